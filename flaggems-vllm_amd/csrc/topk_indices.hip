// gfx950 kernels that turn the sparse indexer's per-token top-k selection
// into the index rows sparse MLA decode reads.
//
//   global_topk_indices_kernel  (compute_global_topk_indices_and_lens;
//     reference src/flaggems_vllm/ops/deepseek_v4_attention_compute_global_topk_indices_and_lens.py:46-160):
//     a request-local index l >= 0 becomes the cache slot
//     block_table[req, l / block_size] * block_size + l % block_size, -1 stays
//     -1, and the row's length is the count of l >= 0 (0 for a token marked
//     invalid).
//   combine_topk_swa_kernel  (combine_topk_swa_indices;
//     reference src/flaggems_vllm/ops/deepseek_v4_attention_combine_topk_swa_indices.py:30-153):
//     for token t of request b at position pos, the first
//     min((pos + 1) / compress_ratio, topk) top-k indices offset by M * b,
//     then the min(pos + 1, window) sliding-window rows
//     M * b + N + pos - swa_len + 1 - gather_start + j, then -1 up to the
//     row width (topk + window rounded up to 128); the row's length.
//
// Both are integer gathers and stores of a few MB, bound by launch and
// latency rather than bandwidth: one wave per token row, lanes striding over
// its columns (coalesced 256-byte accesses), the row's scalars (request,
// position) read once per wave.  Arithmetic is int32 with wrap-around, as
// the reference's Triton kernels compute it.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

__device__ __forceinline__ int32_t wrap_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }

struct GlobalArgs {
    const int32_t* local;
    int64_t local_s0, local_s1;
    const int32_t* req;
    const int32_t* table;
    int64_t table_stride;
    int64_t table_span;  // elements of the block table addressable as req * stride + block
    const int32_t* valid;  // or null: every token valid
    int32_t* out;
    int64_t out_s0, out_s1;
    int32_t* lens;
    int64_t num_tokens;
    int32_t topk, block_size;
};

__global__ void __launch_bounds__(kThreads)
global_topk_indices_kernel(GlobalArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + wave;
    if (t >= a.num_tokens)
        return;
    const int64_t row = (int64_t)a.req[t] * a.table_stride;
    const int32_t* lrow = a.local + t * a.local_s0;
    int32_t* orow = a.out + t * a.out_s0;
    int32_t count = 0;
    // lane 0 runs every pass, so its count is the row's
    for (int32_t i = lane; i < a.topk; i += 64) {
        const int32_t l = lrow[i * a.local_s1];
        int32_t slot = -1;
        if (l >= 0) {
            const int32_t blk = l / a.block_size;
            const int64_t f = row + blk;
            // a block outside the table (an invalid local index or request)
            // has no slot; the reference would read past its row
            if (f >= 0 && f < a.table_span)
                slot = wrap_add(wrap_mul(a.table[f], a.block_size), l - blk * a.block_size);
        }
        orow[i * a.out_s1] = slot;
        count += __popcll(__ballot(l >= 0));
    }
    if (lane == 0)
        a.lens[t] = (a.valid == nullptr || a.valid[t] != 0) ? count : 0;
}

struct CombineArgs {
    const int32_t* topk;
    int64_t topk_s0, topk_s1;
    const int32_t* qsl;
    const int32_t* seq_lens;
    const int32_t* gather_lens;
    int32_t* out;
    int64_t out_s0, out_s1;
    int32_t* lens;
    int32_t num_tokens;  // rows of topk, combined and lens
    int32_t window, ratio, topk_n, m, n, width;
};

// Grid (requests, workers): wave w of worker k takes the request's tokens
// k * 4 + w, stepping by 4 * workers, as the reference's programs stride
// over a request's tokens.  Tokens outside every request are not written, and
// neither are tokens that query_start_loc places outside [0, num_tokens) (the
// tensors' rows), which the reference would read and write out of bounds.
__global__ void __launch_bounds__(kThreads)
combine_topk_swa_kernel(CombineArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int32_t b = blockIdx.x;
    const int32_t base = a.qsl[0];
    const int32_t qs = a.qsl[b] - base, qe = a.qsl[b + 1] - base;
    const int32_t seq = a.seq_lens[b];
    const int32_t start_pos = seq - (qe - qs), gather_start = seq - a.gather_lens[b];
    const int32_t row_off = wrap_mul(a.m, b);
    const int32_t step = (int32_t)gridDim.y * kRowsPerBlock;
    const int32_t end = min(qe, a.num_tokens);
    for (int32_t t = qs + (int32_t)blockIdx.y * kRowsPerBlock + wave; t < end; t += step) {
        if (t < 0)
            continue;
        const int32_t pos = start_pos + (t - qs);
        // C (truncating) division, as Triton divides int32
        const int32_t topk_len = min((pos + 1) / a.ratio, a.topk_n);
        const int32_t swa_len = min(pos + 1, a.window);
        const int32_t swa_base = wrap_add(wrap_add(row_off, a.n), pos - swa_len + 1 - gather_start);
        const int32_t* trow = a.topk + (int64_t)t * a.topk_s0;
        int32_t* orow = a.out + (int64_t)t * a.out_s0;
        for (int32_t c = lane; c < a.width; c += 64) {
            int32_t v = -1;
            if (c < topk_len)
                v = wrap_add(trow[c * a.topk_s1], row_off);
            else if (c - topk_len < swa_len && c - topk_len < a.window)
                v = wrap_add(swa_base, c - topk_len);
            orow[c * a.out_s1] = v;
        }
        if (lane == 0)
            a.lens[t] = topk_len + swa_len;
    }
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_compute_global_topk_indices_and_lens(
    const int32_t* topk_indices, int64_t topk_stride0, int64_t topk_stride1, int64_t num_tokens, int64_t topk,
    const int32_t* token_to_req_indices, const int32_t* block_table, int64_t block_table_stride,
    int64_t num_reqs, int64_t blocks_per_req, int64_t block_size, const int32_t* is_valid_token,
    int32_t* global_indices, int64_t out_stride0, int64_t out_stride1, int32_t* lens, void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || topk < 0 || num_reqs < 0 || blocks_per_req < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (block_size <= 0)
        return fail(FGV_E_BAD_SHAPE, "block_size must be positive");
    if (num_tokens == 0)
        return FGV_OK;
    if (topk > 0x7fffffffLL || block_size > 0x7fffffffLL || num_tokens > (1LL << 40))
        return fail(FGV_E_TOO_LARGE, "top-k and block_size must fit in int32");
    if (!topk_indices || !token_to_req_indices || !global_indices || !lens ||
        (topk > 0 && num_reqs > 0 && blocks_per_req > 0 && !block_table))
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (!aligned(topk_indices, 4) || !aligned(global_indices, 4) || !aligned(lens, 4) ||
        !aligned(token_to_req_indices, 4) || (block_table && !aligned(block_table, 4)) ||
        (is_valid_token && !aligned(is_valid_token, 4)))
        return fail(FGV_E_MISALIGNED, "int32 arguments must be 4-byte aligned");
    GlobalArgs a;
    a.local = topk_indices;
    a.local_s0 = topk_stride0;
    a.local_s1 = topk_stride1;
    a.req = token_to_req_indices;
    a.table = block_table;
    a.table_stride = block_table_stride;
    a.table_span = (num_reqs > 0 && blocks_per_req > 0) ? (num_reqs - 1) * block_table_stride + blocks_per_req : 0;
    a.valid = is_valid_token;
    a.out = global_indices;
    a.out_s0 = out_stride0;
    a.out_s1 = out_stride1;
    a.lens = lens;
    a.num_tokens = num_tokens;
    a.topk = (int32_t)topk;
    a.block_size = (int32_t)block_size;
    const dim3 grid((unsigned)((num_tokens + kRowsPerBlock - 1) / kRowsPerBlock));
    hipLaunchKernelGGL(global_topk_indices_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
    return launch_status();
}

extern "C" int64_t fgv_combine_topk_swa_width(int64_t topk, int64_t window_size) {
    if (topk < 0 || window_size < 0)
        return -1;
    return (topk + window_size + 127) / 128 * 128;
}

extern "C" int fgv_combine_topk_swa_indices(
    const int32_t* topk_indices, int64_t topk_stride0, int64_t topk_stride1, int64_t num_tokens,
    int64_t topk_cols, const int32_t* query_start_loc, const int32_t* seq_lens, const int32_t* gather_lens,
    int64_t num_reqs, int64_t window_size, int64_t compress_ratio, int64_t topk, int64_t M, int64_t N,
    int32_t* combined, int64_t out_stride0, int64_t out_stride1, int32_t* lens, void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || topk_cols < 0 || num_reqs < 0 || window_size < 0 || topk < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (compress_ratio <= 0)
        return fail(FGV_E_BAD_SHAPE, "compress_ratio must be positive");
    if (topk > topk_cols)
        return fail(FGV_E_BAD_SHAPE, "topk exceeds the columns of topk_indices");
    if (num_reqs == 0 || num_tokens == 0)
        return FGV_OK;
    const int64_t width = fgv_combine_topk_swa_width(topk, window_size);
    if (width > 0x7fffffffLL || num_reqs > 0x7fffffffLL || num_tokens > 0x7fffffffLL ||
        compress_ratio > 0x7fffffffLL || M < -0x80000000LL || M > 0x7fffffffLL || N < -0x80000000LL ||
        N > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "sizes must fit in int32");
    if (!topk_indices || !query_start_loc || !seq_lens || !gather_lens || !combined || !lens)
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (!aligned(topk_indices, 4) || !aligned(combined, 4) || !aligned(lens, 4) || !aligned(query_start_loc, 4) ||
        !aligned(seq_lens, 4) || !aligned(gather_lens, 4))
        return fail(FGV_E_MISALIGNED, "int32 arguments must be 4-byte aligned");
    CombineArgs a;
    a.topk = topk_indices;
    a.topk_s0 = topk_stride0;
    a.topk_s1 = topk_stride1;
    a.qsl = query_start_loc;
    a.seq_lens = seq_lens;
    a.gather_lens = gather_lens;
    a.out = combined;
    a.out_s0 = out_stride0;
    a.out_s1 = out_stride1;
    a.lens = lens;
    a.num_tokens = (int32_t)num_tokens;
    a.window = (int32_t)window_size;
    a.ratio = (int32_t)compress_ratio;
    a.topk_n = (int32_t)topk;
    a.m = (int32_t)M;
    a.n = (int32_t)N;
    a.width = (int32_t)width;
    // enough waves for the average request's tokens, at most 128 workers
    // (the reference's grid) per request
    const int64_t per_req = (num_tokens + num_reqs - 1) / num_reqs;
    const int64_t workers = std::min<int64_t>(128, std::max<int64_t>(1, (per_req + kRowsPerBlock - 1) / kRowsPerBlock));
    if (num_reqs > 0x7fffffffLL / workers)
        return fail(FGV_E_TOO_LARGE, "too many requests");
    hipLaunchKernelGGL(combine_topk_swa_kernel, dim3((unsigned)num_reqs, (unsigned)workers), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), a);
    return launch_status();
}
