// gfx950 kernels for the sparse indexer's key cache: the FP8 quantise-and-
// insert of index keys and the gather of a batch's cached keys back out.
//
// Reference semantics:
//   src/flaggems_vllm/ops/indexer_k_quant_and_cache.py:44-132 (and the torch
//     oracle of tests/test_indexer_k_quant_and_cache.py:99-142): per token t
//     with slot s >= 0 and quant block j of quant_block_size (128) elements:
//       scale = max(amax_j, 1e-4) / 448     (ue8m0: 2^ceil(log2(scale)))
//       codes = e4m3fn(k[t, j] / scale)
//     into block s / block_size, row s % block_size of the cache, whose block
//     holds block_size x head_dim codes, then block_size x num_quant_blocks
//     float32 scales.
//   src/flaggems_vllm/ops/cp_gather_indexer_k_quant_cache.py:23-176 (torch
//     oracle tests/test_cp_gather_indexer_k_quant_cache.py:83-114): token t of
//     request b (cu_seqlen[b] <= t < cu_seqlen[b + 1]) copies the head_dim
//     codes and num_quant_blocks scales of position t - cu_seqlen[b] (block
//     block_table[b, pos / block_size], row pos % block_size) into row t of
//     k_fp8 and k_fp8_scale.
//
// Layout: one quant block (128 elements, 256 bytes of bf16 / fp16 input) per
// 16-lane DPP row for the insert, each lane one 16-byte piece; the block's
// maximum is a DPP all-reduce (fgv_device.h), the codes one 8-byte store per
// lane, the scale one 4-byte store.  The gather gives one token per 16-lane
// row.  Both are bandwidth- and launch-bound: a DeepSeek-V4 index key is one
// 128-element head, 256 bytes in and 132 bytes out per token.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = kThreads / 16;
constexpr int kQuantBlock = 128;

struct IndexerKArgs {
    const uint16_t* k;
    uint8_t* cache;
    const int64_t* slots;
    int64_t k_stride;        // elements
    int64_t block_stride;    // bytes
    int64_t num_blocks, block_size;
    int64_t head_dim, units; // units = num_tokens * num_quant_blocks
    int32_t nqb;             // quant blocks per token
    int32_t fp16;            // k is float16 (else bfloat16)
    int32_t ue8m0;
};

// Eight bf16 or fp16 values of a 16-byte piece as binary32 (exact).
__device__ __forceinline__ void unpack8_any(uint4 v, bool fp16, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (fp16) {
            x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
            x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        } else {
            x[2 * i] = bf16_lo(w[i]);
            x[2 * i + 1] = bf16_hi(w[i]);
        }
    }
}

__global__ void __launch_bounds__(kThreads)
indexer_k_quant_kernel(IndexerKArgs a) {
    const int lane16 = threadIdx.x & 15;
    const int64_t u = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 4);
    if (u >= a.units)
        return;
    const int64_t t = u / a.nqb;
    const int j = (int)(u - t * a.nqb);
    const int64_t slot = a.slots[t];
    __builtin_amdgcn_sched_barrier(0);  // the slot load ahead of the key load
    const uint4 v = load16(a.k + t * a.k_stride + (int64_t)j * kQuantBlock + 8 * lane16);
    if (slot < 0)
        return;
    const int64_t blk = slot / a.block_size;
    const int64_t row = slot - blk * a.block_size;
    if (blk >= a.num_blocks)
        return;
    float x[8];
    unpack8_any(v, a.fp16 != 0, x);
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        m = max(m, __float_as_uint(x[i]) & 0x7fffffffu);
    const float amax = __uint_as_float(row16_max(m));
    // max(amax, 1e-4) / 448, correctly rounded (HIP's binary32 division)
    float scale = fmaxf(amax, 1e-4f) / kFp8Max;
    float q[8];
    if (a.ue8m0) {
        // 2^ceil(log2(scale)) from the binary32 fields (scale is a normal
        // number >= 1e-4 / 448): exponent, plus one if any mantissa bit is set
        const uint32_t sb = __float_as_uint(scale);
        const int e = (int)(sb >> 23) - 127 + ((sb & 0x7fffffu) ? 1 : 0);
        scale = __uint_as_float((uint32_t)(e + 127) << 23);
        const float inv = exp2_neg_int(e);  // x / 2^e == x * 2^-e exactly
#pragma unroll
        for (int i = 0; i < 8; ++i)
            q[i] = clamp_fp8(x[i] * inv);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            q[i] = clamp_fp8(x[i] / scale);  // correctly rounded division
    }
    uint8_t* base = a.cache + blk * a.block_stride;
    store8(base + row * a.head_dim + (int64_t)j * kQuantBlock + 8 * lane16, pack_fp8x4(q[0], q[1], q[2], q[3]),
           pack_fp8x4(q[4], q[5], q[6], q[7]));
    if (lane16 == 0)
        *reinterpret_cast<float*>(base + a.block_size * a.head_dim + (row * a.nqb + j) * 4) = scale;
}

struct GatherArgs {
    const uint8_t* cache;
    uint8_t* k_out;
    uint8_t* scale_out;
    const int32_t* block_table;
    const int32_t* cu_seqlen;
    int64_t block_stride, num_blocks, block_size;
    int64_t k_out_stride, scale_out_stride, bt_stride;  // bytes, bytes, elements
    int64_t head_dim, num_tokens;
    int32_t batch, max_blocks, nqb;
};

__global__ void __launch_bounds__(kThreads)
indexer_k_gather_kernel(GatherArgs a) {
    const int lane16 = threadIdx.x & 15;
    const int64_t t = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 4);
    if (t >= a.num_tokens || a.batch <= 0)
        return;
    // largest b < batch with cu_seqlen[b] <= t
    int32_t lo = 0, hi = a.batch - 1;
    while (lo < hi) {
        const int32_t mid = (lo + hi + 1) >> 1;
        if (a.cu_seqlen[mid] <= t)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int64_t start = a.cu_seqlen[lo];
    if (t < start || t >= a.cu_seqlen[lo + 1])
        return;  // not inside any request: left as it is
    const int64_t pos = t - start;
    const int64_t bt = pos / a.block_size;
    if (bt >= a.max_blocks)
        return;
    const int64_t blk = a.block_table[lo * a.bt_stride + bt];
    if (blk < 0 || blk >= a.num_blocks)
        return;
    const int64_t row = pos - bt * a.block_size;
    const uint8_t* src = a.cache + blk * a.block_stride + row * a.head_dim;
    uint8_t* dst = a.k_out + t * a.k_out_stride;
    // head_dim is a multiple of 128: 8 bytes per lane per 128
    for (int64_t off = 8 * lane16; off < a.head_dim; off += 128)
        *reinterpret_cast<uint2*>(dst + off) = *reinterpret_cast<const uint2*>(src + off);
    if (lane16 < a.nqb) {
        const uint8_t* s = a.cache + blk * a.block_stride + a.block_size * a.head_dim + (row * a.nqb + lane16) * 4;
        *reinterpret_cast<uint32_t*>(a.scale_out + t * a.scale_out_stride + 4 * lane16) =
            *reinterpret_cast<const uint32_t*>(s);
    }
}

int check_geometry(int64_t head_dim, int64_t quant_block_size) {
    if (quant_block_size != kQuantBlock)
        return fail(FGV_E_BAD_SHAPE, "quant_block_size must be 128");
    if (head_dim <= 0 || head_dim % kQuantBlock || head_dim > 16 * kQuantBlock)
        return fail(FGV_E_BAD_SHAPE, "head_dim must be a positive multiple of 128, at most 2048");
    return FGV_OK;
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_indexer_k_quant_and_cache(
    const void* k, int64_t k_stride_token, int k_is_fp16,
    int64_t num_tokens, int64_t head_dim, int64_t quant_block_size,
    void* kv_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t block_size,
    const int64_t* slot_mapping, int use_ue8m0, void* stream) {
    using namespace fgv;
    int rc = check_geometry(head_dim, quant_block_size);
    if (rc)
        return rc;
    if (num_tokens < 0 || num_blocks < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_tokens == 0)
        return FGV_OK;
    if (block_size <= 0)
        return fail(FGV_E_BAD_SHAPE, "block_size must be positive");
    if (!k || !kv_cache || !slot_mapping)
        return fail(FGV_E_NULL_POINTER, "null k, kv_cache or slot_mapping");
    const int64_t nqb = head_dim / kQuantBlock;
    if (cache_block_stride < block_size * (head_dim + 4 * nqb))
        return fail(FGV_E_BAD_STRIDE, "cache block stride is below block_size * (head_dim + 4 * head_dim / 128)");
    if (!aligned(k, 16) || k_stride_token % 8)
        return fail(FGV_E_MISALIGNED, "k must be 16-byte aligned with a token stride a multiple of 8 elements");
    if (!aligned(kv_cache, 8) || cache_block_stride % 8)
        return fail(FGV_E_MISALIGNED, "kv_cache and its block stride must be 8-byte aligned");
    if (num_tokens > (1LL << 40))
        return fail(FGV_E_TOO_LARGE, "too many tokens");
    IndexerKArgs a;
    a.k = static_cast<const uint16_t*>(k);
    a.cache = static_cast<uint8_t*>(kv_cache);
    a.slots = slot_mapping;
    a.k_stride = k_stride_token;
    a.block_stride = cache_block_stride;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.head_dim = head_dim;
    a.units = num_tokens * nqb;
    a.nqb = (int32_t)nqb;
    a.fp16 = k_is_fp16 != 0;
    a.ue8m0 = use_ue8m0 != 0;
    const int64_t grid = (a.units + kRows - 1) / kRows;
    if (grid > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "grid exceeds 2^31 - 1 workgroups");
    hipLaunchKernelGGL(indexer_k_quant_kernel, dim3((uint32_t)grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), a);
    return launch_status();
}

extern "C" int fgv_cp_gather_indexer_k_quant_cache(
    const void* kv_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t block_size,
    int64_t head_dim, int64_t quant_block_size,
    void* k_out, int64_t k_out_stride, void* scale_out, int64_t scale_out_stride,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_seq,
    const int32_t* cu_seqlen, int64_t batch_size, int64_t num_tokens, void* stream) {
    using namespace fgv;
    int rc = check_geometry(head_dim, quant_block_size);
    if (rc)
        return rc;
    if (num_tokens < 0 || batch_size < 0 || num_blocks < 0 || max_blocks_per_seq < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_tokens == 0 || batch_size == 0)
        return FGV_OK;
    if (block_size <= 0)
        return fail(FGV_E_BAD_SHAPE, "block_size must be positive");
    if (!kv_cache || !k_out || !scale_out || !block_table || !cu_seqlen)
        return fail(FGV_E_NULL_POINTER, "null kv_cache, k_fp8, k_fp8_scale, block_table or cu_seqlen");
    const int64_t nqb = head_dim / kQuantBlock;
    if (cache_block_stride < block_size * (head_dim + 4 * nqb))
        return fail(FGV_E_BAD_STRIDE, "cache block stride is below block_size * (head_dim + 4 * head_dim / 128)");
    if (!aligned(kv_cache, 8) || cache_block_stride % 8 || !aligned(k_out, 8) || k_out_stride % 8)
        return fail(FGV_E_MISALIGNED, "kv_cache, k_fp8 and their strides must be 8-byte aligned");
    if (!aligned(scale_out, 4) || scale_out_stride % 4)
        return fail(FGV_E_MISALIGNED, "k_fp8_scale and its row stride must be 4-byte aligned");
    if (batch_size > 0x7fffffffLL - 1 || max_blocks_per_seq > 0x7fffffffLL || num_tokens > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "batch, block table and token counts must fit in int32");
    GatherArgs a;
    a.cache = static_cast<const uint8_t*>(kv_cache);
    a.k_out = static_cast<uint8_t*>(k_out);
    a.scale_out = static_cast<uint8_t*>(scale_out);
    a.block_table = block_table;
    a.cu_seqlen = cu_seqlen;
    a.block_stride = cache_block_stride;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.k_out_stride = k_out_stride;
    a.scale_out_stride = scale_out_stride;
    a.bt_stride = block_table_stride;
    a.head_dim = head_dim;
    a.num_tokens = num_tokens;
    a.batch = (int32_t)batch_size;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.nqb = (int32_t)nqb;
    const int64_t grid = (num_tokens + kRows - 1) / kRows;
    hipLaunchKernelGGL(indexer_k_gather_kernel, dim3((uint32_t)grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), a);
    return launch_status();
}
