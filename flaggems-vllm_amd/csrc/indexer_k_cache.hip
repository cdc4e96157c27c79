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
// Layout: the insert gives each 16-lane DPP row four consecutive (token,
// quant block) units; a unit's 128 elements are one 16-byte piece per lane,
// its maximum a DPP all-reduce (fgv_device.h), its codes one 8-byte store per
// lane and its scale one 4-byte store.  The gather gives each wave 4R
// consecutive tokens (R per 16-lane group) and finds their requests with one
// 64-way ballot search plus one load of the following request boundaries.
// Both kernels issue every load of a lane before its first store, so a lane
// keeps 64-128 bytes in flight: both are HBM streams (DeepSeek-V4's index key
// is one 128-element head: 256 bytes in and 132 bytes out per token).
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kQuantBlock = 128;
constexpr int kLanes = 8;                      // lanes per quant block in the insert
constexpr int kElems = kQuantBlock / kLanes;   // 16 elements (32 bytes) per lane
constexpr int kGroups = kThreads / kLanes;     // quant blocks per workgroup

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
    int32_t store_bytes;     // 16, 8 or 4: the widest the cache's block alignment allows
};

// Eight bf16 or fp16 values of a 16-byte piece as binary32 (exact).
__device__ __forceinline__ void unpack8_any(uint4 v, bool fp16, float* x) {
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

// (block, row) of a slot; 32-bit division when both fit.
__device__ __forceinline__ void split_slot(int64_t slot, int64_t block_size, int64_t& blk, int64_t& row) {
    if (((uint64_t)slot | (uint64_t)block_size) >> 31)
        blk = slot / block_size;
    else
        blk = (uint32_t)slot / (uint32_t)block_size;
    row = slot - blk * block_size;
}

// One (token, quant block) unit per 8-lane group: two 16-byte key loads and
// one 16-byte code store per lane, the block maximum a 3-step DPP reduction.
// (Measured against 16 lanes x 16 bytes and 4 lanes x 64 bytes per block, and
// against 2-4 units per group: this layout streams fastest.)
__global__ void __launch_bounds__(kThreads)
indexer_k_quant_kernel(IndexerKArgs a) {
    const int ln = threadIdx.x & (kLanes - 1);
    const int64_t u = (int64_t)blockIdx.x * kGroups + threadIdx.x / kLanes;
    if (u >= a.units)
        return;
    const int64_t t = u / a.nqb;
    const int j = (int)(u - t * a.nqb);
    const int64_t slot = a.slots[t];
    const uint16_t* src = a.k + t * a.k_stride + (int64_t)j * kQuantBlock + kElems * ln;
    const uint4 v0 = load16(src), v1 = load16(src + 8);
    if (slot < 0)
        return;
    int64_t blk, row;
    split_slot(slot, a.block_size, blk, row);
    if (blk >= a.num_blocks)
        return;
    float x[kElems];
    unpack8_any(v0, a.fp16 != 0, x);
    unpack8_any(v1, a.fp16 != 0, x + 8);
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < kElems; ++e)
        m = max(m, __float_as_uint(x[e]) & 0x7fffffffu);
    const float amax = __uint_as_float(row8_max(m));
    // max(amax, 1e-4) / 448, correctly rounded (HIP's binary32 division)
    float scale = fmaxf(amax, 1e-4f) / kFp8Max;
    float q[kElems];
    if (a.ue8m0) {
        // 2^ceil(log2(scale)) from the binary32 fields (scale is a normal
        // number >= 1e-4 / 448): exponent, plus one if any mantissa bit is set
        const uint32_t sb = __float_as_uint(scale);
        const int e = (int)(sb >> 23) - 127 + ((sb & 0x7fffffu) ? 1 : 0);
        scale = __uint_as_float((uint32_t)(e + 127) << 23);
        const float inv = exp2_neg_int(e);  // x / 2^e == x * 2^-e exactly
#pragma unroll
        for (int c = 0; c < kElems; ++c)
            q[c] = clamp_fp8(x[c] * inv);
    } else {
#pragma unroll
        for (int c = 0; c < kElems; ++c)
            q[c] = clamp_fp8(x[c] / scale);  // correctly rounded division
    }
    uint8_t* base = a.cache + blk * a.block_stride;
    uint8_t* dst = base + row * a.head_dim + (int64_t)j * kQuantBlock + kElems * ln;
    const uint4 w = make_uint4(pack_fp8x4(q[0], q[1], q[2], q[3]), pack_fp8x4(q[4], q[5], q[6], q[7]),
                               pack_fp8x4(q[8], q[9], q[10], q[11]), pack_fp8x4(q[12], q[13], q[14], q[15]));
    if (a.store_bytes == 16) {
        store16(dst, w);
    } else if (a.store_bytes == 8) {
        store8(dst, w.x, w.y);
        store8(dst + 8, w.z, w.w);
    } else {
        uint32_t* d4 = reinterpret_cast<uint32_t*>(dst);
        d4[0] = w.x;
        d4[1] = w.y;
        d4[2] = w.z;
        d4[3] = w.w;
    }
    if (ln == 0)
        *reinterpret_cast<float*>(base + a.block_size * a.head_dim + (row * a.nqb + j) * 4) = scale;
}

struct GatherArgs {
    const uint8_t* cache;
    uint8_t* k_out;
    uint8_t* scale_out;
    const int32_t* block_table;
    const int32_t* cu_seqlen;
    int64_t block_stride, num_blocks;
    int64_t k_out_stride, scale_out_stride, bt_stride;  // bytes, bytes, elements
    int64_t head_dim;
    int32_t num_tokens, block_size;
    int32_t batch, max_blocks, nqb, nch;
};

// #{j in [0, batch] : cu[j] <= t} for a wave-uniform t, by 64-way ballot
// search (one load per lane per level: two levels cover 4096 requests).
// Every lane of the wave must call it with the same t.
__device__ __forceinline__ int count_le(const int32_t* cu, int batch, int32_t t, int lane) {
    int base = 0, span = batch + 1;  // entries < base are <= t, entries >= base + span are > t
    while (span > 64) {
        const int stride = (span + 63) >> 6;
        const int off = lane * stride;
        const int k = __popcll(__ballot(off < span && cu[base + off] <= t));
        if (k == 0)
            return base;
        const int end = k * stride < span ? base + k * stride : base + span;
        base += (k - 1) * stride + 1;
        span = end - base;
    }
    return base + __popcll(__ballot(lane < span && cu[base + lane] <= t));
}

template <int CB>
struct Chunk;
template <>
struct Chunk<8> {
    typedef u32x2_t T;
};
template <>
struct Chunk<4> {
    typedef uint32_t T;
};
template <>
struct Chunk<16> {
    typedef u32x4_t T;
};

// Each wave gathers 4 * R consecutive tokens, R per 16-lane group (token
// t0 + 4 r + group).  The requests of all of them come from one ballot search
// for t0 (one load of cu[0..batch] below 64 requests) and the few request
// boundaries inside the wave's tokens; then every lane issues its R
// block-table loads, then its R x nch chunk loads of CB bytes, and only then
// stores.  NCH > 0 fixes the chunk count at compile time;
// NCH < 0 means at most -NCH chunks, a.nch of them.
template <int CB, int NCH, int R, int GL>
__global__ void __launch_bounds__(kThreads)
indexer_k_gather_kernel(GatherArgs a) {
    typedef typename Chunk<CB>::T V;
    constexpr int MAXC = NCH > 0 ? NCH : -NCH;
    constexpr int NG = 64 / GL;  // token groups per wave
    const int nch = NCH > 0 ? NCH : a.nch;
    const int lane = threadIdx.x & 63;
    const int g = lane / GL, lg = lane % GL;
    const int64_t t0l = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * (NG * R);
    if (t0l >= a.num_tokens)
        return;
    const int32_t t0 = (int32_t)t0l;
    const int32_t tl = t0 + NG * R - 1;  // the wave's last token
    // c0 = #{cu <= t0}; the request boundaries after it sit in lanes j0, j0 + 1,
    // ... of bnd, and K of them fall inside the wave's tokens.  With at most 63
    // requests one load of cu[0..batch] gives all of it.
    int c0, j0, K;
    int32_t bnd, prev;
    if (a.batch < 64) {
        bnd = lane <= a.batch ? a.cu_seqlen[lane] : 0x7fffffff;
        c0 = __popcll(__ballot(bnd <= t0));
        j0 = c0;
        K = __popcll(__ballot(bnd <= tl)) - c0;
        prev = c0 >= 1 ? __builtin_amdgcn_readlane(bnd, c0 - 1) : 0;
    } else {
        c0 = count_le(a.cu_seqlen, a.batch, t0, lane);
        bnd = c0 + lane <= a.batch ? a.cu_seqlen[c0 + lane] : 0x7fffffff;
        prev = c0 >= 1 ? a.cu_seqlen[c0 - 1] : 0;
        j0 = 0;
        K = __popcll(__ballot(bnd <= tl));
    }
    int req[R];
    int32_t start[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        req[r] = c0 - 1;
        start[r] = prev;
    }
    if (K < 64 - j0 || a.batch < 64) {
        // usually K is 0 or 1: step each token past the boundaries at or below it
        for (int j = 0; j < K; ++j) {
            const int32_t b = __builtin_amdgcn_readlane(bnd, j0 + j);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (t0 + NG * r + g >= b) {
                    ++req[r];
                    start[r] = b;
                }
            }
        }
    } else {
        // 64 or more requests start inside this wave's tokens (empty
        // requests): search each token on its own
#pragma unroll
        for (int w = 0; w < NG * R; ++w) {
            const int c = count_le(a.cu_seqlen, a.batch, t0 + w, lane);
            const int32_t st = c >= 1 ? a.cu_seqlen[c - 1] : 0;
            if (w % NG == g) {
                req[w / NG] = c - 1;
                start[w / NG] = st;
            }
        }
    }
    int64_t blk[R];
    int32_t row[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int32_t t = t0 + NG * r + g;
        const int b = req[r];
        ok[r] = t < a.num_tokens && b >= 0 && b < a.batch;
        const int32_t pos = t - start[r];
        const int32_t bi = (int32_t)((uint32_t)pos / (uint32_t)a.block_size);
        ok[r] = ok[r] && bi < a.max_blocks;
        blk[r] = ok[r] ? (int64_t)a.block_table[(int64_t)b * a.bt_stride + bi] : -1;
        ok[r] = ok[r] && blk[r] >= 0 && blk[r] < a.num_blocks;
        row[r] = pos - bi * a.block_size;
    }
    V d[R][MAXC];
    uint32_t s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!ok[r])
            continue;
        const uint8_t* base = a.cache + blk[r] * a.block_stride;
        const uint8_t* p = base + (int64_t)row[r] * a.head_dim + CB * lg;
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
            if (i < nch)
                d[r][i] = __builtin_nontemporal_load(reinterpret_cast<const V*>(p + i * GL * CB));
        if (lg < a.nqb)
            s[r] = *reinterpret_cast<const uint32_t*>(base + (int64_t)a.block_size * a.head_dim +
                                                        ((int64_t)row[r] * a.nqb + lg) * 4);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!ok[r])
            continue;
        const int64_t t = t0 + NG * r + g;
        uint8_t* q = a.k_out + t * a.k_out_stride + CB * lg;
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
            if (i < nch)
                __builtin_nontemporal_store(d[r][i], reinterpret_cast<V*>(q + i * GL * CB));
        if (lg < a.nqb)
            *reinterpret_cast<uint32_t*>(a.scale_out + t * a.scale_out_stride + 4 * lg) = s[r];
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
    if (!aligned(kv_cache, 4) || cache_block_stride % 4)
        return fail(FGV_E_MISALIGNED, "kv_cache and its block stride must be 4-byte aligned");
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
    // a block of block_size x (head_dim + head_dim / 32) bytes is 16-byte
    // aligned when block_size is a multiple of 4, 8-byte aligned when even
    a.store_bytes = aligned(kv_cache, 16) && cache_block_stride % 16 == 0  ? 16
                    : aligned(kv_cache, 8) && cache_block_stride % 8 == 0 ? 8
                                                                          : 4;
    const int64_t grid = (a.units + kGroups - 1) / kGroups;
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
    if (!aligned(kv_cache, 4) || cache_block_stride % 4 || !aligned(k_out, 4) || k_out_stride % 4)
        return fail(FGV_E_MISALIGNED, "kv_cache, k_fp8 and their strides must be 4-byte aligned");
    if (!aligned(scale_out, 4) || scale_out_stride % 4)
        return fail(FGV_E_MISALIGNED, "k_fp8_scale and its row stride must be 4-byte aligned");
    if (batch_size > (1LL << 30) || max_blocks_per_seq > 0x7fffffffLL || num_tokens > 0x7fffffffLL - 64)
        return fail(FGV_E_TOO_LARGE, "batch must be at most 2^30, block table and token counts below 2^31 - 64");
    if (block_size > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "block_size must fit in int32");
    GatherArgs a;
    a.cache = static_cast<const uint8_t*>(kv_cache);
    a.k_out = static_cast<uint8_t*>(k_out);
    a.scale_out = static_cast<uint8_t*>(scale_out);
    a.block_table = block_table;
    a.cu_seqlen = cu_seqlen;
    a.block_stride = cache_block_stride;
    a.num_blocks = num_blocks;
    a.k_out_stride = k_out_stride;
    a.scale_out_stride = scale_out_stride;
    a.bt_stride = block_table_stride;
    a.head_dim = head_dim;
    a.num_tokens = (int32_t)num_tokens;
    a.block_size = (int32_t)block_size;
    a.batch = (int32_t)batch_size;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.nqb = (int32_t)nqb;
    // 16-byte chunks where head_dim is 128, 256, 512, 1024 or 2048 and the
    // code rows are 16-byte aligned on both sides, else 8-byte chunks, or
    // 4-byte ones where a row is only 4-byte aligned (an odd block_size)
    const bool wide = (head_dim & (head_dim - 1)) == 0 && aligned(kv_cache, 16) && cache_block_stride % 16 == 0 &&
                      aligned(k_out, 16) && k_out_stride % 16 == 0;
    const bool narrow = !(aligned(kv_cache, 8) && cache_block_stride % 8 == 0 && aligned(k_out, 8) &&
                          k_out_stride % 8 == 0);
    a.nch = (int32_t)(narrow ? head_dim / 64 : head_dim / 128);
    // Below 16384 tokens the launch is latency-bound and one token per lane
    // group is fastest; above, several tokens per group keep more loads in
    // flight (measured on MI355X: 2 at head_dim 512, 4 at 128).
    const bool big = num_tokens >= 16384;
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto launch = [&](auto kernel, int tokens_per_wave) {
        const int64_t per_block = (kThreads / 64) * tokens_per_wave;
        const int64_t grid = (num_tokens + per_block - 1) / per_block;
        hipLaunchKernelGGL(kernel, dim3((uint32_t)grid), dim3(kThreads), 0, st, a);
    };
    if (wide && head_dim == 128)
        big ? launch(indexer_k_gather_kernel<16, 1, 4, 8>, 32) : launch(indexer_k_gather_kernel<16, 1, 1, 8>, 8);
    else if (wide && head_dim == 256)
        big ? launch(indexer_k_gather_kernel<16, 1, 4, 16>, 16) : launch(indexer_k_gather_kernel<16, 1, 1, 16>, 4);
    else if (wide && head_dim == 512)
        big ? launch(indexer_k_gather_kernel<16, 2, 2, 16>, 8) : launch(indexer_k_gather_kernel<16, 2, 1, 16>, 4);
    else if (wide && head_dim == 1024)
        launch(indexer_k_gather_kernel<16, 4, 1, 16>, 4);
    else if (wide)
        launch(indexer_k_gather_kernel<16, 8, 1, 16>, 4);
    else if (narrow)
        launch(indexer_k_gather_kernel<4, -32, 1, 16>, 4);
    else
        launch(indexer_k_gather_kernel<8, -16, 1, 16>, 4);
    return launch_status();
}
