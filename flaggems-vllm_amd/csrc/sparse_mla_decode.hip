// gfx950 kernel for sparse MLA decode over the 584-byte MODEL1 cache: each
// query row attends the top-k cache entries its indices select, K = V = the
// dequantised 512-wide latent of each entry (448 e4m3 NoPE values with one
// E8M0 scale per 64, then 64 bf16 RoPE values).
//
// Reference semantics: src/flaggems_vllm/ops/flash_mla_with_kvcache.py:489-688
// (portable MODEL1 kernel) and src/flaggems_vllm/ops/flash_mla_with_kvcache_model1.py:389-470,
// 699-720 (sm90 kernel: mask, epilogue, attention sink).
//
// One workgroup of 4 waves per (batch row, query position, 64-head block);
// wave w owns heads 16w..16w+15.  The selected entries stream through in
// chunks of 32:
//   1. every thread gathers 4 entries x 8 dims (coalesced 576-byte rows),
//      dequantises them to bf16 (exact: e4m3 value times a power of two) and
//      writes them to LDS twice: row-major K[entry][dim] and dim-major
//      V^T[dim][entry];
//   2. S^T = K q^T on v_mfma_f32_16x16x32_bf16 (A = K from LDS, B = q held in
//      registers for the whole kernel), so each lane ends up with one head
//      and 8 entries of the chunk;
//   3. online softmax in base 2 per head (two cross-lane shuffles), the
//      probabilities rounded to bf16 become the B operand of
//   4. O^T += V^T P^T (A = V^T from LDS), accumulated in fp32 registers.
// The chunk's 32 entries are placed in V^T columns in the order the S^T
// accumulator hands them to each lane, so P needs no data movement between
// the two products.  Both products reduce over the same k permutation in A
// and B, so the MFMA's internal k order does not matter.
#include <math.h>

#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kBlockHeads = 64;
constexpr int kChunk = 32;    // entries per chunk
constexpr int kKRow = 520;    // K row stride in bf16 (1040 B: 8 lanes of a b128 read hit distinct banks)
constexpr int kVRow = 40;     // V^T row stride in bf16 (80 B, same reason)
constexpr float kLn2 = 0.693147180559945309f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct CacheList {
    const uint8_t* cache;
    const int32_t* indices;
    const int32_t* lengths;  // [batch] or null
    int64_t block_stride;    // bytes
    int64_t idx_stride_b, idx_stride_s;
    int32_t num_blocks, page_size, topk, pad;
};

struct MlaArgs {
    const uint16_t* q;
    int64_t q_sb, q_ss, q_sh;
    uint16_t* out;
    int64_t o_sb, o_ss, o_sh;
    float* lse;
    int64_t l_sb, l_sh;
    const float* sink;
    CacheList list[2];
    int32_t num_lists;
    int32_t seq_q, head_blocks;
    float scale_log2;  // softmax scale * log2(e)
};

// V^T column of the first of the 4 entries 4*quad..4*quad+3: lane group g of
// the S^T accumulator holds entries 4g..4g+3 (first 16-entry tile) and
// 16+4g..16+4g+3 (second tile), which become k = 8g..8g+7 of the PV product.
__device__ __forceinline__ int vt_column(int quad) {
    return quad < 4 ? 8 * quad : 8 * (quad - 4) + 4;
}

template <bool kHigh>
__device__ __forceinline__ uint32_t dequant2(uint32_t word, float scale) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, kHigh);
    return pack_bf16x2(f.x * scale, f.y * scale);
}

// 8 e4m3 codes (two words) times a power-of-two scale -> 8 bf16.
__device__ __forceinline__ uint4 dequant8(uint32_t lo, uint32_t hi, float scale) {
    return make_uint4(dequant2<false>(lo, scale), dequant2<true>(lo, scale),
                      dequant2<false>(hi, scale), dequant2<true>(hi, scale));
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__global__ void __launch_bounds__(kThreads, 2)
sparse_mla_decode_kernel(MlaArgs a) {
    __shared__ __align__(16) uint16_t k_lds[kChunk * kKRow];
    __shared__ __align__(16) uint16_t vt_lds[kHeadDim * kVRow];
    __shared__ float mask_lds[kChunk];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int m16 = lane & 15, g = lane >> 4;
    const int hb = blockIdx.x % a.head_blocks;
    const int bs = blockIdx.x / a.head_blocks;
    const int sq = bs % a.seq_q, b = bs / a.seq_q;
    const int head = hb * kBlockHeads + wave * 16 + m16;

    // q as the B operand of S^T = K q^T: step s covers dims 32s..32s+31, lane
    // group g dims 32s+8g..32s+8g+7 of head m16.
    const uint16_t* qrow = a.q + b * a.q_sb + sq * a.q_ss + head * a.q_sh;
    bf16x8_t qf[16];
#pragma unroll
    for (int s = 0; s < 16; ++s)
        qf[s] = __builtin_bit_cast(bf16x8_t, load16(qrow + 32 * s + 8 * g));

    f32x4_t acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
        acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    // Gather geometry: entries 4*quad..4*quad+3 of the chunk, dims 8*d8..8*d8+7
    // for d8 = d8a (NoPE) and d8b = d8a + 32 (NoPE below 56, RoPE from 56 on:
    // exactly wave 3).
    const int quad = tid & 7;
    const int d8a = tid >> 3, d8b = d8a + 32;
    const bool rope_unit = d8b >= kNopeDim / 8;
    const int col0 = vt_column(quad);

    for (int li = 0; li < a.num_lists; ++li) {
        const CacheList& L = a.list[li];
        int len = L.topk;
        if (L.lengths) {
            const int n = L.lengths[b];
            len = n < 0 ? 0 : (n > L.topk ? L.topk : n);
        }
        const int32_t* idx = L.indices + b * L.idx_stride_b + sq * L.idx_stride_s;
        const int64_t scale_off = (int64_t)L.page_size * kTokenDataBytes;

        for (int t0 = 0; t0 < len; t0 += kChunk) {
            // ---- gather + dequantise 4 entries x 2 pieces of 8 dims
            uint4 ka[4], kb[4];
            bool valid[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + 4 * quad + r;
                const int id = t < len ? idx[t] : -1;
                const int page = id >= 0 ? id / L.page_size : 0;
                valid[r] = id >= 0 && page < L.num_blocks;
                ka[r] = make_uint4(0, 0, 0, 0);
                kb[r] = make_uint4(0, 0, 0, 0);
                if (valid[r]) {
                    const int rel = id - page * L.page_size;
                    const uint8_t* blk = L.cache + (int64_t)page * L.block_stride;
                    const uint8_t* tok = blk + (int64_t)rel * kTokenDataBytes;
                    const uint64_t scales =
                        *reinterpret_cast<const uint64_t*>(blk + scale_off + (int64_t)rel * kScaleBytesPerToken);
                    const uint2 na = *reinterpret_cast<const uint2*>(tok + 8 * d8a);
                    const float sa = __uint_as_float((uint32_t)((scales >> (8 * (d8a >> 3))) & 0xff) << 23);
                    ka[r] = dequant8(na.x, na.y, sa);
                    if (rope_unit) {
                        kb[r] = *reinterpret_cast<const uint4*>(tok + kNopeDim + 16 * (d8b - kNopeDim / 8));
                    } else {
                        const uint2 nb = *reinterpret_cast<const uint2*>(tok + 8 * d8b);
                        const float sb = __uint_as_float((uint32_t)((scales >> (8 * (d8b >> 3))) & 0xff) << 23);
                        kb[r] = dequant8(nb.x, nb.y, sb);
                    }
                }
            }

            __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                *reinterpret_cast<uint4*>(&k_lds[(4 * quad + r) * kKRow + 8 * d8a]) = ka[r];
                *reinterpret_cast<uint4*>(&k_lds[(4 * quad + r) * kKRow + 8 * d8b]) = kb[r];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int w = j >> 1;
                uint32_t x0, x1, y0, y1;
                if (j & 1) {
                    x0 = (word_of(ka[0], w) >> 16) | (word_of(ka[1], w) & 0xffff0000u);
                    x1 = (word_of(ka[2], w) >> 16) | (word_of(ka[3], w) & 0xffff0000u);
                    y0 = (word_of(kb[0], w) >> 16) | (word_of(kb[1], w) & 0xffff0000u);
                    y1 = (word_of(kb[2], w) >> 16) | (word_of(kb[3], w) & 0xffff0000u);
                } else {
                    x0 = (word_of(ka[0], w) & 0xffffu) | (word_of(ka[1], w) << 16);
                    x1 = (word_of(ka[2], w) & 0xffffu) | (word_of(ka[3], w) << 16);
                    y0 = (word_of(kb[0], w) & 0xffffu) | (word_of(kb[1], w) << 16);
                    y1 = (word_of(kb[2], w) & 0xffffu) | (word_of(kb[3], w) << 16);
                }
                *reinterpret_cast<uint2*>(&vt_lds[(8 * d8a + j) * kVRow + col0]) = make_uint2(x0, x1);
                *reinterpret_cast<uint2*>(&vt_lds[(8 * d8b + j) * kVRow + col0]) = make_uint2(y0, y1);
            }
            if (tid < 8) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    mask_lds[4 * quad + r] = valid[r] ? 0.f : -INFINITY;
            }
            __syncthreads();

            // ---- S^T = K q^T for the chunk's two 16-entry tiles
            f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(&k_lds[m16 * kKRow + 32 * s + 8 * g]);
                const bf16x8_t a1 =
                    *reinterpret_cast<const bf16x8_t*>(&k_lds[(16 + m16) * kKRow + 32 * s + 8 * g]);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[s], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[s], s1, 0, 0, 0);
            }

            // ---- online softmax (base 2) for head m16 over entries 4g+r, 16+4g+r
            float sv[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sv[r] = s0[r] * a.scale_log2 + mask_lds[4 * g + r];
                sv[4 + r] = s1[r] * a.scale_log2 + mask_lds[16 + 4 * g + r];
            }
            float cmax = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i)
                cmax = fmaxf(cmax, sv[i]);
            cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
            cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
            const float m_new = fmaxf(m_run, cmax);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            float p[8], psum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
                psum += p[i];
            }
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
            l_run = l_run * alpha + psum;
            m_run = m_new;
            const uint4 pw = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                                        pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7]));
            const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pw);

            // ---- O^T = alpha * O^T + V^T P^T over the 32 16-dim tiles
#pragma unroll
            for (int dt = 0; dt < 32; ++dt) {
                const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(&vt_lds[(16 * dt + m16) * kVRow + 8 * g]);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb, acc[dt] * alpha, 0, 0, 0);
            }
        }
    }

    // ---- epilogue: lse excludes the sink; the sink only rescales O
    const bool any = m_run != -INFINITY;
    float factor = 0.f;
    if (any)
        factor = a.sink ? 1.f / (l_run + expf(a.sink[head] - m_run * kLn2)) : 1.f / l_run;
    uint16_t* orow = a.out + b * a.o_sb + sq * a.o_ss + head * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
        const f32x4_t v = acc[dt] * factor;
        *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
    if (g == 0)
        a.lse[b * a.l_sb + head * a.l_sh + sq] = any ? m_run * kLn2 + logf(l_run) : INFINITY;
}

bool fill_list(CacheList& L, const void* cache, int64_t block_stride, int64_t num_blocks, int64_t page_size,
               const int32_t* indices, int64_t idx_sb, int64_t idx_ss, int64_t topk, const int32_t* lengths) {
    L.cache = static_cast<const uint8_t*>(cache);
    L.indices = indices;
    L.lengths = lengths;
    L.block_stride = block_stride;
    L.idx_stride_b = idx_sb;
    L.idx_stride_s = idx_ss;
    L.num_blocks = (int32_t)num_blocks;
    L.page_size = (int32_t)page_size;
    L.topk = (int32_t)topk;
    L.pad = 0;
    return true;
}

int check_list(const char* which, const void* cache, int64_t block_stride, int64_t num_blocks,
               int64_t page_size, const int32_t* indices, int64_t topk) {
    (void)which;
    if (!cache || !indices)
        return fail(FGV_E_NULL_POINTER, "null cache or indices");
    if (page_size <= 0 || num_blocks < 0 || topk < 0)
        return fail(FGV_E_BAD_SHAPE, "page size must be positive, block count and top-k non-negative");
    if (page_size > 0x7fffffffLL / 64 || num_blocks > 0x7fffffffLL || topk > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "page size, block count and top-k must fit in int32");
    if (block_stride < page_size * (kTokenDataBytes + kScaleBytesPerToken))
        return fail(FGV_E_BAD_STRIDE, "cache block stride is below page_size * 584 bytes");
    if (!aligned(cache, 16) || block_stride % 16)
        return fail(FGV_E_MISALIGNED, "cache base and block stride must be 16-byte aligned");
    if (!aligned(indices, 4))
        return fail(FGV_E_MISALIGNED, "indices must be 4-byte aligned");
    return FGV_OK;
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_sparse_mla_decode_model1(
    const void* q, int64_t q_stride_b, int64_t q_stride_s, int64_t q_stride_h,
    const void* k_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t page_size,
    const int32_t* indices, int64_t idx_stride_b, int64_t idx_stride_s, int64_t topk,
    const int32_t* topk_length,
    const void* extra_k_cache, int64_t extra_block_stride, int64_t extra_num_blocks, int64_t extra_page_size,
    const int32_t* extra_indices, int64_t extra_idx_stride_b, int64_t extra_idx_stride_s, int64_t extra_topk,
    const int32_t* extra_topk_length,
    const float* attn_sink, float softmax_scale,
    void* out, int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h,
    float* lse, int64_t lse_stride_b, int64_t lse_stride_h,
    int64_t batch, int64_t seq_q, int64_t num_heads, void* stream) {
    using namespace fgv;
    if (batch < 0 || seq_q < 0 || num_heads < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_heads % kBlockHeads)
        return fail(FGV_E_BAD_SHAPE, "num_heads must be a multiple of 64");
    if (batch == 0 || seq_q == 0 || num_heads == 0)
        return FGV_OK;
    if (batch * seq_q * (num_heads / kBlockHeads) > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "batch * seq_q * num_heads / 64 must be below 2^31");
    if (!q || !out || !lse)
        return fail(FGV_E_NULL_POINTER, "null q, out or lse");
    if (!aligned(q, 16) || q_stride_b % 8 || q_stride_s % 8 || q_stride_h % 8)
        return fail(FGV_E_MISALIGNED, "q must be 16-byte aligned with strides a multiple of 8 elements");
    if (!aligned(out, 8) || out_stride_b % 4 || out_stride_s % 4 || out_stride_h % 4)
        return fail(FGV_E_MISALIGNED, "out must be 8-byte aligned with strides a multiple of 4 elements");
    if (!aligned(lse, 4))
        return fail(FGV_E_MISALIGNED, "lse must be 4-byte aligned");
    int rc = check_list("main", k_cache, cache_block_stride, num_blocks, page_size, indices, topk);
    if (rc)
        return rc;
    MlaArgs a;
    a.num_lists = 1;
    fill_list(a.list[0], k_cache, cache_block_stride, num_blocks, page_size, indices, idx_stride_b,
              idx_stride_s, topk, topk_length);
    if (extra_k_cache) {
        rc = check_list("extra", extra_k_cache, extra_block_stride, extra_num_blocks, extra_page_size,
                        extra_indices, extra_topk);
        if (rc)
            return rc;
        fill_list(a.list[1], extra_k_cache, extra_block_stride, extra_num_blocks, extra_page_size,
                  extra_indices, extra_idx_stride_b, extra_idx_stride_s, extra_topk, extra_topk_length);
        a.num_lists = 2;
    } else if (extra_indices || extra_topk_length) {
        return fail(FGV_E_BAD_SHAPE, "extra indices or lengths given without an extra cache");
    } else {
        a.list[1] = a.list[0];
    }
    a.q = static_cast<const uint16_t*>(q);
    a.q_sb = q_stride_b;
    a.q_ss = q_stride_s;
    a.q_sh = q_stride_h;
    a.out = static_cast<uint16_t*>(out);
    a.o_sb = out_stride_b;
    a.o_ss = out_stride_s;
    a.o_sh = out_stride_h;
    a.lse = lse;
    a.l_sb = lse_stride_b;
    a.l_sh = lse_stride_h;
    a.sink = attn_sink;
    a.seq_q = (int32_t)seq_q;
    a.head_blocks = (int32_t)(num_heads / kBlockHeads);
    a.scale_log2 = (float)((double)softmax_scale * 1.4426950408889634);
    const dim3 grid((unsigned)(batch * seq_q * a.head_blocks));
    hipLaunchKernelGGL(sparse_mla_decode_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
    return launch_status();
}
