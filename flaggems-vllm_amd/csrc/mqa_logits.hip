// gfx950 kernels for the sparse indexer's logits: every query token's
// weighted, ReLU-gated dot products with the cached index keys.
//
// Reference semantics:
//   src/flaggems_vllm/ops/fp8_fp4_mqa_logits.py:88-187 (FP8 kernel), :232-358
//     (MXFP4 kernel), :190-222 (clean), wrapper :523-651, and the float32
//     oracle of tests/test_fp8_fp4_mqa_logits.py:40-66:
//       logits[m, n] = sum_h ReLU((sum_d q[m,h,d] k[n,d]) * k_scale[n]) * w[m,h]
//     with q e4m3fn, or E2M1 times 2^(byte - 127) per 32 elements (MXFP4), and
//     k e4m3fn; clean_logits writes -inf where n < ks[m] or n >= ke[m].
//   src/flaggems_vllm/ops/fp8_fp4_paged_mqa_logits.py:68-181 (kernel),
//     :185-225 (cache layout), :410-579 (wrapper): the same per row of
//     B * next_n query tokens over positions n < context_len[row] of a paged
//     cache [blocks, block_size, 1, 132] (block_size x 128 code bytes, then
//     block_size float32 scales), block index clamped into [0, blocks); every
//     other position of the [rows, max_model_len] output gets the fill value
//     (0, or -inf with clean_logits).
//
// The dot products run on v_mfma_scale_f32_16x16x128_f8f6f4: one
// instruction is one (16 heads) x (16 keys) tile over all 128 dims.  FP8 q
// uses it unscaled; MXFP4 q is the FP4 A operand with its UE8M0 bytes as the
// hardware's per-32-element A scales (B scale 1.0), so no dequantisation pass
// exists.  Register images (measured on MI355X; the tests pin them through
// the results): for 8-bit operands lane (r, g) = (l % 16, l / 16) holds row r,
// k = 16g..16g+15 in its first 16 bytes and 64+16g..64+16g+15 in its last 16;
// for FP4 it holds k = 32g..32g+31 as 32 nibbles (even k low) in its first 16
// bytes; its scale applies to k = 32g..32g+31 of row r; the accumulator holds
// rows 4g..4g+3 of column l % 16.
//
// Epilogue per tile: each lane gates and weights its four heads
// (max(acc, 0) * w, one v_max + one v_fmac each), sums them over the head
// tiles, and the four lane groups are summed with row-swapping permutes; the
// key's scale multiplies the head sum once.  Since k_scale > 0,
// ReLU(x * s) * w = ReLU(x) * w * s exactly; only the summation order differs
// from the reference's.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kIdxDim = 128;        // index head dim: one MFMA K
constexpr int kThreadsM = 256;      // 4 waves
constexpr int kChunk = 64;          // keys per LDS chunk of the dense kernel (128 and 256 measured slower)
constexpr int kKeyPitch = 144;      // LDS bytes per key row (128 + 16)
constexpr int kOneQueryHeads = 128;  // from this many heads a wave holds one query, not two

__device__ __forceinline__ v8i_t fp8_operand(const uint8_t* row, int g) {
    const uint4 lo = *reinterpret_cast<const uint4*>(row + 16 * g);
    const uint4 hi = *reinterpret_cast<const uint4*>(row + 64 + 16 * g);
    const v8i_t v = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return v;
}

__device__ __forceinline__ v8i_t fp4_operand(const uint8_t* row, int g) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + 16 * g);
    const v8i_t r = {(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
    return r;
}

// max(x, 0) as one integer max on the bits (negative values and -0 have the
// sign bit set); fmaxf would add a NaN-quieting canonicalisation
__device__ __forceinline__ float relu(float x) {
    return __int_as_float(max(__float_as_int(x), 0));
}

template <bool FP4>
__device__ __forceinline__ v4f_t qk_tile(v8i_t a, v8i_t b, int scale_a) {
    const v4f_t z = {0.f, 0.f, 0.f, 0.f};
    if constexpr (FP4)
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 4, 0, 0, scale_a, 0, 127);
    else
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

// One query's q image (HT head tiles), weights and MXFP4 scale bytes in registers.
template <bool FP4, int HT>
struct QueryRegs {
    v8i_t q[HT];
    float w[HT][4];
    int sa[HT];

    __device__ __forceinline__ void load(const uint8_t* q_row, int64_t q_sh, const int32_t* qs_row, int64_t qs_sh,
                                         const float* w_row, int64_t w_sh, int c, int g) {
#pragma unroll
        for (int t = 0; t < HT; ++t) {
            const uint8_t* hrow = q_row + (int64_t)(16 * t + c) * q_sh;
            q[t] = FP4 ? fp4_operand(hrow, g) : fp8_operand(hrow, g);
            sa[t] = FP4 ? (int)(((uint32_t)qs_row[(int64_t)(16 * t + c) * qs_sh] >> (8 * g)) & 0xffu) : 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[t][i] = w_row[(int64_t)(16 * t + 4 * g + i) * w_sh];
        }
    }

    // This lane group's share (its 4 rows of every head tile) of
    // sum_h max(q_h . k, 0) * w_h for the lane's key column; every head tile's
    // MFMA is issued before the first is gated.
    __device__ __forceinline__ float gated_part(v8i_t b) const {
        v4f_t acc[HT];
#pragma unroll
        for (int t = 0; t < HT; ++t)
            acc[t] = qk_tile<FP4>(q[t], b, sa[t]);
        float part = 0.f;
#pragma unroll
        for (int t = 0; t < HT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                part = fmaf(relu(acc[t][i]), w[t][i], part);
        return part;
    }

    __device__ __forceinline__ float gated_sum(v8i_t b) const { return group4_sum(gated_part(b)); }
};

// Four key tiles' lane-group shares p[kt] -> lane (c, g) gets the head sum of
// key tile g, column c (key 16 g + c of the 64): a reduce-scatter over the four
// lane groups in two permute steps (v_permlane32_swap pairs tiles 0/2 and 1/3
// across lane groups g, g ^ 2; v_permlane16_swap then pairs g, g ^ 1), six
// VALU operations for the four tiles.  Every total is
// (p[g0] + p[g2]) + (p[g1] + p[g3]).
__device__ __forceinline__ float reduce_scatter4(const float (&p)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[0]), __float_as_uint(p[2]), false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[1]), __float_as_uint(p[3]), false, false);
    const float s02 = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const float s13 = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(s02), __float_as_uint(s13), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

struct MqaArgs {
    const uint8_t* q;
    const int32_t* q_scale;
    const uint8_t* k;
    const float* k_scale;
    const float* w;
    const int32_t* ks;
    const int32_t* ke;
    float* out;
    int64_t q_sm, q_sh;    // bytes
    int64_t qs_sm, qs_sh;  // int32 elements
    int64_t k_sn;          // bytes
    int64_t w_sm, w_sh;    // float elements
    int64_t o_sm;          // float elements
    int32_t M, N;
    int32_t keys_per_block;  // multiple of kChunk
    int32_t clean;
};

// Dense logits.  A workgroup covers WQ * QW queries x keys_per_block keys: its
// four waves are WQ query groups (QW queries each) x (4 / WQ) key-tile slices,
// and every 64-key chunk of K is staged once in LDS (double-buffered, the next
// chunk's loads in flight under the current chunk's MFMAs) for all of them.
// (Staging the workgroup's whole key range at once, with no barrier between
// chunks, measured 14 % slower.)
template <bool FP4, int HT, int QW, int WQ>
__global__ void __launch_bounds__(kThreadsM, 2)
mqa_logits_kernel(MqaArgs a) {
    constexpr int KTW = 4 / (4 / WQ);  // key tiles per wave per chunk
    __shared__ __align__(16) uint8_t kbuf[2][kChunk * kKeyPitch];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int wq = wave % WQ, wk = wave / WQ;
    const int m_first = blockIdx.x * (WQ * QW);
    const int n_begin = blockIdx.y * a.keys_per_block;
    const int n_end = min(a.N, n_begin + a.keys_per_block);

    // the workgroup's key window: the union of its queries' [ks, ke) when
    // cleaning (chunks outside it are only written with -inf)
    int lo = n_begin, hi = n_end;
    int my_ks[QW], my_ke[QW];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        my_ks[j] = 0;
        my_ke[j] = a.N;
    }
    if (a.clean) {
        const int mq = m_first + lane;
        const bool v = lane < WQ * QW && mq < a.M;
        const int qks = v ? a.ks[mq] : 0x7fffffff;
        const int qke = v ? a.ke[mq] : 0;
        int wlo = 0x7fffffff, whi = 0;
        for (int i = 0; i < WQ * QW; ++i) {
            wlo = min(wlo, __builtin_amdgcn_readlane(qks, i));
            whi = max(whi, __builtin_amdgcn_readlane(qke, i));
        }
        lo = max(lo, wlo);
        hi = min(hi, whi);
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            my_ks[j] = __builtin_amdgcn_readlane(qks, wq * QW + j);
            my_ke[j] = __builtin_amdgcn_readlane(qke, wq * QW + j);
        }
    }
    // whole chunks [c_lo, c_hi) hold every computed key
    const int c_lo = lo < hi ? n_begin + (lo - n_begin) / kChunk * kChunk : n_end;
    const int c_hi = lo < hi ? min(n_end, n_begin + (hi - n_begin + kChunk - 1) / kChunk * kChunk) : n_end;

    // -inf on [n_begin, c_lo) and [c_hi, n_end) (cleaning only): lane group g
    // < QW of each wave its query's row, the wave's key slice
    if (a.clean && g < QW && m_first + wq * QW + g < a.M) {
        float* orow = a.out + (int64_t)(m_first + wq * QW + g) * a.o_sm;
        for (int n = n_begin + 16 * wk + c; n < c_lo; n += 16 * (4 / WQ))
            orow[n] = -__builtin_inff();
        for (int n = c_hi + 16 * wk + c; n < n_end; n += 16 * (4 / WQ))
            orow[n] = -__builtin_inff();
    }
    if (c_lo >= c_hi)
        return;  // workgroup-uniform

    QueryRegs<FP4, HT> qr[QW];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int m = min(m_first + wq * QW + j, a.M - 1);
        qr[j].load(a.q + (int64_t)m * a.q_sm, a.q_sh, FP4 ? a.q_scale + (int64_t)m * a.qs_sm : nullptr, a.qs_sh,
                   a.w + (int64_t)m * a.w_sm, a.w_sh, c, g);
    }

    // chunk staging: thread t moves 16-byte pieces (t % 8) of keys t / 8 and t / 8 + 32
    const int lk = threadIdx.x >> 3, lp = threadIdx.x & 7;
    auto fetch = [&](int n0, uint4& r0, uint4& r1) {
        const int k0 = min(n0 + lk, a.N - 1), k1 = min(n0 + lk + 32, a.N - 1);
        // plain loads: every workgroup of the column reads the same keys (L2 reuse)
        r0 = *reinterpret_cast<const uint4*>(a.k + (int64_t)k0 * a.k_sn + 16 * lp);
        r1 = *reinterpret_cast<const uint4*>(a.k + (int64_t)k1 * a.k_sn + 16 * lp);
    };
    auto stage = [&](int b, uint4 r0, uint4 r1) {
        *reinterpret_cast<uint4*>(&kbuf[b][lk * kKeyPitch + 16 * lp]) = r0;
        *reinterpret_cast<uint4*>(&kbuf[b][(lk + 32) * kKeyPitch + 16 * lp]) = r1;
    };
    uint4 r0, r1;
    fetch(c_lo, r0, r1);
    stage(0, r0, r1);
    __syncthreads();
    const int nchunks = (c_hi - c_lo + kChunk - 1) / kChunk;
    for (int ci = 0; ci < nchunks; ++ci) {
        const int n0 = c_lo + ci * kChunk;
        const bool more = ci + 1 < nchunks;
        if (more)
            fetch(n0 + kChunk, r0, r1);
        const uint8_t* kb = kbuf[ci & 1];
        const int n0g = n0;
        if constexpr (KTW == 4) {
            // all four key tiles per query, then one reduce-scatter: lane l
            // holds key n0 + l, stored as one 256-byte row segment per query
            const int n = n0g + lane;
            const float ksc = a.k_scale[min(n, a.N - 1)];
            float p[QW][4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const v8i_t b = fp8_operand(kb + (16 * kt + c) * kKeyPitch, g);
#pragma unroll
                for (int j = 0; j < QW; ++j)
                    p[j][kt] = qr[j].gated_part(b);
            }
#pragma unroll
            for (int j = 0; j < QW; ++j) {
                const float v = reduce_scatter4(p[j]) * ksc;
                const int m = m_first + wq * QW + j;
                const bool outside = n < my_ks[j] || n >= my_ke[j];  // [0, N) unless cleaning
                if (m < a.M && n < n_end)
                    a.out[(int64_t)m * a.o_sm + n] = outside ? -__builtin_inff() : v;
            }
        } else {
            float ksc[KTW];
#pragma unroll
            for (int kt = 0; kt < KTW; ++kt)
                ksc[kt] = a.k_scale[min(n0g + 16 * (wk * KTW + kt) + c, a.N - 1)];
#pragma unroll
            for (int kt = 0; kt < KTW; ++kt) {
                const int tile = wk * KTW + kt;
                const v8i_t b = fp8_operand(kb + (16 * tile + c) * kKeyPitch, g);
                const int n = n0g + 16 * tile + c;
#pragma unroll
                for (int j = 0; j < QW; ++j) {
                    const float v = qr[j].gated_sum(b) * ksc[kt];
                    const int m = m_first + wq * QW + j;
                    const bool outside = n < my_ks[j] || n >= my_ke[j];
                    if (g == j && m < a.M && n < n_end)
                        a.out[(int64_t)m * a.o_sm + n] = outside ? -__builtin_inff() : v;
                }
            }
        }
        if (more)
            stage((ci + 1) & 1, r0, r1);
        __syncthreads();
    }
}

struct PagedArgs {
    const uint8_t* q;
    const int32_t* q_scale;
    const uint8_t* kv;
    const float* w;
    const int32_t* ctx;
    const int32_t* bt;
    float* out;
    int64_t q_sr, q_sh;    // bytes
    int64_t qs_sr, qs_sh;  // int32 elements
    int64_t kv_bs;         // bytes between cache blocks
    int64_t w_sr, w_sh;    // float elements
    int64_t bt_sr;         // int32 elements
    int64_t o_sr;          // float elements
    int32_t rows, bt_row_div, ctx_row_div;
    int32_t num_blocks, block_size, max_blocks;
    int32_t max_model_len, keys_per_block;  // keys_per_block: multiple of 1024
    int32_t vec_fill;                       // output rows 16-byte aligned, max_model_len % 4 == 0
    float fill;
};

// Paged logits: one workgroup per (row, keys_per_block positions); each wave
// takes 64 consecutive positions at a time: all four key tiles' cache loads
// are issued before the first tile is multiplied.
template <bool FP4, int HT>
__global__ void __launch_bounds__(kThreadsM, 2)
paged_mqa_logits_kernel(PagedArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int row = blockIdx.y;
    const int n_begin = blockIdx.x * a.keys_per_block;
    const int n_end = min(a.max_model_len, n_begin + a.keys_per_block);
    const int ctx = min(max(a.ctx[row / a.ctx_row_div], 0), a.max_model_len);
    float* out = a.out + (int64_t)row * a.o_sr;
    if (n_begin >= ctx) {
        if (a.vec_fill) {  // rows 16-byte aligned: one float4 per thread per 1024 positions
            const uint32_t fb = __float_as_uint(a.fill);
            for (int n = n_begin + 4 * threadIdx.x; n < n_end; n += 4 * kThreadsM)
                store16(out + n, make_uint4(fb, fb, fb, fb));
        } else {
            for (int n = n_begin + threadIdx.x; n < n_end; n += kThreadsM)
                out[n] = a.fill;
        }
        return;
    }
    QueryRegs<FP4, HT> qr;
    qr.load(a.q + (int64_t)row * a.q_sr, a.q_sh, FP4 ? a.q_scale + (int64_t)row * a.qs_sr : nullptr, a.qs_sh,
            a.w + (int64_t)row * a.w_sr, a.w_sh, c, g);
    const int32_t* bt_row = a.bt + (int64_t)(row / a.bt_row_div) * a.bt_sr;
    const int64_t scale_off = (int64_t)a.block_size * kIdxDim;
    // each wave: positions n0 .. n0 + 63 per step, the four key tiles' cache
    // loads issued before the first MFMA.  (A two-stage pipeline, the next
    // step's loads issued before the current one is multiplied, measured 1.6x
    // slower: 184 VGPRs halve the waves per SIMD.)
    for (int n0 = n_begin + 64 * wave; n0 < n_end; n0 += 256) {
        v8i_t b[4];
        float ksc[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const int n = n0 + 16 * kt + c;
            if (n < ctx) {
                const int lbn = (int)((uint32_t)n / (uint32_t)a.block_size);
                const int slot = n - lbn * a.block_size;
                // positions past the table read its last block (the table index is clamped)
                const int blk = min(max(bt_row[min(lbn, a.max_blocks - 1)], 0), a.num_blocks - 1);
                const uint8_t* base = a.kv + (int64_t)blk * a.kv_bs;
                b[kt] = fp8_operand(base + (int64_t)slot * kIdxDim, g);
                ksc[kt] = *reinterpret_cast<const float*>(base + scale_off + 4 * slot);
            } else {
                const v8i_t z = {0, 0, 0, 0, 0, 0, 0, 0};
                b[kt] = z;
                ksc[kt] = 0.f;
            }
        }
        float p[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
            p[kt] = qr.gated_part(b[kt]);
        // lane l: position n0 + l (its key tile g's scale sits in lane (c, g)'s ksc[g])
        float my_ksc = ksc[0];
#pragma unroll
        for (int kt = 1; kt < 4; ++kt)
            my_ksc = g == kt ? ksc[kt] : my_ksc;
        const float v = reduce_scatter4(p) * my_ksc;
        const int n = n0 + lane;
        if (n < n_end)
            out[n] = n < ctx ? v : a.fill;
    }
}

// Few queries: the four waves split each chunk's key tiles (one query per
// workgroup); otherwise each wave owns two queries (one from 128 heads, for
// registers) and all four key tiles.
template <bool FP4, int HT>
void launch_dense(bool small, dim3 grid, hipStream_t st, const MqaArgs& a) {
    if (small)
        hipLaunchKernelGGL((mqa_logits_kernel<FP4, HT, 1, 1>), grid, dim3(kThreadsM), 0, st, a);
    else if constexpr (16 * HT >= kOneQueryHeads)
        hipLaunchKernelGGL((mqa_logits_kernel<FP4, HT, 1, 4>), grid, dim3(kThreadsM), 0, st, a);
    else
        hipLaunchKernelGGL((mqa_logits_kernel<FP4, HT, 2, 4>), grid, dim3(kThreadsM), 0, st, a);
}

int check_h(int64_t h) {
    if (h != 16 && h != 32 && h != 64 && h != 128)
        return fail(FGV_E_BAD_SHAPE, "num_heads must be 16, 32, 64 or 128");
    return FGV_OK;
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_fp8_fp4_mqa_logits(
    const void* q, int64_t q_stride_m, int64_t q_stride_h, const int32_t* q_scale, int64_t q_scale_stride_m,
    int64_t q_scale_stride_h, const void* k, int64_t k_stride_n, const float* k_scale, const float* weights,
    int64_t w_stride_m, int64_t w_stride_h, const int32_t* cu_seqlen_ks, const int32_t* cu_seqlen_ke,
    float* logits, int64_t logits_stride_m, int64_t M, int64_t N, int64_t num_heads, int64_t head_dim,
    int clean_logits, void* stream) {
    using namespace fgv;
    int rc = check_h(num_heads);
    if (rc)
        return rc;
    if (head_dim != kIdxDim)
        return fail(FGV_E_BAD_SHAPE, "head_dim must be 128");
    if (M < 0 || N < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (M == 0 || N == 0)
        return FGV_OK;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL - 4096)
        return fail(FGV_E_TOO_LARGE, "M and N must fit in int32");
    if (!q || !k || !k_scale || !weights || !logits || (clean_logits && (!cu_seqlen_ks || !cu_seqlen_ke)))
        return fail(FGV_E_NULL_POINTER, "null q, k, k_scale, weights, logits or ks/ke");
    if (!aligned(q, 16) || q_stride_m % 16 || q_stride_h % 16 || !aligned(k, 16) || k_stride_n % 16)
        return fail(FGV_E_MISALIGNED, "q and k rows must be 16-byte aligned (strides multiples of 16 bytes)");
    MqaArgs a;
    a.q = static_cast<const uint8_t*>(q);
    a.q_scale = q_scale;
    a.k = static_cast<const uint8_t*>(k);
    a.k_scale = k_scale;
    a.w = weights;
    a.ks = cu_seqlen_ks;
    a.ke = cu_seqlen_ke;
    a.out = logits;
    a.q_sm = q_stride_m;
    a.q_sh = q_stride_h;
    a.qs_sm = q_scale_stride_m;
    a.qs_sh = q_scale_stride_h;
    a.k_sn = k_stride_n;
    a.w_sm = w_stride_m;
    a.w_sh = w_stride_h;
    a.o_sm = logits_stride_m;
    a.M = (int32_t)M;
    a.N = (int32_t)N;
    a.clean = clean_logits != 0;
    const bool fp4 = q_scale != nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool small = M < 8;
    const int64_t qw = num_heads >= kOneQueryHeads ? 1 : 2;
    const int64_t qpb = small ? 1 : 4 * qw;
    const int64_t wg_m = (M + qpb - 1) / qpb;
    const int64_t chunks = (N + kChunk - 1) / kChunk;
    const int64_t wg_n = std::min<int64_t>(chunks, std::max<int64_t>(1, (2048 + wg_m - 1) / wg_m));
    a.keys_per_block = (int32_t)(((chunks + wg_n - 1) / wg_n) * kChunk);
    const dim3 grid((uint32_t)wg_m, (uint32_t)((N + a.keys_per_block - 1) / a.keys_per_block));
    if (grid.x > 0x7fffffffu || grid.y > 65535u)
        return fail(FGV_E_TOO_LARGE, "grid too large");
    switch (num_heads) {
        case 16: fp4 ? launch_dense<true, 1>(small, grid, st, a) : launch_dense<false, 1>(small, grid, st, a); break;
        case 32: fp4 ? launch_dense<true, 2>(small, grid, st, a) : launch_dense<false, 2>(small, grid, st, a); break;
        case 64: fp4 ? launch_dense<true, 4>(small, grid, st, a) : launch_dense<false, 4>(small, grid, st, a); break;
        default: fp4 ? launch_dense<true, 8>(small, grid, st, a) : launch_dense<false, 8>(small, grid, st, a); break;
    }
#undef FGV_MQA_LAUNCH
    return launch_status();
}

extern "C" int fgv_fp8_fp4_paged_mqa_logits(
    const void* q, int64_t q_stride_row, int64_t q_stride_h, const int32_t* q_scale, int64_t q_scale_stride_row,
    int64_t q_scale_stride_h, const void* kv_cache, int64_t cache_block_stride, int64_t num_blocks,
    int64_t block_size, int64_t head_dim, const float* weights, int64_t w_stride_row, int64_t w_stride_h,
    const int32_t* context_lens, int64_t rows_per_context_len, const int32_t* block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq, int64_t rows_per_table_row, float* logits,
    int64_t logits_stride_row,
    int64_t rows, int64_t num_heads, int64_t max_model_len, int clean_logits, void* stream) {
    using namespace fgv;
    int rc = check_h(num_heads);
    if (rc)
        return rc;
    if (head_dim != kIdxDim)
        return fail(FGV_E_BAD_SHAPE, "head_dim must be 128");
    if (rows < 0 || max_model_len < 0 || num_blocks < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (rows == 0 || max_model_len == 0)
        return FGV_OK;
    if (block_size <= 0 || num_blocks == 0 || max_blocks_per_seq <= 0 || rows_per_table_row <= 0 ||
        rows_per_context_len <= 0)
        return fail(FGV_E_BAD_SHAPE, "block_size, num_blocks, max_blocks and rows per table / length must be positive");
    if (rows > 65535 || max_model_len > 0x7fffffffLL - 4096 || block_size > 0x7fffffffLL ||
        num_blocks > 0x7fffffffLL || max_blocks_per_seq > 0x7fffffffLL || rows_per_table_row > 65535 ||
        rows_per_context_len > 65535)
        return fail(FGV_E_TOO_LARGE, "at most 65535 rows; sizes must fit in int32");
    if (!q || !kv_cache || !weights || !context_lens || !block_tables || !logits)
        return fail(FGV_E_NULL_POINTER, "null q, kv_cache, weights, context_lens, block_tables or logits");
    if (cache_block_stride < block_size * (kIdxDim + 4))
        return fail(FGV_E_BAD_STRIDE, "cache block stride is below block_size * 132");
    if (!aligned(q, 16) || q_stride_row % 16 || q_stride_h % 16 || !aligned(kv_cache, 16) ||
        cache_block_stride % 16)
        return fail(FGV_E_MISALIGNED, "q rows and cache blocks must be 16-byte aligned");
    PagedArgs a;
    a.q = static_cast<const uint8_t*>(q);
    a.q_scale = q_scale;
    a.kv = static_cast<const uint8_t*>(kv_cache);
    a.w = weights;
    a.ctx = context_lens;
    a.bt = block_tables;
    a.out = logits;
    a.q_sr = q_stride_row;
    a.q_sh = q_stride_h;
    a.qs_sr = q_scale_stride_row;
    a.qs_sh = q_scale_stride_h;
    a.kv_bs = cache_block_stride;
    a.w_sr = w_stride_row;
    a.w_sh = w_stride_h;
    a.bt_sr = block_table_stride;
    a.o_sr = logits_stride_row;
    a.rows = (int32_t)rows;
    a.bt_row_div = (int32_t)rows_per_table_row;
    a.ctx_row_div = (int32_t)rows_per_context_len;
    a.num_blocks = (int32_t)num_blocks;
    a.block_size = (int32_t)block_size;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.max_model_len = (int32_t)max_model_len;
    a.keys_per_block = 1024;
    a.vec_fill = aligned(logits, 16) && logits_stride_row % 4 == 0 && max_model_len % 4 == 0;
    a.fill = clean_logits ? -__builtin_inff() : 0.f;
    const bool fp4 = q_scale != nullptr;
    const dim3 grid((uint32_t)((max_model_len + a.keys_per_block - 1) / a.keys_per_block), (uint32_t)rows);
    hipStream_t st = static_cast<hipStream_t>(stream);
#define FGV_PAGED_LAUNCH(FP4, HT) \
    hipLaunchKernelGGL((paged_mqa_logits_kernel<FP4, HT>), grid, dim3(kThreadsM), 0, st, a)
#define FGV_PAGED_HEADS(HT)             \
    do {                                \
        if (fp4)                        \
            FGV_PAGED_LAUNCH(true, HT);  \
        else                            \
            FGV_PAGED_LAUNCH(false, HT); \
    } while (0)
    switch (num_heads) {
        case 16: FGV_PAGED_HEADS(1); break;
        case 32: FGV_PAGED_HEADS(2); break;
        case 64: FGV_PAGED_HEADS(4); break;
        default: FGV_PAGED_HEADS(8); break;
    }
#undef FGV_PAGED_HEADS
#undef FGV_PAGED_LAUNCH
    return launch_status();
}
