// gfx950 kernel for DeepSeek-V4's sparse-indexer q pre-processing: GPT-J RoPE
// on the last 64 dims of each index head, then FP8 e4m3 quant with one UE8M0
// scale per (token, head) folded into the head weights, or MXFP4 (E2M1 with
// one UE8M0 scale per 32 elements).
//
// Reference semantics: src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py
//   FP8   kernel :64-167   MXFP4 kernel :170-282   wrapper :285-410
// and its test tests/test_fused_indexer_q_rope_quant.py:51-110 (exact codes,
// scales and weights).  The rotated values are rounded to bf16 before the
// amax, as the reference does.
//
// Layout: one (token, head) row per 16-lane DPP row (fgv_device.h); lane l16
// owns elements (l16 + 16*p)*8 .. +8 for p < kPieces (head_dim = 128*kPieces),
// so the 64 rope elements are lanes 8..15 of the last piece, an FP8 row amax
// is one 16-lane DPP max and an MXFP4 32-element block is one lane quad.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 16;

struct IndexerArgs {
    const int64_t* positions;
    const uint16_t* q;
    const void* cos_sin;
    const void* weights;
    float* weights_out;
    uint8_t* q_out;
    uint8_t* scale_out;
    int64_t q_st, q_sh;
    int64_t cs_stride, max_pos;
    int64_t w_st, wo_st;
    int64_t qo_st, qo_sh;
    int64_t so_st, so_sh;
    uint32_t num_rows, num_heads;
    float softmax_scale, head_scale;
    int w_f32, fp4;
};

// Two consecutive cos (or sin) values at element offset `off` (even).
__device__ __forceinline__ float2 load_cs2(const void* base, int64_t off, bool bf16) {
    if (bf16) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(base) + off);
        return make_float2(bf16_lo(v), bf16_hi(v));
    }
    return *reinterpret_cast<const float2*>(static_cast<const float*>(base) + off);
}

// The first of the two RoPE pairs this lane rotates (see rope_words): pairs
// 4(l-8) and 4(l-8)+1 on lanes l = 8..15, pairs 4l+2 and 4l+3 on lanes l < 8.
__device__ __forceinline__ int rope_pair0(int lane16) {
    return lane16 >= 8 ? 4 * (lane16 - 8) : 4 * lane16 + 2;
}

// MXFP4 block exponent k = ceil(log2(max(amax, 6*2^-126) / 6)) from the
// binary32 fields of a = m * 2^E: 6 = 1.5 * 2^2, so k = E - 2 + (m > 1.5).
// Exact for every bf16 amax (amax/6 never rounds across a power of two).
__device__ __forceinline__ int mxfp4_exponent(uint32_t amax_bits) {
    const uint32_t kFloor = 0x01C00000u;  // 6 * 2^-126 = 1.5 * 2^-124
    const uint32_t a = amax_bits > kFloor ? amax_bits : kFloor;
    return (int)(a >> 23) - 127 - 2 + ((a & 0x7fffffu) > 0x400000u ? 1 : 0);
}

// FP8 row exponent k = ceil(log2(max(amax, 1e-4) / 448)) (see the main op).
__device__ __forceinline__ int fp8_row_exponent(uint32_t amax_bits) {
    const uint32_t kFloor = 0x38D1B717u;  // 1e-4f
    const uint32_t a = amax_bits > kFloor ? amax_bits : kFloor;
    return (int)(a >> 23) - 127 - 8 + ((a & 0x7fffffu) > 0x600000u ? 1 : 0);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// GPT-J rotation of one (even, odd) pair held as a packed bf16 word:
// x_even*cos - x_odd*sin, x_odd*cos + x_even*sin, each product and sum rounded
// to binary32 and the result to bf16 (reference kernel :113-123).
__device__ __forceinline__ uint32_t rotate_pair(uint32_t word, float c, float s) {
    const float e = bf16_lo(word), o = bf16_hi(word);
    const float ec = e * c, os = o * s, oc = o * c, es = e * s;
    return pack_bf16x2(ec - os, oc + es);
}

// One row's values stay packed bf16 words (element 2i in the low half of word
// i).  The RoPE half is the last piece of lanes 8..15 (word i of lane l: pair
// 4(l-8)+i).  All 16 lanes rotate two pairs each: lane l >= 8 its words 0 and
// 1; lane j < 8 words 2 and 3 of lane j+8, fetched and returned with a row
// rotation by 8.  c and s hold the lane's two pairs' cos and sin (rope_pair0).
template <int kPieces>
__device__ __forceinline__ void rope_words(const uint4 (&v)[kPieces], float2 c, float2 s, int lane16,
                                           uint32_t (&w)[kPieces][4]) {
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
        w[p][0] = v[p].x; w[p][1] = v[p].y; w[p][2] = v[p].z; w[p][3] = v[p].w;
    }
    uint32_t* r = w[kPieces - 1];
    const bool rope_lane = lane16 >= 8;
    const uint32_t f2 = dpp_u32<kDppRowRor8>(r[2]), f3 = dpp_u32<kDppRowRor8>(r[3]);
    const uint32_t o0 = rotate_pair(rope_lane ? r[0] : f2, c.x, s.x);
    const uint32_t o1 = rotate_pair(rope_lane ? r[1] : f3, c.y, s.y);
    const uint32_t b0 = dpp_u32<kDppRowRor8>(o0), b1 = dpp_u32<kDppRowRor8>(o1);
    if (rope_lane) {
        r[0] = o0;
        r[1] = o1;
        r[2] = b0;
        r[3] = b1;
    }
}

// Binary32 bits of the largest |value| among `n` packed bf16 words: the bf16
// magnitudes compare as integers (two per v_pk_max_u16) and, shifted up 16
// bits, are the binary32 patterns of the same values.
template <int n>
__device__ __forceinline__ uint32_t absmax_bits(const uint32_t* w) {
    u16x2_t m = {0, 0};
#pragma unroll
    for (int i = 0; i < n; ++i)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, w[i] & 0x7fff7fffu));
    return (uint32_t)(m.x > m.y ? m.x : m.y) << 16;
}

// Two bf16 pairs -> four e4m3 codes, each value divided by `scale` (2^k) inside
// v_cvt_scalef32_pk_fp8_bf16.  For every bf16 value and every k the row
// exponent takes (-22..120) with |x / 2^k| <= 448, this gives the same code as
// e4m3(med3(f32(x) * 2^-k, -448, 448)) (checked exhaustively on gfx950), and
// k makes every value of the row that small.
__device__ __forceinline__ uint32_t fp8x4_scaled(uint32_t a, uint32_t b, float scale) {
    short2_t r = {0, 0};
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, a), scale, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, b), scale, true);
    return __builtin_bit_cast(uint32_t, r);
}

// FP8: the row's UE8M0 exponent k (one 16-lane max) and each piece's eight
// e4m3 codes as two words.
template <int kPieces>
__device__ __forceinline__ int fp8_codes(const uint32_t (&w)[kPieces][4], uint32_t (&lo)[kPieces],
                                         uint32_t (&hi)[kPieces]) {
    uint32_t m = absmax_bits<4 * kPieces>(&w[0][0]);
    m = row16_max(m);
    const int k = fp8_row_exponent(m);
    const float scale = __uint_as_float((uint32_t)(k + 127) << 23);
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
        lo[p] = fp8x4_scaled(w[p][0], w[p][1], scale);
        hi[p] = fp8x4_scaled(w[p][2], w[p][3], scale);
    }
    return k;
}

// The FP8 weight ((w * 2^k) * softmax_scale) * head_scale.
__device__ __forceinline__ float fp8_weight(float w_in, int k, const IndexerArgs& a) {
    const float q_scale = __uint_as_float((uint32_t)(k + 127) << 23);
    float w = w_in * q_scale;
    w = w * a.softmax_scale;
    return w * a.head_scale;
}

// MXFP4: 32-element blocks are lane quads (4 lanes x 8 elements).  Per piece,
// this lane's eight E2M1 nibbles, each value divided by the block's 2^k inside
// v_cvt_scalef32_pk_fp4_bf16 (the same nibble as converting f32(x) * 2^-k at
// scale 1, for every bf16 value and every k -124..125: checked exhaustively
// on gfx950), and its quad's UE8M0 byte k + 127.
template <int kPieces>
__device__ __forceinline__ void fp4_codes(const uint32_t (&w)[kPieces][4], uint32_t (&nib)[kPieces],
                                          uint32_t (&ebyte)[kPieces]) {
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
        uint32_t m = absmax_bits<4>(w[p]);
        m = max(m, dpp_u32<kDppQuadXor1>(m));
        m = max(m, dpp_u32<kDppQuadXor2>(m));
        const int k = mxfp4_exponent(m);
        const float scale = __uint_as_float((uint32_t)(k + 127) << 23);
        uint32_t r = 0;
        r = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(r, __builtin_bit_cast(bf16x2_t, w[p][0]), scale, 0);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(r, __builtin_bit_cast(bf16x2_t, w[p][1]), scale, 1);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(r, __builtin_bit_cast(bf16x2_t, w[p][2]), scale, 2);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(r, __builtin_bit_cast(bf16x2_t, w[p][3]), scale, 3);
        nib[p] = r;
        ebyte[p] = (uint32_t)(k + 127) & 0xffu;
    }
}

// The four block bytes of a piece (lanes 0, 4, 8, 12) as one word on lane 0 of
// the row, so they leave in one 32-bit store instead of four byte stores.
__device__ __forceinline__ uint32_t exponent_word(uint32_t e) {
    return e | dpp_u32<kDppRowRor12>(e) << 8 | dpp_u32<kDppRowRor8>(e) << 16 | dpp_u32<kDppRowRor4>(e) << 24;
}

// The MXFP4 weight (w * softmax_scale) * head_scale.
__device__ __forceinline__ float fp4_weight(float w_in, const IndexerArgs& a) {
    const float w = w_in * a.softmax_scale;
    return w * a.head_scale;
}

// One (token, head) row with 64-bit addressing: rotate, quantise, store codes,
// scales and weight.
template <int kPieces>
__device__ __forceinline__ void indexer_row(const IndexerArgs& a, uint32_t t, uint32_t h,
                                            const uint4 (&v)[kPieces], float2 c, float2 s,
                                            float w_in, int lane16) {
    uint32_t xw[kPieces][4];
    rope_words<kPieces>(v, c, s, lane16, xw);
    uint8_t* qo = a.q_out + (int64_t)t * a.qo_st + (int64_t)h * a.qo_sh;
    if (!a.fp4) {
        uint32_t lo[kPieces], hi[kPieces];
        const int k = fp8_codes<kPieces>(xw, lo, hi);
#pragma unroll
        for (int p = 0; p < kPieces; ++p)
            store8(qo + (lane16 + 16 * p) * 8, lo[p], hi[p]);
        if (lane16 == 0)
            a.weights_out[(int64_t)t * a.wo_st + h] = fp8_weight(w_in, k, a);
        return;
    }
    uint8_t* so = a.scale_out + (int64_t)t * a.so_st + (int64_t)h * a.so_sh;
    uint32_t nib[kPieces], ebyte[kPieces];
    fp4_codes<kPieces>(xw, nib, ebyte);
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
        *reinterpret_cast<uint32_t*>(qo + (lane16 + 16 * p) * 4) = nib[p];
        const uint32_t word = exponent_word(ebyte[p]);
        if (lane16 == 0)
            *reinterpret_cast<uint32_t*>(so + 4 * p) = word;
    }
    if (lane16 == 0)
        a.weights_out[(int64_t)t * a.wo_st + h] = fp4_weight(w_in, a);
}

// Each 16-lane group owns kRows rows, 16 rows apart inside the block, so a
// wave's load instruction covers 4 consecutive rows and every lane keeps
// kRows * kPieces = 4 sixteen-byte loads in flight.  Index loads (position,
// weight) are issued before the q loads and the cos/sin loads after them, so
// no load waits on a later one (vmcnt counts in issue order).  kOneToken: all
// rows of the block share one token and its position is a scalar load.
template <int kPieces, bool kCsBf16, bool kOneToken, int kBlock = kThreads>
__global__ void __launch_bounds__(kBlock)
indexer_q_rope_quant_kernel(IndexerArgs a) {
    constexpr int kRows = 4 / kPieces;
    constexpr int kGroups = kBlock / 16;  // 16-lane groups per block
    const int lane16 = threadIdx.x & 15;
    const uint32_t row0 = blockIdx.x * (kGroups * kRows);
    uint32_t tt[kRows], hh[kRows];
    bool valid[kRows];
    int64_t praw[kRows];
    uint32_t w_bits[kRows];
    int64_t pos_block = 0;
    if (kOneToken)
        pos_block = a.positions[row0 / a.num_heads];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
        const uint32_t row = row0 + rr * kGroups + (threadIdx.x >> 4);
        valid[rr] = row < a.num_rows;
        tt[rr] = (valid[rr] ? row : row0) / a.num_heads;
        hh[rr] = (valid[rr] ? row : row0) - tt[rr] * a.num_heads;
        praw[rr] = kOneToken ? pos_block : a.positions[tt[rr]];
        const int64_t wi = (int64_t)tt[rr] * a.w_st + hh[rr];
        // raw bits only: converting here would wait on the load inside the branch
        w_bits[rr] = a.w_f32 ? static_cast<const uint32_t*>(a.weights)[wi]
                             : (uint32_t) static_cast<const uint16_t*>(a.weights)[wi];
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 v[kRows][kPieces];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
        const uint16_t* x = a.q + (int64_t)tt[rr] * a.q_st + (int64_t)hh[rr] * a.q_sh;
#pragma unroll
        for (int p = 0; p < kPieces; ++p)
            v[rr][p] = valid[rr] ? load16(x + (lane16 + 16 * p) * 8) : make_uint4(0, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    float2 c[kRows], s[kRows];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
        if (kOneToken && rr > 0) {  // one token: the first row's cos/sin serve every row
            c[rr] = c[0];
            s[rr] = s[0];
        } else {
            const int64_t pos = clamp_position(praw[rr], a.max_pos);
            const int64_t off = pos * a.cs_stride + rope_pair0(lane16);
            c[rr] = load_cs2(a.cos_sin, off, kCsBf16);
            s[rr] = load_cs2(a.cos_sin, off + kHalfRope, kCsBf16);
        }
    }
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
        const float w_in = __uint_as_float(a.w_f32 ? w_bits[rr] : w_bits[rr] << 16);
        if (valid[rr])
            indexer_row<kPieces>(a, tt[rr], hh[rr], v[rr], c[rr], s[rr], w_in, lane16);
    }
}

// One token per block (num_heads a multiple of the block's rows) and every
// per-head offset below 2^31 bytes: the token, its position and the base
// pointers of its rows are uniform (scalar registers) and each lane addresses
// its rows with 32-bit offsets.  The general kernel's per-row division by
// num_heads and 64-bit address products made it VALU-bound (about 650 VALU
// instructions per wave against ~330 here for the same math).
template <int kPieces, int kRows, bool kCsBf16>
__global__ void __launch_bounds__(kThreads)
indexer_token_kernel(IndexerArgs a) {
    // The block's per-head weights (and MXFP4 exponent words) gather in LDS and
    // leave as one contiguous run per block: from lane 0 of each row they would
    // be 16-byte pieces per store instruction, which measured ~2 us on the
    // DeepSeek-V4 shape for 2 MB of scales.
    constexpr int kBlockRows = kRowsPerBlock * kRows;
    __shared__ float w_lds[kBlockRows];
    __shared__ uint32_t s_lds[kBlockRows * kPieces];  // byte 4 (row * kPieces + p) + quad
    const int lane16 = threadIdx.x & 15;
    const uint32_t row0 = blockIdx.x * kBlockRows;
    const uint32_t t = row0 / a.num_heads;
    const uint32_t hb = row0 - t * a.num_heads;                  // the block's first head
    const uint32_t h = hb + (threadIdx.x >> 4);                  // rows h + 16 * rr
    const int64_t pos_raw = a.positions[t];
    uint32_t w_bits[kRows];
    if (a.w_f32) {
        const uint32_t* wb = static_cast<const uint32_t*>(a.weights) + (int64_t)t * a.w_st;
#pragma unroll
        for (int rr = 0; rr < kRows; ++rr)
            w_bits[rr] = wb[h + 16 * rr];
    } else {
        const uint16_t* wb = static_cast<const uint16_t*>(a.weights) + (int64_t)t * a.w_st;
#pragma unroll
        for (int rr = 0; rr < kRows; ++rr)
            w_bits[rr] = wb[h + 16 * rr];
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* qb = reinterpret_cast<const uint8_t*>(a.q + (int64_t)t * a.q_st);
    const uint32_t q_row = (uint32_t)a.q_sh * 2;  // bytes between heads
    const uint32_t q_off = h * q_row + lane16 * 16;
    uint4 v[kRows][kPieces];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr)
#pragma unroll
        for (int p = 0; p < kPieces; ++p)
            v[rr][p] = load16(qb + (q_off + rr * 16 * q_row + p * 256));
    __builtin_amdgcn_sched_barrier(0);
    const int64_t cs_off = clamp_position(pos_raw, a.max_pos) * a.cs_stride + rope_pair0(lane16);
    const float2 c = load_cs2(a.cos_sin, cs_off, kCsBf16);
    const float2 s = load_cs2(a.cos_sin, cs_off + kHalfRope, kCsBf16);
    uint8_t* qo = a.q_out + (int64_t)t * a.qo_st;
    const uint32_t qo_row = (uint32_t)a.qo_sh;
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
        const uint32_t hr = h + 16 * rr;
        const int local = (threadIdx.x >> 4) + 16 * rr;
        const float w_in = __uint_as_float(a.w_f32 ? w_bits[rr] : w_bits[rr] << 16);
        uint32_t xw[kPieces][4];
        rope_words<kPieces>(v[rr], c, s, lane16, xw);
        if (!a.fp4) {
            uint32_t lo[kPieces], hi[kPieces];
            const int k = fp8_codes<kPieces>(xw, lo, hi);
#pragma unroll
            for (int p = 0; p < kPieces; ++p)
                store8(qo + (hr * qo_row + lane16 * 8 + p * 128), lo[p], hi[p]);
            if (lane16 == 0)
                w_lds[local] = fp8_weight(w_in, k, a);
        } else {
            uint32_t nib[kPieces], ebyte[kPieces];
            fp4_codes<kPieces>(xw, nib, ebyte);
#pragma unroll
            for (int p = 0; p < kPieces; ++p)
                *reinterpret_cast<uint32_t*>(qo + (hr * qo_row + lane16 * 4 + p * 64)) = nib[p];
            if ((lane16 & 3) == 0) {
                uint8_t* sb = reinterpret_cast<uint8_t*>(s_lds);
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    sb[4 * (local * kPieces + p) + (lane16 >> 2)] = (uint8_t)ebyte[p];
            }
            if (lane16 == 0)
                w_lds[local] = fp4_weight(w_in, a);
        }
    }
    __syncthreads();
    if (threadIdx.x < kBlockRows)
        a.weights_out[(int64_t)t * a.wo_st + hb + threadIdx.x] = w_lds[threadIdx.x];
    if (a.fp4 && threadIdx.x < kBlockRows * kPieces) {
        const uint32_t r = threadIdx.x / kPieces, p = threadIdx.x % kPieces;
        uint8_t* so = a.scale_out + (int64_t)t * a.so_st;
        *reinterpret_cast<uint32_t*>(so + ((hb + r) * (uint32_t)a.so_sh + p * 4)) = s_lds[threadIdx.x];
    }
}

// Rows per 16-lane group in the one-token kernel, for head_dim 128, 256, 512.
constexpr int kTokenRows[3] = {4, 2, 1};

template <int kPieces>
void launch_token(const IndexerArgs& a, bool cs_bf16, dim3 grid, hipStream_t s) {
    constexpr int kRows = kTokenRows[kPieces == 1 ? 0 : kPieces == 2 ? 1 : 2];
    if (cs_bf16)
        hipLaunchKernelGGL((indexer_token_kernel<kPieces, kRows, true>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((indexer_token_kernel<kPieces, kRows, false>), grid, dim3(kThreads), 0, s, a);
}

template <int kPieces, int kBlock>
void launch_indexer_block(const IndexerArgs& a, bool cs_bf16, bool one_token, dim3 grid, hipStream_t s) {
    if (cs_bf16) {
        if (one_token)
            hipLaunchKernelGGL((indexer_q_rope_quant_kernel<kPieces, true, true, kBlock>), grid, dim3(kBlock), 0, s, a);
        else
            hipLaunchKernelGGL((indexer_q_rope_quant_kernel<kPieces, true, false, kBlock>), grid, dim3(kBlock), 0, s,
                               a);
    } else {
        if (one_token)
            hipLaunchKernelGGL((indexer_q_rope_quant_kernel<kPieces, false, true, kBlock>), grid, dim3(kBlock), 0, s,
                               a);
        else
            hipLaunchKernelGGL((indexer_q_rope_quant_kernel<kPieces, false, false, kBlock>), grid, dim3(kBlock), 0, s,
                               a);
    }
}

// A grid of fewer workgroups than CUs, with at least one block's worth of
// rows (the reference benchmark's 32 tokens x 8 heads make 4), runs its rows
// over 64-thread workgroups, four times as many: 3.14 -> 2.91 us (FP8) and
// 3.25 -> 3.06 us (MXFP4) there.  Fewer rows stay on one 256-thread block,
// where each 16-lane group has fewer of them (one token x 8 heads: 2.12
// against 2.20 us).
constexpr int kSmallBlock = 64;

template <int kPieces>
void launch_indexer(const IndexerArgs& a, bool cs_bf16, int64_t rows, hipStream_t s) {
    constexpr int kRows = 4 / kPieces;
    const int64_t per_block = kRowsPerBlock * kRows;
    const int64_t blocks = (rows + per_block - 1) / per_block;
    if (blocks < cu_count() && rows >= per_block) {
        constexpr int64_t kSmallRows = kSmallBlock / 16 * kRows;
        launch_indexer_block<kPieces, kSmallBlock>(a, cs_bf16, a.num_heads % kSmallRows == 0,
                                                   dim3((unsigned)((rows + kSmallRows - 1) / kSmallRows)), s);
    } else {
        launch_indexer_block<kPieces, kThreads>(a, cs_bf16, a.num_heads % per_block == 0, dim3((unsigned)blocks), s);
    }
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_fused_indexer_q_rope_quant(
    const int64_t* positions, int64_t num_tokens,
    const void* index_q, int64_t q_stride_token, int64_t q_stride_head,
    int64_t num_heads, int64_t head_dim,
    const void* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos, int cos_sin_is_bf16,
    const void* weights, int64_t weights_stride, int weights_is_fp32,
    float softmax_scale, float head_scale,
    float* weights_out, int64_t weights_out_stride,
    int use_fp4,
    void* q_out, int64_t q_out_stride_token, int64_t q_out_stride_head,
    void* scale_out, int64_t scale_out_stride_token, int64_t scale_out_stride_head,
    void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || num_heads < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    const int64_t rows = num_tokens * num_heads;
    if (rows == 0)
        return FGV_OK;
    if (rows > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "num_tokens * num_heads must be below 2^31");
    if (head_dim != 128 && head_dim != 256 && head_dim != 512)
        return fail(FGV_E_BAD_SHAPE, "head_dim must be 128, 256 or 512 (rope 64)");
    if (!positions || !index_q || !cos_sin_cache || !weights || !weights_out || !q_out ||
        (use_fp4 && !scale_out))
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (max_pos <= 0)
        return fail(FGV_E_BAD_SHAPE, "cos_sin_cache has no rows");
    if (!aligned(index_q, 16) || q_stride_token % 8 || q_stride_head % 8)
        return fail(FGV_E_MISALIGNED, "index_q must be 16-byte aligned, strides multiple of 8");
    if (!aligned(cos_sin_cache, cos_sin_is_bf16 ? 8 : 16) || cos_sin_stride % 4)
        return fail(FGV_E_MISALIGNED, "cos_sin_cache misaligned or row stride not a multiple of 4");
    if (use_fp4) {
        if (!aligned(q_out, 4) || q_out_stride_token % 4 || q_out_stride_head % 4)
            return fail(FGV_E_MISALIGNED, "packed MXFP4 output must be 4-byte aligned");
        if (!aligned(scale_out, 4) || scale_out_stride_token % 4 || scale_out_stride_head % 4)
            return fail(FGV_E_MISALIGNED, "MXFP4 scales must be 4-byte aligned, strides multiples of 4");
    } else if (!aligned(q_out, 8) || q_out_stride_token % 8 || q_out_stride_head % 8) {
        return fail(FGV_E_MISALIGNED, "FP8 output must be 8-byte aligned, strides multiple of 8");
    }

    IndexerArgs a;
    a.positions = positions;
    a.q = static_cast<const uint16_t*>(index_q);
    a.cos_sin = cos_sin_cache;
    a.weights = weights;
    a.weights_out = weights_out;
    a.q_out = static_cast<uint8_t*>(q_out);
    a.scale_out = static_cast<uint8_t*>(scale_out);
    a.q_st = q_stride_token;
    a.q_sh = q_stride_head;
    a.cs_stride = cos_sin_stride;
    a.max_pos = max_pos;
    a.w_st = weights_stride;
    a.wo_st = weights_out_stride;
    a.qo_st = q_out_stride_token;
    a.qo_sh = q_out_stride_head;
    a.so_st = scale_out_stride_token;
    a.so_sh = scale_out_stride_head;
    a.num_rows = (uint32_t)rows;
    a.num_heads = (uint32_t)num_heads;
    a.softmax_scale = softmax_scale;
    a.head_scale = head_scale;
    a.w_f32 = weights_is_fp32 ? 1 : 0;
    a.fp4 = use_fp4 ? 1 : 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the one-token kernel's 32-bit per-head offsets (bytes) must stay below 2^31
    const auto fits = [&](int64_t stride_bytes, int64_t row_bytes) {
        return stride_bytes >= 0 && (num_heads - 1) * stride_bytes + row_bytes < (1LL << 31);
    };
    const int token_rows = kRowsPerBlock * kTokenRows[head_dim == 128 ? 0 : head_dim == 256 ? 1 : 2];
    const dim3 token_grid((unsigned)(rows / token_rows));
    if (num_heads % token_rows == 0 && fits(q_stride_head * 2, head_dim * 2) &&
        fits(q_out_stride_head, use_fp4 ? head_dim / 2 : head_dim) &&
        (!use_fp4 || fits(scale_out_stride_head, head_dim / 32))) {
        if (head_dim == 128)
            launch_token<1>(a, cos_sin_is_bf16, token_grid, s);
        else if (head_dim == 256)
            launch_token<2>(a, cos_sin_is_bf16, token_grid, s);
        else
            launch_token<4>(a, cos_sin_is_bf16, token_grid, s);
        return launch_status();
    }
    if (head_dim == 128)
        launch_indexer<1>(a, cos_sin_is_bf16, rows, s);
    else if (head_dim == 256)
        launch_indexer<2>(a, cos_sin_is_bf16, rows, s);
    else
        launch_indexer<4>(a, cos_sin_is_bf16, rows, s);
    return launch_status();
}
