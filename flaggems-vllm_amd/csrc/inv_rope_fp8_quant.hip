// gfx950 kernel for the fused DeepSeek-V4 inverse RoPE + per-128 FP8 quant of
// the attention output, ahead of the grouped FP8 output projection.
//
// Reference semantics: src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:37-256
// and its torch oracle tests/test_fused_inv_rope_fp8_quant.py:150-198.  The
// rotated rope values are rounded to bf16 before the amax and the quant, as the
// torch oracle does (the Triton kernel keeps them in fp32); this makes codes
// and scales equal to the oracle's bit for bit.
//
// Workgroups of 256 threads own 16 (token, head) rows: 16 consecutive tokens
// of one head.  Each row is one 16-lane DPP row holding four 128-element
// chunks, one per 16-byte piece k (see fgv_device.h), so a chunk's amax is one
// 16-lane DPP max.  One extra workgroup zeroes the scales of the padding
// tokens T..Tpad-1.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kTokensPerBlock = kThreads / 16;

struct InvRopeArgs {
    const uint16_t* o;
    const int64_t* positions;
    const float* cos_sin;
    uint8_t* fp8;
    void* scale;
    int64_t o_st, o_sh;
    int64_t cs_stride, max_pos;
    int64_t fp8_sg, fp8_st;
    int64_t sc_sg, sc_sk;
    uint32_t num_heads, heads_per_group;
    uint32_t num_tokens, padded_tokens, n_groups;
    uint32_t row_blocks;
    float eps;
    int tma;
    // geometry (inv_rope_fp8_quant_any_kernel; the DeepSeek-V4 kernel has
    // head_dim 512, rope 64 from 448, four chunks of 128)
    uint32_t head_dim, rope_dim, rope_start, chunks;
    uint32_t pieces;           // 16-byte pieces per head row: head_dim / 8, a power of two <= 64
    uint32_t seg;              // pieces per chunk: quant_group_size / 8
};

__device__ __forceinline__ void unpack8(uint4 v, float (&x)[8]) {
    x[0] = bf16_lo(v.x); x[1] = bf16_hi(v.x);
    x[2] = bf16_lo(v.y); x[3] = bf16_hi(v.y);
    x[4] = bf16_lo(v.z); x[5] = bf16_hi(v.z);
    x[6] = bf16_lo(v.w); x[7] = bf16_hi(v.w);
}

// Inverse GPT-J rotation of four pairs, separately rounded binary32, result
// rounded to bf16 and widened back (the values the quantiser sees).
__device__ __forceinline__ void inv_rope_piece(float (&x)[8], float4 c, float4 s) {
    const float cc[4] = {c.x, c.y, c.z, c.w};
    const float ss[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float e = x[2 * i], o = x[2 * i + 1];
        float ec = e * cc[i], os = o * ss[i];
        float oc = o * cc[i], es = e * ss[i];
        uint32_t w = pack_bf16x2(ec + os, oc - es);
        x[2 * i] = bf16_lo(w);
        x[2 * i + 1] = bf16_hi(w);
    }
}

// Correctly rounded x / s (s > 0, normal) from y = RN(1/s), which is one IEEE
// division per 128-element chunk instead of one per element.  q0 = RN(x*y) is
// within one ulp of x/s, the negated remainder rn = s*q0 - x is exact in one
// fma, and RN(q0 - rn*y) = RN(x/s) by Markstein's theorem (P. Markstein, IBM
// J. Res. Dev. 34(1), 1990; J.-M. Muller et al., Handbook of Floating-Point
// Arithmetic, 2nd ed., section 4.7).  The remainder stays exact for every
// quotient large enough to reach a non-zero e4m3 code (|x/s| >= 2^-10 keeps
// it far above the binary32 underflow threshold).  For x = +-0 the two fmas
// add zeros of opposite / equal sign so the quotient keeps x's sign, which
// decides between codes 0x00 and 0x80.
__device__ __forceinline__ float div_by_scale(float x, float s, float y) {
    const float q0 = x * y;
    const float rn = __builtin_fmaf(s, q0, -x);
    return __builtin_fmaf(-rn, y, q0);
}

// One workgroup owns kTokensPerBlock consecutive tokens of one head (16-lane
// DPP row r: token t0 + r), so that the scales of a chunk, token-fastest in
// the (G, K, Tpad) layout, come out as one contiguous 64-byte run: they are
// collected in LDS and written by one wave.  Position first (the cos/sin
// loads depend on it; vmcnt counts in issue order), then the row, then
// cos/sin.
__device__ void row_block(const InvRopeArgs& a, uint32_t rb, int lane16, int row_in_block) {
    __shared__ uint32_t scales_lds[4][kTokensPerBlock];
    const bool rope_lane = lane16 >= 8;
    const uint32_t head = rb % a.num_heads, t0 = (rb / a.num_heads) * kTokensPerBlock;
    const uint32_t t = t0 + row_in_block;
    const bool valid = t < a.num_tokens;
    const int64_t praw = a.positions[valid ? t : t0];
    __builtin_amdgcn_sched_barrier(0);
    uint4 v[4];
    const uint16_t* x_row = a.o + (int64_t)(valid ? t : t0) * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = load16(x_row + (lane16 + 16 * k) * 8);
    __builtin_amdgcn_sched_barrier(0);
    float4 cs_c = make_float4(0.f, 0.f, 0.f, 0.f), cs_s = cs_c;
    if (rope_lane) {
        const int64_t pos = clamp_position(praw, a.max_pos);
        const float* cs = a.cos_sin + pos * a.cs_stride + (lane16 - 8) * 4;
        cs_c = *reinterpret_cast<const float4*>(cs);
        cs_s = *reinterpret_cast<const float4*>(cs + kHalfRope);
    }

    const float inv_max = (float)(1.0 / 448.0);
    const uint32_t eps_bits = __float_as_uint(a.eps);
    const uint32_t g = head / a.heads_per_group;
    const uint32_t hig = head - g * a.heads_per_group;
    uint8_t* out = a.fp8 + (int64_t)g * a.fp8_sg + (int64_t)t * a.fp8_st + hig * kHeadDim;
    uint32_t packed = 0;
    float my_scale = 0.0f;  // lane k (k < 4) keeps chunk k's fp32 scale
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float x[8];
        unpack8(v[k], x);
        if (k == 3 && rope_lane)
            inv_rope_piece(x, cs_c, cs_s);
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            m = max(m, __float_as_uint(x[i]) & 0x7fffffffu);
        m = row16_max(m);
        m = m > eps_bits ? m : eps_bits;  // max(amax, eps), eps > 0
        float sc = __uint_as_float(m) * inv_max;
        uint32_t lo, hi;
        if (a.tma) {
            // 2^ceil(log2(max(sc, 1e-10))) from the binary32 fields.
            uint32_t b = __float_as_uint(sc);
            b = b > 0x2EDBE6FFu ? b : 0x2EDBE6FFu;  // 1e-10f
            int e = (int)(b >> 23) - 127 + ((b & 0x7fffffu) ? 1 : 0);
            packed |= (uint32_t)(e + 127) << (8 * k);
            const float inv = exp2_neg_int(e);
            lo = pack_fp8x4(clamp_fp8(x[0] * inv), clamp_fp8(x[1] * inv),
                            clamp_fp8(x[2] * inv), clamp_fp8(x[3] * inv));
            hi = pack_fp8x4(clamp_fp8(x[4] * inv), clamp_fp8(x[5] * inv),
                            clamp_fp8(x[6] * inv), clamp_fp8(x[7] * inv));
        } else {
            if (lane16 == k)
                my_scale = sc;
            const float y = 1.0f / sc;
            float qv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                qv[i] = clamp_fp8(div_by_scale(x[i], sc, y));
            lo = pack_fp8x4(qv[0], qv[1], qv[2], qv[3]);
            hi = pack_fp8x4(qv[4], qv[5], qv[6], qv[7]);
        }
        if (valid)
            store8(out + (lane16 + 16 * k) * 8, lo, hi);
    }
    if (a.tma) {
        if (lane16 == 0)
            scales_lds[0][row_in_block] = packed;
    } else if (lane16 < 4) {
        scales_lds[lane16][row_in_block] = __float_as_uint(my_scale);
    }
    __syncthreads();
    // thread 16 k + r writes chunk k's scale of token t0 + r
    const int k = threadIdx.x >> 4, r = threadIdx.x & 15;
    const bool write = t0 + r < a.num_tokens && k < (a.tma ? 1 : 4);
    if (write) {
        const int64_t off = (int64_t)g * a.sc_sg + (int64_t)(a.tma ? hig : hig * 4 + k) * a.sc_sk + t0 + r;
        static_cast<uint32_t*>(a.scale)[off] = scales_lds[k][r];
    }
}

// Zero the scales of padding tokens T..Tpad-1 (ops/fused_inv_rope_fp8_quant.py:69-88).
__device__ void pad_block(const InvRopeArgs& a) {
    const uint32_t per_group = a.tma ? a.heads_per_group : a.heads_per_group * a.chunks;
    const uint32_t npad = a.padded_tokens - a.num_tokens;
    const uint32_t total = a.n_groups * per_group * npad;
    for (uint32_t i = threadIdx.x; i < total; i += kThreads) {
        uint32_t tp = i % npad, rest = i / npad;
        uint32_t k = rest % per_group, g = rest / per_group;
        int64_t off = (int64_t)g * a.sc_sg + (int64_t)k * a.sc_sk + a.num_tokens + tp;
        static_cast<uint32_t*>(a.scale)[off] = 0u;  // 0.0f and int32 0 share bits
    }
}

__global__ void __launch_bounds__(kThreads)
inv_rope_fp8_quant_kernel(InvRopeArgs a) {
    if (blockIdx.x < a.row_blocks)
        row_block(a, blockIdx.x, threadIdx.x & 15, threadIdx.x >> 4);
    else
        pad_block(a);
}

// ---- every other geometry the reference accepts (nope_dim, rope_dim,
// quant_group_size with head_dim = nope + rope, the rope dims inside the last
// chunk), for head_dim a power of two in [8, 512] and chunks of at least 8.
// One lane per 16-byte piece (8 values): a head row is `pieces` consecutive
// lanes of a wave, a chunk `seg` of them, and a chunk's amax is a butterfly
// over its lanes.  A workgroup takes 256 / pieces consecutive tokens of one
// head.  The same arithmetic as row_block: inverse rotation of each rope pair
// rounded to bf16, scale max(amax, eps) / 448 (or its power of two at least
// 2^ceil(log2(max(s, 1e-10))) for packed scales), codes x / scale correctly
// rounded, clamped to +-448.
__device__ void row_block_any(const InvRopeArgs& a, uint32_t rb) {
    const uint32_t P = a.pieces, S = a.seg;
    const uint32_t rows = kThreads / P;
    const uint32_t row_in_block = threadIdx.x / P, p = threadIdx.x % P;
    const uint32_t head = rb % a.num_heads, t0 = (rb / a.num_heads) * rows;
    const uint32_t t = t0 + row_in_block;
    const bool valid = t < a.num_tokens;
    const uint32_t tt = valid ? t : t0;
    const int64_t praw = a.positions[tt];
    __builtin_amdgcn_sched_barrier(0);
    const uint4 v = load16(a.o + (int64_t)tt * a.o_st + (int64_t)head * a.o_sh + 8 * p);
    float x[8];
    unpack8(v, x);
    const uint32_t i0 = 8 * p;
    if (i0 + 8 > a.rope_start) {
        const int64_t pos = clamp_position(praw, a.max_pos);
        const float* cs = a.cos_sin + pos * a.cs_stride;
        const uint32_t half = a.rope_dim / 2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = i0 + 2 * j;
            if (i >= a.rope_start) {
                const uint32_t jj = (i - a.rope_start) / 2;
                const float c = cs[jj], sn = cs[half + jj];
                const float e = x[2 * j], o = x[2 * j + 1];
                const float ec = e * c, os = o * sn, oc = o * c, es = e * sn;
                const uint32_t w = pack_bf16x2(ec + os, oc - es);
                x[2 * j] = bf16_lo(w);
                x[2 * j + 1] = bf16_hi(w);
            }
        }
    }
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        m = max(m, __float_as_uint(x[i]) & 0x7fffffffu);
    for (uint32_t off = 1; off < S; off <<= 1)  // the chunk's lanes: aligned runs of S
        m = max(m, (uint32_t)__shfl_xor((int)m, (int)off));
    const uint32_t eps_bits = __float_as_uint(a.eps);
    m = m > eps_bits ? m : eps_bits;
    float sc = __uint_as_float(m) * (float)(1.0 / 448.0);
    uint32_t lo, hi, byte = 0;
    if (a.tma) {
        uint32_t b = __float_as_uint(sc);
        b = b > 0x2EDBE6FFu ? b : 0x2EDBE6FFu;  // 1e-10f
        const int e = (int)(b >> 23) - 127 + ((b & 0x7fffffu) ? 1 : 0);
        byte = (uint32_t)(e + 127);
        const float inv = exp2_neg_int(e);
        lo = pack_fp8x4(clamp_fp8(x[0] * inv), clamp_fp8(x[1] * inv), clamp_fp8(x[2] * inv), clamp_fp8(x[3] * inv));
        hi = pack_fp8x4(clamp_fp8(x[4] * inv), clamp_fp8(x[5] * inv), clamp_fp8(x[6] * inv), clamp_fp8(x[7] * inv));
    } else {
        const float y = 1.0f / sc;
        float qv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            qv[i] = clamp_fp8(div_by_scale(x[i], sc, y));
        lo = pack_fp8x4(qv[0], qv[1], qv[2], qv[3]);
        hi = pack_fp8x4(qv[4], qv[5], qv[6], qv[7]);
    }
    const uint32_t g = head / a.heads_per_group, hig = head - g * a.heads_per_group;
    if (valid)
        store8(a.fp8 + (int64_t)g * a.fp8_sg + (int64_t)t * a.fp8_st + hig * a.head_dim + 8 * p, lo, hi);
    if (a.tma) {
        // the row's first lane packs the chunks' bytes (at most four chunks)
        const int base = (int)((threadIdx.x & 63) - p);
        uint32_t packed = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t bc = (uint32_t)__shfl((int)byte, base + (int)(min((uint32_t)c, a.chunks - 1) * S));
            if ((uint32_t)c < a.chunks)
                packed |= bc << (8 * c);
        }
        if (valid && p == 0)
            static_cast<uint32_t*>(a.scale)[(int64_t)g * a.sc_sg + (int64_t)hig * a.sc_sk + t] = packed;
    } else if (valid && p % S == 0) {
        const uint32_t c = p / S;
        static_cast<float*>(a.scale)[(int64_t)g * a.sc_sg + (int64_t)(hig * a.chunks + c) * a.sc_sk + t] = sc;
    }
}

__global__ void __launch_bounds__(kThreads)
inv_rope_fp8_quant_any_kernel(InvRopeArgs a) {
    if (blockIdx.x < a.row_blocks)
        row_block_any(a, blockIdx.x);
    else
        pad_block(a);
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_inv_rope_fp8_quant(
    const void* o, int64_t o_stride_token, int64_t o_stride_head,
    const int64_t* positions,
    const float* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos,
    int64_t num_tokens, int64_t n_groups, int64_t heads_per_group,
    int64_t nope_dim, int64_t rope_dim, int64_t quant_group_size,
    void* fp8_out, int64_t fp8_stride_group, int64_t fp8_stride_token,
    void* scale_out, int64_t scale_stride_group, int64_t scale_stride_k,
    int64_t padded_tokens, float eps, int tma_aligned_scales,
    void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || n_groups <= 0 || heads_per_group <= 0)
        return fail(FGV_E_BAD_SHAPE, "bad num_tokens, n_groups or heads_per_group");
    // the reference's geometry assertions (ops/fused_inv_rope_fp8_quant.py:192-205)
    const int64_t head_dim = nope_dim + rope_dim;
    if (nope_dim < 0 || rope_dim <= 0 || rope_dim % 2 || quant_group_size <= 0 || head_dim % quant_group_size ||
        nope_dim % quant_group_size != quant_group_size - rope_dim)
        return fail(FGV_E_BAD_SHAPE, "geometry: rope_dim even, quant_group_size | head_dim, "
                                     "nope_dim % quant_group_size == quant_group_size - rope_dim");
    const int64_t chunks = head_dim / quant_group_size;
    if (tma_aligned_scales && chunks > 4)
        return fail(FGV_E_BAD_SHAPE, "packed UE8M0 scales take at most 4 chunks per head");
    // this build's limits: head_dim a power of two in [8, 512], chunks of at
    // least 8 values; packed scales need a word per head in the reference's
    // packed scale tensor (four chunks per head, or one head per group)
    const bool pow2 = (head_dim & (head_dim - 1)) == 0 && (quant_group_size & (quant_group_size - 1)) == 0;
    if (!pow2 || head_dim < 8 || head_dim > 512 || quant_group_size < 8)
        return fail(FGV_E_BAD_SHAPE, "head_dim must be a power of two in [8, 512], quant_group_size one >= 8");
    if (tma_aligned_scales && chunks != 4 && heads_per_group != 1)
        return fail(FGV_E_BAD_SHAPE, "packed scales with fewer than 4 chunks per head need heads_per_group 1");
    if (padded_tokens < num_tokens || padded_tokens > num_tokens + 3)
        return fail(FGV_E_BAD_SHAPE, "padded_tokens must be num_tokens rounded up to 4");
    const int64_t num_heads = n_groups * heads_per_group;
    const int64_t rows = num_tokens * num_heads;
    if (rows > 0x7fffffffLL || padded_tokens * num_heads * chunks > 0x7fffffffLL ||
        num_tokens * num_heads * head_dim > (1LL << 46))
        return fail(FGV_E_TOO_LARGE, "num_tokens * num_heads * chunks must be below 2^31");
    if (padded_tokens == 0)
        return FGV_OK;
    if (!scale_out || (rows > 0 && (!o || !positions || !cos_sin_cache || !fp8_out)))
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (max_pos <= 0 && rows > 0)
        return fail(FGV_E_BAD_SHAPE, "cos_sin_cache has no rows");
    if (!(eps > 0.0f))
        return fail(FGV_E_BAD_SHAPE, "eps must be positive");
    // DeepSeek-V4's kernel reads cos/sin rows as 16-byte pieces; the general
    // one reads single floats
    const bool dsv4 = nope_dim == kNopeDim && rope_dim == kRopeDim && quant_group_size == 128;
    if (!aligned(o, 16) || !aligned(cos_sin_cache, dsv4 ? 16 : 4) || !aligned(fp8_out, 8) ||
        !aligned(scale_out, 4))
        return fail(FGV_E_MISALIGNED, "o (and cos_sin_cache for 64 rope dims) must be 16-byte aligned, fp8_out 8");
    if (o_stride_token % 8 || o_stride_head % 8 || (dsv4 && cos_sin_stride % 4) ||
        fp8_stride_group % 8 || fp8_stride_token % 8)
        return fail(FGV_E_BAD_STRIDE, "o/fp8 strides must be multiples of 8 (cos_sin of 4 for 64 rope dims)");

    InvRopeArgs a;
    a.o = static_cast<const uint16_t*>(o);
    a.positions = positions;
    a.cos_sin = cos_sin_cache;
    a.fp8 = static_cast<uint8_t*>(fp8_out);
    a.scale = scale_out;
    a.o_st = o_stride_token;
    a.o_sh = o_stride_head;
    a.cs_stride = cos_sin_stride;
    a.max_pos = max_pos;
    a.fp8_sg = fp8_stride_group;
    a.fp8_st = fp8_stride_token;
    a.sc_sg = scale_stride_group;
    a.sc_sk = scale_stride_k;
    a.num_heads = (uint32_t)num_heads;
    a.heads_per_group = (uint32_t)heads_per_group;
    a.num_tokens = (uint32_t)num_tokens;
    a.padded_tokens = (uint32_t)padded_tokens;
    a.n_groups = (uint32_t)n_groups;
    a.eps = eps;
    a.tma = tma_aligned_scales ? 1 : 0;
    a.head_dim = (uint32_t)head_dim;
    a.rope_dim = (uint32_t)rope_dim;
    a.rope_start = (uint32_t)nope_dim;
    a.chunks = (uint32_t)chunks;
    a.pieces = (uint32_t)(head_dim / 8);
    a.seg = (uint32_t)(quant_group_size / 8);
    const int64_t tokens_per_block = dsv4 ? kTokensPerBlock : kThreads / a.pieces;
    const int64_t row_blocks = (num_tokens + tokens_per_block - 1) / tokens_per_block * num_heads;
    if (row_blocks >= 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "grid exceeds 2^31 - 1 workgroups");
    a.row_blocks = (uint32_t)row_blocks;
    const uint32_t grid = a.row_blocks + (padded_tokens > num_tokens ? 1u : 0u);
    if (dsv4)
        hipLaunchKernelGGL(inv_rope_fp8_quant_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                           a);
    else
        hipLaunchKernelGGL(inv_rope_fp8_quant_any_kernel, dim3(grid), dim3(kThreads), 0,
                           static_cast<hipStream_t>(stream), a);
    return launch_status();
}
