// gfx950 kernel for the fused DeepSeek-V4 q RMSNorm + RoPE and kv RoPE +
// UE8M0 FP8 quant + paged-cache insert.
//
// Reference semantics: src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py
//   q branch  :61-72, 79-97   kv branch :74-93, 98-286   wrapper :289-351
//
// One launch, two kinds of workgroup (256 threads = 4 waves = 16 DPP rows):
//   blocks [0, kv_blocks)          : 16 tokens' kv rows each -> k_cache
//   blocks [kv_blocks, grid)       : kQRowsPerBlock q rows each, in place
// Each 1 KiB row is owned by one 16-lane DPP row (see fgv_device.h).  The op
// is HBM bound (about 98.6% of its bytes are the in-place q read and write):
// every global access is a non-temporal 16-byte (8-byte for the cache) access,
// the per-row math uses DPP reductions only, and q blocks hold one pass of 16
// rows (16 KiB in, 16 KiB out); large grids run four workgroups per CU
// (kOccupancyLds below), 4 waves per SIMD with 4 KiB of loads in flight each.
// The cos/sin row of a token is read from L2 by each row's rope lanes, except
// on one-round grids of 4-8 workgroups per CU with whole tokens per block,
// where it is staged in LDS once per block (q_block's kCsLds: measured faster
// there, slower elsewhere).  One-round grids of 256..1152 workgroups run their
// blocks in XCD-contiguous order, and grids from 1.25 GiB of q in runs of 16
// blocks per XCD (see "Block order" below).
//
// Which 16 rows a q block takes (QMap):
//   kMapRows / kMapRowsOneToken: rows 16b .. 16b+15 in (token, head) order.
//   kMapAligned: q rows that are 1 KiB units of memory (head stride 512, token
//     pitch a multiple of 512 elements, q 1 KiB aligned) but do not tile
//     16 KiB-aligned chunks, e.g. q a slice of a wider [T, H*512 + 512] buffer.
//     Block b takes the 16 units of the 16 KiB-aligned chunk b of the window
//     that starts at q rounded down to 16 KiB; units outside q (the pitch gap,
//     or before q) are skipped.  A stream of misaligned 16 KiB chunks measured
//     ~9 % slower than the same stream in aligned chunks.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerPass = kThreads / 16;   // 16 rows per pass
// One pass of four 16-byte loads per lane; more rows per block (more loads per
// wave, fewer waves) measured slower.
constexpr int kQRowsPerBlock = kRowsPerPass;
constexpr int kKvTokensPerBlock = kRowsPerPass;
// Dynamic LDS reserved per workgroup (the kernel uses none) to cap the launch
// at four workgroups, 16 waves, per CU (160 KiB of LDS).  Each wave keeps 4 KiB
// of loads in flight; with all 32 wave slots of a CU filled the GPU has ~32 MB
// of rows in flight, which measured slower than ~16 MB (c2 168.7 -> 165.5 us,
// c4 1266 -> 1225 us; five per CU the same, three slower).  An in-place stream
// probe with four loads per lane showed the same, and the one-load-per-lane
// stream the probe peaks with fills every slot.
constexpr size_t kOccupancyLds = 40 * 1024;
// The cap applies to grids of more than one uncapped round of workgroups (8 per
// CU on MI355X's 256 CUs).  A smaller grid fits the GPU at once without it,
// while the cap would split it: c1 (T = 256, H = 64) is 1040 workgroups, one
// round uncapped, but 1024 + 16 with four per CU.
constexpr int64_t kUncappedRound = 8 * 256;
// One-round grids of at least four workgroups per CU stage the cos/sin row in
// LDS (q_block's kCsLds); smaller ones load it per row.  Same-box A/B, µs per
// call: c1 (1040 workgroups) 7.12 -> 6.62; T = 64 x H = 128 (516) 4.23 ->
// 4.40, T = 17 x H = 64 (72) 2.20 -> 2.29, T = 1 and 4 unchanged.
constexpr int64_t kCsLdsMinGrid = 4 * 256;

// Block order.  Workgroups are dispatched to the 8 XCDs round-robin (block b
// on XCD b % 8).  Two remaps (bijections on a prefix of the grid; the tail
// maps to itself), measured in same-box A/Bs (bit-identical outputs,
// HIP-graph replay, median of 5):
//   - XCD-contiguous (xcd_per = grid / 8): logical block
//     (b % 8) * xcd_per + b / 8, each XCD a contiguous eighth of the rows.
//     One-round grids of 256..1152 workgroups gain 1.3-3 % (c1, T = 256,
//     H = 64: 6.54 -> 6.35 us; the rows of one token and their cos/sin row
//     stay on one XCD's L2); from 1285 workgroups on it loses (c2 -7 %).
//   - Runs of kXcdRun blocks (group_full > 0): 8 consecutive runs of 16
//     blocks (256 KiB of q each) go one to each XCD, so each XCD streams
//     256 KiB stretches while all XCDs stay inside one 2 MiB window.  From
//     1.5 GiB of q it gains 1.9-5.2 % (c3 1385 -> 1321 us, c4 1231 -> 1178,
//     T = 65536 x H = 128 2772 -> 2627, T = 131072 x H = 128 5523 -> 5268);
//     at 1 GiB it is level, at 0.5 GiB (c2) 1-1.6 % slower.  Runs of 8
//     blocks did 1-3 % worse than 16 on most shapes, runs of 2, 4, 32, 64
//     and 128 worse still.
constexpr int64_t kXcdOrderMinGrid = 256;
constexpr int64_t kXcdOrderMaxOneRound = 1152;
constexpr uint32_t kXcdRun = 16;
constexpr int64_t kXcdRunsMinGrid = 81920;  // 1.25 GiB of q rows

// The block order is a template parameter, so each launch carries only the
// remap its grid uses.
enum BlockOrder { kOrderRoundRobin = 0, kOrderContiguous = 1, kOrderRuns = 2 };

BlockOrder block_order(int64_t grid) {
    if (grid >= kXcdOrderMinGrid && grid <= kXcdOrderMaxOneRound)
        return kOrderContiguous;
    return grid >= kXcdRunsMinGrid ? kOrderRuns : kOrderRoundRobin;
}

struct QnormArgs {
    uint16_t* q;
    const uint16_t* kv;
    uint8_t* k_cache;
    const int64_t* slot_mapping;
    const int64_t* positions;
    const float* cos_sin;
    int64_t q_st, q_sh, kv_st;
    int64_t block_stride, num_blocks, block_size;
    int64_t cs_stride, max_pos;
    uint32_t num_q_rows;       // num_tokens * num_heads
    uint32_t num_heads;
    uint32_t num_tokens;
    uint32_t pitch_units;      // kMapAligned: token pitch in 1 KiB units (>= num_heads)
    uint32_t lead_units;       // kMapAligned: 1 KiB units from the 16 KiB boundary below q to q
    double inv_pitch;          // kMapAligned: 1.0 / pitch_units
    uint32_t num_tokens_insert;
    uint32_t kv_blocks;
    uint32_t xcd_per;          // 0, or grid / 8: blocks [0, 8 xcd_per) run in XCD-contiguous order
    uint32_t group_full;       // 0, or the blocks [0, group_full) run in runs of kXcdRun per XCD
    float eps;
};

// RMSNorm factor r = 1/sqrt(mean(x^2) + eps) of the row owned by this lane's
// 16-lane group.  The sum of squares is accumulated in binary64: squares of
// bf16 values are exact there, and so is their sum unless the row's squares
// span more than 28 binary orders of magnitude; otherwise its rounding error
// (below 2^-44 relative) lies far under the binary32 rounding of the mean, so
// the reduction order matters only when the mean falls that close to a
// binary32 rounding boundary.  Mean and rsqrt are then correctly rounded.
__device__ __forceinline__ float rms_factor(const uint4 (&v)[4], float eps) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            double a = (double)bf16_lo(w[i]);
            double b = (double)bf16_hi(w[i]);
            s = __builtin_fma(a, a, s);
            s = __builtin_fma(b, b, s);
        }
    }
    s = row16_sum(s);
    float var = (float)(s * (1.0 / kHeadDim));
    var = var + eps;
    return (float)(1.0 / __builtin_sqrt((double)var));
}

// GPT-J rotation of the four (even, odd) pairs in one 16-byte piece of bf16,
// each product and sum rounded to binary32 separately (no FMA contraction;
// the file is built with -ffp-contract=off), then packed to bf16 with RNE.
__device__ __forceinline__ uint4 rope_piece(const float (&x)[8], float4 c, float4 s) {
    const float cc[4] = {c.x, c.y, c.z, c.w};
    const float ss[4] = {s.x, s.y, s.z, s.w};
    uint32_t out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float e = x[2 * i], o = x[2 * i + 1];
        float ec = e * cc[i], os = o * ss[i];
        float es = e * ss[i], oc = o * cc[i];
        out[i] = pack_bf16x2(ec - os, es + oc);
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

__device__ __forceinline__ void unpack8(uint4 v, float (&x)[8]) {
    x[0] = bf16_lo(v.x); x[1] = bf16_hi(v.x);
    x[2] = bf16_lo(v.y); x[3] = bf16_hi(v.y);
    x[4] = bf16_lo(v.z); x[5] = bf16_hi(v.z);
    x[6] = bf16_lo(v.w); x[7] = bf16_hi(v.w);
}

// RMSNorm of one q row held in v (this lane's four pieces), GPT-J rotation of
// its rope lanes with this lane's cos/sin, bf16 stores in place.
__device__ __forceinline__ void q_row_math(const QnormArgs& a, uint16_t* rowp, const uint4 (&v)[4], int lane16,
                                           bool rope_lane, float4 cs_c, float4 cs_s) {
    const float r = rms_factor(v, a.eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float x[8];
        unpack8(v[k], x);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            x[i] = x[i] * r;
        uint4 out;
        if (k == 3 && rope_lane) {
            out = rope_piece(x, cs_c, cs_s);
        } else {
            out = make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]),
                             pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
        }
        store16(rowp + (lane16 + 16 * k) * 8, out);
    }
}

enum QMap { kMapRows = 0, kMapRowsOneToken = 1, kMapAligned = 2 };

// v / p for v, p < 2^32 (p >= 1).  The binary64 estimate v * (1/p) is within
// 2^-20 of the quotient (two roundings of relative size 2^-53 on a value
// below 2^32), so its floor is off by at most one; the checks make it exact.
__device__ __forceinline__ uint32_t div_pitch(uint32_t v, uint32_t p, double inv_p) {
    uint32_t t = (uint32_t)((double)v * inv_p);
    if ((uint64_t)t * p > v)
        --t;
    else if (((uint64_t)t + 1) * p <= v)
        ++t;
    return t;
}

// Loads are issued position first: the cos/sin row depends on it, and the
// in-order vmcnt counter would otherwise make that dependent load wait for
// the q loads issued before it.  kMapRowsOneToken (num_heads a multiple of
// 16): all rows of the block share one token, whose position is a scalar load.
// kCsLds (kMapRowsOneToken, one-round grids of 1024..2048 workgroups): the
// cos/sin row is staged in LDS once per block instead of loaded by each row's
// rope lanes.  Measured on MI355X (same-box A/Bs): c1 (T = 256, H = 64, one
// round of 1040 workgroups) 7.07-7.20 -> 6.43-6.62 us; on grids of several
// rounds the block barrier costs more than it saves (c2 +2.7-3.2 %, c3
// +2.4 %), and on one-round grids below four workgroups per CU it is up to
// 4 % slower (kCsLdsMinGrid), so those load per row.  A per-wave variant
// without the barrier (the wave's first row loads, row permutes broadcast)
// measured no faster than per-row loads on c1.
template <int kMap, bool kCsLds>
__device__ void q_block(const QnormArgs& a, uint32_t qb, int lane16, int row_in_pass) {
    const bool rope_lane = lane16 >= 8;
    uint32_t t;
    int64_t pos_raw;
    bool valid;
    uint16_t* rowp;
    if (kMap == kMapAligned) {
        // unit u of the window; v = u - lead wraps for units before q, and
        // then fails the token bound
        const uint32_t u = qb * kQRowsPerBlock + row_in_pass;
        const uint32_t v = u - a.lead_units;
        const uint32_t tt = div_pitch(v, a.pitch_units, a.inv_pitch);
        const uint32_t h = v - tt * a.pitch_units;
        valid = u >= a.lead_units && tt < a.num_tokens && h < a.num_heads;
        t = valid ? tt : 0;
        pos_raw = a.positions[t];  // every lane loads: no branch before the q loads
        __builtin_amdgcn_sched_barrier(0);
        rowp = a.q + (int64_t)v * kHeadDim;  // = q + tt*pitch + h*512 elements
    } else {
        const uint32_t row0 = qb * kQRowsPerBlock;
        const uint32_t row = row0 + row_in_pass;
        valid = row < a.num_q_rows;
        if (kMap == kMapRowsOneToken) {
            t = row0 / a.num_heads;  // uniform across the block
            pos_raw = a.positions[t];
        } else {
            t = (valid ? row : row0) / a.num_heads;
            pos_raw = a.positions[t];  // every lane loads: no branch before the q loads
            __builtin_amdgcn_sched_barrier(0);  // keep it ahead of the q loads
        }
        const uint32_t h = row - t * a.num_heads;
        rowp = a.q + (int64_t)t * a.q_st + (int64_t)h * a.q_sh;
    }
    if (kCsLds) {
        // One-round grids: the token's 256-byte cos/sin row is loaded once
        // per block (by threads 0..15) into LDS.  Every row of the block has
        // that token (kMapRowsOneToken).
        __shared__ float4 cs_row[16];
        uint4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v[k] = load16(rowp + (lane16 + 16 * k) * 8);
        if (threadIdx.x < 16) {
            const int64_t pos = clamp_position(pos_raw, a.max_pos);
            cs_row[threadIdx.x] = *reinterpret_cast<const float4*>(a.cos_sin + pos * a.cs_stride + threadIdx.x * 4);
        }
        __syncthreads();
        float4 cs_c = make_float4(0.f, 0.f, 0.f, 0.f), cs_s = cs_c;
        if (rope_lane) {
            cs_c = cs_row[lane16 - 8];  // cos of pairs 4(lane16-8) ..
            cs_s = cs_row[lane16];      // sin of the same pairs
        }
        q_row_math(a, rowp, v, lane16, rope_lane, cs_c, cs_s);
        return;
    }
    if (!valid)
        return;
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = load16(rowp + (lane16 + 16 * k) * 8);
    const int64_t pos = clamp_position(pos_raw, a.max_pos);
    float4 cs_c = make_float4(0.f, 0.f, 0.f, 0.f), cs_s = cs_c;
    if (rope_lane) {
        const float* cs = a.cos_sin + pos * a.cs_stride + (lane16 - 8) * 4;
        cs_c = *reinterpret_cast<const float4*>(cs);
        cs_s = *reinterpret_cast<const float4*>(cs + kHalfRope);
    }
    q_row_math(a, rowp, v, lane16, rope_lane, cs_c, cs_s);
}


// UE8M0 exponent of a 64-element group: ceil(log2(max(amax, 1e-4) / 448)).
// With a = m * 2^E (1 <= m < 2) and 448 = 1.75 * 2^8 this is
// E - 8 + (m > 1.75), read straight from the binary32 fields of a.
__device__ __forceinline__ int kv_group_exponent(uint32_t amax_bits) {
    const uint32_t kFloor = 0x38D1B717u;  // 1e-4f
    uint32_t a = amax_bits > kFloor ? amax_bits : kFloor;
    int e = (int)(a >> 23) - 127;
    return e - 8 + ((a & 0x7fffffu) > 0x600000u ? 1 : 0);
}

__device__ void kv_block(const QnormArgs& a, uint32_t kvb, int lane16, int row_in_pass) {
    const uint32_t t = kvb * kKvTokensPerBlock + row_in_pass;
    if (t >= a.num_tokens_insert)
        return;
    // slot and position first (see q_block), then the kv row, then cos/sin
    const int64_t slot = a.slot_mapping[t];
    const int64_t pos_raw = a.positions[t];
    __builtin_amdgcn_sched_barrier(0);  // both ahead of the kv loads
    const uint16_t* x = a.kv + (int64_t)t * a.kv_st;
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = load16(x + (lane16 + 16 * k) * 8);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t pos = clamp_position(pos_raw, a.max_pos);
    if (slot < 0)
        return;
    const int64_t blk = slot / a.block_size;
    const int64_t pib = slot - blk * a.block_size;
    if (blk >= a.num_blocks)
        return;
    const bool rope_lane = lane16 >= 8;
    float4 c = make_float4(0.f, 0.f, 0.f, 0.f), s = c;
    if (rope_lane) {
        const float* cs = a.cos_sin + pos * a.cs_stride + (lane16 - 8) * 4;
        c = *reinterpret_cast<const float4*>(cs);
        s = *reinterpret_cast<const float4*>(cs + kHalfRope);
    }

    uint8_t* base = a.k_cache + blk * a.block_stride;
    uint8_t* tok = base + pib * kTokenDataBytes;
    uint8_t* scl = base + a.block_size * kTokenDataBytes + pib * kScaleBytesPerToken;

    // Cache stores are 8 bytes per lane (the codes of the lane's 8 dims; two
    // per RoPE lane).  16-byte stores (odd lanes' codes moved to even lanes by
    // DPP, the RoPE bytes in one store, when the cache allows 16-byte
    // alignment) measured slower in a same-box A/B: c0 2.25 -> 2.61 us, c1
    // unchanged, c2 +1.1 %.  The kv rows are 1.4 % of c2's bytes, and the
    // measured HBM traffic is already 1.008 x the algorithmic bytes.
    // Folding each token's kv row into a fifth wave of that token's first q
    // block (one-round grids, no kv blocks) measured slower too: c1 7.20 ->
    // 8.0 us.
    uint32_t my_bytes = 0;  // byte k = scale byte of the group in piece k
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float xf[8];
        unpack8(v[k], xf);
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            m = max(m, __float_as_uint(xf[i]) & 0x7fffffffu);
        m = row8_max(m);  // lanes 0..7: group 2k, lanes 8..15: group 2k+1
        const int e = kv_group_exponent(m);
        const float inv = exp2_neg_int(e);  // exact, so x * 2^-e == x / 2^e
        const int enc = e + 127;
        my_bytes |= (uint32_t)(enc < 0 ? 0 : (enc > 255 ? 255 : enc)) << (8 * k);
        if (k == 3 && rope_lane) {
            uint4 r = rope_piece(xf, c, s);
            uint8_t* dst = tok + kNopeDim + (lane16 - 8) * 16;
            store8(dst, r.x, r.y);
            store8(dst + 8, r.z, r.w);
        } else {
            uint32_t lo = pack_fp8x4(clamp_fp8(xf[0] * inv), clamp_fp8(xf[1] * inv),
                                     clamp_fp8(xf[2] * inv), clamp_fp8(xf[3] * inv));
            uint32_t hi = pack_fp8x4(clamp_fp8(xf[4] * inv), clamp_fp8(xf[5] * inv),
                                     clamp_fp8(xf[6] * inv), clamp_fp8(xf[7] * inv));
            store8(tok + (lane16 + 16 * k) * 8, lo, hi);
        }
    }
    // Lane 0 holds groups 0,2,4,6 and lane 8 holds groups 1,3,5: gather the
    // seven scale bytes plus the zero pad byte into one 8-byte store.
    const uint32_t other = dpp_u32<kDppRowRor8>(my_bytes);
    if (lane16 == 0) {
        uint32_t lo = (my_bytes & 0xffu) | ((other & 0xffu) << 8) |
                      ((my_bytes & 0xff00u) << 8) | ((other & 0xff00u) << 16);
        uint32_t hi = ((my_bytes >> 16) & 0xffu) | (((other >> 16) & 0xffu) << 8) |
                      (((my_bytes >> 24) & 0xffu) << 16);
        store8(scl, lo, hi);
    }
}

template <int kMap, bool kCsLds, int kOrder>
__global__ void __launch_bounds__(kThreads)
qnorm_rope_kv_insert_kernel(QnormArgs a) {
    const int lane16 = threadIdx.x & 15;
    const int row_in_pass = threadIdx.x >> 4;
    uint32_t b = blockIdx.x;
    if (kOrder == kOrderContiguous && b < 8 * a.xcd_per)
        b = (b % 8) * a.xcd_per + b / 8;
    else if (kOrder == kOrderRuns && b < a.group_full)
        b = b / (8 * kXcdRun) * (8 * kXcdRun) + (b % 8) * kXcdRun + (b / 8) % kXcdRun;
    if (b < a.kv_blocks)
        kv_block(a, b, lane16, row_in_pass);
    else
        q_block<kMap, kCsLds>(a, b - a.kv_blocks, lane16, row_in_pass);
}

template <int kMap, bool kCsLds>
void launch_ordered(BlockOrder order, dim3 grid, size_t lds, hipStream_t st, const QnormArgs& a) {
    if (order == kOrderContiguous)
        hipLaunchKernelGGL((qnorm_rope_kv_insert_kernel<kMap, kCsLds, kOrderContiguous>), grid, dim3(kThreads), lds,
                           st, a);
    else if (order == kOrderRuns)
        hipLaunchKernelGGL((qnorm_rope_kv_insert_kernel<kMap, kCsLds, kOrderRuns>), grid, dim3(kThreads), lds, st,
                           a);
    else
        hipLaunchKernelGGL((qnorm_rope_kv_insert_kernel<kMap, kCsLds, kOrderRoundRobin>), grid, dim3(kThreads), lds,
                           st, a);
}

// cs_lds grids are one round (at most kUncappedRound workgroups), so they never
// take the runs order.
void launch_insert_kernel(int map, bool cs_lds, BlockOrder order, dim3 grid, size_t lds, hipStream_t st,
                     const QnormArgs& a) {
    if (map == kMapAligned)
        launch_ordered<kMapAligned, false>(order, grid, lds, st, a);
    else if (cs_lds && order == kOrderContiguous)
        hipLaunchKernelGGL((qnorm_rope_kv_insert_kernel<kMapRowsOneToken, true, kOrderContiguous>), grid,
                           dim3(kThreads), lds, st, a);
    else if (cs_lds)
        hipLaunchKernelGGL((qnorm_rope_kv_insert_kernel<kMapRowsOneToken, true, kOrderRoundRobin>), grid,
                           dim3(kThreads), lds, st, a);
    else if (map == kMapRowsOneToken)
        launch_ordered<kMapRowsOneToken, false>(order, grid, lds, st, a);
    else
        launch_ordered<kMapRows, false>(order, grid, lds, st, a);
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_qnorm_rope_kv_rope_quant_insert(
    void* q, int64_t q_stride_token, int64_t q_stride_head,
    const void* kv, int64_t kv_stride_token,
    void* k_cache, int64_t cache_block_stride, int64_t num_blocks,
    const int64_t* slot_mapping, int64_t num_tokens_insert,
    const int64_t* position_ids,
    const float* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos,
    int64_t num_tokens, int64_t num_heads,
    float eps, int64_t cache_block_size,
    void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || num_heads < 0 || num_tokens_insert < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_tokens_insert > num_tokens)
        return fail(FGV_E_BAD_SHAPE, "slot_mapping is longer than the number of tokens");
    const int64_t q_rows = num_tokens * num_heads;
    if (q_rows == 0 && num_tokens_insert == 0)
        return FGV_OK;
    if (q_rows > 0x7fffffffLL || num_tokens > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "num_tokens * num_heads must be below 2^31");
    if (!q || !kv || !position_ids || !cos_sin_cache)
        return fail(FGV_E_NULL_POINTER, "null q, kv, position_ids or cos_sin_cache");
    if (num_tokens_insert > 0 && (!k_cache || !slot_mapping))
        return fail(FGV_E_NULL_POINTER, "null k_cache or slot_mapping");
    if (max_pos <= 0)
        return fail(FGV_E_BAD_SHAPE, "cos_sin_cache has no rows");
    if (cache_block_size <= 0)
        return fail(FGV_E_BAD_SHAPE, "cache_block_size must be positive");
    if (!aligned(q, 16) || !aligned(kv, 16) || !aligned(cos_sin_cache, 16))
        return fail(FGV_E_MISALIGNED, "q, kv and cos_sin_cache must be 16-byte aligned");
    if (q_stride_token % 8 || q_stride_head % 8 || kv_stride_token % 8 || cos_sin_stride % 4)
        return fail(FGV_E_BAD_STRIDE,
                    "q/kv strides must be multiples of 8 elements, cos_sin stride of 4");
    if (num_tokens_insert > 0) {
        if (!aligned(k_cache, 8) || cache_block_stride % 8)
            return fail(FGV_E_MISALIGNED, "k_cache and its block stride must be 8-byte aligned");
        if (cache_block_stride < cache_block_size * (kTokenDataBytes + kScaleBytesPerToken))
            return fail(FGV_E_BAD_STRIDE, "k_cache block stride is below cache_block_size * 584");
    }

    QnormArgs a;
    a.q = static_cast<uint16_t*>(q);
    a.kv = static_cast<const uint16_t*>(kv);
    a.k_cache = static_cast<uint8_t*>(k_cache);
    a.slot_mapping = slot_mapping;
    a.positions = position_ids;
    a.cos_sin = cos_sin_cache;
    a.q_st = q_stride_token;
    a.q_sh = q_stride_head;
    a.kv_st = kv_stride_token;
    a.block_stride = cache_block_stride;
    a.num_blocks = num_blocks;
    a.block_size = cache_block_size;
    a.cs_stride = cos_sin_stride;
    a.max_pos = max_pos;
    a.num_q_rows = (uint32_t)q_rows;
    a.num_heads = (uint32_t)(num_heads > 0 ? num_heads : 1);
    a.num_tokens = (uint32_t)num_tokens;
    a.num_tokens_insert = (uint32_t)num_tokens_insert;
    a.kv_blocks = (uint32_t)((num_tokens_insert + kKvTokensPerBlock - 1) / kKvTokensPerBlock);
    a.eps = eps;
    a.pitch_units = a.lead_units = 0;
    a.inv_pitch = 0.0;

    // Row mapping of the q blocks (QMap above).
    constexpr int64_t kUnitBytes = kHeadDim * 2;
    constexpr int64_t kChunkBytes = kUnitBytes * kQRowsPerBlock;
    const int64_t q_addr = (int64_t)reinterpret_cast<uintptr_t>(q);
    const int64_t pitch = num_tokens == 1 ? kHeadDim * num_heads : q_stride_token;
    int map = num_heads > 0 && num_heads % kQRowsPerBlock == 0 ? kMapRowsOneToken : kMapRows;
    int64_t q_blocks = (q_rows + kQRowsPerBlock - 1) / kQRowsPerBlock;
    if (q_rows > 0 && q_stride_head == kHeadDim && pitch % kHeadDim == 0 &&
        pitch >= kHeadDim * num_heads && q_addr % kUnitBytes == 0 &&
        !(pitch == kHeadDim * num_heads && q_addr % kChunkBytes == 0)) {
        const int64_t pitch_units = pitch / kHeadDim;
        const int64_t lead = (q_addr % kChunkBytes) / kUnitBytes;
        const int64_t units = lead + (num_tokens - 1) * pitch_units + num_heads;
        if (units < 0xffffffffLL) {
            map = kMapAligned;
            a.pitch_units = (uint32_t)pitch_units;
            a.lead_units = (uint32_t)lead;
            a.inv_pitch = 1.0 / (double)pitch_units;
            q_blocks = (units + kQRowsPerBlock - 1) / kQRowsPerBlock;
        }
    }
    const int64_t grid = (int64_t)a.kv_blocks + q_blocks;
    if (grid > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "grid exceeds 2^31 - 1 workgroups");
    const BlockOrder order = block_order(grid);
    a.xcd_per = order == kOrderContiguous ? (uint32_t)(grid / 8) : 0u;
    a.group_full = order == kOrderRuns ? (uint32_t)(grid / (8 * kXcdRun) * (8 * kXcdRun)) : 0u;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t lds = grid > kUncappedRound ? kOccupancyLds : 0;
    const bool cs_lds = map == kMapRowsOneToken && grid >= kCsLdsMinGrid && grid <= kUncappedRound;
    launch_insert_kernel(map, cs_lds, order, dim3((uint32_t)grid), lds, st, a);
    return launch_status();
}
