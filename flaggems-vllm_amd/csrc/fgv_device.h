// Device helpers shared by the gfx950 kernels of this library.
//
// Row layout used by every kernel here: one 512-element bf16 row (1 KiB) is
// owned by a 16-lane DPP row of a wave64.  Lane l16 (0..15) holds the four
// 16-byte pieces at element offsets (l16 + 16*k) * 8 for k = 0..3, so each of
// the four global_load_dwordx4 of a wave covers 256 contiguous bytes of each
// of four rows.  With this layout
//   - a 64-element FP8 group (main op) is 8 consecutive lanes of one piece k,
//   - a 128-element FP8 chunk (sibling op) is the 16 lanes of one piece k,
//   - the 64 rope elements 448..511 are lanes 8..15 of piece 3,
// and every reduction is a DPP all-reduce inside one 16-lane row: no LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fgv {

constexpr int kHeadDim = 512;
constexpr int kNopeDim = 448;
constexpr int kRopeDim = 64;
constexpr int kHalfRope = 32;
constexpr int kTokenDataBytes = 576;      // 448 fp8 codes + 64 bf16 rope values
constexpr int kScaleBytesPerToken = 8;    // 7 UE8M0 bytes + 1 zero pad byte
constexpr int kKvGroups = 7;              // 448 / 64
constexpr float kFp8Max = 448.0f;

// GFX9 DPP control words.
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i inside each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i inside each 16 lanes
// row_ror:n rotates right inside each 16 lanes: lane i reads lane (i - n) mod 16
constexpr int kDppRowRor4 = 0x124;     // lane i reads lane (i+12) mod 16
constexpr int kDppRowRor8 = 0x128;     // lane i reads lane (i+8) mod 16
constexpr int kDppRowRor12 = 0x12C;    // lane i reads lane (i+4) mod 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return __builtin_amdgcn_update_dpp(0u, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    uint64_t u = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = dpp_u32<CTRL>((uint32_t)u);
    uint32_t hi = dpp_u32<CTRL>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum over the 16 lanes of a DPP row; every lane gets the total.
__device__ __forceinline__ double row16_sum(double v) {
    v += dpp_f64<kDppQuadXor1>(v);
    v += dpp_f64<kDppQuadXor2>(v);
    v += dpp_f64<kDppHalfMirror>(v);
    v += dpp_f64<kDppMirror>(v);
    return v;
}

// Max of non-negative float bit patterns over each 8-lane half row.
__device__ __forceinline__ uint32_t row8_max(uint32_t v) {
    v = max(v, dpp_u32<kDppQuadXor1>(v));
    v = max(v, dpp_u32<kDppQuadXor2>(v));
    v = max(v, dpp_u32<kDppHalfMirror>(v));
    return v;
}

// Max of non-negative float bit patterns over the 16-lane row.
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
    v = row8_max(v);
    v = max(v, dpp_u32<kDppMirror>(v));
    return v;
}

// Max / sum over the four lanes l, l^16, l^32, l^48 (the four lane groups
// of one column of a 16x16 MFMA tile) with gfx950's row-swapping permutes: with both operands x,
// v_permlane16_swap returns {x[l], x[l^16]} (in row order) and
// v_permlane32_swap {x[l], x[l^32]}, so each step is two VALU operations and
// every lane of the four gets the same result (no LDS round trip).
__device__ __forceinline__ float group4_max(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t w = __float_as_uint(v);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float group4_sum(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const uint32_t w = __float_as_uint(v);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats -> bf16x2, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Four floats (already inside +-448) -> four OCP e4m3fn codes, round to nearest
// even, byte i = code of argument i (v_cvt_pk_fp8_f32, gfx950 OCP format).
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

__device__ __forceinline__ float clamp_fp8(float x) {
    return __builtin_amdgcn_fmed3f(x, -kFp8Max, kFp8Max);
}

// 2^-k as a binary32, exact for -126 <= k <= 126.
__device__ __forceinline__ float exp2_neg_int(int k) {
    return __uint_as_float((uint32_t)(127 - k) << 23);
}

// Streaming (non-temporal) global accesses: every byte these kernels move is
// touched exactly once, so loads and stores carry the nt hint and bypass
// cache allocation.  On MI355X this is worth about 15% of HBM bandwidth for
// the in-place q stream (loads and stores both need it).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load16(const void* p) {
    u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store16(void* p, uint4 v) {
    u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void store8(void* p, uint32_t lo, uint32_t hi) {
    u32x2_t w = {lo, hi};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t*>(p));
}

__device__ __forceinline__ int64_t clamp_position(int64_t p, int64_t max_pos) {
    return p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
}

}  // namespace fgv
