// gfx950 kernel for DeepSeek-V4's fused q/kv RMSNorm: two weighted RMSNorms
// (the q LoRA row and the kv latent row of each token) in one launch.
//
// Reference semantics: src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:24-103
//   y = (x * rsqrt(mean(x^2) + eps)) * w, stored in x's dtype (bf16).
//
// Layout: one row per 16-lane DPP row (fgv_device.h); lane l16 owns the
// 16-byte pieces c = l16 + 16*j, j < kMaxPieces, of its row, so a 1536-wide
// q row is 12 pieces per lane and a 512-wide kv row 4.  Workgroups
// [0, q_blocks) take 16 q rows, the rest 16 kv rows.  As in the main op the
// sum of squares is exact in binary64 and mean and rsqrt are correctly
// rounded, so results do not depend on the reduction order.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 16;

struct RmsArgs {
    const uint16_t* x[2];
    uint16_t* y[2];
    const void* w[2];
    int64_t x_stride[2], y_stride[2];
    int32_t size[2];
    uint32_t num_rows;
    uint32_t q_blocks;
    float eps;
    int weight_f32;
};

__device__ __forceinline__ void weights8(const void* w, int e, bool f32, float (&out)[8]) {
    if (f32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + e);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + e + 4);
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e);
        out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x);
        out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
        out[4] = bf16_lo(v.z); out[5] = bf16_hi(v.z);
        out[6] = bf16_lo(v.w); out[7] = bf16_hi(v.w);
    }
}

template <int kMaxPieces>
__global__ void __launch_bounds__(kThreads)
fused_q_kv_rmsnorm_kernel(RmsArgs a) {
    const int lane16 = threadIdx.x & 15;
    const bool is_kv = blockIdx.x >= a.q_blocks;
    const int which = is_kv ? 1 : 0;
    const uint32_t row = (blockIdx.x - (is_kv ? a.q_blocks : 0)) * kRowsPerBlock + (threadIdx.x >> 4);
    if (row >= a.num_rows)
        return;
    const int size = a.size[which];
    const int pieces = size >> 3;
    const uint16_t* x = a.x[which] + (int64_t)row * a.x_stride[which];
    uint16_t* y = a.y[which] + (int64_t)row * a.y_stride[which];

    uint4 v[kMaxPieces];
#pragma unroll
    for (int j = 0; j < kMaxPieces; ++j) {
        const int c = lane16 + 16 * j;
        v[j] = c < pieces ? load16(x + c * 8) : make_uint4(0, 0, 0, 0);
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kMaxPieces; ++j) {
        const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double lo = (double)bf16_lo(w4[i]), hi = (double)bf16_hi(w4[i]);
            s = __builtin_fma(lo, lo, s);
            s = __builtin_fma(hi, hi, s);
        }
    }
    s = row16_sum(s);
    float var = (float)(s / (double)size);
    var = var + a.eps;
    const float r = (float)(1.0 / __builtin_sqrt((double)var));

#pragma unroll
    for (int j = 0; j < kMaxPieces; ++j) {
        const int c = lane16 + 16 * j;
        if (c < pieces) {
            float wv[8];
            weights8(a.w[which], c * 8, a.weight_f32, wv);
            const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lo = (bf16_lo(w4[i]) * r) * wv[2 * i];
                const float hi = (bf16_hi(w4[i]) * r) * wv[2 * i + 1];
                o[i] = pack_bf16x2(lo, hi);
            }
            store16(y + c * 8, make_uint4(o[0], o[1], o[2], o[3]));
        }
    }
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_fused_q_kv_rmsnorm(
    const void* qr, int64_t qr_stride, void* qr_out, int64_t qr_out_stride,
    const void* q_weight, int64_t q_size,
    const void* kv, int64_t kv_stride, void* kv_out, int64_t kv_out_stride,
    const void* kv_weight, int64_t kv_size,
    int64_t num_tokens, float eps, int weight_is_fp32, void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || q_size < 0 || kv_size < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_tokens == 0)
        return FGV_OK;
    if (num_tokens > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "num_tokens must be below 2^31");
    if (q_size % 8 || kv_size % 8 || q_size == 0 || kv_size == 0)
        return fail(FGV_E_BAD_SHAPE, "row sizes must be positive multiples of 8");
    if (q_size > 4096 || kv_size > 4096)
        return fail(FGV_E_TOO_LARGE, "row sizes above 4096 are not supported");
    if (!qr || !qr_out || !q_weight || !kv || !kv_out || !kv_weight)
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (!aligned(qr, 16) || !aligned(qr_out, 16) || !aligned(kv, 16) || !aligned(kv_out, 16) ||
        !aligned(q_weight, 16) || !aligned(kv_weight, 16))
        return fail(FGV_E_MISALIGNED, "rows and weights must be 16-byte aligned");
    if (qr_stride % 8 || qr_out_stride % 8 || kv_stride % 8 || kv_out_stride % 8)
        return fail(FGV_E_BAD_STRIDE, "row strides must be multiples of 8 elements");

    RmsArgs a;
    a.x[0] = static_cast<const uint16_t*>(qr);
    a.x[1] = static_cast<const uint16_t*>(kv);
    a.y[0] = static_cast<uint16_t*>(qr_out);
    a.y[1] = static_cast<uint16_t*>(kv_out);
    a.w[0] = q_weight;
    a.w[1] = kv_weight;
    a.x_stride[0] = qr_stride;
    a.x_stride[1] = kv_stride;
    a.y_stride[0] = qr_out_stride;
    a.y_stride[1] = kv_out_stride;
    a.size[0] = (int32_t)q_size;
    a.size[1] = (int32_t)kv_size;
    a.num_rows = (uint32_t)num_tokens;
    a.q_blocks = (uint32_t)((num_tokens + kRowsPerBlock - 1) / kRowsPerBlock);
    a.eps = eps;
    a.weight_f32 = weight_is_fp32 ? 1 : 0;
    const dim3 grid(2 * a.q_blocks);
    const int64_t most = q_size > kv_size ? q_size : kv_size;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (most <= 512)
        hipLaunchKernelGGL(fused_q_kv_rmsnorm_kernel<4>, grid, dim3(kThreads), 0, s, a);
    else if (most <= 1536)
        hipLaunchKernelGGL(fused_q_kv_rmsnorm_kernel<12>, grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL(fused_q_kv_rmsnorm_kernel<32>, grid, dim3(kThreads), 0, s, a);
    return launch_status();
}
