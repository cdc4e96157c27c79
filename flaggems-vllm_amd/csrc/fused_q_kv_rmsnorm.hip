// gfx950 kernel for DeepSeek-V4's fused q/kv RMSNorm: two weighted RMSNorms
// (the q LoRA row and the kv latent row of each token) in one launch.
//
// Reference semantics: src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:24-103
//   y = (x * rsqrt(mean(x^2) + eps)) * w, stored in x's dtype (bf16).
//
// Layout: a row of up to 512 elements is one 16-lane DPP row (fgv_device.h),
// one of up to 1536 a half wave, a longer one a whole wave; lane l owns the
// 16-byte pieces l + L*j of its row, so DeepSeek-V4's 1536-wide q row is 6
// pieces on each of 32 lanes and its 512-wide kv row 4 pieces on each of 16.
// Workgroups [0, q_blocks) take q rows, the rest kv rows.  As in the main op
// the sum of squares is exact in binary64 and mean and rsqrt are correctly
// rounded, so results do not depend on the reduction order.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;

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

// Sum over the 64 lanes of the wave: DPP inside each 16-lane row, then the
// four row totals combined with two cross-row lane shuffles (ds_bpermute).
__device__ __forceinline__ double wave_sum(double v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Sum over each 32-lane half of the wave.
__device__ __forceinline__ double half_wave_sum(double v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16);
    return v;
}

// One row of kPieces * 16-byte pieces per lane over kLanes lanes (16: a DPP
// row, 32: a half wave, 64: the whole wave).
template <int kPieces, int kLanes>
__device__ __forceinline__ void rms_row(const RmsArgs& a, int which, uint32_t row, int lane) {
    if (row >= a.num_rows)
        return;
    const int size = a.size[which];
    const int pieces = size >> 3;
    const uint16_t* x = a.x[which] + (int64_t)row * a.x_stride[which];
    uint16_t* y = a.y[which] + (int64_t)row * a.y_stride[which];

    uint4 v[kPieces];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const int c = lane + kLanes * j;
        v[j] = c < pieces ? load16(x + c * 8) : make_uint4(0, 0, 0, 0);
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double lo = (double)bf16_lo(w4[i]), hi = (double)bf16_hi(w4[i]);
            s = __builtin_fma(lo, lo, s);
            s = __builtin_fma(hi, hi, s);
        }
    }
    s = kLanes == 64 ? wave_sum(s) : kLanes == 32 ? half_wave_sum(s) : row16_sum(s);
    float var = (float)(s / (double)size);
    var = var + a.eps;
    const float r = (float)(1.0 / __builtin_sqrt((double)var));

#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const int c = lane + kLanes * j;
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

// Workgroups [0, q_blocks) normalise q rows, the rest kv rows; each row kind
// has its own (pieces per lane, lanes per row) shape.
template <int kQP, int kQL, int kKP, int kKL>
__global__ void __launch_bounds__(kThreads)
fused_q_kv_rmsnorm_kernel(RmsArgs a) {
    if (blockIdx.x < a.q_blocks) {
        const uint32_t row = blockIdx.x * (kThreads / kQL) + threadIdx.x / kQL;
        rms_row<kQP, kQL>(a, 0, row, threadIdx.x % kQL);
    } else {
        const uint32_t row = (blockIdx.x - a.q_blocks) * (kThreads / kKL) + threadIdx.x / kKL;
        rms_row<kKP, kKL>(a, 1, row, threadIdx.x % kKL);
    }
}

// Row shapes (pieces per lane x lanes per row): up to 512 elements -> 4 x 16;
// up to 1536 -> 6 x 32; up to 2048 -> 4 x 64; up to 4096 -> 8 x 64.  The
// 32-lane shape keeps DeepSeek-V4's T = 8192 launch (q 1536, kv 512) inside one
// round of waves, 24 per CU: with a whole wave per 1536-wide row it took 10,240
// waves, 1.25 rounds of the 32 slots per CU, and 13.6 us against 9.8 us.
inline int shape_of(int64_t size) {
    return size <= 512 ? 0 : size <= 1536 ? 1 : size <= 2048 ? 2 : 3;
}
inline int lanes_of(int shape) { return shape == 0 ? 16 : shape == 1 ? 32 : 64; }

template <int kQP, int kQL>
void launch_kv_shape(const RmsArgs& a, int kv_shape, dim3 grid, hipStream_t st) {
    if (kv_shape == 0)
        hipLaunchKernelGGL((fused_q_kv_rmsnorm_kernel<kQP, kQL, 4, 16>), grid, dim3(kThreads), 0, st, a);
    else if (kv_shape == 1)
        hipLaunchKernelGGL((fused_q_kv_rmsnorm_kernel<kQP, kQL, 6, 32>), grid, dim3(kThreads), 0, st, a);
    else if (kv_shape == 2)
        hipLaunchKernelGGL((fused_q_kv_rmsnorm_kernel<kQP, kQL, 4, 64>), grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((fused_q_kv_rmsnorm_kernel<kQP, kQL, 8, 64>), grid, dim3(kThreads), 0, st, a);
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
    a.eps = eps;
    a.weight_f32 = weight_is_fp32 ? 1 : 0;
    const int qs = shape_of(q_size), ks = shape_of(kv_size);
    const int64_t q_rows_per_block = kThreads / lanes_of(qs);
    const int64_t kv_rows_per_block = kThreads / lanes_of(ks);
    a.q_blocks = (uint32_t)((num_tokens + q_rows_per_block - 1) / q_rows_per_block);
    const dim3 grid(a.q_blocks + (uint32_t)((num_tokens + kv_rows_per_block - 1) / kv_rows_per_block));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (qs == 0)
        launch_kv_shape<4, 16>(a, ks, grid, st);
    else if (qs == 1)
        launch_kv_shape<6, 32>(a, ks, grid, st);
    else if (qs == 2)
        launch_kv_shape<4, 64>(a, ks, grid, st);
    else
        launch_kv_shape<8, 64>(a, ks, grid, st);
    return launch_status();
}
