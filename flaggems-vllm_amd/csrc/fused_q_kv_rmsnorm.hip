// gfx950 kernel for DeepSeek-V4's fused q/kv RMSNorm: two weighted RMSNorms
// (the q LoRA row and the kv latent row of each token) in one launch.
//
// Reference semantics: src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:24-103
//   y = (x * rsqrt(mean(x^2) + eps)) * w, stored in x's dtype (bf16).
//
// Layout: a row of up to 512 elements is one 16-lane DPP row (fgv_device.h),
// one of up to 1536 a half wave, one of up to 4096 a whole wave; lane l owns
// the 16-byte pieces l + L*j of its row, so DeepSeek-V4's 1536-wide q row is
// 6 pieces on each of 32 lanes and its 512-wide kv row 4 pieces on each of 16.
// A longer row (the reference benchmark times 64 x 576-wide q rows) takes a
// whole workgroup, read from HBM once up to 49152 values (held in registers).
// Workgroups [0, q_blocks) take q rows, the rest kv rows.  As in the main op
// the sum of squares is accumulated in binary64, where each square of a bf16
// value is exact; the sum is exact too unless a row's squares span more than
// 37 - log2(size) binary orders of magnitude, and its rounding error
// (below size * 2^-53 relative) lies far under the binary32 rounding of the
// mean that follows.  Mean and rsqrt are correctly rounded, so the reduction
// order changes a result only if the mean falls within that error of a
// binary32 rounding boundary.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
// Workgroup size of launches whose 256-thread grid would leave CUs idle
// (short rows only): the same rows spread over four times the workgroups.
// DeepSeek-V4's shapes, per call: T = 32 2.88 -> 2.69 us, 128 3.16 -> 2.94,
// 256 3.40 -> 3.14, 512 3.56 -> 3.36.
constexpr int kSmallBlock = 64;

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

// The eight weights of one 16-byte piece of a row, as stored: one uint4 of
// bf16, or two of float.  The weight dtype is a template parameter and the
// loads take a clamped piece index, so every piece's weight load is issued
// before any is used (a run-time dtype test or a bounds branch around the load
// makes each wait out the one before).
struct WeightBits {
    uint4 a, b;
};

template <bool kF32>
__device__ __forceinline__ WeightBits load_weights8(const void* w, int e) {
    WeightBits r;
    if constexpr (kF32) {
        r.a = *reinterpret_cast<const uint4*>(static_cast<const float*>(w) + e);
        r.b = *reinterpret_cast<const uint4*>(static_cast<const float*>(w) + e + 4);
    } else {
        r.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e);
        r.b = make_uint4(0, 0, 0, 0);
    }
    return r;
}

template <bool kF32>
__device__ __forceinline__ void unpack_weights8(const WeightBits& r, float (&out)[8]) {
    if constexpr (kF32) {
        out[0] = __uint_as_float(r.a.x); out[1] = __uint_as_float(r.a.y);
        out[2] = __uint_as_float(r.a.z); out[3] = __uint_as_float(r.a.w);
        out[4] = __uint_as_float(r.b.x); out[5] = __uint_as_float(r.b.y);
        out[6] = __uint_as_float(r.b.z); out[7] = __uint_as_float(r.b.w);
    } else {
        out[0] = bf16_lo(r.a.x); out[1] = bf16_hi(r.a.x);
        out[2] = bf16_lo(r.a.y); out[3] = bf16_hi(r.a.y);
        out[4] = bf16_lo(r.a.z); out[5] = bf16_hi(r.a.z);
        out[6] = bf16_lo(r.a.w); out[7] = bf16_hi(r.a.w);
    }
}

// y = (x * r) * w for the eight values of one piece, packed to bf16.
__device__ __forceinline__ uint4 scale_piece(const uint4& x, float r, const float (&wv)[8]) {
    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = (bf16_lo(w4[i]) * r) * wv[2 * i];
        const float hi = (bf16_hi(w4[i]) * r) * wv[2 * i + 1];
        o[i] = pack_bf16x2(lo, hi);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
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

__device__ __forceinline__ double sum_squares(const uint4& v, double s) {
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const double lo = (double)bf16_lo(w4[i]), hi = (double)bf16_hi(w4[i]);
        s = __builtin_fma(lo, lo, s);
        s = __builtin_fma(hi, hi, s);
    }
    return s;
}

// 1 / sqrt(mean + eps) from the exact binary64 sum of squares of a row.
__device__ __forceinline__ float inv_rms(double s, int size, float eps) {
    float var = (float)(s / (double)size);
    var = var + eps;
    return (float)(1.0 / __builtin_sqrt((double)var));
}

// One row of kPieces * 16-byte pieces per lane over kLanes lanes (16: a DPP
// row, 32: a half wave, 64: the whole wave).  With kHoist every piece's weight
// load is issued before the reduction, so a lane waits on one L2 round trip
// for all of them; without it the compiler moves each weight load into its
// piece's bounds-checked store, one round trip per piece, in fewer registers
// (the launch picks kHoist only when the grid is small enough that the lost
// occupancy costs nothing).
template <int kPieces, int kLanes, bool kF32, bool kHoist>
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
    for (int j = 0; j < kPieces; ++j)
        s = sum_squares(v[j], s);
    WeightBits wb[kHoist ? kPieces : 1];
    if constexpr (kHoist) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j)
            wb[j] = load_weights8<kF32>(a.w[which], min(lane + kLanes * j, pieces - 1) * 8);
    }
    s = kLanes == 64 ? wave_sum(s) : kLanes == 32 ? half_wave_sum(s) : row16_sum(s);
    const float r = inv_rms(s, size, a.eps);

#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const int c = lane + kLanes * j;
        float wv[8];
        if constexpr (kHoist) {
            unpack_weights8<kF32>(wb[j], wv);
            const uint4 o = scale_piece(v[j], r, wv);
            if (c < pieces)
                store16(y + c * 8, o);
        } else if (c < pieces) {
            unpack_weights8<kF32>(load_weights8<kF32>(a.w[which], c * 8), wv);
            store16(y + c * 8, scale_piece(v[j], r, wv));
        }
    }
}

// Loads the pieces base + tid + kThreads*j of a row (zeros past its end),
// all loads issued before any is used.
template <int kLP>
__device__ __forceinline__ void load_chunk(const uint16_t* x, int base, int tid, int pieces, uint4 (&v)[kLP]) {
#pragma unroll
    for (int j = 0; j < kLP; ++j) {
        const int c = base + tid + kThreads * j;
        v[j] = c < pieces ? load16(x + c * 8) : make_uint4(0, 0, 0, 0);
    }
}

// Normalises and stores one chunk, eight pieces at a time, from the first
// group's weights in wb (load_group0); the next group's weight loads are
// issued before this group's stores.
// The weights of a chunk's first eight pieces (store_chunk's first group).
template <bool kF32>
__device__ __forceinline__ void load_group0(const void* w, int base, int tid, int pieces, WeightBits (&wb)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        wb[j] = load_weights8<kF32>(w, min(base + tid + kThreads * j, pieces - 1) * 8);
}

template <int kLP, bool kF32>
__device__ __forceinline__ void store_chunk(const void* w, uint16_t* y, int base, int tid, int pieces, float r,
                                            uint4 (&v)[kLP], WeightBits (&wb)[8]) {
    static_assert(kLP % 8 == 0, "pieces are stored in groups of eight");
#pragma unroll
    for (int g = 0; g < kLP; g += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float wv[8];
            unpack_weights8<kF32>(wb[j], wv);
            v[g + j] = scale_piece(v[g + j], r, wv);
        }
        if (g + 8 < kLP) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                wb[j] = load_weights8<kF32>(w, min(base + tid + kThreads * (g + 8 + j), pieces - 1) * 8);
        }
#pragma unroll
        for (int j = g; j < g + 8; ++j) {
            const int c = base + tid + kThreads * j;
            if (c < pieces)
                store16(y + c * 8, v[j]);
        }
    }
}

// A row of more than 4096 elements takes the whole workgroup: thread t owns
// pieces t + 256*j.  The first kThreads * kLP pieces stay in registers between
// the sum and the output (kLP 8: rows up to 16384 values; 24: up to 49152);
// pieces past them are read in chunks of that size for the sum and again for
// the output.  The four wave sums are added in a fixed order through LDS.
template <int kLP, bool kF32>
__device__ __forceinline__ void rms_row_long(const RmsArgs& a, int which, uint32_t row, int tid,
                                             double (&red)[kThreads / 64]) {
    const int size = a.size[which];
    const int pieces = size >> 3;
    const uint16_t* x = a.x[which] + (int64_t)row * a.x_stride[which];
    uint16_t* y = a.y[which] + (int64_t)row * a.y_stride[which];
    constexpr int kChunk = kThreads * kLP;

    uint4 v[kLP];
    load_chunk<kLP>(x, 0, tid, pieces, v);
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kLP; ++j)
        s = sum_squares(v[j], s);
    for (int base = kChunk; base < pieces; base += kChunk) {
        uint4 t[kLP];
        load_chunk<kLP>(x, base, tid, pieces, t);
#pragma unroll
        for (int j = 0; j < kLP; ++j)
            s = sum_squares(t[j], s);
    }
    // With 24 pieces per thread the first group's weights load under the
    // reduction (the reference benchmark's 36864-wide rows: 6.67 -> 6.39 us
    // at 32 rows); the 8-piece kernel, which runs several rounds of
    // workgroups, loses occupancy to those registers and loads them after it.
    WeightBits wb[8];
    if constexpr (kLP > 8)
        load_group0<kF32>(a.w[which], 0, tid, pieces, wb);
    s = wave_sum(s);
    if ((tid & 63) == 0)
        red[tid >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = inv_rms(s, size, a.eps);
    if constexpr (kLP <= 8)
        load_group0<kF32>(a.w[which], 0, tid, pieces, wb);

    store_chunk<kLP, kF32>(a.w[which], y, 0, tid, pieces, r, v, wb);
    for (int base = kChunk; base < pieces; base += kChunk) {
        uint4 t[kLP];
        load_chunk<kLP>(x, base, tid, pieces, t);
        load_group0<kF32>(a.w[which], base, tid, pieces, wb);
        store_chunk<kLP, kF32>(a.w[which], y, base, tid, pieces, r, t, wb);
    }
}

// Workgroups [0, q_blocks) normalise q rows, the rest kv rows; each row kind
// has its own (pieces per lane, lanes per row) shape, lanes kThreads meaning
// a workgroup per row (rms_row_long, pieces per lane then its kLP).
template <int kQP, int kQL, int kKP, int kKL, bool kF32, bool kHoist, int kBlock = kThreads>
__global__ void __launch_bounds__(kBlock)
fused_q_kv_rmsnorm_kernel(RmsArgs a) {
    static_assert(kBlock == kThreads || (kQL != kThreads && kKL != kThreads),
                  "long rows take 256-thread workgroups");
    __shared__ double red[kThreads / 64];
    if (blockIdx.x < a.q_blocks) {
        if constexpr (kQL == kThreads) {
            rms_row_long<kQP, kF32>(a, 0, blockIdx.x, threadIdx.x, red);
        } else {
            const uint32_t row = blockIdx.x * (kBlock / kQL) + threadIdx.x / kQL;
            rms_row<kQP, kQL, kF32, kHoist>(a, 0, row, threadIdx.x % kQL);
        }
    } else {
        if constexpr (kKL == kThreads) {
            rms_row_long<kKP, kF32>(a, 1, blockIdx.x - a.q_blocks, threadIdx.x, red);
        } else {
            const uint32_t row = (blockIdx.x - a.q_blocks) * (kBlock / kKL) + threadIdx.x / kKL;
            rms_row<kKP, kKL, kF32, kHoist>(a, 1, row, threadIdx.x % kKL);
        }
    }
}

// Row shapes (pieces per lane x lanes per row): up to 512 elements -> 4 x 16;
// up to 1536 -> 6 x 32; up to 2048 -> 4 x 64; up to 4096 -> 8 x 64; longer ->
// a workgroup per row, 8 pieces per thread in registers up to 16384 values and
// 24 beyond.  The 32-lane shape keeps DeepSeek-V4's T = 8192 launch (q 1536,
// kv 512) inside one round of waves, 24 per CU: with a whole wave per
// 1536-wide row it took 10,240 waves, 1.25 rounds of the 32 slots per CU, and
// 13.6 us against 9.8 us.
inline int shape_of(int64_t size) {
    return size <= 512 ? 0 : size <= 1536 ? 1 : size <= 2048 ? 2 : size <= 4096 ? 3 : size <= 16384 ? 4 : 5;
}
inline int lanes_of(int shape) { return shape == 0 ? 16 : shape == 1 ? 32 : shape <= 3 ? 64 : kThreads; }
constexpr int64_t kMaxRowSize = 1 << 24;

// The hoisted weight loads (rms_row's kHoist) take registers: up to two
// workgroups per CU they are free, above that the lower-occupancy kernel loses
// (DeepSeek-V4's T = 8192 launch: 13.4 us hoisted, 11.3 us not).
constexpr int kHoistMaxBlocksPerCu = 2;

// A grid larger than one round of resident workgroups runs 2-5 % faster with
// fewer of them per CU: the launch then reserves 40 KiB of LDS per workgroup
// (the kernel uses 32 bytes), four per CU.  DeepSeek-V4's shapes, q 1536 and
// kv 512, per call: T = 16384 25.0 -> 24.0 us, 24576 36.2 -> 34.6, 65536
// 91.4 -> 87.1; a one-round grid (T = 8192: 11.3 us) would take 13.3 us
// capped, so it is launched without the reservation, and so is a kernel that
// holds no more than four per CU anyway (the long rows' kernels).
constexpr size_t kMultiRoundLds = 40 << 10;
constexpr int kCappedPerCu = (160 << 10) / kMultiRoundLds;

// Workgroups of `kernel` one CU holds at once (registers and static LDS),
// asked once per instantiation; 0 if the runtime cannot tell (then no cap).
template <typename Kernel>
int resident_per_cu(Kernel kernel, int block) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, 0) != hipSuccess)
        return 0;
    return n;
}

template <int kQP, int kQL, int kKP, int kKL, bool kF32, bool kHoist, int kBlock = kThreads>
void launch_one(const RmsArgs& a, dim3 grid, hipStream_t st) {
    const auto kernel = fused_q_kv_rmsnorm_kernel<kQP, kQL, kKP, kKL, kF32, kHoist, kBlock>;
    static const int resident = resident_per_cu(kernel, kBlock);
    const bool cap = resident > kCappedPerCu && grid.x > (uint32_t)(resident * cu_count());
    hipLaunchKernelGGL(kernel, grid, dim3(kBlock), cap ? kMultiRoundLds : 0, st, a);
}

// small: the grid is in kSmallBlock-thread workgroups (short rows only,
// always with the weight loads hoisted).
template <int kQP, int kQL, int kKP, int kKL>
void launch_kernel(const RmsArgs& a, bool hoist, bool small, dim3 grid, hipStream_t st) {
    constexpr bool kAnyShort = kQL != kThreads || kKL != kThreads;
    if constexpr (kQL != kThreads && kKL != kThreads) {
        if (small) {
            if (a.weight_f32)
                launch_one<kQP, kQL, kKP, kKL, true, true, kSmallBlock>(a, grid, st);
            else
                launch_one<kQP, kQL, kKP, kKL, false, true, kSmallBlock>(a, grid, st);
            return;
        }
    }
    if (a.weight_f32) {
        if (kAnyShort && hoist)
            launch_one<kQP, kQL, kKP, kKL, true, kAnyShort>(a, grid, st);
        else
            launch_one<kQP, kQL, kKP, kKL, true, false>(a, grid, st);
    } else {
        if (kAnyShort && hoist)
            launch_one<kQP, kQL, kKP, kKL, false, kAnyShort>(a, grid, st);
        else
            launch_one<kQP, kQL, kKP, kKL, false, false>(a, grid, st);
    }
}

template <int kQP, int kQL>
void launch_kv_shape(const RmsArgs& a, int kv_shape, bool hoist, bool small, dim3 grid, hipStream_t st) {
    switch (kv_shape) {
    case 0: launch_kernel<kQP, kQL, 4, 16>(a, hoist, small, grid, st); break;
    case 1: launch_kernel<kQP, kQL, 6, 32>(a, hoist, small, grid, st); break;
    case 2: launch_kernel<kQP, kQL, 4, 64>(a, hoist, small, grid, st); break;
    case 3: launch_kernel<kQP, kQL, 8, 64>(a, hoist, small, grid, st); break;
    case 4: launch_kernel<kQP, kQL, 8, kThreads>(a, hoist, small, grid, st); break;
    default: launch_kernel<kQP, kQL, 24, kThreads>(a, hoist, small, grid, st); break;
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
    if (q_size > kMaxRowSize || kv_size > kMaxRowSize)
        return fail(FGV_E_TOO_LARGE, "row sizes above 2^24 are not supported");
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
    const int64_t cus = cu_count();
    // q blocks and the whole grid for workgroups of `block` threads
    auto blocks = [&](int block, uint32_t& q_blocks) {
        const int64_t q_rows = block / lanes_of(qs), kv_rows = block / lanes_of(ks);
        q_blocks = (uint32_t)((num_tokens + q_rows - 1) / q_rows);
        return (int64_t)q_blocks + (num_tokens + kv_rows - 1) / kv_rows;
    };
    int64_t grid_blocks = blocks(kThreads, a.q_blocks);
    const bool small = lanes_of(qs) < kThreads && lanes_of(ks) < kThreads && grid_blocks < cus;
    if (small)
        grid_blocks = blocks(kSmallBlock, a.q_blocks);
    const dim3 grid((uint32_t)grid_blocks);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool hoist = small || grid_blocks <= kHoistMaxBlocksPerCu * cus;
    switch (qs) {
    case 0: launch_kv_shape<4, 16>(a, ks, hoist, small, grid, st); break;
    case 1: launch_kv_shape<6, 32>(a, ks, hoist, small, grid, st); break;
    case 2: launch_kv_shape<4, 64>(a, ks, hoist, small, grid, st); break;
    case 3: launch_kv_shape<8, 64>(a, ks, hoist, small, grid, st); break;
    case 4: launch_kv_shape<8, kThreads>(a, ks, hoist, small, grid, st); break;
    default: launch_kv_shape<24, kThreads>(a, ks, hoist, small, grid, st); break;
    }
    return launch_status();
}
