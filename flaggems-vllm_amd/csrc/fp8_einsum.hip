// gfx950 block-scaled FP8 einsum 'bhr,hdr->bhd': the grouped output
// projection that consumes fused_inv_rope_fp8_quant's e4m3fn activations and
// per-128 scales.
//
// Reference: src/flaggems_vllm/ops/fp8_einsum.py:20-115 (checks :41-97; the
// work goes to a Hopper block-FP8 batched GEMM), test
// tests/test_fp8_einsum.py:124-156 (the dequantise-then-einsum oracle):
//   out[b,h,d] = sum_r (x[b,h,r] xs[b,h,r/128]) (y[h,d,r] ys[h,d/128,r/128])
// with x, y e4m3fn, xs, ys float32, r and d multiples of 128, output bf16,
// fp16 or fp32.
//
// Each 128-wide K block is one v_mfma_f32_16x16x128_f8f6f4 per 16 x 16
// output tile: the MFMA forms the block's exact-input partial sum P (e4m3fn
// products are exact in binary32; the 128-term sum is binary32), and the
// accumulator takes P * (xs[row] * ys) with one FMA per element.  Register
// images (the same instruction as the sparse indexer's logits): lane
// (c, g) = (l % 16, l / 16) holds operand row c, bytes 16g..16g+15 and
// 64+16g..64+16g+15 of the K block; the accumulator holds output rows
// 4g..4g+3 of column c.
//
// Two kernels:
//   - skinny (b <= 64, b <= 128 with few heads, rows not 16-byte aligned,
//     or r = 0): fragments straight from memory into a ring of registers
//     (PD blocks in flight per wave), the K blocks dealt round-robin to KS
//     waves of a workgroup and their partials summed in LDS; y (the
//     weights) streams from HBM once, x is re-read from L2;
//   - tiled (larger b): 256 x 128 (or 128 x 128) output tiles over eight
//     (four) waves of 64 x 64, the K blocks' x and y tiles streamed through a
//     three-stage LDS ring by LDS DMA, two blocks ahead of the MFMAs (one
//     workgroup of eight waves per CU).
// The result depends only on the inputs: a fixed K-block order per wave and
// a fixed order over waves.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kBlockK = 128;   // K block (one scale block, one MFMA)
constexpr int kTile = 128;     // tiled kernel: output tile rows and columns
constexpr int kSkinnyRows = 128;  // b up to this may take the skinny kernel
// skinny configurations for b <= 16, <= 32 and larger: 16-column tiles per
// wave (NW), waves per workgroup splitting K (KS), blocks in flight per wave (PD)
constexpr int kSkinnyNW1 = 2, kSkinnyKS1 = 8, kSkinnyPD1 = 2;
constexpr int kSkinnyNW2 = 2, kSkinnyKS2 = 4, kSkinnyPD2 = 1;
constexpr int kSkinnyNW4 = 2, kSkinnyKS4 = 4, kSkinnyPD4 = 1;

struct EinsumArgs {
    const uint8_t* x;      // x[b, h, r] bytes, r contiguous
    int64_t x_sb, x_sh;
    const float* xs;       // xs[b, h, r / 128]
    int64_t xs_sb, xs_sh, xs_sk;
    const uint8_t* y;      // y[h, d, r] bytes, r contiguous
    int64_t y_sh, y_sd;
    const float* ys;       // ys[h, d / 128, r / 128]
    int64_t ys_sh, ys_sn, ys_sk;
    void* out;             // out[b, h, d] elements
    int64_t o_sb, o_sh, o_sd;
    int32_t b, h, d, nkb;  // nkb = r / 128
};

enum OutType { kOutBf16 = 0, kOutF16 = 1, kOutF32 = 2 };

__device__ __forceinline__ v4f_t mfma_fp8(v8i_t a, v8i_t b) {
    const v4f_t z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);  // zero scales: plain FP8 MFMA
}

// Lane (c, g)'s operand image of one K block of a row (row points at the block).
template <bool ALIGNED>
__device__ __forceinline__ v8i_t load_frag(const uint8_t* row, int g) {
    uint4 lo, hi;
    if constexpr (ALIGNED) {
        lo = *reinterpret_cast<const uint4*>(row + 16 * g);
        hi = *reinterpret_cast<const uint4*>(row + 64 + 16 * g);
    } else {
        __builtin_memcpy(&lo, row + 16 * g, 16);
        __builtin_memcpy(&hi, row + 64 + 16 * g, 16);
    }
    const v8i_t v = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return v;
}

__device__ __forceinline__ v8i_t lds_frag(const uint8_t* row, int g) {
    const uint4 lo = *reinterpret_cast<const uint4*>(row + 16 * g);
    const uint4 hi = *reinterpret_cast<const uint4*>(row + 64 + 16 * g);
    const v8i_t v = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return v;
}

template <int OUT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float v) {
    if constexpr (OUT == kOutBf16)
        reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
    else if constexpr (OUT == kOutF16)
        reinterpret_cast<_Float16*>(out)[i] = (_Float16)v;
    else
        reinterpret_cast<float*>(out)[i] = v;
}

// ---- skinny: rows m0 .. m0 + 16 MT of x (one workgroup row of the grid),
// columns n0 .. n0 + 16 NW of y, head blockIdx.z; wave w takes the K blocks
// w, w + KS, ...  A ring of PD register slots keeps PD blocks' fragments and
// scales in flight: a slot's block is used, then the slot loads the block PD
// turns later.
// With XT, the workgroup first stages its rows' xs for every K block in LDS
// (xt[kb][row], rows past b as 0), so that a K block's scales are one
// 16-byte LDS read per row tile instead of four global loads.
constexpr int kXsTableBlocks = 64;  // K blocks (r <= 8192) whose xs a workgroup stages in LDS

template <int MT, int NW, int KS, int PD, bool ALIGNED, bool XT, int OUT>
__global__ void __launch_bounds__(64 * KS) fp8_einsum_skinny_kernel(EinsumArgs a) {
    __shared__ v4f_t part[KS > 1 ? KS - 1 : 1][MT * NW][64];
    __shared__ __attribute__((aligned(16))) float xt[XT ? 16 * MT * kXsTableBlocks : 4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * NW;
    const int m0 = blockIdx.y * 16 * MT;
    const int hh = blockIdx.z;
    const uint8_t* arow[MT];
    bool aok[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int m = m0 + 16 * i + c;
        aok[i] = m < a.b;
        arow[i] = a.x + (int64_t)hh * a.x_sh + (int64_t)(aok[i] ? m : 0) * a.x_sb;
    }
    const uint8_t* brow[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j)
        brow[j] = a.y + (int64_t)hh * a.y_sh + (int64_t)(n0 + 16 * j + c) * a.y_sd;
    const float* ysp = a.ys + (int64_t)hh * a.ys_sh + (int64_t)(n0 / kBlockK) * a.ys_sn;
    // the lane's output rows m0 + 16 i + 4 g + q: their xs rows (row 0 stands in past b, scaled by 0)
    const float* xsh = a.xs + (int64_t)hh * a.xs_sh;
    int32_t xrow[MT][4];
    bool xok[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = m0 + 16 * i + 4 * g + q;
            xok[i][q] = m < a.b;
            xrow[i][q] = xok[i][q] ? m : 0;
        }

    if constexpr (XT) {
        constexpr int kRows = 16 * MT;
        for (int e = threadIdx.x; e < kRows * a.nkb; e += 64 * KS) {
            const int row = e % kRows, kb = e / kRows, m = m0 + row;
            xt[e] = m < a.b ? xsh[(int64_t)m * a.xs_sb + (int64_t)kb * a.xs_sk] : 0.f;
        }
        __syncthreads();
    }

    v4f_t acc[MT][NW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NW; ++j)
            acc[i][j] = v4f_t{0.f, 0.f, 0.f, 0.f};

    const v8i_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
    v8i_t A[PD][MT], B[PD][NW];
    float X[PD][MT][4], Y[PD];
    auto fetch = [&](int kb, int s) {
        const int64_t k0 = (int64_t)kb * kBlockK;
#pragma unroll
        for (int i = 0; i < MT; ++i)
            A[s][i] = aok[i] ? load_frag<ALIGNED>(arow[i] + k0, g) : zero;
#pragma unroll
        for (int j = 0; j < NW; ++j)
            B[s][j] = load_frag<ALIGNED>(brow[j] + k0, g);
        if constexpr (!XT) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    X[s][i][q] = xsh[(int64_t)xrow[i][q] * a.xs_sb + (int64_t)kb * a.xs_sk];
        }
        Y[s] = ysp[(int64_t)kb * a.ys_sk];
    };
    auto use = [&](int s, int kb) {
        float sx[MT][4];
        if constexpr (XT) {
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(&xt[kb * 16 * MT + 16 * i + 4 * g]);
                sx[i][0] = v.x * Y[s];
                sx[i][1] = v.y * Y[s];
                sx[i][2] = v.z * Y[s];
                sx[i][3] = v.w * Y[s];
            }
        } else {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    sx[i][q] = xok[i][q] ? X[s][i][q] * Y[s] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NW; ++j) {
                const v4f_t p = mfma_fp8(A[s][i], B[s][j]);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[i][j][q] = fmaf(p[q], sx[i][q], acc[i][j][q]);
            }
    };
#pragma unroll
    for (int s = 0; s < PD; ++s)
        if (w + s * KS < a.nkb)
            fetch(w + s * KS, s);
    for (int kb0 = w; kb0 < a.nkb; kb0 += PD * KS) {
#pragma unroll
        for (int s = 0; s < PD; ++s) {
            const int kb = kb0 + s * KS;
            if (kb < a.nkb) {
                use(s, kb);
                if (kb + PD * KS < a.nkb)
                    fetch(kb + PD * KS, s);  // PD blocks ahead
            }
        }
    }

    if constexpr (KS > 1) {
        if (w > 0) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NW; ++j)
                    part[w - 1][i * NW + j][lane] = acc[i][j];
        }
        __syncthreads();
        if (w != 0)
            return;
#pragma unroll
        for (int v = 0; v < KS - 1; ++v)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NW; ++j)
                    acc[i][j] += part[v][i * NW + j][lane];
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = m0 + 16 * i + 4 * g + q;
            if (m >= a.b)
                continue;
#pragma unroll
            for (int j = 0; j < NW; ++j)
                store_out<OUT>(a.out, (int64_t)m * a.o_sb + (int64_t)hh * a.o_sh + (int64_t)(n0 + 16 * j + c) * a.o_sd,
                               acc[i][j][q]);
        }
}

// ---- tiled: output tile (mt, nt) of head blockIdx.y, 64 MW rows x 128
// columns over 2 MW waves (64 x 64 each, MW along rows, 2 along columns); x
// and y rows 16-byte aligned, r > 0.  The K blocks stream through a ring of
// NS LDS stages by LDS DMA (global_load_lds_dwordx4: each wave
// instruction lands 64 lanes x 16 bytes = 8 rows contiguously), issued NS - 1
// blocks ahead of the MFMAs.  Rows are stored unpadded with their 16-byte
// chunks swizzled, chunk c of row r at (c ^ ((r >> 1) & 7)), so that the 16
// rows of a fragment read hit 16 distinct chunk slots.  Rows of x past b read
// row b - 1: they only feed outputs that are not stored.
constexpr int kStages4 = 3;  // LDS stages of the 256-row tiles (49 KB each)
constexpr int kStages2 = 3;  // LDS stages of the 128-row tiles (33 KB each)

// LDS DMA of 16 (4) bytes per lane: lane l's bytes land at LDS address
// lds + 16 l (4 l).  Issued as inline assembly so that the compiler, which
// cannot tell the stages apart, does not wait for every DMA in flight before
// each LDS read; the kernel waits for its own (vmcnt) and has no other vector
// memory loads in flight while DMAs are.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// s_waitcnt operand: vector memory operations outstanding <= n (expcnt and
// lgkmcnt not waited for; gfx9 encoding vmcnt bits 3:0 and 15:14).
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Workgroup barrier over LDS work only: __syncthreads' fence would wait for
// every outstanding LDS DMA, the next blocks' included; each wave waits for
// its own DMAs of the block explicitly before this.  The empty asm statements
// keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0): this wave's LDS accesses done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int MW>
struct TileShape {
    static constexpr int kRows = 64 * MW, kWaves = 2 * MW;
    static constexpr int kABytes = kRows * kBlockK, kBBytes = kTile * kBlockK;
    static constexpr int kXOff = kABytes + kBBytes, kYOff = kXOff + 4 * kRows;
    static constexpr int kStageBytes = kYOff + 256;  // + 64 copies of the block's ys
    static constexpr int kAInstr = kABytes / 1024 / kWaves, kBInstr = kBBytes / 1024 / kWaves;  // DMAs per wave per block
    static constexpr int kXInstr = kRows / 64;                                                   // xs: waves 0 .. kXInstr-1
    static constexpr int kYWave = kWaves - 1;                                                    // ys: the last wave
    static_assert(kAInstr >= 1 && kBInstr >= 1 && kXInstr < kWaves, "tile shape");
};

// Split K: with gridDim.z = S > 1, workgroup z takes K blocks
// [nkb z / S, nkb (z + 1) / S) and writes its fp32 tile to partial slot z of
// `part` ([S][b][h][d]) instead of the output; fp8_einsum_reduce_kernel sums
// the slots in order.
template <int MW, int NS, int OUT>
__global__ void __launch_bounds__(128 * MW) fp8_einsum_tile_kernel(EinsumArgs a, int32_t mtiles, float* part) {
    using S = TileShape<MW>;
    static_assert(NS >= 2 && NS <= 4, "two to four stages");
    // the NS stages, named statically by each step of the NS-unrolled loop
    __shared__ __attribute__((aligned(1024))) uint8_t st0[S::kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t st1[S::kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t st2[NS > 2 ? S::kStageBytes : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t st3[NS > 3 ? S::kStageBytes : 16];
    auto stage = [&](int i) -> uint8_t* { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int hh = blockIdx.y;
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int m0 = mt * S::kRows, n0 = nt * kTile;
    const int kb_lo = (int)((int64_t)a.nkb * blockIdx.z / gridDim.z);
    const int kb_hi = (int)((int64_t)a.nkb * (blockIdx.z + 1) / gridDim.z);

    // this lane's DMA sources: A instruction j of the wave covers tile rows
    // 8 (wave * kAInstr + j) + lane / 8, physical chunk lane % 8
    const int lrow = lane >> 3, lchunk = lane & 7;
    const uint8_t* asrc[S::kAInstr];
#pragma unroll
    for (int j = 0; j < S::kAInstr; ++j) {
        const int row = 8 * (wave * S::kAInstr + j) + lrow;
        const int m = min(m0 + row, a.b - 1);
        asrc[j] = a.x + (int64_t)hh * a.x_sh + (int64_t)m * a.x_sb + 16 * swz(row, lchunk);
    }
    const uint8_t* bsrc[S::kBInstr];
#pragma unroll
    for (int j = 0; j < S::kBInstr; ++j) {
        const int row = 8 * (wave * S::kBInstr + j) + lrow;
        bsrc[j] = a.y + (int64_t)hh * a.y_sh + (int64_t)(n0 + row) * a.y_sd + 16 * swz(row, lchunk);
    }
    const float* xsrc = a.xs + (int64_t)hh * a.xs_sh + (int64_t)min(m0 + 64 * wave + lane, a.b - 1) * a.xs_sb;
    const float* ysg = a.ys + (int64_t)hh * a.ys_sh + (int64_t)nt * a.ys_sn;
    // this wave's DMAs per block (the waitcnt operand while the next block flies)
    const bool xw = wave < S::kXInstr, yw = wave == S::kYWave;

    auto issue = [&](int kb, uint8_t* st) {
        const int64_t k0 = (int64_t)kb * kBlockK;
        const uint32_t base = lds_addr(st);
#pragma unroll
        for (int j = 0; j < S::kAInstr; ++j)
            dma16(asrc[j] + k0, base + 1024 * (wave * S::kAInstr + j));
#pragma unroll
        for (int j = 0; j < S::kBInstr; ++j)
            dma16(bsrc[j] + k0, base + S::kABytes + 1024 * (wave * S::kBInstr + j));
        if (xw)
            dma4(xsrc + (int64_t)kb * a.xs_sk, base + S::kXOff + 256 * wave);
        if (yw)
            dma4(ysg + (int64_t)kb * a.ys_sk, base + S::kYOff);
    };

    v4f_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = v4f_t{0.f, 0.f, 0.f, 0.f};

    // one K block: wait for this wave's DMAs of block kb (the next blocks'
    // may still fly), barrier (everyone's landed; the stage read in the
    // previous step is free), send block kb + NS - 1 into it, then the MFMAs
    // on `cur`
    constexpr int kPer = S::kAInstr + S::kBInstr;  // this wave's DMAs per block (+ 1 with a scale DMA)
    auto step = [&](int kb, const uint8_t* cur, uint8_t* nxt) {
        const int after = min(NS - 2, kb_hi - 1 - kb);  // blocks issued after kb
        if (after >= 2) {
            if (xw || yw)
                __builtin_amdgcn_s_waitcnt(wait_vm(2 * (kPer + 1)));
            else
                __builtin_amdgcn_s_waitcnt(wait_vm(2 * kPer));
        } else if (after == 1) {
            if (xw || yw)
                __builtin_amdgcn_s_waitcnt(wait_vm(kPer + 1));
            else
                __builtin_amdgcn_s_waitcnt(wait_vm(kPer));
        } else {
            __builtin_amdgcn_s_waitcnt(wait_vm(0));
        }
        lds_barrier();
        if (kb + NS - 1 < kb_hi)
            issue(kb + NS - 1, nxt);
        const float sy = reinterpret_cast<const float*>(cur + S::kYOff)[lane];
        v8i_t A[4], B[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = wm * 64 + 16 * i + c;
            const uint8_t* rp = cur + row * kBlockK;
            const uint4 lo = *reinterpret_cast<const uint4*>(rp + 16 * swz(row, g));
            const uint4 hi = *reinterpret_cast<const uint4*>(rp + 16 * swz(row, 4 + g));
            A[i] = v8i_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = wn * 64 + 16 * j + c;
            const uint8_t* rp = cur + S::kABytes + row * kBlockK;
            const uint4 lo = *reinterpret_cast<const uint4*>(rp + 16 * swz(row, g));
            const uint4 hi = *reinterpret_cast<const uint4*>(rp + 16 * swz(row, 4 + g));
            B[j] = v8i_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
        const float* xst = reinterpret_cast<const float*>(cur + S::kXOff);
        float sx[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(xst + wm * 64 + 16 * i + 4 * g);
            sx[i][0] = v.x * sy;
            sx[i][1] = v.y * sy;
            sx[i][2] = v.z * sy;
            sx[i][3] = v.w * sy;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v4f_t p = mfma_fp8(A[i], B[j]);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[i][j][q] = fmaf(p[q], sx[i][q], acc[i][j][q]);
            }
    };

#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
        if (kb_lo + j < kb_hi)
            issue(kb_lo + j, stage(j));
    for (int kb0 = kb_lo; kb0 < kb_hi; kb0 += NS) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
            if (kb0 + j < kb_hi)
                step(kb0 + j, stage(j), stage((j + NS - 1) % NS));
    }

    if (gridDim.z > 1) {
        float* ps = part + (int64_t)blockIdx.z * a.b * a.h * a.d;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = m0 + wm * 64 + 16 * i + 4 * g + q;
                if (m >= a.b)
                    continue;
                float* prow = ps + ((int64_t)m * a.h + hh) * a.d + n0 + wn * 64 + c;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    prow[16 * j] = acc[i][j][q];
            }
        return;
    }

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = m0 + wm * 64 + 16 * i + 4 * g + q;
            if (m >= a.b)
                continue;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                store_out<OUT>(a.out,
                               (int64_t)m * a.o_sb + (int64_t)hh * a.o_sh + (int64_t)(n0 + wn * 64 + 16 * j + c) * a.o_sd,
                               acc[i][j][q]);
        }
}

// out[m, h, n] = sum over z = 0 .. splits-1, in that order, of part[z][m][h][n]:
// four consecutive n per thread.
template <int OUT>
__global__ void __launch_bounds__(256) fp8_einsum_reduce_kernel(EinsumArgs a, const float* part, int32_t splits) {
    const int64_t slot = (int64_t)a.b * a.h * a.d, n4 = slot / 4;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n4; u += (int64_t)gridDim.x * blockDim.x) {
        float4 v = reinterpret_cast<const float4*>(part)[u];
        for (int z = 1; z < splits; ++z) {
            const float4 w = reinterpret_cast<const float4*>(part + z * slot)[u];
            v.x += w.x;
            v.y += w.y;
            v.z += w.z;
            v.w += w.w;
        }
        const int64_t e = 4 * u, row = e / a.d;
        const int n = (int)(e - row * a.d), hh = (int)(row % a.h);
        const int64_t m = row / a.h;
        const int64_t o = m * a.o_sb + (int64_t)hh * a.o_sh + (int64_t)n * a.o_sd;
        store_out<OUT>(a.out, o, v.x);
        store_out<OUT>(a.out, o + a.o_sd, v.y);
        store_out<OUT>(a.out, o + 2 * a.o_sd, v.z);
        store_out<OUT>(a.out, o + 3 * a.o_sd, v.w);
    }
}

template <int MT, int NW, int KS, int PD, bool ALIGNED, int OUT>
void launch_skinny(const EinsumArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)(a.d / (16 * NW)), (unsigned)((a.b + 16 * MT - 1) / (16 * MT)), (unsigned)a.h);
    if (a.nkb <= kXsTableBlocks)
        hipLaunchKernelGGL((fp8_einsum_skinny_kernel<MT, NW, KS, PD, ALIGNED, true, OUT>), grid, dim3(64 * KS), 0, st,
                           a);
    else
        hipLaunchKernelGGL((fp8_einsum_skinny_kernel<MT, NW, KS, PD, ALIGNED, false, OUT>), grid, dim3(64 * KS), 0,
                           st, a);
}

template <bool ALIGNED, int OUT>
void launch_skinny_rows(const EinsumArgs& a, hipStream_t st) {
    if (a.b <= 16)
        launch_skinny<1, kSkinnyNW1, kSkinnyKS1, kSkinnyPD1, ALIGNED, OUT>(a, st);
    else if (a.b <= 32)
        launch_skinny<2, kSkinnyNW2, kSkinnyKS2, kSkinnyPD2, ALIGNED, OUT>(a, st);
    else
        launch_skinny<4, kSkinnyNW4, kSkinnyKS4, kSkinnyPD4, ALIGNED, OUT>(a, st);
}

// Split-K for the 128-row tiles when they would cover at most half the CUs:
// enough splits for two workgroups per CU, at least kSplitMinBlocks K blocks
// each.  The partial tiles need splits * b * h * d fp32 of workspace.
// Measured (graph replay, bf16 out, unsplit -> split): pro (h 16, r 7168,
// d 1024) b 65 / 96 / 128 66 -> 48 / 53 / 57 us; flash (h 8, r 4096,
// d 1024) b 192 / 256 41 -> 37 / 40 us; with three splits (flash b 384) the
// partials' traffic made it slower (44 -> 60 us), hence the half-the-CUs
// condition.
constexpr int kSplitMinBlocks = 8;

int einsum_splits(int64_t b, int64_t h, int64_t nkb, int64_t d) {
    if (b <= 64 || nkb < 2 * kSplitMinBlocks)
        return 1;
    const int64_t tiles128 = ((b + 127) / 128) * (d / kTile) * h;
    const int64_t cus = cu_count();
    if (2 * tiles128 > cus)
        return 1;
    const int64_t want = (2 * cus + tiles128 - 1) / tiles128;
    return (int)std::min<int64_t>(want, nkb / kSplitMinBlocks);
}

int64_t einsum_workspace_bytes(int64_t b, int64_t h, int64_t nkb, int64_t d) {
    const int splits = einsum_splits(b, h, nkb, d);
    return splits > 1 ? ((int64_t)splits * b * h * d * 4 + 255) / 256 * 256 : 0;
}

template <int OUT>
int launch_einsum(const EinsumArgs& a, bool rows_aligned, void* workspace, int64_t workspace_bytes, hipStream_t st) {
    // skinny up to 64 rows, and up to 128 while 128-row tiles would fill
    // fewer than half the CUs (measured: flash b=128 skinny 31 us, tiled 39;
    // pro b=128 skinny 98 us, tiled 67); with a workspace, split-K tiles
    // take b > 64 whenever 128-row tiles would not fill the CUs
    const int64_t tiles128 = (int64_t)((a.b + 127) / 128) * (a.d / kTile) * a.h;
    const int splits = einsum_splits(a.b, a.h, a.nkb, a.d);
    const bool split = rows_aligned && splits > 1 && workspace && aligned(workspace, 16) &&
                       workspace_bytes >= einsum_workspace_bytes(a.b, a.h, a.nkb, a.d);
    const bool skinny = a.b <= 64 || (a.b <= kSkinnyRows && 2 * tiles128 < cu_count());
    if (split) {
        const int32_t mtiles = (a.b + 127) / 128;
        float* part = static_cast<float*>(workspace);
        hipLaunchKernelGGL((fp8_einsum_tile_kernel<2, kStages2, OUT>),
                           dim3((unsigned)(mtiles * (a.d / kTile)), (unsigned)a.h, (unsigned)splits), dim3(256), 0, st,
                           a, mtiles, part);
        const int64_t n4 = (int64_t)a.b * a.h * a.d / 4;
        const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, 8 * (int64_t)cu_count());
        hipLaunchKernelGGL(fp8_einsum_reduce_kernel<OUT>, dim3((unsigned)blocks), dim3(256), 0, st, a,
                           (const float*)part, (int32_t)splits);
    } else if (!rows_aligned)
        launch_skinny_rows<false, OUT>(a, st);
    else if (skinny || a.nkb == 0)
        launch_skinny_rows<true, OUT>(a, st);
    else {
        // 256-row tiles while they give every CU a workgroup, else 128 rows
        const int64_t tiles256 = (int64_t)((a.b + 255) / 256) * (a.d / kTile) * a.h;
        if (tiles256 >= cu_count()) {
            const int32_t mtiles = (a.b + 255) / 256;
            hipLaunchKernelGGL((fp8_einsum_tile_kernel<4, kStages4, OUT>),
                               dim3((unsigned)(mtiles * (a.d / kTile)), (unsigned)a.h), dim3(512), 0, st, a, mtiles,
                               nullptr);
        } else {
            const int32_t mtiles = (a.b + 127) / 128;
            hipLaunchKernelGGL((fp8_einsum_tile_kernel<2, kStages2, OUT>),
                               dim3((unsigned)(mtiles * (a.d / kTile)), (unsigned)a.h), dim3(256), 0, st, a, mtiles,
                               nullptr);
        }
    }
    return launch_status();
}

}  // namespace
}  // namespace fgv

extern "C" int64_t fgv_fp8_einsum_workspace_bytes(int64_t b, int64_t h, int64_t r, int64_t d) {
    if (b <= 0 || h <= 0 || r <= 0 || d <= 0 || r % fgv::kBlockK || d % fgv::kBlockK)
        return 0;
    return fgv::einsum_workspace_bytes(b, h, r / fgv::kBlockK, d);
}

extern "C" int fgv_fp8_einsum_bhr_hdr_ws(const uint8_t* x, int64_t x_sb, int64_t x_sh, const float* xs, int64_t xs_sb,
                                         int64_t xs_sh, int64_t xs_sk, const uint8_t* y, int64_t y_sh, int64_t y_sd,
                                         const float* ys, int64_t ys_sh, int64_t ys_sn, int64_t ys_sk, int64_t b,
                                         int64_t h, int64_t r, int64_t d, void* out, int64_t o_sb, int64_t o_sh,
                                         int64_t o_sd, int32_t out_dtype, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
    using namespace fgv;
    if (b < 0 || h < 0 || r < 0 || d < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (r % kBlockK || d % kBlockK)
        return fail(FGV_E_BAD_SHAPE, "r and d must be multiples of 128");
    if (out_dtype < kOutBf16 || out_dtype > kOutF32)
        return fail(FGV_E_BAD_SHAPE, "out_dtype must be 0 (bf16), 1 (fp16) or 2 (fp32)");
    if (b > 0x7fffffffLL || h > 65535 || r / kBlockK > 0x7fffffffLL || d > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "b, r and d must fit in int32 and h in 65535");
    if (b == 0 || h == 0 || d == 0)
        return FGV_OK;
    if (!out || (r > 0 && (!x || !xs || !y || !ys)))
        return fail(FGV_E_NULL_POINTER, "null tensor");
    const size_t osz = out_dtype == kOutF32 ? 4 : 2;
    if (!aligned(out, osz) || (r > 0 && (!aligned(xs, 4) || !aligned(ys, 4))))
        return fail(FGV_E_MISALIGNED, "out and scales must be aligned to their element size");
    EinsumArgs a{x,  x_sb,  x_sh,  xs,  xs_sb, xs_sh, xs_sk, y,          y_sh,       y_sd,      ys,
                 ys_sh, ys_sn, ys_sk, out, o_sb,  o_sh,  o_sd,  (int32_t)b, (int32_t)h, (int32_t)d, (int32_t)(r / kBlockK)};
    const bool al = aligned(x, 16) && aligned(y, 16) && x_sb % 16 == 0 && x_sh % 16 == 0 && y_sh % 16 == 0 &&
                    y_sd % 16 == 0;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    switch (out_dtype) {
    case kOutBf16:
        return launch_einsum<kOutBf16>(a, al, workspace, workspace_bytes, st);
    case kOutF16:
        return launch_einsum<kOutF16>(a, al, workspace, workspace_bytes, st);
    default:
        return launch_einsum<kOutF32>(a, al, workspace, workspace_bytes, st);
    }
}

extern "C" int fgv_fp8_einsum_bhr_hdr(const uint8_t* x, int64_t x_sb, int64_t x_sh, const float* xs, int64_t xs_sb,
                                      int64_t xs_sh, int64_t xs_sk, const uint8_t* y, int64_t y_sh, int64_t y_sd,
                                      const float* ys, int64_t ys_sh, int64_t ys_sn, int64_t ys_sk, int64_t b,
                                      int64_t h, int64_t r, int64_t d, void* out, int64_t o_sb, int64_t o_sh,
                                      int64_t o_sd, int32_t out_dtype, void* stream) {
    return fgv_fp8_einsum_bhr_hdr_ws(x, x_sb, x_sh, xs, xs_sb, xs_sh, xs_sk, y, y_sh, y_sd, ys, ys_sh, ys_sn, ys_sk, b,
                                     h, r, d, out, o_sb, o_sh, o_sd, out_dtype, nullptr, 0, stream);
}
