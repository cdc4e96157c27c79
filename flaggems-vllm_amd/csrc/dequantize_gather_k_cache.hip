// gfx950 kernel for dequantize_and_gather_k_cache: read each request's last
// gather_len tokens out of the paged FP8 cache that
// qnorm_rope_kv_insert_kernel writes, and expand them to bf16 rows.
//
// Reference semantics: src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:38-172
//   out[r, offset + i, :nope]          = bf16(e4m3(code) * 2^(scale_byte - 127))
//   out[r, offset + i, nope:nope+rope] = the cached bf16 rope values
// for i < gather_len[r], position seq_len[r] - gather_len[r] + i, block
// block_table[r, pos / bs].  Columns past nope + rope are not touched.
//
// Same row ownership as the other kernels (fgv_device.h): one output row per
// 16-lane DPP row, 8 output elements (16 bytes) per lane per step.  The
// decode is exact: an e4m3 value times a power of two fits bf16 unless it
// leaves bf16's exponent range.  The DeepSeek-V4 geometry (448 + 64, 8 scale
// bytes per token) is a compile-time specialisation with one 8-byte load of
// the token's scale bytes; other geometries use the same code with runtime
// sizes.
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 16;
constexpr int kSmallBlock = 64;
// Dynamic LDS reserved per workgroup (the kernel uses none) to cap the launch
// at four workgroups, 16 waves, per CU (160 KiB of LDS).  On c2's 114,967
// whole-sequence rows: none 34.0 us, 24 KiB 33.3, 32-40 KiB 32.5, 52 KiB 34.4,
// 64 KiB and above 39.6.
constexpr size_t kOccupancyLds = 40 * 1024;

struct GatherArgs {
    uint16_t* out;
    const uint8_t* cache;
    const int32_t* seq_lens;
    const int32_t* gather_lens;  // may be null: gather the whole sequence
    const int32_t* block_table;
    int64_t out_s0, out_s1;
    int64_t block_stride, num_blocks;
    int64_t bt_stride;
    int32_t max_blocks, rows_bound, offset;
    int32_t block_size, nope, rope, scale_slots;
};

// 2^(b - 127) for a UE8M0 byte, exactly (b = 0 is the subnormal 2^-127,
// b = 255 is +inf, as exp2 gives).
__device__ __forceinline__ float ue8m0_value(uint32_t b) {
    return __uint_as_float(b ? (b << 23) : 0x00400000u);
}

// Eight e4m3fn codes (two dwords) times a scale, packed to bf16x8.
__device__ __forceinline__ uint4 decode8(uint32_t lo, uint32_t hi, float sc) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
    f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
    f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
    f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
    return make_uint4(pack_bf16x2(a.x * sc, a.y * sc), pack_bf16x2(b.x * sc, b.y * sc),
                      pack_bf16x2(c.x * sc, c.y * sc), pack_bf16x2(d.x * sc, d.y * sc));
}

__device__ __forceinline__ uint2 load8(const void* p) {
    u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_uint2(v.x, v.y);
}

template <bool kDsv4, int kBlock = kThreads>
__global__ void __launch_bounds__(kBlock)
dequantize_gather_kernel(GatherArgs a) {
    const int lane16 = threadIdx.x & 15;
    const int r = blockIdx.y;
    const int32_t i = blockIdx.x * (kBlock / 16) + (threadIdx.x >> 4);
    const int32_t seq_len = a.seq_lens[r];
    const int32_t gl = a.gather_lens ? a.gather_lens[r] : seq_len;
    if (i >= gl || i >= a.rows_bound)
        return;
    const int32_t pos = seq_len - gl + i;
    if (pos < 0)
        return;
    const int32_t bs = a.block_size;
    const int32_t bis = pos / bs;
    if (bis >= a.max_blocks)
        return;
    const int64_t blk = a.block_table[(int64_t)r * a.bt_stride + bis];
    if (blk < 0 || blk >= a.num_blocks)
        return;
    const int32_t pib = pos - bis * bs;
    const int nope = kDsv4 ? kNopeDim : a.nope;
    const int rope = kDsv4 ? kRopeDim : a.rope;
    const int slots = kDsv4 ? kScaleBytesPerToken : a.scale_slots;
    const int token_bytes = nope + 2 * rope;
    const uint8_t* base = a.cache + blk * a.block_stride;
    const uint8_t* tok = base + (int64_t)pib * token_bytes;
    const uint8_t* scl = base + (int64_t)bs * token_bytes + (int64_t)pib * slots;
    uint16_t* out = a.out + (int64_t)r * a.out_s0 + (int64_t)(a.offset + i) * a.out_s1;

    const int chunks = (nope + rope) / 8;
    const int nope_chunks = nope / 8;
    if (kDsv4) {
        // All loads of the row are issued before any store (byte pointers
        // would otherwise pin each load behind the previous store), and piece
        // 3 takes one load shape for both its halves so no lane diverges.
        const uint2 sbytes = load8(scl);  // the 7 group bytes + pad
        uint2 in[3];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            in[k] = load8(tok + (lane16 + 16 * k) * 8);
        // Piece 3 without divergence: lanes 0..7 read codes 384..447 (8 bytes
        // used of 16), lanes 8..15 read the 16 bytes of rope values 4*(l-8)..+3;
        // both stay inside the 576 token bytes.
        const uint8_t* p3 = lane16 < 8 ? tok + 384 + 8 * lane16 : tok + kNopeDim + 16 * (lane16 - 8);
        const uint2 in3a = load8(p3), in3b = load8(p3 + 8);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int g = 2 * k + (lane16 >> 3);
            const uint32_t b = ((g < 4 ? sbytes.x : sbytes.y) >> (8 * (g & 3))) & 0xffu;
            store16(out + (lane16 + 16 * k) * 8, decode8(in[k].x, in[k].y, ue8m0_value(b)));
        }
        const uint4 dec6 = decode8(in3a.x, in3a.y, ue8m0_value((sbytes.y >> 16) & 0xffu));
        const uint4 v3 = lane16 < 8 ? dec6 : make_uint4(in3a.x, in3a.y, in3b.x, in3b.y);
        store16(out + (lane16 + 48) * 8, v3);
        return;
    }
    for (int c = lane16; c < chunks; c += 16) {
        const int e = c * 8;
        uint4 v;
        if (c < nope_chunks) {
            const uint2 codes = load8(tok + e);
            v = decode8(codes.x, codes.y, ue8m0_value(scl[e >> 6]));
        } else {
            const uint8_t* src = tok + nope + 2 * (e - nope);
            const uint2 lo = load8(src), hi = load8(src + 8);
            v = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
        store16(out + e, v);
    }
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_dequantize_and_gather_k_cache(
    void* out, int64_t out_stride_req, int64_t out_stride_row, int64_t out_rows,
    const void* k_cache, int64_t cache_block_stride, int64_t num_blocks,
    const int32_t* seq_lens, const int32_t* gather_lens,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_seq,
    int64_t num_reqs, int64_t block_size, int64_t offset,
    int64_t nope_dim, int64_t rope_dim, int64_t scale_slots,
    void* stream) {
    using namespace fgv;
    if (num_reqs < 0 || out_rows < 0 || offset < 0 || block_size <= 0 || max_blocks_per_seq < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size, offset or non-positive block_size");
    const int64_t rows_bound = out_rows - offset;
    if (num_reqs == 0 || rows_bound <= 0)
        return FGV_OK;
    if (num_reqs > 65535)
        return fail(FGV_E_TOO_LARGE, "at most 65535 requests per call");
    if (out_rows > 0x7fffffffLL || max_blocks_per_seq > 0x7fffffffLL ||
        (int64_t)max_blocks_per_seq * block_size > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "sequence geometry must fit in int32");
    if (!out || !k_cache || !seq_lens || !block_table)
        return fail(FGV_E_NULL_POINTER, "null out, k_cache, seq_lens or block_table");
    if (nope_dim < 0 || rope_dim < 0 || nope_dim % 8 || rope_dim % 8 || nope_dim + rope_dim == 0)
        return fail(FGV_E_BAD_SHAPE, "nope_dim and rope_dim must be multiples of 8");
    if (scale_slots < (nope_dim + 63) / 64)
        return fail(FGV_E_BAD_SHAPE, "scale_slots is below the number of 64-element groups");
    if (!aligned(out, 16) || out_stride_req % 8 || out_stride_row % 8)
        return fail(FGV_E_MISALIGNED, "out must be 16-byte aligned with strides multiple of 8");
    if (!aligned(k_cache, 8) || cache_block_stride % 8)
        return fail(FGV_E_MISALIGNED, "k_cache and its block stride must be 8-byte aligned");
    const int64_t token_bytes = nope_dim + 2 * rope_dim;
    if (cache_block_stride < block_size * (token_bytes + scale_slots))
        return fail(FGV_E_BAD_STRIDE, "k_cache block stride is below block_size * token bytes");

    GatherArgs a;
    a.out = static_cast<uint16_t*>(out);
    a.cache = static_cast<const uint8_t*>(k_cache);
    a.seq_lens = seq_lens;
    a.gather_lens = gather_lens;
    a.block_table = block_table;
    a.out_s0 = out_stride_req;
    a.out_s1 = out_stride_row;
    a.block_stride = cache_block_stride;
    a.num_blocks = num_blocks;
    a.bt_stride = block_table_stride;
    a.max_blocks = (int32_t)max_blocks_per_seq;
    a.rows_bound = (int32_t)rows_bound;
    a.offset = (int32_t)offset;
    a.block_size = (int32_t)block_size;
    a.nope = (int32_t)nope_dim;
    a.rope = (int32_t)rope_dim;
    a.scale_slots = (int32_t)scale_slots;
    const bool dsv4 = nope_dim == kNopeDim && rope_dim == kRopeDim &&
                      scale_slots == kScaleBytesPerToken;
    const dim3 grid((unsigned)((rows_bound + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)num_reqs);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if ((int64_t)grid.x * grid.y < cu_count()) {
        // fewer workgroups than CUs: the rows over 64-thread workgroups
        // (four times as many, one round, so no LDS reservation)
        const dim3 small((unsigned)((rows_bound + kSmallBlock / 16 - 1) / (kSmallBlock / 16)), (unsigned)num_reqs);
        if (dsv4)
            hipLaunchKernelGGL((dequantize_gather_kernel<true, kSmallBlock>), small, dim3(kSmallBlock), 0, st, a);
        else
            hipLaunchKernelGGL((dequantize_gather_kernel<false, kSmallBlock>), small, dim3(kSmallBlock), 0, st, a);
        return launch_status();
    }
    if (dsv4)
        hipLaunchKernelGGL(dequantize_gather_kernel<true>, grid, dim3(kThreads), kOccupancyLds, st, a);
    else
        hipLaunchKernelGGL(dequantize_gather_kernel<false>, grid, dim3(kThreads), kOccupancyLds, st, a);
    return launch_status();
}
