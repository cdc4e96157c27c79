// gfx950 kernel for sparse MLA decode over the 584-byte MODEL1 cache: each
// query row attends the top-k cache entries its indices select, K = V = the
// dequantised 512-wide latent of each entry (448 e4m3 NoPE values with one
// E8M0 scale per 64, then 64 bf16 RoPE values).
//
// Reference semantics: src/flaggems_vllm/ops/flash_mla_with_kvcache.py:489-688
// (portable MODEL1 kernel) and src/flaggems_vllm/ops/flash_mla_with_kvcache_model1.py:389-470,
// 699-720 (sm90 kernel: mask, epilogue, attention sink).
//
// One workgroup of 4 waves per (batch row, query position, 64-head block);
// wave w owns heads 16w..16w+15 and keeps their q (B operand) and fp32 O^T
// accumulators in registers.  The selected entries of the main list, then of
// the extra list, stream through in chunks of 32 with a three-stage pipeline:
//   - the index each lane needs for chunk c+2 is loaded into a register,
//   - the raw 576 token bytes and 8 scale bytes of each entry of chunk c+1 are
//     gathered straight into LDS (global_load_lds_dwordx4: no registers, no
//     wait), into the other half of a double buffer; 8 lanes move one entry,
//     so each lane resolves one index per chunk,
//   - chunk c, gathered one iteration earlier, is dequantised from LDS into a
//     bf16 K tile [32 entries][512] (v_cvt_scalef32_pk_bf16_fp8: e4m3 times a
//     power of two, exact) and attended:
//       S^T = K q^T on v_mfma_f32_16x16x32_bf16 (A = K rows, B = q), giving
//         each lane one head and 8 entries of the chunk;
//       online softmax in base 2 per head (row-swapping permutes) against
//         a reference maximum that is only raised, and O rescaled, when a
//         score exceeds it by more than 2^8 (so probabilities stay below
//         256); the probabilities, rounded to bf16, are the B operand of
//       O^T += V^T P^T, whose A operand (V^T = K^T) is read from the same K
//         tile with ds_read_b64_tr_b16 transposing loads.
// An extra list that is gathered many times per cache entry can instead be
// dequantised once per call into bf16 rows in the workspace
// (mla_expand_cache_kernel); its chunks are then DMA'd straight into a K tile,
// alternating between the K tile and the (then idle) raw gather buffers, with
// no conversion and one barrier per chunk.
// K tile rows are 1056 bytes apart (1024 + 32), so that the row reads of QK,
// the transposing reads of PV and the row writes are all free of LDS bank
// conflicts (measured), while each lane's QK and PV addresses stay one base
// plus constant offsets.  Entries that are
// not attended (past the top-k length, negative, or past the cache) are
// gathered from a zero page, and their scores masked to -inf.
//
// Which workgroup takes which item depends on the grid (C = CUs): up to C
// workgroups, items in runs per XCD; up to 2C (workgroups j and C + j share
// a CU), windows rank their items by list cost, pair long with short, and
// give the workgroups alone on their CU the longest; up to 4C, windows of 256
// take their items longest first.  No result bit depends on the order: every
// item is computed the same way.
//
// The sparse prefill over bf16 rows (flash_mla_sparse_fwd,
// sparse_mla_prefill_kernel near the end of the kernels) reuses the attend
// routine and the row DMAs: its rows need no dequantisation, d_qk may be 576
// (a 64-dim tail that enters the scores only) and it also reports the largest
// score per head.
#include <math.h>

#include <mutex>

#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;
constexpr int kBlockHeads = 64;
constexpr int kChunk = 32;                                    // entries per chunk
constexpr int kPieces = kTokenDataBytes / 16;                 // 36 16-byte pieces per entry
constexpr int kGathers = (kPieces + 7) / 8;                   // 5 wave-wide gathers per wave and chunk
// Raw chunk layout in LDS: gather n of wave w lands at n * kRegion + 1024 w,
// i.e. piece k of entry e at (k / 8) * kRegion + 128 e + 16 (k % 8); the
// region stride is 4096 + 128 so that the 16 lanes of a dequantising read
// that cross into the next region use the other half of the banks.  The
// 8 scale bytes of entry e follow at kRawScaleOff + 32 e.
constexpr int kRegion = kChunk * 128 + 128;
constexpr int kRawScaleOff = kGathers * kRegion;
constexpr int kRawBytes = kRawScaleOff + kChunk * 32;
constexpr float kLn2 = 0.693147180559945309f;
// Split mode: a partial slot holds O [64 heads][512] fp32, then 64 maxima and
// 64 sums; the per-row prefix sums live in the K tile while the schedule is
// computed, which bounds the batch.
constexpr int kSlotFloats = 64 * 512 + 128;
constexpr int kMaxSplitRows = 8000;
constexpr float kRescaleSlack = 8.0f;                         // log2 of the largest probability

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef __attribute__((address_space(3))) uint32_t lds_u32_t;
typedef const __attribute__((address_space(1))) uint32_t global_u32_t;

struct CacheList {
    const uint8_t* cache;
    const int32_t* indices;
    const int32_t* lengths;  // [batch] or null
    const uint8_t* expanded; // bf16 rows [num_entries][512] of the whole cache, or null
    int64_t block_stride;    // bytes
    int64_t idx_stride_b, idx_stride_s;
    int64_t num_entries;     // num_blocks * page_size
    double inv_page;         // 1 / page_size
    int32_t num_blocks, page_size, topk, pad;
};

struct MlaArgs {
    const uint16_t* q;
    int64_t q_sb, q_ss, q_sh;
    uint16_t* out;
    int64_t o_sb, o_ss, o_sh;
    float* lse;
    int64_t l_sb, l_sh;
    const float* sink;
    CacheList list[2];
    int32_t num_lists;
    int32_t batch, seq_q, head_blocks;
    float scale_log2;  // softmax scale * log2(e)
    // split mode
    float* partials;       // 2 slots per workgroup of kSlotFloats
    int32_t* row_prefix;   // batch + 1 prefix sums of per-item chunk counts
    int32_t split_grid;
    // one-item kernel in the paired order: the CU count C (workgroups j and
    // C + j share a CU) and the number of windows
    int32_t pair_cus;
    int32_t order_windows;
};

// K tile addressing: 16-byte block b of row r at r * kKRowBytes + 16 b, rows
// 1056 bytes apart.  Measured with the LDS bank-conflict counter on gfx950
// (one wave, each access pattern alone): QK's ds_read_b128 (lane (m, g) reads
// block 4s+g of row m) and PV's ds_read_b64_tr_b16 (lane j of group g reads
// row 4g + j/4) are both conflict-free at this pitch.  Flipping block bit 0 in
// rows 8..15 (a swizzle meant for 16-lane ds_read_b128 passes) made half of
// QK's LDS cycles conflicts; pitches of 1040, 1072, 1088 or 1152 bytes
// conflict in both.  The dequantising writes and the row DMAs write whole
// rows, which is conflict-free at any pitch.
constexpr int kKRowBytes = kHeadDim * 2 + 32;

__device__ __forceinline__ int kbuf_byte(int row, int block) {
    return row * kKRowBytes + (block << 4);
}

// 8 e4m3 codes times 2^(byte - 127) -> 8 bf16, as the reference computes
// it: bf16(f32(code) * f32 bits (byte << 23)).  v_cvt_scalef32_pk_bf16_fp8
// gives exactly that for bytes 1..254 (tests/test_sparse_mla.py sweeps every
// byte 0..254 with all 254 finite codes through the attention and through
// the expanded copy).  It reads byte 0 as 2^-127 where the bit cast gives 0, so
// byte 0 converts at scale 1 and keeps only the sign bits (+-0, exact for
// finite codes).  Byte 255 is an infinite scale, which the cache writer
// cannot produce; like other non-finite inputs it is out of scope.
template <bool kExact>
__device__ __forceinline__ uint4 dequant8(uint2 codes, uint32_t byte) {
    const float scale = __uint_as_float((kExact && !byte ? 127u : byte) << 23);
    const uint32_t keep = kExact && !byte ? 0x80008000u : 0xffffffffu;
    const uint4 v = make_uint4(
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.x, scale, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.x, scale, true)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.y, scale, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.y, scale, true)));
    if (!kExact)
        return v;
    return make_uint4(keep & v.x, keep & v.y, keep & v.z, keep & v.w);
}

// A zero-filled stand-in for the entries a chunk does not attend (past the
// length, negative, past the cache): gathering them from here makes their
// K rows exactly zero without any select in the dequantisation (e4m3 code 0
// gives 0 at any scale), and keeps every lane of a gather active.
__device__ __align__(256) uint8_t mla_zero_entry[1024];
// The scale bytes gathered for entries that are not attended: 127 (2^0), so
// that a zero scale byte in a gathered chunk always belongs to an attended
// entry (dequantize's exact-route test needs no score mask).
__device__ __align__(16) uint8_t mla_unit_scales[16] = {127, 127, 127, 127, 127, 127, 127, 127,
                                                        127, 127, 127, 127, 127, 127, 127, 127};

// One list (main or extra) as one (batch row, query position) sees it.
struct ListView {
    const uint8_t* cache;
    const int32_t* row;     // this query's index row
    const uint8_t* expanded;
    int64_t block_stride, num_entries;
    double inv_page;
    int page_size, num_blocks, len;
};

// The list's clamped length for batch row b.
__device__ __forceinline__ int list_len(const CacheList& L, bool present, int b) {
    if (!present)
        return 0;
    if (!L.lengths)
        return L.topk;
    const int n = L.lengths[b];
    return n < 0 ? 0 : (n > L.topk ? L.topk : n);
}

// known_len >= 0: the length list_len gives, already loaded by the caller.
__device__ __forceinline__ ListView make_view(const CacheList& L, bool present, int b, int sq, int known_len = -1) {
    ListView v;
    v.cache = L.cache;
    v.row = L.indices + b * L.idx_stride_b + sq * L.idx_stride_s;
    v.expanded = L.expanded;
    v.num_entries = L.num_entries;
    v.block_stride = L.block_stride;
    v.inv_page = L.inv_page;
    v.page_size = L.page_size;
    v.num_blocks = L.num_blocks;
    v.len = known_len >= 0 ? known_len : list_len(L, present, b);
    return v;
}

// Chunk c of the concatenated (main, extra) sequence: its list and first entry.
__device__ __forceinline__ ListView select(const ListView& v0, const ListView& v1, bool second) {
    ListView v;
    v.cache = second ? v1.cache : v0.cache;
    v.row = second ? v1.row : v0.row;
    v.expanded = second ? v1.expanded : v0.expanded;
    v.num_entries = second ? v1.num_entries : v0.num_entries;
    v.block_stride = second ? v1.block_stride : v0.block_stride;
    v.inv_page = second ? v1.inv_page : v0.inv_page;
    v.page_size = second ? v1.page_size : v0.page_size;
    v.num_blocks = second ? v1.num_blocks : v0.num_blocks;
    v.len = second ? v1.len : v0.len;
    return v;
}

// The index of this lane's gather entry (8 * wave + lane / 8) of the chunk
// starting at t0, or -1 past the list's length: one plain load per lane, a
// chunk ahead of its use, so the compiler's own wait on the register is the
// only synchronisation it needs.
__device__ __forceinline__ int load_id(const ListView& v, int t0, int wave, int lane) {
    const int t = t0 + 8 * wave + (lane >> 3);
    return t < v.len ? v.row[t] : -1;
}

// Byte offset of entry `id` inside the cache (page * block stride + `unit` *
// position in page), or -1 if the entry is not attended.
__device__ __forceinline__ int64_t entry_offset(const ListView& v, int id, int64_t unit) {
    if (id < 0)
        return -1;
    int page = (int)((double)id * v.inv_page);
    int rel = id - page * v.page_size;
    if (rel < 0) {
        --page;
        rel += v.page_size;
    } else if (rel >= v.page_size) {
        ++page;
        rel -= v.page_size;
    }
    if (page >= v.num_blocks)
        return -1;
    return (int64_t)page * v.block_stride + unit * rel;
}

// Raw bytes of the chunk's 32 entries -> LDS.  Lane `lane` of wave `wave`
// moves pieces sub, sub+8, ..., sub+32 (sub = lane % 8, pieces past 35 repeat
// piece 35 into padding) of entry 8 * wave + lane / 8 (index `id`, from
// load_id), then a 4-byte scale word (word lane % 2 of that entry's 8 scale
// bytes), and lanes with sub 0 write the entry's score mask (0 or -inf).  The
// mask lives in its own LDS array: LDS written by these gathers is only read
// after the wait at the top of the next chunk.
__device__ __forceinline__ void issue_gather(const ListView& v, const uint8_t* dummy, int wave, int lane, int id,
                                             uint8_t* raw, float* mask) {
    __attribute__((address_space(3))) uint8_t* dst = (__attribute__((address_space(3))) uint8_t*)raw;
    const int e = 8 * wave + (lane >> 3), sub = lane & 7;
    const int64_t off = entry_offset(v, id, kTokenDataBytes);
    const uint8_t* tok = off >= 0 ? v.cache + off : dummy;
#pragma unroll
    for (int n = 0; n < kGathers; ++n) {
        const int k = sub + 8 * n < kPieces ? sub + 8 * n : kPieces - 1;
        __builtin_amdgcn_global_load_lds((global_u32_t*)(tok + 16 * k),
                                         (lds_u32_t*)(dst + n * kRegion + 1024 * wave), 16, 0, 0);
    }
    const int64_t soff = entry_offset(v, id, kScaleBytesPerToken);
    const uint8_t* scl = (soff >= 0 ? v.cache + (int64_t)v.page_size * kTokenDataBytes + soff : mla_unit_scales) +
                         4 * (lane & 1);
    __builtin_amdgcn_global_load_lds((global_u32_t*)scl, (lds_u32_t*)(dst + kRawScaleOff + 256 * wave), 4, 0, 0);
    if (sub == 0)
        mask[e] = off >= 0 ? 0.f : -INFINITY;
}

// A chunk of an expanded list (bf16 rows, 1 KiB per entry) straight into a K
// tile, with no dequantisation: wave w moves entries 8w..8w+7, one row per
// wave-wide 16-byte LDS DMA (64 lanes x 16 bytes land contiguously at the row's
// start, lane l's block l).  Each row's index comes from lane 8j (load_id's
// layout); entries that are not attended come from the zero page, and the
// mask is written as for a gather.
__device__ __forceinline__ void issue_rows(const ListView& v, int wave, int lane, int id, uint8_t* tile,
                                           float* mask) {
    __attribute__((address_space(3))) uint8_t* dst = (__attribute__((address_space(3))) uint8_t*)tile;
    const int src_off = 16 * lane;
    // each lane forms its entry's row address once; row j's is read from lane 8j
    const uint8_t* mine = id >= 0 && id < v.num_entries ? v.expanded + (int64_t)id * (2 * kHeadDim) : mla_zero_entry;
    const uint64_t maddr = reinterpret_cast<uint64_t>(mine);
#pragma unroll
    for (int j = 0; j < kChunk / 4; ++j) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)maddr, 8 * j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(maddr >> 32), 8 * j);
        const uint8_t* row = reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
        __builtin_amdgcn_global_load_lds((global_u32_t*)(row + src_off),
                                         (lds_u32_t*)(dst + (8 * wave + j) * kKRowBytes), 16, 0, 0);
    }
    if ((lane & 7) == 0)
        mask[8 * wave + (lane >> 3)] = id >= 0 && id < v.num_entries ? 0.f : -INFINITY;
}

// Chunk in `raw` -> bf16 K tile: wave w converts entries w, w+4, ..., lane l
// the 8 dims of block l (blocks 0..55 NoPE: half l%2 of piece l/2; 56..63
// RoPE: piece l-28), branch-free, with every LDS read issued before the first
// conversion: each lane reads its whole 16-byte piece.
// (Selects are written per component: a select of whole HIP vector structs
// is lowered through private memory.)
template <bool kExact>
__device__ __forceinline__ uint4 dequant_piece(uint4 piece, uint32_t byte, bool nope, bool hi) {
    const uint2 codes = make_uint2(hi ? piece.z : piece.x, hi ? piece.w : piece.y);
    const uint4 d = dequant8<kExact>(codes, byte);
    return make_uint4(nope ? d.x : piece.x, nope ? d.y : piece.y, nope ? d.z : piece.z, nope ? d.w : piece.w);
}

__device__ __forceinline__ void dequantize(const uint8_t* raw, uint8_t* kbuf, int wave, int lane) {
    const bool nope = lane < kNopeDim / 8, hi = lane & 1;
    const int k = nope ? lane >> 1 : lane - (kNopeDim / 8 - kNopeDim / 16);
    const int piece_off = (k >> 3) * kRegion + 16 * (k & 7);
    const int scale_off = kRawScaleOff + (nope ? lane >> 3 : 0);
    // four entries at a time: loads, then conversions, then stores
#pragma unroll
    for (int j0 = 0; j0 < kChunk / 4; j0 += 4) {
        const int e0 = 4 * j0 + wave, e1 = e0 + 4, e2 = e0 + 8, e3 = e0 + 12;
        const uint4 p0 = *reinterpret_cast<const uint4*>(raw + piece_off + 128 * e0);
        const uint4 p1 = *reinterpret_cast<const uint4*>(raw + piece_off + 128 * e1);
        const uint4 p2 = *reinterpret_cast<const uint4*>(raw + piece_off + 128 * e2);
        const uint4 p3 = *reinterpret_cast<const uint4*>(raw + piece_off + 128 * e3);
        const uint32_t b0 = raw[scale_off + 32 * e0], b1 = raw[scale_off + 32 * e1];
        const uint32_t b2 = raw[scale_off + 32 * e2], b3 = raw[scale_off + 32 * e3];
        // a zero scale byte (never written by the cache writer) takes the
        // exact route for the whole wave; entries that are not attended carry
        // scale byte 127 and zero codes (issue_gather), so they never ask for it
        const bool odd = nope && (b0 == 0 || b1 == 0 || b2 == 0 || b3 == 0);
        if (__builtin_expect(__any(odd), 0)) {
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e0, lane)) = dequant_piece<true>(p0, b0, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e1, lane)) = dequant_piece<true>(p1, b1, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e2, lane)) = dequant_piece<true>(p2, b2, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e3, lane)) = dequant_piece<true>(p3, b3, nope, hi);
        } else {
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e0, lane)) = dequant_piece<false>(p0, b0, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e1, lane)) = dequant_piece<false>(p1, b1, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e2, lane)) = dequant_piece<false>(p2, b2, nope, hi);
            *reinterpret_cast<uint4*>(kbuf + kbuf_byte(e3, lane)) = dequant_piece<false>(p3, b3, nope, hi);
        }
    }
}

// The workgroup's LDS: the double-buffered raw gather, the bf16 K tile, the
// gathered indices and the score masks.  They are separate __shared__ arrays
// (declared in each kernel, passed down by reference) so that the compiler
// can tell the LDS-DMA targets from the tile the MFMAs read; as members of
// one object they would make every tile read wait for the gathers.
#define FGV_MLA_LDS                                              \
    __shared__ __align__(16) uint8_t lds_raw[2][kRawBytes];      \
    __shared__ __align__(16) uint8_t lds_kbuf[kChunk * kKRowBytes]; \
    __shared__ float lds_mask[2][kChunk]

__device__ __forceinline__ uint2 read_tr(const uint8_t* kbuf, int byte) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)((__attribute__((address_space(3))) uint8_t*)kbuf + byte));
    return __builtin_bit_cast(uint2, v);
}

// Attends chunks [c_lo, c_hi) of the (b, sq, hb) item's concatenated (main,
// extra) chunk sequence.  With slot < 0 the item is complete and out/lse are
// written; otherwise the unnormalised O, the reference maximum and the sum go
// to partial slot `slot` of the workspace for the combine kernel.
// q's loads per lane: 16 steps of 32 dims, one 16-byte load each.
constexpr int kQLoads = 16;
// s_waitcnt operand "vmcnt(kQLoads)", expcnt and lgkmcnt not waited for
// (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int kWaitAllButQ = (kQLoads & 15) | ((kQLoads >> 4) << 14) | (7 << 4) | (15 << 8);
static_assert(kQLoads < 64, "vmcnt holds 6 bits");

// s_waitcnt operand "lgkmcnt(0)" alone.
constexpr int kWaitLds = 15 | (3 << 14) | (7 << 4);

// Workgroup barrier over LDS work only.  __syncthreads' fence (even one
// scoped to LDS) waits for every outstanding global load, q's included, since
// LDS-DMA writes count there too; the callers wait for their LDS-DMA gathers
// explicitly before this.  The empty asm statements keep the compiler from
// moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitLds);  // this wave's LDS reads and writes done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Attends one chunk for the wave's 16 heads: its bf16 K tile is at `kt`, its
// score mask (0 or -inf per entry) at `mask`; qf is q (B operand), acc the
// fp32 O^T accumulators, m_run / l_run the reference maximum (base 2) and the
// running sum.  qk_base / tr_base are the lane's K-tile byte offsets for the
// QK row reads and the PV transposing reads, g its 16-lane group.
// (Each call site passes one fixed LDS array, so the compiler can tell the
// tile read from the tile the LDS DMA is filling.)
//
// With TAIL, the scores have 64 more dims (the sparse prefill's d_qk = 576):
// q's in qt (lane group g: dims 512+32t+8g..+7 of step t), the entries' in
// the tail tile `tt` (32 rows of 128 bytes; tl_base = the lane's QK offset
// there); they enter S only, not O.  With MAXL, m_max keeps the exact largest
// score (base 2), which the lazily raised m_run is not.
constexpr int kTailDim = 64;
constexpr int kTailRow = kTailDim * 2;

template <bool MAXL, bool TAIL>
__device__ __forceinline__ void attend_tile(const uint8_t* kt, const uint8_t* tt, const float* mask,
                                            const bf16x8_t (&qf)[kQLoads], const bf16x8_t* qt, f32x4_t (&acc)[32],
                                            float& m_run, float& l_run, float& m_max, int qk_base, int tl_base,
                                            int tr_base, int g, float scale_log2) {
    // ---- S^T = K q^T for the chunk's two 16-entry tiles
    // K operands read two steps ahead of the MFMAs that consume them
    constexpr int kSteps = TAIL ? kQLoads + kTailDim / 32 : kQLoads;
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    bf16x8_t ka[3], kb[3];
    auto read_k = [&](int s, bf16x8_t& x, bf16x8_t& y) {
        if (s < kQLoads) {
            x = *reinterpret_cast<const bf16x8_t*>(kt + qk_base + 64 * s);
            y = *reinterpret_cast<const bf16x8_t*>(kt + qk_base + 64 * s + 16 * kKRowBytes);
        } else {
            x = *reinterpret_cast<const bf16x8_t*>(tt + tl_base + 64 * (s - kQLoads));
            y = *reinterpret_cast<const bf16x8_t*>(tt + tl_base + 64 * (s - kQLoads) + 16 * kTailRow);
        }
    };
    read_k(0, ka[0], kb[0]);
    read_k(1, ka[1], kb[1]);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        if (s + 2 < kSteps)
            read_k(s + 2, ka[(s + 2) % 3], kb[(s + 2) % 3]);
        const bf16x8_t qs = s < kQLoads ? qf[s] : qt[s - kQLoads];
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s % 3], qs, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb[s % 3], qs, s1, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads two steps ahead
    }

    // ---- online softmax (base 2) for head m16 over entries 4g+r, 16+4g+r
    float sv[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sv[r] = s0[r] * scale_log2 + mask[4 * g + r];
        sv[4 + r] = s1[r] * scale_log2 + mask[16 + 4 * g + r];
    }
    float cmax = sv[0];
#pragma unroll
    for (int i = 1; i < 8; ++i)
        cmax = fmaxf(cmax, sv[i]);
    cmax = group4_max(cmax);
    if constexpr (MAXL)
        m_max = fmaxf(m_max, cmax);
    // Raise the reference maximum (and rescale O and the sum) only when a
    // score of this wave's heads exceeds it by more than kRescaleSlack.
    if (__any(cmax > m_run + kRescaleSlack)) {
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 32; ++dt)
            acc[dt] *= alpha;
        m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float p[8], psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        p[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
        psum += p[i];
    }
    psum = group4_sum(psum);
    l_run += psum;
    // k = 8g+i of the PV product is entry 4g+i (i < 4) or 16+4g+i-4
    const uint4 pw = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                                pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7]));
    const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pw);

    // ---- O^T = alpha * O^T + V^T P^T over the 32 16-dim tiles: the
    // transposing read hands lane j of group g dim 16dt+j of rows
    // 4g..4g+3 (then 16+4g..16+4g+3), the A operand of k = 8g..8g+7.
    // (four steps ahead: one MFMA per step covers less LDS latency than
    // the two per step of the QK loop)
    uint2 vlo[5], vhi[5];
    auto read_v = [&](int dt, uint2& x, uint2& y) {
        x = read_tr(kt, tr_base + 32 * dt);
        y = read_tr(kt, tr_base + 32 * dt + 16 * kKRowBytes);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
        read_v(i, vlo[i], vhi[i]);
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
        if (dt + 4 < 32)
            read_v(dt + 4, vlo[(dt + 4) % 5], vhi[(dt + 4) % 5]);
        const uint2 lo = vlo[dt % 5], hi = vhi[dt % 5];
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb, acc[dt], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ void attend_chunk(const uint8_t* kt, const float* mask, const bf16x8_t (&qf)[kQLoads],
                                             f32x4_t (&acc)[32], float& m_run, float& l_run, int qk_base,
                                             int tr_base, int g, float scale_log2) {
    float unused;
    attend_tile<false, false>(kt, nullptr, mask, qf, nullptr, acc, m_run, l_run, unused, qk_base, 0, tr_base, g,
                              scale_log2);
}

// The wave's 16 output rows (lane (m16, g) holds dims 16dt+4g..+3 of head
// m16 in acc[dt]), times `factor`, go out through LDS: the wave stages them at
// `stage` (its own 16 rows, 1040 B apart so the staging writes of 32 lanes hit
// distinct banks), then writes whole 1 KiB rows with 16-byte non-temporal
// stores.  Only this wave touches `stage`, so a wait on its own LDS writes
// is the only synchronisation.
constexpr int kStageRow = kHeadDim * 2 + 16;
static_assert(2 * 16 * kStageRow <= 2 * kRawBytes && 2 * 16 * kStageRow <= kChunk * kKRowBytes,
              "two waves' staging fits the gather buffers and the K tile");

__device__ __forceinline__ void store_rows(uint8_t* stage, const f32x4_t (&acc)[32], float factor, uint16_t* obase,
                                           int64_t o_sh, int m16, int g, int lane) {
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
        const f32x4_t v = acc[dt] * factor;
        *reinterpret_cast<uint2*>(stage + m16 * kStageRow + 32 * dt + 8 * g) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int h = 0; h < 16; ++h)
        store16(obase + h * o_sh + 8 * lane, *reinterpret_cast<const uint4*>(stage + h * kStageRow + 16 * lane));
}

__device__ __forceinline__ void run_segment(const MlaArgs& a, uint8_t (&raw)[2][kRawBytes], uint8_t* kbuf,
                                            float (&mask_lds)[2][kChunk], int b,
                                            int sq, int hb, int c_lo, int c_hi, int slot, int wave, int lane,
                                            int len0 = -1, int len1 = -1) {
    const int m16 = lane & 15, g = lane >> 4;
    const int head = hb * kBlockHeads + wave * 16 + m16;

    const ListView v0 = make_view(a.list[0], true, b, sq, len0);
    const ListView v1 = make_view(a.list[1], a.num_lists > 1, b, sq, len1);
    const int n0 = (v0.len + kChunk - 1) / kChunk;
    const uint8_t* dummy = mla_zero_entry;

    // The first two chunks' indices go first, then the first chunk's gather,
    // then q's 16 loads (the largest transfer), in the same branch: the first
    // chunk waits for its gather alone (vmcnt counts in issue order), so q's
    // loads overlap that chunk's dequantisation.
    auto first_of = [&](int c) { return (c >= n0 ? c - n0 : c) * kChunk; };
    int id_next = -1;

    // q as the B operand of S^T = K q^T: step s covers dims 32s..32s+31, lane
    // group g dims 32s+8g..32s+8g+7 of head m16.
    const uint16_t* qrow = a.q + b * a.q_sb + sq * a.q_ss + head * a.q_sh;
    bf16x8_t qf[kQLoads];
    auto load_q = [&]() __attribute__((always_inline)) {
        asm volatile("" ::: "memory");  // q's loads stay behind the gather
#pragma unroll
        for (int s = 0; s < kQLoads; ++s)
            qf[s] = __builtin_bit_cast(bf16x8_t, load16(qrow + 32 * s + 8 * g));
        asm volatile("" ::: "memory");
    };
    // Chunks [c_lo, c_mid) come from the FP8 cache through the raw gather and
    // the dequantisation; with an expanded extra list, its chunks [c_mid, c_hi)
    // come as bf16 rows, alternating between two K tiles: the raw gather
    // buffers (free then; extra chunk n0 + 2i) and the K tile (n0 + 2i + 1).
    static_assert(kChunk * kKRowBytes <= 2 * kRawBytes, "the raw gather buffers hold a K tile");
    uint8_t* const raw_tile = &raw[0][0];
    const int c_mid = v1.expanded ? max(c_lo, min(c_hi, n0)) : c_hi;
    if (c_lo < c_hi) {
        const int id_cur = load_id(select(v0, v1, c_lo >= n0), first_of(c_lo), wave, lane);
        if (c_lo + 1 < c_hi)
            id_next = load_id(select(v0, v1, c_lo + 1 >= n0), first_of(c_lo + 1), wave, lane);
        if (c_lo < c_mid) {
            issue_gather(select(v0, v1, c_lo >= n0), dummy, wave, lane, id_cur, raw[c_lo & 1], mask_lds[c_lo & 1]);
            load_q();
        } else {
            issue_rows(v1, wave, lane, id_cur, ((c_lo - n0) & 1) ? kbuf : raw_tile, mask_lds[c_lo & 1]);
            load_q();
        }
    } else {
        load_q();
    }

    f32x4_t acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
        acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    // LDS byte offsets of this lane's K-tile reads.  QK: block 4s+g of row
    // m16 (then row 16+m16).  PV: lane j of group g points at row 4g + j/4,
    // dims 16dt + 4(j%4), i.e. block 2dt + (j%4)/2, byte 8(j%2) (then row
    // 16 + 4g + j/4).  s and dt enter as constant offsets 64 s and 32 dt.
    const int qk_base = kbuf_byte(m16, g);
    const int tr_row = 4 * g + (m16 >> 2);
    const int tr_base = kbuf_byte(tr_row, (m16 & 3) >> 1) + 8 * (m16 & 1);

    auto attend = [&](const uint8_t* kt, const float* mask) __attribute__((always_inline)) {
        attend_chunk(kt, mask, qf, acc, m_run, l_run, qk_base, tr_base, g, a.scale_log2);
    };

    for (int c = c_lo; c < c_mid; ++c) {
        uint8_t* cur = raw[c & 1];
        // The gather and dequantisation addresses derive from the lane id; an
        // opaque copy per chunk keeps them from being held (and spilled)
        // across the MFMA loops, which need every register.
        int ln = lane;
        asm volatile("" : "+v"(ln));
        // This wave's gathers of chunk c (and chunk c+1's index); on the first
        // chunk, all but q's loads, which are issued last.
        if (c == c_lo)
            __builtin_amdgcn_s_waitcnt(kWaitAllButQ);
        else
            __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();  // everyone's gathers landed; K tile no longer read
        dequantize(cur, kbuf, wave, ln);
        lds_barrier();
        if (c + 1 < c_mid)
            issue_gather(select(v0, v1, c + 1 >= n0), dummy, wave, ln, id_next, raw[(c + 1) & 1],
                         mask_lds[(c + 1) & 1]);
        else if (c + 1 < c_hi)  // the first expanded chunk (n0) goes to the raw buffers
            issue_rows(v1, wave, ln, id_next, raw_tile, mask_lds[(c + 1) & 1]);
        if (c + 2 < c_hi)
            id_next = load_id(select(v0, v1, c + 2 >= n0), first_of(c + 2), wave, ln);
        attend(kbuf, mask_lds[c & 1]);
    }
    // One expanded chunk: its rows are read from `tile` while the next chunk's
    // rows stream into `other`.  The loop below runs these in (raw, K tile)
    // pairs, so that each step reads one fixed array (two steps under an
    // if / else would merge every accumulator register at the join).
    auto expanded_step = [&](int c, uint8_t* tile, uint8_t* other) __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        __builtin_amdgcn_s_waitcnt(0);  // this wave's rows of chunk c (and chunk c+1's index)
        __syncthreads();                // everyone's rows landed; `other` no longer read
        if (c + 1 < c_hi)
            issue_rows(v1, wave, ln, id_next, other, mask_lds[(c + 1) & 1]);
        if (c + 2 < c_hi)
            id_next = load_id(v1, first_of(c + 2), wave, ln);
        attend(tile, mask_lds[c & 1]);
    };
    int c = c_mid;
    if (c < c_hi && ((c - n0) & 1))  // a segment that starts on an odd extra chunk
        expanded_step(c++, kbuf, raw_tile);
    for (; c < c_hi; c += 2) {
        expanded_step(c, raw_tile, kbuf);
        if (c + 1 < c_hi)
            expanded_step(c + 1, kbuf, raw_tile);
    }

    if (slot >= 0) {
        // partial: O as [head][dim] fp32, then the reference maxima and sums
        float* ws = a.partials + (int64_t)slot * kSlotFloats;
        float* orow = ws + (wave * 16 + m16) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 32; ++dt)
            *reinterpret_cast<f32x4_t*>(orow + 16 * dt + 4 * g) = acc[dt];
        if (g == 0) {
            ws[kBlockHeads * kHeadDim + wave * 16 + m16] = m_run;
            ws[kBlockHeads * kHeadDim + kBlockHeads + wave * 16 + m16] = l_run;
        }
        __syncthreads();  // the next segment reuses the LDS buffers
        return;
    }

    // ---- epilogue: lse excludes the sink; the sink only rescales O.  m_run
    // is the reference maximum (base 2): l_run = sum 2^(s - m_run).
    const bool any = l_run > 0.f;
    float factor = 0.f;
    if (any)
        factor = a.sink ? 1.f / (l_run + expf(a.sink[head] - m_run * kLn2)) : 1.f / l_run;
    // The gather buffers and the K tile are free once every wave has left
    // the chunk loop.
    __syncthreads();
    uint8_t* stage = wave < 2 ? &raw[0][0] + wave * 16 * kStageRow : kbuf + (wave - 2) * 16 * kStageRow;
    store_rows(stage, acc, factor, a.out + b * a.o_sb + sq * a.o_ss + (hb * kBlockHeads + wave * 16) * a.o_sh,
               a.o_sh, m16, g, lane);
    if (g == 0)
        a.lse[b * a.l_sb + head * a.l_sh + sq] = any ? m_run * kLn2 + logf(l_run) : INFINITY;
    __syncthreads();  // the next segment reuses the staging buffers
}


// Items in runs of kItemRun per XCD (kItemsInRuns, grids of at most one
// workgroup per CU): workgroups are dispatched to the 8 XCDs round-robin
// (workgroup w on XCD w % 8); workgroup w takes item floor(w / 8R) 8R +
// (w % 8) R + floor(w / 8) % R instead (R = kItemRun; the tail past the last
// whole 8R takes its own index), so each XCD streams R consecutive items' q
// and output rows.  Same-box A/Bs on the decode bench case when it ran in
// this order (512 items, one round; same bits, medians of 11-15 graph
// replays, four runs): 0.6-1.9 % faster, e.g. 20.22 -> 20.00 us on one input
// set and 21.63 -> 21.45 us over 8 rotating sets; runs of 8 and 32 the same;
// extra512 level (+-0.5 %).  The item count is taken from the grid: computing
// it from the arguments in the prologue cost the gain.  Grids of two
// workgroups per CU take the paired order below instead.
constexpr uint32_t kItemRun = 16;

// Paired order, for grids of C < G <= 2C workgroups (C = CUs).  Workgroups j
// and C + j share a CU: the dispatcher gives every CU one workgroup, then a
// second in the same order (read from HW_ID / XCC_ID on gfx950: pairs
// {j, C + j} in every launch, 256 CUs).  A CU runs to the end of its longer
// item, and a survivor's chunks run almost twice as fast once its partner has
// left; so the P = G - C shared CUs should hold a long item beside a short one,
// and the S = C - P workgroups alone on their CU (j in [P, C)) the longest
// items.  With at least one unpartnered workgroup per two pairs (2 S >= P),
// the grid is cut into the fewest windows W whose largest fits a wave's 64
// lanes: window w holds pairs [P w / W, P (w + 1) / W) (both items of each)
// and unpartnered workgroups [S w / W, S (w + 1) / W), with their own items,
// so each window mixes the two in proportion.  Its items are ranked by cost,
// longest first (ties by position): the unpartnered workgroups take the
// longest, and pair i of the rest takes the i-th longest on j, which is
// dispatched first, and the i-th shortest on C + j.  With fewer unpartnered
// workgroups, windows hold kPairWindow pairs only (no division to place a
// workgroup) and an unpartnered workgroup keeps its own item.  The cost
// counts 2 per FP8 chunk and 1 per expanded chunk (their measured per-chunk
// times are 3.0-3.6 and 1.6-1.8 us).
//   Measured (same bits; same-box A/Bs, graph replays): against items in runs,
// windows of 32 pairs took decode 20.63 -> 18.98 us and extra512 (with its
// expand kernel) 57.91 -> 52.09 us.  Orders computed on the host and read from
// memory: the unpartnered workgroups on the longest items, pairs folding the
// rest, took decode at batch 272 / 300 / 384 from 17.38 / 17.92 / 18.03 us
// (windows of pairs only) to 14.72 / 14.79 / 15.93 us with these windows and
// 14.67 / 14.69 / 15.75 us globally ranked; at batch 512 (no unpartnered
// workgroups) 18.64 against 18.59 us.  A global ranking in the kernel costs
// about 1 us more than a window's.
constexpr uint32_t kPairWindow = 32;  // pairs a window when few workgroups are unpartnered

// floor(n / d) for n, d < 2^20, d > 0: the float estimate n * (1/d) is within
// one of the quotient, and one comparison each way makes it exact.
__device__ __forceinline__ uint32_t small_div(uint32_t n, uint32_t d) {
    uint32_t q = (uint32_t)((float)n * __builtin_amdgcn_rcpf((float)d));
    if (q * d > n)
        --q;
    else if ((q + 1) * d <= n)
        ++q;
    return q;
}

enum ItemOrder { kItemsInOrder = 0, kItemsInRuns = 1, kItemsPaired = 2, kItemsLongestFirst = 3, kItemsPairedMixed = 4 };

// An item's list lengths (n0, n1) and its rank key: 2 per FP8 chunk, 1 per
// expanded chunk, plus 1 (8 bits; 0 is left for a slot with no item).
// (list_len's lengths, with both loads in flight before either is used, and
// no division when each batch row is one item)
__device__ __forceinline__ uint32_t item_key(const MlaArgs& a, uint32_t item, int& n0, int& n1) {
    const uint32_t per_row = (uint32_t)(a.head_blocks * a.seq_q);
    int row = (int)item;
    if (per_row != 1)
        row = (int)(item / per_row);
    const int32_t* p0 = a.list[0].lengths;
    const int32_t* p1 = a.num_lists > 1 ? a.list[1].lengths : nullptr;
    int r0 = 0, r1 = 0;
    if (p0)
        r0 = p0[row];
    if (p1)
        r1 = p1[row];
    const int t0 = a.list[0].topk, t1 = a.list[1].topk;
    n0 = p0 ? (r0 < 0 ? 0 : (r0 > t0 ? t0 : r0)) : t0;
    n1 = a.num_lists > 1 ? (p1 ? (r1 < 0 ? 0 : (r1 > t1 ? t1 : r1)) : t1) : 0;
    const int c0 = (n0 + kChunk - 1) / kChunk, c1 = (n1 + kChunk - 1) / kChunk;
    const int cost = 2 * c0 + (a.list[1].expanded ? c1 : 2 * c1);
    return (uint32_t)min(cost, 254) + 1;
}

// The item workgroup blk takes in the paired order, and that item's two list
// lengths (left at -1 for an unpartnered workgroup that keeps its own item).
// Every wave computes the same answer from one length load per lane: lanes
// [0, np) hold the window's pairs' first items, [np, 2 np) their second,
// [2 np, 2 np + ns) the unpartnered workgroups' own; the rest rank last.
template <bool kMixed>
__device__ __forceinline__ uint32_t paired_item(const MlaArgs& a, uint32_t blk, int lane, int& len0, int& len1) {
    const uint32_t G = gridDim.x, cus = (uint32_t)a.pair_cus, P = G - cus, S = cus - P;
    const uint32_t W = (uint32_t)a.order_windows;
    // this workgroup's place: pair j (first or second) or unpartnered u
    const bool first = blk < P, alone = !first && blk < cus;
    const uint32_t j = first ? blk : blk - cus, u = blk - P;
    const uint32_t l = (uint32_t)lane;
    uint32_t it, want;
    bool valid;
    if (!kMixed) {
        // pairs only, in windows of kPairWindow pairs (shifts, no division);
        // an unpartnered workgroup keeps its own item
        if (alone)
            return blk;
        const uint32_t w0 = j / kPairWindow * kPairWindow, m = min(kPairWindow, P - w0);
        const uint32_t l32 = l & (kPairWindow - 1);
        valid = l32 < m;
        it = valid ? (l < kPairWindow ? w0 + l32 : cus + w0 + l32) : w0;
        want = first ? j - w0 : 2 * m - 1 - (j - w0);
    } else {
        // its window: the largest w whose range starts at or before its index
        // (S > 0 whenever a workgroup is alone; P > 0 always)
        const uint32_t w = alone ? small_div((u + 1) * W - 1, S ? S : 1u) : small_div((j + 1) * W - 1, P);
        const uint32_t p_lo = small_div(P * w, W), np = small_div(P * (w + 1), W) - p_lo;
        const uint32_t s_lo = small_div(S * w, W), ns = small_div(S * (w + 1), W) - s_lo;
        valid = l < 2 * np + ns;
        it = l < np ? p_lo + l : l < 2 * np ? cus + p_lo + (l - np) : valid ? P + s_lo + (l - 2 * np) : blk;
        // unpartnered: ranks [0, ns); pairs: first ns + i, second ns + 2 np - 1 - i
        want = alone ? u - s_lo : first ? ns + (j - p_lo) : ns + 2 * np - 1 - (j - p_lo);
    }
    int n0, n1;
    const uint32_t k = item_key(a, it, n0, n1);
    const uint32_t key = valid ? k : 0;  // 0 ranks last
    // rank = lanes with a larger key + lanes below with the same key: bit
    // planes from the top, `eq` the lanes that match this lane's key so far
    // (an empty plane changes neither, and is skipped)
    uint64_t eq = ~0ull;
    uint32_t above = 0;
#pragma unroll
    for (int bit = 7; bit >= 0; --bit) {
        const bool set = (key >> bit) & 1;
        const uint64_t plane = __builtin_amdgcn_ballot_w64(set);
        if (!plane)
            continue;
        if (set) {
            eq &= plane;
        } else {
            above += __builtin_popcountll(eq & plane);
            eq &= ~plane;
        }
    }
    const uint32_t rank = above + __builtin_popcountll(eq & ((1ull << lane) - 1));
    // ranks are a permutation of 0..63 and the window's valid items take the first ones
    const uint64_t hit = __builtin_amdgcn_ballot_w64(rank == want);
    const int src = hit ? (int)__builtin_ctzll(hit) : 0;
    len0 = __builtin_amdgcn_readlane(n0, src);
    len1 = __builtin_amdgcn_readlane(n1, src);
    return (uint32_t)__builtin_amdgcn_readlane((int)it, src);
}

// Longest first, for grids of 2C < G <= 4C workgroups (three or four
// rounds): workgroups [w0, w0 + 256) take the window's own items in
// descending cost (ties by index), so each round starts its longest items
// first and the last round's tail holds the shortest.  Thread t holds item
// w0 + t; each wave leaves its key's 8 bit planes (ballots) in `scr`, every
// thread ranks its key against all four waves' planes, and the thread whose
// rank is blk - w0 leaves its item and lengths there.  `scr` is the K tile's
// last 512 bytes, which nothing writes before the chunk loop's first barrier.
// Same bits; same-box A/B, medians of 9 graph replays of 20 calls, against
// the grid in order: decode at batch 768 / 1024 33.3 / 42.1 -> 32.0 / 40.3
// us, 128 heads at batch 512 42.3 -> 40.2 us, extra512 at batch 1024 95.0 ->
// 89.6 us; at batch 2048 (eight rounds) 71.2 against 72.3 us, so larger
// grids run in order.  (Host-computed, these windows reach 38.2 / 87.1 us at
// batch 1024: the ranking costs each workgroup the rest.)
constexpr uint32_t kLptWindow = kThreads;

__device__ __forceinline__ uint32_t longest_first_item(const MlaArgs& a, uint32_t blk, int wave, int lane,
                                                       uint8_t* scr, int& len0, int& len1) {
    const uint32_t w0 = blk / kLptWindow * kLptWindow;
    const uint32_t m = min(kLptWindow, gridDim.x - w0);
    const uint32_t t = (uint32_t)(wave * 64 + lane);
    const bool valid = t < m;
    const uint32_t it = valid ? w0 + t : w0;
    int n0, n1;
    const uint32_t k = item_key(a, it, n0, n1);
    const uint32_t key = valid ? k : 0;
    uint64_t* planes = reinterpret_cast<uint64_t*>(scr);             // [4 waves][8 bits]
    int32_t* pick = reinterpret_cast<int32_t*>(scr + 4 * 8 * 8);      // item, n0, n1
    uint32_t* used = reinterpret_cast<uint32_t*>(scr + 4 * 8 * 8 + 16);  // [4]: non-empty planes
    uint32_t mine = 0;
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
        const uint64_t p = __builtin_amdgcn_ballot_w64((key >> bit) & 1);
        mine |= (p != 0 ? 1u : 0u) << bit;
        if (lane == 0)
            planes[wave * 8 + bit] = p;
    }
    if (lane == 0)
        used[wave] = mine;
    lds_barrier();
    const uint4 uw = *reinterpret_cast<const uint4*>(used);
    const uint32_t any = __builtin_amdgcn_readfirstlane(uw.x | uw.y | uw.z | uw.w);
    uint64_t pl[32];  // all planes in one batch of reads
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(planes)[i];
        pl[2 * i] = ((uint64_t)v.y << 32) | v.x;
        pl[2 * i + 1] = ((uint64_t)v.w << 32) | v.z;
    }
    // rank = keys above this one + equal keys at lower positions (waves
    // before this one, lanes below in this one), wave by wave as in
    // paired_item, with `sel` this key's bit as a mask
    uint32_t rank = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        uint64_t eq = ~0ull;
        uint32_t above = 0;
#pragma unroll
        for (int bit = 7; bit >= 0; --bit) {
            if (!((any >> bit) & 1))
                continue;
            const uint64_t p = pl[u * 8 + bit];
            const uint64_t sel = ((key >> bit) & 1) ? ~0ull : 0ull;
            above += __builtin_popcountll(eq & p & ~sel);
            eq &= ~(p ^ sel);
        }
        const uint64_t before = u < wave ? ~0ull : (u == wave ? (1ull << lane) - 1 : 0ull);
        rank += above + __builtin_popcountll(eq & before);
    }
    // ranks are a permutation of 0..255 and the window's items take 0..m-1
    if (valid && rank == blk - w0) {
        pick[0] = (int32_t)it;
        pick[1] = n0;
        pick[2] = n1;
    }
    lds_barrier();
    len0 = __builtin_amdgcn_readfirstlane(pick[1]);
    len1 = __builtin_amdgcn_readfirstlane(pick[2]);
    return (uint32_t)__builtin_amdgcn_readfirstlane(pick[0]);
}

// One workgroup per (batch row, query position, 64-head block).
template <int kOrder>
__global__ void __launch_bounds__(kThreads, 2)
sparse_mla_decode_kernel(MlaArgs a) {
    FGV_MLA_LDS;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    uint32_t item = blockIdx.x;
    int len0 = -1, len1 = -1;
    if (kOrder == kItemsInRuns && item < gridDim.x / (8 * kItemRun) * (8 * kItemRun))
        item = item / (8 * kItemRun) * (8 * kItemRun) + (item % 8) * kItemRun + (item / 8) % kItemRun;
    else if (kOrder == kItemsPaired)
        item = paired_item<false>(a, blockIdx.x, lane, len0, len1);
    else if (kOrder == kItemsPairedMixed)
        item = paired_item<true>(a, blockIdx.x, lane, len0, len1);
    else if (kOrder == kItemsLongestFirst)
        item = longest_first_item(a, blockIdx.x, wave, lane, lds_kbuf + kChunk * kKRowBytes - 512, len0, len1);
    int hb = 0, bs = (int)item;  // (no division for one head block or one query position)
    if (a.head_blocks != 1) {
        hb = item % a.head_blocks;
        bs = item / a.head_blocks;
    }
    int sq = 0, b = bs;
    if (a.seq_q != 1) {
        sq = bs % a.seq_q;
        b = bs / a.seq_q;
    }
    const ListView v0 = make_view(a.list[0], true, b, sq, len0);
    const ListView v1 = make_view(a.list[1], a.num_lists > 1, b, sq, len1);
    const int nchunks = (v0.len + kChunk - 1) / kChunk + (v1.len + kChunk - 1) / kChunk;
    run_segment(a, lds_raw, lds_kbuf, lds_mask, b, sq, hb, 0, nchunks, -1, wave, lane, len0, len1);
}

// ---- sparse prefill (flash_mla_sparse_fwd) over bf16 key/value rows
//
// Reference: src/flaggems_vllm/ops/flashmla_sparse.py:1045-1206 (wrapper,
// asserts) and :50-195 (portable kernel).  Token t's query heads attend the
// kv rows indices[t, 0, i] for i < topk_length[t] (clamped to [0, topk];
// topk without topk_length) that lie in [0, s_kv): K = the row's d_qk dims,
// V = its first 512.  Outputs per (t, head): the largest score, the
// log-sum-exp of the scores (+inf when none is attended) and O (the sink
// only rescales O, as in the decode).
struct PrefillArgs {
    const uint16_t* q;
    int64_t q_st, q_sh;
    const uint8_t* kv;
    int64_t kv_row_bytes;
    const int32_t* indices;
    int64_t idx_st;
    const int32_t* topk_length;  // [s_q] or null
    const float* sink;           // [h_q] or null
    uint16_t* out;
    int64_t o_st, o_sh;
    float* max_logits;
    float* lse;
    int64_t ml_st, l_st;
    int32_t s_kv, topk, head_blocks;
    float scale_log2;
};

// The chunk's 32 rows into a K tile, as issue_rows does (wave w: entries
// 8w..8w+7, one wave-wide 16-byte LDS DMA per 1 KiB row; `id` in load_id's
// layout), and with TAIL each row's 64-dim tail (bytes 1024..1151) into the
// tail tile: one more DMA per wave, lane l moving block l%8 of entry
// 8w + l/8, 8 rows of 128 bytes landing contiguously.  Rows not attended come
// from the zero page.
template <bool TAIL>
__device__ __forceinline__ void issue_kv_rows(const PrefillArgs& a, int wave, int lane, int id, uint8_t* tile,
                                              uint8_t* tail, float* mask) {
    __attribute__((address_space(3))) uint8_t* dst = (__attribute__((address_space(3))) uint8_t*)tile;
    // every lane forms its entry's row address once (vector ALU); row j's
    // address is then read from lane 8j, with no scalar arithmetic or branch
    // per row
    const bool valid = id >= 0 && id < a.s_kv;
    const uint8_t* mine = valid ? a.kv + (int64_t)id * a.kv_row_bytes : mla_zero_entry;
    const uint64_t maddr = reinterpret_cast<uint64_t>(mine);
#pragma unroll
    for (int j = 0; j < kChunk / 4; ++j) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)maddr, 8 * j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(maddr >> 32), 8 * j);
        const uint8_t* row = reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
        __builtin_amdgcn_global_load_lds((global_u32_t*)(row + 16 * lane),
                                         (lds_u32_t*)(dst + (8 * wave + j) * kKRowBytes), 16, 0, 0);
    }
    if constexpr (TAIL) {
        __attribute__((address_space(3))) uint8_t* tdst = (__attribute__((address_space(3))) uint8_t*)tail;
        const uint8_t* row = valid ? mine + 2 * kHeadDim : mla_zero_entry;
        __builtin_amdgcn_global_load_lds((global_u32_t*)(row + 16 * (lane & 7)),
                                         (lds_u32_t*)(tdst + 8 * kTailRow * wave), 16, 0, 0);
    }
    if ((lane & 7) == 0)
        mask[8 * wave + (lane >> 3)] = valid ? 0.f : -INFINITY;
}

// One workgroup per (token, 64-head block).
// The rows alternate between two K tiles (and two tail tiles): chunk c+1's
// DMA runs while chunk c is attended, one barrier per chunk, as the decode's
// expanded chunks do.
template <bool TAIL>
__global__ void __launch_bounds__(kThreads, 2)
sparse_mla_prefill_kernel(PrefillArgs a) {
    __shared__ __align__(16) uint8_t lds_t0[kChunk * kKRowBytes];
    __shared__ __align__(16) uint8_t lds_t1[kChunk * kKRowBytes];
    __shared__ __align__(16) uint8_t lds_x0[TAIL ? kChunk * kTailRow : 16];
    __shared__ __align__(16) uint8_t lds_x1[TAIL ? kChunk * kTailRow : 16];
    __shared__ float lds_mask[2][kChunk];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int m16 = lane & 15, g = lane >> 4;
    // Workgroup i runs on XCD i % 8.  With two head blocks, workgroups i and
    // i + 8 (same XCD, dispatched one round apart) take the two head blocks of
    // one token, so its rows are fetched into one L2 for both (measured 4-7%
    // faster at h_q 128 than head blocks on neighbouring XCDs); a last
    // partial group of 16 keeps the plain order.
    int hb, t;
    {
        const int bid = blockIdx.x, paired = (int)(gridDim.x / 16) * 16;
        if (a.head_blocks == 2 && bid < paired) {
            t = (bid >> 4) * 8 + (bid & 7);
            hb = (bid >> 3) & 1;
        } else {
            hb = bid % a.head_blocks;
            t = bid / a.head_blocks;
        }
    }
    const int head = hb * kBlockHeads + wave * 16 + m16;

    const int32_t* irow = a.indices + t * a.idx_st;
    int len = a.topk;
    if (a.topk_length) {
        const int n = a.topk_length[t];
        len = n < 0 ? 0 : (n > a.topk ? a.topk : n);
    }
    const int nch = (len + kChunk - 1) / kChunk;
    auto load_id = [&](int c, int ln) {
        const int e = c * kChunk + 8 * wave + (ln >> 3);
        return e < len ? irow[e] : -1;
    };
    int id_next = -1;
    if (nch > 0) {
        const int id0 = load_id(0, lane);
        if (nch > 1)
            id_next = load_id(1, lane);
        issue_kv_rows<TAIL>(a, wave, lane, id0, lds_t0, lds_x0, lds_mask[0]);
    }

    // q as the B operand (lane group g: dims 32s+8g..+7 of head m16)
    const uint16_t* qrow = a.q + t * a.q_st + head * a.q_sh;
    bf16x8_t qf[kQLoads], qt[TAIL ? kTailDim / 32 : 1];
#pragma unroll
    for (int s = 0; s < kQLoads; ++s)
        qf[s] = __builtin_bit_cast(bf16x8_t, load16(qrow + 32 * s + 8 * g));
    if constexpr (TAIL) {
#pragma unroll
        for (int s = 0; s < kTailDim / 32; ++s)
            qt[s] = __builtin_bit_cast(bf16x8_t, load16(qrow + kHeadDim + 32 * s + 8 * g));
    }

    f32x4_t acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
        acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f, m_max = -INFINITY;
    const int qk_base = kbuf_byte(m16, g);
    const int tl_base = m16 * kTailRow + 16 * g;
    const int tr_base = kbuf_byte(4 * g + (m16 >> 2), (m16 & 3) >> 1) + 8 * (m16 & 1);

    // Chunk c from (tile, tail) while chunk c+1 streams into (other, other_tail).
    auto step = [&](int c, uint8_t* tile, uint8_t* tail, uint8_t* other, uint8_t* other_tail)
                    __attribute__((always_inline)) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        __builtin_amdgcn_s_waitcnt(0);  // this wave's rows of chunk c (and chunk c+1's index)
        __syncthreads();                // everyone's rows landed; `other` no longer read
        if (c + 1 < nch)
            issue_kv_rows<TAIL>(a, wave, ln, id_next, other, other_tail, lds_mask[(c + 1) & 1]);
        if (c + 2 < nch)
            id_next = load_id(c + 2, ln);
        attend_tile<true, TAIL>(tile, tail, lds_mask[c & 1], qf, qt, acc, m_run, l_run, m_max, qk_base, tl_base,
                                tr_base, g, a.scale_log2);
    };
    for (int c = 0; c < nch; c += 2) {
        step(c, lds_t0, lds_x0, lds_t1, lds_x1);
        if (c + 1 < nch)
            step(c + 1, lds_t1, lds_x1, lds_t0, lds_x0);
    }

    // ---- epilogue, as the decode's: lse and the largest score exclude the
    // sink, which only rescales O; m_run is the reference maximum (base 2).
    const bool any = l_run > 0.f;
    float factor = 0.f;
    if (any)
        factor = a.sink ? 1.f / (l_run + expf(a.sink[head] - m_run * kLn2)) : 1.f / l_run;
    __syncthreads();  // the K tiles are free once every wave has left the loop
    uint8_t* stage = wave < 2 ? lds_t0 + wave * 16 * kStageRow : lds_t1 + (wave - 2) * 16 * kStageRow;
    store_rows(stage, acc, factor, a.out + t * a.o_st + (hb * kBlockHeads + wave * 16) * a.o_sh, a.o_sh, m16, g,
               lane);
    if (g == 0) {
        a.lse[t * a.l_st + head] = any ? m_run * kLn2 + logf(l_run) : INFINITY;
        a.max_logits[t * a.ml_st + head] = m_max * kLn2;
    }
}

// Chunks a batch row's items have (the same for every query position and
// head block of the row).
__device__ __forceinline__ int row_chunks(const MlaArgs& a, int b) {
    const ListView v0 = make_view(a.list[0], true, b, 0);
    const ListView v1 = make_view(a.list[1], a.num_lists > 1, b, 0);
    return (v0.len + kChunk - 1) / kChunk + (v1.len + kChunk - 1) / kChunk;
}

// Split mode: the W chunks of all items, in item order (b, sq, hb), are cut
// into gridDim.x equal ranges, one per workgroup (two per CU), so long and
// short lists share the machine evenly.  A workgroup walks its range item by
// item; an item wholly inside one range is finished there, the pieces of an
// item that crosses range boundaries go to partial slots 2k+1 (the range
// where it starts) and 2k (every later range), which the combine kernel
// merges.  The per-row prefix sums Q are computed by every workgroup in LDS
// (workgroup 0 also leaves them in the workspace for the combine kernel).
__global__ void __launch_bounds__(kThreads, 2)
sparse_mla_decode_split_kernel(MlaArgs a) {
    FGV_MLA_LDS;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int B = a.batch, R = a.seq_q * a.head_blocks, G = gridDim.x;
    int32_t* Q = reinterpret_cast<int32_t*>(lds_kbuf);  // B + 1 prefix sums
    int32_t* part = Q + kMaxSplitRows + 1;              // per-thread slice sums

    // ---- Q[b] = chunks of rows 0..b-1 (per item)
    const int per = (B + kThreads - 1) / kThreads;
    const int lo = min(B, tid * per), hi = min(B, lo + per);
    int sum = 0;
    for (int r = lo; r < hi; ++r)
        sum += row_chunks(a, r);
    part[tid] = sum;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int t = 0; t < kThreads; ++t) {
            const int v = part[t];
            part[t] = run;
            run += v;
        }
        Q[B] = run;
    }
    __syncthreads();
    {
        int run = part[tid];
        for (int r = lo; r < hi; ++r) {
            Q[r] = run;
            run += row_chunks(a, r);
        }
    }
    __syncthreads();
    const int64_t W = (int64_t)Q[B] * R;
    if (blockIdx.x == 0) {
        for (int r = tid; r <= B; r += kThreads)
            a.row_prefix[r] = Q[r];
    }
    const int64_t start = (int64_t)blockIdx.x * W / G, end = ((int64_t)blockIdx.x + 1) * W / G;
    // first row whose items reach past `start`
    int rlo = 0, rhi = B - 1;
    while (rlo < rhi) {
        const int mid = (rlo + rhi + 1) >> 1;
        if ((int64_t)Q[mid] * R <= start)
            rlo = mid;
        else
            rhi = mid - 1;
    }
    int b = rlo;
    int n = Q[b + 1] - Q[b];   // > 0: the largest row starting at or before `start`
    const int64_t off = start - (int64_t)Q[b] * R;   // chunk offset inside row b's items
    __syncthreads();  // Q lives in the K tile, which the segments overwrite
    if (start >= end)
        return;
    int j = (int)(off / n), c = (int)(off - (int64_t)j * n);
    int64_t pos = start;
    while (pos < end) {
        const int c_hi = (int)min((int64_t)n, c + (end - pos));
        const bool whole = c == 0 && c_hi == n;
        const int slot = whole ? -1 : 2 * (int)blockIdx.x + (c > 0 ? 0 : 1);
        // an opaque lane id per segment keeps the lane-derived gather
        // addresses from being held (and spilled) across the segment loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        run_segment(a, lds_raw, lds_kbuf, lds_mask, b, j / a.head_blocks, j % a.head_blocks, c, c_hi,
                    slot, wave, ln);
        pos += c_hi - c;
        c = 0;
        if (++j == R) {
            j = 0;
            do {
                ++b;
                n = b < B ? row_chunks(a, b) : 1;
            } while (b < B && n == 0);
        }
    }
}

// ---- Paired grid: one 8-wave workgroup per CU, both halves on one item.
//
// For long lists over more items than CUs but at most two per CU, one 4-wave
// workgroup per item runs a single round that lasts as long as the longest
// list, and the split grid balances it at the cost of fp32 partial slots
// (128 KiB per crossing piece) and a combine kernel.  Here each CU takes one
// or two items and attends each with both halves of an 8-wave workgroup:
// half h (waves 4h..4h+3; wave hw of a half owns heads 16hw..16hw+15 of the
// block, as in sparse_mla_decode_kernel) takes every other chunk of the item,
// with its own gather buffers, K tile and masks, at its own pace
// (half_barrier).  At the end half 1's O, reference maximum and sum merge into
// half 0 through LDS, and half 0 writes the output: no partials leave the CU.
// A CU with two items gets a short one after a long one: items [0, G) go
// first, one per workgroup, and the workgroup whose first item has rank r in
// ascending chunk count (ties by index) then takes the item of rank r in
// descending chunk count among items [G, I), if there is one.
// Barrier over the four waves of one half of a paired workgroup, on a
// counter in LDS that only grows: each wave adds 1 once its LDS accesses are
// done, then polls until the half's four waves have all added for this
// barrier (`gen` counts the wave's barriers so far, times 4).  Like
// lds_barrier it orders LDS accesses only: callers wait for their own
// LDS-DMA gathers first.  The poll is bounded (2^24 polls of 64 clocks,
// about 0.4 s), so the wait ends even if the counts were ever wrong.  The
// add and the polls are written as ds instructions with their own lgkmcnt
// waits: as builtins the compiler would also wait for every outstanding
// global load before them (it cannot tell the counter from the LDS-DMA
// targets), q's included.
constexpr uint32_t kHalfWaves = 4;

__device__ __forceinline__ void half_barrier(uint32_t* ctr, uint32_t& gen) {
    const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)ctr;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    gen += kHalfWaves;
    if ((threadIdx.x & 63) == 0)
        asm volatile("ds_add_u32 %0, %1" ::"v"(addr), "v"(1u) : "memory");
    for (int i = 0; i < (1 << 24); ++i) {
        uint32_t v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
        if ((int32_t)(__builtin_amdgcn_readfirstlane(v) - gen) >= 0)
            break;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
}

constexpr int kPairThreads = 512;
constexpr int kPairMaxItems = kPairThreads;  // one top-k length per thread and list goes to LDS
constexpr int kPairBuckets = 256;            // chunk counts ordered exactly up to this value

__device__ __forceinline__ int list_chunks(int len, int topk) {
    len = len < 0 ? 0 : (len > topk ? topk : len);
    return (len + kChunk - 1) / kChunk;
}

__global__ void __launch_bounds__(kPairThreads, 1)
sparse_mla_decode_pair_kernel(MlaArgs a) {
    __shared__ __align__(16) uint8_t lds_raw[2][2][kRawBytes];
    __shared__ __align__(16) uint8_t lds_kbuf[2][kChunk * kKRowBytes];
    __shared__ float lds_mask[2][2][kChunk];
    __shared__ int32_t lds_len[2][kPairMaxItems];  // each item's raw top-k lengths (main, extra)
    __shared__ int32_t lds_hist[kPairBuckets];     // items [G, I) per clamped chunk count
    __shared__ int32_t lds_sched[16];              // rank, bucket, rank in bucket, pick, wave partials
    __shared__ uint32_t lds_hbar[2];               // half_barrier counters

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int half = wave >> 2, hw = wave & 3;
    const int m16 = lane & 15, g = lane >> 4;
    const int R = a.seq_q * a.head_blocks, I = a.batch * R, G = gridDim.x;
    uint8_t (&raw)[2][kRawBytes] = lds_raw[half];
    uint8_t* const kbuf = lds_kbuf[half];
    float (&mask_lds)[2][kChunk] = lds_mask[half];
    uint8_t* const raw_tile = &raw[0][0];

    uint32_t gen = 0;  // this wave's half_barrier count so far, times 4
    if (tid < 2)
        lds_hbar[tid] = 0;
    __syncthreads();

    // With more items than workgroups, every item's top-k lengths go to LDS
    // (LDS DMA, counted with the first chunk's gathers) for the choice of the
    // second item, and the counters start at zero (visible after the first
    // barrier).
    const bool pairs = I > G;
    if (pairs) {
        if (tid < kPairBuckets)
            lds_hist[tid] = 0;
        if (tid == 0) {
            lds_sched[0] = 0;
            lds_sched[3] = -1;
        }
        const int i = tid < I ? tid : I - 1;
#pragma unroll
        for (int L = 0; L < 2; ++L)
            if (L < a.num_lists && a.list[L].lengths)
                __builtin_amdgcn_global_load_lds((global_u32_t*)(a.list[L].lengths + i / R),
                                                 (lds_u32_t*)&lds_len[L][64 * wave], 4, 0, 0);
    }
    auto item_chunks = [&](int i) {
        const int t0 = a.list[0].topk, t1 = a.list[1].topk;
        int n = list_chunks(a.list[0].lengths ? lds_len[0][i] : t0, t0);
        if (a.num_lists > 1)
            n += list_chunks(a.list[1].lengths ? lds_len[1][i] : t1, t1);
        return n;
    };

    int item = blockIdx.x;
    for (int it = 0; it < 2 && item >= 0; ++it) {
        const int b = item / R, jr = item - b * R;
        const int sq = jr / a.head_blocks, hb = jr - sq * a.head_blocks;
        const int head = hb * kBlockHeads + hw * 16 + m16;
        const ListView v0 = make_view(a.list[0], true, b, sq);
        const ListView v1 = make_view(a.list[1], a.num_lists > 1, b, sq);
        // Half h takes main chunks h, h+2, ... and extra chunks (h + n0) % 2,
        // +2, ...: K0 + K1 chunks, numbered k = 0.. in its own order.
        const int n0 = (v0.len + kChunk - 1) / kChunk, n1 = (v1.len + kChunk - 1) / kChunk;
        const int p = n0 & 1;
        const int K0 = (n0 + 1 - half) >> 1, K1 = (n1 + 1 - (half ^ p)) >> 1, K = K0 + K1;
        const bool expanded = v1.expanded != nullptr;
        const int Kc = expanded ? K0 : K;  // chunks through the raw gather (the rest are bf16 rows)
        auto view_of = [&](int k) { return select(v0, v1, k >= K0); };
        auto first_of = [&](int k) { return (k < K0 ? 2 * k + half : 2 * (k - K0) + (half ^ p)) * kChunk; };

        const uint16_t* qrow = a.q + b * a.q_sb + sq * a.q_ss + head * a.q_sh;
        bf16x8_t qf[kQLoads];
        auto load_q = [&]() __attribute__((always_inline)) {
            asm volatile("" ::: "memory");  // q's loads stay behind the gather
#pragma unroll
            for (int s = 0; s < kQLoads; ++s)
                qf[s] = __builtin_bit_cast(bf16x8_t, load16(qrow + 32 * s + 8 * g));
            asm volatile("" ::: "memory");
        };
        int id_next = -1;
        if (K > 0) {
            const int id_cur = load_id(view_of(0), first_of(0), hw, lane);
            if (K > 1)
                id_next = load_id(view_of(1), first_of(1), hw, lane);
            if (Kc > 0) {
                issue_gather(view_of(0), mla_zero_entry, hw, lane, id_cur, raw[0], mask_lds[0]);
                load_q();
            } else {
                issue_rows(v1, hw, lane, id_cur, raw_tile, mask_lds[0]);
                load_q();
            }
        } else {
            load_q();
        }

        f32x4_t acc[32];
#pragma unroll
        for (int i = 0; i < 32; ++i)
            acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f;
        const int qk_base = kbuf_byte(m16, g);
        const int tr_base = kbuf_byte(4 * g + (m16 >> 2), (m16 & 3) >> 1) + 8 * (m16 & 1);
        auto attend = [&](const uint8_t* kt, const float* mask) __attribute__((always_inline)) {
            attend_chunk(kt, mask, qf, acc, m_run, l_run, qk_base, tr_base, g, a.scale_log2);
        };

        // The half's chunks k = 0 .. K-1 at its own pace: its barriers are
        // half_barrier's, over its four waves only.  FP8 chunks first (the
        // main list, and the extra list unless it is expanded), as in
        // run_segment's chunk loop.
        for (int k = 0; k < Kc; ++k) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            if (k == 0)
                __builtin_amdgcn_s_waitcnt(kWaitAllButQ);
            else
                __builtin_amdgcn_s_waitcnt(0);
            half_barrier(&lds_hbar[half], gen);  // the half's gathers landed; its K tile no longer read
            dequantize(raw[k & 1], kbuf, hw, ln);
            half_barrier(&lds_hbar[half], gen);
            if (k + 1 < Kc)
                issue_gather(view_of(k + 1), mla_zero_entry, hw, ln, id_next, raw[(k + 1) & 1],
                             mask_lds[(k + 1) & 1]);
            else if (k + 1 < K)  // the half's first expanded chunk goes to the raw buffers
                issue_rows(v1, hw, ln, id_next, raw_tile, mask_lds[(k + 1) & 1]);
            if (k + 2 < K)
                id_next = load_id(view_of(k + 2), first_of(k + 2), hw, ln);
            attend(kbuf, mask_lds[k & 1]);
        }
        // Expanded chunks: chunk k is read from `tile` while the next one
        // streams into `other`, in (raw, K tile) pairs as in run_segment.
        auto expanded_step = [&](int k, uint8_t* tile, uint8_t* other) __attribute__((always_inline)) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            __builtin_amdgcn_s_waitcnt(0);       // this wave's rows of chunk k (and chunk k+1's index)
            half_barrier(&lds_hbar[half], gen);  // the half's rows landed; `other` no longer read
            if (k + 1 < K)
                issue_rows(v1, hw, ln, id_next, other, mask_lds[(k + 1) & 1]);
            if (k + 2 < K)
                id_next = load_id(v1, first_of(k + 2), hw, ln);
            attend(tile, mask_lds[k & 1]);
        };
        for (int k = Kc; k < K; k += 2) {
            expanded_step(k, raw_tile, kbuf);
            if (k + 1 < K)
                expanded_step(k + 1, kbuf, raw_tile);
        }
        __syncthreads();  // both halves done: every K tile and gather buffer is free

        // ---- the second item (first pass only): this item's rank among
        // items [0, G), then the item of that rank from the top among [G, I)
        int next = -1;
        if (it == 0 && pairs) {
            const int nf = item_chunks(item);
            int cnt = 0;
            for (int x0 = 0; x0 < G; x0 += kPairThreads) {
                const int x = x0 + tid;
                bool before = false;
                if (x < G) {
                    const int nx = item_chunks(x);
                    before = nx < nf || (nx == nf && x < item);
                }
                cnt += __popcll(__ballot(before));
            }
            for (int y = G + tid; y < I; y += kPairThreads)
                atomicAdd(&lds_hist[min(item_chunks(y), kPairBuckets - 1)], 1);
            if (lane == 0)
                atomicAdd(&lds_sched[0], cnt);
            __syncthreads();
            const int r = lds_sched[0];
            if (r < I - G) {
                // descending prefix over the buckets: thread t holds bucket 255 - t
                int h = 0, incl = 0;
                const int v = kPairBuckets - 1 - tid;
                if (tid < kPairBuckets) {
                    h = lds_hist[v];
                    incl = h;
#pragma unroll
                    for (int d = 1; d < 64; d <<= 1) {
                        const int t = __shfl_up(incl, d);
                        if (lane >= d)
                            incl += t;
                    }
                    if (lane == 63)
                        lds_sched[8 + wave] = incl;
                }
                __syncthreads();
                if (tid < kPairBuckets) {
                    int excl = incl - h;
                    for (int w = 0; w < wave; ++w)
                        excl += lds_sched[8 + w];
                    if (h > 0 && excl <= r && r < excl + h) {
                        lds_sched[1] = v;
                        lds_sched[2] = r - excl;
                    }
                }
                __syncthreads();
                const int vstar = lds_sched[1], j = lds_sched[2];
                // the j-th item of [G, I) (in index order) in bucket vstar
                int base = 0;
                for (int y0 = G; y0 < I; y0 += kPairThreads) {
                    const int y = y0 + tid;
                    const bool m = y < I && min(item_chunks(y), kPairBuckets - 1) == vstar;
                    const uint64_t bal = __ballot(m);
                    if (lane == 0)
                        lds_sched[8 + wave] = __popcll(bal);
                    __syncthreads();
                    int before = base, total = base;
                    for (int w = 0; w < kPairThreads / 64; ++w) {
                        const int c = lds_sched[8 + w];
                        before += w < wave ? c : 0;
                        total += c;
                    }
                    if (m && before + __popcll(bal & ((1ull << lane) - 1)) == j)
                        lds_sched[3] = y;
                    __syncthreads();
                    base = total;
                    if (base > j)
                        break;
                }
                next = __builtin_amdgcn_readfirstlane(lds_sched[3]);
            }
        }

        // ---- half 1's O, reference maximum and sum merge into half 0: wave
        // hw of half 1 leaves them in one of four LDS arrays (33280 bytes each),
        // lane-major, and wave hw of half 0 (the same heads) reads them.
        float* mrg = hw == 0   ? reinterpret_cast<float*>(&lds_raw[0][0][0])
                     : hw == 1 ? reinterpret_cast<float*>(&lds_raw[1][0][0])
                     : hw == 2 ? reinterpret_cast<float*>(&lds_kbuf[0][0])
                               : reinterpret_cast<float*>(&lds_kbuf[1][0]);
        static_assert((32 * 64 * 4 + 128) * 4 <= kChunk * kKRowBytes && kChunk * kKRowBytes <= 2 * kRawBytes,
                      "a wave's merge data fits each of the four arrays");
        if (half == 1) {
#pragma unroll
            for (int dt = 0; dt < 32; ++dt)
                *reinterpret_cast<f32x4_t*>(mrg + (dt * 64 + lane) * 4) = acc[dt];
            mrg[32 * 64 * 4 + lane] = m_run;
            mrg[32 * 64 * 4 + 64 + lane] = l_run;
        }
        __syncthreads();
        if (half == 0) {
            const float m1 = mrg[32 * 64 * 4 + lane], l1 = mrg[32 * 64 * 4 + 64 + lane];
            const float m_new = fmaxf(m_run, m1);
            const float m_ref = m_new == -INFINITY ? 0.f : m_new;
            const float w0 = __builtin_amdgcn_exp2f(m_run - m_ref), w1 = __builtin_amdgcn_exp2f(m1 - m_ref);
            l_run = l_run * w0 + l1 * w1;
            // eight reads in flight at a time (q's registers are free here)
#pragma unroll
            for (int d0 = 0; d0 < 32; d0 += 8) {
                f32x4_t o1[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    o1[i] = *reinterpret_cast<const f32x4_t*>(mrg + ((d0 + i) * 64 + lane) * 4);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc[d0 + i] = acc[d0 + i] * w0 + o1[i] * w1;
            }
            m_run = m_new;
        }
        __syncthreads();  // the merge arrays are free again

        // ---- epilogue (half 0), as in run_segment
        if (half == 0) {
            const bool any = l_run > 0.f;
            float factor = 0.f;
            if (any)
                factor = a.sink ? 1.f / (l_run + expf(a.sink[head] - m_run * kLn2)) : 1.f / l_run;
            uint8_t* stage = hw < 2 ? raw_tile + hw * 16 * kStageRow : kbuf + (hw - 2) * 16 * kStageRow;
            store_rows(stage, acc, factor,
                       a.out + b * a.o_sb + sq * a.o_ss + (hb * kBlockHeads + hw * 16) * a.o_sh, a.o_sh, m16,
                       g, lane);
            if (g == 0)
                a.lse[b * a.l_sb + head * a.l_sh + sq] = any ? m_run * kLn2 + logf(l_run) : INFINITY;
        }
        __syncthreads();  // the next item reuses the staging buffers
        item = next;
    }
}

// Merges the partial slots of every item that crosses a split range
// boundary, and writes the items that attend nothing.  Four workgroups per
// item, one per quarter of its 64 heads; wave w of a workgroup merges 4 head
// rows, lane l dims 8l..8l+7 of each, so every read of a 2 KiB partial row and
// every 1 KiB output row is contiguous.  Each slot's reads for the wave's four
// heads (reference maxima and sums, then the rows) are issued together and
// unconditionally: a slot whose segment attended nothing holds zero rows and
// a zero sum, and takes weight 0.
__global__ void __launch_bounds__(kThreads)
sparse_mla_combine_kernel(MlaArgs a) {
    constexpr int kHeadsPerWave = kBlockHeads / 4 / (kThreads / 64);
    const int item = blockIdx.x >> 2, quarter = blockIdx.x & 3;
    const int R = a.seq_q * a.head_blocks, G = a.split_grid;
    const int b = item / R, jr = item % R;
    const int sq = jr / a.head_blocks, hb = jr % a.head_blocks;
    const int64_t W = (int64_t)a.row_prefix[a.batch] * R;
    const int n = a.row_prefix[b + 1] - a.row_prefix[b];
    const int64_t p0 = (int64_t)a.row_prefix[b] * R + (int64_t)jr * n, p1 = p0 + n;
    auto range_of = [&](int64_t p) { return (int)min((int64_t)G - 1, ((p + 1) * G - 1) / W); };
    auto start_of = [&](int k) { return (int64_t)k * W / G; };
    int k_lo = 0, k_hi = -1;
    if (n > 0) {
        k_lo = range_of(p0);
        k_hi = range_of(p1 - 1);
        if (k_lo == k_hi)
            return;  // finished by its workgroup
    }
    auto slot_of = [&](int k) {
        return a.partials + (int64_t)(k == k_lo ? 2 * k + 1 : 2 * k) * kSlotFloats;
    };
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h0 = quarter * (kBlockHeads / 4) + wave * kHeadsPerWave;

    float M[kHeadsPerWave];
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i)
        M[i] = -INFINITY;
    for (int k = k_lo; k <= k_hi; ++k) {
        if (start_of(k) == start_of(k + 1))  // skip empty ranges
            continue;
        const float* mk = slot_of(k) + kBlockHeads * kHeadDim + h0;
#pragma unroll
        for (int i = 0; i < kHeadsPerWave; ++i)
            M[i] = fmaxf(M[i], mk[i]);
    }
    float M_use[kHeadsPerWave], L[kHeadsPerWave];
    f32x4_t o[kHeadsPerWave][2];
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i) {
        M_use[i] = M[i] == -INFINITY ? 0.f : M[i];
        L[i] = 0.f;
        o[i][0] = o[i][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int k = k_lo; k <= k_hi; ++k) {
        if (start_of(k) == start_of(k + 1))
            continue;
        const float* ws = slot_of(k);
        float m[kHeadsPerWave], l[kHeadsPerWave];
        f32x4_t r0[kHeadsPerWave], r1[kHeadsPerWave];
#pragma unroll
        for (int i = 0; i < kHeadsPerWave; ++i) {
            m[i] = ws[kBlockHeads * kHeadDim + h0 + i];
            l[i] = ws[kBlockHeads * kHeadDim + kBlockHeads + h0 + i];
            const f32x4_t* row = reinterpret_cast<const f32x4_t*>(ws + (h0 + i) * kHeadDim + 8 * lane);
            r0[i] = row[0];
            r1[i] = row[1];
        }
#pragma unroll
        for (int i = 0; i < kHeadsPerWave; ++i) {
            const float w = l[i] > 0.f ? __builtin_amdgcn_exp2f(m[i] - M_use[i]) : 0.f;
            L[i] += l[i] * w;
            o[i][0] += r0[i] * w;
            o[i][1] += r1[i] * w;
        }
    }
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i) {
        const int head = hb * kBlockHeads + h0 + i;
        const bool any = L[i] > 0.f;
        float factor = 0.f;
        if (any)
            factor = a.sink ? 1.f / (L[i] + expf(a.sink[head] - M_use[i] * kLn2)) : 1.f / L[i];
        const f32x4_t v0 = o[i][0] * factor, v1 = o[i][1] * factor;
        store16(a.out + b * a.o_sb + sq * a.o_ss + head * a.o_sh + 8 * lane,
                make_uint4(pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]), pack_bf16x2(v1[0], v1[1]),
                           pack_bf16x2(v1[2], v1[3])));
        if (lane == 0)
            a.lse[b * a.l_sb + head * a.l_sh + sq] = any ? M_use[i] * kLn2 + logf(L[i]) : INFINITY;
    }
}

// Dequantises every entry of a list's cache into bf16 rows [num_entries][512]
// (the expanded copy the chunk loop then DMAs without converting), with the
// conversion the chunk loop uses (scale byte 0 included), so either route
// gives the same K rows.  Each 32-lane half of a wave does kPerHalf entries,
// all loads first (the kernel is short, and latency-bound with fewer bytes in
// flight); lane k makes output blocks k and k + 32, so each store instruction
// writes two whole 512-byte halves: blocks below 56 from 8 code bytes and
// their scale byte, blocks 56..63 from 16 RoPE bytes.  Four entries per half
// while that leaves at least kExpandWideMinBlocks workgroups, else two: same
// bits; same-box A/B, extra512 (32768 entries) 51.35 -> 50.87 us per call
// on one input set and 53.86 -> 52.43 us over four, eight per half 52.21 /
// 54.38 us; extra8192 (1024 entries) 296.8 against 297.9 us with four.
constexpr int kExpandWideMinBlocks = 256;

template <int kPerHalf>
constexpr int expand_per_block() { return kThreads / 32 * kPerHalf; }

template <int kPerHalf>
__global__ void __launch_bounds__(kThreads)
mla_expand_cache_kernel(CacheList L, uint8_t* out) {
    constexpr int kExpandPerHalf = kPerHalf;
    constexpr int kExpandPerBlock = expand_per_block<kPerHalf>();
    const int k = threadIdx.x & 31, k2 = k + 32;
    const int64_t e0 = (int64_t)blockIdx.x * kExpandPerBlock + (threadIdx.x >> 5) * kExpandPerHalf;
    uint2 c0[kExpandPerHalf];
    uint4 c1[kExpandPerHalf];  // codes of block k2 in .x/.y, or its RoPE bytes
    uint32_t b0[kExpandPerHalf], b1[kExpandPerHalf];
#pragma unroll
    for (int i = 0; i < kExpandPerHalf; ++i) {
        // (entries < 2^16 here: the copy is at most 64 MiB of 1 KiB rows)
        const uint32_t e = (uint32_t)(e0 + i < L.num_entries ? e0 + i : L.num_entries - 1);
        const uint32_t page = e / (uint32_t)L.page_size, rel = e - page * (uint32_t)L.page_size;
        const uint8_t* base = L.cache + (int64_t)page * L.block_stride;
        const uint8_t* tok = base + rel * kTokenDataBytes;
        const uint8_t* scl = base + (int64_t)L.page_size * kTokenDataBytes + rel * kScaleBytesPerToken;
        c0[i] = *reinterpret_cast<const uint2*>(tok + 8 * k);
        b0[i] = scl[k >> 3];
        if (k2 < kNopeDim / 8) {
            const uint2 c = *reinterpret_cast<const uint2*>(tok + 8 * k2);
            c1[i] = make_uint4(c.x, c.y, 0u, 0u);
            b1[i] = scl[k2 >> 3];
        } else {
            c1[i] = *reinterpret_cast<const uint4*>(tok + kNopeDim + 16 * (k2 - kNopeDim / 8));
            b1[i] = 0;
        }
    }
#pragma unroll
    for (int i = 0; i < kExpandPerHalf; ++i) {
        if (e0 + i >= L.num_entries)
            break;
        const uint4 r0 = dequant8<true>(c0[i], b0[i]);
        const uint4 r1 = k2 < kNopeDim / 8 ? dequant8<true>(make_uint2(c1[i].x, c1[i].y), b1[i]) : c1[i];
        uint8_t* row = out + (e0 + i) * (2 * kHeadDim);
        store16(row + 16 * k, r0);
        store16(row + 16 * k2, r1);
    }
}

void fill_list(CacheList& L, const void* cache, int64_t block_stride, int64_t num_blocks, int64_t page_size,
               const int32_t* indices, int64_t idx_sb, int64_t idx_ss, int64_t topk, const int32_t* lengths) {
    L.cache = static_cast<const uint8_t*>(cache);
    L.indices = indices;
    L.lengths = lengths;
    L.expanded = nullptr;
    L.num_entries = num_blocks * page_size;
    L.block_stride = block_stride;
    L.idx_stride_b = idx_sb;
    L.idx_stride_s = idx_ss;
    L.inv_page = 1.0 / (double)page_size;
    L.num_blocks = (int32_t)num_blocks;
    L.page_size = (int32_t)page_size;
    L.topk = (int32_t)topk;
    L.pad = 0;
}

int check_list(const void* cache, int64_t block_stride, int64_t num_blocks, int64_t page_size,
               const int32_t* indices, int64_t topk) {
    if (!cache || !indices)
        return fail(FGV_E_NULL_POINTER, "null cache or indices");
    if (page_size <= 0 || num_blocks < 0 || topk < 0)
        return fail(FGV_E_BAD_SHAPE, "page size must be positive, block count and top-k non-negative");
    if (page_size > 0x7fffffffLL / 64 || num_blocks > 0x7fffffffLL || topk > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "page size, block count and top-k must fit in int32");
    if (block_stride < page_size * (kTokenDataBytes + kScaleBytesPerToken))
        return fail(FGV_E_BAD_STRIDE, "cache block stride is below page_size * 584 bytes");
    if (!aligned(cache, 16) || block_stride % 16)
        return fail(FGV_E_MISALIGNED, "cache base and block stride must be 16-byte aligned");
    if (!aligned(indices, 4))
        return fail(FGV_E_MISALIGNED, "indices must be 4-byte aligned");
    return FGV_OK;
}

// Lists this long (in 32-entry chunks, main + extra) make the one-item-per-
// workgroup grid wait on its longest rows; from here on the split grid's
// balance outweighs the partials it writes.
constexpr int64_t kSplitMinChunks = 64;

int64_t chunks_of(int64_t topk) { return (topk + kChunk - 1) / kChunk; }

// Workgroups of the split grid: two per CU of the current device.
int split_grid() { return 2 * cu_count(); }

// The grids (fgv_sparse_mla_decode_grid's values).
enum MlaGrid { kGridOneItem = 0, kGridSplit = 1, kGridPair = 2 };

int64_t items_of(int64_t batch, int64_t seq_q, int64_t num_heads) { return batch * seq_q * (num_heads / kBlockHeads); }

// Lists this long (main + extra chunks) need the split or the paired grid.
bool long_lists(int64_t batch, int64_t items, int64_t topk, int64_t extra_topk) {
    return chunks_of(topk) + chunks_of(extra_topk) >= kSplitMinChunks && batch <= kMaxSplitRows &&
           4 * items <= 0x7fffffffLL;
}

// Long lists over more items than CUs but at most two per CU (and at most
// kPairMaxItems) take the paired grid: the items already fill the machine,
// so the split grid's partial slots and combine buy nothing that pairing a
// short item with a long one does not.  Short lists stay one workgroup per
// item: each item then waits on a few chunks only, and two items per CU in
// flight hide each other's latency (measured: the paired grid costs a few
// microseconds per item, which only long lists amortise).
bool pair_fits(int64_t batch, int64_t items, int64_t topk, int64_t extra_topk) {
    const int64_t cus = cu_count();
    return long_lists(batch, items, topk, extra_topk) && items > cus && items <= 2 * cus && items <= kPairMaxItems;
}

// The grid a call runs when it gets the workspace it asks for.
int mla_grid(int64_t batch, int64_t seq_q, int64_t num_heads, int64_t topk, int64_t extra_topk) {
    const int64_t items = items_of(batch, seq_q, num_heads);
    if (pair_fits(batch, items, topk, extra_topk))
        return kGridPair;
    return long_lists(batch, items, topk, extra_topk) ? kGridSplit : kGridOneItem;
}

// An extra list gathered at least this many times per cache entry (counting
// every row, query position and head block at its full top-k) is dequantised
// once per call into a bf16 copy in the workspace, up to this size; its chunks
// then skip the dequantisation (2.0 bytes of L2 -> LDS per byte of K instead
// of 1.14, no conversion, one barrier per chunk instead of two).
constexpr int64_t kExpandMinReuse = 8;
constexpr int64_t kExpandMaxBytes = 64LL << 20;
static_assert(kExpandMaxBytes / (2 * kHeadDim) <= (1LL << 31), "the expand kernel counts entries in 32 bits");

int64_t expand_bytes(int64_t batch, int64_t seq_q, int64_t num_heads, int64_t extra_topk, int64_t extra_entries) {
    if (extra_entries <= 0 || extra_topk <= 0 || extra_entries * 2 * kHeadDim > kExpandMaxBytes)
        return 0;
    const int64_t gathers = batch * seq_q * (num_heads / kBlockHeads) * extra_topk;
    return gathers >= kExpandMinReuse * extra_entries ? extra_entries * 2 * kHeadDim : 0;
}

int64_t split_bytes(int64_t batch, int64_t seq_q, int64_t num_heads, int64_t topk, int64_t extra_topk) {
    if (mla_grid(batch, seq_q, num_heads, topk, extra_topk) != kGridSplit)
        return 0;
    const int64_t slots = 2 * (int64_t)split_grid() * kSlotFloats * 4;
    return slots + ((batch + 1) * 4 + 255) / 256 * 256;
}

}  // namespace
}  // namespace fgv

extern "C" int64_t fgv_sparse_mla_decode_workspace_bytes(int64_t batch, int64_t seq_q, int64_t num_heads,
                                                         int64_t topk, int64_t extra_topk,
                                                         int64_t extra_num_entries) {
    if (batch <= 0 || seq_q <= 0 || num_heads <= 0 || num_heads % fgv::kBlockHeads || topk < 0 || extra_topk < 0 ||
        extra_num_entries < 0)
        return 0;
    return fgv::expand_bytes(batch, seq_q, num_heads, extra_topk, extra_num_entries) +
           fgv::split_bytes(batch, seq_q, num_heads, topk, extra_topk);
}

extern "C" int fgv_sparse_mla_decode_grid(int64_t batch, int64_t seq_q, int64_t num_heads, int64_t topk,
                                          int64_t extra_topk) {
    if (batch <= 0 || seq_q <= 0 || num_heads <= 0 || num_heads % fgv::kBlockHeads || topk < 0 || extra_topk < 0)
        return -1;
    return fgv::mla_grid(batch, seq_q, num_heads, topk, extra_topk);
}

// The argument list of fgv_sparse_mla_decode_model1 up to (not including) the
// workspace, shared by both entry points.
#define FGV_MLA_PARAMS                                                                                           \
    const void *q, int64_t q_stride_b, int64_t q_stride_s, int64_t q_stride_h, const void *k_cache,             \
        int64_t cache_block_stride, int64_t num_blocks, int64_t page_size, const int32_t *indices,               \
        int64_t idx_stride_b, int64_t idx_stride_s, int64_t topk, const int32_t *topk_length,                    \
        const void *extra_k_cache, int64_t extra_block_stride, int64_t extra_num_blocks, int64_t extra_page_size, \
        const int32_t *extra_indices, int64_t extra_idx_stride_b, int64_t extra_idx_stride_s, int64_t extra_topk, \
        const int32_t *extra_topk_length, const float *attn_sink, float softmax_scale, void *out,                \
        int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h, float *lse, int64_t lse_stride_b,      \
        int64_t lse_stride_h, int64_t batch, int64_t seq_q, int64_t num_heads
#define FGV_MLA_ARGS                                                                                        \
    q, q_stride_b, q_stride_s, q_stride_h, k_cache, cache_block_stride, num_blocks, page_size, indices,     \
        idx_stride_b, idx_stride_s, topk, topk_length, extra_k_cache, extra_block_stride, extra_num_blocks, \
        extra_page_size, extra_indices, extra_idx_stride_b, extra_idx_stride_s, extra_topk,                 \
        extra_topk_length, attn_sink, softmax_scale, out, out_stride_b, out_stride_s, out_stride_h, lse,    \
        lse_stride_b, lse_stride_h, batch, seq_q, num_heads

namespace fgv {
namespace {

int mla_decode(FGV_MLA_PARAMS, void* workspace, int64_t workspace_bytes, void* stream) {
    if (batch < 0 || seq_q < 0 || num_heads < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (num_heads % kBlockHeads)
        return fail(FGV_E_BAD_SHAPE, "num_heads must be a multiple of 64");
    if (batch == 0 || seq_q == 0 || num_heads == 0)
        return FGV_OK;
    if (batch * seq_q * (num_heads / kBlockHeads) > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "batch * seq_q * num_heads / 64 must be below 2^31");
    if (!q || !out || !lse)
        return fail(FGV_E_NULL_POINTER, "null q, out or lse");
    if (!aligned(q, 16) || q_stride_b % 8 || q_stride_s % 8 || q_stride_h % 8)
        return fail(FGV_E_MISALIGNED, "q must be 16-byte aligned with strides a multiple of 8 elements");
    if (!aligned(out, 16) || out_stride_b % 8 || out_stride_s % 8 || out_stride_h % 8)
        return fail(FGV_E_MISALIGNED, "out must be 16-byte aligned with strides a multiple of 8 elements");
    if (!aligned(lse, 4))
        return fail(FGV_E_MISALIGNED, "lse must be 4-byte aligned");
    int rc = check_list(k_cache, cache_block_stride, num_blocks, page_size, indices, topk);
    if (rc)
        return rc;
    MlaArgs a;
    a.num_lists = 1;
    fill_list(a.list[0], k_cache, cache_block_stride, num_blocks, page_size, indices, idx_stride_b,
              idx_stride_s, topk, topk_length);
    if (extra_k_cache) {
        rc = check_list(extra_k_cache, extra_block_stride, extra_num_blocks, extra_page_size, extra_indices,
                        extra_topk);
        if (rc)
            return rc;
        fill_list(a.list[1], extra_k_cache, extra_block_stride, extra_num_blocks, extra_page_size,
                  extra_indices, extra_idx_stride_b, extra_idx_stride_s, extra_topk, extra_topk_length);
        a.num_lists = 2;
    } else if (extra_indices || extra_topk_length) {
        return fail(FGV_E_BAD_SHAPE, "extra indices or lengths given without an extra cache");
    } else {
        a.list[1] = a.list[0];
    }
    a.q = static_cast<const uint16_t*>(q);
    a.q_sb = q_stride_b;
    a.q_ss = q_stride_s;
    a.q_sh = q_stride_h;
    a.out = static_cast<uint16_t*>(out);
    a.o_sb = out_stride_b;
    a.o_ss = out_stride_s;
    a.o_sh = out_stride_h;
    a.lse = lse;
    a.l_sb = lse_stride_b;
    a.l_sh = lse_stride_h;
    a.sink = attn_sink;
    a.batch = (int32_t)batch;
    a.seq_q = (int32_t)seq_q;
    a.head_blocks = (int32_t)(num_heads / kBlockHeads);
    a.scale_log2 = (float)((double)softmax_scale * 1.4426950408889634);
    a.partials = nullptr;
    a.row_prefix = nullptr;
    a.split_grid = 0;
    a.pair_cus = 0;
    a.order_windows = 0;
    const int64_t items = batch * seq_q * a.head_blocks;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Workspace: [expanded extra cache][split slots][row prefix sums].  A
    // workspace too small for both drops the expansion first, then the split.
    // (the combine kernel runs four workgroups per item)
    const int64_t need_split = split_bytes(batch, seq_q, num_heads, topk, extra_k_cache ? extra_topk : 0);
    const int64_t need_expand =
        extra_k_cache ? expand_bytes(batch, seq_q, num_heads, extra_topk, a.list[1].num_entries) : 0;
    const int64_t have = workspace ? workspace_bytes : 0;
    const bool use_expand = need_expand > 0 && have >= need_expand + need_split;
    const bool use_split = need_split > 0 && have >= need_split + (use_expand ? need_expand : 0);
    if ((use_expand || use_split) && !aligned(workspace, 256))
        return fail(FGV_E_MISALIGNED, "workspace must be 256-byte aligned");
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (use_expand) {
        a.list[1].expanded = ws;
        const int64_t entries = a.list[1].num_entries;
        constexpr int64_t wide = expand_per_block<4>(), narrow = expand_per_block<2>();
        if (entries >= kExpandWideMinBlocks * wide)
            hipLaunchKernelGGL(mla_expand_cache_kernel<4>, dim3((unsigned)((entries + wide - 1) / wide)),
                               dim3(kThreads), 0, st, a.list[1], ws);
        else
            hipLaunchKernelGGL(mla_expand_cache_kernel<2>, dim3((unsigned)((entries + narrow - 1) / narrow)),
                               dim3(kThreads), 0, st, a.list[1], ws);
        rc = launch_status();
        if (rc)
            return rc;
        ws += need_expand;
    }
    if (use_split) {
        a.split_grid = split_grid();
        a.partials = reinterpret_cast<float*>(ws);
        a.row_prefix = reinterpret_cast<int32_t*>(ws + 2 * (int64_t)a.split_grid * kSlotFloats * 4);
        hipLaunchKernelGGL(sparse_mla_decode_split_kernel, dim3((unsigned)a.split_grid), dim3(kThreads), 0, st, a);
        rc = launch_status();
        if (rc)
            return rc;
        hipLaunchKernelGGL(sparse_mla_combine_kernel, dim3((unsigned)(4 * items)), dim3(kThreads), 0, st, a);
        return launch_status();
    }
    if (pair_fits(batch, items, topk, extra_k_cache ? extra_topk : 0)) {
        hipLaunchKernelGGL(sparse_mla_decode_pair_kernel, dim3((unsigned)min(items, (int64_t)cu_count())),
                           dim3(kPairThreads), 0, st, a);
        return launch_status();
    }
    // one round: items in runs per XCD while each has a CU to itself, paired
    // long with short once two share one; three or four rounds: longest
    // first in windows; more rounds: in order
    const int64_t cus = cu_count();
    if (items > cus && items <= 2 * cus) {
        a.pair_cus = (int32_t)cus;
        // with at least one unpartnered workgroup per two pairs, the fewest
        // windows whose largest (2 ceil(P / W) + ceil(S / W) items) fits a
        // wave; else pairs only (0)
        const int64_t pairs = items - cus, alone = cus - pairs;
        int64_t windows = 0;
        if (2 * alone >= pairs) {
            windows = 1;
            while (2 * ((pairs + windows - 1) / windows) + (alone + windows - 1) / windows > 64)
                ++windows;
        }
        a.order_windows = (int32_t)windows;
        if (windows)
            hipLaunchKernelGGL(sparse_mla_decode_kernel<kItemsPairedMixed>, dim3((unsigned)items), dim3(kThreads), 0,
                               st, a);
        else
            hipLaunchKernelGGL(sparse_mla_decode_kernel<kItemsPaired>, dim3((unsigned)items), dim3(kThreads), 0, st, a);
    } else if (items <= cus) {
        hipLaunchKernelGGL(sparse_mla_decode_kernel<kItemsInRuns>, dim3((unsigned)items), dim3(kThreads), 0, st, a);
    } else if (items <= 4 * cus) {
        hipLaunchKernelGGL(sparse_mla_decode_kernel<kItemsLongestFirst>, dim3((unsigned)items), dim3(kThreads), 0,
                           st, a);
    } else {
        hipLaunchKernelGGL(sparse_mla_decode_kernel<kItemsInOrder>, dim3((unsigned)items), dim3(kThreads), 0, st, a);
    }
    return launch_status();
}

// ---- the no-allocation entry point's scratch: a fixed device array in
// place of the caller's workspace.  Each device that loads the library holds
// its own copy until the process ends.  Nothing in it needs clearing between
// calls: every byte a call reads (the expanded cache, the split partial
// slots, the row prefix sums) is written earlier in the same call.
constexpr int64_t kScratchBytes = FGV_MLA_NO_ALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the current device, looked up once per
// device with that device current (the array's name in host code is only a
// host-side stand-in).
int scratch_of_current_device(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(FGV_E_BAD_SHAPE, "device index beyond the 64 devices the scratch table holds");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return static_cast<int>(e);
        if (!p)
            return fail(FGV_E_NULL_POINTER, "hipGetSymbolAddress gave no address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return FGV_OK;
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_sparse_mla_decode_model1(FGV_MLA_PARAMS, void* workspace, int64_t workspace_bytes,
                                            void* stream) {
    return fgv::mla_decode(FGV_MLA_ARGS, workspace, workspace_bytes, stream);
}

extern "C" int fgv_sparse_mla_decode_model1_no_alloc(FGV_MLA_PARAMS, void* stream) {
    using namespace fgv;
    // the schedule fgv_sparse_mla_decode_model1 runs with the workspace the
    // query asks for, or an error when that does not fit the scratch
    const int64_t extra_entries = extra_k_cache ? extra_num_blocks * extra_page_size : 0;
    const int64_t need = fgv_sparse_mla_decode_workspace_bytes(batch, seq_q, num_heads, topk,
                                                               extra_k_cache ? extra_topk : 0, extra_entries);
    if (need > kScratchBytes)
        return fail(FGV_E_TOO_LARGE,
                    "fgv_sparse_mla_decode_model1_no_alloc: this call's schedule needs more workspace than the "
                    "64 MiB scratch (fgv_sparse_mla_decode_workspace_bytes); call "
                    "fgv_sparse_mla_decode_model1 with a workspace instead");
    void* ws = nullptr;
    if (need > 0) {
        const int rc = scratch_of_current_device(&ws);
        if (rc)
            return rc;
    }
    return mla_decode(FGV_MLA_ARGS, ws, need, stream);
}

// Sparse prefill over bf16 rows (sparse_mla_prefill_kernel).
extern "C" int fgv_flash_mla_sparse_fwd(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* kv,
                                        int64_t kv_stride_row, int64_t s_kv, const int32_t* indices,
                                        int64_t idx_stride_t, int64_t topk, const int32_t* topk_length,
                                        const float* attn_sink, float sm_scale, int64_t s_q, int64_t h_q,
                                        int64_t d_qk, void* out, int64_t out_stride_t, int64_t out_stride_h,
                                        float* max_logits, int64_t max_logits_stride_t, float* lse,
                                        int64_t lse_stride_t, void* stream) {
    using namespace fgv;
    if (s_q < 0 || h_q < 0 || s_kv < 0 || topk < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (d_qk != kHeadDim && d_qk != kHeadDim + kTailDim)
        return fail(FGV_E_BAD_SHAPE, "d_qk must be 512 or 576");
    if (h_q % kBlockHeads)
        return fail(FGV_E_BAD_SHAPE, "h_q must be a multiple of 64");
    if (s_q == 0 || h_q == 0)
        return FGV_OK;
    if (kv_stride_row < d_qk)
        return fail(FGV_E_BAD_STRIDE, "kv rows overlap (kv_stride_row < d_qk)");
    if (out_stride_h < kHeadDim || out_stride_t < h_q * out_stride_h || max_logits_stride_t < h_q ||
        lse_stride_t < h_q)
        return fail(FGV_E_BAD_STRIDE, "out, max_logits or lse rows overlap");
    if (s_q * (h_q / kBlockHeads) > 0x7fffffffLL || s_kv > 0x7fffffffLL || topk > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "s_q * h_q / 64, s_kv and topk must fit in int32");
    if (!q || !out || !lse || !max_logits || (topk > 0 && (!indices || (s_kv > 0 && !kv))))
        return fail(FGV_E_NULL_POINTER, "null q, kv, indices, out, max_logits or lse");
    if (!aligned(q, 16) || q_stride_t % 8 || q_stride_h % 8)
        return fail(FGV_E_MISALIGNED, "q must be 16-byte aligned with strides a multiple of 8 elements");
    if (!aligned(out, 16) || out_stride_t % 8 || out_stride_h % 8)
        return fail(FGV_E_MISALIGNED, "out must be 16-byte aligned with strides a multiple of 8 elements");
    if (!aligned(kv, 16) || kv_stride_row % 8)
        return fail(FGV_E_MISALIGNED, "kv must be 16-byte aligned with a row stride a multiple of 8 elements");
    if (!aligned(indices, 4) || !aligned(lse, 4) || !aligned(max_logits, 4))
        return fail(FGV_E_MISALIGNED, "indices, lse and max_logits must be 4-byte aligned");
    PrefillArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.q_st = q_stride_t;
    a.q_sh = q_stride_h;
    a.kv = static_cast<const uint8_t*>(kv);
    a.kv_row_bytes = 2 * kv_stride_row;
    a.indices = indices;
    a.idx_st = idx_stride_t;
    a.topk_length = topk_length;
    a.sink = attn_sink;
    a.out = static_cast<uint16_t*>(out);
    a.o_st = out_stride_t;
    a.o_sh = out_stride_h;
    a.max_logits = max_logits;
    a.lse = lse;
    a.ml_st = max_logits_stride_t;
    a.l_st = lse_stride_t;
    a.s_kv = (int32_t)s_kv;
    a.topk = (int32_t)topk;
    a.head_blocks = (int32_t)(h_q / kBlockHeads);
    a.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
    const dim3 grid((unsigned)(s_q * a.head_blocks));
    if (d_qk == kHeadDim)
        hipLaunchKernelGGL(sparse_mla_prefill_kernel<false>, grid, dim3(kThreads), 0,
                           static_cast<hipStream_t>(stream), a);
    else
        hipLaunchKernelGGL(sparse_mla_prefill_kernel<true>, grid, dim3(kThreads), 0,
                           static_cast<hipStream_t>(stream), a);
    return launch_status();
}
