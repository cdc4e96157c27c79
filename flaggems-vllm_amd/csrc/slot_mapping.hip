// gfx950 kernel for paged-KV slot-mapping generation: the step that produces
// the slot_mapping consumed by qnorm_rope_kv_insert_kernel.
//
// Reference semantics: src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:42-144
// (vLLM's per-request slot-mapping kernel, parallelised):
//   for token t of request r (query_start_loc[r] <= t < query_start_loc[r+1]):
//     pos = positions[t]; vbs = block_size * cp_world
//     blk = block_table[r, pos / vbs]; voff = pos % vbs
//     slot = blk * block_size + (voff / (cp_world*il)) * il + voff % il
//            if (voff / il) % cp_world == cp_rank, else pad_id
//   tokens num_tokens..max_num_tokens-1 get pad_id.
//
// One thread per output slot; the owning request is found by binary search
// over query_start_loc (num_reqs + 1 int32 values, cache resident), so the
// grid does not depend on how tokens split into requests.  Slots are
// computed in int64 (the reference's int32 product would wrap past 2^31).
#include "fgv_device.h"
#include "fgv_host.h"

namespace fgv {
namespace {

constexpr int kThreads = 256;

struct SlotArgs {
    const int32_t* qsl;
    const void* positions;
    const int32_t* block_table;
    int64_t* out;
    int64_t bt_stride;
    int64_t pad_id;
    int32_t num_tokens, max_num_tokens, num_reqs;
    int32_t block_size, cp_world, cp_rank, interleave;
    int32_t max_blocks;
    int pos64;
};

__global__ void __launch_bounds__(kThreads)
slot_mapping_kernel(SlotArgs a) {
    const int32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= a.max_num_tokens)
        return;
    if (t >= a.num_tokens) {
        a.out[t] = a.pad_id;
        return;
    }
    if (a.num_reqs == 0)
        return;
    // largest r < num_reqs with qsl[r] <= t
    int32_t lo = 0, hi = a.num_reqs - 1;
    while (lo < hi) {
        const int32_t mid = (lo + hi + 1) >> 1;
        if (a.qsl[mid] <= t)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int32_t r = lo;
    if (t < a.qsl[r] || t >= a.qsl[r + 1])
        return;  // not inside any request: left as it is
    const int32_t pos = a.pos64 ? (int32_t) static_cast<const int64_t*>(a.positions)[t]
                                : static_cast<const int32_t*>(a.positions)[t];
    const int32_t vbs = a.block_size * a.cp_world;
    const int32_t bi = pos / vbs;
    if (pos < 0 || bi >= a.max_blocks) {
        a.out[t] = a.pad_id;  // outside the block table: not a cache slot
        return;
    }
    const int64_t blk = a.block_table[(int64_t)r * a.bt_stride + bi];
    const int32_t voff = pos - bi * vbs;
    const bool local = (voff / a.interleave) % a.cp_world == a.cp_rank;
    const int32_t loff = voff / (a.cp_world * a.interleave) * a.interleave + voff % a.interleave;
    a.out[t] = local ? blk * a.block_size + loff : a.pad_id;
}

}  // namespace
}  // namespace fgv

extern "C" int fgv_compute_slot_mapping(
    int64_t num_tokens, int64_t max_num_tokens,
    const int32_t* query_start_loc, int64_t num_reqs,
    const void* positions, int positions_are_int64,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_req,
    int64_t* slot_mapping, int64_t block_size,
    int64_t cp_world_size, int64_t cp_rank, int64_t cp_kv_cache_interleave_size,
    int64_t pad_id, void* stream) {
    using namespace fgv;
    if (num_tokens < 0 || max_num_tokens < 0 || num_reqs < 0)
        return fail(FGV_E_BAD_SHAPE, "negative size");
    if (max_num_tokens == 0)
        return FGV_OK;
    if (max_num_tokens > 0x7fffffffLL || num_reqs > 0x7ffffffeLL || max_blocks_per_req > 0x7fffffffLL)
        return fail(FGV_E_TOO_LARGE, "sizes must fit in int32");
    if (block_size <= 0 || cp_world_size <= 0 || cp_kv_cache_interleave_size <= 0 ||
        cp_rank < 0 || cp_rank >= cp_world_size ||
        block_size * cp_world_size > 0x7fffffffLL)
        return fail(FGV_E_BAD_SHAPE, "bad block_size or context-parallel geometry");
    if (!slot_mapping || (num_tokens > 0 && num_reqs > 0 && (!query_start_loc || !positions || !block_table)))
        return fail(FGV_E_NULL_POINTER, "null pointer argument");
    if (!aligned(slot_mapping, 8))
        return fail(FGV_E_MISALIGNED, "slot_mapping must be 8-byte aligned");

    SlotArgs a;
    a.qsl = query_start_loc;
    a.positions = positions;
    a.block_table = block_table;
    a.out = slot_mapping;
    a.bt_stride = block_table_stride;
    a.pad_id = pad_id;
    a.num_tokens = (int32_t)(num_tokens < max_num_tokens ? num_tokens : max_num_tokens);
    a.max_num_tokens = (int32_t)max_num_tokens;
    a.num_reqs = (int32_t)num_reqs;
    a.block_size = (int32_t)block_size;
    a.cp_world = (int32_t)cp_world_size;
    a.cp_rank = (int32_t)cp_rank;
    a.interleave = (int32_t)cp_kv_cache_interleave_size;
    a.max_blocks = (int32_t)max_blocks_per_req;
    a.pos64 = positions_are_int64 ? 1 : 0;
    const dim3 grid((unsigned)((max_num_tokens + kThreads - 1) / kThreads));
    hipLaunchKernelGGL(slot_mapping_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
    return launch_status();
}
