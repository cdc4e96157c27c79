// Host-side torch bindings of the path's ops:
//   fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert  (reference wrapper
//     src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:289-351)
//   fused_inv_rope_fp8_quant                            (reference wrapper
//     src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:157-256)
// and of the four ops beside them (fused_q_kv_rmsnorm,
// dequantize_and_gather_k_cache, fused_indexer_q_rope_quant,
// compute_slot_mapping_parallel).
//
// The argument checks, the output allocation and the launch run here in C++,
// so an eager call costs a few microseconds of host time instead of the
// Python asserts plus a ctypes call of some twenty arguments.  The main op and
// the sibling are reachable two ways, both ending in the same function:
//   - the module functions (pybind11), which the Python drop-ins call.  They
//     return a status: 0, kAssertFailed (a reference assertion failed: the
//     Python side raises AssertionError with assert_message()), or the C ABI's
//     code (negative: argument error, positive: hipError_t);
//   - the dispatcher ops torch.ops.flaggems_vllm.<name> (TORCH_LIBRARY_FRAGMENT;
//     schemas mark q and k_cache written), for torch.compile and graph capture.
//     These raise RuntimeError on any failure, as vLLM's own compiled op does.
// The other four are module functions only; their torch.ops registrations
// call the Python drop-ins.
// Launches go on torch's current HIP stream of the tensors' device; nothing
// synchronises and nothing is read back from the device.
#include <torch/extension.h>
#include <torch/library.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <string>
#include <tuple>

#include "flaggems_vllm_amd.h"

namespace {

constexpr int kAssertFailed = -1000;
constexpr int64_t kHeadDim = 512;
constexpr int64_t kRopeDim = 64;

thread_local std::string g_assert_message;

int assert_failed(const char* msg) {
    g_assert_message = msg;
    return kAssertFailed;
}

#define FGV_ASSERT(cond, msg)              \
    do {                                   \
        if (!(cond))                       \
            return assert_failed(msg);     \
    } while (0)

void* current_stream(const at::Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Whether each block t[i] is contiguous bytes: the dims after the first are
// dense in row-major order (dims of size 1 may have any stride), the test
// Tensor.is_contiguous() makes on t[0].
bool blocks_contiguous(const at::Tensor& t) {
    int64_t expected = 1;
    for (int64_t d = t.dim() - 1; d >= 1; --d) {
        const int64_t n = t.size(d);
        if (n != 1 && t.stride(d) != expected)
            return false;
        expected *= n;
    }
    return true;
}

// The reference's assertions (same conditions, same order), the extensions
// documented in the Python drop-in (strided q and kv, cos_sin row stride, a
// 1-D cache as one block), then one C-ABI launch.
int qnorm_rope_kv_insert(const at::Tensor& q, const at::Tensor& kv, const at::Tensor& k_cache,
                         const at::Tensor& slot_mapping, const at::Tensor& position_ids,
                         const at::Tensor& cos_sin_cache, double eps, int64_t cache_block_size) {
    FGV_ASSERT(q.dim() == 3 && kv.dim() == 2, "q must be 3-D and kv 2-D");
    FGV_ASSERT(q.stride(2) == 1 && kv.stride(1) == 1, "q and kv need a unit last stride");
    const int64_t num_tokens = q.size(0), num_heads = q.size(1);
    FGV_ASSERT(q.size(2) == kHeadDim, "q's head_dim must be 512");
    FGV_ASSERT(kv.size(0) == num_tokens && kv.size(1) == kHeadDim, "kv must be [num_tokens, 512]");
    FGV_ASSERT(q.scalar_type() == at::kBFloat16 && kv.scalar_type() == at::kBFloat16,
               "q and kv must be bfloat16");
    FGV_ASSERT(k_cache.scalar_type() == at::kByte, "k_cache must be uint8");
    FGV_ASSERT(slot_mapping.dim() == 1, "slot_mapping must be 1-D");
    const int64_t num_tokens_insert = slot_mapping.size(0);
    FGV_ASSERT(num_tokens_insert <= num_tokens, "slot_mapping is longer than the number of tokens");
    FGV_ASSERT(slot_mapping.scalar_type() == at::kLong, "slot_mapping must be int64");
    FGV_ASSERT(position_ids.dim() == 1 && position_ids.size(0) == num_tokens,
               "position_ids must be [num_tokens]");
    FGV_ASSERT(position_ids.scalar_type() == at::kLong, "position_ids must be int64");
    FGV_ASSERT(cos_sin_cache.dim() == 2 && cos_sin_cache.size(1) == kRopeDim,
               "cos_sin_cache must be [max_pos, 64]");
    FGV_ASSERT(cos_sin_cache.scalar_type() == at::kFloat, "cos_sin_cache must be float32");
    FGV_ASSERT(cos_sin_cache.stride(1) == 1, "cos_sin_cache rows must be contiguous");
    FGV_ASSERT(slot_mapping.stride(0) == 1 || num_tokens_insert <= 1, "slot_mapping must be contiguous");
    FGV_ASSERT(position_ids.stride(0) == 1 || num_tokens <= 1, "position_ids must be contiguous");
    FGV_ASSERT(k_cache.dim() >= 1 && blocks_contiguous(k_cache), "each k_cache block must be contiguous bytes");
    const c10::Device dev = q.device();
    FGV_ASSERT(kv.device() == dev && k_cache.device() == dev && slot_mapping.device() == dev &&
                   position_ids.device() == dev && cos_sin_cache.device() == dev,
               "all tensors must be on q's device");
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");

    if (num_tokens == 0)
        return 0;
    // A [num_blocks, block_bytes] cache (or more dims) has size(0) blocks,
    // stride(0) bytes apart; a 1-D cache is one block of numel bytes.
    const bool one_block = k_cache.dim() == 1;
    const int64_t num_blocks = one_block ? 1 : k_cache.size(0);
    const int64_t block_stride = one_block ? k_cache.numel() : k_cache.stride(0);
    const c10::DeviceGuard guard(dev);
    return fgv_qnorm_rope_kv_rope_quant_insert(
        q.data_ptr(), q.stride(0), q.stride(1), kv.data_ptr(), kv.stride(0), k_cache.data_ptr(), block_stride,
        num_blocks, slot_mapping.data_ptr<int64_t>(), num_tokens_insert, position_ids.data_ptr<int64_t>(),
        cos_sin_cache.data_ptr<float>(), cos_sin_cache.stride(0), cos_sin_cache.size(0), num_tokens, num_heads,
        static_cast<float>(eps), cache_block_size, current_stream(q));
}

using SiblingOut = std::tuple<at::Tensor, at::Tensor>;

// The reference's assertions in its order (:184-205, plus this build's
// geometry limits), its output allocation (:207-227): codes [G, T, hpg * D]
// e4m3fn and scales stored (G, K, Tpad4) token-fastest, returned transposed to
// [T, G, d] and [T, G, K]; then one C-ABI launch.
int inv_rope_fp8_quant(const at::Tensor& o, const at::Tensor& positions_in, const at::Tensor& cos_sin_cache,
                       int64_t n_groups, int64_t heads_per_group, int64_t nope_dim, int64_t rope_dim,
                       int64_t quant_group_size, double eps, bool fp8_e4m3fn, bool tma_aligned_scales,
                       SiblingOut* out) {
    FGV_ASSERT(fp8_e4m3fn, "only torch.float8_e4m3fn is supported");
    FGV_ASSERT(o.dim() == 3, "`o` must be [num_tokens, num_heads, head_dim]");
    FGV_ASSERT(positions_in.dim() == 1, "`positions` must be 1D");
    FGV_ASSERT(cos_sin_cache.dim() == 2, "`cos_sin_cache` must be 2D");
    FGV_ASSERT(o.stride(2) == 1, "head_dim must be contiguous");
    FGV_ASSERT(positions_in.size(0) == o.size(0), "positions and o token count mismatch");
    const int64_t num_tokens = o.size(0), num_heads = o.size(1), head_dim = o.size(2);
    FGV_ASSERT(num_heads == n_groups * heads_per_group, "num_heads must be n_groups * heads_per_group");
    FGV_ASSERT(head_dim == nope_dim + rope_dim, "head_dim must be nope_dim + rope_dim");
    FGV_ASSERT(quant_group_size > 0 && head_dim % quant_group_size == 0,
               "head_dim must be a multiple of quant_group_size");
    FGV_ASSERT(nope_dim % quant_group_size == quant_group_size - rope_dim,
               "nope_dim % quant_group_size must be quant_group_size - rope_dim");
    FGV_ASSERT(rope_dim % 2 == 0, "rope_dim must be even");
    FGV_ASSERT(cos_sin_cache.size(1) == rope_dim, "cos_sin_cache's last dim must be rope_dim");
    FGV_ASSERT(cos_sin_cache.scalar_type() == at::kFloat, "cos_sin_cache must be float32");
    FGV_ASSERT((head_dim & (head_dim - 1)) == 0 && head_dim >= 8 && head_dim <= 512 &&
                   (quant_group_size & (quant_group_size - 1)) == 0 && quant_group_size >= 8,
               "this build takes head_dim a power of two in [8, 512] and quant_group_size a power of two >= 8");
    FGV_ASSERT(o.scalar_type() == at::kBFloat16, "`o` must be bfloat16");
    FGV_ASSERT(cos_sin_cache.stride(1) == 1, "cos_sin_cache rows must be contiguous");
    const c10::Device dev = o.device();
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");
    FGV_ASSERT(positions_in.device() == dev && cos_sin_cache.device() == dev, "all tensors must be on o's device");
    const int64_t chunks_per_head = head_dim / quant_group_size;
    if (tma_aligned_scales) {
        FGV_ASSERT(chunks_per_head <= 4, "packed UE8M0 path currently expects at most 4 scale blocks per head");
        // the reference's packed tensor holds (hpg * chunks + 3) / 4 words per
        // (group, token) and its kernel writes one per head: below four chunks
        // that is past the tensor unless there is one head per group
        FGV_ASSERT(chunks_per_head == 4 || heads_per_group == 1,
                   "packed scales with fewer than 4 scale blocks per head need heads_per_group 1");
    }

    const at::Tensor positions = (positions_in.scalar_type() != at::kLong || positions_in.stride(0) != 1)
                                     ? positions_in.to(at::kLong).contiguous()
                                     : positions_in;
    const int64_t d = heads_per_group * head_dim;
    const int64_t num_scale_blocks = d / quant_group_size;
    const int64_t tpad = (num_tokens + 3) / 4 * 4;
    const int64_t scale_inner = tma_aligned_scales ? (num_scale_blocks + 3) / 4 : num_scale_blocks;
    const auto opts = o.options();
    // both outputs allocated straight in the returned layouts (no transposed
    // views to make): codes [T, G, d] over storage [G][T][d]; scales
    // [T, G, K] over storage [G][K][Tpad] (all Tpad columns: the kernel writes
    // the padding tokens' zero scales)
    at::Tensor fp8 = at::empty_strided({num_tokens, n_groups, d}, {d, num_tokens * d, 1},
                                       opts.dtype(at::kFloat8_e4m3fn));
    at::Tensor scale = at::empty({n_groups * scale_inner * tpad}, opts.dtype(tma_aligned_scales ? at::kInt : at::kFloat))
                           .as_strided({num_tokens, n_groups, scale_inner}, {1, scale_inner * tpad, tpad});
    int rc = 0;
    if (tpad > 0) {
        const c10::DeviceGuard guard(dev);
        rc = fgv_inv_rope_fp8_quant(o.data_ptr(), o.stride(0), o.stride(1), positions.data_ptr<int64_t>(),
                                    cos_sin_cache.data_ptr<float>(), cos_sin_cache.stride(0), cos_sin_cache.size(0),
                                    num_tokens, n_groups, heads_per_group, nope_dim, rope_dim, quant_group_size,
                                    fp8.data_ptr(), fp8.stride(1),
                                    fp8.stride(0), scale.data_ptr(), scale.stride(1), scale.stride(2), tpad,
                                    static_cast<float>(eps), tma_aligned_scales ? 1 : 0, current_stream(o));
    }
    *out = SiblingOut(fp8, scale);
    return rc;
}

// ---- the ops beside the path: checks, allocation and launch of their Python drop-ins ----

using TensorPair = std::tuple<at::Tensor, at::Tensor>;

int32_t* i32_ptr(const at::Tensor& t) { return t.data_ptr<int32_t>(); }

at::Tensor to_i32(const at::Tensor& t) { return t.scalar_type() == at::kInt ? t : t.to(at::kInt); }

// fused_q_kv_rmsnorm (reference wrapper
// src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:65-103):
// outputs like qr and kv, one C-ABI launch.
int q_kv_rmsnorm(const at::Tensor& qr, const at::Tensor& kv, const at::Tensor& q_weight, const at::Tensor& kv_weight,
                 double eps, TensorPair* out) {
    FGV_ASSERT(qr.dim() == 2 && kv.dim() == 2, "qr and kv must be 2D [num_tokens, size]");
    FGV_ASSERT(qr.size(0) == kv.size(0), "qr and kv token count mismatch");
    FGV_ASSERT(qr.stride(-1) == 1 && kv.stride(-1) == 1, "qr and kv rows must be contiguous");
    FGV_ASSERT(q_weight.is_contiguous() && kv_weight.is_contiguous(), "weights must be contiguous");
    const int64_t q_size = qr.size(1), kv_size = kv.size(1), num_tokens = qr.size(0);
    at::Tensor qr_out = at::empty_like(qr), kv_out = at::empty_like(kv);
    *out = TensorPair(qr_out, kv_out);
    if (num_tokens == 0)
        return 0;
    FGV_ASSERT(qr.scalar_type() == at::kBFloat16 && kv.scalar_type() == at::kBFloat16, "bf16 activations");
    FGV_ASSERT(q_weight.scalar_type() == kv_weight.scalar_type() &&
                   (q_weight.scalar_type() == at::kBFloat16 || q_weight.scalar_type() == at::kFloat),
               "weights must be both bf16 or both float32");
    FGV_ASSERT(q_weight.numel() == q_size && kv_weight.numel() == kv_size, "weight sizes must match the row sizes");
    const c10::Device dev = qr.device();
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");
    FGV_ASSERT(kv.device() == dev && q_weight.device() == dev && kv_weight.device() == dev,
               "all tensors must be on qr's device");
    const c10::DeviceGuard guard(dev);
    return fgv_fused_q_kv_rmsnorm(qr.data_ptr(), qr.stride(0), qr_out.data_ptr(), qr_out.stride(0),
                                  q_weight.data_ptr(), q_size, kv.data_ptr(), kv.stride(0), kv_out.data_ptr(),
                                  kv_out.stride(0), kv_weight.data_ptr(), kv_size, num_tokens,
                                  static_cast<float>(eps), q_weight.scalar_type() == at::kFloat ? 1 : 0,
                                  current_stream(qr));
}

// dequantize_and_gather_k_cache (reference wrapper
// src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:123-172):
// out written in place; int64 index tensors converted to int32.
int dequantize_gather(const at::Tensor& out, const at::Tensor& k_cache, const at::Tensor& seq_lens_in,
                      const std::optional<at::Tensor>& gather_lens_in, const at::Tensor& block_table_in,
                      int64_t block_size, int64_t offset, int64_t rope_dim, std::optional<int64_t> nope_dim_in,
                      std::optional<int64_t> scale_slots_in) {
    FGV_ASSERT(out.dim() == 3 && out.scalar_type() == at::kBFloat16, "out must be 3D bfloat16");
    FGV_ASSERT(seq_lens_in.dim() == 1 && block_table_in.dim() == 2, "seq_lens must be 1D and block_table 2D");
    FGV_ASSERT(seq_lens_in.size(0) == block_table_in.size(0) && block_table_in.size(0) <= out.size(0),
               "seq_lens, block_table and out must agree on the request count");
    const int64_t nope_dim = nope_dim_in.has_value() ? *nope_dim_in : out.size(2) - rope_dim;
    const int64_t scale_slots =
        scale_slots_in.has_value() ? *scale_slots_in : (nope_dim + 63) / 64 + (nope_dim % 64 == 0 ? 1 : 0);
    FGV_ASSERT(nope_dim + rope_dim <= out.size(2), "nope_dim + rope_dim must fit out's last dim");
    FGV_ASSERT(k_cache.dim() == 2 || k_cache.dim() == 3, "k_cache must be 2D or 3D");
    FGV_ASSERT(out.stride(2) == 1, "out rows must be contiguous");
    FGV_ASSERT(blocks_contiguous(k_cache), "each k_cache block must be contiguous bytes");
    FGV_ASSERT(block_table_in.stride(1) == 1, "block_table rows must be contiguous");
    const c10::Device dev = out.device();
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");
    FGV_ASSERT(k_cache.device() == dev && seq_lens_in.device() == dev && block_table_in.device() == dev &&
                   (!gather_lens_in.has_value() || gather_lens_in->device() == dev),
               "all tensors must be on out's device");
    const at::Tensor seq_lens = to_i32(seq_lens_in).contiguous();
    const at::Tensor gather_lens =
        gather_lens_in.has_value() ? to_i32(*gather_lens_in).contiguous() : at::Tensor();
    const at::Tensor block_table = to_i32(block_table_in);
    const int64_t num_reqs = seq_lens.size(0);
    if (num_reqs == 0)
        return 0;
    const c10::DeviceGuard guard(dev);
    return fgv_dequantize_and_gather_k_cache(
        out.data_ptr(), out.stride(0), out.stride(1), out.size(1), k_cache.data_ptr(), k_cache.stride(0),
        k_cache.size(0), i32_ptr(seq_lens), gather_lens.defined() ? i32_ptr(gather_lens) : nullptr,
        i32_ptr(block_table), block_table.stride(0), block_table.size(1), num_reqs, block_size, offset, nope_dim,
        rope_dim, scale_slots, current_stream(out));
}

using IndexerOut = std::tuple<at::Tensor, at::Tensor, at::Tensor>;

// fused_indexer_q_rope_quant (reference wrapper
// src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py:285-410): returns
// (q codes, the UE8M0 scale bytes viewed as int32 [T, H, D/128] and squeezed
// to [T, H] for D = 128 (MXFP4), or an undefined tensor (FP8), folded weights).
int indexer_q_rope_quant(const at::Tensor& positions_in, const at::Tensor& index_q, const at::Tensor& cos_sin,
                         const at::Tensor& weights, double softmax_scale, double head_scale, bool use_fp4,
                         IndexerOut* out) {
    FGV_ASSERT(positions_in.dim() == 1, "positions must be 1D");
    FGV_ASSERT(index_q.dim() == 3, "index_q must be [num_tokens, num_heads, head_dim]");
    FGV_ASSERT(cos_sin.dim() == 2, "index_q_cos_sin_cache must be 2D");
    const int64_t num_tokens = positions_in.size(0), num_heads = index_q.size(1), head_dim = index_q.size(2);
    at::Tensor weights_out = at::empty_like(weights, weights.options().dtype(at::kFloat));
    FGV_ASSERT(index_q.scalar_type() == at::kBFloat16 && index_q.stride(2) == 1,
               "index_q must be bfloat16 with contiguous rows");
    FGV_ASSERT(index_q.size(0) >= num_tokens, "index_q has fewer rows than positions");
    FGV_ASSERT(cos_sin.size(-1) == 64, "rope dim 64");
    FGV_ASSERT(cos_sin.scalar_type() == at::kFloat || cos_sin.scalar_type() == at::kBFloat16,
               "index_q_cos_sin_cache must be float32 or bfloat16");
    FGV_ASSERT(cos_sin.stride(-1) == 1, "index_q_cos_sin_cache rows must be contiguous");
    FGV_ASSERT(weights.scalar_type() == at::kBFloat16 || weights.scalar_type() == at::kFloat,
               "index_weights must be bfloat16 or float32");
    FGV_ASSERT(weights.dim() == 2 && weights.stride(-1) == 1, "index_weights must be 2D with contiguous rows");
    FGV_ASSERT(weights.size(0) >= num_tokens && weights.size(1) == num_heads,
               "index_weights must be [>= num_tokens, num_heads]");
    FGV_ASSERT(head_dim == 128 || head_dim == 256 || head_dim == 512, "head_dim 128, 256 or 512");
    const c10::Device dev = index_q.device();
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");
    FGV_ASSERT(positions_in.device() == dev && cos_sin.device() == dev && weights.device() == dev,
               "all tensors must be on index_q's device");
    const at::Tensor positions = (positions_in.scalar_type() != at::kLong || positions_in.stride(0) != 1)
                                     ? positions_in.to(at::kLong).contiguous()
                                     : positions_in;
    at::Tensor q_out, scale;
    if (use_fp4) {
        q_out = at::empty({num_tokens, num_heads, head_dim / 2}, index_q.options().dtype(at::kByte));
        scale = at::empty({num_tokens, num_heads, head_dim / 32}, index_q.options().dtype(at::kByte));
    } else {
        // as the reference allocates it: index_q's shape and layout
        q_out = at::empty_like(index_q, index_q.options().dtype(at::kFloat8_e4m3fn));
        FGV_ASSERT(q_out.stride(2) == 1, "q codes must have contiguous rows");
    }
    *out = IndexerOut(q_out, scale.defined() ? scale.view(at::kInt).squeeze(-1) : scale, weights_out);
    const c10::DeviceGuard guard(dev);
    return fgv_fused_indexer_q_rope_quant(
        positions.data_ptr<int64_t>(), num_tokens, index_q.data_ptr(), index_q.stride(0), index_q.stride(1),
        num_heads, head_dim, cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.size(0),
        cos_sin.scalar_type() == at::kBFloat16 ? 1 : 0, weights.data_ptr(), weights.stride(0),
        weights.scalar_type() == at::kFloat ? 1 : 0, static_cast<float>(softmax_scale),
        static_cast<float>(head_scale), weights_out.data_ptr<float>(), weights_out.stride(0), use_fp4 ? 1 : 0,
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1), scale.defined() ? scale.data_ptr() : nullptr,
        scale.defined() ? scale.stride(0) : 0, scale.defined() ? scale.stride(1) : 0, current_stream(index_q));
}

// compute_slot_mapping_parallel (reference
// src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:109-144):
// slot_mapping written in place.
int slot_mapping(int64_t num_tokens, int64_t max_num_tokens, const at::Tensor& query_start_loc_in, int64_t num_reqs,
                 const at::Tensor& positions, const at::Tensor& block_table, const at::Tensor& slot_mapping_out,
                 int64_t block_size, int64_t cp_world_size, int64_t cp_rank, int64_t cp_interleave, int64_t pad_id) {
    FGV_ASSERT(slot_mapping_out.scalar_type() == at::kLong && slot_mapping_out.stride(-1) == 1,
               "slot_mapping must be contiguous int64");
    FGV_ASSERT(slot_mapping_out.numel() >= max_num_tokens, "slot_mapping holds fewer than max_num_tokens entries");
    FGV_ASSERT(query_start_loc_in.scalar_type() == at::kInt && query_start_loc_in.numel() >= num_reqs + 1,
               "query_start_loc must be int32 with num_reqs + 1 entries");
    FGV_ASSERT((positions.scalar_type() == at::kInt || positions.scalar_type() == at::kLong) &&
                   positions.stride(-1) == 1,
               "positions must be contiguous int32 or int64");
    FGV_ASSERT(block_table.scalar_type() == at::kInt && block_table.dim() == 2, "block_table must be 2D int32");
    FGV_ASSERT(block_table.stride(-1) == 1, "block_table rows must be contiguous");
    const c10::Device dev = slot_mapping_out.device();
    FGV_ASSERT(dev.is_cuda(), "flaggems_vllm runs on the GPU (HIP) only");
    FGV_ASSERT(query_start_loc_in.device() == dev && positions.device() == dev && block_table.device() == dev,
               "all tensors must be on slot_mapping's device");
    const at::Tensor query_start_loc = query_start_loc_in.contiguous();
    const c10::DeviceGuard guard(dev);
    return fgv_compute_slot_mapping(num_tokens, max_num_tokens, i32_ptr(query_start_loc), num_reqs,
                                    positions.data_ptr(), positions.scalar_type() == at::kLong ? 1 : 0,
                                    i32_ptr(block_table), block_table.stride(0), block_table.size(1),
                                    slot_mapping_out.data_ptr<int64_t>(), block_size, cp_world_size, cp_rank,
                                    cp_interleave, pad_id, current_stream(slot_mapping_out));
}

// ---- dispatcher ops: the same functions, failures raised as RuntimeError ----

void raise_on_status(int rc, const char* op) {
    if (rc == 0)
        return;
    if (rc == kAssertFailed)
        TORCH_CHECK(false, op, ": ", g_assert_message);
    if (rc < 0)
        TORCH_CHECK(false, op, ": ", fgv_last_error(), " (code ", rc, ")");
    TORCH_CHECK(false, op, ": HIP launch failed with hipError_t ", rc);
}

void qnorm_rope_kv_insert_op(at::Tensor& q, const at::Tensor& kv, at::Tensor& k_cache,
                             const at::Tensor& slot_mapping, const at::Tensor& position_ids,
                             const at::Tensor& cos_sin_cache, double eps, int64_t cache_block_size) {
    raise_on_status(qnorm_rope_kv_insert(q, kv, k_cache, slot_mapping, position_ids, cos_sin_cache, eps,
                                         cache_block_size),
                    "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert");
}

SiblingOut inv_rope_fp8_quant_op(const at::Tensor& o, const at::Tensor& positions, const at::Tensor& cos_sin_cache,
                                 int64_t n_groups, int64_t heads_per_group, int64_t nope_dim, int64_t rope_dim,
                                 int64_t quant_group_size, double eps, bool tma_aligned_scales) {
    SiblingOut out;
    raise_on_status(inv_rope_fp8_quant(o, positions, cos_sin_cache, n_groups, heads_per_group, nope_dim, rope_dim,
                                       quant_group_size, eps, true, tma_aligned_scales, &out),
                    "fused_inv_rope_fp8_quant");
    return out;
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(flaggems_vllm, m) {
    // positional order of vLLM's torch.ops._C op of the same name
    m.def("fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(Tensor(a0!) q, Tensor kv, Tensor(a2!) k_cache, "
          "Tensor slot_mapping, Tensor position_ids, Tensor cos_sin_cache, float eps, int cache_block_size) -> ()");
    m.def("fused_inv_rope_fp8_quant(Tensor o, Tensor positions, Tensor cos_sin_cache, int n_groups, "
          "int heads_per_group, int nope_dim=448, int rope_dim=64, int quant_group_size=128, float eps=1e-10, "
          "bool tma_aligned_scales=False) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(flaggems_vllm, CUDA, m) {
    m.impl("fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert", &qnorm_rope_kv_insert_op);
    m.impl("fused_inv_rope_fp8_quant", &inv_rope_fp8_quant_op);
}

PYBIND11_MODULE(_fgv_torch, m) {
    m.doc() = "C++ checks and launches of fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert, "
              "fused_inv_rope_fp8_quant and the four ops beside them (status-returning; the Python drop-ins map "
              "the status)";
    m.attr("ASSERT_FAILED") = kAssertFailed;
    m.def("qnorm_rope_kv_insert", &qnorm_rope_kv_insert);
    m.def("inv_rope_fp8_quant",
          [](const at::Tensor& o, const at::Tensor& positions, const at::Tensor& cos_sin_cache, int64_t n_groups,
             int64_t heads_per_group, int64_t nope_dim, int64_t rope_dim, int64_t quant_group_size, double eps,
             bool fp8_e4m3fn, bool tma_aligned_scales) {
              SiblingOut out;
              const int rc = inv_rope_fp8_quant(o, positions, cos_sin_cache, n_groups, heads_per_group, nope_dim,
                                                rope_dim, quant_group_size, eps, fp8_e4m3fn, tma_aligned_scales,
                                                &out);
              return std::make_tuple(rc, std::get<0>(out), std::get<1>(out));
          });
    m.def("q_kv_rmsnorm",
          [](const at::Tensor& qr, const at::Tensor& kv, const at::Tensor& q_weight, const at::Tensor& kv_weight,
             double eps) {
              TensorPair out;
              const int rc = q_kv_rmsnorm(qr, kv, q_weight, kv_weight, eps, &out);
              return std::make_tuple(rc, std::get<0>(out), std::get<1>(out));
          });
    m.def("dequantize_gather", &dequantize_gather);
    m.def("indexer_q_rope_quant",
          [](const at::Tensor& positions, const at::Tensor& index_q, const at::Tensor& cos_sin,
             const at::Tensor& weights, double softmax_scale, double head_scale, bool use_fp4) {
              IndexerOut out;
              const int rc = indexer_q_rope_quant(positions, index_q, cos_sin, weights, softmax_scale, head_scale,
                                                  use_fp4, &out);
              return std::make_tuple(rc, std::get<0>(out), std::get<1>(out), std::get<2>(out));
          });
    m.def("slot_mapping", &slot_mapping);
    m.def("assert_message", []() { return g_assert_message; });
}
