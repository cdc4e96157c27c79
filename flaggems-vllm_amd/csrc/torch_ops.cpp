// Host-side torch bindings of the path's two ops:
//   fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert  (reference wrapper
//     src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:289-351)
//   fused_inv_rope_fp8_quant                            (reference wrapper
//     src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:157-256)
//
// The argument checks, the output allocation (sibling) and the launch run
// here in C++, so an eager call costs a few microseconds of host time instead
// of the Python asserts plus a 19-argument ctypes call.  Each op is reachable
// two ways, both ending in the same function:
//   - the module functions qnorm_rope_kv_insert / inv_rope_fp8_quant (pybind11),
//     which the Python drop-ins call.  They return a status: 0, kAssertFailed
//     (a reference assertion failed: the Python side raises AssertionError with
//     assert_message()), or the C ABI's code (negative: argument error,
//     positive: hipError_t);
//   - the dispatcher ops torch.ops.flaggems_vllm.<name> (TORCH_LIBRARY_FRAGMENT;
//     schemas mark q and k_cache written), for torch.compile and graph capture.
//     These raise RuntimeError on any failure, as vLLM's own compiled op does.
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
    m.doc() = "C++ checks and launches of fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert and "
              "fused_inv_rope_fp8_quant (status-returning; the Python drop-ins map the status)";
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
    m.def("assert_message", []() { return g_assert_message; });
}
