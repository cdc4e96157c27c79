/*
 * flaggems_vllm_amd — C ABI of the MI355X (gfx950) DeepSeek-V4 attention
 * pre-processing path.
 *
 * Plain pointers, element strides and sizes; no torch types.  Every launcher
 * is asynchronous on the given HIP stream (NULL = the null stream), performs
 * no host synchronisation, no device->host read and no allocation, so it can
 * be recorded into a HIP graph.  Return value: 0 on success, a negative
 * FGV_E_* code for an invalid argument (nothing is launched; fgv_last_error()
 * describes it), or a positive hipError_t from the launch.
 *
 * Element strides are in elements of the tensor's own type (bf16 = 2 bytes,
 * float = 4 bytes, int32 = 4 bytes); k_cache strides are in bytes.
 */
#ifndef FLAGGEMS_VLLM_AMD_H
#define FLAGGEMS_VLLM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGV_OK 0
#define FGV_E_NULL_POINTER (-1)
#define FGV_E_BAD_SHAPE (-2)
#define FGV_E_MISALIGNED (-3)
#define FGV_E_BAD_STRIDE (-4)
#define FGV_E_TOO_LARGE (-5)

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int fgv_version(void);

/* Human-readable description of the last negative return on this thread. */
const char* fgv_last_error(void);

/*
 * Fused DeepSeek-V4 q RMSNorm + RoPE, kv RoPE + UE8M0 FP8 quant + paged insert.
 *
 * Replaces flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
 * (reference: src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:289-351,
 * kernel :20-286) and vLLM's torch.ops._C op of the same name.
 *
 *   q             bf16 [num_tokens, num_heads, 512], element (t,h,i) at
 *                 q + t*q_stride_token + h*q_stride_head + i.  Updated in place:
 *                 i < 448 -> bf16(x_i * r); i >= 448 -> GPT-J RoPE of x*r,
 *                 r = 1/sqrt(mean(x^2) + eps) over all 512 dims.
 *   kv            bf16 [num_tokens, 512] (row stride kv_stride_token); read only.
 *   k_cache       uint8 paged cache, block b at k_cache + b*cache_block_stride
 *                 bytes; per block: cache_block_size x 576 B token data
 *                 (448 e4m3fn codes, 64 bf16 roped values), then
 *                 cache_block_size x 8 B scales (7 UE8M0 bytes, 1 zero byte).
 *   slot_mapping  int64 [num_tokens_insert]; token t < num_tokens_insert with
 *                 slot s >= 0 is written to block s / cache_block_size, row
 *                 s % cache_block_size.  Slots < 0 (padding) are skipped, as
 *                 are slots whose block is >= num_blocks.
 *   position_ids  int64 [num_tokens]; clamped into [0, max_pos).
 *   cos_sin_cache float [max_pos, 64] (row stride cos_sin_stride): cos in
 *                 columns 0..31, sin in 32..63.
 *
 * Alignment: q, kv 16-byte aligned with strides multiple of 8 elements;
 * k_cache 8-byte aligned with cache_block_stride multiple of 8;
 * cos_sin_cache 16-byte aligned with cos_sin_stride multiple of 4.
 */
int fgv_qnorm_rope_kv_rope_quant_insert(
    void* q, int64_t q_stride_token, int64_t q_stride_head,
    const void* kv, int64_t kv_stride_token,
    void* k_cache, int64_t cache_block_stride, int64_t num_blocks,
    const int64_t* slot_mapping, int64_t num_tokens_insert,
    const int64_t* position_ids,
    const float* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos,
    int64_t num_tokens, int64_t num_heads,
    float eps, int64_t cache_block_size,
    void* stream);

/*
 * Fused DeepSeek-V4 inverse GPT-J RoPE + per-group FP8 e4m3fn quant.
 *
 * Replaces flaggems_vllm.fused_inv_rope_fp8_quant
 * (reference: src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:157-256,
 * kernel :37-154), with its geometry arguments: head_dim D = nope_dim +
 * rope_dim, quant_group_size Q dividing D, nope_dim % Q == Q - rope_dim (the
 * rope dims inside the last chunk), rope_dim even (the reference's
 * assertions, :192-205).  This build takes D a power of two in [8, 512] and
 * Q a power of two >= 8; DeepSeek-V4's (448, 64, 128) runs a kernel of its
 * own, every other geometry a general one.  Packed scales need at most four
 * chunks per head, and four unless heads_per_group is 1: the reference's
 * packed scale tensor has a word per head only then.
 *
 *   o          bf16 [num_tokens, n_groups*heads_per_group, D], element
 *              (t,h,i) at o + t*o_stride_token + h*o_stride_head + i.
 *   positions  int64 [num_tokens], clamped into [0, max_pos).
 *   fp8_out    uint8 e4m3fn codes, element (g,t,i), i < heads_per_group*D,
 *              at fp8_out + g*fp8_stride_group + t*fp8_stride_token + i.
 *   scale_out  tma_aligned_scales == 0: float scale of chunk k
 *              (k < (D/Q)*heads_per_group) at scale_out + g*scale_stride_group
 *              + k*scale_stride_k + t;  != 0: int32 with the UE8M0 bytes of
 *              head j's chunks (byte c for chunk c) at scale_out +
 *              g*scale_stride_group + j*scale_stride_k + t.  Tokens
 *              num_tokens..padded_tokens-1 get zero scales.
 */
int fgv_inv_rope_fp8_quant(
    const void* o, int64_t o_stride_token, int64_t o_stride_head,
    const int64_t* positions,
    const float* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos,
    int64_t num_tokens, int64_t n_groups, int64_t heads_per_group,
    int64_t nope_dim, int64_t rope_dim, int64_t quant_group_size,
    void* fp8_out, int64_t fp8_stride_group, int64_t fp8_stride_token,
    void* scale_out, int64_t scale_stride_group, int64_t scale_stride_k,
    int64_t padded_tokens, float eps, int tma_aligned_scales,
    void* stream);

/*
 * Dequantise and gather cached K rows into bf16.
 *
 * Replaces flaggems_vllm.dequantize_and_gather_k_cache
 * (reference: src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:123-172,
 * kernel :38-120), the consumer of the cache that
 * fgv_qnorm_rope_kv_rope_quant_insert writes.
 *
 *   out          bf16 [>= num_reqs, out_rows, >= nope_dim + rope_dim]; element
 *                (r, j, c) at out + r*out_stride_req + j*out_stride_row + c.
 *   k_cache      uint8 paged cache: block b at k_cache + b*cache_block_stride;
 *                per block block_size x (nope_dim + 2*rope_dim) token bytes, then
 *                block_size x scale_slots UE8M0 bytes.
 *   seq_lens     int32 [num_reqs]; gather_lens int32 [num_reqs] or NULL (= seq_lens).
 *   block_table  int32 [num_reqs, max_blocks_per_seq], row stride block_table_stride.
 *
 * For request r and i < gather_lens[r] (and offset + i < out_rows), position
 * p = seq_lens[r] - gather_lens[r] + i is read from block
 * block_table[r, p / block_size] and written to out row offset + i:
 * columns < nope_dim get e4m3(code) * 2^(scale_byte - 127) of their 64-element
 * group, the next rope_dim columns the cached bf16 values.  Rows whose block
 * index or physical block is out of range are left untouched.
 * nope_dim and rope_dim must be multiples of 8.
 */
int fgv_dequantize_and_gather_k_cache(
    void* out, int64_t out_stride_req, int64_t out_stride_row, int64_t out_rows,
    const void* k_cache, int64_t cache_block_stride, int64_t num_blocks,
    const int32_t* seq_lens, const int32_t* gather_lens,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_seq,
    int64_t num_reqs, int64_t block_size, int64_t offset,
    int64_t nope_dim, int64_t rope_dim, int64_t scale_slots,
    void* stream);

/*
 * Fused weighted RMSNorm of DeepSeek-V4's q LoRA rows and kv latent rows.
 *
 * Replaces flaggems_vllm.fused_q_kv_rmsnorm
 * (reference: src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:65-103,
 * kernel :24-62).  For every token t:
 *   qr_out[t] = (qr[t] * rsqrt(mean(qr[t]^2) + eps)) * q_weight
 *   kv_out[t] = (kv[t] * rsqrt(mean(kv[t]^2) + eps)) * kv_weight
 * Rows are bf16 with row strides in elements; weights are bf16, or float when
 * weight_is_fp32.  Sizes must be multiples of 8, at most 2^24.
 */
int fgv_fused_q_kv_rmsnorm(
    const void* qr, int64_t qr_stride, void* qr_out, int64_t qr_out_stride,
    const void* q_weight, int64_t q_size,
    const void* kv, int64_t kv_stride, void* kv_out, int64_t kv_out_stride,
    const void* kv_weight, int64_t kv_size,
    int64_t num_tokens, float eps, int weight_is_fp32, void* stream);

/*
 * Fused sparse-indexer q RoPE + quant with head-weight folding.
 *
 * Replaces flaggems_vllm.fused_indexer_q_rope_quant
 * (reference: src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py:285-410,
 * kernels :64-167 (FP8) and :170-282 (MXFP4)).
 *
 *   index_q      bf16 [num_tokens, num_heads, head_dim], head_dim 128/256/512;
 *                GPT-J RoPE on the last 64 dims, result rounded to bf16.
 *   cos_sin      [max_pos, 64] float (or bf16 if cos_sin_is_bf16), cos | sin.
 *   weights      [num_tokens, num_heads] bf16 (or float), row stride given.
 *   use_fp4 == 0: q_out = e4m3fn codes of x * 2^-k per (t, h), with
 *                k = ceil(log2(max(amax, 1e-4) / 448));
 *                weights_out = ((w * 2^k) * softmax_scale) * head_scale.
 *   use_fp4 != 0: q_out = packed E2M1 nibbles [.., head_dim/2] (even element
 *                in the low nibble), scale_out = UE8M0 byte per 32 elements
 *                (4-byte aligned, strides multiples of 4),
 *                k = ceil(log2(max(amax, 6*2^-126) / 6));
 *                weights_out = (w * softmax_scale) * head_scale.
 */
int fgv_fused_indexer_q_rope_quant(
    const int64_t* positions, int64_t num_tokens,
    const void* index_q, int64_t q_stride_token, int64_t q_stride_head,
    int64_t num_heads, int64_t head_dim,
    const void* cos_sin_cache, int64_t cos_sin_stride, int64_t max_pos, int cos_sin_is_bf16,
    const void* weights, int64_t weights_stride, int weights_is_fp32,
    float softmax_scale, float head_scale,
    float* weights_out, int64_t weights_out_stride,
    int use_fp4,
    void* q_out, int64_t q_out_stride_token, int64_t q_out_stride_head,
    void* scale_out, int64_t scale_out_stride_token, int64_t scale_out_stride_head,
    void* stream);

/*
 * Paged-KV slot mapping, parallel over tokens.
 *
 * Replaces flaggems_vllm.compute_slot_mapping_parallel
 * (reference: src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:109-144,
 * kernel :42-106).  For token t of request r (query_start_loc[r] <= t <
 * query_start_loc[r + 1], t < num_tokens):
 *   pos = positions[t] (int32, or int64 if positions_are_int64)
 *   v = block_size * cp_world_size; blk = block_table[r, pos / v]; o = pos % v
 *   slot_mapping[t] = blk * block_size + (o / (cp_world_size * il)) * il + o % il
 *     if (o / il) % cp_world_size == cp_rank, else pad_id   (il = interleave size)
 * and slot_mapping[t] = pad_id for num_tokens <= t < max_num_tokens.  Tokens
 * outside every request are not written; positions outside the block table
 * give pad_id.
 */
int fgv_compute_slot_mapping(
    int64_t num_tokens, int64_t max_num_tokens,
    const int32_t* query_start_loc, int64_t num_reqs,
    const void* positions, int positions_are_int64,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_req,
    int64_t* slot_mapping, int64_t block_size,
    int64_t cp_world_size, int64_t cp_rank, int64_t cp_kv_cache_interleave_size,
    int64_t pad_id, void* stream);

/*
 * Sparse-indexer key quantise + paged insert.
 *
 * Replaces flaggems_vllm.ops.indexer_k_quant_and_cache
 * (reference: src/flaggems_vllm/ops/indexer_k_quant_and_cache.py:100-132,
 * kernel :44-96; torch oracle tests/test_indexer_k_quant_and_cache.py:99-142).
 *
 *   k         bf16 (or fp16 if k_is_fp16) [num_tokens, head_dim], row stride
 *             k_stride_token elements (multiple of 8), 16-byte aligned
 *   kv_cache  uint8 blocks cache_block_stride bytes apart (pointer and stride
 *             4-byte aligned; 16-byte alignment, i.e. block_size a multiple
 *             of 4 in a packed cache, gives 16-byte code stores); block b
 *             holds block_size x head_dim e4m3fn codes, then block_size x
 *             (head_dim / 128) float32 scales
 *   slot_mapping  int64 [num_tokens]; < 0 skips the token
 *
 * For token t with slot s >= 0 (block s / block_size < num_blocks) and quant
 * block j of 128 elements:
 *   scale = max(amax_j, 1e-4) / 448 (IEEE binary32 division);
 *           use_ue8m0: 2^ceil(log2(scale))
 *   codes = e4m3fn(k / scale), scale stored as float32
 * at row s % block_size of block s / block_size.  quant_block_size must be
 * 128; head_dim a multiple of 128, at most 2048.
 */
int fgv_indexer_k_quant_and_cache(
    const void* k, int64_t k_stride_token, int k_is_fp16,
    int64_t num_tokens, int64_t head_dim, int64_t quant_block_size,
    void* kv_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t block_size,
    const int64_t* slot_mapping, int use_ue8m0, void* stream);

/*
 * Gather of a batch's cached sparse-indexer keys.
 *
 * Replaces flaggems_vllm.ops.cp_gather_indexer_k_quant_cache
 * (reference: src/flaggems_vllm/ops/cp_gather_indexer_k_quant_cache.py:114-176,
 * kernel :23-111; torch oracle tests/test_cp_gather_indexer_k_quant_cache.py:83-114).
 * Cache layout as fgv_indexer_k_quant_and_cache writes it.  Token
 * t < num_tokens of request b (cu_seqlen[b] <= t < cu_seqlen[b + 1]) at
 * position p = t - cu_seqlen[b] copies the head_dim code bytes and
 * head_dim / 128 float32 scales of row p % block_size of block
 * block_table[b, p / block_size] to k_out + t * k_out_stride and
 * scale_out + t * scale_out_stride (byte strides; kv_cache, k_out, scale_out
 * and their strides 4-byte aligned).
 * Tokens outside every request, and tokens whose block-table index or block
 * is out of range, are left untouched.  cu_seqlen has batch_size + 1 entries,
 * non-decreasing.
 */
int fgv_cp_gather_indexer_k_quant_cache(
    const void* kv_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t block_size,
    int64_t head_dim, int64_t quant_block_size,
    void* k_out, int64_t k_out_stride, void* scale_out, int64_t scale_out_stride,
    const int32_t* block_table, int64_t block_table_stride, int64_t max_blocks_per_seq,
    const int32_t* cu_seqlen, int64_t batch_size, int64_t num_tokens, void* stream);

/*
 * Sparse-indexer logits over dense keys.
 *
 * Replaces flaggems_vllm.ops.fp8_fp4_mqa_logits
 * (reference: src/flaggems_vllm/ops/fp8_fp4_mqa_logits.py:523-651, kernels
 * :88-187 (FP8), :232-358 (MXFP4), :190-222 (clean); float32 oracle
 * tests/test_fp8_fp4_mqa_logits.py:40-66).  For m < M, n < N:
 *   logits[m, n] = sum_h ReLU((sum_d q[m,h,d] k[n,d]) * k_scale[n]) * w[m,h]
 * and, with clean_logits, -inf where n < ks[m] or n >= ke[m].
 *   q        q_scale == NULL: e4m3fn [M, H, 128]; else packed E2M1 [M, H, 64]
 *            (even d in the low nibble) with q_scale int32 [M, H] holding the
 *            UE8M0 byte of d = 32b..32b+31 in byte b.  Byte strides, multiples
 *            of 16, 16-byte aligned rows.
 *   k        e4m3fn [N, 128] (byte row stride, multiple of 16); k_scale float [N]
 *            (positive, as the producers write it).
 *   weights  float [M, H]; ks, ke int32 [M] (read only with clean_logits).
 *   logits   float [M, N], row stride in elements.
 * num_heads 16, 32, 64 or 128; head_dim 128.  The head sum is taken in
 * binary32 in an order of this library's choosing, with k_scale applied once
 * after it.  Precondition: k_scale[n] >= 0 (the producers write amax / 448 >
 * 0).  For k_scale > 0 this equals the reference's per-head product; for
 * k_scale = 0 both give 0.  A negative k_scale[n] is not rejected (that would
 * need a device read) and gives k_scale[n] * sum_h ReLU(dot_h) * w[m,h], not
 * the reference's sum_h ReLU(dot_h * k_scale[n]) * w[m,h].  The paged
 * variant below has the same precondition on the cache's scales.
 */
int fgv_fp8_fp4_mqa_logits(
    const void* q, int64_t q_stride_m, int64_t q_stride_h, const int32_t* q_scale, int64_t q_scale_stride_m,
    int64_t q_scale_stride_h, const void* k, int64_t k_stride_n, const float* k_scale, const float* weights,
    int64_t w_stride_m, int64_t w_stride_h, const int32_t* cu_seqlen_ks, const int32_t* cu_seqlen_ke,
    float* logits, int64_t logits_stride_m, int64_t M, int64_t N, int64_t num_heads, int64_t head_dim,
    int clean_logits, void* stream);

/*
 * Sparse-indexer logits over the paged key cache (decode).
 *
 * Replaces flaggems_vllm.ops.fp8_fp4_paged_mqa_logits
 * (reference: src/flaggems_vllm/ops/fp8_fp4_paged_mqa_logits.py:410-579,
 * kernel :68-181, cache layout :185-225).  For each of `rows` query rows
 * (q, q_scale and weights as in fgv_fp8_fp4_mqa_logits, per row):
 *   ctx = context_lens[row / rows_per_context_len], clamped to [0, max_model_len];
 *   position n < ctx reads entry n % block_size of cache block
 *   clamp(block_tables[(row / rows_per_table_row) * block_table_stride +
 *   min(n / block_size, max_blocks_per_seq - 1)], 0, num_blocks - 1)
 *   (block_size x 128 e4m3fn bytes, then block_size float32 scales: the
 *   cache fgv_indexer_k_quant_and_cache writes at head_dim 128) and gets the
 *   logit above; every position ctx <= n < max_model_len gets 0, or -inf
 *   with clean_logits.  Every element of the [rows, max_model_len] output is
 *   written.  At most 65535 rows.
 */
int fgv_fp8_fp4_paged_mqa_logits(
    const void* q, int64_t q_stride_row, int64_t q_stride_h, const int32_t* q_scale, int64_t q_scale_stride_row,
    int64_t q_scale_stride_h, const void* kv_cache, int64_t cache_block_stride, int64_t num_blocks,
    int64_t block_size, int64_t head_dim, const float* weights, int64_t w_stride_row, int64_t w_stride_h,
    const int32_t* context_lens, int64_t rows_per_context_len, const int32_t* block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq, int64_t rows_per_table_row, float* logits,
    int64_t logits_stride_row, int64_t rows, int64_t num_heads, int64_t max_model_len, int clean_logits,
    void* stream);

/*
 * Sparse MLA decode over the 584-byte MODEL1 cache.
 *
 * Replaces the sparse MODEL1 branch of flaggems_vllm.flash_mla_with_kvcache
 * (reference: src/flaggems_vllm/ops/flash_mla_with_kvcache.py:852-1073 wrapper,
 * :1096-1171 dispatch, kernel :489-688; sm90 kernel
 * src/flaggems_vllm/ops/flash_mla_with_kvcache_model1.py:1464-1695).
 *
 *   q    bf16 [batch, seq_q, num_heads, 512] (strides in elements, last dim contiguous)
 *   k_cache / extra_k_cache  uint8 [num_blocks, page_size, 1, 584]: per page,
 *        page_size x 576 token bytes (448 e4m3 + 64 bf16) then page_size x 8
 *        E8M0 scale bytes; block strides in bytes
 *   indices / extra_indices  int32 [batch, seq_q, topk] (last dim contiguous)
 *   topk_length / extra_topk_length  int32 [batch] or NULL (then topk); clamped
 *        to [0, topk]
 *   attn_sink  float [num_heads] or NULL
 *   out  bf16 [batch, seq_q, num_heads, 512];  lse  float [batch, num_heads, seq_q]
 *        (stride over seq_q is 1)
 *
 * Entry t of a list is attended when t < its length, id >= 0 and
 * id / page_size < num_blocks.  K = V = bf16(e4m3 * 2^(scale_byte - 127)) for
 * dims 0..447 (one scale per 64) and the cached bf16 RoPE for 448..511.  Per
 * head: s = softmax_scale * q.K, lse = m + log(sum exp(s - m)) (+inf if nothing
 * is attended), out = sum exp(s - m) V / (sum exp(s - m) + exp(sink - m)) (no
 * sink term without attn_sink; 0 if nothing is attended).  num_heads must be a
 * multiple of 64.
 */
int fgv_sparse_mla_decode_model1(
    const void* q, int64_t q_stride_b, int64_t q_stride_s, int64_t q_stride_h,
    const void* k_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t page_size,
    const int32_t* indices, int64_t idx_stride_b, int64_t idx_stride_s, int64_t topk,
    const int32_t* topk_length,
    const void* extra_k_cache, int64_t extra_block_stride, int64_t extra_num_blocks,
    int64_t extra_page_size,
    const int32_t* extra_indices, int64_t extra_idx_stride_b, int64_t extra_idx_stride_s,
    int64_t extra_topk,
    const int32_t* extra_topk_length,
    const float* attn_sink, float softmax_scale,
    void* out, int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h,
    float* lse, int64_t lse_stride_b, int64_t lse_stride_h,
    int64_t batch, int64_t seq_q, int64_t num_heads,
    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace (256-byte aligned) that fgv_sparse_mla_decode_model1
 * can use, the sum of two optional parts:
 *   - an expanded extra cache: when the extra list is gathered at least 8 times
 *     per cache entry (batch * seq_q * num_heads/64 * extra_topk >=
 *     8 * extra_num_entries) and the copy is at most 64 MiB, the extra cache is
 *     dequantised once per call into bf16 rows (1 KiB per entry) that the
 *     attention reads without converting.  The results are the same bits.
 *   - the split schedule: for long lists (topk + extra_topk at least 2048
 *     entries, batch at most 8000 rows) over at most one (row, head block)
 *     item per CU, or over more than two per CU, a grid of two workgroups per
 *     CU splits all items' chunks evenly, and a combine kernel merges the
 *     items that cross a split (the reference's split-KV schedule and
 *     combine, ops/flash_mla_with_kvcache_model1.py:1212-1395).  Its size
 *     depends on the current device's CU count.
 * extra_num_entries is extra_num_blocks * extra_page_size (0 without an extra
 * cache).  0 means the workspace argument is ignored.  Passing no workspace
 * (NULL or too small) always works: a workspace too small for both parts drops
 * the expansion first, then the split (one workgroup per item).
 */
int64_t fgv_sparse_mla_decode_workspace_bytes(int64_t batch, int64_t seq_q, int64_t num_heads,
                                              int64_t topk, int64_t extra_topk, int64_t extra_num_entries);

/*
 * Which grid fgv_sparse_mla_decode_model1 runs for these sizes on the current
 * device, given the workspace fgv_sparse_mla_decode_workspace_bytes asks for:
 *   0  one workgroup per (row, query position, 64-head block) item
 *      (sparse_mla_decode_kernel);
 *   1  the split grid and its combine (sparse_mla_decode_split_kernel,
 *      sparse_mla_combine_kernel);
 *   2  the paired grid (sparse_mla_decode_pair_kernel): lists as long as the
 *      split grid's over more items than CUs but at most two per CU (and at
 *      most 512); one 8-wave workgroup per CU attends each of its items with
 *      both halves, a short item after a long one, and writes no partials.
 * -1 for sizes the decode rejects.  No counterpart in the reference: it is
 * for benchmarks, profilers and tests that need the kernel's name.
 */
int fgv_sparse_mla_decode_grid(int64_t batch, int64_t seq_q, int64_t num_heads, int64_t topk,
                               int64_t extra_topk);

/*
 * Size of the fixed device scratch of fgv_sparse_mla_decode_model1_no_alloc.
 * Two costs every caller of this library carries:
 *   - Memory: the array is part of the library's GPU code object, so every
 *     process that runs any op of this library on a device holds these
 *     64 MiB of that device's memory until it exits, whether or not it ever
 *     calls the no-allocation entry point.
 *   - Concurrency: all no-allocation calls on one device share the array.
 *     Calls that overlap in time (two streams, two host threads) race on it
 *     and give wrong results; nothing in the library detects or prevents
 *     this, so the caller must order them (one stream, or events).
 */
#define FGV_MLA_NO_ALLOC_SCRATCH_BYTES (64LL << 20)

/*
 * Sparse MLA decode exactly as fgv_sparse_mla_decode_model1 with the workspace
 * fgv_sparse_mla_decode_workspace_bytes asks for (same arguments, same
 * schedule, same output bits), but with no workspace argument and no
 * allocation of any kind: the workspace is a fixed device array of
 * FGV_MLA_NO_ALLOC_SCRATCH_BYTES (64 MiB) inside the library, one per device,
 * held from the library's first use on that device until the process ends.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.
 *
 * Limit: a call whose workspace query exceeds 64 MiB returns FGV_E_TOO_LARGE
 * and launches nothing (with today's schedule: expanded extra caches above
 * 64 MiB, and every call long enough for the split grid, whose partial slots
 * take ~135 MB); call fgv_sparse_mla_decode_model1 with a workspace for those.
 * Calls on one device share its scratch: calls that overlap in time on one
 * device (concurrent streams, other host threads) race and must be serialised
 * by the caller.  The scratch of the device current at the call is used; the
 * stream must belong to that device.
 */
int fgv_sparse_mla_decode_model1_no_alloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_s, int64_t q_stride_h,
    const void* k_cache, int64_t cache_block_stride, int64_t num_blocks, int64_t page_size,
    const int32_t* indices, int64_t idx_stride_b, int64_t idx_stride_s, int64_t topk,
    const int32_t* topk_length,
    const void* extra_k_cache, int64_t extra_block_stride, int64_t extra_num_blocks,
    int64_t extra_page_size,
    const int32_t* extra_indices, int64_t extra_idx_stride_b, int64_t extra_idx_stride_s,
    int64_t extra_topk,
    const int32_t* extra_topk_length,
    const float* attn_sink, float softmax_scale,
    void* out, int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h,
    float* lse, int64_t lse_stride_b, int64_t lse_stride_h,
    int64_t batch, int64_t seq_q, int64_t num_heads,
    void* stream);

/*
 * Sparse MLA prefill over bf16 key/value rows.
 *
 * Replaces flaggems_vllm.flash_mla_sparse_fwd (reference:
 * src/flaggems_vllm/ops/flashmla_sparse.py:1045-1206 wrapper and asserts,
 * kernel :50-195; definitions of the outputs in tests/test_flash_mla_sparse_fwd.py:93-150).
 *
 *   q    bf16 [s_q, h_q, d_qk] (strides in elements, last dim contiguous)
 *   kv   bf16 [s_kv, d_qk] rows kv_stride_row elements apart (h_kv = 1)
 *   indices  int32 [s_q, topk] (token stride idx_stride_t, last dim contiguous)
 *   topk_length  int32 [s_q] or NULL (then topk); clamped to [0, topk]
 *   attn_sink  float [h_q] or NULL
 *   out  bf16 [s_q, h_q, 512];  max_logits, lse  float [s_q, h_q] (head stride 1)
 *
 * Entry i of token t is attended when i < its length and 0 <= id < s_kv.
 * Per (t, head): s = sm_scale * q . kv[id] over the d_qk dims (512 or 576),
 * max_logits = max s (-inf if nothing is attended), lse = log sum exp s (+inf
 * if nothing is attended), out = sum exp(s - m) V / (sum exp(s - m) +
 * exp(sink - m)) with V = kv[id][0:512] (no sink term without attn_sink; 0
 * if nothing is attended).  The sink does not enter max_logits or lse.
 * h_q must be a multiple of 64 (the reference allows 64 and 128).
 */
int fgv_flash_mla_sparse_fwd(
    const void* q, int64_t q_stride_t, int64_t q_stride_h,
    const void* kv, int64_t kv_stride_row, int64_t s_kv,
    const int32_t* indices, int64_t idx_stride_t, int64_t topk,
    const int32_t* topk_length, const float* attn_sink, float sm_scale,
    int64_t s_q, int64_t h_q, int64_t d_qk,
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    float* max_logits, int64_t max_logits_stride_t,
    float* lse, int64_t lse_stride_t, void* stream);

/*
 * Request-local top-k indices -> global cache slots, and the row lengths.
 *
 * Replaces flaggems_vllm.compute_global_topk_indices_and_lens
 * (reference: src/flaggems_vllm/ops/deepseek_v4_attention_compute_global_topk_indices_and_lens.py:122-160,
 * kernel :46-119).  For token t with request r = token_to_req_indices[t] and
 * each column i < topk with l = topk_indices[t, i]:
 *   global_indices[t, i] = block_table[r, l / block_size] * block_size + l % block_size   (l >= 0)
 *                        = -1                                                           (l < 0)
 *   lens[t] = #{i : l >= 0} if is_valid_token[t] != 0 (or is_valid_token is NULL), else 0.
 * int32 arithmetic with wrap-around, as the reference computes it.  A block
 * outside the block table ([num_reqs, blocks_per_req] with row stride
 * block_table_stride, all in elements) gives -1 and still counts; the
 * reference reads past the row there.  Strides are in elements.
 */
int fgv_compute_global_topk_indices_and_lens(
    const int32_t* topk_indices, int64_t topk_stride0, int64_t topk_stride1, int64_t num_tokens, int64_t topk,
    const int32_t* token_to_req_indices, const int32_t* block_table, int64_t block_table_stride,
    int64_t num_reqs, int64_t blocks_per_req, int64_t block_size, const int32_t* is_valid_token,
    int32_t* global_indices, int64_t out_stride0, int64_t out_stride1, int32_t* lens, void* stream);

/*
 * Row width of combine_topk_swa_indices' output: topk + window_size rounded
 * up to a multiple of 128 (the reference's _SPARSE_PREFILL_TOPK_ALIGNMENT),
 * or -1 for negative arguments.
 */
int64_t fgv_combine_topk_swa_width(int64_t topk, int64_t window_size);

/*
 * Top-k indices and sliding-window rows combined into one index row per token.
 *
 * Replaces flaggems_vllm.combine_topk_swa_indices
 * (reference: src/flaggems_vllm/ops/deepseek_v4_attention_combine_topk_swa_indices.py:105-150,
 * kernel :30-102).  For request b (query_start_loc[b] - query_start_loc[0] <=
 * t < query_start_loc[b + 1] - query_start_loc[0]) with q = its query length,
 * pos = seq_lens[b] - q + (t - start), gather_start = seq_lens[b] - gather_lens[b]:
 *   topk_len = min((pos + 1) / compress_ratio, topk), swa_len = min(pos + 1, window_size)
 *   combined[t, j] = topk_indices[t, j] + M * b                               j < topk_len
 *   combined[t, topk_len + j] = M * b + N + j + pos - swa_len + 1 - gather_start   j < swa_len
 *   combined[t, j] = -1 for the rest of the fgv_combine_topk_swa_width columns
 *   lens[t] = topk_len + swa_len
 * int32 arithmetic with wrap-around and truncating division, as the
 * reference computes it.  Rows of tokens outside every request are not
 * written.  topk must not exceed topk_cols (the reference would read past
 * the row).  Strides are in elements.
 */
int fgv_combine_topk_swa_indices(
    const int32_t* topk_indices, int64_t topk_stride0, int64_t topk_stride1, int64_t num_tokens,
    int64_t topk_cols, const int32_t* query_start_loc, const int32_t* seq_lens, const int32_t* gather_lens,
    int64_t num_reqs, int64_t window_size, int64_t compress_ratio, int64_t topk, int64_t M, int64_t N,
    int32_t* combined, int64_t out_stride0, int64_t out_stride1, int32_t* lens, void* stream);

/*
 * Top-k per row of float32 logits (the sparse indexer's selection).
 *
 * Replace flaggems_vllm.top_k_per_row_decode and top_k_per_row_prefill
 * (reference: src/flaggems_vllm/ops/top_k_per_row_decode.py:1263-1399, job
 * :877-1043; src/flaggems_vllm/ops/top_k_per_row_prefill.py:1232-1331).  Row r
 * of logits [num_rows, width] (strides in elements) holds candidates
 *   decode:  [0, seq_lens[r / next_n] - next_n + r % next_n + 1)
 *   prefill: [row_starts[r], row_ends[r])
 * (clamped to [0, width)).  indices[r, :] receives the column indices,
 * relative to the row's start, of its top_k largest values in no particular
 * order; a row of at most top_k values gives 0, 1, ..., len - 1 then -1.
 * Values equal to the k-th largest are taken lowest index first, so the set
 * is a function of the values; NaN orders above +inf (as torch.topk).
 * workspace (16-byte aligned, fgv_top_k_per_row_workspace_bytes of it) lets
 * few rows of 12 or more 16384-value parts (192K+ values; at most two parts
 * per CU in all) be split into parts and merged; without it (NULL or too
 * small), or otherwise, each row is streamed by one workgroup.  The index
 * sets are the same either way.  The reference allocates its split's
 * buffers per call likewise (ops/top_k_per_row_decode.py:1303-1312).
 */
int fgv_top_k_per_row_decode(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                             int64_t width, int64_t next_n, const int32_t* seq_lens, int32_t* indices,
                             int64_t out_stride0, int64_t out_stride1, int64_t top_k, void* workspace,
                             int64_t workspace_bytes, void* stream);
int fgv_top_k_per_row_prefill(const float* logits, int64_t stride0, int64_t stride1, int64_t num_rows,
                              int64_t width, const int32_t* row_starts, const int32_t* row_ends, int32_t* indices,
                              int64_t out_stride0, int64_t out_stride1, int64_t top_k, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* Workspace bytes the top-k entry points can use for these sizes on the
 * current device (0: they use none). */
int64_t fgv_top_k_per_row_workspace_bytes(int64_t num_rows, int64_t width, int64_t top_k);

/*
 * Block-scaled FP8 einsum 'bhr,hdr->bhd' (the grouped output projection that
 * consumes fgv_inv_rope_fp8_quant's codes and per-128 scales).
 *
 * Replaces flaggems_vllm.fp8_einsum (reference: src/flaggems_vllm/ops/fp8_einsum.py:20-115,
 * which hands the work to a Hopper block-FP8 batched GEMM):
 *   out[b,h,d] = sum_r (x[b,h,r] xs[b,h,r/128]) (y[h,d,r] ys[h,d/128,r/128])
 * x [b,h,r] and y [h,d,r] are e4m3fn codes with r contiguous; xs [b,h,r/128]
 * and ys [h,d/128,r/128] float32; every stride is in elements of its tensor.
 * r and d are multiples of 128.  out [b,h,d] is bf16 (out_dtype 0), fp16
 * (1) or fp32 (2), rounded to nearest even; r = 0 writes zeros, b, h or
 * d = 0 writes nothing.  Each 128-wide K block's partial sum is formed in
 * binary32 and accumulated times xs * ys in binary32, in a fixed order, so
 * the result depends only on the inputs.  Rows of x and y need no
 * alignment (16-byte aligned ones take the fast paths).
 */
int fgv_fp8_einsum_bhr_hdr(const uint8_t* x, int64_t x_stride_b, int64_t x_stride_h, const float* xs,
                           int64_t xs_stride_b, int64_t xs_stride_h, int64_t xs_stride_k, const uint8_t* y,
                           int64_t y_stride_h, int64_t y_stride_d, const float* ys, int64_t ys_stride_h,
                           int64_t ys_stride_n, int64_t ys_stride_k, int64_t b, int64_t h, int64_t r, int64_t d,
                           void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_d,
                           int32_t out_dtype, void* stream);

/*
 * Bytes of device workspace fgv_fp8_einsum_bhr_hdr_ws can use for these
 * sizes on the current device, or 0 when it would not use any.  With b > 64
 * and at most CUs / 2 128-row output tiles, the K blocks are split over up to
 * 2 x CUs / tiles workgroups per tile (at least 8 blocks each); each writes
 * its fp32 partial tile, and a second kernel sums the partials in a fixed
 * order (splits * b * h * d * 4 bytes, rounded up to 256).  Same call as
 * fgv_fp8_einsum_bhr_hdr (reference: src/flaggems_vllm/ops/fp8_einsum.py:20-115).
 */
int64_t fgv_fp8_einsum_workspace_bytes(int64_t b, int64_t h, int64_t r, int64_t d);

/*
 * fgv_fp8_einsum_bhr_hdr with a caller workspace (16-byte aligned) for the
 * split-K schedule above.  A NULL or too small workspace runs the unsplit
 * schedule of fgv_fp8_einsum_bhr_hdr.  The results depend only on the inputs
 * and on whether the workspace was used: the split sums each K range's
 * scaled blocks in fp32, then the ranges in order, a different fp32
 * summation order from the unsplit kernel's.  Calls that share a workspace
 * must be ordered on one stream.
 */
int fgv_fp8_einsum_bhr_hdr_ws(const uint8_t* x, int64_t x_stride_b, int64_t x_stride_h, const float* xs,
                              int64_t xs_stride_b, int64_t xs_stride_h, int64_t xs_stride_k, const uint8_t* y,
                              int64_t y_stride_h, int64_t y_stride_d, const float* ys, int64_t ys_stride_h,
                              int64_t ys_stride_n, int64_t ys_stride_k, int64_t b, int64_t h, int64_t r, int64_t d,
                              void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_d,
                              int32_t out_dtype, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLAGGEMS_VLLM_AMD_H */
