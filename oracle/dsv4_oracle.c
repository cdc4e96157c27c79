/*
 * CPU oracle for the DeepSeek-V4 attention pre-processing path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library or the
 * flaggems_vllm Python package) links, loads or calls this file.  It is loaded
 * by tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of
 * bench.py, always as the checker and never as the thing measured or shipped.
 *
 * It restates, in plain scalar C, what the reference computes:
 *
 *   oracle_qnorm_rope_kv_insert
 *     reference op   src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:20-351
 *     reference test tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:93-243, 316-333
 *   oracle_inv_rope_fp8_quant
 *     reference op   src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:37-256
 *     reference test tests/test_fused_inv_rope_fp8_quant.py:150-198
 *   oracle_fused_q_kv_rmsnorm
 *     reference op   src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:24-103
 *     reference test tests/test_deepseek_v4_attention_fused_q_kv_rmsnorm.py:40-76
 *   oracle_fused_indexer_q_rope_quant
 *     reference op   src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py:64-410
 *     reference test tests/test_fused_indexer_q_rope_quant.py:51-110
 *   oracle_compute_slot_mapping
 *     reference op   src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:42-144
 *     reference test tests/test_slot_mapping.py:53-66
 *   oracle_dequantize_and_gather_k_cache
 *     reference op   src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:38-172
 *     reference test tests/test_deepseek_v4_attention_dequantize_and_gather_k_cache.py:42-119
 *   oracle_indexer_k_quant_and_cache, oracle_cp_gather_indexer_k_quant_cache
 *     reference ops  src/flaggems_vllm/ops/indexer_k_quant_and_cache.py:44-132
 *                    src/flaggems_vllm/ops/cp_gather_indexer_k_quant_cache.py:23-176
 *     reference test tests/test_indexer_k_quant_and_cache.py:99-142 (torch_indexer)
 *                    tests/test_cp_gather_indexer_k_quant_cache.py:83-114 (torch_gather)
 *   oracle_mqa_logits, oracle_paged_mqa_logits (binary64 logits with an error
 *   bound for a binary32 implementation, see their comment)
 *     reference ops  src/flaggems_vllm/ops/fp8_fp4_mqa_logits.py:88-358, 523-651
 *                    src/flaggems_vllm/ops/fp8_fp4_paged_mqa_logits.py:68-225, 410-579
 *     reference test tests/test_fp8_fp4_mqa_logits.py:40-66 (reference_fp4_mqa_logits)
 *                    tests/test_fp8_fp4_paged_mqa_logits.py:196-249
 *   oracle_compute_global_topk_indices
 *     reference op   src/flaggems_vllm/ops/deepseek_v4_attention_compute_global_topk_indices_and_lens.py:46-160
 *     reference test tests/test_deepseek_v4_attention_compute_global_topk_indices_and_lens.py:78-98
 *   oracle_combine_topk_swa_indices
 *     reference op   src/flaggems_vllm/ops/deepseek_v4_attention_combine_topk_swa_indices.py:30-150
 *     reference test tests/test_deepseek_v4_attention_combine_topk_swa_indices.py:119-141
 *   oracle_top_k_per_row
 *     reference ops  src/flaggems_vllm/ops/top_k_per_row_decode.py:877-1043, 1263-1399
 *                    src/flaggems_vllm/ops/top_k_per_row_prefill.py:1232-1331
 *     reference test tests/test_top_k_per_row_decode.py:98-119 (_torch_topk_ref)
 *                    tests/test_top_k_per_row_prefill.py:79-100 (reference_top_k_per_row)
 *   oracle_fp8_einsum (binary64 with an error bound, see its comment)
 *     reference op   src/flaggems_vllm/ops/fp8_einsum.py:20-115
 *     reference test tests/test_fp8_einsum.py:124-156 (torch_fp8_block_einsum_reference)
 *   oracle_sparse_mla_decode_model1 (binary64 attention, see its comment)
 *     reference op   src/flaggems_vllm/ops/flash_mla_with_kvcache.py:489-688, 852-1073
 *                    src/flaggems_vllm/ops/flash_mla_with_kvcache_model1.py:389-470, 699-720
 *     reference test tests/test_flash_mla_with_kvcache.py:94-140, 236-360
 *
 * Numerics (compile with -ffp-contract=off and without -ffast-math):
 *   - every product and sum is a separately rounded binary32 operation, as in
 *     the torch oracle, so RoPE output and FP8 codes are fully determined;
 *   - float -> bf16 is round-to-nearest-even;
 *   - float -> e4m3fn is round-to-nearest-even with subnormals kept and no
 *     saturation (values rounding past 448 become NaN 0x7f), which is what
 *     torch's CPU cast does; the op clamps to +-448 first;
 *   - the RMSNorm factor is evaluated as
 *         w = (float)(sum_i (double)x_i^2 / 512) + eps      (binary32 add)
 *         r = (float)(1 / sqrt((double)w))
 *     i.e. the variance and the reciprocal square root are correctly rounded.
 *     The reference's fp32 sum (tl.sum / torch mean) and rsqrt are within a
 *     few fp32 ulps of this; the bar on q is 1 bf16 ulp.  The HIP kernel uses
 *     the same formulation so that it can be compared bit for bit.
 *
 * Parity pins (tests/test_oracle_*.py): e4m3fn encoder against torch's cast
 * exhaustively over every bf16 value times every reachable power-of-two scale;
 * bf16 rounding against torch's cast; the UE8M0 exponent against log2/ceil and
 * against exact rational arithmetic; RMS factor against exact rational
 * arithmetic; RoPE against closed-form rotations (identity, quarter turn,
 * forward-then-inverse); cache placement by brute force over small caches.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 512
#define NOPE_DIM 448
#define ROPE_DIM 64
#define HALF_ROPE 32
#define KV_QUANT_BLOCK 64
#define KV_NUM_QUANT_BLOCKS 7
#define TOKEN_DATA_BYTES 576
#define SCALE_BYTES_PER_TOKEN 8
#define FP8_MAX 448.0f

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16 -> binary32 (exact; subnormals kept). */
float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0x1f)
        return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0)
        return (sign ? -1.0f : 1.0f) * ldexpf((float)m, -24);
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

/* binary32 -> bfloat16, round to nearest, ties to even. NaN -> quiet NaN. */
uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t keep_lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + keep_lsb) >> 16);
}

/*
 * binary32 -> OCP e4m3fn code, round to nearest even.
 * Grid: subnormals m * 2^-9 (m = 0..7), normals (1 + m/8) * 2^e, e = -6..8,
 * code 0x7e = 448 is the largest finite value, 0x7f / 0xff are NaN.
 */
uint8_t oracle_e4m3fn(float x)
{
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) /* NaN */
        return (uint8_t)(sign | 0x7f);
    uint32_t code;
    if (a < 0x3c800000u) {
        /* |x| < 2^-6: the grid is k * 2^-9 for k = 0..8 (k = 8 is the
           smallest normal 2^-6, code 0x08).  |x| * 2^9 is exact. */
        float scaled = u2f(a) * 512.0f;
        code = (uint32_t)nearbyintf(scaled); /* default mode: ties to even */
    } else {
        int e = (int)(a >> 23) - 127; /* >= -6 */
        if (e > 15)
            return (uint8_t)(sign | 0x7f); /* far beyond 448, incl. inf */
        uint32_t mant = a & 0x7fffffu;
        code = ((uint32_t)(e + 7) << 3) | (mant >> 20);
        uint32_t rest = mant & 0xfffffu;
        if (rest > 0x80000u || (rest == 0x80000u && (code & 1u)))
            code += 1; /* a carry moves into the exponent field, as it should */
    }
    if (code > 0x7eu)
        code = 0x7fu; /* rounds past 448: NaN, there is no infinity */
    return (uint8_t)(sign | code);
}

/* OCP e4m3fn code -> binary32 (exact): 0x7f / 0xff are NaN, codes 1..7 are
   the subnormals m * 2^-9, others (1 + m/8) * 2^(e-7). */
float oracle_e4m3fn_to_f32(uint8_t code)
{
    int sign = code >> 7, e = (code >> 3) & 15, m = code & 7;
    float v;
    if (e == 15 && m == 7)
        v = NAN;
    else if (e == 0)
        v = ldexpf((float)m, -9);
    else
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -v : v;
}

void oracle_e4m3fn_decode_array(const uint8_t* codes, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_e4m3fn_to_f32(codes[i]);
}

void oracle_e4m3fn_array(const float* x, uint8_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_e4m3fn(x[i]);
}

void oracle_f32_to_bf16_array(const float* x, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_f32_to_bf16(x[i]);
}

/* The KV UE8M0 exponent as the reference writes it:
   k = ceil(log2(max(amax, 1e-4) / 448))   (ops/...insert.py:127-132). */
int oracle_kv_ue8m0_exponent(float amax)
{
    float a = amax > 1e-4f ? amax : 1e-4f;
    float raw = a / FP8_MAX;
    return (int)ceilf(log2f(raw));
}

/* RMSNorm factor of one 512-element bf16 row (see the header comment). */
float oracle_rms_factor(const uint16_t* row, float eps)
{
    double s = 0.0;
    for (int i = 0; i < HEAD_DIM; ++i) {
        double v = (double)oracle_bf16_to_f32(row[i]);
        s += v * v;
    }
    float w = (float)(s / (double)HEAD_DIM);
    w = w + eps;
    return (float)(1.0 / sqrt((double)w));
}

/* GPT-J pair rotation, separately rounded binary32 (tests/...insert.py:134-135). */
static inline void rope_pair(float e, float o, float c, float s, float* e_out, float* o_out)
{
    float ec = e * c, os = o * s, es = e * s, oc = o * c;
    *e_out = ec - os;
    *o_out = es + oc;
}

static inline int64_t clamp_pos(int64_t p, int64_t max_pos)
{
    if (p < 0) return 0;
    if (p >= max_pos) return max_pos - 1;
    return p;
}

/*
 * Main op.  q[t, h, :] at q + t*q_st + h*q_sh (bf16 elements), updated in place.
 * kv[t, :] at kv + t*kv_st, read only.  k_cache block b at k_cache + b*block_stride.
 */
void oracle_qnorm_rope_kv_insert(uint16_t* q, int64_t q_st, int64_t q_sh,
                                 const uint16_t* kv, int64_t kv_st,
                                 uint8_t* k_cache, int64_t block_stride, int64_t num_blocks,
                                 const int64_t* slot_mapping, int64_t num_tokens_insert,
                                 const int64_t* position_ids,
                                 const float* cos_sin, int64_t cs_stride, int64_t max_pos,
                                 int64_t num_tokens, int64_t num_heads,
                                 float eps, int64_t block_size, int nthreads)
{
    (void)nthreads;
    /* Q: RMSNorm over all 512 dims, store nope, rotate rope (ops/...insert.py:61-97). */
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t row = 0; row < num_tokens * num_heads; ++row) {
        int64_t t = row / num_heads, h = row % num_heads;
        uint16_t* x = q + t * q_st + h * q_sh;
        const float* cs = cos_sin + clamp_pos(position_ids[t], max_pos) * cs_stride;
        float r = oracle_rms_factor(x, eps);
        float y[ROPE_DIM];
        for (int i = 0; i < ROPE_DIM; ++i)
            y[i] = oracle_bf16_to_f32(x[NOPE_DIM + i]) * r;
        for (int i = 0; i < NOPE_DIM; ++i)
            x[i] = oracle_f32_to_bf16(oracle_bf16_to_f32(x[i]) * r);
        for (int j = 0; j < HALF_ROPE; ++j) {
            float e2, o2;
            rope_pair(y[2 * j], y[2 * j + 1], cs[j], cs[HALF_ROPE + j], &e2, &o2);
            x[NOPE_DIM + 2 * j] = oracle_f32_to_bf16(e2);
            x[NOPE_DIM + 2 * j + 1] = oracle_f32_to_bf16(o2);
        }
    }

    /* KV: rope slice to bf16, UE8M0 FP8 quant of the nope slice, paged insert
       (ops/...insert.py:98-286; tests/...insert.py:178-243). */
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t t = 0; t < num_tokens_insert; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0)
            continue;
        int64_t blk = slot / block_size, pos_in_block = slot % block_size;
        if (blk >= num_blocks)
            continue; /* the HIP kernel ignores out-of-range slots likewise */
        uint8_t* base = k_cache + blk * block_stride;
        uint8_t* tok = base + pos_in_block * TOKEN_DATA_BYTES;
        uint8_t* scl = base + block_size * TOKEN_DATA_BYTES + pos_in_block * SCALE_BYTES_PER_TOKEN;
        const uint16_t* x = kv + t * kv_st;
        const float* cs = cos_sin + clamp_pos(position_ids[t], max_pos) * cs_stride;

        for (int j = 0; j < HALF_ROPE; ++j) {
            float e2, o2;
            rope_pair(oracle_bf16_to_f32(x[NOPE_DIM + 2 * j]), oracle_bf16_to_f32(x[NOPE_DIM + 2 * j + 1]),
                      cs[j], cs[HALF_ROPE + j], &e2, &o2);
            uint16_t be = oracle_f32_to_bf16(e2), bo = oracle_f32_to_bf16(o2);
            memcpy(tok + NOPE_DIM + 4 * j, &be, 2); /* little-endian bf16 */
            memcpy(tok + NOPE_DIM + 4 * j + 2, &bo, 2);
        }
        for (int g = 0; g < KV_NUM_QUANT_BLOCKS; ++g) {
            float v[KV_QUANT_BLOCK];
            float amax = 0.0f;
            for (int i = 0; i < KV_QUANT_BLOCK; ++i) {
                v[i] = oracle_bf16_to_f32(x[g * KV_QUANT_BLOCK + i]);
                float a = fabsf(v[i]);
                amax = a > amax ? a : amax;
            }
            int k = oracle_kv_ue8m0_exponent(amax);
            float scale = ldexpf(1.0f, k); /* exact power of two */
            for (int i = 0; i < KV_QUANT_BLOCK; ++i) {
                float s = v[i] / scale;
                s = s < -FP8_MAX ? -FP8_MAX : (s > FP8_MAX ? FP8_MAX : s);
                tok[g * KV_QUANT_BLOCK + i] = oracle_e4m3fn(s);
            }
            int enc = k + 127;
            scl[g] = (uint8_t)(enc < 0 ? 0 : (enc > 255 ? 255 : enc));
        }
        scl[KV_NUM_QUANT_BLOCKS] = 0;
    }
}

/*
 * Sibling op.  Inverse GPT-J RoPE on the last rope_dim dims of each head
 * (head_dim = nope_dim + rope_dim), rope part rounded to bf16
 * (tests/test_fused_inv_rope_fp8_quant.py:163-170), then one scale per
 * quant_group_size-element chunk and e4m3fn codes (:177-198); the geometry
 * follows ops/fused_inv_rope_fp8_quant.py:192-205 (the kernel's rope start
 * ROPE_START = nope_dim % quant_group_size inside the last chunk, :229-247).
 *
 * fp8 output element (g, t, i) at fp8 + g*fp8_sg + t*fp8_st + i.
 * Scales: fp32 (tma == 0) at scale + g*sc_sg + k*sc_sk + t with
 * k = hig*chunks + c; packed int32 (tma != 0) at scale + g*sc_sg + hig*sc_sk
 * + t, byte c for chunk c < chunks (<= 4).  Tokens T..Tpad-1 get zero
 * scales (ops/fused_inv_rope_fp8_quant.py:69-88).
 */
void oracle_inv_rope_fp8_quant(const uint16_t* o, int64_t o_st, int64_t o_sh,
                               const int64_t* positions, const float* cos_sin, int64_t cs_stride,
                               int64_t max_pos, int64_t num_tokens, int64_t n_groups,
                               int64_t heads_per_group, int64_t nope_dim, int64_t rope_dim, int64_t group,
                               uint8_t* fp8, int64_t fp8_sg, int64_t fp8_st,
                               void* scale, int64_t sc_sg, int64_t sc_sk, int64_t tpad,
                               float eps, int tma, int nthreads)
{
    (void)nthreads;
    const float inv_max = (float)(1.0 / 448.0);
    const int64_t num_heads = n_groups * heads_per_group;
    const int64_t head_dim = nope_dim + rope_dim, half = rope_dim / 2, chunks = head_dim / group;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t row = 0; row < num_tokens * num_heads; ++row) {
        int64_t t = row / num_heads, h = row % num_heads;
        int64_t g = h / heads_per_group, hig = h % heads_per_group;
        const uint16_t* x = o + t * o_st + h * o_sh;
        const float* cs = cos_sin + clamp_pos(positions[t], max_pos) * cs_stride;
        float* v = (float*)malloc(sizeof(float) * (size_t)head_dim);
        for (int64_t i = 0; i < nope_dim; ++i)
            v[i] = oracle_bf16_to_f32(x[i]);
        for (int64_t j = 0; j < half; ++j) {
            float e = oracle_bf16_to_f32(x[nope_dim + 2 * j]);
            float od = oracle_bf16_to_f32(x[nope_dim + 2 * j + 1]);
            float c = cs[j], s = cs[half + j];
            float ec = e * c, os = od * s, oc = od * c, es = e * s;
            float e2 = ec + os; /* inverse rotation */
            float o2 = oc - es;
            v[nope_dim + 2 * j] = oracle_bf16_to_f32(oracle_f32_to_bf16(e2));
            v[nope_dim + 2 * j + 1] = oracle_bf16_to_f32(oracle_f32_to_bf16(o2));
        }
        uint8_t* out = fp8 + g * fp8_sg + t * fp8_st + hig * head_dim;
        uint32_t packed = 0;
        for (int64_t c = 0; c < chunks; ++c) {
            float amax = 0.0f;
            for (int64_t i = 0; i < group; ++i) {
                float a = fabsf(v[c * group + i]);
                amax = a > amax ? a : amax;
            }
            float absmax = amax > eps ? amax : eps;
            float sc = absmax * inv_max;
            if (tma) {
                float cl = sc > 1e-10f ? sc : 1e-10f;
                sc = ldexpf(1.0f, (int)ceilf(log2f(cl)));
                packed |= ((f2u(sc) >> 23) & 0xffu) << (8 * c);
            } else {
                ((float*)scale)[g * sc_sg + (hig * chunks + c) * sc_sk + t] = sc;
            }
            for (int64_t i = 0; i < group; ++i) {
                float qv = v[c * group + i] / sc;
                qv = qv < -FP8_MAX ? -FP8_MAX : (qv > FP8_MAX ? FP8_MAX : qv);
                out[c * group + i] = oracle_e4m3fn(qv);
            }
        }
        if (tma)
            ((int32_t*)scale)[g * sc_sg + hig * sc_sk + t] = (int32_t)packed;
        free(v);
    }
    for (int64_t t = num_tokens; t < tpad; ++t)
        for (int64_t g = 0; g < n_groups; ++g) {
            if (tma) {
                for (int64_t hig = 0; hig < heads_per_group; ++hig)
                    ((int32_t*)scale)[g * sc_sg + hig * sc_sk + t] = 0;
            } else {
                for (int64_t k = 0; k < heads_per_group * chunks; ++k)
                    ((float*)scale)[g * sc_sg + k * sc_sk + t] = 0.0f;
            }
        }
}

/*
 * dequantize_and_gather_k_cache: out element (r, j, c) at out + r*out_s0 +
 * j*out_s1 + c (bf16).  For request r and i < gather_len (and offset + i <
 * out_rows): pos = seq_len - gather_len + i, block block_table[r*bt_stride +
 * pos / bs]; nope column c -> bf16(e4m3(code_c) * 2^(scale[c/64] - 127)),
 * rope columns copy the cached bf16 values (reference kernel :61-120).  Rows
 * whose block index or block is out of range are skipped, as in the kernel.
 */
void oracle_dequantize_and_gather_k_cache(uint16_t* out, int64_t out_s0, int64_t out_s1, int64_t out_rows,
                                          const uint8_t* cache, int64_t block_stride, int64_t num_blocks,
                                          const int32_t* seq_lens, const int32_t* gather_lens,
                                          const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                                          int64_t num_reqs, int64_t bs, int64_t offset,
                                          int64_t nope, int64_t rope, int64_t scale_slots)
{
    int64_t token_bytes = nope + 2 * rope;
    for (int64_t r = 0; r < num_reqs; ++r) {
        int64_t seq_len = seq_lens[r];
        int64_t gl = gather_lens ? gather_lens[r] : seq_len;
        for (int64_t i = 0; i < gl && offset + i < out_rows; ++i) {
            int64_t pos = seq_len - gl + i;
            if (pos < 0 || pos / bs >= max_blocks)
                continue;
            int64_t blk = block_table[r * bt_stride + pos / bs];
            if (blk < 0 || blk >= num_blocks)
                continue;
            int64_t pib = pos % bs;
            const uint8_t* base = cache + blk * block_stride;
            const uint8_t* tok = base + pib * token_bytes;
            const uint8_t* scl = base + bs * token_bytes + pib * scale_slots;
            uint16_t* row = out + r * out_s0 + (offset + i) * out_s1;
            for (int64_t c = 0; c < nope; ++c) {
                float scale = ldexpf(1.0f, (int)scl[c / 64] - 127);
                row[c] = oracle_f32_to_bf16(oracle_e4m3fn_to_f32(tok[c]) * scale);
            }
            for (int64_t c = 0; c < rope; ++c)
                memcpy(row + nope + c, tok + nope + 2 * c, 2);
        }
    }
}

/* Weighted RMSNorm of one bf16 row: y = (x * r) * w with r as in
   oracle_rms_factor but over `size` elements (reference kernel :55-62). */
static void rmsnorm_row(const uint16_t* x, uint16_t* y, const void* w, int w_f32, int64_t size,
                        float eps)
{
    double s = 0.0;
    for (int64_t i = 0; i < size; ++i) {
        double v = (double)oracle_bf16_to_f32(x[i]);
        s += v * v;
    }
    float var = (float)(s / (double)size);
    var = var + eps;
    float r = (float)(1.0 / sqrt((double)var));
    for (int64_t i = 0; i < size; ++i) {
        float wi = w_f32 ? ((const float*)w)[i] : oracle_bf16_to_f32(((const uint16_t*)w)[i]);
        float t = oracle_bf16_to_f32(x[i]) * r;
        y[i] = oracle_f32_to_bf16(t * wi);
    }
}

void oracle_fused_q_kv_rmsnorm(const uint16_t* qr, int64_t qr_st, uint16_t* qr_out, int64_t qo_st,
                               const void* q_w, int64_t q_size,
                               const uint16_t* kv, int64_t kv_st, uint16_t* kv_out, int64_t ko_st,
                               const void* kv_w, int64_t kv_size,
                               int64_t num_tokens, float eps, int w_f32, int nthreads)
{
    (void)nthreads;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t t = 0; t < num_tokens; ++t) {
        rmsnorm_row(qr + t * qr_st, qr_out + t * qo_st, q_w, w_f32, q_size, eps);
        rmsnorm_row(kv + t * kv_st, kv_out + t * ko_st, kv_w, w_f32, kv_size, eps);
    }
}

/*
 * binary32 -> E2M1 nibble (FP4: values 0, 0.5, 1, 1.5, 2, 3, 4, 6), round to
 * nearest with ties to the even code, saturating at 6; bit 3 is the sign of x
 * (so -0 and negative values that round to 0 keep it).  On [0, 2) the grid
 * step is 0.5, on [2, 4) 1 and on [4, 6] 2, so the code is the step index
 * rounded to nearest even, offset by the first code of the interval.
 */
uint8_t oracle_e2m1(float x)
{
    uint8_t sign = (uint8_t)((f2u(x) >> 31) << 3);
    float a = fabsf(x);
    if (a > 6.0f)
        a = 6.0f;
    uint32_t code;
    if (a < 2.0f)
        code = (uint32_t)nearbyintf(a * 2.0f);
    else if (a < 4.0f)
        code = 4u + (uint32_t)nearbyintf(a - 2.0f);
    else
        code = 6u + (uint32_t)nearbyintf((a - 4.0f) * 0.5f);
    return (uint8_t)(sign | code);
}

void oracle_e2m1_array(const float* x, uint8_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_e2m1(x[i]);
}

/*
 * fused_indexer_q_rope_quant.  q[t, h, i] at q + t*q_st + h*q_sh (bf16);
 * GPT-J RoPE on the last 64 dims rounded to bf16 (reference kernel :113-123),
 * then FP8 (one 2^k per row, folded into the weights, :125-167) or MXFP4
 * (one 2^k per 32 elements, :39-58, :211-282).
 */
void oracle_fused_indexer_q_rope_quant(const int64_t* positions, int64_t T,
                                       const uint16_t* q, int64_t q_st, int64_t q_sh, int64_t H, int64_t D,
                                       const void* cs, int64_t cs_st, int64_t max_pos, int cs_bf16,
                                       const void* w, int64_t w_st, int w_f32,
                                       float softmax_scale, float head_scale,
                                       float* wo, int64_t wo_st, int fp4,
                                       uint8_t* qo, int64_t qo_st, int64_t qo_sh,
                                       uint8_t* so, int64_t so_st, int64_t so_sh)
{
    int64_t nope = D - ROPE_DIM;
    float x[4096];
    for (int64_t t = 0; t < T; ++t) {
        int64_t pos = clamp_pos(positions[t], max_pos);
        for (int64_t h = 0; h < H; ++h) {
            const uint16_t* row = q + t * q_st + h * q_sh;
            for (int64_t i = 0; i < D; ++i)
                x[i] = oracle_bf16_to_f32(row[i]);
            for (int j = 0; j < HALF_ROPE; ++j) {
                float c, s;
                if (cs_bf16) {
                    c = oracle_bf16_to_f32(((const uint16_t*)cs)[pos * cs_st + j]);
                    s = oracle_bf16_to_f32(((const uint16_t*)cs)[pos * cs_st + HALF_ROPE + j]);
                } else {
                    c = ((const float*)cs)[pos * cs_st + j];
                    s = ((const float*)cs)[pos * cs_st + HALF_ROPE + j];
                }
                float e = x[nope + 2 * j], o = x[nope + 2 * j + 1];
                float ec = e * c, os = o * s, oc = o * c, es = e * s;
                float re = ec - os, ro = oc + es;
                x[nope + 2 * j] = oracle_bf16_to_f32(oracle_f32_to_bf16(re));
                x[nope + 2 * j + 1] = oracle_bf16_to_f32(oracle_f32_to_bf16(ro));
            }
            float wv = w_f32 ? ((const float*)w)[t * w_st + h]
                             : oracle_bf16_to_f32(((const uint16_t*)w)[t * w_st + h]);
            uint8_t* out = qo + t * qo_st + h * qo_sh;
            if (!fp4) {
                float amax = 0.0f;
                for (int64_t i = 0; i < D; ++i)
                    amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
                float a = amax > 1e-4f ? amax : 1e-4f;
                float scale = ldexpf(1.0f, (int)ceilf(log2f(a / FP8_MAX)));
                for (int64_t i = 0; i < D; ++i)
                    out[i] = oracle_e4m3fn(x[i] / scale);
                float r = wv * scale;
                r = r * softmax_scale;
                wo[t * wo_st + h] = r * head_scale;
            } else {
                uint8_t* sc = so + t * so_st + h * so_sh;
                for (int64_t b = 0; b < D / 32; ++b) {
                    float amax = 0.0f;
                    for (int i = 0; i < 32; ++i)
                        amax = fabsf(x[b * 32 + i]) > amax ? fabsf(x[b * 32 + i]) : amax;
                    const float floor6 = 6.0f * 0x1p-126f;
                    float a = amax > floor6 ? amax : floor6;
                    float k = ceilf(log2f(a * (1.0f / 6.0f)));
                    k = k < -127.0f ? -127.0f : (k > 127.0f ? 127.0f : k);
                    float scale = ldexpf(1.0f, (int)k);
                    sc[b] = (uint8_t)(k + 127.0f);
                    for (int i = 0; i < 32; i += 2) {
                        uint8_t lo = oracle_e2m1(x[b * 32 + i] / scale);
                        uint8_t hi = oracle_e2m1(x[b * 32 + i + 1] / scale);
                        out[(b * 32 + i) / 2] = (uint8_t)(lo | (hi << 4));
                    }
                }
                float r = wv * softmax_scale;
                wo[t * wo_st + h] = r * head_scale;
            }
        }
    }
}

/* Slot mapping, request by request as the stock per-request kernel walks it
   (reference test :53-66 for cp_world = 1, CP arithmetic from the op :88-105). */
void oracle_compute_slot_mapping(int64_t num_tokens, int64_t max_num_tokens, const int32_t* qsl,
                                 int64_t num_reqs, const void* positions, int pos64,
                                 const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                                 int64_t* out, int64_t bs, int64_t cpw, int64_t cp_rank, int64_t il,
                                 int64_t pad_id)
{
    for (int64_t t = num_tokens; t < max_num_tokens; ++t)
        out[t] = pad_id;
    for (int64_t r = 0; r < num_reqs; ++r) {
        for (int64_t t = qsl[r]; t < qsl[r + 1] && t < num_tokens && t < max_num_tokens; ++t) {
            int64_t pos = pos64 ? (int32_t)((const int64_t*)positions)[t] : ((const int32_t*)positions)[t];
            int64_t vbs = bs * cpw;
            int64_t bi = pos / vbs;
            if (pos < 0 || bi >= max_blocks) {
                out[t] = pad_id;
                continue;
            }
            int64_t blk = block_table[r * bt_stride + bi];
            int64_t voff = pos - bi * vbs;
            int local = (voff / il) % cpw == cp_rank;
            int64_t loff = voff / (cpw * il) * il + voff % il;
            out[t] = local ? blk * bs + loff : pad_id;
        }
    }
}

/*
 * Sparse MLA decode over the 584-byte MODEL1 cache
 * (reference portable kernel ops/flash_mla_with_kvcache.py:489-688 and the
 * sm90 kernel ops/flash_mla_with_kvcache_model1.py:389-470, 699-720):
 *
 *   K = V = the dequantised 512-wide latent of each selected token:
 *     dims [0,448):   bf16(e4m3(code) * 2^(scale_byte[d/64] - 127))  (f32 product, RNE)
 *     dims [448,512): the cached bf16 RoPE values
 *   A selected entry t of a list is used when t < len, id >= 0 and
 *   id / page < num_blocks (len = topk, or topk_length[b] clamped to
 *   [0, topk]).  The extra list is attended together with the main one.
 *   For each head: s_t = sm_scale * q . K_t, m = max s_t,
 *   l = sum exp(s_t - m), lse = m + log(l)   (+inf when nothing is used),
 *   out = sum_t exp(s_t - m) V_t / (l + exp(sink - m))   (sink term only with
 *   attn_sink; out = 0 when nothing is used).
 *
 * Everything after the dequantisation is evaluated in binary64, so this is
 * the exact attention the reference's fp32/bf16 kernels approximate.
 * q, out: [B][SQ][HQ][512] contiguous; lse: [B][HQ][SQ].
 */
void oracle_model1_token_row(const uint8_t* cache, int64_t block_stride, int64_t page, int64_t id,
                             uint16_t* row)
{
    int64_t blk = id / page, rel = id % page;
    const uint8_t* tok = cache + blk * block_stride + rel * TOKEN_DATA_BYTES;
    const uint8_t* scl = cache + blk * block_stride + page * TOKEN_DATA_BYTES + rel * SCALE_BYTES_PER_TOKEN;
    for (int c = 0; c < NOPE_DIM; ++c) {
        float scale = u2f((uint32_t)scl[c / KV_QUANT_BLOCK] << 23);
        row[c] = oracle_f32_to_bf16(oracle_e4m3fn_to_f32(tok[c]) * scale);
    }
    memcpy(row + NOPE_DIM, tok + NOPE_DIM, 2 * ROPE_DIM);
}

struct mla_list {
    const uint8_t* cache;
    int64_t num_blocks, page, block_stride;
    const int32_t* idx;
    int64_t topk;
    const int32_t* len;
};

static int64_t mla_collect(const struct mla_list* L, int64_t b, int64_t sq, int64_t SQ, int64_t* ids)
{
    if (!L->cache)
        return 0;
    int64_t len = L->topk;
    if (L->len) {
        len = L->len[b];
        len = len < 0 ? 0 : len > L->topk ? L->topk : len;
    }
    const int32_t* row = L->idx + (b * SQ + sq) * L->topk;
    int64_t n = 0;
    for (int64_t t = 0; t < len; ++t) {
        int64_t id = row[t];
        if (id >= 0 && id / L->page < L->num_blocks)
            ids[n++] = id;
    }
    return n;
}

void oracle_sparse_mla_decode_model1(const uint16_t* q, int64_t B, int64_t SQ, int64_t HQ,
                                     const uint8_t* cache, int64_t num_blocks, int64_t page,
                                     int64_t block_stride, const int32_t* idx, int64_t topk,
                                     const int32_t* topk_len,
                                     const uint8_t* ecache, int64_t enum_blocks, int64_t epage,
                                     int64_t eblock_stride, const int32_t* eidx, int64_t etopk,
                                     const int32_t* etopk_len,
                                     const float* sink, double sm_scale, double* out, double* lse)
{
    struct mla_list lists[2] = {
        {cache, num_blocks, page, block_stride, idx, topk, topk_len},
        {ecache, enum_blocks, epage, eblock_stride, eidx, etopk, etopk_len},
    };
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t sq = 0; sq < SQ; ++sq) {
            int64_t cap = topk + (ecache ? etopk : 0);
            int64_t* ids = (int64_t*)malloc(sizeof(int64_t) * (cap ? cap : 1));
            int* which = (int*)malloc(sizeof(int) * (cap ? cap : 1));
            int64_t n = 0;
            for (int li = 0; li < 2; ++li) {
                int64_t k = mla_collect(&lists[li], b, sq, SQ, ids + n);
                for (int64_t i = 0; i < k; ++i)
                    which[n + i] = li;
                n += k;
            }
            double* kv = (double*)malloc(sizeof(double) * HEAD_DIM * (n ? n : 1));
            uint16_t row[HEAD_DIM];
            for (int64_t t = 0; t < n; ++t) {
                const struct mla_list* L = &lists[which[t]];
                oracle_model1_token_row(L->cache, L->block_stride, L->page, ids[t], row);
                for (int d = 0; d < HEAD_DIM; ++d)
                    kv[t * HEAD_DIM + d] = oracle_bf16_to_f32(row[d]);
            }
            #pragma omp parallel for schedule(static)
            for (int64_t h = 0; h < HQ; ++h) {
                const uint16_t* qh = q + ((b * SQ + sq) * HQ + h) * HEAD_DIM;
                double* oh = out + ((b * SQ + sq) * HQ + h) * HEAD_DIM;
                double* lh = lse + (b * HQ + h) * SQ + sq;
                double qd[HEAD_DIM];
                for (int d = 0; d < HEAD_DIM; ++d)
                    qd[d] = oracle_bf16_to_f32(qh[d]);
                for (int d = 0; d < HEAD_DIM; ++d)
                    oh[d] = 0.0;
                if (n == 0) {
                    *lh = INFINITY;
                    continue;
                }
                double* s = (double*)malloc(sizeof(double) * n);
                double m = -INFINITY;
                for (int64_t t = 0; t < n; ++t) {
                    double acc = 0.0;
                    for (int d = 0; d < HEAD_DIM; ++d)
                        acc += qd[d] * kv[t * HEAD_DIM + d];
                    s[t] = acc * sm_scale;
                    if (s[t] > m)
                        m = s[t];
                }
                double l = 0.0;
                for (int64_t t = 0; t < n; ++t) {
                    s[t] = exp(s[t] - m);
                    l += s[t];
                }
                *lh = m + log(l);
                double denom = l + (sink ? exp((double)sink[h] - m) : 0.0);
                for (int64_t t = 0; t < n; ++t) {
                    double w = s[t] / denom;
                    for (int d = 0; d < HEAD_DIM; ++d)
                        oh[d] += w * kv[t * HEAD_DIM + d];
                }
                free(s);
            }
            free(kv);
            free(which);
            free(ids);
        }
    }
}

/*
 * Sparse MLA prefill over bf16 kv rows (reference wrapper
 * ops/flashmla_sparse.py:1045-1206, kernel :50-195; the outputs as the
 * reference test defines them, tests/test_flash_mla_sparse_fwd.py:93-150):
 *
 *   Token t attends entry i of indices[t] when i < len (topk, or
 *   topk_length[t] clamped to [0, topk]) and 0 <= id < s_kv.
 *   K = kv[id][0:d_qk], V = kv[id][0:512].  For each head:
 *   s_i = sm_scale * q . K_i, max_logits = max s_i (-inf when nothing is
 *   used), lse = m + log sum exp(s_i - m) (+inf when nothing is used),
 *   out = sum exp(s_i - m) V_i / (l + exp(sink - m)) (sink term only with
 *   attn_sink; 0 when nothing is used).  Binary64 throughout.
 * q: [s_q][h_q][d_qk] contiguous; kv rows kv_row elements apart;
 * indices [s_q][topk]; out [s_q][h_q][512]; max_logits, lse [s_q][h_q].
 */
void oracle_sparse_mla_prefill(const uint16_t* q, const uint16_t* kv, int64_t kv_row, int64_t s_kv,
                               const int32_t* idx, int64_t topk, const int32_t* topk_len, const float* sink,
                               double sm_scale, int64_t s_q, int64_t h_q, int64_t d_qk, double* out,
                               double* max_logits, double* lse)
{
    for (int64_t t = 0; t < s_q; ++t) {
        int64_t len = topk;
        if (topk_len) {
            len = topk_len[t];
            len = len < 0 ? 0 : len > topk ? topk : len;
        }
        int64_t* ids = (int64_t*)malloc(sizeof(int64_t) * (topk ? topk : 1));
        int64_t n = 0;
        for (int64_t i = 0; i < len; ++i) {
            int64_t id = idx[t * topk + i];
            if (id >= 0 && id < s_kv)
                ids[n++] = id;
        }
        double* k = (double*)malloc(sizeof(double) * d_qk * (n ? n : 1));
        for (int64_t i = 0; i < n; ++i)
            for (int64_t d = 0; d < d_qk; ++d)
                k[i * d_qk + d] = oracle_bf16_to_f32(kv[ids[i] * kv_row + d]);
        #pragma omp parallel for schedule(static)
        for (int64_t h = 0; h < h_q; ++h) {
            const uint16_t* qh = q + (t * h_q + h) * d_qk;
            double* oh = out + (t * h_q + h) * HEAD_DIM;
            for (int d = 0; d < HEAD_DIM; ++d)
                oh[d] = 0.0;
            if (n == 0) {
                max_logits[t * h_q + h] = -INFINITY;
                lse[t * h_q + h] = INFINITY;
                continue;
            }
            double* s = (double*)malloc(sizeof(double) * n);
            double m = -INFINITY;
            for (int64_t i = 0; i < n; ++i) {
                double acc = 0.0;
                for (int64_t d = 0; d < d_qk; ++d)
                    acc += (double)oracle_bf16_to_f32(qh[d]) * k[i * d_qk + d];
                s[i] = acc * sm_scale;
                if (s[i] > m)
                    m = s[i];
            }
            double l = 0.0;
            for (int64_t i = 0; i < n; ++i) {
                s[i] = exp(s[i] - m);
                l += s[i];
            }
            max_logits[t * h_q + h] = m;
            lse[t * h_q + h] = m + log(l);
            double denom = l + (sink ? exp((double)sink[h] - m) : 0.0);
            for (int64_t i = 0; i < n; ++i) {
                double w = s[i] / denom;
                for (int d = 0; d < HEAD_DIM; ++d)
                    oh[d] += w * k[i * d_qk + d];
            }
            free(s);
        }
        free(k);
        free(ids);
    }
}

/* ------------------------------------------------------------------------
 * Sparse indexer key cache (reference test torch_indexer / torch_gather).
 * Cache block b at cache + b * block_stride: block_size x head_dim e4m3fn
 * codes, then block_size x (head_dim / qbs) float32 scales.
 * ------------------------------------------------------------------------ */

/* k: [T, head_dim] bf16 (k_fp16 = 0) or fp16 (k_fp16 = 1), row stride k_st
 * elements.  For token t with slot s >= 0 and quant block j:
 *   scale = fl32(max(amax_j, 1e-4) / 448), ue8m0: 2^ceil(log2(scale))
 *   code  = e4m3fn(fl32(k / scale)) (division IEEE; |k / scale| <= 448(1+eps)
 *           rounds to 448 at most, so no clamp is needed)
 * exactly as the torch oracle writes them (tests/test_indexer_k_quant_and_cache.py:118-142). */
void oracle_indexer_k_quant_and_cache(const uint16_t* k, int64_t k_st, int k_fp16, int64_t T, int64_t head_dim,
                                      int64_t qbs, uint8_t* cache, int64_t block_stride, int64_t num_blocks,
                                      int64_t block_size, const int64_t* slots, int ue8m0)
{
    if (qbs <= 0 || qbs > 1024)
        return; /* v[] below holds one quant block */
    int64_t nqb = head_dim / qbs;
    for (int64_t t = 0; t < T; ++t) {
        int64_t slot = slots[t];
        if (slot < 0)
            continue;
        int64_t blk = slot / block_size, row = slot % block_size;
        if (blk >= num_blocks)
            continue;
        uint8_t* base = cache + blk * block_stride;
        for (int64_t j = 0; j < nqb; ++j) {
            float v[1024];
            float amax = 0.0f;
            for (int64_t i = 0; i < qbs; ++i) {
                uint16_t h = k[t * k_st + j * qbs + i];
                v[i] = k_fp16 ? oracle_f16_to_f32(h) : oracle_bf16_to_f32(h);
                float a = fabsf(v[i]);
                amax = a > amax ? a : amax;
            }
            float scale = (amax > 1e-4f ? amax : 1e-4f) / 448.0f;
            if (ue8m0)
                scale = exp2f(ceilf(log2f(scale)));
            for (int64_t i = 0; i < qbs; ++i)
                base[row * head_dim + j * qbs + i] = oracle_e4m3fn(v[i] / scale);
            memcpy(base + block_size * head_dim + (row * nqb + j) * 4, &scale, 4);
        }
    }
}

/* Token t of request b (cu[b] <= t < cu[b + 1], t < T) takes position
 * pos = t - cu[b] from block block_table[b, pos / block_size], row
 * pos % block_size: head_dim code bytes into k_out + t * k_out_st and
 * nqb float32 scales into scale_out + t * scale_out_st (byte strides).
 * A position whose table index is >= max_blocks, or whose block is outside
 * [0, num_blocks), is skipped (its rows keep their contents): the product's
 * documented contract where the reference's behaviour is undefined. */
void oracle_cp_gather_indexer_k_quant_cache(const uint8_t* cache, int64_t block_stride, int64_t num_blocks,
                                            int64_t block_size, int64_t head_dim, int64_t qbs, uint8_t* k_out,
                                            int64_t k_out_st, uint8_t* scale_out, int64_t scale_out_st,
                                            const int32_t* block_table, int64_t bt_stride, int64_t max_blocks,
                                            const int32_t* cu, int64_t batch, int64_t T)
{
    int64_t nqb = head_dim / qbs;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t t = cu[b]; t < cu[b + 1] && t < T; ++t) {
            if (t < 0)
                continue;
            int64_t pos = t - cu[b];
            if (pos / block_size >= max_blocks)
                continue;
            int64_t blk = block_table[b * bt_stride + pos / block_size], row = pos % block_size;
            if (blk < 0 || blk >= num_blocks)
                continue;
            const uint8_t* base = cache + blk * block_stride;
            memcpy(k_out + t * k_out_st, base + row * head_dim, (size_t)head_dim);
            memcpy(scale_out + t * scale_out_st, base + block_size * head_dim + row * nqb * 4, (size_t)(nqb * 4));
        }
    }
}

/* ------------------------------------------------------------------------
 * Sparse-indexer logits (reference fp8_fp4_mqa_logits / paged variant):
 *   logit[m, n] = sum_h ReLU((sum_d q[m,h,d] k[n,d]) * k_scale[n]) * w[m,h]
 * q is e4m3fn, or E2M1 nibbles (even d in the low nibble) times
 * 2^(byte - 127), byte b of q_scale[m, h] covering d = 32b..32b+31 (MXFP4);
 * k is e4m3fn.  Everything is binary64: the products of two 4-bit
 * significands and their 128-term sums are exact.  bound[] receives an error
 * bound for an implementation that forms each head's dot product with the
 * FP8 matrix instruction (128 products added in groups of 8 consecutive d,
 * each truncated toward zero to a multiple of 2^(E_g - 13), E_g the group's
 * largest exponent sum e(q) + e(k), the group sums added in binary32: the
 * behaviour tests/test_fp8_einsum.py pins for e4m3 x e4m3), gates it, sums
 * the H weighted heads in any order and multiplies by k_scale:
 *   k_scale * sum_h |w_h| (t_h + (H + 3) 2^-24 (|dot_h| + t_h)),
 *   t_h = T_h + gamma (a_h + T_h),  T_h = sum_g n_g 2^(E_g - 13),
 * with a_h = sum_d |q_hd k_d| and gamma = D 2^-24.  e is the unbiased
 * exponent (-6 for zero and subnormal e4m3 codes).  For MXFP4 q, whose
 * grouping in the instruction is not pinned, a group is the whole 32-element
 * scale block (n_g = 32) and e(q) = e(E2M1) + byte - 127 with 0 and 0.5
 * taken at exponent 0: larger than any grouping of those 32 products gives.
 * Positions a cleaned output leaves at -inf (or a paged row's fill value)
 * get that value and bound 0.
 * ------------------------------------------------------------------------ */

static double oracle_e2m1_value(unsigned nib)
{
    static const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    return (nib & 8u) ? -mag[nib & 7u] : mag[nib & 7u];
}

/* q row of one query: H x D binary64 values into qd. */
static int oracle_e4m3_exp(uint8_t code)
{
    const int e = (code >> 3) & 15;
    return e ? e - 7 : -6;
}

/* q row of one query: H x D binary64 values into qd, exponents (for the
 * bound) into qe. */
static void oracle_query_values(const uint8_t* q_row, int64_t q_sh, const int32_t* qs_row, int64_t qs_sh, int64_t H,
                                int64_t D, double* qd, int* qe)
{
    for (int64_t h = 0; h < H; ++h) {
        const uint8_t* hr = q_row + h * q_sh;
        for (int64_t d = 0; d < D; ++d) {
            if (qs_row) {
                uint32_t sb = (uint32_t)qs_row[h * qs_sh];
                int byte = (int)((sb >> (8 * (d / 32))) & 0xffu);
                unsigned nib = (hr[d / 2] >> (4 * (d % 2))) & 0xfu;
                const unsigned m = nib & 7u;
                qd[h * D + d] = ldexp(oracle_e2m1_value(nib), byte - 127);
                qe[h * D + d] = (m >= 6 ? 2 : m >= 4 ? 1 : 0) + byte - 127;
            } else {
                qd[h * D + d] = (double)oracle_e4m3fn_to_f32(hr[d]);
                qe[h * D + d] = oracle_e4m3_exp(hr[d]);
            }
        }
    }
}

/* group: 8 products (e4m3 q) or 32 (MXFP4 q) per truncation group. */
static void oracle_logit_one(const double* qd, const int* qe, int64_t group, const float* w_row, int64_t w_sh,
                             int64_t H, int64_t D, const uint8_t* krow, float kscale, double* out, double* bound)
{
    const double u = ldexp(1.0, -24), gamma = (double)D * u;
    double kv[1024];
    int ke[1024];
    for (int64_t d = 0; d < D; ++d) {
        kv[d] = (double)oracle_e4m3fn_to_f32(krow[d]);
        ke[d] = oracle_e4m3_exp(krow[d]);
    }
    double sum = 0.0, err = 0.0;
    for (int64_t h = 0; h < H; ++h) {
        double dot = 0.0, a = 0.0, tr = 0.0;
        for (int64_t g0 = 0; g0 < D; g0 += group) {
            int eg = -1000;
            for (int64_t d = g0; d < g0 + group && d < D; ++d) {
                const double t = qd[h * D + d] * kv[d];
                dot += t;
                a += fabs(t);
                const int e = qe[h * D + d] + ke[d];
                eg = e > eg ? e : eg;
            }
            tr += (double)group * ldexp(1.0, eg - 13);
        }
        const double td = tr + gamma * (a + tr);
        double s = dot * (double)kscale;
        double wh = (double)w_row[h * w_sh];
        sum += (s > 0.0 ? s : 0.0) * wh;
        err += fabs(wh) * (td + (double)(H + 3) * u * (fabs(dot) + td));
    }
    *out = sum;
    *bound = fabs((double)kscale) * err;
}

/* Dense: the listed query rows (row r of out/bound = query rows[r]) x all N keys. */
void oracle_mqa_logits(const uint8_t* q, int64_t q_sm, int64_t q_sh, const int32_t* q_scale, int64_t qs_sm,
                       int64_t qs_sh, const uint8_t* k, int64_t k_sn, const float* k_scale, const float* w,
                       int64_t w_sm, int64_t w_sh, const int32_t* ks, const int32_t* ke, int clean, int64_t N,
                       int64_t H, int64_t D, const int64_t* rows, int64_t nrows, double* out, double* bound)
{
    if (D > 1024)
        return;
#pragma omp parallel for schedule(dynamic)
    for (int64_t r = 0; r < nrows; ++r) {
        const int64_t m = rows[r];
        double* qd = (double*)malloc(sizeof(double) * (size_t)(H * D));
        int* qe = (int*)malloc(sizeof(int) * (size_t)(H * D));
        if (!qd || !qe) {
            free(qd);
            free(qe);
            continue;
        }
        oracle_query_values(q + m * q_sm, q_sh, q_scale ? q_scale + m * qs_sm : NULL, qs_sh, H, D, qd, qe);
        for (int64_t n = 0; n < N; ++n) {
            if (clean && (n < ks[m] || n >= ke[m])) {
                out[r * N + n] = -INFINITY;
                bound[r * N + n] = 0.0;
                continue;
            }
            oracle_logit_one(qd, qe, q_scale ? 32 : 8, w + m * w_sm, w_sh, H, D, k + n * k_sn, k_scale[n],
                             &out[r * N + n], &bound[r * N + n]);
        }
        free(qd);
        free(qe);
    }
}

/* Paged: the listed rows x positions 0..max_model_len-1.  Row `row` reads
 * context_lens[row / rows_per_context_len] positions through block-table row
 * row / rows_per_table_row;
 * position n is entry n % block_size of block clamp(table[min(n / block_size,
 * max_blocks - 1)], 0, num_blocks - 1) (a position past the table reads
 * the table's last block); codes at block + slot * 128 (D bytes),
 * the float32 scale at block + block_size * D + 4 slot. */
void oracle_paged_mqa_logits(const uint8_t* q, int64_t q_sr, int64_t q_sh, const int32_t* q_scale, int64_t qs_sr,
                             int64_t qs_sh, const uint8_t* kv, int64_t block_stride, int64_t num_blocks,
                             int64_t block_size, const float* w, int64_t w_sr, int64_t w_sh, const int32_t* ctx,
                             int64_t rows_per_context_len, const int32_t* bt, int64_t bt_sr, int64_t max_blocks,
                             int64_t rows_per_table_row,
                             int64_t H, int64_t D, int64_t max_model_len, float fill, const int64_t* rows,
                             int64_t nrows, double* out, double* bound)
{
    if (D > 1024)
        return;
#pragma omp parallel for schedule(dynamic)
    for (int64_t r = 0; r < nrows; ++r) {
        const int64_t row = rows[r];
        double* qd = (double*)malloc(sizeof(double) * (size_t)(H * D));
        int* qe = (int*)malloc(sizeof(int) * (size_t)(H * D));
        if (!qd || !qe) {
            free(qd);
            free(qe);
            continue;
        }
        oracle_query_values(q + row * q_sr, q_sh, q_scale ? q_scale + row * qs_sr : NULL, qs_sh, H, D, qd, qe);
        int64_t c = ctx[row / rows_per_context_len];
        if (c < 0)
            c = 0;
        if (c > max_model_len)
            c = max_model_len;
        const int32_t* tab = bt + (row / rows_per_table_row) * bt_sr;
        for (int64_t n = 0; n < max_model_len; ++n) {
            if (n >= c) {
                out[r * max_model_len + n] = (double)fill;
                bound[r * max_model_len + n] = 0.0;
                continue;
            }
            int64_t lb = n / block_size;
            const int64_t slot = n - lb * block_size;
            if (lb > max_blocks - 1)
                lb = max_blocks - 1;
            int64_t blk = tab[lb];
            if (blk < 0)
                blk = 0;
            if (blk > num_blocks - 1)
                blk = num_blocks - 1;
            const uint8_t* base = kv + blk * block_stride;
            float ksc;
            memcpy(&ksc, base + block_size * D + 4 * slot, 4);
            oracle_logit_one(qd, qe, q_scale ? 32 : 8, w + row * w_sr, w_sh, H, D, base + slot * D, ksc,
                             &out[r * max_model_len + n], &bound[r * max_model_len + n]);
        }
        free(qd);
        free(qe);
    }
}

/*
 * Request-local top-k indices -> global cache slots, token by token and column
 * by column as the reference test's loop walks them (test :78-98): local
 * l >= 0 maps to block_table[req][l / bs] * bs + l % bs (int32 with
 * wrap-around, like the reference's Triton arithmetic), l < 0 to -1; the
 * length counts l >= 0, or is 0 for a token marked invalid (valid NULL: all
 * valid).  A block outside the table ([num_reqs][bpr], row stride bt_stride)
 * gives -1 and still counts.
 */
void oracle_compute_global_topk_indices(const int32_t* local, int64_t ls0, int64_t ls1, int64_t T, int64_t K,
                                        const int32_t* req, const int32_t* bt, int64_t bt_stride, int64_t num_reqs,
                                        int64_t bpr, int64_t bs, const int32_t* valid, int32_t* out, int64_t os0,
                                        int64_t os1, int32_t* lens)
{
    const int64_t span = (num_reqs > 0 && bpr > 0) ? (num_reqs - 1) * bt_stride + bpr : 0;
    for (int64_t t = 0; t < T; ++t) {
        int32_t count = 0;
        for (int64_t i = 0; i < K; ++i) {
            const int32_t l = local[t * ls0 + i * ls1];
            int32_t slot = -1;
            if (l >= 0) {
                ++count;
                const int64_t blk = l / bs, off = l % bs;
                const int64_t f = (int64_t)req[t] * bt_stride + blk;
                if (f >= 0 && f < span)
                    slot = (int32_t)((uint32_t)bt[f] * (uint32_t)bs + (uint32_t)off);
            }
            out[t * os0 + i * os1] = slot;
        }
        lens[t] = (!valid || valid[t] != 0) ? count : 0;
    }
}

/*
 * Top-k plus sliding-window index rows, request by request and token by
 * token as the reference test's loop builds them (test :119-141): the row is
 * [topk_indices[t, :topk_len] + M*b, the swa_len window rows, -1 ...] over
 * `width` columns, lens[t] = topk_len + swa_len, with
 * topk_len = min((pos + 1) / ratio, topk) (truncating division, as Triton
 * divides int32) and swa_len = min(pos + 1, window).  Rows of tokens outside
 * every request are not written.
 */
void oracle_combine_topk_swa_indices(const int32_t* topk_idx, int64_t ts0, int64_t ts1, int64_t num_tokens,
                                     const int32_t* qsl, const int32_t* seq_lens, const int32_t* gather_lens,
                                     int64_t num_reqs, int64_t window, int64_t ratio, int64_t topk, int64_t M,
                                     int64_t N, int32_t* out, int64_t os0, int64_t os1, int64_t width, int32_t* lens)
{
    for (int64_t b = 0; b < num_reqs; ++b) {
        const int64_t start = (int64_t)qsl[b] - qsl[0], end = (int64_t)qsl[b + 1] - qsl[0];
        const int64_t seq = seq_lens[b];
        const int64_t start_pos = seq - (end - start), gather_start = seq - gather_lens[b];
        const uint32_t row_off = (uint32_t)((int32_t)M * (int32_t)b);
        for (int64_t t = start; t < end; ++t) {
            if (t < 0 || t >= num_tokens)  /* rows outside the tensors are not touched */
                continue;
            const int32_t pos = (int32_t)(start_pos + (t - start));
            int32_t topk_len = (pos + 1) / (int32_t)ratio;
            if (topk_len > topk)
                topk_len = (int32_t)topk;
            const int32_t swa_len = pos + 1 < window ? pos + 1 : (int32_t)window;
            for (int64_t c = 0; c < width; ++c)
                out[t * os0 + c * os1] = -1;
            for (int32_t j = 0; j < topk_len; ++j)
                out[t * os0 + j * os1] = (int32_t)((uint32_t)topk_idx[t * ts0 + j * ts1] + row_off);
            for (int32_t j = 0; j < swa_len; ++j)
                out[t * os0 + (topk_len + j) * os1] =
                    (int32_t)(row_off + (uint32_t)(int32_t)N + (uint32_t)(j + pos - swa_len + 1 - (int32_t)gather_start));
            lens[t] = topk_len + swa_len;
        }
    }
}

/*
 * Top-k per row by sorting: each candidate (value, index) of the row is sorted
 * by value, largest first, equal values lowest index first (NaN above +inf,
 * as torch.topk orders it); the first k indices, relative to the row's start,
 * are written in ascending order.  A row of at most k values gives
 * 0..len-1 then -1.  Row r holds [starts[r], ends[r]) (prefill, starts
 * non-NULL) or [0, seq_lens[r / next_n] - next_n + r % next_n + 1) (decode),
 * clamped to [0, width).  out is [num_rows][k] contiguous.
 */
struct topk_item {
    float v;
    int32_t i;
};

static int topk_before(const struct topk_item* a, const struct topk_item* b)
{
    const int an = a->v != a->v, bn = b->v != b->v;
    if (an != bn)
        return an;  /* NaN first */
    if (!an && a->v != b->v)
        return a->v > b->v;
    return a->i < b->i;
}

static int topk_cmp(const void* pa, const void* pb)
{
    const struct topk_item* a = (const struct topk_item*)pa;
    const struct topk_item* b = (const struct topk_item*)pb;
    return topk_before(a, b) ? -1 : (topk_before(b, a) ? 1 : 0);
}

static int int_cmp(const void* pa, const void* pb)
{
    const int32_t a = *(const int32_t*)pa, b = *(const int32_t*)pb;
    return (a > b) - (a < b);
}

void oracle_top_k_per_row(const float* logits, int64_t s0, int64_t s1, int64_t num_rows, int64_t width,
                          const int32_t* starts, const int32_t* ends, const int32_t* seq_lens, int64_t next_n,
                          int64_t k, int32_t* out)
{
#pragma omp parallel for schedule(dynamic)
    for (int64_t r = 0; r < num_rows; ++r) {
        int64_t start = 0, end;
        if (starts) {
            start = starts[r];
            end = ends[r];
        } else {
            end = (int64_t)seq_lens[r / next_n] - next_n + r % next_n + 1;
        }
        if (start < 0)
            start = 0;
        if (end > width)
            end = width;
        const int64_t len = end > start ? end - start : 0;
        int32_t* o = out + r * k;
        if (len <= k) {
            for (int64_t i = 0; i < k; ++i)
                o[i] = i < len ? (int32_t)i : -1;
            continue;
        }
        struct topk_item* it = (struct topk_item*)malloc(sizeof(struct topk_item) * (size_t)len);
        if (!it)
            continue;
        for (int64_t i = 0; i < len; ++i) {
            it[i].v = logits[r * s0 + (start + i) * s1];
            it[i].i = (int32_t)i;
        }
        qsort(it, (size_t)len, sizeof(*it), topk_cmp);
        for (int64_t i = 0; i < k; ++i)
            o[i] = it[i].i;
        qsort(o, (size_t)k, sizeof(int32_t), int_cmp);
        free(it);
    }
}

/* ------------------------------------------------------------------------
 * Block-scaled FP8 einsum 'bhr,hdr->bhd' (reference fp8_einsum):
 *   out[b,h,d] = sum_kb s_kb P_kb,  s_kb = xs[b,h,kb] ys[h,d/128,kb],
 *   P_kb = sum_{r in block kb} e4m3(x[b,h,r]) e4m3(y[h,d,r])
 * in binary64.  Each P_kb is exact (products of two e4m3 values span
 * 2^-18..2^17.6, so 128 of them sum exactly in 53 bits) and so is s_kb (two
 * binary32 factors); only the sum over blocks rounds (2^-53 relative).
 *
 * bound[] receives an error bound for an implementation whose block sums
 * come from a matrix instruction that adds the 128 products in groups of 8
 * consecutive K, each product truncated toward zero to a multiple of
 * 2^(E_g - 13), E_g the group's largest exponent sum e(x) + e(y) (e = the
 * unbiased exponent, -6 for zero and subnormal codes), the group sums then
 * added in binary32 (at most 16 roundings of 2^-23); that rounds s_kb to
 * binary32 and accumulates the blocks with one rounding of 2^-24 each:
 *   sum_kb |s_kb| (T_kb + (2^-19 + (nkb + 3) 2^-24) (A_kb + T_kb)),
 *   T_kb = sum_g 8 2^(E_g - 13),  A_kb = sum_r |x y|,
 * before any rounding to the output type.  (The 16x16x128 FP8 MFMA of
 * gfx950 behaves so: tests/test_fp8_einsum.py pins the groups, the window
 * and the truncation with crafted sums.)  Tensors are contiguous:
 * x [B][H][R] codes, xs [B][H][R/128], y [H][D][R] codes, ys [H][D/128][R/128];
 * out and bound [B][H][D].
 * ------------------------------------------------------------------------ */
void oracle_fp8_einsum(const uint8_t* x, const float* xs, const uint8_t* y, const float* ys, int64_t B, int64_t H,
                       int64_t R, int64_t D, double* out, double* bound)
{
    const int64_t nkb = R / 128;
    const double c = ldexp(1.0, -19) + (double)(nkb + 3) * ldexp(1.0, -24);
    double lut[256];
    int ex[256];
    for (int i = 0; i < 256; ++i) {
        lut[i] = (double)oracle_e4m3fn_to_f32((uint8_t)i);
        ex[i] = oracle_e4m3_exp((uint8_t)i);
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h) {
            const uint8_t* xr = x + (b * H + h) * R;
            for (int64_t d = 0; d < D; ++d) {
                const uint8_t* yr = y + (h * D + d) * R;
                double sum = 0.0, err = 0.0;
                for (int64_t kb = 0; kb < nkb; ++kb) {
                    double p = 0.0, a = 0.0, tr = 0.0;
                    for (int64_t g0 = kb * 128; g0 < kb * 128 + 128; g0 += 8) {
                        int eg = -12;
                        for (int64_t i = g0; i < g0 + 8; ++i) {
                            const double t = lut[xr[i]] * lut[yr[i]];
                            p += t;
                            a += fabs(t);
                            const int e = ex[xr[i]] + ex[yr[i]];
                            eg = e > eg ? e : eg;
                        }
                        tr += 8.0 * ldexp(1.0, eg - 13);
                    }
                    const double s = (double)xs[(b * H + h) * nkb + kb] * (double)ys[(h * (D / 128) + d / 128) * nkb + kb];
                    sum += s * p;
                    err += fabs(s) * (tr + c * (a + tr));
                }
                out[(b * H + h) * D + d] = sum;
                bound[(b * H + h) * D + d] = err;
            }
        }
}
