/*
 * sp_oracle.h — CPU restatement of the reference's ragged-batch attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (sketchpad_amd/, include/) links or calls
 * this code. It is used by tests/ as the checker, by __graft_entry__.smoke() as the checker and
 * by bench.py's cpu_baseline leg as the timed CPU port of the reference's op sequence.
 *
 * Every function restates a reference item (file:line under rhi-zone/sketchpad) and states how
 * it is pinned (see the test named after it):
 *   spo_get_block / spo_get_slot / spo_needs_new_block    paged_attention.rs:124-137
 *       pinned: the reference's test_block_table known answers (paged_attention.rs:568-598)
 *   spo_blocks_needed                                     paged_attention.rs:403-404, :504-505
 *       pinned: test_paged_scheduler counts (3 tokens -> 1 block, 5 -> 2; :623-645)
 *   spo_blocks_from_memory_budget                         paged_attention.rs:67-85
 *       pinned: test_config_from_memory_budget (1 GiB -> 256 blocks; :648-661)
 *   spo_store_kv / spo_slot_mapping                       paged_attention.rs:230-310
 *       pinned: gather(store(x)) == x, untouched slots stay zero, closed-form addresses,
 *               and the numpy restatement (oracle/np_oracle.py)
 *   spo_gather_kv                                         paged_attention.rs:313-378
 *       pinned: empty gather (test_gather_kv_empty, :664-674) + round trip + concat-cache
 *               equivalence (KvCache::update, kv_cache.rs:108-130)
 *   spo_causal_mask / spo_sliding_window_mask             transformer.rs:415-451
 *       pinned: test_causal_mask and test_sliding_window_mask entries (transformer.rs:524-561)
 *   spo_prefill_causal_mask                               llama.rs:374-388
 *   spo_sliding_window_prefill_mask                       gemma4.rs:1086-1108
 *       pinned: reduce to causal_mask when new_len == total_len; brute-force predicate checks
 *   spo_attention_f64                                     transformer.rs:227-243 (+ repeat_kv :257-271)
 *       pinned: torch.nn.functional.scaled_dot_product_attention in float64 (a library
 *               routine), closed forms (one key -> v; equal keys -> mean(v); dominant key -> its v),
 *               GQA == repeated-head MHA, mask-rule == explicit additive mask
 *   spo_attention_f64_cap                                 + the logit soft cap, gemma4.rs:366-377
 *       pinned: the two-key closed form p1 = 1 / (1 + exp(c tanh(l2/c) - c tanh(l1/c))) with
 *               math.tanh, saturation (logits far past +-c weigh as e^{+-c}), a cap far above
 *               the logits equal to no cap, and the cap applied before the window mask
 *   spo_attention_f32_refops                              transformer.rs:234-243 op order in f32
 *       pinned: within f32 rounding of spo_attention_f64 on every test case
 *   spo_rope_caches                                       rope.rs:60-102 (with_base + repeat_interleave)
 *       pinned: position 0 -> (1, 0) exactly, pair 0 -> (cos p, sin p) within 1 ulp of the
 *               float64 values, every entry within a few ulp of float64 cos / sin of p / base^(2i/d),
 *               duplicated entries equal
 *   spo_rope_apply                                        rope.rs:136-170 (apply_rotary, rotate_half)
 *       pinned: the reference's rope tests (zeros stay zeros, ones change, position 0 is the
 *               identity; rope.rs:180-230), complex multiplication (x0 + i x1) e^{i angle} in
 *               float64, pair norms preserved, rotating back by -angle restores x, and
 *               <R(m) q, R(n) k> depends only on m - n (float64)
 *   spo_f32_to_f16_bits / spo_f16_bits_to_f32             f16::from_f32 / to_f32 (kv_cache.rs:449, :496)
 *       pinned: numpy's float16 conversion (a library routine) on every binary16 value and on
 *               ties, overflow, subnormal and NaN inputs
 *   spo_polar_compress / spo_polar_decompress             kv_cache.rs:437-532 (PolarQuant)
 *   spo_polar_record_bytes / spo_polar_compression_ratio  kv_cache.rs:441-443, :315-318
 *   spo_qjl_lcg_normal / spo_qjl_projection               kv_cache.rs:373-396, :417-424 (QJL)
 *   spo_qjl_compress / spo_qjl_decompress                 kv_cache.rs:534-617
 *   spo_qjl_record_bytes / spo_qjl_compression_ratio      kv_cache.rs:536-540, :319-321
 *       pinned: hand-derived records (one-hot, negative, zero, odd head_dim, a half-way code that
 *               f32::round takes away from zero), decompress(compress(x)) within the closed-form
 *               bound |x_j - x'_j| <= |x|/14 + (f16 rounding of |x|), codes = sign-correct
 *               rounded 7 x_j/|x| (float64 brute force away from ties), record size against
 *               compression_ratio for even head_dim (the reference test's QJL ratio at :871-876
 *               pins the same formula's shape), NaN / infinity / zero rows
 *   spo_cpu_decode_baseline / spo_cpu_prefill_baseline    the reference's whole decode / prefill
 *       op sequence (store, gather+concat, repeat_kv, matmul, scale, mask, softmax, matmul), f32,
 *       OpenMP over sequences; the prefill's two products run on a packed 6x16 AVX2/FMA GEMM
 *       (burn-ndarray's matmul is the matrixmultiply crate's packed sgemm), the decode's are
 *       matrix-vector products (bandwidth-bound); pinned against spo_attention_f64.
 */
#ifndef SP_ORACLE_H
#define SP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order as sp_cache_layout (include/sketchpad_attn.h). */
typedef struct spo_layout {
  int32_t num_blocks, num_layers, layer, num_kv_heads, block_size, head_dim;
} spo_layout;

/* element types of the tensors handed to the oracle */
enum { SPO_F32 = 0, SPO_BF16 = 1, SPO_F16 = 2 };

int64_t spo_get_block(const int32_t* table, int64_t num_table_blocks, int64_t pos, int block_size);
int64_t spo_get_slot(int64_t pos, int block_size);
int spo_needs_new_block(int64_t seq_len, int block_size);
int64_t spo_blocks_needed(int64_t new_len, int block_size);
int64_t spo_blocks_from_memory_budget(int64_t memory_bytes, int64_t num_kv_heads, int64_t head_dim,
                                      int64_t num_layers, int64_t block_size);

int spo_slot_mapping(const int32_t* table, int64_t num_table_blocks, int64_t start_pos,
                     int64_t count, int block_size, int32_t* out);
int spo_store_kv(void* k_pool, void* v_pool, const spo_layout* layout, const int32_t* table,
                 int64_t num_table_blocks, const void* k, const void* v, int64_t seq_len,
                 int64_t start_pos, int elem_size);
int spo_gather_kv(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                  const spo_layout* layout, const int32_t* table, int64_t num_table_blocks,
                  int64_t seq_len, int elem_size);

void spo_causal_mask(int64_t n, float* out);
void spo_prefill_causal_mask(int64_t new_len, int64_t total_len, float* out);
void spo_sliding_window_mask(int64_t n, int64_t window, float* out);
void spo_sliding_window_prefill_mask(int64_t new_len, int64_t total_len, int64_t window,
                                     float* out);

/*
 * Attention of one sequence. q element (i, h, d) is at q[i*q_tok + h*q_head + d]; k/v (j, g, d)
 * at [j*kv_tok + g*kv_head + d]. Query head h reads KV head h / (Hq / Hkv). Key j is visible to
 * query i when mask == NULL and
 *   (!causal || j <= q_pos0 + i) && (window_left < 0 || j >= q_pos0 + i - window_left)
 * or, with an explicit mask, the additive mask[i*Lk + j] is added to the scaled score.
 * out is [Sq, Hq, D] (double for _f64, float for _f32_refops). A row with no visible key is 0.
 */
void spo_attention_f64(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                       const void* v, int64_t kv_tok, int64_t kv_head, int64_t sq, int64_t lk,
                       int hq, int hkv, int d, double scale, const float* mask, int causal,
                       int64_t q_pos0, int64_t window_left, int dtype, double* out);
/* spo_attention_f64 with V of its own head dim dv and strides (out [sq][hq][dv]): the value
 * head dim of flash_attention (sketchpad-cubecl attention.rs:135-143). */
void spo_attention_f64_v(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                         int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                         int64_t v_head, int dv, int64_t sq, int64_t lk, int hq, int hkv, int d,
                         double scale, const float* mask, int causal, int64_t q_pos0,
                         int64_t window_left, int dtype, double* out);
/* spo_attention_f64_v with Gemma-4's logit soft cap: every scaled logit x becomes
 * softcap * tanh(x / softcap) before the mask (gemma4.rs:366-377); softcap <= 0: none. */
void spo_attention_f64_cap(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                           int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                           int64_t v_head, int dv, int64_t sq, int64_t lk, int hq, int hkv,
                           int d, double scale, double softcap, const float* mask, int causal,
                           int64_t q_pos0, int64_t window_left, int dtype, double* out);
void spo_attention_f32_refops(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                              const void* v, int64_t kv_tok, int64_t kv_head, int64_t sq,
                              int64_t lk, int hq, int hkv, int d, float scale, const float* mask,
                              int causal, int64_t q_pos0, int64_t window_left, int dtype,
                              float* out);

/*
 * Timed CPU baseline of one decode step in the reference's op order, OpenMP over sequences.
 * For each sequence s: store the new token's k/v ([Hkv, D] at position L_s-1) into the pools,
 * gather [Hkv, L_s, D], materialise repeat_kv, scores = (q k^T) * scale, softmax, out = p v.
 * Pools are f32 (the reference's NdArray<f32>); q/k_new/v_new are f32. out is [B, Hq, D].
 */
void spo_cpu_decode_baseline(float* out, const float* q, const float* k_new, const float* v_new,
                             float* k_pool, float* v_pool, const spo_layout* layout,
                             const int32_t* block_tables, int64_t max_blocks_per_seq,
                             const int32_t* context_lens, int64_t num_seqs, int hq, float scale,
                             int64_t window_left, int threads);

/*
 * Timed CPU baseline of causal prefill over packed sequences in the reference's op order:
 * per sequence, repeat_kv, [Hq, L, L] f32 scores, scale, + causal mask, softmax, matmul; both
 * products in full (as the reference computes them) on a packed AVX2/FMA GEMM.
 * q [T, Hq, D], k/v [T, Hkv, D] f32, cu_seqlens [num_seqs+1]; out [T, Hq, D].
 */
void spo_cpu_prefill_baseline(float* out, const float* q, const float* k, const float* v,
                              const int32_t* cu_seqlens, int64_t num_seqs, int hq, int hkv,
                              int d, float scale, int threads);

void spo_rope_caches(float* cos_full, float* sin_full, int64_t rows, int64_t head_dim, float base);
int spo_rope_apply(float* x, int64_t tokens, int64_t heads, int64_t head_dim, int64_t tok_stride,
                   int64_t head_stride, const int32_t* positions, const float* cos_full,
                   const float* sin_full, int64_t rows);

uint16_t spo_f32_to_f16_bits(float f);
float spo_f16_bits_to_f32(uint16_t h);
int64_t spo_polar_record_bytes(int64_t head_dim);
void spo_polar_compress(uint8_t* out, const float* x, int64_t num_vecs, int64_t head_dim);
void spo_polar_decompress(float* out, const uint8_t* bytes, int64_t num_vecs, int64_t head_dim);
double spo_polar_compression_ratio(int64_t head_dim);
void spo_qjl_lcg_normal(float* out, int64_t count, float scale);
void spo_qjl_projection(float* out, int64_t proj_dim, int64_t head_dim);
int64_t spo_qjl_record_bytes(int64_t proj_dim);
void spo_qjl_compress(uint8_t* out, const float* x, int64_t num_vecs, int64_t head_dim,
                      const float* proj, int64_t proj_dim);
void spo_qjl_decompress(float* out, const uint8_t* bytes, int64_t num_vecs, int64_t head_dim,
                        const float* proj, int64_t proj_dim);
double spo_qjl_compression_ratio(int64_t proj_dim, int64_t head_dim);

#ifdef __cplusplus
}
#endif

#endif
