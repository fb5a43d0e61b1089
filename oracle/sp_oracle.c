/*
 * sp_oracle.c — CPU restatement of the reference's ragged-batch attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and bench.py's cpu_baseline leg.
 * The product never links it. See sp_oracle.h for the reference file:line each function
 * restates and the check that pins it.
 */
#include "sp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include <immintrin.h>

/* ------------------------------------------------------------------------------------------ */
/* element conversion                                                                          */
/* ------------------------------------------------------------------------------------------ */

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: renormalise */
      exp = 127 - 15 + 1;
      while ((man & 0x400u) == 0) {
        man <<= 1;
        exp--;
      }
      man &= 0x3ffu;
      u = sign | (exp << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float load_elem(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case SPO_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case SPO_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

/* ------------------------------------------------------------------------------------------ */
/* BlockTable / PagedKvCacheConfig arithmetic (paged_attention.rs:67-85, :124-137, :403-404)    */
/* ------------------------------------------------------------------------------------------ */

int64_t spo_get_block(const int32_t* table, int64_t num_table_blocks, int64_t pos,
                      int block_size) {
  const int64_t block_num = pos / block_size; /* paged_attention.rs:125 */
  if (block_num < 0 || block_num >= num_table_blocks) return -1; /* None (:126) */
  return table[block_num];
}

int64_t spo_get_slot(int64_t pos, int block_size) { return pos % block_size; /* :131 */ }

int spo_needs_new_block(int64_t seq_len, int block_size) {
  return seq_len > 0 && seq_len % block_size == 0; /* :136 */
}

int64_t spo_blocks_needed(int64_t new_len, int block_size) {
  return (new_len + block_size - 1) / block_size; /* div_ceil, :404 */
}

int64_t spo_blocks_from_memory_budget(int64_t memory_bytes, int64_t num_kv_heads,
                                      int64_t head_dim, int64_t num_layers, int64_t block_size) {
  /* 2 (K+V) * layers * heads * head_dim * block_size * 4 bytes (f32), :75-76 */
  const int64_t per_block = 2 * num_layers * num_kv_heads * head_dim * block_size * 4;
  return per_block > 0 ? memory_bytes / per_block : 0;
}

/* ------------------------------------------------------------------------------------------ */
/* store_kv / gather_kv (paged_attention.rs:230-378)                                            */
/* ------------------------------------------------------------------------------------------ */

int spo_slot_mapping(const int32_t* table, int64_t num_table_blocks, int64_t start_pos,
                     int64_t count, int block_size, int32_t* out) {
  for (int64_t i = 0; i < count; ++i) {
    const int64_t pos = start_pos + i;
    const int64_t blk = spo_get_block(table, num_table_blocks, pos, block_size);
    if (blk < 0) return -1; /* "Block not allocated", :242 */
    out[i] = (int32_t)(blk * block_size + spo_get_slot(pos, block_size));
  }
  return 0;
}

static int64_t pool_offset(const spo_layout* l, int64_t blk, int64_t head, int64_t slot) {
  /* [num_blocks][num_layers][Hkv][BS][D] element offset of row (blk, layer, head, slot) */
  return (((blk * l->num_layers + l->layer) * l->num_kv_heads + head) * l->block_size + slot) *
         l->head_dim;
}

int spo_store_kv(void* k_pool, void* v_pool, const spo_layout* l, const int32_t* table,
                 int64_t num_table_blocks, const void* k, const void* v, int64_t seq_len,
                 int64_t start_pos, int elem_size) {
  const int64_t row = (int64_t)l->head_dim * elem_size;
  for (int64_t i = 0; i < seq_len; ++i) { /* :240 */
    const int64_t pos = start_pos + i;
    const int64_t blk = spo_get_block(table, num_table_blocks, pos, l->block_size);
    if (blk < 0 || blk >= l->num_blocks) return -1; /* panic "Block not allocated" */
    const int64_t slot = spo_get_slot(pos, l->block_size);
    for (int64_t h = 0; h < l->num_kv_heads; ++h) {
      /* k is [Hkv, seq_len, D] (:234); cache[blk, layer, h, slot, :] = k[h, i, :] (:289-298) */
      const int64_t src = (h * seq_len + i) * row;
      const int64_t dst = pool_offset(l, blk, h, slot) * elem_size;
      memcpy((char*)k_pool + dst, (const char*)k + src, (size_t)row);
      memcpy((char*)v_pool + dst, (const char*)v + src, (size_t)row);
    }
  }
  return 0;
}

int spo_gather_kv(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                  const spo_layout* l, const int32_t* table, int64_t num_table_blocks,
                  int64_t seq_len, int elem_size) {
  if (seq_len == 0) return 0; /* [Hkv, 0, D], :322-327 */
  if (spo_blocks_needed(seq_len, l->block_size) > num_table_blocks) return -1;
  const int64_t row = (int64_t)l->head_dim * elem_size;
  for (int64_t b = 0; b < num_table_blocks; ++b) { /* :333 */
    const int64_t start = b * l->block_size;
    if (start >= seq_len) break;
    int64_t end = start + l->block_size;
    if (end > seq_len) end = seq_len; /* :335 */
    const int64_t blk = table[b];
    if (blk < 0 || blk >= l->num_blocks) return -1;
    for (int64_t h = 0; h < l->num_kv_heads; ++h) {
      for (int64_t t = start; t < end; ++t) { /* slice + reshape + cat along seq (:340-375) */
        const int64_t src = pool_offset(l, blk, h, t - start) * elem_size;
        const int64_t dst = (h * seq_len + t) * row;
        memcpy((char*)k_out + dst, (const char*)k_pool + src, (size_t)row);
        memcpy((char*)v_out + dst, (const char*)v_pool + src, (size_t)row);
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* masks                                                                                       */
/* ------------------------------------------------------------------------------------------ */

void spo_causal_mask(int64_t n, float* out) { /* transformer.rs:415-424 */
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < n; ++j) out[i * n + j] = j > i ? -INFINITY : 0.f;
}

void spo_prefill_causal_mask(int64_t new_len, int64_t total_len, float* out) {
  const int64_t start = total_len - new_len; /* llama.rs:379 */
  for (int64_t i = 0; i < new_len; ++i)
    for (int64_t j = 0; j < total_len; ++j) out[i * total_len + j] = j > start + i ? -INFINITY : 0.f;
}

void spo_sliding_window_mask(int64_t n, int64_t window, float* out) { /* transformer.rs:436-451 */
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < n; ++j)
      out[i * n + j] = (j > i || i > j + window) ? -INFINITY : 0.f; /* :445 */
}

void spo_sliding_window_prefill_mask(int64_t new_len, int64_t total_len, int64_t window,
                                     float* out) { /* gemma4.rs:1086-1108 */
  const int64_t start = total_len - new_len;
  for (int64_t i = 0; i < new_len; ++i) {
    const int64_t p = start + i;
    for (int64_t j = 0; j < total_len; ++j) {
      float m = 0.f;
      if (j > p) m = -INFINITY;
      if (p >= window && j < p - window + 1) m = -INFINITY; /* :1102 */
      out[i * total_len + j] = m;
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* attention                                                                                   */
/* ------------------------------------------------------------------------------------------ */

static int visible(int causal, int64_t q_pos0, int64_t window_left, int64_t i, int64_t j) {
  const int64_t p = q_pos0 + i;
  if (causal && j > p) return 0;
  if (window_left >= 0 && j < p - window_left) return 0;
  return 1;
}

void spo_attention_f64(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                       const void* v, int64_t kv_tok, int64_t kv_head, int64_t sq, int64_t lk,
                       int hq, int hkv, int d, double scale, const float* mask, int causal,
                       int64_t q_pos0, int64_t window_left, int dtype, double* out) {
  spo_attention_f64_v(q, q_tok, q_head, k, kv_tok, kv_head, v, kv_tok, kv_head, d, sq, lk, hq,
                      hkv, d, scale, mask, causal, q_pos0, window_left, dtype, out);
}

void spo_attention_f64_v(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                         int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                         int64_t v_head, int dv, int64_t sq, int64_t lk, int hq, int hkv, int d,
                         double scale, const float* mask, int causal, int64_t q_pos0,
                         int64_t window_left, int dtype, double* out) {
  spo_attention_f64_cap(q, q_tok, q_head, k, k_tok, k_head, v, v_tok, v_head, dv, sq, lk, hq,
                        hkv, d, scale, 0.0, mask, causal, q_pos0, window_left, dtype, out);
}

void spo_attention_f64_cap(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                           int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                           int64_t v_head, int dv, int64_t sq, int64_t lk, int hq, int hkv,
                           int d, double scale, double softcap, const float* mask, int causal,
                           int64_t q_pos0, int64_t window_left, int dtype, double* out) {
  const int rep = hq / hkv; /* repeat_kv: head h reads KV head h / rep (transformer.rs:263-270) */
  /* Work items are (head, block of 64 query rows), spread over OpenMP threads. Each output row
   * is still one sequential sum over the keys in ascending order, so the thread count does not
   * change any result. Without an additive mask, keys the causal / window predicate hides are
   * skipped: they would enter as exp(-inf) = 0 and change neither the maximum nor the sums. */
  const int64_t rb = 64, nrb = (sq + rb - 1) / rb;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)(lk > 0 ? lk : 1));
    double* kd = (double*)malloc(sizeof(double) * (size_t)(lk > 0 ? lk : 1) * (size_t)d);
    double* vd = (double*)malloc(sizeof(double) * (size_t)(lk > 0 ? lk : 1) * (size_t)dv);
    double* qd = (double*)malloc(sizeof(double) * (size_t)d);
    int g_have = -1;
#pragma omp for schedule(dynamic, 1)
    for (int64_t item = 0; item < (int64_t)hq * nrb; ++item) {
      const int h = (int)(item / nrb);
      const int64_t i0 = (item % nrb) * rb, i1 = i0 + rb < sq ? i0 + rb : sq;
      const int g = h / rep;
      if (g != g_have) { /* this KV head's rows, converted once per thread */
        for (int64_t j = 0; j < lk; ++j) {
          for (int c = 0; c < d; ++c)
            kd[j * d + c] = (double)load_elem(k, j * k_tok + g * k_head + c, dtype);
          for (int c = 0; c < dv; ++c)
            vd[j * dv + c] = (double)load_elem(v, j * v_tok + g * v_head + c, dtype);
        }
        g_have = g;
      }
      for (int64_t i = i0; i < i1; ++i) {
        for (int c = 0; c < d; ++c) qd[c] = (double)load_elem(q, i * q_tok + h * q_head + c, dtype);
        int64_t jlo = 0, jhi = lk; /* keys [jlo, jhi) can be visible */
        if (!mask) {
          const int64_t p = q_pos0 + i;
          if (causal && p + 1 < jhi) jhi = p + 1 > 0 ? p + 1 : 0;
          if (window_left >= 0 && p - window_left > jlo) jlo = p - window_left;
          if (jlo > jhi) jlo = jhi;
        }
        double m = -INFINITY;
        for (int64_t j = jlo; j < jhi; ++j) {
          double acc = 0.0;
          for (int c = 0; c < d; ++c) acc += qd[c] * kd[j * d + c];
          acc *= scale; /* scale after the product (transformer.rs:234-235) */
          /* Gemma-4's logit soft cap, on the scaled logits and before the mask
           * (gemma4.rs:366-377) */
          if (softcap > 0.0) acc = softcap * tanh(acc / softcap);
          if (mask)
            acc += (double)mask[i * lk + j];
          else if (!visible(causal, q_pos0, window_left, i, j))
            acc = -INFINITY;
          s[j] = acc;
          if (acc > m) m = acc;
        }
        double* o = out + (i * hq + h) * dv;
        for (int c = 0; c < dv; ++c) o[c] = 0.0;
        if (m == -INFINITY) continue; /* no visible key (or no keys): zeros */
        double sum = 0.0;
        for (int64_t j = jlo; j < jhi; ++j) {
          s[j] = exp(s[j] - m); /* softmax(dim 3), max-subtracted (transformer.rs:242) */
          sum += s[j];
        }
        for (int64_t j = jlo; j < jhi; ++j) {
          if (s[j] == 0.0) continue;
          const double pj = s[j] / sum;
          for (int c = 0; c < dv; ++c) o[c] += pj * vd[j * dv + c];
        }
      }
    }
    free(s);
    free(kd);
    free(vd);
    free(qd);
  }
}

void spo_attention_f32_refops(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                              const void* v, int64_t kv_tok, int64_t kv_head, int64_t sq,
                              int64_t lk, int hq, int hkv, int d, float scale, const float* mask,
                              int causal, int64_t q_pos0, int64_t window_left, int dtype,
                              float* out) {
  const int rep = hq / hkv;
  const int64_t lk1 = lk > 0 ? lk : 1;
  float* s = (float*)malloc(sizeof(float) * (size_t)lk1);
  float* kr = (float*)malloc(sizeof(float) * (size_t)(lk1 * d)); /* repeat_kv copy, per head */
  float* vr = (float*)malloc(sizeof(float) * (size_t)(lk1 * d));
  for (int h = 0; h < hq; ++h) {
    const int g = h / rep;
    for (int64_t j = 0; j < lk; ++j)
      for (int c = 0; c < d; ++c) {
        kr[j * d + c] = load_elem(k, j * kv_tok + g * kv_head + c, dtype);
        vr[j * d + c] = load_elem(v, j * kv_tok + g * kv_head + c, dtype);
      }
    for (int64_t i = 0; i < sq; ++i) {
      float m = -INFINITY;
      for (int64_t j = 0; j < lk; ++j) {
        float acc = 0.f; /* q.matmul(k^T) */
        for (int c = 0; c < d; ++c) acc += load_elem(q, i * q_tok + h * q_head + c, dtype) * kr[j * d + c];
        acc = acc * scale; /* * scale */
        if (mask)
          acc = acc + mask[i * lk + j]; /* + mask */
        else if (!visible(causal, q_pos0, window_left, i, j))
          acc = -INFINITY;
        s[j] = acc;
        if (acc > m) m = acc;
      }
      float* o = out + (i * hq + h) * d;
      for (int c = 0; c < d; ++c) o[c] = 0.f;
      if (m == -INFINITY) continue;
      float sum = 0.f; /* softmax: exp(x - max) / sum */
      for (int64_t j = 0; j < lk; ++j) {
        s[j] = expf(s[j] - m);
        sum += s[j];
      }
      for (int64_t j = 0; j < lk; ++j) s[j] = s[j] / sum;
      for (int64_t j = 0; j < lk; ++j) /* attn.matmul(v) */
        for (int c = 0; c < d; ++c) o[c] += s[j] * vr[j * d + c];
    }
  }
  free(s);
  free(kr);
  free(vr);
}

/* ------------------------------------------------------------------------------------------ */
/* timed CPU baselines (the reference's op sequence, f32, OpenMP)                              */
/* ------------------------------------------------------------------------------------------ */

static float dot_f32(const float* a, const float* b, int n) {
  float acc = 0.f;
#pragma omp simd reduction(+ : acc)
  for (int c = 0; c < n; ++c) acc += a[c] * b[c];
  return acc;
}

/* softmax over row[0..n), in place, max-subtracted; returns 0 when every entry is -inf */
static int softmax_row(float* row, int64_t n) {
  float m = -INFINITY;
  for (int64_t j = 0; j < n; ++j) m = row[j] > m ? row[j] : m;
  if (m == -INFINITY) return 0;
  float sum = 0.f;
  for (int64_t j = 0; j < n; ++j) {
    row[j] = expf(row[j] - m);
    sum += row[j];
  }
  const float inv = 1.f / sum;
  for (int64_t j = 0; j < n; ++j) row[j] *= inv;
  return 1;
}

void spo_cpu_decode_baseline(float* out, const float* q, const float* k_new, const float* v_new,
                             float* k_pool, float* v_pool, const spo_layout* l,
                             const int32_t* block_tables, int64_t max_blocks_per_seq,
                             const int32_t* context_lens, int64_t num_seqs, int hq, float scale,
                             int64_t window_left, int threads) {
  const int hkv = l->num_kv_heads, d = l->head_dim;
  const int rep = hq / hkv;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t s = 0; s < num_seqs; ++s) {
    const int64_t len = context_lens[s];
    const int32_t* table = block_tables + s * max_blocks_per_seq;
    float* o = out + s * hq * d;
    if (len <= 0) {
      memset(o, 0, sizeof(float) * (size_t)hq * d);
      continue;
    }
    /* 1. store the new token at position len-1 (store_kv, per head) */
    spo_store_kv(k_pool, v_pool, l, table, max_blocks_per_seq, k_new + s * hkv * d,
                 v_new + s * hkv * d, 1, len - 1, 4);
    /* 2. gather: per-block slices concatenated into [Hkv, len, D] */
    float* kg = (float*)malloc(sizeof(float) * (size_t)(hkv * len * d));
    float* vg = (float*)malloc(sizeof(float) * (size_t)(hkv * len * d));
    spo_gather_kv(kg, vg, k_pool, v_pool, l, table, max_blocks_per_seq, len, 4);
    /* 3. repeat_kv materialised: [Hq, len, D] */
    float* kr = (float*)malloc(sizeof(float) * (size_t)(hq * len * d));
    float* vr = (float*)malloc(sizeof(float) * (size_t)(hq * len * d));
    for (int h = 0; h < hq; ++h) {
      memcpy(kr + (int64_t)h * len * d, kg + (int64_t)(h / rep) * len * d, sizeof(float) * (size_t)(len * d));
      memcpy(vr + (int64_t)h * len * d, vg + (int64_t)(h / rep) * len * d, sizeof(float) * (size_t)(len * d));
    }
    /* 4. scores = (q k^T) * scale (+ window mask), softmax, out = p v */
    float* sc = (float*)malloc(sizeof(float) * (size_t)(hq * len));
    for (int h = 0; h < hq; ++h) {
      const float* qh = q + (s * hq + h) * d;
      float* row = sc + (int64_t)h * len;
      for (int64_t j = 0; j < len; ++j) row[j] = dot_f32(qh, kr + ((int64_t)h * len + j) * d, d) * scale;
      if (window_left >= 0)
        for (int64_t j = 0; j < len; ++j)
          if (j < len - 1 - window_left) row[j] += -INFINITY;
      float* oh = o + h * d;
      for (int c = 0; c < d; ++c) oh[c] = 0.f;
      if (!softmax_row(row, len)) continue;
      for (int64_t j = 0; j < len; ++j) {
        const float pj = row[j];
        const float* vj = vr + ((int64_t)h * len + j) * d;
#pragma omp simd
        for (int c = 0; c < d; ++c) oh[c] += pj * vj[c];
      }
    }
    free(sc);
    free(kr);
    free(vr);
    free(kg);
    free(vg);
  }
}

/* Blocked single-precision GEMM for the prefill baseline: the reference's two matmuls go through
 * burn-ndarray, i.e. the matrixmultiply crate's packed sgemm with AVX2/FMA micro-kernels, so the
 * port uses the same kind of kernel rather than a dot product per output. B is packed into
 * panels of 16 columns (panel p, row kk at bp[(p * k + kk) * 16], zero padded); a 6 x 16 block of
 * C is held in 12 AVX registers while kk runs over the shared dimension. */
#define GEMM_MR 6
#define GEMM_NR 16

/* C[i, j] = alpha * sum_kk A[i, kk] * B[kk, j] over rows [0, m), columns [0, n) */
static void gemm_packed(float* c, int64_t ldc, const float* a, int64_t lda, const float* bp,
                        int64_t m, int64_t n, int64_t k, float alpha) {
  for (int64_t p = 0; p * GEMM_NR < n; ++p) {
    const float* panel = bp + p * k * GEMM_NR;
    const int64_t j0 = p * GEMM_NR, nc = n - j0 < GEMM_NR ? n - j0 : GEMM_NR;
    for (int64_t i0 = 0; i0 < m; i0 += GEMM_MR) {
      const int mr = m - i0 < GEMM_MR ? (int)(m - i0) : GEMM_MR;
      const float* a0 = a + i0 * lda;
      const float* a1 = a + (i0 + (mr > 1 ? 1 : 0)) * lda;
      const float* a2 = a + (i0 + (mr > 2 ? 2 : 0)) * lda;
      const float* a3 = a + (i0 + (mr > 3 ? 3 : 0)) * lda;
      const float* a4 = a + (i0 + (mr > 4 ? 4 : 0)) * lda;
      const float* a5 = a + (i0 + (mr > 5 ? 5 : 0)) * lda;
      __m256 c00 = _mm256_setzero_ps(), c01 = c00, c10 = c00, c11 = c00, c20 = c00, c21 = c00;
      __m256 c30 = c00, c31 = c00, c40 = c00, c41 = c00, c50 = c00, c51 = c00;
      for (int64_t kk = 0; kk < k; ++kk) {
        const __m256 b0 = _mm256_loadu_ps(panel + kk * GEMM_NR);
        const __m256 b1 = _mm256_loadu_ps(panel + kk * GEMM_NR + 8);
        __m256 av = _mm256_broadcast_ss(a0 + kk);
        c00 = _mm256_fmadd_ps(av, b0, c00);
        c01 = _mm256_fmadd_ps(av, b1, c01);
        av = _mm256_broadcast_ss(a1 + kk);
        c10 = _mm256_fmadd_ps(av, b0, c10);
        c11 = _mm256_fmadd_ps(av, b1, c11);
        av = _mm256_broadcast_ss(a2 + kk);
        c20 = _mm256_fmadd_ps(av, b0, c20);
        c21 = _mm256_fmadd_ps(av, b1, c21);
        av = _mm256_broadcast_ss(a3 + kk);
        c30 = _mm256_fmadd_ps(av, b0, c30);
        c31 = _mm256_fmadd_ps(av, b1, c31);
        av = _mm256_broadcast_ss(a4 + kk);
        c40 = _mm256_fmadd_ps(av, b0, c40);
        c41 = _mm256_fmadd_ps(av, b1, c41);
        av = _mm256_broadcast_ss(a5 + kk);
        c50 = _mm256_fmadd_ps(av, b0, c50);
        c51 = _mm256_fmadd_ps(av, b1, c51);
      }
      const __m256 al = _mm256_set1_ps(alpha);
      float tmp[GEMM_MR][GEMM_NR];
      _mm256_storeu_ps(tmp[0], _mm256_mul_ps(c00, al));
      _mm256_storeu_ps(tmp[0] + 8, _mm256_mul_ps(c01, al));
      _mm256_storeu_ps(tmp[1], _mm256_mul_ps(c10, al));
      _mm256_storeu_ps(tmp[1] + 8, _mm256_mul_ps(c11, al));
      _mm256_storeu_ps(tmp[2], _mm256_mul_ps(c20, al));
      _mm256_storeu_ps(tmp[2] + 8, _mm256_mul_ps(c21, al));
      _mm256_storeu_ps(tmp[3], _mm256_mul_ps(c30, al));
      _mm256_storeu_ps(tmp[3] + 8, _mm256_mul_ps(c31, al));
      _mm256_storeu_ps(tmp[4], _mm256_mul_ps(c40, al));
      _mm256_storeu_ps(tmp[4] + 8, _mm256_mul_ps(c41, al));
      _mm256_storeu_ps(tmp[5], _mm256_mul_ps(c50, al));
      _mm256_storeu_ps(tmp[5] + 8, _mm256_mul_ps(c51, al));
      for (int r = 0; r < mr; ++r)
        memcpy(c + (i0 + r) * ldc + j0, tmp[r], sizeof(float) * (size_t)nc);
    }
  }
}

/* pack B = X^T for X [n rows, k cols] (row stride ldx): panel rows are X's columns */
static void pack_transposed(float* bp, const float* x, int64_t ldx, int64_t n, int64_t k) {
  for (int64_t p = 0; p * GEMM_NR < n; ++p)
    for (int64_t kk = 0; kk < k; ++kk)
      for (int c = 0; c < GEMM_NR; ++c) {
        const int64_t j = p * GEMM_NR + c;
        bp[(p * k + kk) * GEMM_NR + c] = j < n ? x[j * ldx + kk] : 0.f;
      }
}

/* pack B = X for X [k rows, n cols] (row stride ldx) */
static void pack_rows(float* bp, const float* x, int64_t ldx, int64_t k, int64_t n) {
  for (int64_t p = 0; p * GEMM_NR < n; ++p)
    for (int64_t kk = 0; kk < k; ++kk)
      for (int c = 0; c < GEMM_NR; ++c) {
        const int64_t j = p * GEMM_NR + c;
        bp[(p * k + kk) * GEMM_NR + c] = j < n ? x[kk * ldx + j] : 0.f;
      }
}

void spo_cpu_prefill_baseline(float* out, const float* q, const float* k, const float* v,
                              const int32_t* cu_seqlens, int64_t num_seqs, int hq, int hkv,
                              int d, float scale, int threads) {
  const int rep = hq / hkv;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t s = 0; s < num_seqs; ++s) {
    for (int h = 0; h < hq; ++h) {
      const int64_t t0 = cu_seqlens[s], len = cu_seqlens[s + 1] - cu_seqlens[s];
      if (len <= 0) continue;
      const int g = h / rep;
      const int64_t lp = (len + GEMM_NR - 1) / GEMM_NR * GEMM_NR;
      const int64_t dp = ((int64_t)d + GEMM_NR - 1) / GEMM_NR * GEMM_NR;
      /* repeat_kv of this head's K/V, packed for the two products: K^T [D, L] and V [L, D] */
      float* kt = (float*)malloc(sizeof(float) * (size_t)(lp * d));
      float* vp = (float*)malloc(sizeof(float) * (size_t)(dp * len));
      pack_transposed(kt, k + (t0 * hkv + g) * d, (int64_t)hkv * d, len, d);
      pack_rows(vp, v + (t0 * hkv + g) * d, (int64_t)hkv * d, len, d);
      /* [L, L] scores = (q k^T) * scale, + causal mask, softmax, then p v: both full products,
       * as the reference computes them */
      float* sc = (float*)malloc(sizeof(float) * (size_t)(len * len));
      gemm_packed(sc, len, q + (t0 * hq + h) * d, (int64_t)hq * d, kt, len, len, d, scale);
      for (int64_t i = 0; i < len; ++i) {
        float* row = sc + i * len;
        for (int64_t j = i + 1; j < len; ++j) row[j] += -INFINITY;
        softmax_row(row, len);
      }
      gemm_packed(out + (t0 * hq + h) * d, (int64_t)hq * d, sc, len, vp, len, d, len, 1.f);
      free(sc);
      free(kt);
      free(vp);
    }
  }
}

/* ---------------------------------------------------------------------------------------------
 * Rotary position embedding (crates/sketchpad-core/src/rope.rs). Compiled without floating-point
 * contraction: the reference evaluates x * cos + rotate_half(x) * sin as separate tensor ops,
 * each product and the sum rounded to f32.
 * ------------------------------------------------------------------------------------------- */
#pragma GCC push_options
#pragma GCC optimize("fp-contract=off")

/* RotaryEmbedding::with_base (rope.rs:60-92) + repeat_interleave (:95-102): the full caches
 * [rows][head_dim], each pair's cos / sin stored twice. inv_freq = 1 / base^(2i/d) in f32
 * (:66-68), angles = positions x inv_freq (a [rows,1] x [1,d/2] matmul: one f32 product,
 * :75-78), cos / sin in f32 (:81-82). */
void spo_rope_caches(float* cos_full, float* sin_full, int64_t rows, int64_t head_dim, float base) {
  const int64_t half = head_dim / 2;
  for (int64_t i = 0; i < half; ++i) {
    const float inv_freq = 1.0f / powf(base, (float)(2 * i) / (float)head_dim);
    for (int64_t p = 0; p < rows; ++p) {
      const float angle = (float)p * inv_freq;
      const float c = cosf(angle), sn = sinf(angle);
      cos_full[p * head_dim + 2 * i] = c;
      cos_full[p * head_dim + 2 * i + 1] = c;
      sin_full[p * head_dim + 2 * i] = sn;
      sin_full[p * head_dim + 2 * i + 1] = sn;
    }
  }
}

/* apply_rotary + rotate_half (rope.rs:136-170) on f32 rows, in place: token t of x (element
 * (t, h, d) at t*tok_stride + h*head_stride + d) at position positions[t] becomes
 * x * cos[pos] + rotate_half(x) * sin[pos], rotate_half([x0, x1, ...]) = [-x1, x0, ...].
 * Returns -1 if a position is outside the caches (the reference's slice would panic). */
int spo_rope_apply(float* x, int64_t tokens, int64_t heads, int64_t head_dim, int64_t tok_stride,
                   int64_t head_stride, const int32_t* positions, const float* cos_full,
                   const float* sin_full, int64_t rows) {
  for (int64_t t = 0; t < tokens; ++t) {
    const int64_t pos = positions[t];
    if (pos < 0 || pos >= rows) return -1;
    const float* c = cos_full + pos * head_dim;
    const float* sn = sin_full + pos * head_dim;
    for (int64_t h = 0; h < heads; ++h) {
      float* r = x + t * tok_stride + h * head_stride;
      for (int64_t i = 0; i < head_dim; i += 2) {
        const float x0 = r[i], x1 = r[i + 1];
        const float rot0 = -x1, rot1 = x0; /* rotate_half */
        const float a0 = x0 * c[i], b0 = rot0 * sn[i];
        const float a1 = x1 * c[i + 1], b1 = rot1 * sn[i + 1];
        r[i] = a0 + b0;
        r[i + 1] = a1 + b1;
      }
    }
  }
  return 0;
}

#pragma GCC pop_options


/* ---------------------------------------------------------------------------------------------
 * PolarQuant codec of CompressedKvCache (crates/sketchpad-core/src/kv_cache.rs:437-532). Each
 * head_dim vector becomes one record: its Euclidean norm as an IEEE binary16 (2 bytes, little
 * endian) followed by ceil(head_dim / 2) bytes of 4-bit two's-complement direction codes, the
 * even dimension of a pair in the high nibble. Compiled without contraction: the reference sums
 * the squares as separate f32 products and additions.
 * ------------------------------------------------------------------------------------------- */
#pragma GCC push_options
#pragma GCC optimize("fp-contract=off")

/* binary32 -> binary16 bits, IEEE 754 round to nearest even: overflow to infinity, results below
 * the smallest normal rounded to a subnormal (or zero), NaN kept quiet with its sign and top
 * payload bits. This is the conversion the reference's f16::from_f32 performs (kv_cache.rs:449).
 * Written from the format definition; the tests compare it with numpy's float16 conversion. */
uint16_t spo_f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((x >> 23) & 0xffu);
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x0200u | (man >> 13) : 0u));
  const int32_t e = exp - 127 + 15; /* binary16 biased exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    /* subnormal result: value = M * 2^(exp-150) with M the 24-bit significand, in units of
     * 2^-24 that is M >> (14 - e) */
    if (e < -10) return (uint16_t)sign; /* below 2^-25: rounds to zero */
    const uint32_t m = man | 0x800000u;
    const int shift = 14 - e;
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r; /* may carry into the smallest normal */
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r; /* may carry into infinity */
  return (uint16_t)(sign | r);
}

/* binary16 bits -> binary32 (exact). */
float spo_f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t x;
  if (exp == 0x1f) {
    x = sign | 0x7f800000u | (man << 13);
  } else if (exp != 0) {
    x = sign | ((exp + 112u) << 23) | (man << 13);
  } else {
    const float v = ldexpf((float)man, -24); /* subnormal (or zero): man * 2^-24, exact */
    memcpy(&x, &v, 4);
    x |= sign;
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* One direction code: (d * 7.0).round().clamp(-7.0, 7.0) as i8 (kv_cache.rs:462-469). f32::round
 * rounds half away from zero (C roundf); clamp keeps a NaN and `as i8` maps it to 0. */
static int polar_code(float d) {
  const float t = roundf(d * 7.0f);
  if (t != t) return 0;
  return t < -7.0f ? -7 : (t > 7.0f ? 7 : (int)t);
}

int64_t spo_polar_record_bytes(int64_t head_dim) { return 2 + (head_dim + 1) / 2; }

/* polar_quant_compress (kv_cache.rs:437-483): num_vecs rows of head_dim f32 -> num_vecs records
 * of spo_polar_record_bytes(head_dim) bytes. */
void spo_polar_compress(uint8_t* out, const float* x, int64_t num_vecs, int64_t head_dim) {
  const int64_t nb = (head_dim + 1) / 2, rec = 2 + nb;
  for (int64_t i = 0; i < num_vecs; ++i) {
    const float* r = x + i * head_dim;
    uint8_t* o = out + i * rec;
    float ss = 0.0f; /* Sum::<f32> over the squares: a left fold */
    for (int64_t j = 0; j < head_dim; ++j) ss = ss + r[j] * r[j];
    const float mag = sqrtf(ss);
    const uint16_t mb = spo_f32_to_f16_bits(mag);
    o[0] = (uint8_t)(mb & 0xffu);
    o[1] = (uint8_t)(mb >> 8);
    memset(o + 2, 0, (size_t)nb);
    if (mag == 0.0f) continue;
    const float inv = 1.0f / mag;
    for (int64_t j = 0; j < head_dim; j += 2) {
      const int q0 = polar_code(r[j] * inv);
      const int q1 = j + 1 < head_dim ? polar_code(r[j + 1] * inv) : 0;
      o[2 + j / 2] = (uint8_t)(((q0 & 0xf) << 4) | (q1 & 0xf));
    }
  }
}

/* 4-bit two's complement nibble -> integer (kv_cache.rs:510-528). */
static int polar_nibble(unsigned raw) { return raw > 7 ? (int)raw - 16 : (int)raw; }

/* polar_quant_decompress (kv_cache.rs:486-532): records -> num_vecs rows of head_dim f32,
 * element = code * (magnitude / 7); a zero magnitude gives a zero row. */
void spo_polar_decompress(float* out, const uint8_t* bytes, int64_t num_vecs, int64_t head_dim) {
  const int64_t rec = spo_polar_record_bytes(head_dim);
  for (int64_t i = 0; i < num_vecs; ++i) {
    const uint8_t* b = bytes + i * rec;
    float* o = out + i * head_dim;
    const float mag = spo_f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    for (int64_t j = 0; j < head_dim; ++j) o[j] = 0.0f;
    if (mag == 0.0f) continue;
    const float scale = mag / 7.0f;
    for (int64_t j = 0; j < head_dim; j += 2) {
      const uint8_t byte = b[2 + j / 2];
      o[j] = (float)polar_nibble((byte >> 4) & 0xfu) * scale;
      if (j + 1 < head_dim) o[j + 1] = (float)polar_nibble(byte & 0xfu) * scale;
    }
  }
}

/* KvQuantMethod::PolarQuant.compression_ratio (kv_cache.rs:315-318): (2 + D/2) / (2 D). */
double spo_polar_compression_ratio(int64_t head_dim) {
  return (2.0 + (double)head_dim / 2.0) / ((double)head_dim * 2.0);
}

/* ---- QJL (KvQuantMethod::QJL, kv_cache.rs:300-324, :371-396, :534-617) ---- */

/* lcg_normal_f32 (kv_cache.rs:373-396): the 64-bit LCG state from 42 (Numerical Recipes
 * constants, wrapping), uniforms (state >> 11) as f32 / 2^53 (u1 floored at 1e-10), Box-Muller
 * r = sqrt(-2 ln u1) * scale giving r cos(2 pi u2) then r sin(2 pi u2), all in f32. */
void spo_qjl_lcg_normal(float* out, int64_t count, float scale) {
  uint64_t state = 42u;
  int64_t i = 0;
  while (i < count) {
    state = state * 1664525u + 1013904223u;
    float u1 = (float)(state >> 11) / (float)(1ull << 53);
    if (!(u1 > 1e-10f)) u1 = 1e-10f;
    state = state * 1664525u + 1013904223u;
    const float u2 = (float)(state >> 11) / (float)(1ull << 53);
    const float r = sqrtf(-2.0f * logf(u1)) * scale;
    const float t = 6.28318548f * u2;
    out[i++] = r * cosf(t);
    if (i < count) out[i++] = r * sinf(t);
  }
}

/* CompressedKvCache::new (kv_cache.rs:417-424): R [proj_dim, head_dim] ~ N(0, 1/proj_dim). */
void spo_qjl_projection(float* out, int64_t proj_dim, int64_t head_dim) {
  spo_qjl_lcg_normal(out, proj_dim * head_dim, sqrtf(1.0f / (float)proj_dim));
}

int64_t spo_qjl_record_bytes(int64_t proj_dim) { return 2 + (proj_dim + 7) / 8; }

/* qjl_compress (kv_cache.rs:534-569): per vector the f16 magnitude (left fold of x*x, sqrt),
 * then if it is nonzero bit k of the sign bytes = (R[k,:] . x >= 0), the dot a left fold. */
void spo_qjl_compress(uint8_t* out, const float* x, int64_t num_vecs, int64_t head_dim,
                      const float* proj, int64_t proj_dim) {
  const int64_t rec = spo_qjl_record_bytes(proj_dim);
  memset(out, 0, (size_t)(num_vecs * rec));
  for (int64_t i = 0; i < num_vecs; ++i) {
    const float* v = x + i * head_dim;
    uint8_t* o = out + i * rec;
    float ss = 0.0f;
    for (int64_t j = 0; j < head_dim; ++j) ss = ss + v[j] * v[j];
    const float mag = sqrtf(ss);
    const uint16_t bits = spo_f32_to_f16_bits(mag);
    o[0] = (uint8_t)(bits & 0xff);
    o[1] = (uint8_t)(bits >> 8);
    if (mag == 0.0f) continue;
    for (int64_t k = 0; k < proj_dim; ++k) {
      const float* r = proj + k * head_dim;
      float dot = 0.0f;
      for (int64_t j = 0; j < head_dim; ++j) dot = dot + r[j] * v[j];
      if (dot >= 0.0f) o[2 + k / 8] |= (uint8_t)(1u << (k % 8));
    }
  }
}

/* qjl_decompress (kv_cache.rs:571-617): out[j] = (sum_k s_k R[k, j]) * (|x| * (pi/2 / proj_dim)),
 * the sum in k order from 0, s_k = +1 for a set bit, -1 otherwise; zeros for a zero magnitude. */
void spo_qjl_decompress(float* out, const uint8_t* bytes, int64_t num_vecs, int64_t head_dim,
                        const float* proj, int64_t proj_dim) {
  const int64_t rec = spo_qjl_record_bytes(proj_dim);
  const float scale_factor = 1.57079637f / (float)proj_dim; /* FRAC_PI_2 as f32 */
  for (int64_t i = 0; i < num_vecs; ++i) {
    const uint8_t* b = bytes + i * rec;
    float* o = out + i * head_dim;
    for (int64_t j = 0; j < head_dim; ++j) o[j] = 0.0f;
    const float mag = spo_f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    if (mag == 0.0f) continue;
    const float scale = mag * scale_factor;
    for (int64_t k = 0; k < proj_dim; ++k) {
      const float sign = ((b[2 + k / 8] >> (k % 8)) & 1) ? 1.0f : -1.0f;
      const float* r = proj + k * head_dim;
      for (int64_t j = 0; j < head_dim; ++j) o[j] = o[j] + sign * r[j];
    }
    for (int64_t j = 0; j < head_dim; ++j) o[j] = o[j] * scale;
  }
}

/* KvQuantMethod::QJL.compression_ratio (kv_cache.rs:319-321): (2 + P/8) / (2 D). */
double spo_qjl_compression_ratio(int64_t proj_dim, int64_t head_dim) {
  return (2.0 + (double)proj_dim / 8.0) / ((double)head_dim * 2.0);
}

#pragma GCC pop_options
