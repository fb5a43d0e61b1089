// C-ABI entry points (include/sketchpad_attn.h): argument validation, geometry, launches.
//
// Every entry point checks its arguments on the host before anything is enqueued, turns each
// failure into an sp_status plus a thread-local message, and never throws across the ABI.
#include <stdarg.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <mutex>
#include <utility>
#include <string>

#include "kv_cache.hpp"
#include "linear.hpp"
#include "paged_decode.hpp"
#include "polar_cache.hpp"
#include "prefill.hpp"
#include "qjl.hpp"
#include "rope_append.hpp"
#include "sp_common.hpp"

namespace sp {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SP_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SP_OK;
}

static int check_dtype(sp_dtype dt, const char* fn) {
  if (dt != SP_F32 && dt != SP_BF16 && dt != SP_F16)
    return fail(SP_EINVAL, "%s: unknown dtype %d", fn, (int)dt);
  return SP_OK;
}

static int check_layout(const sp_cache_layout* l, const char* fn) {
  if (!l) return fail(SP_EINVAL, "%s: layout is NULL", fn);
  if (l->num_blocks <= 0 || l->num_layers <= 0 || l->num_kv_heads <= 0 || l->block_size <= 0 ||
      l->head_dim <= 0)
    return fail(SP_EINVAL,
                "%s: layout sizes must be positive (num_blocks=%d num_layers=%d num_kv_heads=%d "
                "block_size=%d head_dim=%d)",
                fn, l->num_blocks, l->num_layers, l->num_kv_heads, l->block_size, l->head_dim);
  if (l->layer < 0 || l->layer >= l->num_layers)
    return fail(SP_EOOB, "%s: layer %d outside [0, %d)", fn, l->layer, l->num_layers);
  return SP_OK;
}

// Byte strides of the reference pool layout [num_blocks][num_layers][Hkv][BS][D].
static void pool_strides(const sp_cache_layout* l, int es, int64_t* block_stride_b,
                         int64_t* layer_off_b) {
  const int64_t layer_elems = (int64_t)l->num_kv_heads * l->block_size * l->head_dim;
  *block_stride_b = layer_elems * l->num_layers * es;
  *layer_off_b = layer_elems * l->layer * es;
}

}  // namespace sp

using namespace sp;

extern "C" {

int sp_version(void) { return SP_ABI_VERSION; }

const char* sp_last_error(void) { return g_last_error.c_str(); }

int sp_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout, const void* k_new,
                 const void* v_new, int64_t token_stride, int64_t head_stride,
                 const int32_t* slot_mapping, int32_t num_tokens, sp_dtype dtype, void* stream) {
  const char* fn = "sp_kv_append";
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_tokens < 0) return fail(SP_EINVAL, "%s: num_tokens %d < 0", fn, num_tokens);
  if (num_tokens == 0) return SP_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !slot_mapping)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (token_stride < 0 || head_stride < 0)
    return fail(SP_EINVAL, "%s: negative stride", fn);
  const int es = dtype_size(dtype);
  KvAppendArgs a{};
  a.kpool = (char*)k_pool;
  a.vpool = (char*)v_pool;
  a.knew = (const char*)k_new;
  a.vnew = (const char*)v_new;
  a.tok_stride_b = token_stride * es;
  a.head_stride_b = head_stride * es;
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.hkv = layout->num_kv_heads;
  a.row_bytes = layout->head_dim * es;
  a.block_size = layout->block_size;
  pool_strides(layout, es, &a.block_stride_b, &a.layer_off_b);
  a.num_slots = (int64_t)layout->num_blocks * layout->block_size;
  return launch_kv_append(a, (hipStream_t)stream);
}

int sp_rope_tables(float* cos_table, float* sin_table, int32_t rows, int32_t head_dim,
                   float base) {
  const char* fn = "sp_rope_tables";
  if (rows < 0 || head_dim <= 0 || (head_dim & 1))
    return fail(SP_EINVAL, "%s: rows %d, head_dim %d (must be even and > 0)", fn, rows, head_dim);
  if (rows == 0) return SP_OK;
  if (!cos_table || !sin_table) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (!(base > 0.f) || !isfinite(base)) return fail(SP_EINVAL, "%s: base must be > 0", fn);
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    // fp32 throughout, as the reference: 1.0 / base.powf((2 * i) as f32 / head_dim as f32)
    const float inv_freq = 1.0f / powf(base, (float)(2 * i) / (float)head_dim);
    for (int p = 0; p < rows; ++p) {
      const float angle = (float)p * inv_freq;
      cos_table[(int64_t)p * half + i] = cosf(angle);
      sin_table[(int64_t)p * half + i] = sinf(angle);
    }
  }
  return SP_OK;
}

int sp_rope_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout,
                      const void* k_new, const void* v_new, int64_t token_stride,
                      int64_t head_stride, void* q, int64_t q_token_stride, int64_t q_head_stride,
                      int32_t num_q_heads, const int32_t* positions, const int32_t* slot_mapping,
                      int32_t num_tokens, const float* cos_table, const float* sin_table,
                      int32_t table_rows, sp_dtype dtype, void* stream) {
  const char* fn = "sp_rope_kv_append";
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_tokens < 0 || table_rows < 0)
    return fail(SP_EINVAL, "%s: num_tokens %d, table_rows %d", fn, num_tokens, table_rows);
  if (layout->head_dim & 1) return fail(SP_EINVAL, "%s: head_dim %d is odd", fn, layout->head_dim);
  if (num_tokens == 0) return SP_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !positions || !slot_mapping || !cos_table ||
      !sin_table)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (token_stride < 0 || head_stride < 0 || q_token_stride < 0 || q_head_stride < 0)
    return fail(SP_EINVAL, "%s: negative stride", fn);
  if (q && num_q_heads <= 0) return fail(SP_EINVAL, "%s: num_q_heads %d", fn, num_q_heads);
  const int es = dtype_size(dtype);
  RopeAppendArgs a{};
  a.kpool = (char*)k_pool;
  a.vpool = (char*)v_pool;
  a.knew = (const char*)k_new;
  a.vnew = (const char*)v_new;
  a.kv_tok_b = token_stride * es;
  a.kv_head_b = head_stride * es;
  a.q = (char*)q;
  a.q_tok_b = q_token_stride * es;
  a.q_head_b = q_head_stride * es;
  a.positions = positions;
  a.slots = slot_mapping;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.table_rows = table_rows;
  a.num_tokens = num_tokens;
  a.hkv = layout->num_kv_heads;
  a.hq = q ? num_q_heads : 0;
  a.head_dim = layout->head_dim;
  a.block_size = layout->block_size;
  pool_strides(layout, es, &a.block_stride_b, &a.layer_off_b);
  a.num_slots = (int64_t)layout->num_blocks * layout->block_size;
  return launch_rope_kv_append(a, dtype, (hipStream_t)stream);
}

int sp_kv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                 const sp_cache_layout* layout, const int32_t* block_table,
                 int32_t num_table_blocks, int32_t seq_len, sp_dtype dtype, void* stream) {
  const char* fn = "sp_kv_gather";
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (seq_len < 0) return fail(SP_EINVAL, "%s: seq_len %d < 0", fn, seq_len);
  if (seq_len == 0) return SP_OK;
  if (!k_out || !v_out || !k_pool || !v_pool || !block_table)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  const int64_t needed = ((int64_t)seq_len + layout->block_size - 1) / layout->block_size;
  if (num_table_blocks < needed)
    return fail(SP_EOOB, "%s: seq_len %d needs %lld blocks, the table holds %d", fn, seq_len,
                (long long)needed, num_table_blocks);
  const int es = dtype_size(dtype);
  KvGatherArgs a{};
  a.kout = (char*)k_out;
  a.vout = (char*)v_out;
  a.kpool = (const char*)k_pool;
  a.vpool = (const char*)v_pool;
  a.table = block_table;
  a.seq_len = seq_len;
  a.hkv = layout->num_kv_heads;
  a.row_bytes = layout->head_dim * es;
  a.block_size = layout->block_size;
  pool_strides(layout, es, &a.block_stride_b, &a.layer_off_b);
  a.num_blocks = layout->num_blocks;
  return launch_kv_gather(a, (hipStream_t)stream);
}

size_t sp_paged_decode_workspace_size(int32_t num_seqs, int32_t num_q_heads,
                                      int32_t max_context_len, int32_t window_left,
                                      const sp_cache_layout* layout) {
  if (!layout || layout->num_kv_heads <= 0 || num_seqs <= 0 || num_q_heads <= 0 ||
      max_context_len <= 0)
    return 0;
  // one size for both pool kinds: the larger of the dense and the PolarQuant plans
  const DecodePlan p = plan_decode(num_seqs, num_q_heads, layout->num_kv_heads, layout->head_dim,
                                   max_context_len, window_left, DecodeKind::Dense);
  const DecodePlan pq = plan_decode(num_seqs, num_q_heads, layout->num_kv_heads,
                                    layout->head_dim, max_context_len, window_left,
                                    DecodeKind::Polar);
  return p.ws_bytes > pq.ws_bytes ? p.ws_bytes : pq.ws_bytes;
}

// Validation and arguments shared by the dense and the PolarQuant decode entry points. The pool
// strides are left to the caller.
static int decode_setup(const char* fn, void* out, const void* q, const void* k_pool,
                        const void* v_pool, const sp_cache_layout* layout,
                        const int32_t* block_tables, int32_t max_blocks_per_seq,
                        const int32_t* context_lens, int32_t max_context_len, int32_t num_seqs,
                        int32_t num_q_heads, float scale, int32_t window_left, sp_dtype dtype,
                        void* workspace, size_t workspace_bytes, DecodeArgs* a,
                        DecodeKind kind = DecodeKind::Dense) {
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_seqs < 0 || num_q_heads <= 0 || max_context_len < 0 || max_blocks_per_seq < 0)
    return fail(SP_EINVAL,
                "%s: invalid sizes (num_seqs=%d num_q_heads=%d max_context_len=%d "
                "max_blocks_per_seq=%d)",
                fn, num_seqs, num_q_heads, max_context_len, max_blocks_per_seq);
  if (num_seqs == 0) return SP_OK;
  if (!out || !q || !k_pool || !v_pool || !block_tables || !context_lens)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  const int hkv = layout->num_kv_heads;
  if (num_q_heads % hkv != 0)
    return fail(SP_EINVAL, "%s: num_q_heads %d is not a multiple of num_kv_heads %d", fn,
                num_q_heads, hkv);
  const int group = num_q_heads / hkv;
  if (group > kDecodeMaxGroup)
    return fail(SP_EUNSUPPORTED, "%s: GQA group %d > %d has no kernel", fn, group,
                kDecodeMaxGroup);
  const int D = layout->head_dim;
  const bool wide = (D == 256 || D == 512) && dtype != SP_F32 && kind == DecodeKind::Dense;
  if (D != 64 && D != 128 && !wide)
    return fail(SP_EUNSUPPORTED,
                "%s: head_dim %d has no kernel (64, 128; 256 and 512 for 16-bit dense pools)", fn,
                D);
  if (window_left < -1) return fail(SP_EINVAL, "%s: window_left %d < -1", fn, window_left);
  if ((int64_t)max_context_len > (int64_t)max_blocks_per_seq * layout->block_size)
    return fail(SP_EOOB, "%s: max_context_len %d exceeds the block tables (%d blocks of %d)", fn,
                max_context_len, max_blocks_per_seq, layout->block_size);
  if (!isfinite(scale)) return fail(SP_EINVAL, "%s: scale is not finite", fn);
  const DecodePlan p =
      plan_decode(num_seqs, num_q_heads, hkv, D, max_context_len < 1 ? 1 : max_context_len,
                  window_left, kind);
  // dense pools: any block size (one that is not a multiple of the tile takes the per-row path,
  // where a tile spans several blocks); PolarQuant pools: multiples of the tile
  if (kind != DecodeKind::Dense && layout->block_size % p.tt != 0)
    return fail(SP_EUNSUPPORTED,
                "%s: block_size %d is not a multiple of the %d-token tile of PolarQuant pools", fn,
                layout->block_size, p.tt);
  if (p.ws_bytes > 0 && (!workspace || workspace_bytes < p.ws_bytes))
    return fail(SP_ENOSPACE, "%s: workspace of %zu bytes, %zu required", fn, workspace_bytes,
                p.ws_bytes);
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool |
       (uintptr_t)workspace) & 15)
    return fail(SP_EINVAL, "%s: out, q, pools and workspace must be 16-byte aligned", fn);
  a->out = out;
  a->q = q;
  a->kpool = (const char*)k_pool;
  a->vpool = (const char*)v_pool;
  a->block_tables = block_tables;
  a->context_lens = context_lens;
  a->partials = (float*)workspace;
  a->max_blocks_per_seq = max_blocks_per_seq;
  a->max_context_len = max_context_len;
  a->num_blocks = layout->num_blocks;
  a->block_size = layout->block_size;
  a->num_seqs = num_seqs;
  a->hq = num_q_heads;
  a->hkv = hkv;
  a->group = group;
  a->window_left = window_left;
  a->tps = p.tps;
  a->max_splits = p.max_splits;
  a->scale_log2 = scale * 1.4426950408889634f;
  return SP_OK;
}

}  // extern "C"

// The logit soft cap of the *_softcap entry points (Gemma-4's attn_logit_softcap: logits =
// cap * tanh(logits / cap) on the scaled product, before the mask, gemma4.rs:366-377). 0: none;
// > 0 runs on the head-dim-256 and -512 bf16 / f16 kernels (Gemma-4's two head dims), which take
// it as cap_in = 2 log2(e) scale / cap and cap_out = cap log2(e) (softcap_log2: the softmax's
// exponent units).
static int softcap_args(const char* fn, float softcap, float scale, int head_dim, sp_dtype dtype,
                        float* cap_in, float* cap_out) {
  *cap_in = *cap_out = 0.f;
  if (softcap == 0.f) return SP_OK;
  if (!(softcap > 0.f) || !isfinite(softcap))
    return fail(SP_EINVAL, "%s: logit_softcap must be finite and >= 0 (got %g)", fn,
                (double)softcap);
  if ((head_dim != 256 && head_dim != 512) || dtype == SP_F32)
    return fail(SP_EUNSUPPORTED,
                "%s: the logit soft cap runs at head_dims 256 and 512 on bf16 / f16 tensors (got "
                "head_dim %d, %s)",
                fn, head_dim, dtype_name(dtype));
  *cap_in = (float)(2.0 * 1.4426950408889634 * (double)scale / (double)softcap);
  *cap_out = (float)((double)softcap * 1.4426950408889634);
  return SP_OK;
}

static int paged_decode_impl(const char* fn, void* out, const void* q, const void* k_pool,
                             const void* v_pool, const sp_cache_layout* layout,
                             const int32_t* block_tables, int32_t max_blocks_per_seq,
                             const int32_t* context_lens, int32_t max_context_len,
                             int32_t num_seqs, int32_t num_q_heads, float scale,
                             int32_t window_left, sp_dtype dtype, void* workspace,
                             size_t workspace_bytes, float softcap, void* stream) {
  DecodeArgs a{};
  if (int rc = decode_setup(fn, out, q, k_pool, v_pool, layout, block_tables, max_blocks_per_seq,
                            context_lens, max_context_len, num_seqs, num_q_heads, scale,
                            window_left, dtype, workspace, workspace_bytes, &a))
    return rc;
  if (int rc = softcap_args(fn, softcap, scale, layout->head_dim, dtype, &a.cap_in, &a.cap_out))
    return rc;
  if (num_seqs == 0) return SP_OK;
  pool_strides(layout, dtype_size(dtype), &a.block_stride_b, &a.layer_off_b);
  return launch_paged_decode(a, dtype, layout->head_dim, (hipStream_t)stream);
}

static int paged_append_decode_impl(const char* fn, void* out, const void* q, void* k_pool,
                                    void* v_pool, const sp_cache_layout* layout,
                                    const void* k_new, const void* v_new, int64_t token_stride,
                                    int64_t head_stride, const int32_t* block_tables,
                                    int32_t max_blocks_per_seq, const int32_t* context_lens,
                                    int32_t max_context_len, int32_t num_seqs,
                                    int32_t num_q_heads, float scale, int32_t window_left,
                                    sp_dtype dtype, void* workspace, size_t workspace_bytes,
                                    float softcap, void* stream) {
  DecodeArgs a{};
  if (int rc = decode_setup(fn, out, q, k_pool, v_pool, layout, block_tables, max_blocks_per_seq,
                            context_lens, max_context_len, num_seqs, num_q_heads, scale,
                            window_left, dtype, workspace, workspace_bytes, &a))
    return rc;
  if (int rc = softcap_args(fn, softcap, scale, layout->head_dim, dtype, &a.cap_in, &a.cap_out))
    return rc;
  if (num_seqs == 0) return SP_OK;
  if (!k_new || !v_new) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (token_stride < 0 || head_stride < 0) return fail(SP_EINVAL, "%s: negative stride", fn);
  const int es = dtype_size(dtype);
  if ((((uintptr_t)k_new | (uintptr_t)v_new) & 15) || ((token_stride * es) & 15) ||
      ((head_stride * es) & 15))
    return fail(SP_EINVAL, "%s: k_new, v_new and their strides must be 16-byte aligned", fn);
  pool_strides(layout, es, &a.block_stride_b, &a.layer_off_b);
  a.k_new = (const char*)k_new;
  a.v_new = (const char*)v_new;
  a.new_tok_stride_b = token_stride * es;
  a.new_head_stride_b = head_stride * es;
  return launch_paged_decode(a, dtype, layout->head_dim, (hipStream_t)stream);
}

extern "C" {

int sp_paged_decode(void* out, const void* q, const void* k_pool, const void* v_pool,
                    const sp_cache_layout* layout, const int32_t* block_tables,
                    int32_t max_blocks_per_seq, const int32_t* context_lens,
                    int32_t max_context_len, int32_t num_seqs, int32_t num_q_heads, float scale,
                    int32_t window_left, sp_dtype dtype, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return paged_decode_impl("sp_paged_decode", out, q, k_pool, v_pool, layout, block_tables,
                           max_blocks_per_seq, context_lens, max_context_len, num_seqs,
                           num_q_heads, scale, window_left, dtype, workspace, workspace_bytes,
                           0.f, stream);
}

int sp_paged_decode_softcap(void* out, const void* q, const void* k_pool, const void* v_pool,
                            const sp_cache_layout* layout, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* context_lens,
                            int32_t max_context_len, int32_t num_seqs, int32_t num_q_heads,
                            float scale, float logit_softcap, int32_t window_left,
                            sp_dtype dtype, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return paged_decode_impl("sp_paged_decode_softcap", out, q, k_pool, v_pool, layout,
                           block_tables, max_blocks_per_seq, context_lens, max_context_len,
                           num_seqs, num_q_heads, scale, window_left, dtype, workspace,
                           workspace_bytes, logit_softcap, stream);
}

int sp_paged_append_decode(void* out, const void* q, void* k_pool, void* v_pool,
                           const sp_cache_layout* layout, const void* k_new, const void* v_new,
                           int64_t token_stride, int64_t head_stride, const int32_t* block_tables,
                           int32_t max_blocks_per_seq, const int32_t* context_lens,
                           int32_t max_context_len, int32_t num_seqs, int32_t num_q_heads,
                           float scale, int32_t window_left, sp_dtype dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return paged_append_decode_impl("sp_paged_append_decode", out, q, k_pool, v_pool, layout,
                                  k_new, v_new, token_stride, head_stride, block_tables,
                                  max_blocks_per_seq, context_lens, max_context_len, num_seqs,
                                  num_q_heads, scale, window_left, dtype, workspace,
                                  workspace_bytes, 0.f, stream);
}

int sp_paged_append_decode_softcap(void* out, const void* q, void* k_pool, void* v_pool,
                                   const sp_cache_layout* layout, const void* k_new,
                                   const void* v_new, int64_t token_stride, int64_t head_stride,
                                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* context_lens, int32_t max_context_len,
                                   int32_t num_seqs, int32_t num_q_heads, float scale,
                                   float logit_softcap, int32_t window_left, sp_dtype dtype,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  return paged_append_decode_impl("sp_paged_append_decode_softcap", out, q, k_pool, v_pool,
                                  layout, k_new, v_new, token_stride, head_stride, block_tables,
                                  max_blocks_per_seq, context_lens, max_context_len, num_seqs,
                                  num_q_heads, scale, window_left, dtype, workspace,
                                  workspace_bytes, logit_softcap, stream);
}

int sp_paged_decode_noalloc(void* out, const void* q, const void* k_pool, const void* v_pool,
                            const sp_cache_layout* layout, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* context_lens,
                            int32_t max_context_len, int32_t num_seqs, int32_t num_q_heads,
                            float scale, int32_t window_left, sp_dtype dtype, void* stream) {
  const char* fn = "sp_paged_decode_noalloc";
  // The split plan (and so the partials' size) is sp_paged_decode's for the same shape, so both
  // entry points run the same kernels on the same split boundaries.
  size_t need = 0;
  if (layout && layout->num_kv_heads > 0 && num_seqs > 0 && num_q_heads > 0 &&
      max_context_len > 0)
    need = plan_decode(num_seqs, num_q_heads, layout->num_kv_heads, layout->head_dim,
                       max_context_len, window_left, DecodeKind::Dense)
               .ws_bytes;
  if (need > kDecodeScratchBytes)
    return fail(SP_ENOSPACE,
                "%s: this batch needs %zu bytes of split partials, past the library's %zu-byte "
                "scratch; call sp_paged_decode with a workspace instead",
                fn, need, kDecodeScratchBytes);
  void* ws = nullptr;
  if (need > 0 && !(ws = decode_scratch_on_current_device())) return SP_EHIP;
  return sp_paged_decode(out, q, k_pool, v_pool, layout, block_tables, max_blocks_per_seq,
                         context_lens, max_context_len, num_seqs, num_q_heads, scale,
                         window_left, dtype, ws, need > 0 ? kDecodeScratchBytes : 0, stream);
}

// dense_f32: the dense f32 path (flash_attention), which also takes head dims 40, 80, 160 and
// 256 and a value head dim of its own; everything else runs head_dim 64 or 128, Dv == D (and
// 256 and 512 for 16-bit tensors).
static int check_prefill_common(const char* fn, int32_t num_seqs, int32_t max_seqlen_q,
                                int32_t hq, int32_t hkv, int32_t D, float scale,
                                int32_t causal, int32_t window_left, sp_dtype dtype,
                                int32_t Dv = -1, bool dense = false) {
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_seqs < 0 || max_seqlen_q < 0 || hq <= 0 || hkv <= 0)
    return fail(SP_EINVAL, "%s: invalid sizes (num_seqs=%d max_seqlen_q=%d hq=%d hkv=%d)", fn,
                num_seqs, max_seqlen_q, hq, hkv);
  if (hq % hkv != 0)
    return fail(SP_EINVAL, "%s: num_q_heads %d is not a multiple of num_kv_heads %d", fn, hq, hkv);
  if (Dv < 0) Dv = D;
  if (D <= 0 || Dv <= 0)
    return fail(SP_EINVAL, "%s: head_dim %d / value head_dim %d must be positive", fn, D, Dv);
  if (dense && dtype == SP_F32) {
    if (!prefill_f32_supports(D, Dv, false))
      return fail(SP_EUNSUPPORTED,
                  "%s: f32 head_dim %d / value head_dim %d has no kernel (head_dim 40, 64, 80, "
                  "128, 160 or 256; value head_dim a multiple of 4 up to 256)",
                  fn, D, Dv);
  } else if ((D != 64 && D != 128 && !((D == 256 || D == 512) && dtype != SP_F32)) || Dv != D) {
    return fail(SP_EUNSUPPORTED,
                "%s: head_dim %d / value head_dim %d has no %s kernel (64 or 128, and 256 and 512 "
                "for 16-bit tensors; equal)",
                fn, D, Dv, dtype_name(dtype));
  }
  if (causal < SP_CAUSAL_NONE || causal > SP_CAUSAL_TOP_LEFT)
    return fail(SP_EINVAL, "%s: unknown causal mode %d", fn, causal);
  if (window_left < -1) return fail(SP_EINVAL, "%s: window_left %d < -1", fn, window_left);
  // The kernel folds the scale into the exponent after taking the row maximum of the raw
  // scores, which needs scale > 0 (the reference always uses head_dim^-0.5).
  if (!isfinite(scale) || !(scale > 0.f))
    return fail(SP_EINVAL, "%s: scale must be finite and > 0 (got %g)", fn, (double)scale);
  return SP_OK;
}

static bool misaligned16(const void* p) { return ((uintptr_t)p & 15) != 0; }

static int varlen_prefill_impl(const char* fn, void* out, const void* q, const void* k,
                               const void* v, const int32_t* cu_seqlens_q,
                               const int32_t* cu_seqlens_k, int32_t num_seqs,
                               int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, float scale, int32_t causal,
                               int32_t window_left, sp_dtype dtype, float softcap,
                               void* stream) {
  if (int rc = check_prefill_common(fn, num_seqs, max_seqlen_q, num_q_heads, num_kv_heads,
                                    head_dim, scale, causal, window_left, dtype))
    return rc;
  if (num_seqs == 0 || max_seqlen_q == 0) return SP_OK;
  if (!out || !q || !k || !v || !cu_seqlens_q || !cu_seqlens_k)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (misaligned16(out) || misaligned16(q) || misaligned16(k) || misaligned16(v))
    return fail(SP_EINVAL, "%s: q, k, v and out must be 16-byte aligned", fn);
  PrefillArgs a{};
  a.out = out;
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_tok = a.o_tok = (int64_t)num_q_heads * head_dim;
  a.q_head = a.o_head = head_dim;
  a.kv_tok = a.v_tok = (int64_t)num_kv_heads * head_dim;
  a.kv_head = a.v_head = head_dim;
  a.dv = head_dim;
  a.out_dtype = dtype;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.num_seqs = num_seqs;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.num_qblocks = (max_seqlen_q + kPrefillBM - 1) / kPrefillBM;
  a.causal = causal;
  a.window_left = window_left;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (int rc = softcap_args(fn, softcap, scale, head_dim, dtype, &a.cap_in, &a.cap_out))
    return rc;
  return launch_prefill(a, dtype, head_dim, false, (hipStream_t)stream);
}

int sp_varlen_prefill(void* out, const void* q, const void* k, const void* v,
                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                      int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, float scale, int32_t causal, int32_t window_left,
                      sp_dtype dtype, void* stream) {
  return varlen_prefill_impl("sp_varlen_prefill", out, q, k, v, cu_seqlens_q, cu_seqlens_k,
                             num_seqs, max_seqlen_q, num_q_heads, num_kv_heads, head_dim, scale,
                             causal, window_left, dtype, 0.f, stream);
}

int sp_varlen_prefill_softcap(void* out, const void* q, const void* k, const void* v,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, float scale,
                              float logit_softcap, int32_t causal, int32_t window_left,
                              sp_dtype dtype, void* stream) {
  return varlen_prefill_impl("sp_varlen_prefill_softcap", out, q, k, v, cu_seqlens_q,
                             cu_seqlens_k, num_seqs, max_seqlen_q, num_q_heads, num_kv_heads,
                             head_dim, scale, causal, window_left, dtype, logit_softcap, stream);
}

// Key-range splits of a chunked prefill: the planner's count for the batch shape (the context
// bound is the block tables' width), lowered until the partials fit the caller's workspace.
static int prefill_splits(int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                          int32_t head_dim, int64_t max_context, size_t workspace_bytes) {
  if (head_dim >= 256) return 1;  // the head-dim-256 / 512 kernels walk every key tile themselves
  const int64_t base = (int64_t)((max_seqlen_q + kPrefillBM - 1) / kPrefillBM) * num_seqs *
                       num_q_heads;
  int s = plan_prefill_splits(base, (max_context + kPrefillBN - 1) / kPrefillBN);
  while (s > 1 &&
         prefill_partials_bytes(num_seqs, max_seqlen_q, num_q_heads, head_dim, s) > workspace_bytes)
    --s;
  return s;
}

size_t sp_paged_prefill_workspace_size(int32_t num_seqs, int32_t max_seqlen_q,
                                       int32_t num_q_heads, const sp_cache_layout* layout,
                                       int32_t max_blocks_per_seq) {
  if (!layout || num_seqs <= 0 || max_seqlen_q <= 0 || num_q_heads <= 0 ||
      layout->num_kv_heads <= 0 || max_blocks_per_seq <= 0 ||
      (layout->head_dim != 64 && layout->head_dim != 128))
    return 0;
  const int64_t max_context = (int64_t)max_blocks_per_seq * layout->block_size;
  const int s = prefill_splits(num_seqs, max_seqlen_q, num_q_heads, layout->head_dim,
                               max_context, SIZE_MAX);
  return prefill_partials_bytes(num_seqs, max_seqlen_q, num_q_heads, layout->head_dim, s);
}

static int paged_prefill_impl(const char* fn, void* out, const void* q, const void* k_pool,
                              const void* v_pool, const sp_cache_layout* layout,
                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                              const int32_t* cu_seqlens_q, const int32_t* context_lens,
                              int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                              float scale, int32_t window_left, sp_dtype dtype, void* workspace,
                              size_t workspace_bytes, float softcap, void* stream) {
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_prefill_common(fn, num_seqs, max_seqlen_q, num_q_heads,
                                    layout->num_kv_heads, layout->head_dim, scale,
                                    SP_CAUSAL_BOTTOM_RIGHT, window_left, dtype))
    return rc;
  float cap_in = 0.f, cap_out = 0.f;
  if (int rc = softcap_args(fn, softcap, scale, layout->head_dim, dtype, &cap_in, &cap_out))
    return rc;
  if (num_seqs == 0 || max_seqlen_q == 0) return SP_OK;
  if (!out || !q || !k_pool || !v_pool || !block_tables || !cu_seqlens_q || !context_lens)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (max_blocks_per_seq <= 0) return fail(SP_EINVAL, "%s: max_blocks_per_seq must be > 0", fn);
  if (misaligned16(out) || misaligned16(q) || misaligned16(k_pool) || misaligned16(v_pool))
    return fail(SP_EINVAL, "%s: q, out and pools must be 16-byte aligned", fn);
  const int D = layout->head_dim;
  PrefillArgs a{};
  a.out = out;
  a.q = q;
  a.q_tok = a.o_tok = (int64_t)num_q_heads * D;
  a.q_head = a.o_head = D;
  a.cu_q = cu_seqlens_q;
  a.num_seqs = num_seqs;
  a.hq = num_q_heads;
  a.hkv = layout->num_kv_heads;
  a.group = num_q_heads / layout->num_kv_heads;
  a.num_qblocks = (max_seqlen_q + kPrefillBM - 1) / kPrefillBM;
  a.causal = SP_CAUSAL_BOTTOM_RIGHT;
  a.window_left = window_left;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.dv = D;
  a.out_dtype = dtype;
  a.kpool = (const char*)k_pool;
  a.vpool = (const char*)v_pool;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.max_blocks_per_seq = max_blocks_per_seq;
  a.block_size = layout->block_size;
  a.num_blocks = layout->num_blocks;
  pool_strides(layout, dtype_size(dtype), &a.block_stride_b, &a.layer_off_b);
  if (workspace && misaligned16(workspace))
    return fail(SP_EINVAL, "%s: workspace must be 16-byte aligned", fn);
  a.nsplit = workspace ? prefill_splits(num_seqs, max_seqlen_q, num_q_heads, D,
                                        (int64_t)max_blocks_per_seq * layout->block_size,
                                        workspace_bytes)
                       : 1;
  a.partials = a.nsplit > 1 ? (float*)workspace : nullptr;
  a.max_q = max_seqlen_q;
  a.cap_in = cap_in;
  a.cap_out = cap_out;
  return launch_prefill(a, dtype, D, true, (hipStream_t)stream);
}

int sp_paged_prefill(void* out, const void* q, const void* k_pool, const void* v_pool,
                     const sp_cache_layout* layout, const int32_t* block_tables,
                     int32_t max_blocks_per_seq, const int32_t* cu_seqlens_q,
                     const int32_t* context_lens, int32_t num_seqs, int32_t max_seqlen_q,
                     int32_t num_q_heads, float scale, int32_t window_left, sp_dtype dtype,
                     void* workspace, size_t workspace_bytes, void* stream) {
  return paged_prefill_impl("sp_paged_prefill", out, q, k_pool, v_pool, layout, block_tables,
                            max_blocks_per_seq, cu_seqlens_q, context_lens, num_seqs,
                            max_seqlen_q, num_q_heads, scale, window_left, dtype, workspace,
                            workspace_bytes, 0.f, stream);
}

int sp_paged_prefill_softcap(void* out, const void* q, const void* k_pool, const void* v_pool,
                             const sp_cache_layout* layout, const int32_t* block_tables,
                             int32_t max_blocks_per_seq, const int32_t* cu_seqlens_q,
                             const int32_t* context_lens, int32_t num_seqs,
                             int32_t max_seqlen_q, int32_t num_q_heads, float scale,
                             float logit_softcap, int32_t window_left, sp_dtype dtype,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return paged_prefill_impl("sp_paged_prefill_softcap", out, q, k_pool, v_pool, layout,
                            block_tables, max_blocks_per_seq, cu_seqlens_q, context_lens,
                            num_seqs, max_seqlen_q, num_q_heads, scale, window_left, dtype,
                            workspace, workspace_bytes, logit_softcap, stream);
}

// Byte offset of the prefill's region in a mixed batch's workspace: the decode's partials come
// first, rounded up to 256 bytes.
static size_t ragged_decode_bytes(int32_t num_decode_seqs, int32_t num_q_heads,
                                  int32_t decode_max_context_len, int32_t window_left,
                                  const sp_cache_layout* layout) {
  if (num_decode_seqs <= 0) return 0;
  const size_t d = sp_paged_decode_workspace_size(num_decode_seqs, num_q_heads,
                                                  decode_max_context_len, window_left, layout);
  return (d + 255) & ~(size_t)255;
}

size_t sp_ragged_attention_workspace_size(int32_t num_seqs, int32_t num_prefill_seqs,
                                          int32_t prefill_max_seqlen_q,
                                          int32_t decode_max_context_len, int32_t num_q_heads,
                                          int32_t window_left, const sp_cache_layout* layout,
                                          int32_t max_blocks_per_seq) {
  if (num_seqs <= 0 || num_prefill_seqs < 0 || num_prefill_seqs > num_seqs) return 0;
  size_t need = ragged_decode_bytes(num_seqs - num_prefill_seqs, num_q_heads,
                                    decode_max_context_len, window_left, layout);
  if (num_prefill_seqs > 0)
    need += sp_paged_prefill_workspace_size(num_prefill_seqs, prefill_max_seqlen_q, num_q_heads,
                                            layout, max_blocks_per_seq);
  return need;
}

// The side stream and fork / join events of mixed batches issued on one caller stream of one
// device, made on first use (default priority, events without timing). Each (device, caller
// stream) pair has its own, so mixed steps on independent caller streams never queue behind each
// other on a shared side stream, and a caller stream under graph capture pulls only its own side
// stream into the capture. g_fork_mu guards the table and keeps each call's record / wait pairs
// together when several host threads issue mixed batches on one caller stream.
struct ForkJoin {
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
static std::mutex g_fork_mu;
// Past this many (device, caller stream) pairs a mixed batch runs both halves on the caller's
// stream, one after the other (the table is never pruned: a stream handle may be reused).
constexpr size_t kMaxForkJoins = 256;

// *out = the pair's resources, or nullptr when the table is full. Call with g_fork_mu held.
static int fork_join_for(hipStream_t caller, ForkJoin** out) {
  static std::map<std::pair<int, uintptr_t>, ForkJoin> table;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SP_EHIP, "mixed batch: hipGetDevice: %s", hipGetErrorString(e));
  const auto key = std::make_pair(dev, (uintptr_t)caller);
  auto it = table.find(key);
  if (it != table.end()) {
    *out = &it->second;
    return SP_OK;
  }
  if (table.size() >= kMaxForkJoins) {
    *out = nullptr;
    return SP_OK;
  }
  hipStream_t s = nullptr;
  hipEvent_t f = nullptr, j = nullptr;
  if ((e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&f, hipEventDisableTiming)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&j, hipEventDisableTiming)) != hipSuccess) {
    if (j) (void)hipEventDestroy(j);
    if (f) (void)hipEventDestroy(f);
    if (s) (void)hipStreamDestroy(s);
    return fail(SP_EHIP, "mixed batch: side stream on device %d: %s", dev, hipGetErrorString(e));
  }
  ForkJoin& fj = table[key];
  fj.side = s;
  fj.fork = f;
  fj.join = j;
  *out = &fj;
  return SP_OK;
}

static int ragged_paged_attention_impl(
    const char* fn, void* out, const void* q, const void* k_pool, const void* v_pool,
    const sp_cache_layout* layout, const int32_t* block_tables, int32_t max_blocks_per_seq,
    const int32_t* cu_seqlens_q, const int32_t* context_lens, int32_t num_seqs,
    int32_t num_prefill_seqs, int32_t num_prefill_tokens, int32_t prefill_max_seqlen_q,
    int32_t decode_max_context_len, int32_t num_q_heads, float scale, int32_t window_left,
    sp_dtype dtype, void* workspace, size_t workspace_bytes, float softcap, void* stream) {
  if (int rc = check_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  float cap_in = 0.f, cap_out = 0.f;
  if (int rc = softcap_args(fn, softcap, scale, layout->head_dim, dtype, &cap_in, &cap_out))
    return rc;
  if (num_seqs < 0 || num_prefill_seqs < 0 || num_prefill_seqs > num_seqs ||
      num_prefill_tokens < 0 || num_q_heads <= 0 || max_blocks_per_seq < 0)
    return fail(SP_EINVAL,
                "%s: invalid sizes (num_seqs=%d num_prefill_seqs=%d num_prefill_tokens=%d "
                "num_q_heads=%d max_blocks_per_seq=%d)",
                fn, num_seqs, num_prefill_seqs, num_prefill_tokens, num_q_heads,
                max_blocks_per_seq);
  if (num_seqs == 0) return SP_OK;
  if (!out || !q || !block_tables || !context_lens || (num_prefill_seqs > 0 && !cu_seqlens_q))
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  const int nd = num_seqs - num_prefill_seqs;
  const int64_t row = (int64_t)num_q_heads * layout->head_dim * dtype_size(dtype);
  auto decode_half = [&](void* ws, size_t ws_bytes, void* st) {
    return paged_decode_impl(fn, (char*)out + num_prefill_tokens * row,
                             (const char*)q + num_prefill_tokens * row, k_pool, v_pool, layout,
                             block_tables + (int64_t)num_prefill_seqs * max_blocks_per_seq,
                             max_blocks_per_seq, context_lens + num_prefill_seqs,
                             decode_max_context_len, nd, num_q_heads, scale, window_left, dtype,
                             ws, ws_bytes, softcap, st);
  };
  auto prefill_half = [&](void* ws, size_t ws_bytes, void* st) {
    return paged_prefill_impl(fn, out, q, k_pool, v_pool, layout, block_tables,
                              max_blocks_per_seq, cu_seqlens_q, context_lens, num_prefill_seqs,
                              prefill_max_seqlen_q, num_q_heads, scale, window_left, dtype, ws,
                              ws_bytes, softcap, st);
  };
  if (nd == 0) return prefill_half(workspace, workspace_bytes, stream);
  if (num_prefill_seqs == 0) return decode_half(workspace, workspace_bytes, stream);

  // Both halves: the decode's partials take the front of the workspace, the prefill's split
  // partials (if its plan splits) the rest. The decode runs on the side stream, forked from and
  // joined back into the caller's stream, so its workgroups fill the slots the chunks' long key
  // walks leave idle (C4: 250-300 us for the pair against 345 us one after the other).
  const size_t d_bytes =
      ragged_decode_bytes(nd, num_q_heads, decode_max_context_len, window_left, layout);
  void* pws = workspace && workspace_bytes > d_bytes ? (char*)workspace + d_bytes : nullptr;
  const size_t pws_bytes = pws ? workspace_bytes - d_bytes : 0;
  // the decode half is validated before anything is enqueued (the prefill validates itself
  // before its launch)
  DecodeArgs da{};
  if (int rc = decode_setup(fn, (char*)out + num_prefill_tokens * row,
                            (const char*)q + num_prefill_tokens * row, k_pool, v_pool, layout,
                            block_tables + (int64_t)num_prefill_seqs * max_blocks_per_seq,
                            max_blocks_per_seq, context_lens + num_prefill_seqs,
                            decode_max_context_len, nd, num_q_heads, scale, window_left, dtype,
                            workspace, workspace_bytes < d_bytes ? workspace_bytes : d_bytes, &da))
    return rc;
  da.cap_in = cap_in;
  da.cap_out = cap_out;
  pool_strides(layout, dtype_size(dtype), &da.block_stride_b, &da.layer_off_b);
  const hipStream_t caller = (hipStream_t)stream;
  std::lock_guard<std::mutex> lock(g_fork_mu);
  ForkJoin* fj = nullptr;
  if (int rc = fork_join_for(caller, &fj)) return rc;
  if (!fj) {  // no side stream left for this caller stream: both halves on the caller's
    if (int rc = prefill_half(pws, pws_bytes, stream)) return rc;
    return launch_paged_decode(da, dtype, layout->head_dim, caller);
  }
  hipError_t e = hipEventRecord(fj->fork, caller);
  if (e == hipSuccess) e = hipStreamWaitEvent(fj->side, fj->fork, 0);
  if (e != hipSuccess) return fail(SP_EHIP, "%s: fork: %s", fn, hipGetErrorString(e));
  // the chunks' long key walks are dispatched first, the decode's short workgroups after them
  const int rc_p = prefill_half(pws, pws_bytes, stream);
  const int rc = rc_p ? rc_p : launch_paged_decode(da, dtype, layout->head_dim, fj->side);
  // the join is recorded whatever the launches returned, so the side stream never stays forked
  e = hipEventRecord(fj->join, fj->side);
  if (e == hipSuccess) e = hipStreamWaitEvent(caller, fj->join, 0);
  if (e != hipSuccess) return fail(SP_EHIP, "%s: join: %s", fn, hipGetErrorString(e));
  return rc;
}

int sp_ragged_paged_attention(void* out, const void* q, const void* k_pool, const void* v_pool,
                              const sp_cache_layout* layout, const int32_t* block_tables,
                              int32_t max_blocks_per_seq, const int32_t* cu_seqlens_q,
                              const int32_t* context_lens, int32_t num_seqs,
                              int32_t num_prefill_seqs, int32_t num_prefill_tokens,
                              int32_t prefill_max_seqlen_q, int32_t decode_max_context_len,
                              int32_t num_q_heads, float scale, int32_t window_left,
                              sp_dtype dtype, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return ragged_paged_attention_impl(
      "sp_ragged_paged_attention", out, q, k_pool, v_pool, layout, block_tables,
      max_blocks_per_seq, cu_seqlens_q, context_lens, num_seqs, num_prefill_seqs,
      num_prefill_tokens, prefill_max_seqlen_q, decode_max_context_len, num_q_heads, scale,
      window_left, dtype, workspace, workspace_bytes, 0.f, stream);
}

int sp_ragged_paged_attention_softcap(
    void* out, const void* q, const void* k_pool, const void* v_pool,
    const sp_cache_layout* layout, const int32_t* block_tables, int32_t max_blocks_per_seq,
    const int32_t* cu_seqlens_q, const int32_t* context_lens, int32_t num_seqs,
    int32_t num_prefill_seqs, int32_t num_prefill_tokens, int32_t prefill_max_seqlen_q,
    int32_t decode_max_context_len, int32_t num_q_heads, float scale, float logit_softcap,
    int32_t window_left, sp_dtype dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return ragged_paged_attention_impl(
      "sp_ragged_paged_attention_softcap", out, q, k_pool, v_pool, layout, block_tables,
      max_blocks_per_seq, cu_seqlens_q, context_lens, num_seqs, num_prefill_seqs,
      num_prefill_tokens, prefill_max_seqlen_q, decode_max_context_len, num_q_heads, scale,
      window_left, dtype, workspace, workspace_bytes, logit_softcap, stream);
}

static int flash_attention_impl(const char* fn, void* out, const void* q, const void* k,
                                const void* v, const float* mask, int64_t mask_stride_b,
                                int64_t mask_stride_h, int64_t mask_stride_q, int32_t batch,
                                int32_t num_heads, int32_t seq_q, int32_t seq_k, int32_t head_dim,
                                int32_t v_head_dim, float scale, int32_t causal, sp_dtype dtype,
                                sp_dtype out_dtype, void* stream) {
  if (int rc = check_prefill_common(fn, batch, seq_q, num_heads, num_heads, head_dim, scale,
                                    causal ? SP_CAUSAL_TOP_LEFT : SP_CAUSAL_NONE, -1, dtype,
                                    v_head_dim, true))
    return rc;
  if (int rc = check_dtype(out_dtype, fn)) return rc;
  if (seq_k < 0) return fail(SP_EINVAL, "%s: seq_k %d < 0", fn, seq_k);
  if (mask_stride_b < 0 || mask_stride_h < 0 || mask_stride_q < 0)
    return fail(SP_EINVAL, "%s: negative mask stride", fn);
  if (batch == 0 || seq_q == 0) return SP_OK;
  if (!out || !q || !k || !v) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (misaligned16(out) || misaligned16(q) || misaligned16(k) || misaligned16(v))
    return fail(SP_EINVAL, "%s: q, k, v and out must be 16-byte aligned", fn);
  if (mask && ((uintptr_t)mask & 3)) return fail(SP_EINVAL, "%s: mask is not 4-byte aligned", fn);
  PrefillArgs a{};
  a.out = out;
  a.q = q;
  a.k = k;
  a.v = v;
  // [B, H, S, D] (q, k) and [B, H, S, Dv] (v, out): token stride D or Dv, head stride S * that
  a.q_tok = head_dim;
  a.q_head = (int64_t)seq_q * head_dim;
  a.q_batch = (int64_t)num_heads * seq_q * head_dim;
  a.o_tok = v_head_dim;
  a.o_head = (int64_t)seq_q * v_head_dim;
  a.o_batch = (int64_t)num_heads * seq_q * v_head_dim;
  a.kv_tok = head_dim;
  a.kv_head = (int64_t)seq_k * head_dim;
  a.kv_batch = (int64_t)num_heads * seq_k * head_dim;
  a.v_tok = v_head_dim;
  a.v_head = (int64_t)seq_k * v_head_dim;
  a.v_batch = (int64_t)num_heads * seq_k * v_head_dim;
  a.dv = v_head_dim;
  a.out_dtype = out_dtype;
  a.lq = seq_q;
  a.lk = seq_k;
  a.num_seqs = batch;
  a.hq = a.hkv = num_heads;
  a.group = 1;
  a.num_qblocks = (seq_q + kPrefillBM - 1) / kPrefillBM;
  a.causal = causal ? SP_CAUSAL_TOP_LEFT : SP_CAUSAL_NONE;
  a.window_left = -1;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.mask = mask;
  a.mask_b = mask_stride_b;
  a.mask_h = mask_stride_h;
  a.mask_q = mask_stride_q;
  a.inv_scale = 1.f / scale;
  return launch_prefill(a, dtype, head_dim, false, (hipStream_t)stream);
}

int sp_flash_attention_ex(void* out, const void* q, const void* k, const void* v,
                          const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                          int64_t mask_stride_q, int32_t batch, int32_t num_heads, int32_t seq_q,
                          int32_t seq_k, int32_t head_dim, int32_t v_head_dim, float scale,
                          int32_t causal, sp_dtype dtype, sp_dtype out_dtype, void* stream) {
  return flash_attention_impl("sp_flash_attention_ex", out, q, k, v, mask, mask_stride_b,
                              mask_stride_h, mask_stride_q, batch, num_heads, seq_q, seq_k,
                              head_dim, v_head_dim, scale, causal, dtype, out_dtype, stream);
}

int sp_flash_attention(void* out, const void* q, const void* k, const void* v, int32_t batch,
                       int32_t num_heads, int32_t seq_q, int32_t seq_k, int32_t head_dim,
                       float scale, int32_t causal, sp_dtype dtype, void* stream) {
  return flash_attention_impl("sp_flash_attention", out, q, k, v, nullptr, 0, 0, 0, batch,
                              num_heads, seq_q, seq_k, head_dim, head_dim, scale, causal, dtype,
                              dtype, stream);
}

int sp_flash_attention_masked(void* out, const void* q, const void* k, const void* v,
                              const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                              int64_t mask_stride_q, int32_t batch, int32_t num_heads,
                              int32_t seq_q, int32_t seq_k, int32_t head_dim, float scale,
                              int32_t causal, sp_dtype dtype, void* stream) {
  const char* fn = "sp_flash_attention_masked";
  if (!mask && batch > 0 && seq_q > 0 && seq_k > 0)
    return fail(SP_EINVAL, "%s: NULL mask", fn);
  return flash_attention_impl(fn, out, q, k, v, mask, mask_stride_b, mask_stride_h, mask_stride_q,
                              batch, num_heads, seq_q, seq_k, head_dim, head_dim, scale, causal,
                              dtype, dtype, stream);
}

// ---------------------------------------------------------------------------------------------
// PolarQuant compressed paged cache
// ---------------------------------------------------------------------------------------------
int64_t sp_polar_record_bytes(int32_t head_dim) {
  if (head_dim <= 0) return -1;
  return 2 + ((int64_t)head_dim + 1) / 2;
}

static int check_polar_layout(const sp_cache_layout* l, const char* fn) {
  if (int rc = check_layout(l, fn)) return rc;
  if (l->head_dim & 1)
    return fail(SP_EUNSUPPORTED, "%s: a paged PolarQuant pool needs an even head_dim (got %d)",
                fn, l->head_dim);
  if (l->block_size % 4)
    return fail(SP_EUNSUPPORTED,
                "%s: a paged PolarQuant pool needs block_size a multiple of 4 (got %d)", fn,
                l->block_size);
  return SP_OK;
}

static void polar_strides(const sp_cache_layout* l, int64_t* block_stride_b,
                          int64_t* layer_off_b) {
  const int64_t layer_b = (int64_t)l->num_kv_heads * polar_region_bytes(l->block_size, l->head_dim);
  *block_stride_b = layer_b * l->num_layers;
  *layer_off_b = layer_b * l->layer;
}

size_t sp_polar_pool_bytes(const sp_cache_layout* layout) {
  if (check_polar_layout(layout, "sp_polar_pool_bytes")) return 0;
  int64_t stride, off;
  polar_strides(layout, &stride, &off);
  return (size_t)stride * (size_t)layout->num_blocks;
}

int sp_polar_compress(void* records, const void* x, int64_t num_vecs, int32_t head_dim,
                      sp_dtype dtype, void* stream) {
  const char* fn = "sp_polar_compress";
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_vecs < 0 || head_dim <= 0)
    return fail(SP_EINVAL, "%s: num_vecs %lld, head_dim %d", fn, (long long)num_vecs, head_dim);
  if (num_vecs == 0) return SP_OK;
  if (!records || !x) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if ((uintptr_t)x % dtype_size(dtype))
    return fail(SP_EINVAL, "%s: x is not aligned to its element type", fn);
  return launch_polar_compress(records, x, num_vecs, head_dim, dtype, (hipStream_t)stream);
}

int sp_polar_decompress(void* out, const void* records, int64_t num_vecs, int32_t head_dim,
                        sp_dtype dtype, void* stream) {
  const char* fn = "sp_polar_decompress";
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_vecs < 0 || head_dim <= 0)
    return fail(SP_EINVAL, "%s: num_vecs %lld, head_dim %d", fn, (long long)num_vecs, head_dim);
  if (num_vecs == 0) return SP_OK;
  if (!records || !out) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if ((uintptr_t)out % dtype_size(dtype))
    return fail(SP_EINVAL, "%s: out is not aligned to its element type", fn);
  return launch_polar_decompress(out, records, num_vecs, head_dim, dtype, (hipStream_t)stream);
}

int sp_polar_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout,
                       const void* k_new, const void* v_new, int64_t token_stride,
                       int64_t head_stride, const int32_t* slot_mapping, int32_t num_tokens,
                       sp_dtype dtype, void* stream) {
  const char* fn = "sp_polar_kv_append";
  if (int rc = check_polar_layout(layout, fn)) return rc;
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_tokens < 0) return fail(SP_EINVAL, "%s: num_tokens %d < 0", fn, num_tokens);
  if (num_tokens == 0) return SP_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !slot_mapping)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (token_stride < 0 || head_stride < 0) return fail(SP_EINVAL, "%s: negative stride", fn);
  if (((uintptr_t)k_pool | (uintptr_t)v_pool) & 15)
    return fail(SP_EINVAL, "%s: pools must be 16-byte aligned", fn);
  if (((uintptr_t)k_new | (uintptr_t)v_new) % dtype_size(dtype))
    return fail(SP_EINVAL, "%s: k_new / v_new are not aligned to their element type", fn);
  PolarAppendArgs a{};
  a.kpool = (char*)k_pool;
  a.vpool = (char*)v_pool;
  a.knew = (const char*)k_new;
  a.vnew = (const char*)v_new;
  a.tok_stride_e = token_stride;
  a.head_stride_e = head_stride;
  a.slots = slot_mapping;
  polar_strides(layout, &a.block_stride_b, &a.layer_off_b);
  a.num_slots = (int64_t)layout->num_blocks * layout->block_size;
  a.num_tokens = num_tokens;
  a.hkv = layout->num_kv_heads;
  a.head_dim = layout->head_dim;
  a.block_size = layout->block_size;
  return launch_polar_append(a, dtype, (hipStream_t)stream);
}

static int polar_gather_common(const char* fn, void* k_out, void* v_out, const void* k_pool,
                               const void* v_pool, const sp_cache_layout* layout,
                               const int32_t* block_table, int32_t num_table_blocks,
                               int32_t seq_len, int dtype, void* stream) {
  if (int rc = check_polar_layout(layout, fn)) return rc;
  if (seq_len < 0) return fail(SP_EINVAL, "%s: seq_len %d < 0", fn, seq_len);
  if (seq_len == 0) return SP_OK;
  if (!k_out || !v_out || !k_pool || !v_pool || !block_table)
    return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (((uintptr_t)k_pool | (uintptr_t)v_pool) & 15)
    return fail(SP_EINVAL, "%s: pools must be 16-byte aligned", fn);
  if (dtype >= 0 && ((uintptr_t)k_out | (uintptr_t)v_out) % dtype_size((sp_dtype)dtype))
    return fail(SP_EINVAL, "%s: outputs are not aligned to their element type", fn);
  const int64_t needed = ((int64_t)seq_len + layout->block_size - 1) / layout->block_size;
  if (num_table_blocks < needed)
    return fail(SP_EOOB, "%s: seq_len %d needs %lld blocks, the table holds %d", fn, seq_len,
                (long long)needed, num_table_blocks);
  PolarGatherArgs a{};
  a.kout = (char*)k_out;
  a.vout = (char*)v_out;
  a.kpool = (const char*)k_pool;
  a.vpool = (const char*)v_pool;
  a.table = block_table;
  polar_strides(layout, &a.block_stride_b, &a.layer_off_b);
  a.seq_len = seq_len;
  a.hkv = layout->num_kv_heads;
  a.head_dim = layout->head_dim;
  a.block_size = layout->block_size;
  a.num_blocks = layout->num_blocks;
  return launch_polar_gather(a, dtype, (hipStream_t)stream);
}

int sp_polar_kv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                       const sp_cache_layout* layout, const int32_t* block_table,
                       int32_t num_table_blocks, int32_t seq_len, sp_dtype dtype, void* stream) {
  const char* fn = "sp_polar_kv_gather";
  if (int rc = check_dtype(dtype, fn)) return rc;
  return polar_gather_common(fn, k_out, v_out, k_pool, v_pool, layout, block_table,
                             num_table_blocks, seq_len, (int)dtype, stream);
}

int sp_polar_kv_export(void* k_records, void* v_records, const void* k_pool, const void* v_pool,
                       const sp_cache_layout* layout, const int32_t* block_table,
                       int32_t num_table_blocks, int32_t seq_len, void* stream) {
  return polar_gather_common("sp_polar_kv_export", k_records, v_records, k_pool, v_pool, layout,
                             block_table, num_table_blocks, seq_len, -1, stream);
}

int sp_polar_paged_decode(void* out, const void* q, const void* k_pool, const void* v_pool,
                          const sp_cache_layout* layout, const int32_t* block_tables,
                          int32_t max_blocks_per_seq, const int32_t* context_lens,
                          int32_t max_context_len, int32_t num_seqs, int32_t num_q_heads,
                          float scale, int32_t window_left, sp_dtype dtype, void* workspace,
                          size_t workspace_bytes, void* stream) {
  const char* fn = "sp_polar_paged_decode";
  if (dtype != SP_BF16 && dtype != SP_F16)
    return fail(dtype == SP_F32 ? SP_EUNSUPPORTED : SP_EINVAL,
                "%s: dtype %d has no kernel (bf16, f16)", fn, (int)dtype);
  DecodeArgs a{};
  // the PolarQuant split plan (sp_paged_decode_workspace_size covers both plans)
  if (int rc = decode_setup(fn, out, q, k_pool, v_pool, layout, block_tables, max_blocks_per_seq,
                            context_lens, max_context_len, num_seqs, num_q_heads, scale,
                            window_left, dtype, workspace, workspace_bytes, &a, DecodeKind::Polar))
    return rc;
  if (num_seqs == 0) return SP_OK;
  polar_strides(layout, &a.block_stride_b, &a.layer_off_b);
  return launch_polar_decode(a, dtype, layout->head_dim, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------
// Projections
// ---------------------------------------------------------------------------------------------
size_t sp_linear_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return plan_linear(M, K, N, SIZE_MAX).ws_bytes;
}

int sp_linear(void* y, const void* x, const void* w, const void* bias, int64_t M, int64_t K,
              int64_t N, sp_dtype dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "sp_linear";
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (M < 0 || K <= 0 || N <= 0)
    return fail(SP_EINVAL, "%s: M=%lld K=%lld N=%lld", fn, (long long)M, (long long)K,
                (long long)N);
  if (M == 0) return SP_OK;
  if (!y || !x || !w) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (M > kLinearMaxRows || K > INT32_MAX || N > INT32_MAX)
    return fail(SP_EUNSUPPORTED, "%s: M past %lld or K / N past 2^31", fn,
                (long long)kLinearMaxRows);
  const int es = dtype_size(dtype);
  if (((uintptr_t)y | (uintptr_t)bias) % es)
    return fail(SP_EINVAL, "%s: y / bias are not aligned to the element type", fn);
  if (dtype == SP_F32) {
    if (((uintptr_t)x | (uintptr_t)w) % 4)
      return fail(SP_EINVAL, "%s: x / w are not aligned to the element type", fn);
  } else {
    if (K % 8)
      return fail(SP_EUNSUPPORTED, "%s: K = %lld is not a multiple of 8 (16-byte rows)", fn,
                  (long long)K);
    if (((uintptr_t)x | (uintptr_t)w) % 16)
      return fail(SP_EINVAL, "%s: x / w are not 16-byte aligned", fn);
  }
  if (workspace && (uintptr_t)workspace % 16)
    return fail(SP_EINVAL, "%s: workspace is not 16-byte aligned", fn);
  return launch_linear(y, x, w, bias, M, K, N, dtype, workspace, workspace ? workspace_bytes : 0,
                       (hipStream_t)stream);
}

int sp_linear_weight_nk(void* dst, const void* src, int64_t K, int64_t N, sp_dtype dtype,
                        void* stream) {
  const char* fn = "sp_linear_weight_nk";
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (K <= 0 || N <= 0)
    return fail(SP_EINVAL, "%s: K=%lld N=%lld", fn, (long long)K, (long long)N);
  if (!dst || !src) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if (dst == src) return fail(SP_EINVAL, "%s: dst and src must not alias", fn);
  if (K > 65535LL * 32 || N > INT32_MAX)
    return fail(SP_EUNSUPPORTED, "%s: K past 65535 * 32 or N past 2^31", fn);
  if (((uintptr_t)dst | (uintptr_t)src) % dtype_size(dtype))
    return fail(SP_EINVAL, "%s: pointers are not aligned to the element type", fn);
  return launch_weight_transpose(dst, src, K, N, dtype, (hipStream_t)stream);
}


// ---------------------------------------------------------------------------------------------
// QJL codec (KvQuantMethod::QJL, kv_cache.rs:300-324, :371-396, :534-617)
// ---------------------------------------------------------------------------------------------
int64_t sp_qjl_record_bytes(int32_t proj_dim) {
  return proj_dim > 0 ? 2 + ((int64_t)proj_dim + 7) / 8 : 0;
}

int sp_qjl_projection(float* out, int32_t proj_dim, int32_t head_dim) {
  const char* fn = "sp_qjl_projection";
  if (proj_dim <= 0 || head_dim <= 0)
    return fail(SP_EINVAL, "%s: proj_dim %d, head_dim %d", fn, proj_dim, head_dim);
  if (!out) return fail(SP_EINVAL, "%s: NULL output", fn);
  const float scale = sqrtf(1.0f / (float)proj_dim);  // R ~ N(0, 1 / proj_dim)
  qjl_projection_host(out, proj_dim, head_dim, scale);
  return SP_OK;
}

static int check_qjl(const char* fn, int64_t num_vecs, int32_t head_dim, const float* proj,
                     int32_t proj_dim, sp_dtype dtype) {
  if (int rc = check_dtype(dtype, fn)) return rc;
  if (num_vecs < 0 || head_dim <= 0 || proj_dim <= 0)
    return fail(SP_EINVAL, "%s: num_vecs %lld, head_dim %d, proj_dim %d", fn,
                (long long)num_vecs, head_dim, proj_dim);
  if (num_vecs > 0 && !proj) return fail(SP_EINVAL, "%s: NULL projection", fn);
  return SP_OK;
}

int sp_qjl_compress(void* records, const void* x, int64_t num_vecs, int32_t head_dim,
                    const float* projection, int32_t proj_dim, sp_dtype dtype, void* stream) {
  const char* fn = "sp_qjl_compress";
  if (int rc = check_qjl(fn, num_vecs, head_dim, projection, proj_dim, dtype)) return rc;
  if (num_vecs == 0) return SP_OK;
  if (!records || !x) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if ((uintptr_t)x % dtype_size(dtype) || (uintptr_t)projection % 4)
    return fail(SP_EINVAL, "%s: x or projection is not aligned to its element type", fn);
  return launch_qjl_compress(records, x, num_vecs, head_dim, projection, proj_dim, dtype,
                             (hipStream_t)stream);
}

int sp_qjl_decompress(void* out, const void* records, int64_t num_vecs, int32_t head_dim,
                      const float* projection, int32_t proj_dim, sp_dtype dtype, void* stream) {
  const char* fn = "sp_qjl_decompress";
  if (int rc = check_qjl(fn, num_vecs, head_dim, projection, proj_dim, dtype)) return rc;
  if (num_vecs == 0) return SP_OK;
  if (!records || !out) return fail(SP_EINVAL, "%s: NULL pointer argument", fn);
  if ((uintptr_t)out % dtype_size(dtype) || (uintptr_t)projection % 4)
    return fail(SP_EINVAL, "%s: out or projection is not aligned to its element type", fn);
  return launch_qjl_decompress(out, records, num_vecs, head_dim, projection, proj_dim, dtype,
                               (hipStream_t)stream);
}

}  // extern "C"
