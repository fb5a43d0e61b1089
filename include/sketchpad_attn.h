/*
 * sketchpad_attn.h — C ABI of the MI355X (gfx950) ragged-batch attention path.
 *
 * The library replaces the attention hot path of rhi-zone/sketchpad:
 *   - the paged KV-cache append      (PagedKvCache::store_kv,  crates/sketchpad-core/src/paged_attention.rs:230-310)
 *   - the paged KV-cache gather      (PagedKvCache::gather_kv, crates/sketchpad-core/src/paged_attention.rs:313-378)
 *   - cached decode attention         (MultiHeadAttention::forward_cached with Sq == 1,
 *                                      crates/sketchpad-core/src/transformer.rs:184-271)
 *   - causal / windowed prefill        (flash_attention, crates/sketchpad-cubecl/src/attention.rs:97-178,
 *                                      and the dense masked path, transformer.rs:103-168, :415-451)
 *   - chunked prefill against a cache  (forward_cached with Sq > 1 and prefill_causal_mask,
 *                                      crates/sketchpad-llm/src/llama.rs:250-260, :374-388)
 *
 * Conventions (all entry points):
 *   - Plain pointers and sizes only. Device pointers are HIP device addresses; the stream is a
 *     hipStream_t passed as void* (NULL = the default stream) of the current HIP device. Work
 *     is enqueued on that stream and nothing synchronises the host.
 *   - Return SP_OK (0) on success, a nonzero sp_status otherwise; sp_last_error() then returns a
 *     thread-local message. Nothing is thrown, aborted or exited across the ABI.
 *   - No entry point allocates device memory. Scratch space is caller-owned (workspace).
 *   - Calls are stateless and re-entrant; two calls that share a workspace must not overlap.
 *     (sp_ragged_paged_attention keeps one side stream and two events per device and caller
 *     stream, made on the first mixed batch issued on that stream; sp_paged_decode_noalloc one
 *     scratch array per device.)
 *
 * Paged pool layout (the reference's, paged_attention.rs:152-155):
 *   pool[num_blocks][num_layers][num_kv_heads][block_size][head_dim], one pool for K, one for V.
 *   A position `pos` of a sequence with block table `table` lives at
 *   block = table[pos / block_size], slot = pos % block_size (BlockTable::get_block/get_slot,
 *   paged_attention.rs:124-132). A slot-mapping entry is block * block_size + slot.
 *
 * Grouped-query attention (repeat_kv, transformer.rs:257-271): query head h reads KV head
 * h / (num_q_heads / num_kv_heads).
 *
 * Attention window: `window_left` = how many keys before the query's own position stay visible;
 * -1 means no limit. The reference's two conventions map to it as:
 *   sliding_window_mask(W)          (transformer.rs:436-451, keys [i-W, i])   -> window_left = W
 *   sliding_window_prefill_mask(W)  (gemma4.rs:1086-1108, keys [p-W+1, p])    -> window_left = W-1
 */
#ifndef SKETCHPAD_ATTN_H
#define SKETCHPAD_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SP_ABI_VERSION 1

typedef enum sp_status {
    SP_OK = 0,
    SP_EINVAL = 1,        /* a size, pointer or combination of arguments is invalid          */
    SP_EUNSUPPORTED = 2,  /* valid, but this build has no kernel for it (dtype, head_dim...) */
    SP_EHIP = 3,          /* the HIP runtime reported an error (launch, device query)          */
    SP_EOOB = 4,          /* an index addresses memory outside the pool / table               */
    SP_ENOSPACE = 5       /* the caller's workspace is smaller than required                  */
} sp_status;

typedef enum sp_dtype {
    SP_F32 = 0,
    SP_BF16 = 1,
    SP_F16 = 2
} sp_dtype;

/* Causal alignment of the prefill mask when a sequence has Lq queries and Lk keys. */
typedef enum sp_causal {
    SP_CAUSAL_NONE = 0,          /* no causal mask (bidirectional)                                  */
    SP_CAUSAL_BOTTOM_RIGHT = 1,  /* query i sits at position Lk-Lq+i: prefill_causal_mask,
                                    llama.rs:374-388 (== causal_mask when Lq == Lk)              */
    SP_CAUSAL_TOP_LEFT = 2       /* query i sits at position i: the flash-attention test oracle,
                                    sketchpad-cubecl/tests/correctness_cpu.rs:1066-1074         */
} sp_causal;

/* Geometry of one layer's view into a paged pool (PagedKvCacheConfig, paged_attention.rs:35-86). */
typedef struct sp_cache_layout {
    int32_t num_blocks;    /* blocks in the pool                                  */
    int32_t num_layers;    /* layers interleaved in every block                   */
    int32_t layer;         /* the layer this call reads or writes (0..num_layers) */
    int32_t num_kv_heads;  /* Hkv                                                 */
    int32_t block_size;    /* tokens per block (BS)                               */
    int32_t head_dim;      /* D                                                   */
} sp_cache_layout;

/* ABI version (SP_ABI_VERSION) and the message of the last failed call on this thread. */
int sp_version(void);
const char* sp_last_error(void);

/*
 * Cache append: scatter new K/V rows into the paged pools through a slot mapping.
 * Replaces PagedKvCache::store_kv + store_single_kv (paged_attention.rs:230-310), batched over
 * any number of sequences: token t of the batch is written to
 *   pool[slot_mapping[t] / BS][layer][h][slot_mapping[t] % BS][:] = new[t, h, :]
 * for every KV head h. The copy is bit-exact. A negative slot skips the token; a slot at or past
 * num_blocks * block_size is skipped by the kernel (never written) — callers validate slots on
 * the host first (the reference panics "Block not allocated", paged_attention.rs:242).
 * k_new / v_new element (t, h, d) lives at t*token_stride + h*head_stride + d (elements), so
 * token-major [T, Hkv, D] input uses (Hkv*D, D) and the reference's head-major [Hkv, T, D] uses
 * (D, T*D).
 */
int sp_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout,
                 const void* k_new, const void* v_new,
                 int64_t token_stride, int64_t head_stride,
                 const int32_t* slot_mapping, int32_t num_tokens,
                 sp_dtype dtype, void* stream);

/*
 * Rotary tables for sp_rope_kv_append, built on the host exactly as the reference builds its
 * caches (RotaryEmbedding::with_base, crates/sketchpad-core/src/rope.rs:60-92), in fp32:
 *   inv_freq[i] = 1 / powf(base, (2i) / head_dim),  angle = p * inv_freq[i],
 *   cos_table[p * head_dim/2 + i] = cosf(angle),   sin_table[...] = sinf(angle)
 * for p < rows, i < head_dim / 2 (the reference stores each value twice, once per element of the
 * pair; these tables keep one per pair). Host memory; copy them to the device once.
 * head_dim must be even and positive, rows >= 0.
 */
int sp_rope_tables(float* cos_table, float* sin_table, int32_t rows, int32_t head_dim,
                   float base);

/*
 * RoPE fused into the cache append. Rotates the new K rows and writes them, with the V rows,
 * into the pools (as sp_kv_append), and rotates Q in place, in one pass. Replaces
 * RotaryEmbedding::forward (rope.rs:115-170) on q and k followed by PagedKvCache::store_kv
 * (paged_attention.rs:230-310), as called from MultiHeadAttention::forward_cached
 * (transformer.rs:221-227). Adjacent dimensions (2i, 2i+1) of token t rotate by the angle of
 * row positions[t] of the tables (rope.rs:145-170, rotate_half maps (x0, x1) to (-x1, x0)):
 *   y[2i] = x[2i] c - x[2i+1] s,   y[2i+1] = x[2i+1] c + x[2i] s
 * in fp32 with each product and the sum rounded (no fused multiply-add), then stored in the
 * element type: bit-identical to the reference's fp32 op sequence for f32; bf16 / f16 round
 * once from the fp32 result.
 *   k_new, v_new : element (t, h, d) at t*token_stride + h*head_stride + d (as sp_kv_append)
 *   q            : [T, num_q_heads, D] with element (t, h, d) at t*q_token_stride +
 *                  h*q_head_stride + d, rotated in place; NULL to skip Q
 *   positions    : [num_tokens] int32 (device), each token's position in its sequence
 *   cos_table, sin_table : device copies of sp_rope_tables(rows = table_rows)
 * A token whose slot is negative or past the pool has its K/V write skipped (as sp_kv_append;
 * its Q is still rotated); a token whose position is outside [0, table_rows) is skipped entirely
 * (K/V not written, Q not rotated). The reference panics on both (paged_attention.rs:242, the
 * cache slice in rope.rs:124-131).
 */
int sp_rope_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout,
                      const void* k_new, const void* v_new,
                      int64_t token_stride, int64_t head_stride,
                      void* q, int64_t q_token_stride, int64_t q_head_stride,
                      int32_t num_q_heads,
                      const int32_t* positions, const int32_t* slot_mapping, int32_t num_tokens,
                      const float* cos_table, const float* sin_table, int32_t table_rows,
                      sp_dtype dtype, void* stream);

/*
 * Cache gather: copy one sequence's first seq_len positions out of the pools into contiguous
 * k_out / v_out of shape [Hkv, seq_len, D]. Replaces PagedKvCache::gather_kv
 * (paged_attention.rs:313-378); seq_len == 0 is a no-op (the reference returns [Hkv, 0, D]).
 * block_table is a device array of num_table_blocks block ids; positions whose block index is
 * past the table make the call fail with SP_EOOB before any launch.
 */
int sp_kv_gather(void* k_out, void* v_out,
                 const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                 const int32_t* block_table, int32_t num_table_blocks, int32_t seq_len,
                 sp_dtype dtype, void* stream);

/*
 * Bytes of workspace sp_paged_decode needs for the given batch shape. max_context_len bounds
 * every context_lens[] entry.
 */
size_t sp_paged_decode_workspace_size(int32_t num_seqs, int32_t num_q_heads,
                                      int32_t max_context_len, int32_t window_left,
                                      const sp_cache_layout* layout);

/*
 * Paged decode attention: one query token per sequence against its paged context.
 * Replaces, for Sq == 1, PagedAttentionCache::update_layer's gather (paged_attention.rs:519-548)
 * followed by repeat_kv + softmax((q k^T) * scale) v (transformer.rs:227-243). Decode applies
 * no mask in the reference (llama.rs:255-260); window_left >= 0 restricts sequence s to keys
 * [context_lens[s]-1-window_left, context_lens[s]) (Mistral window: window_left = W).
 *   q, out         : [num_seqs, num_q_heads, D] contiguous, dtype; q, out, the pools and the
 *                    workspace 16-byte aligned (else SP_EINVAL)
 *   block_tables   : [num_seqs, max_blocks_per_seq] int32 (device)
 *   context_lens   : [num_seqs] int32 (device), each in [0, max_context_len]; the count
 *                    includes the token just appended. A zero-length context yields zeros.
 *   workspace      : device scratch of at least sp_paged_decode_workspace_size() bytes (no
 *                    initialisation needed). Calls that share a workspace must not overlap.
 * Softmax and accumulation are fp32 for every dtype. GQA groups (Hq / Hkv) up to 16, head_dim
 * 64 or 128 (and 256 and 512 for bf16 / f16: Gemma-4's sliding and global layers,
 * gemma4.rs:82-107), any block_size
 * (BlockTable takes any, paged_attention.rs:89-148; one that is not a multiple of 16 makes a
 * 16-token tile span several blocks, each row read from the block its position maps to).
 */
int sp_paged_decode(void* out, const void* q,
                    const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                    const int32_t* block_tables, int32_t max_blocks_per_seq,
                    const int32_t* context_lens, int32_t max_context_len,
                    int32_t num_seqs, int32_t num_q_heads,
                    float scale, int32_t window_left, sp_dtype dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * The logit soft cap of Gemma-4's attention (Gemma4Attention::forward, gemma4.rs:366-377, with
 * attn_logit_softcap = 50, :96): every logit becomes logit_softcap * tanh(logit / logit_softcap),
 * logit = (q . k) * scale, before the mask and the softmax. Each *_softcap entry point below is
 * its namesake with that one argument added after `scale`; logit_softcap == 0 is the namesake
 * itself, > 0 runs at head_dims 256 and 512 on bf16 / f16 tensors (Gemma-4's sliding-window
 * layers, which come with the W-key window of gemma4.rs:1086-1108, window_left = W - 1, and its
 * global layers, causal without a window) and returns SP_EUNSUPPORTED elsewhere; a negative or
 * non-finite cap is SP_EINVAL.
 */
int sp_paged_decode_softcap(void* out, const void* q,
                            const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                            const int32_t* block_tables, int32_t max_blocks_per_seq,
                            const int32_t* context_lens, int32_t max_context_len,
                            int32_t num_seqs, int32_t num_q_heads,
                            float scale, float logit_softcap, int32_t window_left, sp_dtype dtype,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step's append and attention in a single call: sp_kv_append of each sequence's new
 * token followed by sp_paged_decode, with the append done inside the decode kernel. Replaces
 * PagedAttentionCache::update_layer for one new token per sequence (store_kv,
 * paged_attention.rs:230-310, :519-548) followed by the decode attention (transformer.rs:227-243).
 *   k_new, v_new : the step's new token of sequence s, KV head h, at element offset
 *                  s*token_stride + h*head_stride (for [num_seqs, Hkv, D] contiguous:
 *                  token_stride = Hkv*D, head_stride = D); 16-byte aligned, as are the strides
 *                  in bytes.
 * The new token of sequence s is its last position, context_lens[s] - 1: it is written into the
 * pools at the slot its block table gives that position (not written when that block id lies
 * outside the pool, as sp_kv_append skips such a slot) and attended from k_new / v_new in the
 * same launch. Everything else is sp_paged_decode's (same arguments, workspace and results, bit
 * for bit, as sp_kv_append with those slots followed by sp_paged_decode). A sequence with
 * context_lens[s] == 0 has no new token: nothing is written and its output is zeros.
 */
int sp_paged_append_decode(void* out, const void* q, void* k_pool, void* v_pool,
                           const sp_cache_layout* layout, const void* k_new, const void* v_new,
                           int64_t token_stride, int64_t head_stride,
                           const int32_t* block_tables, int32_t max_blocks_per_seq,
                           const int32_t* context_lens, int32_t max_context_len,
                           int32_t num_seqs, int32_t num_q_heads,
                           float scale, int32_t window_left, sp_dtype dtype,
                           void* workspace, size_t workspace_bytes, void* stream);
/* sp_paged_append_decode with Gemma-4's logit soft cap (see sp_paged_decode_softcap). */
int sp_paged_append_decode_softcap(void* out, const void* q, void* k_pool, void* v_pool,
                                   const sp_cache_layout* layout, const void* k_new,
                                   const void* v_new, int64_t token_stride, int64_t head_stride,
                                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* context_lens, int32_t max_context_len,
                                   int32_t num_seqs, int32_t num_q_heads,
                                   float scale, float logit_softcap, int32_t window_left,
                                   sp_dtype dtype, void* workspace, size_t workspace_bytes,
                                   void* stream);

/*
 * sp_paged_decode without a workspace argument: the split partials go to a scratch array the
 * library holds on each GPU it runs on (32 MiB, kept until the process ends), so the call
 * allocates nothing. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Same arguments and results as sp_paged_decode with the workspace it asks for
 * (the same split plan, so the same kernels and merge order). A batch whose dense split plan
 * needs more than 32 MiB of partials returns SP_ENOSPACE before any launch. The figure
 * sp_paged_decode_workspace_size() returns is the larger of the dense and the PolarQuant plans'
 * needs, so it can exceed 32 MiB for a batch that still runs here.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialised by the caller.
 */
int sp_paged_decode_noalloc(void* out, const void* q,
                            const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                            const int32_t* block_tables, int32_t max_blocks_per_seq,
                            const int32_t* context_lens, int32_t max_context_len,
                            int32_t num_seqs, int32_t num_q_heads,
                            float scale, int32_t window_left, sp_dtype dtype, void* stream);

/*
 * Prefill attention over packed variable-length sequences (FlashAttention-2 style, MFMA).
 * Replaces MultiHeadAttention::forward with causal_mask / sliding_window_mask
 * (transformer.rs:103-168, :415-451) and flash_attention (sketchpad-cubecl attention.rs:97-178),
 * for a ragged batch packed into one token stream:
 *   q, out : [total_q, Hq, D] contiguous;  k, v : [total_k, Hkv, D] contiguous
 *   sequence s owns queries cu_seqlens_q[s]..cu_seqlens_q[s+1] and keys
 *   cu_seqlens_k[s]..cu_seqlens_k[s+1] (device int32 arrays of num_seqs + 1 entries; pass the same
 *   array twice for self-attention). max_seqlen_q must bound every sequence's query count.
 *   causal : sp_causal; window_left >= 0 adds the sliding window (see above).
 * Softmax and accumulation are fp32; a query that sees no key gets zeros. f32 (fp32 MFMA, fp32
 * weights: the reference flash_attention's element type), bf16 and f16 (16-bit weights on the
 * bf16/f16 MFMA), head_dim 64 or 128 (and 256 and 512 for bf16 / f16), GQA groups of any size.
 */
int sp_varlen_prefill(void* out, const void* q, const void* k, const void* v,
                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                      int32_t num_seqs, int32_t max_seqlen_q,
                      int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                      float scale, int32_t causal, int32_t window_left,
                      sp_dtype dtype, void* stream);
/* sp_varlen_prefill with Gemma-4's logit soft cap (see sp_paged_decode_softcap). */
int sp_varlen_prefill_softcap(void* out, const void* q, const void* k, const void* v,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int32_t num_seqs, int32_t max_seqlen_q,
                              int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                              float scale, float logit_softcap, int32_t causal,
                              int32_t window_left, sp_dtype dtype, void* stream);

/*
 * Chunked prefill against a paged cache: the new tokens of every sequence attend to that
 * sequence's whole paged context, which already holds them (append first with sp_kv_append).
 * Replaces forward_cached with seq_len > 1 and prefill_causal_mask (llama.rs:250-260, :374-388):
 * sequence s has context_lens[s] keys in the pools and cu_seqlens_q[s+1] - cu_seqlens_q[s] new
 * queries, which sit at the last positions of the context (bottom-right causal).
 *   q, out    : [total_q, Hq, D] contiguous; block_tables [num_seqs, max_blocks_per_seq] (device).
 *   workspace : optional device scratch (16-byte aligned). Batches of few query blocks over long
 *               contexts split each sequence's keys over several workgroups when the workspace
 *               holds their fp32 partials, sp_paged_prefill_workspace_size() bytes for the full
 *               split; a smaller (or NULL) workspace lowers the split (NULL: none). The result
 *               does not depend on whether the keys were split beyond fp32 rounding of the
 *               merge. Calls sharing one workspace must not overlap. Head dims 256 and 512
 *               take no split (their workspace size is 0).
 * Dtypes, head dims and GQA groups as sp_varlen_prefill.
 */
size_t sp_paged_prefill_workspace_size(int32_t num_seqs, int32_t max_seqlen_q,
                                       int32_t num_q_heads, const sp_cache_layout* layout,
                                       int32_t max_blocks_per_seq);
int sp_paged_prefill(void* out, const void* q,
                     const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                     const int32_t* block_tables, int32_t max_blocks_per_seq,
                     const int32_t* cu_seqlens_q, const int32_t* context_lens,
                     int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                     float scale, int32_t window_left, sp_dtype dtype,
                     void* workspace, size_t workspace_bytes, void* stream);
/* sp_paged_prefill with Gemma-4's logit soft cap (see sp_paged_decode_softcap). */
int sp_paged_prefill_softcap(void* out, const void* q,
                             const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                             const int32_t* block_tables, int32_t max_blocks_per_seq,
                             const int32_t* cu_seqlens_q, const int32_t* context_lens,
                             int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                             float scale, float logit_softcap, int32_t window_left,
                             sp_dtype dtype, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * One mixed ragged batch over a paged cache: every sequence's new tokens attend to its whole
 * paged context (append them first with sp_kv_append / sp_rope_kv_append). Sequences
 * [0, num_prefill_seqs) are prompt chunks: chunked prefill (sp_paged_prefill, the bottom-right
 * causal rule of prefill_causal_mask, llama.rs:374-388); sequences [num_prefill_seqs, num_seqs)
 * add one token each: decode (sp_paged_decode, no mask, llama.rs:255-260). Replaces the
 * per-sequence forward_cached calls of one scheduler iteration (transformer.rs:184-254 with
 * start_pos and the mask chosen per sequence as Llama::forward does, llama.rs:247-260). With
 * both groups present the decode runs on a library-owned side stream that belongs to `stream`
 * (one per device and caller stream, created on first use, default priority), forked from
 * `stream` and joined back into it with events, so it overlaps the chunks' prefill; the call is
 * ordered on `stream` like one launch (work after it on `stream` sees both halves), mixed steps
 * on different caller streams do not wait for each other, and the call can be captured into a
 * graph. Past 256 caller streams the library makes no more side streams: later ones run the
 * two halves one after the other on `stream`.
 *   q, out          : [total_q, Hq, D], the chunks' tokens first (num_prefill_tokens of them),
 *                     then one token per decode sequence
 *   cu_seqlens_q    : [num_prefill_seqs + 1] token offsets of the chunks (device); may be NULL
 *                     when num_prefill_seqs == 0
 *   context_lens    : [num_seqs] (device), block_tables [num_seqs, max_blocks_per_seq] (device)
 *   prefill_max_seqlen_q, decode_max_context_len : bounds over the respective groups
 *   workspace       : sp_ragged_attention_workspace_size() bytes: the decode's partials first
 *                     (its need rounded up to 256 bytes), then the prefill's split partials
 *                     (none when the prefill plan does not split). Calls sharing it must not
 *                     overlap.
 */
size_t sp_ragged_attention_workspace_size(int32_t num_seqs, int32_t num_prefill_seqs,
                                          int32_t prefill_max_seqlen_q,
                                          int32_t decode_max_context_len, int32_t num_q_heads,
                                          int32_t window_left, const sp_cache_layout* layout,
                                          int32_t max_blocks_per_seq);
int sp_ragged_paged_attention(void* out, const void* q,
                              const void* k_pool, const void* v_pool,
                              const sp_cache_layout* layout,
                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                              const int32_t* cu_seqlens_q, const int32_t* context_lens,
                              int32_t num_seqs, int32_t num_prefill_seqs,
                              int32_t num_prefill_tokens, int32_t prefill_max_seqlen_q,
                              int32_t decode_max_context_len, int32_t num_q_heads, float scale,
                              int32_t window_left, sp_dtype dtype, void* workspace,
                              size_t workspace_bytes, void* stream);
/* sp_ragged_paged_attention with Gemma-4's logit soft cap on both halves (see
 * sp_paged_decode_softcap). */
int sp_ragged_paged_attention_softcap(void* out, const void* q,
                                      const void* k_pool, const void* v_pool,
                                      const sp_cache_layout* layout,
                                      const int32_t* block_tables, int32_t max_blocks_per_seq,
                                      const int32_t* cu_seqlens_q, const int32_t* context_lens,
                                      int32_t num_seqs, int32_t num_prefill_seqs,
                                      int32_t num_prefill_tokens, int32_t prefill_max_seqlen_q,
                                      int32_t decode_max_context_len, int32_t num_q_heads,
                                      float scale, float logit_softcap, int32_t window_left,
                                      sp_dtype dtype, void* workspace, size_t workspace_bytes,
                                      void* stream);

/*
 * Dense attention on [batch, heads, seq, dim] tensors with every option of the reference's
 * flash_attention_impl (sketchpad-cubecl attention.rs:130-178; FlashAttentionOptions
 * :39-69): q, k [batch, heads, seq_q / seq_k, head_dim], v [batch, heads, seq_k, v_head_dim],
 * out [batch, heads, seq_q, v_head_dim] of out_dtype (FlashAttentionOptions.out_dtype; the
 * reference defaults it to q's dtype), out = softmax(q k^T scale + mask) v with fp32 softmax and
 * accumulation. Equal head counts for q and k/v (the reference has no GQA there). causal != 0
 * masks key j > query i (the reference's test oracle, correctness_cpu.rs:1066-1074, top-left).
 *   mask : optional additive f32 mask (NULL: none; flash_attention_masked's argument),
 *          element (b, h, i, j) at b*mask_stride_b + h*mask_stride_h + i*mask_stride_q + j
 *          (stride 0 broadcasts, as the reference's tests expand one [seq_q, seq_k] mask).
 *          Masked entries are -inf or large negatives; a query whose every key is masked gets
 *          zeros.
 * f32 tensors (the element type the reference's flash_attention runs, attention.rs:21-25):
 * head_dim 40, 64, 80, 128, 160 or 256 (so the SD-1.x UNet's head dims 40 / 80 / 160 run
 * without padding, sketchpad-unet/src/cubecl.rs:256-316), v_head_dim a multiple of 4 up to
 * 256. bf16 / f16 tensors: head_dim == v_head_dim, 64, 128, 256 or 512. out_dtype any of
 * f32 / bf16 / f16.
 * The reference scales by head_dim^-0.5.
 */
int sp_flash_attention_ex(void* out, const void* q, const void* k, const void* v,
                          const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                          int64_t mask_stride_q, int32_t batch, int32_t num_heads,
                          int32_t seq_q, int32_t seq_k, int32_t head_dim, int32_t v_head_dim,
                          float scale, int32_t causal, sp_dtype dtype, sp_dtype out_dtype,
                          void* stream);

/*
 * flash_attention(q, k, v, FlashAttentionOptions{causal}) (sketchpad-cubecl
 * attention.rs:97-104): sp_flash_attention_ex with no mask, v_head_dim = head_dim and out of
 * q's dtype.
 */
int sp_flash_attention(void* out, const void* q, const void* k, const void* v,
                       int32_t batch, int32_t num_heads, int32_t seq_q, int32_t seq_k,
                       int32_t head_dim, float scale, int32_t causal, sp_dtype dtype,
                       void* stream);

/*
 * flash_attention_masked (sketchpad-cubecl attention.rs:119-128): sp_flash_attention_ex with a
 * required mask, v_head_dim = head_dim and out of q's dtype. mask is f32 for every dtype of
 * q / k / v; causal != 0 also applies the j > i mask.
 */
int sp_flash_attention_masked(void* out, const void* q, const void* k, const void* v,
                              const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                              int64_t mask_stride_q, int32_t batch, int32_t num_heads,
                              int32_t seq_q, int32_t seq_k, int32_t head_dim, float scale,
                              int32_t causal, sp_dtype dtype, void* stream);

/*
 * ---- PolarQuant compressed paged cache ----------------------------------------------------
 * KvQuantMethod::PolarQuant of CompressedKvCache (crates/sketchpad-core/src/kv_cache.rs:300-324,
 * :437-532, used at :640-727). A head_dim vector x is stored as a record of
 *   2 bytes   |x| (f32 norm, summed left to right without fused multiply-add) as IEEE binary16,
 *             little endian (f16::from_f32: round to nearest even)
 *   ceil(head_dim/2) bytes of 4-bit two's-complement direction codes
 *             n_j = (x_j * (1/|x|) * 7).round().clamp(-7, 7)  (half away from zero; NaN -> 0),
 *             dimension 2p in the high nibble of byte p, 2p+1 in the low nibble
 * (all codes zero when |x| == 0) and read back as n_j * (|x| / 7), a zero row when the stored
 * norm is 0. Encoding is bit-exact with the reference's polar_quant_compress.
 *
 * Paged pools (one for K, one for V): pool[num_blocks][num_layers][num_kv_heads] regions of
 * block_size * (head_dim/2 + 2) bytes; sp_polar_pool_bytes() gives the size of one pool. Within
 * a region the codes come first (K: [block_size][head_dim/2], token-major; V:
 * [block_size/4][head_dim/2][4], four consecutive tokens interleaved per byte pair), then the
 * block_size binary16 norms. Paged pools need an even head_dim, block_size a multiple of 4 and
 * 16-byte aligned pools; the decode kernel also needs block_size a multiple of 16.
 */

/* Bytes of one record: 2 + ceil(head_dim / 2); -1 when head_dim <= 0. The ratio to an f16 row
 * (2 * head_dim bytes) is KvQuantMethod::PolarQuant.compression_ratio for even head_dim. */
int64_t sp_polar_record_bytes(int32_t head_dim);

/* Bytes of one paged PolarQuant pool for this layout (0 if the layout is not valid for one). */
size_t sp_polar_pool_bytes(const sp_cache_layout* layout);

/*
 * polar_quant_compress / polar_quant_decompress (kv_cache.rs:437-532) on contiguous rows:
 * x [num_vecs, head_dim] (dtype, converted exactly to f32 first) <-> records
 * [num_vecs, sp_polar_record_bytes(head_dim)] bytes. Any head_dim > 0 (odd ones pad the last
 * byte's low nibble with 0). Decompression computes the f32 value and rounds once to dtype.
 */
int sp_polar_compress(void* records, const void* x, int64_t num_vecs, int32_t head_dim,
                      sp_dtype dtype, void* stream);
int sp_polar_decompress(void* out, const void* records, int64_t num_vecs, int32_t head_dim,
                        sp_dtype dtype, void* stream);

/*
 * QJL codec (KvQuantMethod::QJL, kv_cache.rs:300-324, :534-617), the reference's other
 * compressed cache method: 2 + ceil(proj_dim / 8) bytes per vector, the binary16 magnitude
 * then bit k = (R[k,:] . x >= 0) (little-endian within each byte); decompression gives
 * |x| * (pi/2 / proj_dim) * sum_k (+-1)_k R[k,:]. Bit for bit the reference's values.
 *   sp_qjl_projection : fills host memory out[proj_dim * head_dim] with the reference's fixed
 *                       projection R ~ N(0, 1/proj_dim) (its seed-42 LCG + Box-Muller,
 *                       CompressedKvCache::new, kv_cache.rs:371-396, :417-424); copy it to the
 *                       device for the two calls below.
 *   sp_qjl_compress   : x [num_vecs, head_dim] (dtype, converted exactly to f32) -> records
 *                       [num_vecs, sp_qjl_record_bytes(proj_dim)] (qjl_compress, :534-569)
 *   sp_qjl_decompress : records -> out [num_vecs, head_dim] (f32 value rounded once to dtype;
 *                       qjl_decompress, :571-617)
 */
int64_t sp_qjl_record_bytes(int32_t proj_dim);
int sp_qjl_projection(float* out, int32_t proj_dim, int32_t head_dim);
int sp_qjl_compress(void* records, const void* x, int64_t num_vecs, int32_t head_dim,
                    const float* projection, int32_t proj_dim, sp_dtype dtype, void* stream);
int sp_qjl_decompress(void* out, const void* records, int64_t num_vecs, int32_t head_dim,
                      const float* projection, int32_t proj_dim, sp_dtype dtype, void* stream);

/*
 * Encode on append: the PolarQuant form of sp_kv_append (same slot mapping, strides and skip
 * rules). Replaces the compress-and-extend step of CompressedKvCache::update_layer
 * (kv_cache.rs:665-676) for a paged pool and a ragged batch.
 */
int sp_polar_kv_append(void* k_pool, void* v_pool, const sp_cache_layout* layout,
                       const void* k_new, const void* v_new,
                       int64_t token_stride, int64_t head_stride,
                       const int32_t* slot_mapping, int32_t num_tokens,
                       sp_dtype dtype, void* stream);

/*
 * One sequence's first seq_len positions out of PolarQuant pools (rules of sp_kv_gather):
 *   sp_polar_kv_gather : decompressed into k_out / v_out [Hkv, seq_len, D] of dtype — the full
 *                        K / V that CompressedKvCache::update_layer returns (kv_cache.rs:682-724)
 *   sp_polar_kv_export : the records themselves, [Hkv, seq_len, sp_polar_record_bytes(D)] bytes
 *                        (the reference's k_bytes / v_bytes of a batch-1 cache filled in one
 *                        update, kv_cache.rs:670-671)
 * Positions whose block id lies outside the pool give a zero record / zeros.
 */
int sp_polar_kv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool,
                       const sp_cache_layout* layout, const int32_t* block_table,
                       int32_t num_table_blocks, int32_t seq_len, sp_dtype dtype, void* stream);
int sp_polar_kv_export(void* k_records, void* v_records, const void* k_pool, const void* v_pool,
                       const sp_cache_layout* layout, const int32_t* block_table,
                       int32_t num_table_blocks, int32_t seq_len, void* stream);

/*
 * Paged decode attention on PolarQuant pools: sp_paged_decode with every cached key / value read
 * as n_j * (|x| / 7) straight from the codes (same arguments, same workspace size:
 * sp_paged_decode_workspace_size). Replaces the decompress-then-attend step of
 * CompressedKvCache::update_layer + MultiHeadAttention::forward_cached (transformer.rs:227-243).
 * q / out dtype bf16 or f16 (f32 -> SP_EUNSUPPORTED). Scores take q . n exactly in fp32 MFMA
 * accumulation, times |k|/7 and scale; softmax and accumulation are fp32; the probabilities
 * times |v|/7 enter the PV product as bf16.
 */
int sp_polar_paged_decode(void* out, const void* q,
                          const void* k_pool, const void* v_pool, const sp_cache_layout* layout,
                          const int32_t* block_tables, int32_t max_blocks_per_seq,
                          const int32_t* context_lens, int32_t max_context_len,
                          int32_t num_seqs, int32_t num_q_heads,
                          float scale, int32_t window_left, sp_dtype dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * ---- Projections on either side of the path ------------------------------------------------
 * y[M, N] = x[M, K] . w[N, K]^T (+ bias[N]): burn's nn::Linear as MultiHeadAttention applies it
 * for q_proj / k_proj / v_proj (transformer.rs:196-208) and o_proj (:249-253). The weight is
 * taken [out, in] = [N, K] (K contiguous, the PyTorch / Hugging Face layout); burn stores it
 * [in, out] = [K, N], which sp_linear_weight_nk turns into [N, K] once at load time.
 * Row-major contiguous x, w, y; dtype f32 / bf16 / f16. The product accumulates in fp32 and is
 * rounded once to dtype (the reference upcasts f16 activations to f32 for these projections and
 * casts back); a bias is then added in fp32 and rounded again (matmul, then + bias, as two ops).
 * bias may be NULL. bf16 / f16: K % 8 == 0 and x, w 16-byte aligned (else SP_EUNSUPPORTED /
 * SP_EINVAL); M <= 65535 * 64. Hand-written MFMA kernels; no library GEMM is called.
 *   workspace : optional device scratch (16-byte aligned) for split-K partials. Skinny shapes
 *               (few output tiles, long K) split K over workgroups when the workspace holds
 *               the fp32 partials, sp_linear_workspace_size(M, K, N) bytes for the full split;
 *               a smaller (or NULL) workspace caps the split. Partials are summed in a fixed
 *               order: the result is a deterministic function of the inputs, the shape and
 *               workspace_bytes. Calls sharing one workspace must not overlap.
 */
size_t sp_linear_workspace_size(int64_t M, int64_t K, int64_t N);
int sp_linear(void* y, const void* x, const void* w, const void* bias,
              int64_t M, int64_t K, int64_t N, sp_dtype dtype,
              void* workspace, size_t workspace_bytes, void* stream);

/*
 * dst[N, K] = src[K, N]^T: burn's [in, out] Linear weight (transformer.rs:75-86 builds the
 * projections with LinearConfig; burn keeps the weight as [d_input, d_output]) into sp_linear's
 * [out, in].
 * One pass, done once when weights are loaded; dst and src must not alias.
 */
int sp_linear_weight_nk(void* dst, const void* src, int64_t K, int64_t N, sp_dtype dtype,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SKETCHPAD_ATTN_H */
