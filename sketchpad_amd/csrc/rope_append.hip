// Rotary position embedding fused into the paged KV-cache append, for gfx950.
//
// Semantics (reference: RotaryEmbedding::forward / apply_rotary / rotate_half,
// crates/sketchpad-core/src/rope.rs:115-170, applied to q and k before the cache update at
// crates/sketchpad-core/src/transformer.rs:221-227; the append is PagedKvCache::store_kv,
// crates/sketchpad-core/src/paged_attention.rs:230-310): adjacent dimensions (2i, 2i+1) of a
// row at position p rotate by the angle whose cosine / sine are cos_t[p][i] / sin_t[p][i]:
//   y[2i]   = x[2i]   * c - x[2i+1] * s
//   y[2i+1] = x[2i+1] * c + x[2i]   * s
// computed in fp32 as two products and one sum, each rounded (the reference's
// x * cos + rotate_half(x) * sin; no fused multiply-add), then stored in the element type.
// K rows are rotated on their way into the pool, V rows copied, and Q rows (optional) rotated in
// place. A token whose slot or position is invalid is skipped (nothing written).
//
// Memory-bound: one thread moves one VB-byte chunk of a (token, head) row; consecutive threads
// take consecutive chunks of a row so every wave reads and writes contiguous rows. The cos / sin
// rows of a token are read once per chunk and stay in L1/L2 across the token's heads.
#include "rope_append.hpp"

namespace sp {

template <typename T, int VB> struct RopeVec;
template <typename T> struct RopeVec<T, 16> { using V = uint4; };
template <typename T> struct RopeVec<T, 8> { using V = uint2; };
template <typename T> struct RopeVec<T, 4> { using V = uint32_t; };

// Rotate the element pairs of one VB-byte chunk in place (registers).
template <typename T, int VB>
__device__ __forceinline__ void rope_chunk(char* buf, const float* __restrict__ c,
                                           const float* __restrict__ s) {
#pragma clang fp contract(off)
  constexpr int E = VB / Elem<T>::bytes;  // elements in the chunk (even)
#pragma unroll
  for (int j = 0; j < E / 2; ++j) {
    const float x0 = Elem<T>::load(buf, 2 * j);
    const float x1 = Elem<T>::load(buf, 2 * j + 1);
    const float cj = c[j], sj = s[j];
    const float y0 = x0 * cj + (-x1) * sj;
    const float y1 = x1 * cj + x0 * sj;
    Elem<T>::store(buf, 2 * j, y0);
    Elem<T>::store(buf, 2 * j + 1, y1);
  }
}

template <typename T, int VB>
__global__ void __launch_bounds__(256) rope_kv_append_kernel(RopeAppendArgs a) {
  using V = typename RopeVec<T, VB>::V;
  constexpr int ES = Elem<T>::bytes;
  constexpr int E = VB / ES;  // elements per chunk
  const uint32_t cpr = a.head_dim / E;            // chunks per row
  const uint32_t rows = a.hkv + (a.q ? a.hq : 0);  // K/V rows first, then Q rows
  const uint32_t total = (uint32_t)a.num_tokens * rows * cpr;  // < 2^31 (host splits launches)
  const int half = a.head_dim / 2;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += gridDim.x * blockDim.x) {
    const int ch = (int)(i % cpr);
    const uint32_t tr = i / cpr;
    const int r = (int)(tr % rows);
    const int t = (int)(tr / rows);
    const int pos = a.positions[t];
    if (pos < 0 || pos >= a.table_rows) continue;
    const float* ct = a.cos_t + (int64_t)pos * half + ch * (E / 2);
    const float* st = a.sin_t + (int64_t)pos * half + ch * (E / 2);
    float cv[E / 2], sv[E / 2];
#pragma unroll
    for (int j = 0; j < E / 2; ++j) {
      cv[j] = ct[j];
      sv[j] = st[j];
    }
    if (r < a.hkv) {
      const int32_t slot = a.slots[t];
      if (slot < 0 || (int64_t)slot >= a.num_slots) continue;
      const int blk = slot / a.block_size, sl = slot - blk * a.block_size;
      const int64_t src = (int64_t)t * a.kv_tok_b + (int64_t)r * a.kv_head_b + (int64_t)ch * VB;
      const int64_t dst = (int64_t)blk * a.block_stride_b + a.layer_off_b +
                          ((int64_t)r * a.block_size + sl) * a.head_dim * ES + (int64_t)ch * VB;
      V kx = *(const V*)(a.knew + src);
      const V vx = *(const V*)(a.vnew + src);
      rope_chunk<T, VB>((char*)&kx, cv, sv);
      *(V*)(a.kpool + dst) = kx;
      *(V*)(a.vpool + dst) = vx;
    } else {
      const int h = r - a.hkv;
      char* qp = a.q + (int64_t)t * a.q_tok_b + (int64_t)h * a.q_head_b + (int64_t)ch * VB;
      V qx = *(const V*)qp;
      rope_chunk<T, VB>((char*)&qx, cv, sv);
      *(V*)qp = qx;
    }
  }
}

template <typename T, int VB>
static void launch_tv(const RopeAppendArgs& a, hipStream_t stream) {
  constexpr int E = VB / Elem<T>::bytes;
  const int rows = a.hkv + (a.q ? a.hq : 0);
  const int64_t items = (int64_t)a.num_tokens * rows * (a.head_dim / E);
  int64_t blocks = (items + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;  // grid-stride beyond this
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((rope_kv_append_kernel<T, VB>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     a);
}

template <typename T>
static int launch_t(const RopeAppendArgs& a, int64_t align_mask, hipStream_t stream) {
  constexpr int ES = Elem<T>::bytes;
  // widest chunk that every row start and stride allows, at least one element pair
  if ((align_mask & 15) == 0 && (a.head_dim * ES) % 16 == 0) {
    launch_tv<T, 16>(a, stream);
  } else if ((align_mask & 7) == 0 && (a.head_dim * ES) % 8 == 0) {
    launch_tv<T, 8>(a, stream);
  } else {
    if constexpr (ES == 2) {
      if ((align_mask & 3) == 0) {
        launch_tv<T, 4>(a, stream);
        return check_launch("rope_kv_append_kernel");
      }
    }
    return fail(SP_EINVAL, "rope_kv_append: rows must be aligned to an element pair");
  }
  return check_launch("rope_kv_append_kernel");
}

static int launch_chunk(const RopeAppendArgs& a, sp_dtype dtype, hipStream_t stream) {
  int64_t mask = a.kv_tok_b | a.kv_head_b | a.block_stride_b | a.layer_off_b |
                 (int64_t)(uintptr_t)a.kpool | (int64_t)(uintptr_t)a.vpool |
                 (int64_t)(uintptr_t)a.knew | (int64_t)(uintptr_t)a.vnew;
  if (a.q) mask |= a.q_tok_b | a.q_head_b | (int64_t)(uintptr_t)a.q;
  switch (dtype) {
    case SP_F32: return launch_t<float>(a, mask, stream);
    case SP_BF16: return launch_t<bf16_t>(a, mask, stream);
    case SP_F16: return launch_t<f16_t>(a, mask, stream);
  }
  return fail(SP_EUNSUPPORTED, "rope_kv_append: dtype %d has no kernel", (int)dtype);
}

int launch_rope_kv_append(const RopeAppendArgs& a, sp_dtype dtype, hipStream_t stream) {
  // The kernel indexes work items with 32 bits: launch at most 2^30 items' worth of tokens at a
  // time (items per token = rows * head_dim / 2 at the narrowest chunk, one element pair).
  const int64_t per_token = (int64_t)(a.hkv + (a.q ? a.hq : 0)) * (a.head_dim / 2);
  const int64_t max_tokens = per_token > 0 ? ((int64_t)1 << 30) / per_token : a.num_tokens;
  if (max_tokens < 1) return fail(SP_EUNSUPPORTED, "rope_kv_append: rows too wide");
  for (int64_t t0 = 0; t0 < a.num_tokens; t0 += max_tokens) {
    RopeAppendArgs c = a;
    c.num_tokens = (int)((a.num_tokens - t0 < max_tokens) ? a.num_tokens - t0 : max_tokens);
    c.knew = a.knew + t0 * a.kv_tok_b;
    c.vnew = a.vnew + t0 * a.kv_tok_b;
    if (a.q) c.q = a.q + t0 * a.q_tok_b;
    c.positions = a.positions + t0;
    c.slots = a.slots + t0;
    if (int rc = launch_chunk(c, dtype, stream)) return rc;
  }
  return SP_OK;
}

}  // namespace sp
