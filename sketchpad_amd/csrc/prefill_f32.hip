// fp32 attention prefill (dense, packed variable-length and paged/chunked) on the fp32 MFMA.
//
// Same semantics and entry points as prefill.hip (MultiHeadAttention::forward / forward_cached
// with causal, chunked or sliding-window masks, crates/sketchpad-core/src/transformer.rs:103-271,
// :415-451, crates/sketchpad-llm/src/llama.rs:374-388), for f32 tensors. f32 is the one element
// type the reference's flash_attention runs (crates/sketchpad-cubecl/src/attention.rs:21-25,
// :93-96: cubek's f16/bf16 path is broken) and the reference cache's default, so this is the
// path its f32 callers (the UNet's padded f32 attention, f32 paged caches) take. Scores, softmax
// and accumulation stay fp32 end to end (no 16-bit P), for the reference's 1e-5 relative bar.
//
// Tiling: a workgroup of four waves owns 128 queries of one head (32 per wave) and walks the keys
// in tiles of 32, staged global -> registers -> LDS in a double buffer (one barrier per tile).
// Both products run on v_mfma_f32_32x32x2_f32:
//   S^T[32 keys, 32 q] = K Q^T   k-step s covers dims {s, s + D/2} (lane half hh takes
//                                s + hh D/2): A = K[key l32][s + hh D/2] from LDS (one 16-byte
//                                read feeds four steps), B = Q^T in registers (loaded once).
//                                Lane l ends up with the 16 scores of query l32 for keys
//                                4hh + 8(r/4) + r%4.
//   O^T[32 d, 32 q]   += V^T P^T step r covers keys {4hh + 8(r/4) + r%4 : hh}: B = P^T is the
//                                lane's own score register r, A = V[key][d0 + l32] from LDS.
// fp32 online softmax (FlashAttention-2, Dao 2023) with the row maximum taken per tile; a query
// with no visible key gets zeros.
#include "prefill.hpp"

#include <math.h>

namespace sp {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
// Tile chunks in the native vector type: arrays of HIP's float4 struct are copied with memcpy,
// which keeps them in scratch memory and makes every load wait as soon as it is issued.
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kF32BN = 32;  // keys per tile

template <int D, int DB>
struct F32Cfg {
  // LDS row pitches in floats: K rows are read 16 bytes per lane down a column (pitch = 4 mod 64
  // banks spreads 16 lanes over all banks at D = 64 / 128), V rows by two lane halves four rows
  // apart (4 pitch = 32 mod 64 puts the halves on disjoint banks). V rows hold DB * 32 columns:
  // the PV product works in 32-column blocks, and columns past the value head dim only feed
  // output columns that are never stored.
  static constexpr int PITCH_K = D + 4;
  static constexpr int PITCH_V = DB * 32 + 8;
  static constexpr int TILE_K = kF32BN * PITCH_K;
  static constexpr int BUF = TILE_K + kF32BN * PITCH_V;  // K tile then V tile
  static constexpr int CPR = D / 4;                 // float4 chunks per K row
  static constexpr int CPRV = DB * 8;               // float4 chunks per (padded) V row
  static constexpr int LOADS_K = (kF32BN * CPR + 255) / 256;  // per thread per K tile
  static constexpr int LOADS_V = kF32BN * CPRV / 256;         // per thread per V tile
  static_assert(LOADS_V * 256 == kF32BN * CPRV, "V tile load split");
};

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void swap_halves_f32(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

template <int D, int DB, bool PAGED>
__global__ void __launch_bounds__(256, (DB >= 8 || D >= 256 || (D >= 160 && DB >= 4)) ? 1 : 2) prefill_f32_kernel(PrefillArgs a) {
  using C = F32Cfg<D, DB>;
  constexpr int BN = kF32BN, CPR = C::CPR;
  constexpr int PITCH_K = C::PITCH_K, PITCH_V = C::PITCH_V;
  constexpr int RB = D * 4;  // bytes per K row in memory (paged pools: K and V rows alike)
  static_assert(D % 8 == 0, "the QK steps split a row into two halves of float4 chunks");
  __shared__ __attribute__((aligned(16))) float lds[2][C::BUF];
  const int dv = a.dv;           // value head dim (<= 32 DB, a multiple of 4)
  const int last_v = dv / 4 - 1; // last float4 chunk of a V row in memory

  // ---- workgroup -> (kv head, group member, sequence, query block), heavy query blocks first
  int id = blockIdx.x;
  const int kvh = id % a.hkv;
  id /= a.hkv;
  const int gm = id % a.group;
  id /= a.group;
  const int seq = id % a.num_seqs;
  const int qblk = a.num_qblocks - 1 - id / a.num_seqs;
  const int h = kvh * a.group + gm;

  const int q_begin = a.cu_q ? a.cu_q[seq] : 0;
  const int Lq = a.cu_q ? a.cu_q[seq + 1] - q_begin : a.lq;
  const int qs = qblk * kPrefillBM;
  if (qs >= Lq) return;
  const int qe = min(qs + kPrefillBM, Lq);
  int Lk, k_begin = 0;
  if constexpr (PAGED) {
    Lk = min(a.context_lens[seq], a.max_blocks_per_seq * a.block_size);
  } else {
    k_begin = a.cu_k ? a.cu_k[seq] : 0;
    Lk = a.cu_k ? a.cu_k[seq + 1] - k_begin : a.lk;
  }
  const int pos_off = (a.causal == SP_CAUSAL_TOP_LEFT) ? 0 : Lk - Lq;
  // keys any query of this workgroup can see: [kv_lo, kv_hi)
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  const int t_first = (kv_lo / BN) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;

  // ---- per-sequence base addresses (elements are 4 bytes)
  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 4;
  const int oes = dtype_size((sp_dtype)a.out_dtype);
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) *
          oes;
  const char* kbase = nullptr;
  const char* vbase = nullptr;
  const int32_t* table = nullptr;
  int64_t head_off = 0;
  if constexpr (PAGED) {
    table = a.block_tables + (int64_t)seq * a.max_blocks_per_seq;
    head_off = a.layer_off_b + (int64_t)kvh * a.block_size * RB;
  } else {
    kbase = (const char*)a.k +
            ((a.cu_k ? (int64_t)k_begin * a.kv_tok : (int64_t)seq * a.kv_batch) +
             (int64_t)kvh * a.kv_head) * 4;
    vbase = (const char*)a.v +
            ((a.cu_k ? (int64_t)k_begin * a.v_tok : (int64_t)seq * a.v_batch) +
             (int64_t)kvh * a.v_head) * 4;
  }

  // ---- Q^T operand: query my_q, dims hh D/2 .. hh D/2 + D/2 - 1 (step s reads qreg[s])
  const int wq0 = qs + 32 * wave;
  const int my_q = wq0 + l32;
  float qreg[D / 2];
  {
    const float* qp = (const float*)(qbase + (int64_t)min(my_q, qe - 1) * a.q_tok * 4) + hh * (D / 2);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      const float4 v = my_q < qe ? *(const float4*)(qp + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
      qreg[4 * c] = v.x;
      qreg[4 * c + 1] = v.y;
      qreg[4 * c + 2] = v.z;
      qreg[4 * c + 3] = v.w;
    }
  }

  // ---- tile loads: thread tid moves float4 chunk (tid + 256 u) of the K tile and of the V tile;
  // rows outside [kv_lo, kv_hi) are clamped to a valid row (their scores are masked). Every load
  // is unconditional (a load under a condition makes the compiler wait for all outstanding loads
  // before each tile): chunks past the K tile (head dims 40, 80) repeat its last row, and V
  // chunks past the value head dim repeat the row's last chunk into LDS columns that only feed
  // output columns which are never stored.
  auto row_src = [&](int j, bool is_v) __attribute__((always_inline)) {
    j = min(max(j, kv_lo), kv_hi - 1);
    if constexpr (PAGED) {
      int blk = table[j / a.block_size];
      blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;  // never dereference outside the pool
      return (is_v ? a.vpool : a.kpool) + (int64_t)blk * a.block_stride_b + head_off +
             (int64_t)(j % a.block_size) * RB;
    } else {
      return is_v ? vbase + (int64_t)j * a.v_tok * 4 : kbase + (int64_t)j * a.kv_tok * 4;
    }
  };
  f32x4 kreg[C::LOADS_K], vreg[C::LOADS_V];
  auto k_chunk = [&](int u, int& r, int& c) __attribute__((always_inline)) {
    const int ch = tid + 256 * u;
    r = ch / CPR;
    c = ch % CPR;
    if constexpr (C::LOADS_K * 256 != BN * CPR) {
      if (r >= BN) {
        r = BN - 1;
        c = ch % CPR;  // the same (row, chunk) as another thread: an identical LDS store
      }
    }
  };
  auto load_tile = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < C::LOADS_K; ++u) {
      int r, c;
      k_chunk(u, r, c);
      kreg[u] = *(const f32x4*)(row_src(t0 + r, false) + c * 16);
    }
#pragma unroll
    for (int u = 0; u < C::LOADS_V; ++u) {
      const int ch = tid + 256 * u, r = ch / C::CPRV, c = min(ch % C::CPRV, last_v);
      vreg[u] = *(const f32x4*)(row_src(t0 + r, true) + c * 16);
    }
  };
  auto store_tile = [&](float* buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < C::LOADS_K; ++u) {
      int r, c;
      k_chunk(u, r, c);
      *(f32x4*)(buf + r * PITCH_K + 4 * c) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < C::LOADS_V; ++u) {
      const int ch = tid + 256 * u, r = ch / C::CPRV, c = ch % C::CPRV;
      *(f32x4*)(buf + C::TILE_K + r * PITCH_V + 4 * c) = vreg[u];
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  const int wq_lo = wq0, wq_hi = min(wq0 + 32, qe) - 1;  // this wave's queries (inclusive)
  const bool wave_active = wq_lo < qe;
  const int qpos = my_q + pos_off;
  const float c2 = a.scale_log2;  // > 0 (checked on the host)
  // this lane's row of the additive mask (dense path: the sequence index is the batch index)
  const float* mrow = a.mask ? a.mask + (int64_t)seq * a.mask_b + (int64_t)h * a.mask_h +
                                   (int64_t)min(my_q, qe - 1) * a.mask_q
                             : nullptr;
  // masks only on tiles that start before kv_lo or this wave's window edge, or run past the
  // sequence end or this wave's first causal diagonal
  int mask_below = kv_lo, mask_above = Lk - BN;
  if (a.causal != SP_CAUSAL_NONE) mask_above = min(mask_above, wq_lo + pos_off - BN + 1);
  if (a.window_left >= 0) mask_below = max(mask_below, wq_hi + pos_off - a.window_left);
  mask_below = wave_uniform(mask_below);
  mask_above = wave_uniform(mask_above);

  auto compute_tile = [&](int t0, const float* kl) __attribute__((always_inline)) {
    const float* vl = kl + C::TILE_K;
    // S^T = K Q^T over D/2 steps in two independent accumulator chains; one 16-byte LDS read
    // gives a lane four consecutive steps
    f32x16 s, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = s1[r] = 0.f;
    const float* krow = kl + l32 * PITCH_K + hh * (D / 2);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      const float4 kv = *(const float4*)(krow + 4 * c);
      s = mfma_f32(kv.x, qreg[4 * c], s);
      s1 = mfma_f32(kv.y, qreg[4 * c + 1], s1);
      s = mfma_f32(kv.z, qreg[4 * c + 2], s);
      s1 = mfma_f32(kv.w, qreg[4 * c + 3], s1);
    }
    s += s1;
    // score r of this lane is key t0 + 4hh + 8(r/4) + r%4
    if (a.mask) {
      // additive mask (flash_attention_masked): softmax(q.k scale + mask) = softmax over
      // (q.k + mask / scale) scale. Keys past the sequence end read its last column; their
      // scores are masked below (such tiles always take the mask).
      const int jb = t0 + 4 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = min(jb + 8 * (r >> 2) + (r & 3), Lk - 1);
        s[r] += mrow[key] * a.inv_scale;
      }
    }
    if (t0 < mask_below || t0 > mask_above) {
      int lo = kv_lo, hi = Lk - 1;
      if (a.causal != SP_CAUSAL_NONE) hi = min(hi, qpos);
      if (a.window_left >= 0) lo = max(lo, qpos - a.window_left);
      const int jb = t0 + 4 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = jb + 8 * (r >> 2) + (r & 3);
        s[r] = (key >= lo && key <= hi) ? s[r] : -INFINITY;
      }
    }
    // online softmax for query l32 (both halves of the wave hold its 32 keys)
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = __builtin_fmaxf(mx, s[r]);
    float x0, x1;
    swap_halves_f32(mx, x0, x1);
    const float m_new = __builtin_fmaxf(m_run, __builtin_fmaxf(x0, x1) * c2);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);  // 0 while m_run = -inf
    m_run = m_new;
    float p[16], ls = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c2, -m_use));
      ls += p[r];
    }
    l_run = l_run * alpha + ls;
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    // O^T += V^T P^T: step r covers keys 8(r/4) + r%4 (+ 4 for the upper half)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float* vrow = vl + (4 * hh + 8 * (r >> 2) + (r & 3)) * PITCH_V + l32;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] = mfma_f32(vrow[32 * db], p[r], acc[db]);
    }
  };

  // wave-uniform: does this wave see any key of the tile
  auto visits = [&](int t0) __attribute__((always_inline)) {
    bool v = wave_active;
    if (a.causal != SP_CAUSAL_NONE) v = v && t0 <= wq_hi + pos_off;
    if (a.window_left >= 0) v = v && t0 + BN - 1 >= wq_lo + pos_off - a.window_left;
    return v;
  };

  // Double buffer, one barrier per tile: tile t is read from buf[cur] while tile t+1 sits in
  // registers; the registers go to buf[cur ^ 1], which every wave finished reading before the
  // previous barrier.
  if (t_first < kv_hi) {
    load_tile(t_first);
    store_tile(lds[0]);
  }
  __syncthreads();
  int cur = 0;
  for (int t0 = t_first; t0 < kv_hi; t0 += BN) {
    // unconditional: past the last tile the rows clamp to the last key and the copy lands in
    // the buffer nobody reads again
    load_tile(t0 + BN);
    if (visits(t0)) compute_tile(t0, lds[cur]);
    store_tile(lds[cur ^ 1]);
    __syncthreads();
    cur ^= 1;
  }

  // ---- normalise and store: lane holds O^T[d][query l32], d = 32db + 8(r/4) + 4hh + r%4
  float x0, x1;
  swap_halves_f32(l_run, x0, x1);
  const float l = x0 + x1;
  if (my_q >= qe) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  char* op = obase + (int64_t)my_q * a.o_tok * oes;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d0 = db * 32 + rg * 8 + hh * 4;  // four consecutive columns, all < dv or none
      if (d0 >= dv) continue;
      const float o0 = acc[db][rg * 4] * inv, o1 = acc[db][rg * 4 + 1] * inv;
      const float o2 = acc[db][rg * 4 + 2] * inv, o3 = acc[db][rg * 4 + 3] * inv;
      if (a.out_dtype == SP_F32) {
        *(float4*)(op + d0 * 4) = make_float4(o0, o1, o2, o3);
      } else if (a.out_dtype == SP_BF16) {
        *(uint2*)(op + d0 * 2) =
            make_uint2(f32_to_bf16_bits(o0) | ((uint32_t)f32_to_bf16_bits(o1) << 16),
                       f32_to_bf16_bits(o2) | ((uint32_t)f32_to_bf16_bits(o3) << 16));
      } else {
        *(uint2*)(op + d0 * 2) =
            make_uint2(f32_to_f16_bits(o0) | ((uint32_t)f32_to_f16_bits(o1) << 16),
                       f32_to_f16_bits(o2) | ((uint32_t)f32_to_f16_bits(o3) << 16));
      }
    }
}

template <int D, int DB>
int launch_f32_d(const PrefillArgs& a, bool paged, hipStream_t stream) {
  const int64_t blocks = (int64_t)a.num_qblocks * a.num_seqs * a.hq;
  if (blocks <= 0) return SP_OK;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "prefill: grid of %lld workgroups", (long long)blocks);
  if (paged) {
    // paged pools hold K and V rows of one head dim: only the matching instantiations exist
    if constexpr ((D == 64 && DB == 2) || (D == 128 && DB == 4))
      hipLaunchKernelGGL((prefill_f32_kernel<D, DB, true>), dim3((unsigned)blocks), dim3(256), 0,
                         stream, a);
    else
      return fail(SP_EUNSUPPORTED, "prefill: paged f32 head_dim %d has no kernel", D);
  } else {
    hipLaunchKernelGGL((prefill_f32_kernel<D, DB, false>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, a);
  }
  return check_launch("prefill_f32_kernel");
}

}  // namespace

bool prefill_f32_supports(int head_dim, int v_head_dim, bool paged) {
  if (paged) return (head_dim == 64 || head_dim == 128) && v_head_dim == head_dim;
  const bool dk = head_dim == 40 || head_dim == 64 || head_dim == 80 || head_dim == 128 ||
                  head_dim == 160 || head_dim == 256;
  return dk && v_head_dim > 0 && v_head_dim % 4 == 0 && v_head_dim <= 256;
}

int launch_prefill_f32(const PrefillArgs& a, int head_dim, bool paged, hipStream_t stream) {
  if (!prefill_f32_supports(head_dim, a.dv, paged))
    return fail(SP_EUNSUPPORTED,
                "prefill: f32 head_dim %d / value head_dim %d has no kernel (head_dim 40, 64, 80, "
                "128, 160 or 256 with a value head_dim <= 256, a multiple of 4; paged and packed "
                "K/V: 64 or 128 with equal value head_dim)",
                head_dim, a.dv);
  // V blocks of 32 columns: 2, 4 or 8 (value head dims up to 64, 128, 256)
  const int db = a.dv <= 64 ? 2 : (a.dv <= 128 ? 4 : 8);
  switch (head_dim) {
    case 40: return db == 2 ? launch_f32_d<40, 2>(a, paged, stream)
                   : db == 4 ? launch_f32_d<40, 4>(a, paged, stream)
                             : launch_f32_d<40, 8>(a, paged, stream);
    case 64: return db == 2 ? launch_f32_d<64, 2>(a, paged, stream)
                   : db == 4 ? launch_f32_d<64, 4>(a, paged, stream)
                             : launch_f32_d<64, 8>(a, paged, stream);
    case 80: return db == 2 ? launch_f32_d<80, 2>(a, paged, stream)
                   : db == 4 ? launch_f32_d<80, 4>(a, paged, stream)
                             : launch_f32_d<80, 8>(a, paged, stream);
    case 128: return db == 2 ? launch_f32_d<128, 2>(a, paged, stream)
                    : db == 4 ? launch_f32_d<128, 4>(a, paged, stream)
                              : launch_f32_d<128, 8>(a, paged, stream);
    case 160: return db == 2 ? launch_f32_d<160, 2>(a, paged, stream)
                    : db == 4 ? launch_f32_d<160, 4>(a, paged, stream)
                              : launch_f32_d<160, 8>(a, paged, stream);
    case 256: return db == 2 ? launch_f32_d<256, 2>(a, paged, stream)
                    : db == 4 ? launch_f32_d<256, 4>(a, paged, stream)
                              : launch_f32_d<256, 8>(a, paged, stream);
  }
  return fail(SP_EUNSUPPORTED, "prefill: f32 head_dim %d has no kernel", head_dim);
}

}  // namespace sp
