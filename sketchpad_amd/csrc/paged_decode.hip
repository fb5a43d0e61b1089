// Split-K paged decode attention for gfx950.
//
// Semantics (reference: MultiHeadAttention::forward_cached with one new token,
// crates/sketchpad-core/src/transformer.rs:227-243, fed by PagedAttentionCache::update_layer,
// crates/sketchpad-core/src/paged_attention.rs:519-548): for every sequence s and query head h,
//   out[s,h,:] = softmax_j( (q[s,h,:] . K[s, h/G, j, :]) * scale ) @ V[s, h/G, j, :]
// over keys j in [start, L_s), start = 0 or L_s-1-window_left; fp32 softmax and accumulation.
//
// Work decomposition: one workgroup of four waves per (split, KV head, sequence). A split is
// `tps` consecutive tiles of TT tokens (TT = 16 for GQA groups up to 4). The GQA group's query
// heads are all served by the same workgroup, so every K/V byte is read from HBM exactly once.
// Each wave takes every fourth tile of the split and runs its own online softmax:
//   1. the tile's K and V rows (TT x D each, contiguous inside one pool block) are loaded with
//      16-byte per-lane loads (a wave instruction covers 1 KiB contiguous) into registers, one
//      tile ahead of the compute, then staged in LDS with a 16-byte row pad (bank-conflict free);
//   2. lane (head g, token t[, part]) computes the full q_g . k_t from LDS (v_dot2_f32_bf16 for
//      16-bit types), so no cross-lane reduction is needed for the scores;
//   3. per-head tile max/exp2 with shuffles inside the head's lane group, p written to LDS;
//   4. lane (head g, dim chunk) accumulates p_t * V[t, chunk] over the tile's tokens.
// The four waves are merged in LDS at the end. A sequence that fits in one split writes its
// output directly; otherwise each split writes (m, l, acc[D]) and decode_combine_kernel merges.
#include "paged_decode.hpp"

#include <math.h>

namespace sp {

template <int GP> struct DecodeShape {
  static constexpr int TT = GP <= 4 ? 16 : 64 / GP;  // tokens per tile
  static constexpr int LPH = 64 / GP;                // lanes per head
  static constexpr int LPS = LPH / TT;               // lanes per score
};

// Copy BYTES (4, 8 or 16) from LDS into 32-bit words.
template <int BYTES>
__device__ __forceinline__ void lds_words(const char* p, uint32_t* w) {
  if constexpr (BYTES == 16) {
    const uint4 v = *(const uint4*)p;
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BYTES == 8) {
    const uint2 v = *(const uint2*)p;
    w[0] = v.x; w[1] = v.y;
  } else {
    static_assert(BYTES == 4, "LDS chunk must be 4, 8 or 16 bytes");
    w[0] = *(const uint32_t*)p;
  }
}

template <typename T, int D, int GP>
__global__ void __launch_bounds__(64 * kDecodeWaves) paged_decode_kernel(DecodeArgs a) {
  using S = DecodeShape<GP>;
  constexpr int TT = S::TT, LPH = S::LPH, LPS = S::LPS;
  constexpr int ES = Elem<T>::bytes;
  constexpr bool kF32 = (ES == 4);
  constexpr int RB = D * ES;              // bytes per K/V row
  constexpr int RBP = RB + 16;            // LDS row pitch (pad breaks the 256-byte bank stride)
  constexpr int NL = TT * RB / 1024;      // 16-byte loads per lane per tile (K or V)
  constexpr int SEG = D / LPS;            // dims per score lane
  constexpr int QW = SEG * ES / 4;        // 32-bit words of q held per lane
  constexpr int DPL = D / LPH;            // dims per accumulation lane
  constexpr int PVB = DPL * ES;           // bytes of one V row read by one lane
  constexpr int WAVE_LDS = 2 * TT * RBP + GP * TT * 4;
  static_assert(TT * RB % 1024 == 0 && NL >= 1, "tile must be a whole number of wave loads");
  static_assert(SEG * ES % 16 == 0, "score segment must be 16-byte aligned");
  static_assert(DPL >= 1, "head_dim too small for this group");
  static_assert(kDecodeWaves * GP * (D + 2) * 4 <= kDecodeWaves * WAVE_LDS, "merge area");

  __shared__ __attribute__((aligned(16))) char smem[kDecodeWaves * WAVE_LDS];

  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform(threadIdx.x >> 6);
  const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int G = a.group;

  int L = a.context_lens[seq];
  L = min(L, min(a.max_context_len, a.max_blocks_per_seq * a.block_size));
  if (L <= 0) {
    if (split == 0) {
      for (int i = threadIdx.x; i < G * D; i += blockDim.x)
        Elem<T>::store(a.out, ((int64_t)seq * a.hq + kvh * G) * D + i, 0.f);
    }
    return;
  }
  const int start_tok = a.window_left >= 0 ? max(0, L - 1 - a.window_left) : 0;
  const int first_tile = start_tok / TT, last_tile = (L - 1) / TT;
  const int nsplit = (last_tile - first_tile + a.tps) / a.tps;
  if (split >= nsplit) return;
  const int t_begin = first_tile + split * a.tps;
  const int t_end = min(t_begin + a.tps, last_tile + 1);

  // Lane roles: score lane (head hs, token tok_s, part) and accumulation lane (head hs, chunk dc).
  const int hs = lane / LPH;
  const int rem = lane % LPH;
  const int tok_s = rem / LPS;
  const int part = rem % LPS;
  const int dc = rem;
  const int hq_lane = kvh * G + min(hs, G - 1);

  // q segment of this score lane, as raw 32-bit words.
  uint32_t qw[QW];
  {
    const char* qp = (const char*)a.q + (((int64_t)seq * a.hq + hq_lane) * D + part * SEG) * ES;
#pragma unroll
    for (int i = 0; i < QW / 4; ++i) {
      const uint4 v = ((const uint4*)qp)[i];
      qw[4 * i + 0] = v.x; qw[4 * i + 1] = v.y; qw[4 * i + 2] = v.z; qw[4 * i + 3] = v.w;
    }
  }

  char* lds_k = smem + wave * WAVE_LDS;
  char* lds_v = lds_k + TT * RBP;
  float* lds_p = (float*)(lds_v + TT * RBP);

  const int32_t* table = a.block_tables + (int64_t)seq * a.max_blocks_per_seq;
  const int64_t head_off = a.layer_off_b + (int64_t)kvh * a.block_size * RB;

  uint4 kr[NL], vr[NL];
  bool next_ok = false;
  auto load_tile = [&](int t) {
    const int pos0 = t * TT;
    const int blk = table[pos0 / a.block_size];
    next_ok = blk >= 0 && blk < a.num_blocks;
    const int64_t base = (int64_t)(next_ok ? blk : 0) * a.block_stride_b + head_off +
                         (int64_t)(pos0 % a.block_size) * RB;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int off = (i * 64 + lane) * 16;
      const int pos = pos0 + off / RB;
      if (next_ok && pos >= start_tok && pos < L) {
        kr[i] = *(const uint4*)(a.kpool + base + off);
        vr[i] = *(const uint4*)(a.vpool + base + off);
      } else {
        kr[i] = make_uint4(0, 0, 0, 0);
        vr[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;

  int t = t_begin + wave;
  if (t < t_end) load_tile(t);
  for (; t < t_end; t += kDecodeWaves) {
    const bool tile_ok = next_ok;
    // Stage the tile in LDS, then start fetching the next one.
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int off = (i * 64 + lane) * 16;
      const int lds_off = (off / RB) * RBP + off % RB;
      *(uint4*)(lds_k + lds_off) = kr[i];
      *(uint4*)(lds_v + lds_off) = vr[i];
    }
    wave_lds_sync();
    if (t + kDecodeWaves < t_end) load_tile(t + kDecodeWaves);

    // Score of (head hs, token tok_s) over this lane's dims.
    float s = 0.f;
    {
      const char* kp = lds_k + tok_s * RBP + part * SEG * ES;
#pragma unroll
      for (int i = 0; i < QW / 4; ++i) {
        uint32_t kw[4];
        lds_words<16>(kp + 16 * i, kw);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (kF32)
            s = fmaf(__uint_as_float(qw[4 * i + j]), __uint_as_float(kw[j]), s);
          else
            s = Dot2<T>::fma(qw[4 * i + j], kw[j], s);
        }
      }
    }
    if constexpr (LPS > 1) s = group_sum<LPS>(s);
    const int pos = t * TT + tok_s;
    const bool valid = tile_ok && pos >= start_tok && pos < L;
    s = valid ? s * a.scale_log2 : -INFINITY;

    const float m_tile = group_max<LPH>(s);
    const float m_new = fmaxf(m_run, m_tile);
    const float alpha = (m_run == -INFINITY) ? 0.f : exp2f(m_run - m_new);
    const float p = valid ? exp2f(s - m_new) : 0.f;
    l_run = l_run * alpha + (part == 0 ? p : 0.f);
    m_run = m_new;
    if (part == 0) lds_p[hs * TT + tok_s] = p;
    wave_lds_sync();

    // acc[hs, dc*DPL ..] = alpha * acc + sum_t p_t * V[t, dc*DPL ..]
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int t4 = 0; t4 < TT; t4 += 4) {
      const float4 p4 = *(const float4*)(lds_p + hs * TT + t4);
      const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const char* vp = lds_v + (t4 + j) * RBP + dc * PVB;
        if constexpr (kF32) {
          constexpr int NW = DPL;  // one word per element
          uint32_t w[NW];
          if constexpr (PVB >= 16) {
#pragma unroll
            for (int c = 0; c < PVB / 16; ++c) lds_words<16>(vp + 16 * c, w + 4 * c);
          } else {
            lds_words<PVB>(vp, w);
          }
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[e] = fmaf(pv[j], __uint_as_float(w[e]), acc[e]);
        } else if constexpr (PVB >= 4) {
          constexpr int NW = PVB / 4;
          uint32_t w[NW];
          if constexpr (PVB >= 16) {
#pragma unroll
            for (int c = 0; c < PVB / 16; ++c) lds_words<16>(vp + 16 * c, w + 4 * c);
          } else {
            lds_words<PVB>(vp, w);
          }
#pragma unroll
          for (int e = 0; e < NW; ++e) {
            acc[2 * e] = fmaf(pv[j], Dot2<T>::lo(w[e]), acc[2 * e]);
            acc[2 * e + 1] = fmaf(pv[j], Dot2<T>::hi(w[e]), acc[2 * e + 1]);
          }
        } else {
          acc[0] = fmaf(pv[j], Elem<T>::load(vp, 0), acc[0]);
        }
      }
    }
    wave_lds_sync();
  }

  // Merge the four waves' (m, l, acc) in LDS.
  l_run = group_sum<LPH>(l_run);
  __syncthreads();
  float* cm = (float*)smem;                  // [waves][GP]
  float* cl = cm + kDecodeWaves * GP;        // [waves][GP]
  float* ca = cl + kDecodeWaves * GP;        // [waves][GP][D]
  if (rem == 0) {
    cm[wave * GP + hs] = m_run;
    cl[wave * GP + hs] = l_run;
  }
#pragma unroll
  for (int e = 0; e < DPL; ++e) ca[(wave * GP + hs) * D + dc * DPL + e] = acc[e];
  __syncthreads();

  for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
    const int h = i / D, d = i % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, cm[w * GP + h]);
    float lsum = 0.f, accsum = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecodeWaves; ++w) {
        const float mw = cm[w * GP + h];
        const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
        lsum = fmaf(cl[w * GP + h], f, lsum);
        accsum = fmaf(ca[(w * GP + h) * D + d], f, accsum);
      }
    }
    const int hq = kvh * G + h;
    if (nsplit == 1) {
      Elem<T>::store(a.out, ((int64_t)seq * a.hq + hq) * D + d, lsum > 0.f ? accsum / lsum : 0.f);
    } else {
      float* pp = a.partials + (((int64_t)seq * a.hq + hq) * a.max_splits + split) * (D + 4);
      if (d == 0) {
        pp[0] = M;
        pp[1] = lsum;
      }
      pp[4 + d] = accsum;
    }
  }
}

// Merge the per-split partials of sequences that needed more than one split.
template <typename T, int D, int TT>
__global__ void __launch_bounds__(D) decode_combine_kernel(DecodeArgs a) {
  const int hq = blockIdx.x, seq = blockIdx.y, d = threadIdx.x;
  int L = a.context_lens[seq];
  L = min(L, min(a.max_context_len, a.max_blocks_per_seq * a.block_size));
  if (L <= 0) return;
  const int start_tok = a.window_left >= 0 ? max(0, L - 1 - a.window_left) : 0;
  const int nsplit = ((L - 1) / TT - start_tok / TT + a.tps) / a.tps;
  if (nsplit <= 1) return;
  const float* pp = a.partials + ((int64_t)seq * a.hq + hq) * a.max_splits * (D + 4);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, pp[s * (D + 4)]);
  float lsum = 0.f, accsum = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ms = pp[s * (D + 4)];
      const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
      lsum = fmaf(pp[s * (D + 4) + 1], f, lsum);
      accsum = fmaf(pp[s * (D + 4) + 4 + d], f, accsum);
    }
  }
  Elem<T>::store(a.out, ((int64_t)seq * a.hq + hq) * D + d, lsum > 0.f ? accsum / lsum : 0.f);
}

DecodePlan plan_decode(int num_seqs, int hq, int hkv, int head_dim, int max_context_len,
                       int window_left) {
  DecodePlan p{};
  p.group = hkv > 0 ? hq / hkv : 0;
  p.gp = decode_group_pow2(p.group < 1 ? 1 : p.group);
  p.tt = decode_tile_tokens(p.gp);
  int max_tiles = (max_context_len + p.tt - 1) / p.tt;
  if (window_left >= 0) {
    const int wt = (window_left + 1 + p.tt - 1) / p.tt + 1;  // a window straddles one extra tile
    if (wt < max_tiles) max_tiles = wt;
  }
  p.max_tiles = max_tiles < 1 ? 1 : max_tiles;
  // Tiles per split: 16 (4 per wave) unless the batch is too small to fill 256 CUs.
  int tps = 16;
  const char* env = getenv("SP_DECODE_TPS");
  if (env && atoi(env) > 0) {
    tps = atoi(env);
  } else {
    const int64_t units = (int64_t)num_seqs * (hkv > 0 ? hkv : 1);
    while (tps > kDecodeWaves && units * ((p.max_tiles + tps - 1) / tps) < 2048) tps >>= 1;
  }
  p.tps = tps;
  p.max_splits = (p.max_tiles + tps - 1) / tps;
  p.ws_bytes = p.max_splits > 1
                   ? (size_t)num_seqs * hq * p.max_splits * (head_dim + 4) * sizeof(float)
                   : 0;
  return p;
}

template <typename T, int D, int GP>
static void launch_typed(const DecodeArgs& a, int nsplit_grid, hipStream_t stream) {
  const dim3 grid(nsplit_grid, a.hkv, a.num_seqs);
  hipLaunchKernelGGL((paged_decode_kernel<T, D, GP>), grid, dim3(64 * kDecodeWaves), 0, stream, a);
  if (a.max_splits > 1) {
    hipLaunchKernelGGL((decode_combine_kernel<T, D, DecodeShape<GP>::TT>), dim3(a.hq, a.num_seqs),
                       dim3(D), 0, stream, a);
  }
}

template <typename T, int D>
static int launch_d(const DecodeArgs& a, int gp, hipStream_t stream) {
  switch (gp) {
    case 1: launch_typed<T, D, 1>(a, a.max_splits, stream); break;
    case 2: launch_typed<T, D, 2>(a, a.max_splits, stream); break;
    case 4: launch_typed<T, D, 4>(a, a.max_splits, stream); break;
    case 8: launch_typed<T, D, 8>(a, a.max_splits, stream); break;
    default: return fail(SP_EUNSUPPORTED, "paged decode: GQA group %d has no kernel", a.group);
  }
  return check_launch("paged_decode_kernel");
}

template <typename T>
static int launch_t(const DecodeArgs& a, int head_dim, int gp, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_d<T, 64>(a, gp, stream);
    case 128: return launch_d<T, 128>(a, gp, stream);
    default: return fail(SP_EUNSUPPORTED, "paged decode: head_dim %d has no kernel", head_dim);
  }
}

int launch_paged_decode(const DecodeArgs& a, sp_dtype dtype, int head_dim, int gp,
                        hipStream_t stream) {
  switch (dtype) {
    case SP_F32: return launch_t<float>(a, head_dim, gp, stream);
    case SP_BF16: return launch_t<bf16_t>(a, head_dim, gp, stream);
    case SP_F16: return launch_t<f16_t>(a, head_dim, gp, stream);
  }
  return fail(SP_EUNSUPPORTED, "paged decode: dtype %d has no kernel", (int)dtype);
}

}  // namespace sp
