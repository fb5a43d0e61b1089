// Causal / windowed attention prefill over packed variable-length sequences, on gfx950 MFMA.
//
// Semantics (reference: MultiHeadAttention::forward / forward_cached with a causal or sliding
// window mask, crates/sketchpad-core/src/transformer.rs:103-168, :184-271, :415-451; the chunked
// prefill mask of crates/sketchpad-llm/src/llama.rs:374-388; flash_attention,
// crates/sketchpad-cubecl/src/attention.rs:97-178): for query i of a sequence with Lq queries and
// Lk keys, sitting at position p = i + (Lk - Lq) (bottom-right) or p = i (top-left),
//   out[i, h, :] = softmax_j((q[i,h,:] . k[j, h/G, :]) * scale) @ v[j, h/G, :]
// over keys j < Lk with j <= p when causal and j >= p - window_left when windowed; fp32 softmax
// and accumulation; a query with no visible key gets zeros.
//
// Tiling: a workgroup of four waves owns 128 queries of one head (32 per wave, two 16-query MFMA
// column blocks) and walks the keys in steps of 64. Each step's K and V tiles (64 x D) are loaded
// cooperatively with 16-byte coalesced loads one step ahead into registers and staged in a double
// buffer in LDS. Per wave and step:
//   S^T[64 keys, 32 q]  = K Q^T        MFMA 16x16x32; K from LDS (A operand, 16-byte reads),
//                                      Q^T held in registers for the whole kernel (B operand)
//   online softmax per query column: the 16 keys of a lane are local, two shuffles per step
//   O^T[D, 32 q]       += V^T P^T      MFMA 16x16x16; P^T is the S^T accumulator layout as is,
//                                      V^T comes from row-major V in LDS through ds_read_tr16_b64
// Only tiles that cross the causal diagonal, the window edge or the sequence end are masked.
// Workgroups are ordered with the KV head fastest (all query heads of one KV head share an XCD's
// L2) and the heaviest causal query blocks first.
#include "prefill.hpp"

#include <math.h>

namespace sp {

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_f16x8 __attribute__((ext_vector_type(8)));
typedef short pf_s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 pf_f16x4 __attribute__((ext_vector_type(4)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_s16x4 lds_s16x4;

template <typename T> struct PrefillMfma;
template <> struct PrefillMfma<bf16_t> {
  __device__ __forceinline__ static pf_f32x4 qk(uint4 k, uint4 q, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8, k),
                                                   __builtin_bit_cast(pf_bf16x8, q), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x4 pv(pf_s16x4 v, uint2 p, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v, __builtin_bit_cast(pf_s16x4, p), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
  }
};
template <> struct PrefillMfma<f16_t> {
  __device__ __forceinline__ static pf_f32x4 qk(uint4 k, uint4 q, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pf_f16x8, k),
                                                  __builtin_bit_cast(pf_f16x8, q), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x4 pv(pf_s16x4 v, uint2 p, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(pf_f16x4, v),
                                                 __builtin_bit_cast(pf_f16x4, p), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
  }
};

template <int D>
struct PrefillCfg {
  static constexpr int RB = D * 2;             // bytes per K/V row (16-bit elements)
  static constexpr int KP = RB + 16;           // K LDS pitch: 16-byte reads of 8 rows hit 8 bank groups
  static constexpr int VP = RB + 32;           // V LDS pitch: transpose reads of 4 rows hit 4 bank groups
  static constexpr int KT = kPrefillBN * KP;   // bytes of one K tile
  static constexpr int VT = kPrefillBN * VP;
  static constexpr int BUF = KT + VT;
  static constexpr int LDS = 2 * BUF;          // double buffered
  static constexpr int CPR = RB / 16;          // 16-byte chunks per row
  static constexpr int NLD = kPrefillBN * CPR / 256;  // 16-byte loads per thread per tile (K or V)
  static constexpr int DC = D / 32;            // QK k-chunks
  static constexpr int DB = D / 16;            // PV output dim blocks
};

template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(256, 2) prefill_kernel(PrefillArgs a) {
  using C = PrefillCfg<D>;
  constexpr int BN = kPrefillBN, KP = C::KP, VP = C::VP, DC = C::DC, DB = C::DB;
  constexpr int CPR = C::CPR, NLD = C::NLD, RB = C::RB;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

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
  // keys any query of this workgroup can see
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  const int t_first = kv_lo > 0 ? (kv_lo / BN) * BN : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int b = lane >> 4, i16 = lane & 15;

  // ---- per-sequence base addresses
  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 2;
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) * 2;
  const char* kbase = nullptr;
  const char* vbase = nullptr;
  const int32_t* table = nullptr;
  int64_t head_off = 0;
  if constexpr (PAGED) {
    table = a.block_tables + (int64_t)seq * a.max_blocks_per_seq;
    head_off = a.layer_off_b + (int64_t)kvh * a.block_size * RB;
  } else {
    const int64_t kv0 = (a.cu_k ? (int64_t)k_begin * a.kv_tok : (int64_t)seq * a.kv_batch) +
                        (int64_t)kvh * a.kv_head;
    kbase = (const char*)a.k + kv0 * 2;
    vbase = (const char*)a.v + kv0 * 2;
  }

  // ---- Q^T operand in registers: wave's queries qs + 32*wave + 16*qb + i16, dims 32c + 8b..+8
  const int wq0 = qs + 32 * wave;
  uint4 qreg[2][DC];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = wq0 + 16 * qb + i16;
    const char* qp = qbase + (int64_t)qi * a.q_tok * 2;
#pragma unroll
    for (int c = 0; c < DC; ++c)
      qreg[qb][c] = qi < qe ? *(const uint4*)(qp + (32 * c + 8 * b) * 2) : make_uint4(0, 0, 0, 0);
  }

  // ---- cooperative tile loads (16-byte chunks, rows = keys)
  uint4 kr[NLD], vr[NLD];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int idx = u * 256 + tid;
      const int r = idx / CPR, c = idx % CPR;
      const int j = t0 + r;
      bool ok = j >= kv_lo && j < kv_hi;
      const char* kp;
      const char* vp;
      if constexpr (PAGED) {
        const int blk = ok ? table[j / a.block_size] : 0;
        ok = ok && blk >= 0 && blk < a.num_blocks;
        const int64_t off = (int64_t)(ok ? blk : 0) * a.block_stride_b + head_off +
                            (int64_t)(j % a.block_size) * RB + c * 16;
        kp = a.kpool + off;
        vp = a.vpool + off;
      } else {
        const int64_t off = (int64_t)j * a.kv_tok * 2 + c * 16;
        kp = kbase + off;
        vp = vbase + off;
      }
      kr[u] = ok ? *(const uint4*)kp : make_uint4(0, 0, 0, 0);
      vr[u] = ok ? *(const uint4*)vp : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
    char* kl = smem + buf * C::BUF;
    char* vl = kl + C::KT;
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int idx = u * 256 + tid;
      const int r = idx / CPR, c = idx % CPR;
      *(uint4*)(kl + r * KP + c * 16) = kr[u];
      *(uint4*)(vl + r * VP + c * 16) = vr[u];
    }
  };

  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  pf_f32x4 acc[2][DB];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[qb][db] = pf_f32x4{0.f, 0.f, 0.f, 0.f};

  // query positions of this wave (for masking) and whether the wave has queries at all
  const int wq_lo = wq0, wq_hi = min(wq0 + 32, qe) - 1;  // inclusive
  const bool wave_active = wq_lo < qe;

  int t0 = t_first;
  if (t0 < kv_hi) {
    load_tile(t0);
    store_tile(0);
    if (t0 + BN < kv_hi) load_tile(t0 + BN);
  }
  __syncthreads();

  int buf = 0;
  for (; t0 < kv_hi; t0 += BN, buf ^= 1) {
    // wave-uniform: does this wave see any key of the tile, and does it need per-element masks
    bool visit = wave_active;
    bool need_mask = t0 + BN > Lk;
    if (a.causal != SP_CAUSAL_NONE) {
      visit = visit && t0 <= wq_hi + pos_off;
      need_mask = need_mask || (t0 + BN - 1 > wq_lo + pos_off);
    }
    if (a.window_left >= 0) {
      visit = visit && t0 + BN - 1 >= wq_lo + pos_off - a.window_left;
      need_mask = need_mask || (t0 < wq_hi + pos_off - a.window_left);
    }
    if (visit) {
      const char* kl = smem + buf * C::BUF;
      char* vl = smem + buf * C::BUF + C::KT;
      // S^T = K Q^T
      pf_f32x4 s[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        s[kb][0] = pf_f32x4{0.f, 0.f, 0.f, 0.f};
        s[kb][1] = pf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const uint4 kop = *(const uint4*)(kl + (16 * kb + i16) * KP + (32 * c + 8 * b) * 2);
          s[kb][0] = PrefillMfma<T>::qk(kop, qreg[0][c], s[kb][0]);
          s[kb][1] = PrefillMfma<T>::qk(kop, qreg[1][c], s[kb][1]);
        }
      }
      // online softmax per query column
      uint2 pb[4][2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qpos = wq0 + 16 * qb + i16 + pos_off;
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = s[kb][qb][e] * a.scale_log2;
            if (need_mask) {
              const int j = t0 + 16 * kb + 4 * b + e;
              bool ok = j < Lk && j >= kv_lo;
              if (a.causal != SP_CAUSAL_NONE) ok = ok && j <= qpos;
              if (a.window_left >= 0) ok = ok && j >= qpos - a.window_left;
              x = ok ? x : -INFINITY;
            }
            s[kb][qb][e] = x;
            mloc = fmaxf(mloc, x);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run[qb], mloc);
        const float alpha = (m_run[qb] == -INFINITY) ? 0.f : exp2f(m_run[qb] - m_new);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        float lsum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          float p[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p[e] = exp2f(s[kb][qb][e] - m_use);  // exp2(-inf) = 0 for masked keys
            lsum += p[e];
          }
          pb[kb][qb] = make_uint2(PrefillMfma<T>::pack(p[0], p[1]), PrefillMfma<T>::pack(p[2], p[3]));
        }
        l_run[qb] = l_run[qb] * alpha + lsum;
        m_run[qb] = m_new;
        if (alpha != 1.f) {  // skipped wave-wide once the running max stops moving
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[qb][db] *= alpha;
        }
      }
      // O^T += V^T P^T, V^T through the LDS transpose read
      const int vrow = 4 * b + (i16 >> 2), vcol = 4 * (i16 & 3);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          lds_s16x4* vptr = (lds_s16x4*)(vl + (16 * kb + vrow) * VP + (16 * db + vcol) * 2);
          const pf_s16x4 vop = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vptr);
          acc[0][db] = PrefillMfma<T>::pv(vop, pb[kb][0], acc[0][db]);
          acc[1][db] = PrefillMfma<T>::pv(vop, pb[kb][1], acc[1][db]);
        }
      }
    }
    // stage the next tile (loaded one step ahead) and fetch the one after
    if (t0 + BN < kv_hi) {
      store_tile(buf ^ 1);
      if (t0 + 2 * BN < kv_hi) load_tile(t0 + 2 * BN);
    }
    __syncthreads();
  }

  // ---- normalise and store: lane (b, i16) holds O^T[16db + 4b + e][query 16qb + i16]
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int qi = wq0 + 16 * qb + i16;
    if (qi >= qe) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    char* op = obase + (int64_t)qi * a.o_tok * 2;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      uint2 w;
      if constexpr (sizeof(T) == 2) {
        w.x = PrefillMfma<T>::pack(acc[qb][db][0] * inv, acc[qb][db][1] * inv);
        w.y = PrefillMfma<T>::pack(acc[qb][db][2] * inv, acc[qb][db][3] * inv);
      }
      *(uint2*)(op + (16 * db + 4 * b) * 2) = w;
    }
  }
}

template <typename T, int D>
static int launch_td(const PrefillArgs& a, bool paged, hipStream_t stream) {
  const int64_t blocks = (int64_t)a.num_qblocks * a.num_seqs * a.hq;
  if (blocks <= 0) return SP_OK;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "prefill: grid of %lld workgroups", (long long)blocks);
  if (paged)
    hipLaunchKernelGGL((prefill_kernel<T, D, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((prefill_kernel<T, D, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return check_launch("prefill_kernel");
}

template <typename T>
static int launch_t(const PrefillArgs& a, int head_dim, bool paged, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_td<T, 64>(a, paged, stream);
    case 128: return launch_td<T, 128>(a, paged, stream);
    default: return fail(SP_EUNSUPPORTED, "prefill: head_dim %d has no kernel (64, 128)", head_dim);
  }
}

int launch_prefill(const PrefillArgs& a, sp_dtype dtype, int head_dim, bool paged,
                   hipStream_t stream) {
  switch (dtype) {
    case SP_BF16: return launch_t<bf16_t>(a, head_dim, paged, stream);
    case SP_F16: return launch_t<f16_t>(a, head_dim, paged, stream);
    default: return fail(SP_EUNSUPPORTED, "prefill: dtype %s has no kernel", dtype_name(dtype));
  }
}

}  // namespace sp
