// Causal / windowed attention prefill over packed variable-length sequences, on gfx950 MFMA.
//
// Semantics (reference: MultiHeadAttention::forward / forward_cached with a causal or sliding
// window mask, crates/sketchpad-core/src/transformer.rs:103-168, :184-271, :415-451; the chunked
// prefill mask of crates/sketchpad-llm/src/llama.rs:374-388; flash_attention,
// crates/sketchpad-cubecl/src/attention.rs:97-178): for query i of a sequence with Lq queries and
// Lk keys, sitting at position p = i + (Lk - Lq) (bottom-right) or p = i (top-left),
//   out[i, h, :] = softmax_j((q[i,h,:] . k[j, h/G, :]) * scale) @ v[j, h/G, :]
// over keys j < Lk with j <= p when causal and j >= p - window_left when windowed; fp32 softmax
// and accumulation (FlashAttention-2 online softmax, Dao 2023); a query with no visible key gets
// zeros.
//
// Tiling: a workgroup of four waves owns 128 queries of one head (32 per wave) and walks the keys
// in tiles of 64. Both products run on v_mfma_f32_32x32x16 (bf16 / f16):
//   S^T[32 keys, 32 q] = K Q^T   A = K rows from LDS (16 bytes per lane), B = Q^T in registers
//                                (loaded once). Lane l ends up holding 16 scores of query l%32, so
//                                the softmax max / sum are in-lane plus one permlane32 swap.
//   O^T[32 d, 32 q]   += V^T P^T B = P^T straight from the S^T registers (the 16 tokens of one
//                                MFMA are taken in the order the S^T layout hands them out); A = V^T
//                                from row-major V in LDS through ds_read_tr16_b64.
// The key loop is software-pipelined inside each wave: while the QK MFMAs of tile j+1 run, the
// same wave computes tile j's softmax (one slice of exponentials, packs and row sums after each
// MFMA, in an order sched_barriers pin), then issues tile j's PV MFMAs. So the wave keeps the
// MFMA and VALU pipes busy at once instead of leaving the overlap to the other wave on its SIMD.
// K/V tiles go HBM -> LDS with global_load_lds_dwordx4 (no register staging) into double
// buffers: K runs two tiles ahead of the PV product (its QK product runs one tile early), V one
// tile ahead; interior tiles take one scalar base per tile (per block when paged, with the block
// ids fetched a tile ahead), and their loads go out four per M0 write through the instruction
// offset. Rows are stored with the 16-byte chunks XOR-swizzled so that the K
// reads (16 rows x one chunk) and the V transpose reads (4 rows x 64 bytes) are bank-conflict
// free.
// Only tiles that cross the causal diagonal, the window edge or the sequence end are masked.
// Workgroups are ordered with the KV head fastest (all query heads of one KV head share an XCD's
// L2) and the heaviest causal query blocks first.
// Outputs in the input type leave through LDS: each wave stages its block in a tile buffer that
// no wave needs any more and stores whole rows (store_rows_staged), where a store from the O^T
// registers would write 16 bytes into each of 32 rows.
#include "prefill.hpp"

#include <math.h>

#include <type_traits>

namespace sp {

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 pf_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 pf_f16x2 __attribute__((ext_vector_type(2)));
typedef float pf_f32x2 __attribute__((ext_vector_type(2)));
typedef float pf_f32x16 __attribute__((ext_vector_type(16)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));
typedef short pf_s16x4 __attribute__((ext_vector_type(4)));
typedef short pf_s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) pf_s16x4 lds_s16x4;
typedef unsigned pf_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_u32x4 lds_u32x4;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const char* p) {
  return (unsigned)(uintptr_t)(lds_void*)p;
}

template <typename T> struct PrefillMfma;
template <> struct PrefillMfma<bf16_t> {
  __device__ __forceinline__ static pf_f32x16 mma(uint4 a, uint4 b, pf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(pf_bf16x8, a),
                                                   __builtin_bit_cast(pf_bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x16 mma(pf_s16x8 a, uint4 b, pf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(pf_bf16x8, a),
                                                   __builtin_bit_cast(pf_bf16x8, b), c, 0, 0, 0);
  }
  // v_mfma_f32_16x16x32: A 16 x 32 (lane l: row l % 16, k 8(l / 16) .. +7), B 32 x 16 (lane l:
  // column l % 16, the same k), D 16 x 16 (lane l: column l % 16, rows 4(l / 16) .. +3)
  __device__ __forceinline__ static pf_f32x4 mma16(uint4 a, uint4 b, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8, a),
                                                   __builtin_bit_cast(pf_bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x4 mma16(pf_s16x8 a, uint4 b, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8, a),
                                                   __builtin_bit_cast(pf_bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {  // v_cvt_pk_bf16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((pf_f32x2){lo, hi}, pf_bf16x2));
  }
  // c + lo + hi of a packed pair (v_dot2_f32_bf16 against (1, 1))
  __device__ __forceinline__ static float sum2(uint32_t w, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(pf_bf16x2, w),
                                           __builtin_bit_cast(pf_bf16x2, 0x3f803f80u), c, false);
  }
};
template <> struct PrefillMfma<f16_t> {
  __device__ __forceinline__ static pf_f32x16 mma(uint4 a, uint4 b, pf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(pf_f16x8, a),
                                                  __builtin_bit_cast(pf_f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x16 mma(pf_s16x8 a, uint4 b, pf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(pf_f16x8, a),
                                                  __builtin_bit_cast(pf_f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x4 mma16(uint4 a, uint4 b, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pf_f16x8, a),
                                                  __builtin_bit_cast(pf_f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static pf_f32x4 mma16(pf_s16x8 a, uint4 b, pf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pf_f16x8, a),
                                                  __builtin_bit_cast(pf_f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((pf_f32x2){lo, hi}, pf_f16x2));
  }
  __device__ __forceinline__ static float sum2(uint32_t w, float c) {  // v_dot2_f32_f16
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(pf_f16x2, w),
                                  __builtin_bit_cast(pf_f16x2, 0x3c003c00u), c, false);
  }
};

template <int D>
struct PrefillCfg {
  static constexpr int RB = D * 2;                 // bytes per K/V row (16-bit elements)
  static constexpr int CPR = RB / 16;              // 16-byte chunks per row
  static constexpr int TILE = kPrefillBN * RB;     // bytes of one K (or V) tile
  static constexpr int BUF = 2 * TILE;             // K tile then V tile
  static constexpr int NLD = BUF / 1024 / 4;       // 1 KiB global_load_lds per wave per tile
  static constexpr int KC = D / 16;                // QK k-steps (16 dims each)
  static constexpr int DB = D / 32;                // PV output blocks (32 dims each)
  // XOR swizzle of a row's 16-byte chunks (a permutation of 0..CPR-1 that depends on the row's
  // low four bits). Chosen so that 16 consecutive rows at one logical chunk, and 4 consecutive
  // rows x 64 logical bytes, land on distinct LDS banks.
  // (Rows of 32 chunks, D = 256, take the 16-chunk permutation: it only has to separate rows
  // within 256 bytes of banks.) Rows of 64 chunks, D = 512, are read by transposes of 8 rows x
  // 32 bytes per 32 lanes (prefill_d512_kernel), which need the row's permutation to move the
  // chunk pair by a different even offset for each of 8 consecutive rows: 2(row % 8) + row / 8 % 2.
  __device__ __forceinline__ static int swz(int row) {
    if constexpr (CPR >= 64) return ((row & 7) << 1) | ((row >> 3) & 1);
    else if constexpr (CPR >= 16) return ((row & 3) << 2) | ((row >> 2) & 3);
    else return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
  }
};

__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// Value of the lane's partner in the other half of the wave (lane ^ 32), via v_permlane32_swap.
__device__ __forceinline__ void swap_halves(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Four 1 KiB LDS DMAs that share one M0 write: load u (0-3) reads base_u + v_u + 1024u and
// writes lds_dst + 1024u + 16 lane (the instruction offset applies to both addresses). The s_nop
// covers the M0 write (and, for bases read out of vector lanes, the SGPR write) -> LDS DMA wait
// states. Completion is awaited explicitly (s_waitcnt vmcnt(0) + barrier) before the data is read.
__device__ __forceinline__ void lds_dma16x4(const char* b0, const char* b1, const char* b2,
                                            const char* b3, int v0, int v1, int v2, int v3,
                                            char* lds_dst) {
  const unsigned m0 = (unsigned)(uintptr_t)(lds_void*)lds_dst;
  asm volatile(
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %4\n\t"
      "global_load_lds_dwordx4 %1, %5 offset:1024\n\t"
      "global_load_lds_dwordx4 %2, %6 offset:2048\n\t"
      "global_load_lds_dwordx4 %3, %7 offset:3072" ::"v"(v0),
      "v"(v1), "v"(v2), "v"(v3), "s"(b0), "s"(b1), "s"(b2), "s"(b3), "{m0}"(m0)
      : "memory");
}

// A wave's normalised 32 x D output block, stored as whole rows in the input's 16-bit type. In
// the O^T MFMA layout lane (l32, hh) holds dims 32db + 8rg + 4hh .. +3 of query l32, so a store
// straight from there would put 16 bytes into each of 32 rows. The block goes instead through
// `stage`, 32 rows x SD dims (SD = min(D, 128)) of LDS that no other wave touches meanwhile, in
// D / SD passes: the lanes write their values there (chunk c of row r at chunk c ^ (r % CPS), so
// that the writes and the row reads spread over the banks), then read it back row-wise and
// store CPS lanes x 16 bytes per row. A wave's LDS accesses run in order, so a pass's writes do
// not overtake the previous pass's reads. Rows at or past qe are not stored.
template <typename M, int D>
__device__ __forceinline__ void store_rows_staged(const pf_f32x16* acc, float inv, char* stage,
                                                  char* obase, int64_t o_tok, int wq0, int qe,
                                                  int lane) {
  constexpr int SD = D < 128 ? D : 128, SRB = SD * 2, CPS = SRB / 16, DBS = SD / 32;
  constexpr int RPS = 64 / CPS;  // rows per store instruction
  static_assert(D % SD == 0 && CPS * 16 == SRB, "whole passes of 16-byte chunks");
  const int l32 = lane & 31, hh = lane >> 5, rsw = l32 & (CPS - 1), cc = lane % CPS;
#pragma unroll
  for (int p = 0; p < D / SD; ++p) {
#pragma unroll
    for (int db = 0; db < DBS; ++db)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const pf_f32x16& A = acc[p * DBS + db];
        *(uint2*)(stage + l32 * SRB + 16 * ((db * 4 + rg) ^ rsw) + 8 * hh) =
            make_uint2(M::pack(A[rg * 4 + 0] * inv, A[rg * 4 + 1] * inv),
                       M::pack(A[rg * 4 + 2] * inv, A[rg * 4 + 3] * inv));
      }
#pragma unroll
    for (int j = 0; j < 32 / RPS; ++j) {
      const int row = RPS * j + lane / CPS;
      const uint4 v = *(const uint4*)(stage + row * SRB + 16 * (cc ^ (row & (CPS - 1))));
      const int q = wq0 + row;
      if (q < qe) *(uint4*)(obase + (int64_t)q * o_tok * 2 + p * SRB + 16 * cc) = v;
    }
  }
}

// The same for a wave of 16 queries on v_mfma_f32_16x16x32 (head dim 512): lane (n, g) holds
// dims 16db + 4g .. +3 of query n, so a direct store puts 32 bytes into each of 16 rows. The
// 16 x 512 block goes through a 16-row x 256-dim stage (8 KiB) in two passes; chunk c of row r
// sits at chunk c ^ (r % 16), and every store writes 32 lanes x 16 bytes of a row.
template <typename M>
__device__ __forceinline__ void store_rows_staged16(const pf_f32x4* acc, float inv, char* stage,
                                                    char* obase, int64_t o_tok, int wq0, int qe,
                                                    int lane) {
  constexpr int D = 512, SD = 256, SRB = SD * 2, CPS = SRB / 16, DBS = SD / 16;
  const int n = lane & 15, g = lane >> 4, cc = lane & 31;
#pragma unroll
  for (int p = 0; p < D / SD; ++p) {
#pragma unroll
    for (int db = 0; db < DBS; ++db) {
      const pf_f32x4& A = acc[p * DBS + db];
      *(uint2*)(stage + n * SRB + 16 * ((2 * db + (g >> 1)) ^ n) + 8 * (g & 1)) =
          make_uint2(M::pack(A[0] * inv, A[1] * inv), M::pack(A[2] * inv, A[3] * inv));
    }
#pragma unroll
    for (int j = 0; j < 16 / (64 / CPS); ++j) {
      const int row = 2 * j + (lane >> 5);
      const uint4 v = *(const uint4*)(stage + row * SRB + 16 * (cc ^ row));
      const int q = wq0 + row;
      if (q < qe) *(uint4*)(obase + (int64_t)q * o_tok * 2 + p * SRB + 16 * cc) = v;
    }
  }
}

// Stands in for cu_seqlens when a batch has none, so the kernel's length loads need no branch.
__constant__ int32_t kPrefillZeroPair[2] = {0, 0};

// Metadata the kernel only reads, seen through the constant address space so that uniform
// loads of it become scalar loads.
typedef const __attribute__((address_space(4))) int32_t* kconst_i32;
__device__ __forceinline__ kconst_i32 as_const(const int32_t* p) { return (kconst_i32)p; }

template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(256, 2) prefill_kernel(PrefillArgs a) {
  using C = PrefillCfg<D>;
  using M = PrefillMfma<T>;
  constexpr int BN = kPrefillBN, RB = C::RB, CPR = C::CPR, TILE = C::TILE;
  constexpr int KC = C::KC, DB = C::DB;
  constexpr int RPI = 1024 / RB;       // rows per 1 KiB load
  constexpr int NLD = TILE / 2048;     // loads per wave per tile: waves 0-1 fill K, 2-3 fill V
  constexpr int WROWS = NLD * RPI;     // rows of a tile one wave loads (half the tile)
  static_assert(BN == 64, "the S^T layout below assumes two 32-key MFMA blocks per tile");
  static_assert(WROWS * 2 == BN, "two waves fill one tile");
  __shared__ __attribute__((aligned(1024))) char kl[2][TILE];
  __shared__ __attribute__((aligned(1024))) char vl[2][TILE];

  // ---- workgroup -> (kv head, group member, sequence, split, query block), heavy query blocks
  // first; wave w takes queries 32w .. 32w + 31 of the block
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  // the metadata pointers are read with the grid shape, in the first batch of argument loads
  const int32_t* const cu_q_p = a.cu_q;
  const int32_t* const cu_k_p = PAGED ? a.context_lens : a.cu_k;
  int id = blockIdx.x;
  const int kvh = id % a.hkv;
  id /= a.hkv;
  const int gm = id % a.group;
  id /= a.group;
  const int seq = id % a.num_seqs;
  id /= a.num_seqs;
  const int split = id % a.nsplit;
  const int qblk = a.num_qblocks - 1 - id / a.nsplit;
  const int h = kvh * a.group + gm;

  // Sequence offsets and lengths. The scalar loads are issued whatever the layout (a batch
  // without cu_q / cu_k reads a zero pair instead), so they go out together and are waited for
  // once.
  const kconst_i32 cq = cu_q_p ? as_const(cu_q_p) + seq : as_const(kPrefillZeroPair);
  const kconst_i32 ck = PAGED || cu_k_p ? as_const(cu_k_p) + seq : as_const(kPrefillZeroPair);
  const int cq0 = cq[0], cq1 = cq[1], ck0 = ck[0], ck1 = PAGED ? 0 : ck[1];
  asm volatile("" ::"s"(ck0), "s"(ck1));  // keep the key-length loads ahead of the early exit
  const int q_begin = cq0;
  const int Lq = cu_q_p ? cq1 - cq0 : a.lq;
  int Lk, k_begin = 0;
  if constexpr (PAGED) {
    Lk = min(ck0, a.max_blocks_per_seq * a.block_size);
  } else {
    k_begin = ck0;
    Lk = cu_k_p ? ck1 - ck0 : a.lk;
  }
  const int qs = qblk * kPrefillBM;
  if (qs >= Lq) return;
  const int qe = min(qs + kPrefillBM, Lq);
  const int pos_off = (a.causal == SP_CAUSAL_TOP_LEFT) ? 0 : Lk - Lq;
  // keys any query of this workgroup can see: [kv_lo, kv_hi)
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  // This workgroup's key tiles: all of [kv_lo, kv_hi), or its 1/nsplit share of them (masks and
  // row clamps keep using the full range; only the walk stops at kv_end).
  int t_first = (kv_lo / BN) * BN, kv_end = kv_hi;
  if (a.nsplit > 1) {
    const int ntiles = kv_hi > t_first ? (kv_hi - t_first + BN - 1) / BN : 0;
    const int tps = (ntiles + a.nsplit - 1) / a.nsplit;
    t_first += split * tps * BN;
    kv_end = min(kv_hi, t_first + tps * BN);
  }

  const int l32 = lane & 31, hh = lane >> 5;        // MFMA column (query) and half
  const int i16 = lane & 15, g4 = lane >> 4;        // 16-lane group for the transpose reads

  // ---- per-sequence base addresses
  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 2;
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) *
          dtype_size((sp_dtype)a.out_dtype);
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

  // ---- Q^T operand (B of the S^T MFMA): query wq0 + l32, dims 16c + 8hh .. +7, unscaled.
  const int wq0 = qs + 32 * wave;
  const int my_q = wq0 + l32;
  const float c2 = a.scale_log2;  // > 0 (checked on the host)
  uint4 qreg[KC];
  {
    const char* qp = qbase + (int64_t)min(my_q, qe - 1) * a.q_tok * 2;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[c] = my_q < qe ? *(const uint4*)(qp + (16 * c + 8 * hh) * 2) : make_uint4(0, 0, 0, 0);
  }

  // ---- HBM -> LDS tile loads. Waves 0-1 fill K tiles, running two tiles ahead of the PV product
  // (the QK product of tile j+1 runs while tile j's softmax is computed); waves 2-3 fill V tiles,
  // one tile ahead. Wave w's load u moves 1 KiB = RPI rows, r_u = (w & 1) * WROWS + u * RPI ..;
  // lane `lane` takes physical chunk p = lane % CPR of row r_u + lane / CPR and fetches the
  // logical chunk that the swizzle puts there. Interior tiles (every row inside [kv_lo, kv_hi))
  // take the fast path: one scalar base per tile (non-paged) or per block (paged) plus a constant
  // lane offset per load. Edge tiles clamp rows outside [kv_lo, kv_hi) to a valid row (their
  // scores are masked) and compute per-lane addresses.
  const bool v_wave = wave >= 2;
  const int lead = v_wave ? 1 : 2;  // tiles ahead of the PV product this wave loads
  const int wrow0 = (wave & 1) * WROWS;
  const int64_t row_pitch = PAGED ? (int64_t)RB : (int64_t)a.kv_tok * 2;
  const char* src_base = PAGED ? (v_wave ? a.vpool : a.kpool) : (v_wave ? vbase : kbase);
  // paged fast path: a wave's WROWS rows of a tile lie in whole blocks (block_size divides the
  // 64-row tile, and a load never straddles blocks)
  const bool paged_fast = PAGED && a.block_size % RPI == 0 && BN % a.block_size == 0;
  int voff[NLD];  // lane part of each load's source offset (bytes), row offset included
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = wrow0 + u * RPI + lane / CPR;  // tile row
    const int64_t row_b = PAGED ? (int64_t)(r % max(a.block_size, 1)) * RB : (int64_t)r * row_pitch;
    voff[u] = (int)row_b + 16 * ((lane % CPR) ^ C::swz(r));
  }
  static_assert(NLD % 4 == 0, "tile loads go out in groups of four");
  // Interior tiles issue their loads in groups of four with instruction offsets 0, 1, 2, 3 KiB.
  // Contiguous K/V: the offsets come out of the lane offsets (still >= 0: load u's rows start at
  // u RPI rows of at least RB bytes, u RPI RB = 1024 u). Paged with blocks that hold whole groups
  // (block_size a multiple of 4 RPI rows, so a group's rows lie in one block): the same, with one
  // base per group. Smaller blocks: out of the per-load bases.
  const bool group_blk = wave_uniform(PAGED && a.block_size % (4 * RPI) == 0);
  int voff_g[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u)
    voff_g[u] = (!PAGED || group_blk) ? voff[u] - (u & 3) * 1024 : voff[u];
  auto tile_interior = [&](int t0) __attribute__((always_inline)) {
    return t0 >= kv_lo && t0 + BN <= kv_hi;
  };
  // Paged fast path: the block ids of the rows of the next tile this wave loads, fetched one
  // tile ahead so that no load waits on a dependent block-table read. Lane u < NLD fetches load
  // u's id with a vector load: it completes with the tile loads at the next step's wait, where a
  // scalar load would sit in lgkmcnt ahead of the LDS operand reads of the QK product and make
  // each of their waits a wait for the table read.
  // block_size divides the 64-key tile here, so it is a power of two and every tile start t0 is
  // a multiple of it: the id of the block holding row t0 + r is table[(t0 >> shift) + (r >> shift)].
  int nblk = 0;
  const int bs_shift = paged_fast ? wave_uniform(31 - __builtin_clz(max(a.block_size, 1))) : 0;
  const int lane_blk = (wrow0 + min(lane, NLD - 1) * RPI) >> bs_shift;
  auto fetch_blocks = [&](int t0) __attribute__((always_inline)) {
    if constexpr (PAGED) {
      if (paged_fast && t0 < kv_end && tile_interior(t0)) nblk = table[(t0 >> bs_shift) + lane_blk];
    }
  };
  // Interior tile: its loads go out in groups of four that share one M0 write.
  auto issue_interior = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if constexpr (PAGED) {
      // block ids fetched by fetch_blocks(t0), load u's in lane u: every lane turns its id into
      // its load's base address at once (vector ops), and each load reads its base out of lane u
      // (two readlanes), instead of a scalar chain of compares and 64-bit multiplies per load.
      // The base is taken less the load's instruction offset; the sum is the block's row address.
      const int bl = (nblk >= 0 && nblk < a.num_blocks) ? nblk : 0;  // never outside the pool
      const uint64_t vb = (uint64_t)(uintptr_t)(src_base + head_off) +
                          (uint64_t)bl * (uint64_t)a.block_stride_b - (uint64_t)((lane & 3) * 1024);
      const int vb_lo = (int)(uint32_t)vb, vb_hi = (int)(uint32_t)(vb >> 32);
      auto base_of = [&](int u) __attribute__((always_inline)) {
        const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane(vb_lo, u);
        const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane(vb_hi, u);
        return (const char*)(uintptr_t)((hi << 32) | lo);
      };
      if (group_blk) {  // lane g (g % 4 == 0) holds its group's block; no offset taken off
#pragma unroll
        for (int g = 0; g < NLD; g += 4) {
          const char* b = base_of(g);
          lds_dma16x4(b, b, b, b, voff_g[g], voff_g[g + 1], voff_g[g + 2], voff_g[g + 3],
                      dst + g * 1024);
        }
      } else {
#pragma unroll
        for (int g = 0; g < NLD; g += 4)
          lds_dma16x4(base_of(g), base_of(g + 1), base_of(g + 2), base_of(g + 3), voff_g[g],
                      voff_g[g + 1], voff_g[g + 2], voff_g[g + 3], dst + g * 1024);
      }
    } else {
      const char* sb = src_base + (int64_t)t0 * row_pitch;
#pragma unroll
      for (int g = 0; g < NLD; g += 4)
        lds_dma16x4(sb, sb, sb, sb, voff_g[g], voff_g[g + 1], voff_g[g + 2], voff_g[g + 3],
                    dst + g * 1024);
    }
  };
  auto issue_tile = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if (tile_interior(t0) && (!PAGED || paged_fast)) {
      issue_interior(t0, buf);
      return;
    }
    // Edge tiles are rare: the lane id goes through an empty asm so that the per-lane source
    // addresses are derived here, not hoisted out of the key loop as live registers.
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int R = wrow0 + u * RPI + ln / CPR, p = ln % CPR;
      const int c = p ^ C::swz(R);
      const int j = min(max(t0 + R, kv_lo), kv_hi - 1);
      const char* src;
      if constexpr (PAGED) {
        int blk = table[j / a.block_size];
        blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;  // never dereference outside the pool
        src = src_base + (int64_t)blk * a.block_stride_b + head_off +
              (int64_t)(j % a.block_size) * RB + c * 16;
      } else {
        src = src_base + (int64_t)j * row_pitch + c * 16;
      }
      lds_dma16(src, dst + u * 1024);
    }
  };

  // Online softmax state of query l32 (both lanes of a query hold the same values).
  // m_run: running maximum of the exponents x = q.k * scale * log2(e) seen (-inf before the
  // first visible key); m_used: the offset subtracted from x (m_run once that is finite, else 0).
  float m_run = -INFINITY, m_used = 0.f, l_run = 0.f;
  pf_f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  pf_f32x16 zero16;
#pragma unroll
  for (int r = 0; r < 16; ++r) zero16[r] = 0.f;

  const int wq_lo = wq0, wq_hi = min(wq0 + 32, qe) - 1;  // this wave's queries (inclusive)
  const bool wave_active = wq_lo < qe;
  const int qpos = my_q + pos_off;
  const int sw = C::swz(l32);     // swizzle of the K rows this lane reads (row & 15 == l32 & 15)
  // A tile needs masking iff t0 < mask_below or t0 > mask_above (wave-uniform bounds): it starts
  // before kv_lo or before the window edge of this wave's last query, or it runs past the
  // sequence end or past the causal diagonal of this wave's first query.
  int mask_below = kv_lo, mask_above = Lk - BN;
  if (a.causal != SP_CAUSAL_NONE) mask_above = min(mask_above, wq_lo + pos_off - BN + 1);
  if (a.window_left >= 0) mask_below = max(mask_below, wq_hi + pos_off - a.window_left);
  mask_below = wave_uniform(mask_below);
  mask_above = wave_uniform(mask_above);

  // Lane parts of the LDS operand addresses (byte offsets inside a tile). With the XOR swizzle
  // an operand's logical chunk index only flips bits the lane part owns alone, so every operand
  // of a tile sits at (lane part ^ constant) + immediate offset.
  const int k_lane = (l32 * RB) | (16 * (hh ^ sw));
  const int rl = (g4 >> 1) * 4 + (i16 >> 2);
  const int chl = (g4 & 1) * 2 + ((i16 & 3) >> 1);
  const int v_lane0 = rl * RB + 16 * (chl ^ C::swz(rl)) + 8 * (i16 & 1);
  const int v_lane1 = (rl + 8) * RB + 16 * (chl ^ C::swz(rl + 8)) + 8 * (i16 & 1);

  // Causal diagonal at 32-key granularity (see the mask below).
  const int diag0 = wave_uniform(wq_lo + pos_off);
  const bool tri_ok = a.causal != SP_CAUSAL_NONE && pos_off >= 0 && (pos_off & 31) == 0 &&
                      qe - 1 + pos_off < Lk;
  const int tri_lim = l32 - 4 * hh;

  // ---- the pieces of one key tile -------------------------------------------------------------
  // QK product S^T = K Q^T of the tile in LDS buffer kb into s (two 32-key blocks). K operand i
  // (k-step i/2, key block i%2) is row 32(i%2) + l32, chunk 2(i/2) + hh: (k_lane ^ 32(i/2)) +
  // 32(i%2) RB. `between(i)` runs after MFMA i: the softmax of the previous tile is interleaved
  // with these MFMAs, one slice per MFMA, in an order the sched_barriers pin.
  constexpr int NK = 2 * KC, AHK = 4;
  auto qk = [&](const char* kb, pf_f32x16 (&s)[2], auto&& between) __attribute__((always_inline)) {
    int kbl = k_lane;
    asm volatile("" : "+v"(kbl));
    auto read_k = [&](int i) __attribute__((always_inline)) {
      return *(const uint4*)(kb + (i & 1) * 32 * RB + (kbl ^ (32 * (i >> 1))));
    };
    uint4 kop[AHK];
#pragma unroll
    for (int i = 0; i < AHK; ++i) kop[i] = read_k(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const uint4 cur = kop[i % AHK];
      if (i + AHK < NK) kop[i % AHK] = read_k(i + AHK);
      s[i & 1] = M::mma(cur, qreg[i >> 1], i < 2 ? zero16 : s[i & 1]);
      between(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Masks, only on tiles that cross the sequence end, the window edge, kv_lo or the causal
  // diagonal. Score (mb, r) of this lane is key t0 + 4hh + off, off = 32mb + 8(r/4) + r%4.
  // this lane's row of the additive mask (dense path: the sequence index is the batch index)
  const float* mrow = a.mask ? a.mask + (int64_t)seq * a.mask_b + (int64_t)h * a.mask_h +
                                   (int64_t)min(my_q, qe - 1) * a.mask_q
                             : nullptr;
  auto apply_mask = [&](int t0, pf_f32x16 (&s)[2]) __attribute__((always_inline)) {
    if (mrow) {
      // additive mask (flash_attention_masked): softmax(q.k scale + mask) = softmax over
      // (q.k + mask / scale) scale. Keys past the sequence end read its last column; their
      // scores are masked below (such tiles always take the mask).
      const int jb = t0 + 4 * hh;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = min(jb + 32 * mb + 8 * (r >> 2) + (r & 3), Lk - 1);
          s[mb][r] += mrow[key] * a.inv_scale;
        }
    }
    if (t0 < mask_below || t0 > mask_above) {
      if (tri_ok && t0 >= mask_below && (t0 == diag0 || t0 + 32 == diag0)) {
        // 32-aligned causal diagonal: the diagonal block is the triangle 8(r/4) + r%4 <=
        // l32 - 4hh; with the diagonal at the tile start, block 1 lies wholly above it.
        int tl = tri_lim;
        asm volatile("" : "+v"(tl));
        if (t0 == diag0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[0][r] = (8 * (r >> 2) + (r & 3) <= tl) ? s[0][r] : -INFINITY;
            s[1][r] = -INFINITY;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            s[1][r] = (8 * (r >> 2) + (r & 3) <= tl) ? s[1][r] : -INFINITY;
        }
      } else {
        // general: visible iff lo <= key <= hi, a compile-time offset against two per-lane bounds
        int lo = kv_lo, hi = Lk - 1;
        if (a.causal != SP_CAUSAL_NONE) hi = min(hi, qpos);
        if (a.window_left >= 0) lo = max(lo, qpos - a.window_left);
        const int jb = t0 + 4 * hh;
        const int olo = lo - jb, ohi = hi - jb;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = 32 * mb + (r >> 2) * 8 + (r & 3);
            s[mb][r] = (off >= olo && off <= ohi) ? s[mb][r] : -INFINITY;
          }
      }
    }
  };

  // Softmax weights of one tile for query l32 (FlashAttention-2 online softmax, Dao 2023) with a
  // lazily raised maximum: p = 2^(s * scale * log2 e - m_used), packed to 16 bits for the PV
  // product; the row sum adds the 16-bit values the PV product uses (v_dot2 against ones).
  // Slice e (of 16) computes the two scores 2e, 2e+1 (score k of the lane is s[k/16][k%16]).
  uint4 pb[4];
  float la = 0.f, lb = 0.f;
  auto weights_slice = [&](const pf_f32x16 (&s)[2], int e, float off) __attribute__((always_inline)) {
    const int k0 = 2 * e;
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[k0 >> 4][k0 & 15], c2, -off));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[(k0 + 1) >> 4][(k0 + 1) & 15], c2, -off));
    const uint32_t w = M::pack(p0, p1);
    const int ks = k0 >> 3, c = (k0 >> 1) & 3;  // pb[ks] word c holds scores 8ks + 2c, +1
    if (c == 0) pb[ks].x = w;
    else if (c == 1) pb[ks].y = w;
    else if (c == 2) pb[ks].z = w;
    else pb[ks].w = w;
    if (ks < 2) la = M::sum2(w, la);
    else lb = M::sum2(w, lb);
  };
  auto weights_all = [&](const pf_f32x16 (&s)[2], float off) __attribute__((always_inline)) {
    la = 0.f;
    lb = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) weights_slice(s, e, off);
  };
  constexpr float kLazyBound = 4096.f;  // 2^kLazy, kLazy = 12
  // After the weights of a tile: raise the maximum when this lane's weights of the tile sum past
  // 2^kLazy (so every weight that enters the accumulators is <= 2^kLazy) or while the query has
  // no maximum yet; the weights are then recomputed against the exact new maximum, so the largest
  // weight of a row never underflows whatever the score range.
  auto finish_weights = [&](const pf_f32x16 (&s)[2]) __attribute__((always_inline)) {
    float lsum = la + lb;
    if (__any(lsum > kLazyBound || m_run == -INFINITY)) {
      float mq[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // four independent max3 chains over 8 scores each
        const int mb = k >> 1, r0 = (k & 1) * 8;
        float x = max3f(s[mb][r0], s[mb][r0 + 1], s[mb][r0 + 2]);
        x = max3f(x, s[mb][r0 + 3], s[mb][r0 + 4]);
        x = max3f(x, s[mb][r0 + 5], s[mb][r0 + 6]);
        mq[k] = __builtin_fmaxf(x, s[mb][r0 + 7]);
      }
      float mx = __builtin_fmaxf(max3f(mq[0], mq[1], mq[2]), mq[3]);
      float x0, x1;
      swap_halves(mx, x0, x1);
      const float m_new = __builtin_fmaxf(m_run, __builtin_fmaxf(x0, x1) * c2);
      const float used_new = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - used_new);  // 0 while m_run = -inf
      weights_all(s, used_new);
      lsum = la + lb;
      m_run = m_new;
      m_used = used_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    }
    l_run += lsum;
  };

  // PV product O^T += V^T P^T of the tile in LDS buffer vb: K-step ks covers tile tokens
  // 16ks .. 16ks+15 in the S^T order. The V^T operand (ks, db) is rows 16ks + rl (+ 8), chunk
  // 4db + chl: (v_lane0 ^ 64db) + 16ks RB (v_lane1 for the second row group), read AH ahead.
  auto pv = [&](const char* vb) __attribute__((always_inline)) {
    int vb0 = v_lane0, vb1 = v_lane1;
    asm volatile("" : "+v"(vb0), "+v"(vb1));
    auto read_v = [&](int ks, int db) __attribute__((always_inline)) {
      const char* a0 = vb + 16 * ks * RB + (vb0 ^ (64 * db));
      const char* a1 = vb + 16 * ks * RB + (vb1 ^ (64 * db));
      const pf_s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0));
      const pf_s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a1));
      return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    constexpr int NV = 4 * DB, AH = 4;
    pf_s16x8 vop[AH];
#pragma unroll
    for (int i = 0; i < AH; ++i) vop[i] = read_v(i / DB, i % DB);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const pf_s16x8 cur = vop[i % AH];
      if (i + AH < NV) vop[i % AH] = read_v((i + AH) / DB, (i + AH) % DB);
      acc[i % DB] = M::mma(cur, pb[i / DB], acc[i % DB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // wave-uniform: does this wave see any key of the tile. The conditions (the wave has queries,
  // the tile starts before kv_end, at or before the causal diagonal of the wave's last query, and
  // ends at or after the window edge of its first query) bound t0 from both sides, so they
  // reduce to one range [vis_lo, vis_hi) worked out once.
  int vis_lo = -(1 << 30), vis_hi = wave_active ? kv_end : -(1 << 30);
  if (a.causal != SP_CAUSAL_NONE) vis_hi = min(vis_hi, wq_hi + pos_off + 1);
  if (a.window_left >= 0) vis_lo = wq_lo + pos_off - a.window_left - BN + 1;
  vis_lo = wave_uniform(vis_lo);
  vis_hi = wave_uniform(vis_hi);
  auto visits = [&](int t0) __attribute__((always_inline)) { return t0 >= vis_lo && t0 < vis_hi; };

  // One pipeline step on tile t0 (its K in kcur's tile one step ago, now its S^T in sc; its V
  // in vcur): wait until this step's tiles are in (own loads, then everyone's), start the loads
  // that run ahead (K of t0 + 2 BN into kload, V of t0 + BN into vload; the barrier also
  // guarantees every wave is done reading both buffers), then the QK product of the next tile
  // (K in knext, S^T into sn) with this tile's softmax interleaved, and this tile's PV product.
  auto step = [&](int t0, pf_f32x16 (&sc)[2], pf_f32x16 (&sn)[2], const char* knext,
                  const char* vcur, char* kload, char* vload) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    {
      const int lt = t0 + lead * BN;
      if (lt < kv_end) {
        issue_tile(lt, v_wave ? vload : kload);
        fetch_blocks(lt + BN);
      }
    }
    const bool vis_c = visits(t0), vis_n = visits(t0 + BN);
    if (vis_c) {
      apply_mask(t0, sc);
      la = 0.f;
      lb = 0.f;
      // The offset goes through an empty asm in each branch so that the compiler cannot hoist
      // the (identical) weight computations of both branches above them, which would take the
      // exponentials out of the MFMA slots they are meant to fill.
      float off = m_used;
      if (vis_n) {
        asm volatile("" : "+v"(off));
        // 16 weight slices over the NK MFMAs of the QK product (NK = 16 at D = 128, 8 at D = 64)
        qk(knext, sn, [&](int i) __attribute__((always_inline)) {
#pragma unroll
          for (int e = i * 16 / NK; e < (i + 1) * 16 / NK; ++e) weights_slice(sc, e, off);
        });
      } else {
        asm volatile("" : "+v"(off));
#pragma unroll
        for (int e = 0; e < 16; ++e) weights_slice(sc, e, off);
      }
      finish_weights(sc);
      pv(vcur);
    } else if (vis_n) {
      qk(knext, sn, [](int) {});
    }
  };

  // Prologue: K of the first two tiles and V of the first go out while the Q loads are still in
  // flight; the wait below covers both, so no wait inside the key loop refers to Q (the tile
  // loads issued there are awaited explicitly). Then the first tile's QK product.
  pf_f32x16 sa[2], sb[2];
  int t0 = t_first;
  if (t0 < kv_end) {
    fetch_blocks(t0);
    if (v_wave) {
      issue_tile(t0, vl[0]);
      fetch_blocks(t0 + BN);
    } else {
      issue_tile(t0, kl[0]);
      fetch_blocks(t0 + BN);
      if (t0 + BN < kv_end) {
        issue_tile(t0 + BN, kl[1]);
        fetch_blocks(t0 + 2 * BN);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (visits(t0)) qk(kl[0], sa, [](int) {});
  // the loop's first barrier has nothing to wait for but keeps the step uniform
  while (t0 < kv_end) {
    step(t0, sa, sb, kl[1], vl[0], kl[0], vl[1]);
    t0 += BN;
    if (t0 >= kv_end) break;
    step(t0, sb, sa, kl[0], vl[1], kl[1], vl[0]);
    t0 += BN;
  }

  // ---- normalise and store: lane holds O^T[d][query l32], d = 32db + 8(r/4) + 4hh + r%4
  float x0, x1;
  swap_halves(l_run, x0, x1);
  const float l = x0 + x1;
  constexpr int kSelf = std::is_same<T, bf16_t>::value ? SP_BF16 : SP_F16;  // out = in type
  if (a.nsplit <= 1 && a.out_dtype == kSelf) {
    // Whole output rows through an LDS stage (store_rows_staged). The stage is half of a K
    // buffer: after the last step's barrier no wave reads K (the last step has no next tile) and
    // no load is pending (every wave waited for all before that barrier); only the V buffer of
    // the last tile may still be read. Waves 0-1 take kl[0], waves 2-3 kl[1].
    static_assert(TILE >= 64 * RB, "two 32-row stages per K buffer");
    store_rows_staged<M, D>(acc, l > 0.f ? 1.f / l : 0.f, kl[wave >> 1] + (wave & 1) * 32 * RB,
                            obase, a.o_tok, wq0, qe, lane);
    return;
  }
  if (my_q >= qe) return;
  if (a.nsplit > 1) {
    // partial record (m, l, -, -, acc[D]) of this split; m is the offset the weights are
    // relative to, -inf when the split saw no visible key (then l = 0 and acc = 0), so that the
    // merge never takes an empty split's offset as the row maximum. Rows past max_q (a caller
    // whose cu_seqlens exceed max_seqlen_q) have no record slot and are not written.
    if (my_q >= a.max_q) return;
    float* rec = a.partials +
        ((((int64_t)seq * a.max_q + my_q) * a.hq + h) * a.nsplit + split) * (D + 4);
    if (hh == 0) *(float2*)rec = make_float2(m_run == -INFINITY ? -INFINITY : m_used, l);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
        *(float4*)(rec + 4 + db * 32 + rg * 8 + hh * 4) =
            make_float4(acc[db][rg * 4 + 0], acc[db][rg * 4 + 1], acc[db][rg * 4 + 2],
                        acc[db][rg * 4 + 3]);
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int oes = dtype_size((sp_dtype)a.out_dtype);
  char* op = obase + (int64_t)my_q * a.o_tok * oes;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d0 = db * 32 + rg * 8 + hh * 4;
      const float o0 = acc[db][rg * 4 + 0] * inv, o1 = acc[db][rg * 4 + 1] * inv;
      const float o2 = acc[db][rg * 4 + 2] * inv, o3 = acc[db][rg * 4 + 3] * inv;
      if (a.out_dtype == SP_F32) {
        *(float4*)(op + d0 * 4) = make_float4(o0, o1, o2, o3);
      } else if (a.out_dtype == kSelf) {
        *(uint2*)(op + d0 * 2) = make_uint2(M::pack(o0, o1), M::pack(o2, o3));
      } else {  // the other 16-bit type
        using O = PrefillMfma<typename std::conditional<kSelf == SP_BF16, f16_t, bf16_t>::type>;
        *(uint2*)(op + d0 * 2) = make_uint2(O::pack(o0, o1), O::pack(o2, o3));
      }
    }
}

// Contiguous-K/V variant for grids of several rounds of workgroups: 32-key tiles, so that the
// workgroup fits three per CU (32 x 168 VGPRs per lane and 48 KiB of LDS), and a plain per-wave
// order QK -> softmax -> PV on each tile, with the waves of the two other workgroups on the SIMD
// filling its MFMA pipe while one wave runs its softmax (where prefill_kernel, at two workgroups
// per CU, overlaps the two inside each wave instead). A workgroup's start-up (metadata, Q, the
// first tiles) is then hidden behind two other workgroups rather than one. Tiles go HBM -> LDS
// two ahead through three buffers. Same semantics, masks and arguments as prefill_kernel
// (contiguous K/V, no key split).
template <typename T, int D>
__global__ void __launch_bounds__(256, 3) prefill_k32_kernel(PrefillArgs a) {
  using M = PrefillMfma<T>;
  constexpr int BN = 32, RB = D * 2, CPR = RB / 16, TILE = BN * RB;
  constexpr int KC = D / 16, DB = D / 32;
  constexpr int RPI = 1024 / RB;    // rows per 1 KiB load
  constexpr int NLD = TILE / 2048;  // loads per wave per tile: waves 0-1 fill K, 2-3 fill V
  constexpr int WROWS = NLD * RPI;  // rows of a tile one wave loads (half the tile)
  static_assert(WROWS * 2 == BN, "two waves fill one tile");
  static_assert(NLD == 4, "one group of four loads per wave and tile");
  using C = PrefillCfg<D>;  // the row swizzle
  __shared__ __attribute__((aligned(1024))) char kl[3][TILE];
  __shared__ __attribute__((aligned(1024))) char vl[3][TILE];

  // ---- workgroup -> (kv head, group member, sequence, query block), heavy query blocks first
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int32_t* const cu_q_p = a.cu_q;
  const int32_t* const cu_k_p = a.cu_k;
  int id = blockIdx.x;
  const int kvh = id % a.hkv;
  id /= a.hkv;
  const int gm = id % a.group;
  id /= a.group;
  const int seq = id % a.num_seqs;
  const int qblk = a.num_qblocks - 1 - id / a.num_seqs;
  const int h = kvh * a.group + gm;

  const kconst_i32 cq = cu_q_p ? as_const(cu_q_p) + seq : as_const(kPrefillZeroPair);
  const kconst_i32 ck = cu_k_p ? as_const(cu_k_p) + seq : as_const(kPrefillZeroPair);
  const int cq0 = cq[0], cq1 = cq[1], ck0 = ck[0], ck1 = ck[1];
  asm volatile("" ::"s"(ck0), "s"(ck1));  // keep the key-length loads ahead of the early exit
  const int q_begin = cq0;
  const int Lq = cu_q_p ? cq1 - cq0 : a.lq;
  const int k_begin = ck0;
  const int Lk = cu_k_p ? ck1 - ck0 : a.lk;
  const int qs = qblk * kPrefillBM;
  if (qs >= Lq) return;
  const int qe = min(qs + kPrefillBM, Lq);
  const int pos_off = (a.causal == SP_CAUSAL_TOP_LEFT) ? 0 : Lk - Lq;
  // keys any query of this workgroup can see: [kv_lo, kv_hi)
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  const int t_first = (kv_lo / BN) * BN, kv_end = kv_hi;

  const int l32 = lane & 31, hh = lane >> 5;  // MFMA column (query) and half
  const int i16 = lane & 15, g4 = lane >> 4;  // 16-lane group for the transpose reads

  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 2;
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) *
          dtype_size((sp_dtype)a.out_dtype);
  const int64_t kv0 = (a.cu_k ? (int64_t)k_begin * a.kv_tok : (int64_t)seq * a.kv_batch) +
                      (int64_t)kvh * a.kv_head;
  const bool v_wave = wave >= 2;
  const int64_t row_pitch = (int64_t)a.kv_tok * 2;
  const char* src_base = (const char*)(v_wave ? a.v : a.k) + kv0 * 2;
  const int wrow0 = (wave & 1) * WROWS;

  // ---- HBM -> LDS tile loads: wave w's load u moves rows (w & 1) WROWS + u RPI .. of the tile
  // (K for waves 0-1, V for waves 2-3); lane `lane` takes physical chunk lane % CPR of row
  // lane / CPR and fetches the logical chunk the swizzle puts there. Interior tiles share one
  // scalar base and one M0 write for the four loads (instruction offsets 0-3 KiB); edge tiles
  // clamp their rows into [kv_lo, kv_hi) (those scores are masked) with per-lane addresses.
  int voff_g[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = wrow0 + u * RPI + lane / CPR;
    voff_g[u] = (int)((int64_t)r * row_pitch) + 16 * ((lane % CPR) ^ C::swz(r)) - u * 1024;
  }
  auto issue_tile = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if (t0 >= kv_lo && t0 + BN <= kv_hi) {
      const char* sb = src_base + (int64_t)t0 * row_pitch;
      lds_dma16x4(sb, sb, sb, sb, voff_g[0], voff_g[1], voff_g[2], voff_g[3], dst);
      return;
    }
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int R = wrow0 + u * RPI + ln / CPR, p = ln % CPR;
      const int j = min(max(t0 + R, kv_lo), kv_hi - 1);
      lds_dma16(src_base + (int64_t)j * row_pitch + (p ^ C::swz(R)) * 16, dst + u * 1024);
    }
  };

  // Prologue: the first two tiles' loads go out ahead of the Q loads, and one wait covers all
  // of them, so that no wait inside the key loop refers to Q.
  int t0 = t_first;
  if (t0 < kv_end) {
    issue_tile(t0, v_wave ? vl[0] : kl[0]);
    if (t0 + BN < kv_end) issue_tile(t0 + BN, v_wave ? vl[1] : kl[1]);
  }
  // ---- Q^T operand (B of the S^T MFMA): query wq0 + l32, dims 16c + 8hh .. +7, unscaled.
  const int wq0 = qs + 32 * wave;
  const int my_q = wq0 + l32;
  const float c2 = a.scale_log2;  // > 0 (checked on the host)
  uint4 qreg[KC];
  {
    const char* qp = qbase + (int64_t)min(my_q, qe - 1) * a.q_tok * 2;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[c] = my_q < qe ? *(const uint4*)(qp + (16 * c + 8 * hh) * 2) : make_uint4(0, 0, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

  // Online softmax state of query l32 (both lanes of a query hold the same values): m_run, the
  // running maximum of the exponents x = q.k * scale * log2(e) (-inf before the first visible
  // key); m_used, the offset subtracted from x (m_run once that is finite, else 0).
  float m_run = -INFINITY, m_used = 0.f, l_run = 0.f;
  pf_f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  pf_f32x16 zero16;
#pragma unroll
  for (int r = 0; r < 16; ++r) zero16[r] = 0.f;

  const int wq_lo = wq0, wq_hi = min(wq0 + 32, qe) - 1;  // this wave's queries (inclusive)
  const bool wave_active = wq_lo < qe;
  const int qpos = my_q + pos_off;
  const int sw = C::swz(l32);
  // A tile needs masking iff t0 < mask_below or t0 > mask_above (wave-uniform bounds).
  int mask_below = kv_lo, mask_above = Lk - BN;
  if (a.causal != SP_CAUSAL_NONE) mask_above = min(mask_above, wq_lo + pos_off - BN + 1);
  if (a.window_left >= 0) mask_below = max(mask_below, wq_hi + pos_off - a.window_left);
  mask_below = wave_uniform(mask_below);
  mask_above = wave_uniform(mask_above);

  // Lane parts of the LDS operand addresses: every operand of a tile sits at (lane part ^
  // constant) + immediate offset.
  const int k_lane = (l32 * RB) | (16 * (hh ^ sw));
  const int rl = (g4 >> 1) * 4 + (i16 >> 2);
  const int chl = (g4 & 1) * 2 + ((i16 & 3) >> 1);
  const int v_lane0 = rl * RB + 16 * (chl ^ C::swz(rl)) + 8 * (i16 & 1);
  const int v_lane1 = (rl + 8) * RB + 16 * (chl ^ C::swz(rl + 8)) + 8 * (i16 & 1);

  // 32-aligned causal diagonal: the tile that starts at the wave's first query position is the
  // triangle 8(r/4) + r%4 <= l32 - 4hh (later tiles are not visited).
  const int diag0 = wave_uniform(wq_lo + pos_off);
  const bool tri_ok = a.causal != SP_CAUSAL_NONE && pos_off >= 0 && (pos_off & 31) == 0 &&
                      qe - 1 + pos_off < Lk;
  const int tri_lim = l32 - 4 * hh;

  // QK product S^T = K Q^T of the tile in LDS buffer kb: K operand i (k-step i) is row l32,
  // chunk 2i + hh: k_lane ^ 32i. Four operand reads run ahead of the MFMAs.
  constexpr int AHK = 4;
  auto qk = [&](const char* kb, pf_f32x16& s) __attribute__((always_inline)) {
    int kbl = k_lane;
    asm volatile("" : "+v"(kbl));
    auto read_k = [&](int i) __attribute__((always_inline)) {
      return *(const uint4*)(kb + (kbl ^ (32 * i)));
    };
    uint4 kop[AHK];
#pragma unroll
    for (int i = 0; i < AHK; ++i) kop[i] = read_k(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const uint4 cur = kop[i % AHK];
      if (i + AHK < KC) kop[i % AHK] = read_k(i + AHK);
      s = M::mma(cur, qreg[i], i < 1 ? zero16 : s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Masks, only on tiles that cross the sequence end, the window edge, kv_lo or the causal
  // diagonal. Score r of this lane is key t0 + 4hh + 8(r/4) + r%4.
  const float* mrow = a.mask ? a.mask + (int64_t)seq * a.mask_b + (int64_t)h * a.mask_h +
                                   (int64_t)min(my_q, qe - 1) * a.mask_q
                             : nullptr;
  auto apply_mask = [&](int t0, pf_f32x16& s) __attribute__((always_inline)) {
    if (mrow) {
      const int jb = t0 + 4 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = min(jb + 8 * (r >> 2) + (r & 3), Lk - 1);
        s[r] += mrow[key] * a.inv_scale;
      }
    }
    if (t0 < mask_below || t0 > mask_above) {
      if (tri_ok && t0 >= mask_below && t0 == diag0) {
        int tl = tri_lim;
        asm volatile("" : "+v"(tl));
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = (8 * (r >> 2) + (r & 3) <= tl) ? s[r] : -INFINITY;
      } else {
        int lo = kv_lo, hi = Lk - 1;
        if (a.causal != SP_CAUSAL_NONE) hi = min(hi, qpos);
        if (a.window_left >= 0) lo = max(lo, qpos - a.window_left);
        const int jb = t0 + 4 * hh;
        const int olo = lo - jb, ohi = hi - jb;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = (r >> 2) * 8 + (r & 3);
          s[r] = (off >= olo && off <= ohi) ? s[r] : -INFINITY;
        }
      }
    }
  };

  // Softmax weights of one tile (FlashAttention-2 online softmax, Dao 2023) with a lazily raised
  // maximum, as in prefill_kernel: p = 2^(s * scale * log2 e - m_used) packed to 16 bits; pb[ks]
  // word c holds scores 8ks + 2c, +1; the row sums add the 16-bit values the PV product uses.
  uint4 pb[2];
  float la = 0.f, lb = 0.f;
  auto weights_all = [&](const pf_f32x16& s, float off) __attribute__((always_inline)) {
    la = 0.f;
    lb = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k0 = 2 * e;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[k0], c2, -off));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[k0 + 1], c2, -off));
      const uint32_t w = M::pack(p0, p1);
      const int ks = k0 >> 3, c = (k0 >> 1) & 3;
      if (c == 0) pb[ks].x = w;
      else if (c == 1) pb[ks].y = w;
      else if (c == 2) pb[ks].z = w;
      else pb[ks].w = w;
      if (ks < 1) la = M::sum2(w, la);
      else lb = M::sum2(w, lb);
    }
  };
  constexpr float kLazyBound = 4096.f;  // 2^12
  // Raise the maximum when this lane's weights of the tile sum past 2^12 or while the query has
  // no maximum yet, and recompute the weights against the exact new maximum.
  auto finish_weights = [&](const pf_f32x16& s) __attribute__((always_inline)) {
    float lsum = la + lb;
    if (__any(lsum > kLazyBound || m_run == -INFINITY)) {
      float x = max3f(s[0], s[1], s[2]);
      float y = max3f(s[8], s[9], s[10]);
      x = max3f(x, s[3], s[4]);
      y = max3f(y, s[11], s[12]);
      x = max3f(x, s[5], s[6]);
      y = max3f(y, s[13], s[14]);
      x = max3f(x, s[7], y);
      x = __builtin_fmaxf(x, s[15]);
      float x0, x1;
      swap_halves(x, x0, x1);
      const float m_new = __builtin_fmaxf(m_run, __builtin_fmaxf(x0, x1) * c2);
      const float used_new = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - used_new);  // 0 while m_run = -inf
      weights_all(s, used_new);
      lsum = la + lb;
      m_run = m_new;
      m_used = used_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    }
    l_run += lsum;
  };

  // PV product O^T += V^T P^T of the tile in LDS buffer vb: K-step ks covers tile tokens
  // 16ks .. 16ks+15 in the S^T order; the V^T operand (ks, db) is rows 16ks + rl (+ 8), chunk
  // 4db + chl. The first AH operands are read before the softmax (their LDS latency runs under
  // it), the rest AH ahead of the MFMAs.
  constexpr int NV = 2 * DB, AH = 2;
  pf_s16x8 vop[AH];
  auto read_v = [&](const char* vb, int ks, int db) __attribute__((always_inline)) {
    const char* a0 = vb + 16 * ks * RB + (v_lane0 ^ (64 * db));
    const char* a1 = vb + 16 * ks * RB + (v_lane1 ^ (64 * db));
    const pf_s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0));
    const pf_s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a1));
    return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  auto pv_pre = [&](const char* vb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < AH; ++i) vop[i] = read_v(vb, i / DB, i % DB);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto pv = [&](const char* vb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const pf_s16x8 cur = vop[i % AH];
      if (i + AH < NV) vop[i % AH] = read_v(vb, (i + AH) / DB, (i + AH) % DB);
      acc[i % DB] = M::mma(cur, pb[i / DB], acc[i % DB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // wave-uniform: does this wave see any key of the tile ([vis_lo, vis_hi), worked out once)
  int vis_lo = -(1 << 30), vis_hi = wave_active ? kv_end : -(1 << 30);
  if (a.causal != SP_CAUSAL_NONE) vis_hi = min(vis_hi, wq_hi + pos_off + 1);
  if (a.window_left >= 0) vis_lo = wq_lo + pos_off - a.window_left - BN + 1;
  vis_lo = wave_uniform(vis_lo);
  vis_hi = wave_uniform(vis_hi);

  // One step on tile t0 (K in kcur, V in vcur): wait for this wave's loads of t0 (those of
  // t0 + BN, NLD DMAs issued after them, may stay in flight; the last tile waits for all), then
  // for every wave's; the barrier also frees the buffers of t0 - BN, which take t0 + 2 BN.
  pf_f32x16 sc;
  auto step = [&](int t0, const char* kcur, const char* vcur, char* kload, char* vload)
      __attribute__((always_inline)) {
    if (t0 + BN < kv_end) __builtin_amdgcn_s_waitcnt(0x0F70 | NLD);
    else __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (t0 + 2 * BN < kv_end) issue_tile(t0 + 2 * BN, v_wave ? vload : kload);
    if (t0 >= vis_lo && t0 < vis_hi) {
      qk(kcur, sc);
      pv_pre(vcur);
      apply_mask(t0, sc);
      float off = m_used;
      asm volatile("" : "+v"(off));
      weights_all(sc, off);
      finish_weights(sc);
      pv(vcur);
    }
  };
  while (t0 < kv_end) {
    step(t0, kl[0], vl[0], kl[2], vl[2]);
    t0 += BN;
    if (t0 >= kv_end) break;
    step(t0, kl[1], vl[1], kl[0], vl[0]);
    t0 += BN;
    if (t0 >= kv_end) break;
    step(t0, kl[2], vl[2], kl[1], vl[1]);
    t0 += BN;
  }

  // ---- normalise and store: lane holds O^T[d][query l32], d = 32db + 8(r/4) + 4hh + r%4
  float x0, x1;
  swap_halves(l_run, x0, x1);
  const float l = x0 + x1;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  constexpr int kSelf = std::is_same<T, bf16_t>::value ? SP_BF16 : SP_F16;  // out = in type
  if (a.out_dtype == kSelf) {
    // Whole output rows through an LDS stage (store_rows_staged). The stage is a ring buffer the
    // last step's barrier freed: not the last tile's (other waves may still read it), and no
    // load is pending into it (the last step waited for all). With n steps, the last used
    // buffer is (n - 1) % 3; the free ones are n % 3 (waves 0-1) and (n + 1) % 3 (waves 2-3),
    // K half or V half by wave parity.
    static_assert(TILE >= 32 * RB, "a 32-row stage per K or V buffer");
    const int nsteps = kv_end > t_first ? (kv_end - t_first + BN - 1) / BN : 0;
    const int fb = wave_uniform((nsteps + (wave >> 1)) % 3);
    store_rows_staged<M, D>(acc, inv, (wave & 1) ? vl[fb] : kl[fb], obase, a.o_tok, wq0, qe,
                            lane);
    return;
  }
  if (my_q >= qe) return;
  const int oes = dtype_size((sp_dtype)a.out_dtype);
  char* op = obase + (int64_t)my_q * a.o_tok * oes;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d0 = db * 32 + rg * 8 + hh * 4;
      const float o0 = acc[db][rg * 4 + 0] * inv, o1 = acc[db][rg * 4 + 1] * inv;
      const float o2 = acc[db][rg * 4 + 2] * inv, o3 = acc[db][rg * 4 + 3] * inv;
      if (a.out_dtype == SP_F32) {
        *(float4*)(op + d0 * 4) = make_float4(o0, o1, o2, o3);
      } else if (a.out_dtype == kSelf) {
        *(uint2*)(op + d0 * 2) = make_uint2(M::pack(o0, o1), M::pack(o2, o3));
      } else {  // the other 16-bit type
        using O = PrefillMfma<typename std::conditional<kSelf == SP_BF16, f16_t, bf16_t>::type>;
        *(uint2*)(op + d0 * 2) = make_uint2(O::pack(o0, o1), O::pack(o2, o3));
      }
    }
}

// Head dim 256 (Gemma-4's sliding-window layers, gemma4.rs:94-102; griffin.rs:63): prefill_kernel's
// per-wave state does not fit at this width (O^T alone is 128 VGPRs per lane), so 32-key tiles
// (one 32 x 32 score block, 16 VGPRs) with the softmax between the two products, two workgroups
// per CU and the tiles loaded one ahead through two buffers (64 KiB of LDS). Contiguous and
// paged K/V, the same masks and arguments as prefill_kernel; no key split. CAP: the logit soft
// cap (a.cap_in / a.cap_out) applied to each tile's raw products before the masks.
template <typename T, int D, bool PAGED, bool CAP = false>
__global__ void __launch_bounds__(256, 2) prefill_wide_kernel(PrefillArgs a) {
  using C = PrefillCfg<D>;  // the row swizzle
  using M = PrefillMfma<T>;
  constexpr int BN = 32, RB = C::RB, CPR = C::CPR, TILE = BN * RB;
  constexpr int KC = C::KC, DB = C::DB;
  constexpr int RPI = 1024 / RB;       // rows per 1 KiB load
  constexpr int NLD = TILE / 2048;     // loads per wave per tile: waves 0-1 fill K, 2-3 fill V
  constexpr int WROWS = NLD * RPI;     // rows of a tile one wave loads (half the tile)
  static_assert(WROWS * 2 == BN, "two waves fill one tile");
  __shared__ __attribute__((aligned(1024))) char kl[2][TILE];
  __shared__ __attribute__((aligned(1024))) char vl[2][TILE];

  // ---- workgroup -> (kv head, group member, sequence, split, query block), heavy query blocks
  // first; wave w takes queries 32w .. 32w + 31 of the block
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  // the metadata pointers are read with the grid shape, in the first batch of argument loads
  const int32_t* const cu_q_p = a.cu_q;
  const int32_t* const cu_k_p = PAGED ? a.context_lens : a.cu_k;
  int id = blockIdx.x;
  const int kvh = id % a.hkv;
  id /= a.hkv;
  const int gm = id % a.group;
  id /= a.group;
  const int seq = id % a.num_seqs;
  id /= a.num_seqs;
  const int split = id % a.nsplit;
  const int qblk = a.num_qblocks - 1 - id / a.nsplit;
  const int h = kvh * a.group + gm;

  // Sequence offsets and lengths. The scalar loads are issued whatever the layout (a batch
  // without cu_q / cu_k reads a zero pair instead), so they go out together and are waited for
  // once.
  const kconst_i32 cq = cu_q_p ? as_const(cu_q_p) + seq : as_const(kPrefillZeroPair);
  const kconst_i32 ck = PAGED || cu_k_p ? as_const(cu_k_p) + seq : as_const(kPrefillZeroPair);
  const int cq0 = cq[0], cq1 = cq[1], ck0 = ck[0], ck1 = PAGED ? 0 : ck[1];
  asm volatile("" ::"s"(ck0), "s"(ck1));  // keep the key-length loads ahead of the early exit
  const int q_begin = cq0;
  const int Lq = cu_q_p ? cq1 - cq0 : a.lq;
  int Lk, k_begin = 0;
  if constexpr (PAGED) {
    Lk = min(ck0, a.max_blocks_per_seq * a.block_size);
  } else {
    k_begin = ck0;
    Lk = cu_k_p ? ck1 - ck0 : a.lk;
  }
  const int qs = qblk * kPrefillBM;
  if (qs >= Lq) return;
  const int qe = min(qs + kPrefillBM, Lq);
  const int pos_off = (a.causal == SP_CAUSAL_TOP_LEFT) ? 0 : Lk - Lq;
  // keys any query of this workgroup can see: [kv_lo, kv_hi)
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  // This workgroup's key tiles: all of [kv_lo, kv_hi), or its 1/nsplit share of them (masks and
  // row clamps keep using the full range; only the walk stops at kv_end).
  int t_first = (kv_lo / BN) * BN, kv_end = kv_hi;
  if (a.nsplit > 1) {
    const int ntiles = kv_hi > t_first ? (kv_hi - t_first + BN - 1) / BN : 0;
    const int tps = (ntiles + a.nsplit - 1) / a.nsplit;
    t_first += split * tps * BN;
    kv_end = min(kv_hi, t_first + tps * BN);
  }

  const int l32 = lane & 31, hh = lane >> 5;        // MFMA column (query) and half
  const int i16 = lane & 15, g4 = lane >> 4;        // 16-lane group for the transpose reads

  // ---- per-sequence base addresses
  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 2;
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) *
          dtype_size((sp_dtype)a.out_dtype);
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

  // ---- Q^T operand (B of the S^T MFMA): query wq0 + l32, dims 16c + 8hh .. +7, unscaled.
  const int wq0 = qs + 32 * wave;
  const int my_q = wq0 + l32;
  // > 0 (checked on the host); with the soft cap the scores already are exponents
  const float c2 = CAP ? 1.f : a.scale_log2;
  uint4 qreg[KC];
  {
    const char* qp = qbase + (int64_t)min(my_q, qe - 1) * a.q_tok * 2;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[c] = my_q < qe ? *(const uint4*)(qp + (16 * c + 8 * hh) * 2) : make_uint4(0, 0, 0, 0);
  }

  // ---- HBM -> LDS tile loads. Waves 0-1 fill K tiles and waves 2-3 V tiles, one tile ahead of
  // the step that reads them. Wave w's load u moves 1 KiB = RPI rows, r_u = (w & 1) * WROWS + u * RPI ..;
  // lane `lane` takes physical chunk p = lane % CPR of row r_u + lane / CPR and fetches the
  // logical chunk that the swizzle puts there. Interior tiles (every row inside [kv_lo, kv_hi))
  // take the fast path: one scalar base per tile (non-paged) or per block (paged) plus a constant
  // lane offset per load. Edge tiles clamp rows outside [kv_lo, kv_hi) to a valid row (their
  // scores are masked) and compute per-lane addresses.
  const bool v_wave = wave >= 2;
  const int wrow0 = (wave & 1) * WROWS;
  const int64_t row_pitch = PAGED ? (int64_t)RB : (int64_t)a.kv_tok * 2;
  const char* src_base = PAGED ? (v_wave ? a.vpool : a.kpool) : (v_wave ? vbase : kbase);
  // paged fast path: a wave's WROWS rows of a tile lie in whole blocks (block_size divides the
  // 32-row tile, and a load never straddles blocks)
  const bool paged_fast = PAGED && a.block_size % RPI == 0 && BN % a.block_size == 0;
  int voff[NLD];  // lane part of each load's source offset (bytes), row offset included
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = wrow0 + u * RPI + lane / CPR;  // tile row
    const int64_t row_b = PAGED ? (int64_t)(r % max(a.block_size, 1)) * RB : (int64_t)r * row_pitch;
    voff[u] = (int)row_b + 16 * ((lane % CPR) ^ C::swz(r));
  }
  static_assert(NLD % 4 == 0, "tile loads go out in groups of four");
  // Interior tiles issue their loads in groups of four with instruction offsets 0, 1, 2, 3 KiB.
  // Contiguous K/V: the offsets come out of the lane offsets (still >= 0: load u's rows start at
  // u RPI rows of at least RB bytes, u RPI RB = 1024 u). Paged with blocks that hold whole groups
  // (block_size a multiple of 4 RPI rows, so a group's rows lie in one block): the same, with one
  // base per group. Smaller blocks: out of the per-load bases.
  const bool group_blk = wave_uniform(PAGED && a.block_size % (4 * RPI) == 0);
  int voff_g[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u)
    voff_g[u] = (!PAGED || group_blk) ? voff[u] - (u & 3) * 1024 : voff[u];
  auto tile_interior = [&](int t0) __attribute__((always_inline)) {
    return t0 >= kv_lo && t0 + BN <= kv_hi;
  };
  // Paged fast path: the block ids of the rows of the next tile this wave loads, fetched one
  // tile ahead so that no load waits on a dependent block-table read. Lane u < NLD fetches load
  // u's id with a vector load: it completes with the tile loads at the next step's wait, where a
  // scalar load would sit in lgkmcnt ahead of the LDS operand reads of the QK product and make
  // each of their waits a wait for the table read.
  // block_size divides the 32-key tile here, so it is a power of two and every tile start t0 is
  // a multiple of it: the id of the block holding row t0 + r is table[(t0 >> shift) + (r >> shift)].
  int nblk = 0;
  const int bs_shift = paged_fast ? wave_uniform(31 - __builtin_clz(max(a.block_size, 1))) : 0;
  const int lane_blk = (wrow0 + min(lane, NLD - 1) * RPI) >> bs_shift;
  auto fetch_blocks = [&](int t0) __attribute__((always_inline)) {
    if constexpr (PAGED) {
      if (paged_fast && t0 < kv_end && tile_interior(t0)) nblk = table[(t0 >> bs_shift) + lane_blk];
    }
  };
  // Interior tile: its loads go out in groups of four that share one M0 write.
  auto issue_interior = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if constexpr (PAGED) {
      // block ids fetched by fetch_blocks(t0), load u's in lane u: every lane turns its id into
      // its load's base address at once (vector ops), and each load reads its base out of lane u
      // (two readlanes), instead of a scalar chain of compares and 64-bit multiplies per load.
      // The base is taken less the load's instruction offset; the sum is the block's row address.
      const int bl = (nblk >= 0 && nblk < a.num_blocks) ? nblk : 0;  // never outside the pool
      const uint64_t vb = (uint64_t)(uintptr_t)(src_base + head_off) +
                          (uint64_t)bl * (uint64_t)a.block_stride_b - (uint64_t)((lane & 3) * 1024);
      const int vb_lo = (int)(uint32_t)vb, vb_hi = (int)(uint32_t)(vb >> 32);
      auto base_of = [&](int u) __attribute__((always_inline)) {
        const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane(vb_lo, u);
        const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane(vb_hi, u);
        return (const char*)(uintptr_t)((hi << 32) | lo);
      };
      if (group_blk) {  // lane g (g % 4 == 0) holds its group's block; no offset taken off
#pragma unroll
        for (int g = 0; g < NLD; g += 4) {
          const char* b = base_of(g);
          lds_dma16x4(b, b, b, b, voff_g[g], voff_g[g + 1], voff_g[g + 2], voff_g[g + 3],
                      dst + g * 1024);
        }
      } else {
#pragma unroll
        for (int g = 0; g < NLD; g += 4)
          lds_dma16x4(base_of(g), base_of(g + 1), base_of(g + 2), base_of(g + 3), voff_g[g],
                      voff_g[g + 1], voff_g[g + 2], voff_g[g + 3], dst + g * 1024);
      }
    } else {
      const char* sb = src_base + (int64_t)t0 * row_pitch;
#pragma unroll
      for (int g = 0; g < NLD; g += 4)
        lds_dma16x4(sb, sb, sb, sb, voff_g[g], voff_g[g + 1], voff_g[g + 2], voff_g[g + 3],
                    dst + g * 1024);
    }
  };
  auto issue_tile = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if (tile_interior(t0) && (!PAGED || paged_fast)) {
      issue_interior(t0, buf);
      return;
    }
    // Edge tiles are rare: the lane id goes through an empty asm so that the per-lane source
    // addresses are derived here, not hoisted out of the key loop as live registers.
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int R = wrow0 + u * RPI + ln / CPR, p = ln % CPR;
      const int c = p ^ C::swz(R);
      const int j = min(max(t0 + R, kv_lo), kv_hi - 1);
      const char* src;
      if constexpr (PAGED) {
        int blk = table[j / a.block_size];
        blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;  // never dereference outside the pool
        src = src_base + (int64_t)blk * a.block_stride_b + head_off +
              (int64_t)(j % a.block_size) * RB + c * 16;
      } else {
        src = src_base + (int64_t)j * row_pitch + c * 16;
      }
      lds_dma16(src, dst + u * 1024);
    }
  };

  // Online softmax state of query l32 (both lanes of a query hold the same values).
  // m_run: running maximum of the exponents x = q.k * scale * log2(e) seen (-inf before the
  // first visible key); m_used: the offset subtracted from x (m_run once that is finite, else 0).
  float m_run = -INFINITY, m_used = 0.f, l_run = 0.f;
  pf_f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  pf_f32x16 zero16;
#pragma unroll
  for (int r = 0; r < 16; ++r) zero16[r] = 0.f;

  const int wq_lo = wq0, wq_hi = min(wq0 + 32, qe) - 1;  // this wave's queries (inclusive)
  const bool wave_active = wq_lo < qe;
  const int qpos = my_q + pos_off;
  const int sw = C::swz(l32);     // swizzle of the K rows this lane reads (row & 15 == l32 & 15)
  // A tile needs masking iff t0 < mask_below or t0 > mask_above (wave-uniform bounds): it starts
  // before kv_lo or before the window edge of this wave's last query, or it runs past the
  // sequence end or past the causal diagonal of this wave's first query.
  int mask_below = kv_lo, mask_above = Lk - BN;
  if (a.causal != SP_CAUSAL_NONE) mask_above = min(mask_above, wq_lo + pos_off - BN + 1);
  if (a.window_left >= 0) mask_below = max(mask_below, wq_hi + pos_off - a.window_left);
  mask_below = wave_uniform(mask_below);
  mask_above = wave_uniform(mask_above);

  // Lane parts of the LDS operand addresses (byte offsets inside a tile). With the XOR swizzle
  // an operand's logical chunk index only flips bits the lane part owns alone, so every operand
  // of a tile sits at (lane part ^ constant) + immediate offset.
  const int k_lane = (l32 * RB) | (16 * (hh ^ sw));
  const int rl = (g4 >> 1) * 4 + (i16 >> 2);
  const int chl = (g4 & 1) * 2 + ((i16 & 3) >> 1);
  const int v_lane0 = rl * RB + 16 * (chl ^ C::swz(rl)) + 8 * (i16 & 1);
  const int v_lane1 = (rl + 8) * RB + 16 * (chl ^ C::swz(rl + 8)) + 8 * (i16 & 1);

  // Causal diagonal at 32-key granularity (see the mask below).
  const int diag0 = wave_uniform(wq_lo + pos_off);
  const bool tri_ok = a.causal != SP_CAUSAL_NONE && pos_off >= 0 && (pos_off & 31) == 0 &&
                      qe - 1 + pos_off < Lk;
  const int tri_lim = l32 - 4 * hh;

  // ---- the pieces of one key tile -------------------------------------------------------------
  // QK product S^T = K Q^T of the tile in LDS buffer kb into s (one 32 x 32 block). K operand i
  // (k-step i) is row l32, chunk 2i + hh: k_lane ^ 32i. `between(i)` runs after MFMA i.
  constexpr int NK = KC, AHK = PAGED ? 1 : 2;  // paged: four VGPRs for the block bases
  auto qk = [&](const char* kb, pf_f32x16& s, auto&& between) __attribute__((always_inline)) {
    int kbl = k_lane;
    asm volatile("" : "+v"(kbl));
    auto read_k = [&](int i) __attribute__((always_inline)) {
      return *(const uint4*)(kb + (kbl ^ (32 * i)));
    };
    uint4 kop[AHK];
#pragma unroll
    for (int i = 0; i < AHK; ++i) kop[i] = read_k(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const uint4 cur = kop[i % AHK];
      if (i + AHK < NK) kop[i % AHK] = read_k(i + AHK);
      s = M::mma(cur, qreg[i], i < 1 ? zero16 : s);
      between(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Masks, only on tiles that cross the sequence end, the window edge, kv_lo or the causal
  // diagonal. Score r of this lane is key t0 + 4hh + off, off = 8(r/4) + r%4.
  // this lane's row of the additive mask (dense path: the sequence index is the batch index)
  const float* mrow = a.mask ? a.mask + (int64_t)seq * a.mask_b + (int64_t)h * a.mask_h +
                                   (int64_t)min(my_q, qe - 1) * a.mask_q
                             : nullptr;
  auto apply_mask = [&](int t0, pf_f32x16& s) __attribute__((always_inline)) {
    if (mrow) {
      const int jb = t0 + 4 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = min(jb + 8 * (r >> 2) + (r & 3), Lk - 1);
        s[r] += mrow[key] * a.inv_scale;
      }
    }
    if (t0 < mask_below || t0 > mask_above) {
      if (tri_ok && t0 >= mask_below && t0 == diag0) {
        int tl = tri_lim;
        asm volatile("" : "+v"(tl));
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = (8 * (r >> 2) + (r & 3) <= tl) ? s[r] : -INFINITY;
      } else {
        int lo = kv_lo, hi = Lk - 1;
        if (a.causal != SP_CAUSAL_NONE) hi = min(hi, qpos);
        if (a.window_left >= 0) lo = max(lo, qpos - a.window_left);
        const int jb = t0 + 4 * hh;
        const int olo = lo - jb, ohi = hi - jb;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = (r >> 2) * 8 + (r & 3);
          s[r] = (off >= olo && off <= ohi) ? s[r] : -INFINITY;
        }
      }
    }
  };

  // Softmax weights of one tile for query l32 (FlashAttention-2 online softmax, Dao 2023) with a
  // lazily raised maximum: p = 2^(s * scale * log2 e - m_used), packed to 16 bits for the PV
  // product; the row sum adds the 16-bit values the PV product uses (v_dot2 against ones).
  // Slice e (of 8) computes the two scores 2e, 2e+1 of the lane.
  uint4 pb[2];
  float la = 0.f, lb = 0.f;
  auto weights_slice = [&](const pf_f32x16& s, int e, float off) __attribute__((always_inline)) {
    const int k0 = 2 * e;
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[k0], c2, -off));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[k0 + 1], c2, -off));
    const uint32_t w = M::pack(p0, p1);
    const int ks = k0 >> 3, c = (k0 >> 1) & 3;  // pb[ks] word c holds scores 8ks + 2c, +1
    if (c == 0) pb[ks].x = w;
    else if (c == 1) pb[ks].y = w;
    else if (c == 2) pb[ks].z = w;
    else pb[ks].w = w;
    if (ks < 1) la = M::sum2(w, la);
    else lb = M::sum2(w, lb);
  };
  auto weights_all = [&](const pf_f32x16& s, float off) __attribute__((always_inline)) {
    la = 0.f;
    lb = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) weights_slice(s, e, off);
  };
  constexpr float kLazyBound = 4096.f;  // 2^kLazy, kLazy = 12
  auto finish_weights = [&](const pf_f32x16& s) __attribute__((always_inline)) {
    float lsum = la + lb;
    if (__any(lsum > kLazyBound || m_run == -INFINITY)) {
      float mq[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int r0 = k * 8;
        float x = max3f(s[r0], s[r0 + 1], s[r0 + 2]);
        x = max3f(x, s[r0 + 3], s[r0 + 4]);
        x = max3f(x, s[r0 + 5], s[r0 + 6]);
        mq[k] = __builtin_fmaxf(x, s[r0 + 7]);
      }
      float mx = __builtin_fmaxf(mq[0], mq[1]);
      float x0, x1;
      swap_halves(mx, x0, x1);
      const float m_new = __builtin_fmaxf(m_run, __builtin_fmaxf(x0, x1) * c2);
      const float used_new = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - used_new);
      weights_all(s, used_new);
      lsum = la + lb;
      m_run = m_new;
      m_used = used_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    }
    l_run += lsum;
  };

  // PV product O^T += V^T P^T of the tile in LDS buffer vb: K-step ks covers tile tokens
  // 16ks .. 16ks+15 in the S^T order. The V^T operand (ks, db) is rows 16ks + rl (+ 8), chunk
  // 4db + chl: (v_lane0 ^ 64db) + 16ks RB (v_lane1 for the second row group), read AH ahead.
  auto pv = [&](const char* vb) __attribute__((always_inline)) {
    int vb0 = v_lane0, vb1 = v_lane1;
    asm volatile("" : "+v"(vb0), "+v"(vb1));
    auto read_v = [&](int ks, int db) __attribute__((always_inline)) {
      const char* a0 = vb + 16 * ks * RB + (vb0 ^ (64 * db));
      const char* a1 = vb + 16 * ks * RB + (vb1 ^ (64 * db));
      const pf_s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0));
      const pf_s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a1));
      return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    constexpr int NV = 2 * DB, AH = PAGED ? 1 : 2;
    pf_s16x8 vop[AH];
#pragma unroll
    for (int i = 0; i < AH; ++i) vop[i] = read_v(i / DB, i % DB);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const pf_s16x8 cur = vop[i % AH];
      if (i + AH < NV) vop[i % AH] = read_v((i + AH) / DB, (i + AH) % DB);
      acc[i % DB] = M::mma(cur, pb[i / DB], acc[i % DB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // wave-uniform: does this wave see any key of the tile. The conditions (the wave has queries,
  // the tile starts before kv_end, at or before the causal diagonal of the wave's last query, and
  // ends at or after the window edge of its first query) bound t0 from both sides, so they
  // reduce to one range [vis_lo, vis_hi) worked out once.
  int vis_lo = -(1 << 30), vis_hi = wave_active ? kv_end : -(1 << 30);
  if (a.causal != SP_CAUSAL_NONE) vis_hi = min(vis_hi, wq_hi + pos_off + 1);
  if (a.window_left >= 0) vis_lo = wq_lo + pos_off - a.window_left - BN + 1;
  vis_lo = wave_uniform(vis_lo);
  vis_hi = wave_uniform(vis_hi);
  auto visits = [&](int t0) __attribute__((always_inline)) { return t0 >= vis_lo && t0 < vis_hi; };

  // One step on tile t0 (its K in kcur, its V in vcur): wait until this step's tiles are in (own
  // loads, then everyone's; the barrier also guarantees every wave is done with the other
  // buffers), start the next tile's loads into kload / vload, then QK product, softmax, PV.
  pf_f32x16 sc;
  auto step = [&](int t0, const char* kcur, const char* vcur, char* kload, char* vload)
      __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    {
      const int lt = t0 + BN;
      if (lt < kv_end) {
        issue_tile(lt, v_wave ? vload : kload);
        fetch_blocks(lt + BN);
      }
    }
    if (visits(t0)) {
      qk(kcur, sc, [](int) {});
      if constexpr (CAP) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = softcap_log2(sc[r], a.cap_in, a.cap_out);
      }
      apply_mask(t0, sc);
      float off = m_used;
      asm volatile("" : "+v"(off));
      la = 0.f;
      lb = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) weights_slice(sc, e, off);
      finish_weights(sc);
      pv(vcur);
    }
  };

  int t0 = t_first;
  if (t0 < kv_end) {
    fetch_blocks(t0);
    issue_tile(t0, v_wave ? vl[0] : kl[0]);
    fetch_blocks(t0 + BN);
  }
  while (t0 < kv_end) {
    step(t0, kl[0], vl[0], kl[1], vl[1]);
    t0 += BN;
    if (t0 >= kv_end) break;
    step(t0, kl[1], vl[1], kl[0], vl[0]);
    t0 += BN;
  }

  // ---- normalise and store: lane holds O^T[d][query l32], d = 32db + 8(r/4) + 4hh + r%4
  float x0, x1;
  swap_halves(l_run, x0, x1);
  const float l = x0 + x1;
  constexpr int kSelf = std::is_same<T, bf16_t>::value ? SP_BF16 : SP_F16;  // out = in type
  if (a.nsplit <= 1 && a.out_dtype == kSelf) {
    // Whole output rows through an LDS stage (store_rows_staged, two passes of 128 dims). The
    // stage is a quarter of the buffer pair the last step did not read: with n steps the last
    // read pair n - 1 (mod 2), and no load is pending into pair n % 2 (the last step issued
    // none and waited for all before its barrier, which also ended every read of that pair).
    // Waves 0-1 take kl, waves 2-3 vl, 8 KiB each.
    static_assert(TILE >= 2 * 32 * 256, "two 32-row x 128-dim stages per buffer");
    const int nsteps = kv_end > t_first ? (kv_end - t_first + BN - 1) / BN : 0;
    const int fb = wave_uniform(nsteps % 2);
    store_rows_staged<M, D>(acc, l > 0.f ? 1.f / l : 0.f,
                            ((wave >> 1) ? vl[fb] : kl[fb]) + (wave & 1) * 32 * 256, obase,
                            a.o_tok, wq0, qe, lane);
    return;
  }
  if (my_q >= qe) return;
  if (a.nsplit > 1) {
    // partial record (m, l, -, -, acc[D]) of this split; m is the offset the weights are
    // relative to, -inf when the split saw no visible key (then l = 0 and acc = 0), so that the
    // merge never takes an empty split's offset as the row maximum. Rows past max_q (a caller
    // whose cu_seqlens exceed max_seqlen_q) have no record slot and are not written.
    if (my_q >= a.max_q) return;
    float* rec = a.partials +
        ((((int64_t)seq * a.max_q + my_q) * a.hq + h) * a.nsplit + split) * (D + 4);
    if (hh == 0) *(float2*)rec = make_float2(m_run == -INFINITY ? -INFINITY : m_used, l);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg)
        *(float4*)(rec + 4 + db * 32 + rg * 8 + hh * 4) =
            make_float4(acc[db][rg * 4 + 0], acc[db][rg * 4 + 1], acc[db][rg * 4 + 2],
                        acc[db][rg * 4 + 3]);
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int oes = dtype_size((sp_dtype)a.out_dtype);
  char* op = obase + (int64_t)my_q * a.o_tok * oes;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d0 = db * 32 + rg * 8 + hh * 4;
      const float o0 = acc[db][rg * 4 + 0] * inv, o1 = acc[db][rg * 4 + 1] * inv;
      const float o2 = acc[db][rg * 4 + 2] * inv, o3 = acc[db][rg * 4 + 3] * inv;
      if (a.out_dtype == SP_F32) {
        *(float4*)(op + d0 * 4) = make_float4(o0, o1, o2, o3);
      } else if (a.out_dtype == kSelf) {
        *(uint2*)(op + d0 * 2) = make_uint2(M::pack(o0, o1), M::pack(o2, o3));
      } else {  // the other 16-bit type
        using O = PrefillMfma<typename std::conditional<kSelf == SP_BF16, f16_t, bf16_t>::type>;
        *(uint2*)(op + d0 * 2) = make_uint2(O::pack(o0, o1), O::pack(o2, o3));
      }
    }
}

// Head dim 512 (Gemma-4's global-attention layers, gemma4.rs:82-107): a wave of 32 queries would
// hold 128 VGPRs of Q and 256 of O at this width, so each wave takes 16 queries on
// v_mfma_f32_16x16x32 (S^T blocks of 16 keys x 16 queries, O^T blocks of 16 dims x 16 queries)
// and eight waves cover the 128-query block. The K / V tiles (32 keys, 32 KiB each) go HBM -> LDS
// one ahead through two buffers (128 KiB: one workgroup of two waves per SIMD on each CU); waves
// 0-3 load K, 4-7 V, one 1 KiB row per load. Lane (g, n) (g = lane / 16, n = lane % 16) holds
// query n's scores of the tile's keys 4g .. 4g+3 and 16 + 4g .. +3, which are also the k slots
// 8g .. 8g+7 of its P^T operand; the V^T operand takes the same keys through two transpose reads.
// Contiguous and paged K/V, the masks and arguments of prefill_kernel; no key split. CAP: the
// logit soft cap (a.cap_in / a.cap_out) on each tile's raw products before the masks.
template <typename T, bool PAGED, bool CAP = false>
__global__ void __launch_bounds__(512, 1) prefill_d512_kernel(PrefillArgs a) {
  using C = PrefillCfg<512>;  // the row swizzle
  using M = PrefillMfma<T>;
  constexpr int D = 512, BN = 32, RB = C::RB, TILE = BN * RB;
  constexpr int KC = D / 32;  // QK k-steps (32 dims each)
  constexpr int DB = D / 16;  // PV output blocks (16 dims each)
  constexpr int NLD = 8;      // one-row loads per wave and tile
  static_assert(RB == 1024 && NLD * 4 == BN, "four waves fill one tile, a row per load");
  __shared__ __attribute__((aligned(1024))) char kl[2][TILE];
  __shared__ __attribute__((aligned(1024))) char vl[2][TILE];

  // ---- workgroup -> (kv head, group member, sequence, query block), heavy query blocks first;
  // wave w takes queries 16w .. 16w + 15 of the block
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int32_t* const cu_q_p = a.cu_q;
  const int32_t* const cu_k_p = PAGED ? a.context_lens : a.cu_k;
  int id = blockIdx.x;
  const int kvh = id % a.hkv;
  id /= a.hkv;
  const int gm = id % a.group;
  id /= a.group;
  const int seq = id % a.num_seqs;
  const int qblk = a.num_qblocks - 1 - id / a.num_seqs;
  const int h = kvh * a.group + gm;

  const kconst_i32 cq = cu_q_p ? as_const(cu_q_p) + seq : as_const(kPrefillZeroPair);
  const kconst_i32 ck = PAGED || cu_k_p ? as_const(cu_k_p) + seq : as_const(kPrefillZeroPair);
  const int cq0 = cq[0], cq1 = cq[1], ck0 = ck[0], ck1 = PAGED ? 0 : ck[1];
  asm volatile("" ::"s"(ck0), "s"(ck1));  // keep the key-length loads ahead of the early exit
  const int q_begin = cq0;
  const int Lq = cu_q_p ? cq1 - cq0 : a.lq;
  int Lk, k_begin = 0;
  if constexpr (PAGED) {
    Lk = min(ck0, a.max_blocks_per_seq * a.block_size);
  } else {
    k_begin = ck0;
    Lk = cu_k_p ? ck1 - ck0 : a.lk;
  }
  const int qs = qblk * kPrefillBM;
  if (qs >= Lq) return;
  const int qe = min(qs + kPrefillBM, Lq);
  const int pos_off = (a.causal == SP_CAUSAL_TOP_LEFT) ? 0 : Lk - Lq;
  // keys any query of this workgroup can see: [kv_lo, kv_hi)
  int kv_lo = 0, kv_hi = Lk;
  if (a.causal != SP_CAUSAL_NONE) kv_hi = min(Lk, qe - 1 + pos_off + 1);
  if (a.window_left >= 0) kv_lo = max(0, qs + pos_off - a.window_left);
  const int t_first = (kv_lo / BN) * BN, kv_end = kv_hi;

  const int n = lane & 15, g = lane >> 4;  // MFMA column (query) and row group

  // ---- per-sequence base addresses
  const char* qbase = (const char*)a.q +
      ((a.cu_q ? (int64_t)q_begin * a.q_tok : (int64_t)seq * a.q_batch) + (int64_t)h * a.q_head) * 2;
  char* obase = (char*)a.out +
      ((a.cu_q ? (int64_t)q_begin * a.o_tok : (int64_t)seq * a.o_batch) + (int64_t)h * a.o_head) *
          dtype_size((sp_dtype)a.out_dtype);
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

  // ---- HBM -> LDS tile loads. Wave w (w & 3 = j) loads rows 8j .. 8j + 7 of each tile (K for
  // waves 0-3, V for 4-7), one row per load; lane `lane` takes physical chunk `lane` of the row
  // and fetches the logical chunk the swizzle puts there. Interior tiles go out in two groups of
  // four loads that share one M0 write (instruction offsets 0-3 KiB): contiguous K/V from one
  // scalar base per tile, paged K/V from one base per block (block_size divides the tile) or per
  // group (block_size a multiple of four). Edge tiles clamp rows outside [kv_lo, kv_hi) to a
  // valid row (their scores are masked) and compute per-lane addresses.
  const bool v_wave = wave >= 4;
  const int wrow0 = (wave & 3) * NLD;
  const int64_t row_pitch = PAGED ? (int64_t)RB : (int64_t)a.kv_tok * 2;
  const char* src_base = PAGED ? (v_wave ? a.vpool : a.kpool) : (v_wave ? vbase : kbase);
  const bool paged_fast = PAGED && BN % a.block_size == 0;
  const bool group_blk = wave_uniform(PAGED && a.block_size % 4 == 0);
  // lane part of load u's source offset less its instruction offset (u % 4) KiB; >= 0: load u's
  // row lies u rows of at least RB = 1 KiB past the group's base (contiguous), or its group
  // starts a block's rows (paged, whole groups)
  int voff_g[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = wrow0 + u;
    const int chunk = 16 * (lane ^ C::swz(r));
    if constexpr (PAGED)
      voff_g[u] = (r % max(a.block_size, 1)) * RB + chunk - (group_blk ? (u & 3) * 1024 : 0);
    else
      voff_g[u] = (int)((int64_t)(u & 4) * row_pitch) + (u & 3) * (int)(row_pitch - 1024) + chunk;
  }
  auto tile_interior = [&](int t0) __attribute__((always_inline)) {
    return t0 >= kv_lo && t0 + BN <= kv_hi;
  };
  // paged: block ids of this wave's rows of the next tile, fetched a tile ahead in lanes 0-7
  int nblk = 0;
  const int bs_shift = paged_fast ? wave_uniform(31 - __builtin_clz(max(a.block_size, 1))) : 0;
  const int lane_blk = (wrow0 + min(lane, NLD - 1)) >> bs_shift;
  auto fetch_blocks = [&](int t0) __attribute__((always_inline)) {
    if constexpr (PAGED) {
      if (paged_fast && t0 < kv_end && tile_interior(t0)) nblk = table[(t0 >> bs_shift) + lane_blk];
    }
  };
  auto issue_tile = [&](int t0, char* buf) __attribute__((always_inline)) {
    char* dst = buf + wrow0 * RB;
    if (tile_interior(t0) && (!PAGED || paged_fast)) {
      if constexpr (PAGED) {
        const int bl = (nblk >= 0 && nblk < a.num_blocks) ? nblk : 0;  // never outside the pool
        const uint64_t vb = (uint64_t)(uintptr_t)(src_base + head_off) +
                            (uint64_t)bl * (uint64_t)a.block_stride_b -
                            (group_blk ? 0ull : (uint64_t)((lane & 3) * 1024));
        const int vb_lo = (int)(uint32_t)vb, vb_hi = (int)(uint32_t)(vb >> 32);
        auto base_of = [&](int u) __attribute__((always_inline)) {
          const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane(vb_lo, u);
          const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane(vb_hi, u);
          return (const char*)(uintptr_t)((hi << 32) | lo);
        };
#pragma unroll
        for (int gq = 0; gq < NLD; gq += 4) {
          if (group_blk) {
            const char* b = base_of(gq);
            lds_dma16x4(b, b, b, b, voff_g[gq], voff_g[gq + 1], voff_g[gq + 2], voff_g[gq + 3],
                        dst + gq * 1024);
          } else {
            lds_dma16x4(base_of(gq), base_of(gq + 1), base_of(gq + 2), base_of(gq + 3),
                        voff_g[gq], voff_g[gq + 1], voff_g[gq + 2], voff_g[gq + 3],
                        dst + gq * 1024);
          }
        }
      } else {
        const char* sb = src_base + (int64_t)(t0 + wrow0) * row_pitch;
#pragma unroll
        for (int gq = 0; gq < NLD; gq += 4)
          lds_dma16x4(sb, sb, sb, sb, voff_g[gq], voff_g[gq + 1], voff_g[gq + 2], voff_g[gq + 3],
                      dst + gq * 1024);
      }
      return;
    }
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int R = wrow0 + u;
      const int c = ln ^ C::swz(R);
      const int j = min(max(t0 + R, kv_lo), kv_hi - 1);
      const char* src;
      if constexpr (PAGED) {
        int blk = table[j / a.block_size];
        blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;  // never dereference outside the pool
        src = src_base + (int64_t)blk * a.block_stride_b + head_off +
              (int64_t)(j % a.block_size) * RB + c * 16;
      } else {
        src = src_base + (int64_t)j * row_pitch + c * 16;
      }
      lds_dma16(src, dst + u * 1024);
    }
  };

  // First tile's loads ahead of the Q loads.
  int t0 = t_first;
  if (t0 < kv_end) {
    fetch_blocks(t0);
    issue_tile(t0, v_wave ? vl[0] : kl[0]);
    fetch_blocks(t0 + BN);
  }

  // ---- Q^T operand (B of the S^T MFMA): query wq0 + n, dims 32c + 8g .. +7, unscaled.
  const int wq0 = qs + 16 * wave;
  const int my_q = wq0 + n;
  const float c2 = CAP ? 1.f : a.scale_log2;  // with the cap the scores already are exponents
  uint4 qreg[KC];
  {
    const char* qp = qbase + (int64_t)min(my_q, qe - 1) * a.q_tok * 2;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[c] = my_q < qe ? *(const uint4*)(qp + (32 * c + 8 * g) * 2) : make_uint4(0, 0, 0, 0);
  }

  float m_run = -INFINITY, m_used = 0.f, l_run = 0.f;
  pf_f32x4 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = pf_f32x4{0.f, 0.f, 0.f, 0.f};

  const int wq_lo = wq0, wq_hi = min(wq0 + 16, qe) - 1;  // this wave's queries (inclusive)
  const bool wave_active = wq_lo < qe;
  const int qpos = my_q + pos_off;
  int mask_below = kv_lo, mask_above = Lk - BN;
  if (a.causal != SP_CAUSAL_NONE) mask_above = min(mask_above, wq_lo + pos_off - BN + 1);
  if (a.window_left >= 0) mask_below = max(mask_below, wq_hi + pos_off - a.window_left);
  mask_below = wave_uniform(mask_below);
  mask_above = wave_uniform(mask_above);

  // LDS operand addresses: K operand (half b, k-step c) is row 16b + n, logical chunk 4c + g:
  // b 16 RB + (k_lane ^ 64c). V^T operand (keys 16b + 4g .., dims 16db ..) by transpose read: lane
  // n addresses row 16b + 4g + n / 4, dims 16db + 4(n % 4) .. +3: b 16 RB + (v_lane ^ 32db).
  const int k_lane = (n * RB) | (16 * (g ^ C::swz(n)));
  const int vr = 4 * g + (n >> 2);
  const int v_lane = (vr * RB) | (16 * (((n & 3) >> 1) ^ C::swz(vr))) | (8 * (n & 1));

  // The operand reads take LDS byte addresses: the buffer base (1 KiB aligned, so its low ten
  // bits are zero) plus the lane part, then an XOR of bits 5-9 per operand and the half's
  // 16 KiB as the instruction offset. One VALU op per read address, where pointer arithmetic
  // from the buffer's pointer cost an add more (a base past 64 KiB does not fit the offset).
  // score i of this lane is key t0 + koff(i), koff(i) = 16(i / 4) + 4g + i % 4
  float sc[8];
  auto qk = [&](const char* kb) __attribute__((always_inline)) {
    unsigned kbl = lds_addr(kb) + k_lane;
    asm volatile("" : "+v"(kbl));
    auto read_k = [&](int i) __attribute__((always_inline)) {  // operand i: half i & 1, step i / 2
      return __builtin_bit_cast(
          uint4, *(const lds_u32x4*)(uintptr_t)((kbl ^ (64u * (i >> 1))) + (i & 1) * 16 * RB));
    };
    constexpr int AHK = 2;
    uint4 kop[AHK];
#pragma unroll
    for (int i = 0; i < AHK; ++i) kop[i] = read_k(i);
    __builtin_amdgcn_sched_barrier(0);
    pf_f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 2 * KC; ++i) {
      const uint4 cur = kop[i % AHK];
      if (i + AHK < 2 * KC) kop[i % AHK] = read_k(i + AHK);
      if (i & 1) s1 = M::mma16(cur, qreg[i >> 1], s1);
      else s0 = M::mma16(cur, qreg[i >> 1], s0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sc[r] = s0[r];
      sc[4 + r] = s1[r];
    }
  };

  const float* mrow = a.mask ? a.mask + (int64_t)seq * a.mask_b + (int64_t)h * a.mask_h +
                                   (int64_t)min(my_q, qe - 1) * a.mask_q
                             : nullptr;
  auto apply_mask = [&](int t0) __attribute__((always_inline)) {
    const int jb = t0 + 4 * g;
    if (mrow) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sc[i] += mrow[min(jb + 16 * (i >> 2) + (i & 3), Lk - 1)] * a.inv_scale;
    }
    if (t0 < mask_below || t0 > mask_above) {
      int lo = kv_lo, hi = Lk - 1;
      if (a.causal != SP_CAUSAL_NONE) hi = min(hi, qpos);
      if (a.window_left >= 0) lo = max(lo, qpos - a.window_left);
      const int olo = lo - jb, ohi = hi - jb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int off = 16 * (i >> 2) + (i & 3);
        sc[i] = (off >= olo && off <= ohi) ? sc[i] : -INFINITY;
      }
    }
  };

  // Softmax weights (FlashAttention-2 online softmax, Dao 2023) with the lazily raised maximum
  // of prefill_kernel: p = 2^(s c2 - m_used), packed to 16 bits in k-slot order (pb word e holds
  // scores 2e, 2e + 1); the row sum adds the 16-bit values the PV product uses.
  uint4 pb;
  float la = 0.f;
  auto weights_all = [&](float off) __attribute__((always_inline)) {
    uint32_t w[4];
    la = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[2 * e], c2, -off));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[2 * e + 1], c2, -off));
      w[e] = M::pack(p0, p1);
      la = M::sum2(w[e], la);
    }
    pb = make_uint4(w[0], w[1], w[2], w[3]);
  };
  constexpr float kLazyBound = 4096.f;  // 2^12
  auto finish_weights = [&]() __attribute__((always_inline)) {
    float lsum = la;
    if (__any(lsum > kLazyBound || m_run == -INFINITY)) {
      float x = max3f(sc[0], sc[1], sc[2]);
      x = max3f(x, sc[3], sc[4]);
      x = max3f(x, sc[5], sc[6]);
      x = __builtin_fmaxf(x, sc[7]);
      x = __builtin_fmaxf(x, xor16(x));  // the query's four lanes: n, n + 16, n + 32, n + 48
      x = __builtin_fmaxf(x, xor32(x));
      const float m_new = __builtin_fmaxf(m_run, x * c2);
      const float used_new = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - used_new);  // 0 while m_run = -inf
      weights_all(used_new);
      lsum = la;
      m_run = m_new;
      m_used = used_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    }
    l_run += lsum;
  };

  // PV product O^T += V^T P^T: output block db (dims 16db ..) takes the V^T operand of keys
  // 4g .. 4g+3 (first transpose read) and 16 + 4g .. +3 (second), k slots 8g .. 8g+7.
  auto pv = [&](const char* vb) __attribute__((always_inline)) {
    unsigned vbl = lds_addr(vb) + v_lane;
    asm volatile("" : "+v"(vbl));
    auto read_v = [&](int db) __attribute__((always_inline)) {
      const unsigned a0 = vbl ^ (32u * db);
      const pf_s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a0);
      const pf_s16x4 v1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(a0 + 16 * RB));
      return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    constexpr int AH = 2;
    pf_s16x8 vop[AH];
#pragma unroll
    for (int i = 0; i < AH; ++i) vop[i] = read_v(i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const pf_s16x8 cur = vop[db % AH];
      if (db + AH < DB) vop[db % AH] = read_v(db + AH);
      acc[db] = M::mma16(cur, pb, acc[db]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  int vis_lo = -(1 << 30), vis_hi = wave_active ? kv_end : -(1 << 30);
  if (a.causal != SP_CAUSAL_NONE) vis_hi = min(vis_hi, wq_hi + pos_off + 1);
  if (a.window_left >= 0) vis_lo = wq_lo + pos_off - a.window_left - BN + 1;
  vis_lo = wave_uniform(vis_lo);
  vis_hi = wave_uniform(vis_hi);

  // One step on tile t0: wait for its tiles (own loads, then everyone's; the barrier also frees
  // the other buffers), start the next tile's loads, then QK product, softmax, PV product.
  auto step = [&](int t0, const char* kcur, const char* vcur, char* kload, char* vload)
      __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (t0 + BN < kv_end) {
      issue_tile(t0 + BN, v_wave ? vload : kload);
      fetch_blocks(t0 + 2 * BN);
    }
    if (t0 >= vis_lo && t0 < vis_hi) {
      qk(kcur);
      if constexpr (CAP) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = softcap_log2(sc[i], a.cap_in, a.cap_out);
      }
      apply_mask(t0);
      float off = m_used;
      asm volatile("" : "+v"(off));
      weights_all(off);
      finish_weights();
      pv(vcur);
    }
  };
  while (t0 < kv_end) {
    step(t0, kl[0], vl[0], kl[1], vl[1]);
    t0 += BN;
    if (t0 >= kv_end) break;
    step(t0, kl[1], vl[1], kl[0], vl[0]);
    t0 += BN;
  }

  // ---- normalise and store: lane holds O^T[dims 16db + 4g .. +3][query n]
  float l = l_run;
  l += xor16(l);
  l += xor32(l);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  constexpr int kSelf = std::is_same<T, bf16_t>::value ? SP_BF16 : SP_F16;  // out = in type
  if (a.out_dtype == kSelf) {
    // Whole output rows through an LDS stage (store_rows_staged16). The stage is an eighth of
    // the buffer pair the last step did not read: with n steps the last read pair n - 1 (mod 2),
    // and no load is pending into pair n % 2 (the last step issued none and waited for all
    // before its barrier, which also ended every read of that pair). Waves 0-3 take kl, waves
    // 4-7 vl, 8 KiB each.
    static_assert(TILE >= 4 * 16 * 512, "four 16-row x 256-dim stages per buffer");
    const int nsteps = kv_end > t_first ? (kv_end - t_first + BN - 1) / BN : 0;
    const int fb = wave_uniform(nsteps % 2);
    store_rows_staged16<M>(acc, inv, ((wave >> 2) ? vl[fb] : kl[fb]) + (wave & 3) * 16 * 512,
                           obase, a.o_tok, wq0, qe, lane);
    return;
  }
  if (my_q >= qe) return;
  const int oes = dtype_size((sp_dtype)a.out_dtype);
  char* op = obase + (int64_t)my_q * a.o_tok * oes;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int d0 = db * 16 + 4 * g;
    const float o0 = acc[db][0] * inv, o1 = acc[db][1] * inv;
    const float o2 = acc[db][2] * inv, o3 = acc[db][3] * inv;
    if (a.out_dtype == SP_F32) {
      *(float4*)(op + d0 * 4) = make_float4(o0, o1, o2, o3);
    } else if (a.out_dtype == kSelf) {
      *(uint2*)(op + d0 * 2) = make_uint2(M::pack(o0, o1), M::pack(o2, o3));
    } else {  // the other 16-bit type
      using O = PrefillMfma<typename std::conditional<kSelf == SP_BF16, f16_t, bf16_t>::type>;
      *(uint2*)(op + d0 * 2) = make_uint2(O::pack(o0, o1), O::pack(o2, o3));
    }
  }
}

// Merge the split partials of one (sequence, head, group of kCombineRows query rows):
// out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s, M = max_s m_s (zeros when no split saw
// a key). D/4 lanes per row, four output elements each, one row per lane group, so every row's
// loads are in flight at once.
constexpr int kCombineRows = 8;

template <typename T, int D>
__global__ void __launch_bounds__(256) prefill_combine_kernel(PrefillArgs a) {
  using M = PrefillMfma<T>;
  constexpr int TPR = D / 4, RPP = 256 / TPR;  // lanes per row, rows per workgroup pass
  static_assert(RPP >= kCombineRows, "a workgroup covers its row group in one pass");
  const int h = blockIdx.x % a.hq;
  const int id = blockIdx.x / a.hq;
  const int seq = id % a.num_seqs, grp = id / a.num_seqs;
  const int q_begin = a.cu_q[seq];
  const int Lq = min(a.cu_q[seq + 1] - q_begin, a.max_q);  // rows with a record slot
  const int qs = grp * kCombineRows;
  if (qs >= Lq) return;
  const int qe = min(qs + kCombineRows, Lq);
  const int c = threadIdx.x % TPR;
  for (int q = qs + (int)threadIdx.x / TPR; q < qe; q += RPP) {
    const float* rec =
        a.partials + ((((int64_t)seq * a.max_q + q) * a.hq + h) * a.nsplit) * (D + 4);
    // M: the largest offset of the splits that saw a key (an empty split records -inf)
    float m = -INFINITY;
    for (int sp = 0; sp < a.nsplit; ++sp) m = fmaxf(m, rec[sp * (D + 4)]);
    float l = 0.f, o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    for (int sp = 0; sp < a.nsplit && m != -INFINITY; ++sp) {
      const float* r = rec + sp * (D + 4);
      if (r[0] == -INFINITY) continue;  // no key in this split: weight 0, and no -inf - -inf
      const float w = __builtin_amdgcn_exp2f(r[0] - m);
      const float4 v = *(const float4*)(r + 4 + 4 * c);
      l += w * r[1];
      o0 += w * v.x;
      o1 += w * v.y;
      o2 += w * v.z;
      o3 += w * v.w;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    char* op = (char*)a.out + ((int64_t)(q_begin + q) * a.o_tok + (int64_t)h * a.o_head + 4 * c) * 2;
    *(uint2*)op = make_uint2(M::pack(o0 * inv, o1 * inv), M::pack(o2 * inv, o3 * inv));
  }
}

int plan_prefill_splits(int64_t base_wgs, int64_t max_ctx_tiles) {
  // A split pays for its partial records and merge only while it turns idle resident slots into
  // shorter walks: past one round of workgroups the extra ones queue behind the first.
  constexpr int64_t kResidentWgs = 2 * 256;
  if (base_wgs <= 0 || base_wgs * 2 > kResidentWgs) return 1;
  int64_t s = kResidentWgs / base_wgs;
  s = s > 8 ? 8 : s;
  const int64_t by_len = max_ctx_tiles / 16;
  s = s > by_len ? by_len : s;
  return s < 1 ? 1 : (int)s;
}

size_t prefill_partials_bytes(int num_seqs, int max_seqlen_q, int hq, int head_dim, int nsplit) {
  if (nsplit <= 1) return 0;
  return (size_t)num_seqs * max_seqlen_q * hq * nsplit * (head_dim + 4) * sizeof(float);
}

#ifndef SP_K32_MIN_WGS
#define SP_K32_MIN_WGS 1536
#endif
// Contiguous 16-bit prefills of at least this many workgroups (two rounds of prefill_k32_kernel's
// three per CU on 256 CUs) run on prefill_k32_kernel; smaller grids keep prefill_kernel, whose
// in-wave overlap of softmax and MFMA does not depend on other workgroups sharing the SIMD.
constexpr int64_t kK32MinWorkgroups = SP_K32_MIN_WGS;

template <typename T, int D>
static int launch_td(const PrefillArgs& a, bool paged, hipStream_t stream) {
  const int64_t base = (int64_t)a.num_qblocks * a.num_seqs * a.hq;
  const int64_t blocks = base * (a.nsplit > 1 ? a.nsplit : 1);
  if (blocks <= 0) return SP_OK;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "prefill: grid of %lld workgroups", (long long)blocks);
  // the split merge writes the input element type at head_dim columns
  constexpr int kSelf = std::is_same<T, bf16_t>::value ? SP_BF16 : SP_F16;
  if (a.nsplit > 1 && (a.out_dtype != kSelf || a.dv != D))
    return fail(SP_EUNSUPPORTED, "prefill: a key split needs out_dtype = the input type and Dv = D");
  if constexpr (D == 128) {
    if (!paged && a.nsplit <= 1 && base >= kK32MinWorkgroups) {
      hipLaunchKernelGGL((prefill_k32_kernel<T, D>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
      return check_launch("prefill_k32_kernel");
    }
  }
  if (paged)
    hipLaunchKernelGGL((prefill_kernel<T, D, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((prefill_kernel<T, D, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  if (int rc = check_launch("prefill_kernel")) return rc;
  if (a.nsplit > 1) {
    const int64_t groups = (int64_t)((a.max_q + kCombineRows - 1) / kCombineRows) * a.num_seqs * a.hq;
    if (groups > 0x7fffffff) return fail(SP_EINVAL, "prefill: combine grid of %lld", (long long)groups);
    hipLaunchKernelGGL((prefill_combine_kernel<T, D>), dim3((unsigned)groups), dim3(256), 0, stream, a);
    return check_launch("prefill_combine_kernel");
  }
  return SP_OK;
}

template <typename T>
static int launch_wide(const PrefillArgs& a, bool paged, hipStream_t stream) {
  if (a.nsplit > 1) return fail(SP_EUNSUPPORTED, "prefill: head_dim 256 takes no key split");
  const int64_t blocks = (int64_t)a.num_qblocks * a.num_seqs * a.hq;
  if (blocks <= 0) return SP_OK;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "prefill: grid of %lld workgroups", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(256);
  if (a.cap_out > 0.f) {
    if (paged)
      hipLaunchKernelGGL((prefill_wide_kernel<T, 256, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_wide_kernel<T, 256, false, true>), grid, block, 0, stream, a);
  } else if (paged) {
    hipLaunchKernelGGL((prefill_wide_kernel<T, 256, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((prefill_wide_kernel<T, 256, false>), grid, block, 0, stream, a);
  }
  return check_launch("prefill_wide_kernel");
}

template <typename T>
static int launch_d512(const PrefillArgs& a, bool paged, hipStream_t stream) {
  if (a.nsplit > 1) return fail(SP_EUNSUPPORTED, "prefill: head_dim 512 takes no key split");
  const int64_t blocks = (int64_t)a.num_qblocks * a.num_seqs * a.hq;
  if (blocks <= 0) return SP_OK;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "prefill: grid of %lld workgroups", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(512);
  if (a.cap_out > 0.f) {
    if (paged)
      hipLaunchKernelGGL((prefill_d512_kernel<T, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_d512_kernel<T, false, true>), grid, block, 0, stream, a);
  } else if (paged) {
    hipLaunchKernelGGL((prefill_d512_kernel<T, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((prefill_d512_kernel<T, false>), grid, block, 0, stream, a);
  }
  return check_launch("prefill_d512_kernel");
}

template <typename T>
static int launch_t(const PrefillArgs& a, int head_dim, bool paged, hipStream_t stream) {
  if (a.cap_out > 0.f && head_dim != 256 && head_dim != 512)
    return fail(SP_EUNSUPPORTED, "prefill: logit soft cap at head_dim %d", head_dim);
  switch (head_dim) {
    case 64: return launch_td<T, 64>(a, paged, stream);
    case 128: return launch_td<T, 128>(a, paged, stream);
    case 256: return launch_wide<T>(a, paged, stream);
    case 512: return launch_d512<T>(a, paged, stream);
    default:
      return fail(SP_EUNSUPPORTED, "prefill: head_dim %d has no kernel (64, 128, 256, 512)",
                  head_dim);
  }
}

int launch_prefill(const PrefillArgs& args, sp_dtype dtype, int head_dim, bool paged,
                   hipStream_t stream) {
  PrefillArgs a = args;
  if (a.nsplit < 1 || !a.partials) a.nsplit = 1;
  if (dtype == SP_F32) {
    if (a.cap_out > 0.f) return fail(SP_EUNSUPPORTED, "prefill: logit soft cap on f32 tensors");
    a.nsplit = 1;  // the fp32 kernel walks every key tile itself (no split partials)
    return launch_prefill_f32(a, head_dim, paged, stream);
  }
  switch (dtype) {
    case SP_BF16: return launch_t<bf16_t>(a, head_dim, paged, stream);
    case SP_F16: return launch_t<f16_t>(a, head_dim, paged, stream);
    default: return fail(SP_EUNSUPPORTED, "prefill: dtype %s has no kernel", dtype_name(dtype));
  }
}

}  // namespace sp
