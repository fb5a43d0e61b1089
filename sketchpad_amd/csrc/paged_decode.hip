// Split-K paged decode attention for gfx950, on MFMA.
//
// Semantics (reference: MultiHeadAttention::forward_cached with one new token,
// crates/sketchpad-core/src/transformer.rs:227-243, fed by PagedAttentionCache::update_layer,
// crates/sketchpad-core/src/paged_attention.rs:519-548): for every sequence s and query head h,
//   out[s,h,:] = softmax_j( (q[s,h,:] . K[s, h/G, j, :]) * scale ) @ V[s, h/G, j, :]
// over keys j in [start, L_s), start = 0 or L_s-1-window_left; fp32 softmax and accumulation.
//
// Work decomposition: one workgroup of four waves per (split, KV head, sequence); a split is
// `tps` consecutive 16-token tiles and the waves take every fourth tile (head_dim 512: the four
// waves take every tile together, each a quarter of its dims, and add up their partial products
// through LDS before one shared softmax). All query heads of the GQA group (up to 16) ride in
// the N = 16 columns of the MFMA tiles, so each K/V byte is read from HBM once. Per tile, per
// wave:
//   S^T[16 tok, 16 heads]  = K[16 tok, D] . Q^T[D, 16 heads]     MFMA 16x16x32 (16-bit) / 16x16x4 (f32)
//     16-bit: the tile's K and V rows are loaded lane-linear (coalesced 16-byte chunks) and
//     staged in the wave's LDS with an XOR chunk swizzle; the K operand of lane (g, n) is read
//     back as 16 bytes of token n. f32: K is the A operand loaded straight from the pool (lane
//     (g, n) loads 16 bytes of token n). Lane (g, n) then holds scores of tokens 4g..4g+3 for
//     head n.
//   online softmax per head column (two cross-row shuffles per tile), fp32.
//   O^T[D, 16 heads]     += V^T[D, 16 tok] . P^T[16 tok, 16 heads] MFMA 16x16x16 / 16x16x4
//     The score registers are already the B-operand layout of P^T; V^T comes from the stage by
//     transpose reads (ds_read_b64_tr_b16; f32: a padded pitch read column-wise).
// The next tile's loads are issued as soon as the current tile is in LDS (f32: as soon as K has
// entered the MFMAs and V is in LDS), so they stay in flight through the MFMAs and softmax of
// the current tile.
// sp_paged_append_decode runs the step's append in the same launch: the last split of each
// (sequence, KV head) unit stores the new token's rows (store_kv, paged_attention.rs:230-310)
// and reads them from the input rather than the pool.
// The four waves merge in LDS. A sequence that needs one split writes its output directly;
// otherwise each split stores (m, l, acc[D]) and decode_combine_kernel merges them. (Merging in
// the last-arriving split instead needs an agent-scope release/acquire per split, which on
// gfx950 is an L2 writeback + invalidate per workgroup: measured 10x slower. Without the fences,
// with the partials stored and loaded agent-coherent and a relaxed counter per unit, it is
// correct but every split then holds its slot through a write-through and an atomic round trip:
// Llama-3-8B decode 104.5 -> 107.6 us, Qwen2.5-7B 110.3 -> 115.1 us, and only the single-round
// windowed Mistral grid gains, 47.0 -> 46.4 us.)
#include "paged_decode.hpp"

#include <math.h>

#include <mutex>

namespace sp {

// Scratch of the entry point that allocates nothing (sp_paged_decode_noalloc). Each GPU the
// library runs on holds its own copy at its own address; host code reaches it only through the
// address hipGetSymbolAddress returns on that device (the array's name is a host-side stand-in).
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

void* decode_scratch_on_current_device() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(SP_EHIP, "decode scratch: hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(SP_EUNSUPPORTED, "decode scratch: device %d past the %d the library tracks", dev,
         kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(SP_EHIP, "decode scratch: hipGetSymbolAddress on device %d: %s", dev,
           hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef short s16x4_v __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_v __attribute__((ext_vector_type(4)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

constexpr int kTile = 16;  // tokens per tile

template <typename T> struct DecodeMfma;
template <> struct DecodeMfma<bf16_t> {
  __device__ __forceinline__ static f32x4_v qk(uint4 k, uint4 q, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, k),
                                                   __builtin_bit_cast(bf16x8_v, q), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4_v pv(uint2 v, uint2 p, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_v, v),
                                                     __builtin_bit_cast(s16x4_v, p), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {  // v_cvt_pk_bf16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){lo, hi}, bf16x2_v));
  }
};
template <> struct DecodeMfma<f16_t> {
  __device__ __forceinline__ static f32x4_v qk(uint4 k, uint4 q, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, k),
                                                  __builtin_bit_cast(f16x8_v, q), c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x4_v pv(uint2 v, uint2 p, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_v, v),
                                                 __builtin_bit_cast(f16x4_v, p), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {  // RNE
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){lo, hi}, f16x2_v));
  }
};

__device__ __forceinline__ f32x4_v mfma_f32(float a, float b, f32x4_v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <typename T, int D>
struct DecodeCfg {
  static constexpr int ES = Elem<T>::bytes;
  static constexpr bool kF32 = (ES == 4);
  static constexpr int RB = D * ES;                    // bytes per K/V row
  // Head dim 512 (16-bit): the four waves of a workgroup share every tile, each taking a slice
  // of D / 4 dims of its rows (one wave's registers cannot hold a whole row's Q, K, V and O);
  // otherwise one slice, the whole row, and the waves take every fourth tile.
  static constexpr int NSL = (D == 512) ? kDecodeWaves : 1;  // slices per row
  static constexpr int SD = D / NSL;                   // dims of a wave's slice
  static constexpr int SB = SD * ES;                   // bytes of a row's slice
  static constexpr int NL = SB / 64;                   // 16-byte loads per lane per tile (K or V)
  static constexpr int VP = RB + (kF32 ? 16 : 0);      // f32: V staging pitch (new banks per row)
  // 16-bit: K and V stages of 16 rows (slices) each, 16-byte chunks XOR-swizzled per row (swz
  // below); f32: a padded V stage only (K is read from HBM straight into the MFMA operand).
  static constexpr int WAVE_LDS = kF32 ? kTile * VP : 2 * kTile * SB;
  static constexpr int CPR = SB / 16;                  // 16-byte chunks per staged row
  static constexpr int ND = SD / 16;                   // 16-dim output blocks of a wave
  // the four waves' (m, l, O) merge; with slices the waves share one softmax and do not merge
  static constexpr int MERGE_LDS = NSL > 1 ? 0 : kDecodeWaves * (2 * 16 + 16 * D) * 4;
  // slices: each wave's partial products of a tile, [tile parity][wave][lane] x 4 floats
  static constexpr int XCHG_LDS = NSL > 1 ? 2 * kDecodeWaves * 64 * 16 : 0;
  static constexpr int STAGE_LDS = kDecodeWaves * WAVE_LDS + XCHG_LDS;
  static constexpr int LDS = STAGE_LDS > MERGE_LDS ? STAGE_LDS : MERGE_LDS;
  // Chunk swizzle of the 16-bit stages: the K operand read (16 rows at one logical chunk) and
  // the V transpose read (8 consecutive rows x 32 bytes per 32 lanes) hit distinct banks.
  // (Rows of 32 chunks, D = 256, take the 16-chunk pattern: it only needs to separate the rows
  // within 256 bytes of banks.)
  __device__ __forceinline__ static int swz(int row) {
    if constexpr (CPR >= 16) return ((row & 7) << 1) | ((row >> 3) & 1);
    else return (((row >> 1) & 3) << 1) | ((row >> 3) & 1);
  }
};
typedef __attribute__((address_space(3))) s16x4_v lds_s16x4_v;

// 16-bit kernels fit four waves per SIMD (<= 128 VGPRs, no spills), three for sub-tile blocks
// and two at head_dim 256 (head_dim 512 holds a quarter row per wave, like 128); f32 D=128
// would spill.
template <typename T, int D, bool SUB>
constexpr int decode_min_waves() {
  return Elem<T>::bytes == 4 ? 1 : (D == 256 ? 2 : (SUB ? 3 : 4));
}

// SUB: block sizes that are not multiples of the 16-token tile (1-15, 24, 40, ...), so that a
// tile spans several blocks or straddles a block edge; every row of a tile then takes the block
// its position maps to.
// CAP: the logit soft cap (a.cap_in / a.cap_out), instantiated for head_dims 256 and 512.
template <typename T, int D, bool SUB, bool CAP = false>
__global__ void __launch_bounds__(64 * kDecodeWaves, (decode_min_waves<T, D, SUB>()))
    paged_decode_kernel(DecodeArgs a) {
  using C = DecodeCfg<T, D>;
  constexpr int ES = C::ES, RB = C::RB, SD = C::SD, SB = C::SB, NL = C::NL, VP = C::VP;
  constexpr int ND = C::ND;
  constexpr bool kF32 = C::kF32;
  constexpr bool kSlices = C::NSL > 1;
  static_assert(SB % 64 == 0, "a slice must split into 64-byte MFMA K chunks");
  static_assert(!kSlices || !kF32, "dim slices are for 16-bit pools");
  // the waves' tile order: every fourth tile each, or (slices) every tile together
  constexpr int kStep = kSlices ? 1 : kDecodeWaves;

  __shared__ __attribute__((aligned(16))) char smem[C::LDS];

  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform(threadIdx.x >> 6);
  const int g = lane >> 4, n = lane & 15;
  // blockIdx.x enumerates (sequence, KV head) units, blockIdx.y the split. Workgroups are handed
  // to the eight XCDs round-robin in id order, so the unit must vary fastest: with the split
  // fastest, split s always lands on XCD s % 8 and the early splits (present in every sequence)
  // pile up on a few XCDs.
  const int unit = blockIdx.x, split = blockIdx.y;
  const int seq = unit / a.hkv, kvh = unit - seq * a.hkv;
  const int G = a.group;
  const int slice_b = kSlices ? wave * SB : 0;  // byte offset of this wave's slice in a row

  const int L_raw = a.context_lens[seq];
  const int L = min(L_raw, min(a.max_context_len, a.max_blocks_per_seq * a.block_size));
  if (L <= 0) {
    if (split == 0) {
      for (int i = threadIdx.x; i < G * D; i += blockDim.x)
        Elem<T>::store(a.out, ((int64_t)seq * a.hq + kvh * G) * D + i, 0.f);
      if (a.max_splits > 1 && threadIdx.x < G)  // split count 0: nothing for the combine
        a.partials[((int64_t)seq * a.hq + kvh * G + threadIdx.x) * a.max_splits * (D + 4) + 2] =
            0.f;
    }
    return;
  }
  const int start_tok = a.window_left >= 0 ? max(0, L - 1 - a.window_left) : 0;
  const int first_tile = start_tok / kTile, last_tile = (L - 1) / kTile;
  const int nsplit = (last_tile - first_tile + a.tps) / a.tps;
  if (split >= nsplit) return;
  const int t_begin = first_tile + split * a.tps;
  const int t_end = min(t_begin + a.tps, last_tile + 1);

  // Q^T operand: lane (g, n) holds head n's bytes [c*64 + g*16, +16) of the slice for every
  // chunk c.
  uint4 qv[NL];
  {
    const bool real = n < G;
    const char* qp =
        (const char*)a.q + ((int64_t)seq * a.hq + kvh * G + (real ? n : 0)) * RB + slice_b;
#pragma unroll
    for (int c = 0; c < NL; ++c) {
      const uint4 x = *(const uint4*)(qp + c * 64 + g * 16);  // padding heads read head 0
      qv[c] = real ? x : make_uint4(0, 0, 0, 0);
    }
  }

  const int32_t* table = a.block_tables + (int64_t)seq * a.max_blocks_per_seq;
  const int64_t head_off = a.layer_off_b + (int64_t)kvh * a.block_size * RB;
  char* vst = smem + wave * C::WAVE_LDS;

  // Fused append (sp_paged_append_decode): the step's new token of this sequence sits at position
  // context_lens[seq] - 1. The last split stores the token's K and V rows of this KV head in the
  // pool, at the slot the block table gives that position (skipped when the position lies past
  // the table or its block id outside the pool, as sp_kv_append skips such a slot). When the
  // token is attended (the length was not clamped to max_context_len or the table), the tile
  // holding it reads the row from k_new / v_new instead of the pool, so no other kernel has to
  // run first; a clamped length attends [0, L) without it, as sp_paged_decode would.
  const char* knew_row = nullptr;
  const char* vnew_row = nullptr;
  if (a.k_new) {
    const int64_t off_new = (int64_t)seq * a.new_tok_stride_b + (int64_t)kvh * a.new_head_stride_b;
    if (L == L_raw) {
      knew_row = a.k_new + off_new;
      vnew_row = a.v_new + off_new;
    }
    const int p = L_raw - 1;
    if (split == nsplit - 1 && wave == 0 && p < a.max_blocks_per_seq * a.block_size) {
      const int blk = table[p / a.block_size];
      const char* kn = a.k_new + off_new;
      const char* vn = a.v_new + off_new;
      if (blk >= 0 && blk < a.num_blocks) {
        const int64_t dst = (int64_t)blk * a.block_stride_b + head_off + (int64_t)(p % a.block_size) * RB;
        for (int o = lane * 16; o < RB; o += 64 * 16) {
          *(uint4*)((char*)a.kpool + dst + o) = *(const uint4*)(kn + o);
          *(uint4*)((char*)a.vpool + dst + o) = *(const uint4*)(vn + o);
        }
      }
    }
  }

  // Block ids of this split's tiles, fetched once up front: lane j holds the block of tile
  // t_begin + j in blk0 and of tile t_begin + 64 + j in blk1 (tps <= 128), so no tile load waits
  // on a dependent block-table read.
  int blk0 = 0, blk1 = 0;
  if constexpr (!SUB) {
    const int n_tiles = t_end - t_begin;
    if (lane < n_tiles) blk0 = table[((t_begin + lane) * kTile) / a.block_size];
    if (lane + 64 < n_tiles) blk1 = table[((t_begin + 64 + lane) * kTile) / a.block_size];
  }

  // Tile loads. K in MFMA A-operand order (token n, 16 bytes at c*64 + g*16); V coalesced
  // (lane-linear 16-byte chunks of the contiguous 16 x RB tile). Rows outside [start_tok, L)
  // read a valid row of the same tile instead (their scores are masked to -inf, so their
  // values are weighted by 0); a block id outside the pool reads block 0 and masks the tile.
  // K/V are streamed once: nontemporal loads keep them from displacing reusable L2 lines.
  typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));
  auto ldnt = [](const char* p) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4_v*)p));
  };
  auto load_tile_blk = [&](int t, uint4* kr, uint4* vr, uint32_t& okm) {
    const int pos0 = t * kTile;
    const int ti = t - t_begin;  // wave-uniform, < tps
    const int b0 = __builtin_amdgcn_readlane(blk0, ti & 63);
    const int b1 = __builtin_amdgcn_readlane(blk1, ti & 63);
    const int blk = ti < 64 ? b0 : b1;
    const bool ok = blk >= 0 && blk < a.num_blocks;
    okm = ok ? 0xFFFFu : 0u;
    const int64_t base = (int64_t)(ok ? blk : 0) * a.block_stride_b + head_off +
                         (int64_t)(pos0 % a.block_size) * RB;
    const int rlo = max(start_tok - pos0, 0), rhi = min(L - pos0, kTile) - 1;  // valid rows
    if (knew_row && pos0 + kTile > L - 1) {
      // the tile holding the fused append's token: its row rhi = L - 1 - pos0 (and the rows
      // clamped onto it) come from k_new / v_new
      if constexpr (kF32) {
        const int kr_row = min(max(n, rlo), rhi);
        const char* kb = kr_row == rhi ? knew_row : a.kpool + base + kr_row * RB;
#pragma unroll
        for (int c = 0; c < NL; ++c) kr[c] = ldnt(kb + c * 64 + g * 16);
      }
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int off = (i * 64 + lane) * 16;
        const int row = min(max(off / SB, rlo), rhi);
        const bool nw = row == rhi;
        const int so = slice_b + off % SB;  // byte of the row
        const int o = row * RB + so;
        if constexpr (!kF32) kr[i] = ldnt(nw ? knew_row + so : a.kpool + base + o);
        vr[i] = ldnt(nw ? vnew_row + so : a.vpool + base + o);
      }
      return;
    }
    if constexpr (kF32) {
      const int kr_row = min(max(n, rlo), rhi);
#pragma unroll
      for (int c = 0; c < NL; ++c) kr[c] = ldnt(a.kpool + base + kr_row * RB + c * 64 + g * 16);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int off = (i * 64 + lane) * 16;
      const int row = off / SB;
      const int o = min(max(row, rlo), rhi) * RB + slice_b + off % SB;
      if constexpr (!kF32) kr[i] = ldnt(a.kpool + base + o);  // coalesced, staged through LDS
      vr[i] = ldnt(a.vpool + base + o);
    }
  };
  // SUB: the rows of one tile lie in several blocks. Lane r < 16 reads the block id of row r
  // (ok: bit r set when that block lies in the pool) and works out the row's byte offset in the
  // pool once; each load takes its row's offset through a lane shuffle (every lane takes part).
  const unsigned bsz = (unsigned)a.block_size;
  auto load_tile_sub = [&](int t, uint4* kr, uint4* vr, uint32_t& okm) {
    const int pos0 = t * kTile;
    const int rlo = max(start_tok - pos0, 0), rhi = min(L - pos0, kTile) - 1;  // valid rows
    const unsigned p = (unsigned)min(pos0 + (lane & (kTile - 1)), L - 1);
    const unsigned bi = p / bsz;
    int rblk = 0;
    if (lane < kTile) rblk = table[bi];
    const bool okr = rblk >= 0 && rblk < a.num_blocks;
    okm = (uint32_t)__builtin_amdgcn_ballot_w64(okr) & 0xFFFFu;
    rblk = okr ? rblk : 0;
    const int64_t roff =
        (int64_t)rblk * a.block_stride_b + head_off + (int64_t)(p - bi * bsz) * RB;
    auto row_off = [&](int r) -> int64_t {
      const int lo = __shfl((int)(uint32_t)roff, r, 64);
      const int hi = __shfl((int)(roff >> 32), r, 64);
      return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    };
    const bool has_new = knew_row && pos0 + kTile > L - 1;  // the fused append's token (row rhi)
    if constexpr (kF32) {
      const int kr_row = min(max(n, rlo), rhi);
      const int64_t ko = row_off(kr_row);
      const char* kb = has_new && kr_row == rhi ? knew_row : a.kpool + ko;
#pragma unroll
      for (int c = 0; c < NL; ++c) kr[c] = ldnt(kb + c * 64 + g * 16);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int off = (i * 64 + lane) * 16;
      const int row = min(max(off / SB, rlo), rhi);
      const int so = slice_b + off % SB;  // byte of the row
      const int64_t o = row_off(row) + so;
      const bool nw = has_new && row == rhi;
      if constexpr (!kF32) kr[i] = ldnt(nw ? knew_row + so : a.kpool + o);
      vr[i] = ldnt(nw ? vnew_row + so : a.vpool + o);
    }
  };
  auto load_tile = [&](int t, uint4* kr, uint4* vr, uint32_t& okm) {
    if constexpr (SUB) load_tile_sub(t, kr, vr, okm);
    else load_tile_blk(t, kr, vr, okm);
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4_v acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};

  uint4 kc[NL], vc[NL];
  uint32_t ok_c = 0;
  int t = kSlices ? t_begin : t_begin + wave;
  if (t < t_end) load_tile(t, kc, vc, ok_c);
  for (; t < t_end; t += kStep) {
    const uint32_t tile_ok = ok_c;

    f32x4_v s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kF32) {
      // Stage V rows in LDS (two 8-byte stores per 16-byte chunk: the pitch is 8-byte aligned).
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int off = (i * 64 + lane) * 16;
        char* dst = vst + (off / RB) * VP + off % RB;
        *(uint2*)dst = make_uint2(vc[i].x, vc[i].y);
        *(uint2*)(dst + 8) = make_uint2(vc[i].z, vc[i].w);
      }
      // S^T = K Q^T
#pragma unroll
      for (int c = 0; c < NL; ++c) {
        s = mfma_f32(__uint_as_float(kc[c].x), __uint_as_float(qv[c].x), s);
        s = mfma_f32(__uint_as_float(kc[c].y), __uint_as_float(qv[c].y), s);
        s = mfma_f32(__uint_as_float(kc[c].z), __uint_as_float(qv[c].z), s);
        s = mfma_f32(__uint_as_float(kc[c].w), __uint_as_float(qv[c].w), s);
      }
      // K went into the MFMAs and V into LDS: the registers take the next tile's loads, which
      // stay in flight through this tile's softmax and PV.
      if (t + kStep < t_end) load_tile(t + kStep, kc, vc, ok_c);
    } else {
      // Stage K and V rows (slices): lane-linear 16-byte chunks at swizzled chunk positions.
      char* kst = vst + kTile * SB;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int off = (i * 64 + lane) * 16;
        const int row = off / SB, lc = (off % SB) / 16;
        const int dst = row * SB + 16 * (lc ^ C::swz(row));
        *(uint4*)(kst + dst) = kc[i];
        *(uint4*)(vst + dst) = vc[i];
      }
      wave_lds_sync();
      // both tiles are in LDS: the registers take the next tile's loads, which stay in flight
      // through this tile's MFMAs and softmax
      if (t + kStep < t_end) load_tile(t + kStep, kc, vc, ok_c);
      // S^T = K Q^T: the K operand of chunk c is row n, logical chunk 4c + g
      const int ksw = C::swz(n);
#pragma unroll
      for (int c = 0; c < NL; ++c)
        s = DecodeMfma<T>::qk(*(const uint4*)(kst + n * SB + 16 * ((4 * c + g) ^ ksw)), qv[c], s);
      if constexpr (kSlices) {
        // s holds the products over this wave's dims only: add up the four waves' partials, in
        // the same order in every wave, so that all four hold the same scores (and from them
        // the same softmax state). Two exchange buffers by tile parity: a wave writes tile t + 2's
        // partials only after the barrier of tile t + 1, which every wave reaches after reading
        // tile t's.
        f32x4_v* xs = (f32x4_v*)(smem + kDecodeWaves * C::WAVE_LDS) +
                      ((t - t_begin) & 1) * kDecodeWaves * 64;
        xs[wave * 64 + lane] = s;
        lds_barrier();
        s = xs[lane];
#pragma unroll
        for (int w = 1; w < kDecodeWaves; ++w) s += xs[w * 64 + lane];
      }
    }

    // Online softmax for head column n over tokens 4g..4g+3 of this tile.
    const int pos = t * kTile + 4 * g;
    float sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = ((tile_ok >> (4 * g + j)) & 1) && pos + j >= start_tok && pos + j < L;
      if constexpr (CAP)
        sv[j] = valid ? softcap_log2(s[j], a.cap_in, a.cap_out) : -INFINITY;
      else
        sv[j] = valid ? s[j] * a.scale_log2 : -INFINITY;
    }
    float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mt = fmaxf(mt, xor16(mt));
    mt = fmaxf(mt, xor32(mt));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      p[j] = (sv[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sv[j] - m_new);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] *= alpha;

    if constexpr (kF32) wave_lds_sync();  // V staging visible to the whole wave

    // O^T += V^T P^T
    if constexpr (kF32) {
#pragma unroll
      for (int db = 0; db < ND; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = *(const float*)(vst + (4 * g + j) * VP + (db * 16 + n) * 4);
          acc[db] = mfma_f32(v, p[j], acc[db]);
        }
      }
    } else {
      // A operand = V^T[16 dims][tokens 4g..4g+3] straight from the row-major stage by a
      // transpose read: lane n addresses row 4g + n/4, dims 16db + 4(n%4) .. +3
      const uint2 pp = make_uint2(DecodeMfma<T>::pack(p[0], p[1]), DecodeMfma<T>::pack(p[2], p[3]));
      const int vrow = 4 * g + (n >> 2);
      const int vsw = C::swz(vrow);
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const int colb = (db * 16 + 4 * (n & 3)) * ES;
        const char* ap = vst + vrow * SB + 16 * ((colb >> 4) ^ vsw) + (colb & 15);
        const s16x4_v vop = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_v*)ap);
        acc[db] = DecodeMfma<T>::pv(__builtin_bit_cast(uint2, vop), pp, acc[db]);
      }
    }
    wave_lds_sync();  // reads done before the next tile overwrites the staging area
  }

  // Per-head sums over the four token groups of the wave, then (whole rows) merge the four waves
  // in LDS.
  l_run += xor16(l_run);
  l_run += xor32(l_run);
  if constexpr (kSlices) {
    // The four waves hold the same softmax state and each the output of its own dims: no merge.
    // Lane (g, n) holds O^T[dims SD wave + 16 db + 4g .. +3][head n].
    if (n >= G) return;
    const int hq = kvh * G + n;
    const int d0 = SD * wave + 4 * g;
    if (nsplit == 1) {
      const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
      char* op = (char*)a.out + (((int64_t)seq * a.hq + hq) * D + d0) * ES;
#pragma unroll
      for (int db = 0; db < ND; ++db)
        *(uint2*)(op + db * 16 * ES) =
            make_uint2(DecodeMfma<T>::pack(acc[db][0] * inv, acc[db][1] * inv),
                       DecodeMfma<T>::pack(acc[db][2] * inv, acc[db][3] * inv));
    } else {
      float* pp = a.partials + (((int64_t)seq * a.hq + hq) * a.max_splits + split) * (D + 4);
      if (wave == 0 && g == 0) {
        pp[0] = m_run;
        pp[1] = l_run;
      }
#pragma unroll
      for (int db = 0; db < ND; ++db)
        *(float4*)(pp + 4 + d0 + db * 16) =
            make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
    }
    // word 2 of split 0's record: the split count, read by the combine (1: the output is final)
    if (split == 0 && wave == 0 && g == 0 && a.max_splits > 1)
      a.partials[((int64_t)seq * a.hq + hq) * a.max_splits * (D + 4) + 2] = (float)nsplit;
  } else {
    __syncthreads();
    float* cm = (float*)smem;             // [waves][16]
    float* cl = cm + kDecodeWaves * 16;   // [waves][16]
    float* ca = cl + kDecodeWaves * 16;   // [waves][16][D]
    if (g == 0) {
      cm[wave * 16 + n] = m_run;
      cl[wave * 16 + n] = l_run;
    }
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) ca[(wave * 16 + n) * D + db * 16 + 4 * g + r] = acc[db][r];
    __syncthreads();

    for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
      const int h = i / D, d = i % D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, cm[w * 16 + h]);
      float lsum = 0.f, asum = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) {
          const float mw = cm[w * 16 + h];
          const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
          lsum = fmaf(cl[w * 16 + h], f, lsum);
          asum = fmaf(ca[(w * 16 + h) * D + d], f, asum);
        }
      }
      const int hq = kvh * G + h;
      if (nsplit == 1) {
        Elem<T>::store(a.out, ((int64_t)seq * a.hq + hq) * D + d, lsum > 0.f ? asum / lsum : 0.f);
      } else {
        float* pp = a.partials + (((int64_t)seq * a.hq + hq) * a.max_splits + split) * (D + 4);
        if (d == 0) {
          pp[0] = M;
          pp[1] = lsum;
        }
        pp[4 + d] = asum;
      }
      // word 2 of split 0's record: the split count, read by the combine in the same round trip as
      // the partials (1: the output is final)
      if (split == 0 && d == 0 && a.max_splits > 1)
        a.partials[((int64_t)seq * a.hq + hq) * a.max_splits * (D + 4) + 2] = (float)nsplit;
    }
  }
}

// Merge the per-split partials (m, l, acc[D]) of sequences that needed more than one split.
// One wave per (query head, sequence). The split count (word 2 of split 0's record, written by
// the decode kernel) and the first 16 splits' (m, l) and the lane's D/64 accumulator columns are
// loaded together, so the merge waits on a single memory round trip; slots past the split count
// may hold stale data from earlier calls and are masked out.
template <typename T, int D>
__global__ void __launch_bounds__(64) decode_combine_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  constexpr int B = 16;  // splits per batch
  const int hq = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  const float* pp = a.partials + ((int64_t)seq * a.hq + hq) * a.max_splits * (D + 4);
  float M = -INFINITY, lsum = 0.f;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  int nsplit = B;  // refined by the header once the first batch is in
  for (int s0 = 0; s0 < nsplit; s0 += B) {
    float ms[B], ls[B], v[B][DPL];
    const float hdr = pp[2];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const float* src = pp + min(s0 + u, a.max_splits - 1) * (D + 4);
      ms[u] = src[0];
      ls[u] = src[1];
#pragma unroll
      for (int e = 0; e < DPL; ++e) v[u][e] = src[4 + lane * DPL + e];
    }
    nsplit = (int)hdr;
    if (nsplit <= 1) return;  // output written by the decode kernel (or an empty context)
    float mb = M;
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (s0 + u >= nsplit) ms[u] = -INFINITY;
      mb = fmaxf(mb, ms[u]);
    }
    if (mb == -INFINITY) continue;
    const float alpha = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - mb);
    lsum *= alpha;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (ms[u] == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ms[u] - mb);
      lsum = fmaf(ls[u], w, lsum);
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] = fmaf(v[u][e], w, acc[e]);
    }
    M = mb;
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int e = 0; e < DPL; ++e)
    Elem<T>::store(a.out, ((int64_t)seq * a.hq + hq) * D + lane * DPL + e, acc[e] * inv);
}

DecodePlan plan_decode(int num_seqs, int hq, int hkv, int head_dim, int max_context_len,
                       int window_left, DecodeKind kind) {
  DecodePlan p{};
  p.group = hkv > 0 ? hq / hkv : 0;
  p.tt = kTile;
  int max_tiles = (max_context_len + kTile - 1) / kTile;
  if (window_left >= 0) {
    const int wt = (window_left + 1 + kTile - 1) / kTile + 1;  // a window straddles one extra tile
    if (wt < max_tiles) max_tiles = wt;
  }
  p.max_tiles = max_tiles < 1 ? 1 : max_tiles;
  // Workgroups the batch launches with splits of t tiles if every sequence spanned max_tiles
  // (the host does not read the context lengths).
  const int64_t units = (int64_t)num_seqs * (hkv > 0 ? hkv : 1);
  auto wgs = [&](int t) { return units * ((p.max_tiles + t - 1) / t); };
  int tps;
  if (kind == DecodeKind::Dense && head_dim == 512) {
    // The four waves of a workgroup share each tile (a quarter of its dims each), so a tile is a
    // whole-workgroup step. 32 tiles, halved while the batch launches fewer than 512 workgroups:
    // measured on Gemma-4's global shape (16 / 8 heads) at 8-128 sequences of 0.3k-32k tokens,
    // 32-tile splits were 0.5-7 % faster than 16 and 8-15 % faster than 8; 64 was 1 % faster on
    // 16 contexts of 8k-32k tokens and 0.5-7 % slower on the others.
    tps = 32;
    while (tps > 4 && wgs(tps) < 512) tps /= 2;
  } else if (kind == DecodeKind::Dense) {
    // A rule fitted to measurements (24 batches: groups 1-16, 64-1024 units, contexts of
    // 256-16k tokens, windowed and not; it is within 2 % of the best of 32 / 64 / 128 tiles on
    // each, where one fixed length loses up to 20 %):
    //  - 64 tiles (1024 tokens) by default;
    //  - batches that would launch fewer than two workgroups per CU (256 CUs) with 64-tile
    //    splits take 32, halved while they still launch fewer;
    //  - 128 when that plan launches 384-512 workgroups: its longest splits then fill the GPU
    //    about once and a half to twice, with the fewest partials to merge (the windowed
    //    Mistral batch, 16-head groups, 256 units of 4k-token contexts);
    //  - 80 for groups of at most 4 query heads over contexts of 129-256 tiles with 512 or
    //    more units (measured on six such batches against 32, the earlier choice for them, and
    //    96: 80 was 0.5-5 % faster than 32 on all six, e.g. Llama-3-8B at 64 sequences
    //    105.0 -> 102.1 us, and level with 96 on average);
    //  - 96 for the other batches of at least 256 units: fewer, longer splits whose busy
    //    workgroups come closer to whole rounds of resident slots (measured against 64 on seven
    //    batches of groups 1-16: 2-7 % faster on all five with 256-2,048 units, e.g. the
    //    Qwen2.5-7B batch 111.8 -> 108.5 us; 1 % and 11 % slower on the two with 128 and 64
    //    units, which keep 64).
    // (Splitting each sequence's tiles into near-equal parts instead of full splits plus a
    // remainder measured slower on most of these batches.)
    tps = 64;
    if (wgs(64) < 512) {
      tps = 32;
      while (tps > kDecodeWaves && wgs(tps) < 512) tps /= 2;
    } else if (wgs(128) >= 384 && wgs(128) <= 512) {
      tps = 128;
    } else if (p.group <= 4 && units >= 512 && p.max_tiles > 128 && p.max_tiles <= 256) {
      tps = 80;
    } else if (units >= 256) {
      tps = 96;
    }
  } else {
    // Compressed tiles are a quarter of a dense one's bytes: 56-tile splits, halved while the
    // batch launches fewer than 512 workgroups (two per CU). Measured against 32, 40, 48 and 64
    // on the C2, C4 and C5 batches: 56 was the fastest or within 0.5 % of it on each (C2
    // 46.2 -> 45.6 us and C4 50.0 -> 49.2 against the earlier 64, C5 24.8 -> 23.8 against the
    // earlier 32).
    tps = 56;
    while (tps > kDecodeWaves && wgs(tps) < 512) tps /= 2;
  }
  p.tps = tps;
  p.max_splits = (p.max_tiles + tps - 1) / tps;
  if (p.max_splits > 1)
    p.ws_bytes = (size_t)num_seqs * hq * p.max_splits * (head_dim + 4) * sizeof(float);
  return p;
}

template <typename T, int D>
static int launch_typed(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.num_seqs * a.hkv, a.max_splits);
  const dim3 block(64 * kDecodeWaves);
  const bool sub = a.block_size % kTile != 0;
  if (a.cap_out > 0.f) {  // the host admits the soft cap at head_dims 256 and 512 only
    if constexpr (D >= 256) {
      if (sub)
        hipLaunchKernelGGL((paged_decode_kernel<T, D, true, true>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((paged_decode_kernel<T, D, false, true>), grid, block, 0, stream, a);
    } else {
      return fail(SP_EUNSUPPORTED, "paged decode: logit soft cap at head_dim %d", D);
    }
  } else if (sub) {
    hipLaunchKernelGGL((paged_decode_kernel<T, D, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((paged_decode_kernel<T, D, false>), grid, block, 0, stream, a);
  }
  if (a.max_splits > 1)
    hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3(a.hq, a.num_seqs), dim3(64), 0, stream,
                       a);
  return check_launch("paged_decode_kernel");
}

template <typename T>
static int launch_t(const DecodeArgs& a, int head_dim, hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_typed<T, 64>(a, stream);
    case 128: return launch_typed<T, 128>(a, stream);
    case 256:  // 16-bit pools only (Gemma-4's sliding layers, griffin)
      if constexpr (Elem<T>::bytes == 2) return launch_typed<T, 256>(a, stream);
      break;
    case 512:  // 16-bit pools only (Gemma-4's global layers)
      if constexpr (Elem<T>::bytes == 2) return launch_typed<T, 512>(a, stream);
      break;
    default: break;
  }
  return fail(SP_EUNSUPPORTED, "paged decode: head_dim %d has no kernel", head_dim);
}

template <typename T>
static int combine_t(const DecodeArgs& a, int head_dim, hipStream_t stream) {
  const dim3 grid(a.hq, a.num_seqs);
  if (head_dim == 64)
    hipLaunchKernelGGL((decode_combine_kernel<T, 64>), grid, dim3(64), 0, stream, a);
  else if (head_dim == 128)
    hipLaunchKernelGGL((decode_combine_kernel<T, 128>), grid, dim3(64), 0, stream, a);
  else
    return fail(SP_EUNSUPPORTED, "decode combine: head_dim %d has no kernel", head_dim);
  return check_launch("decode_combine_kernel");
}

int launch_decode_combine(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream) {
  if (a.max_splits <= 1) return SP_OK;
  switch (dtype) {
    case SP_F32: return combine_t<float>(a, head_dim, stream);
    case SP_BF16: return combine_t<bf16_t>(a, head_dim, stream);
    case SP_F16: return combine_t<f16_t>(a, head_dim, stream);
  }
  return fail(SP_EUNSUPPORTED, "decode combine: dtype %d has no kernel", (int)dtype);
}

int launch_paged_decode(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream) {
  switch (dtype) {
    case SP_F32: return launch_t<float>(a, head_dim, stream);
    case SP_BF16: return launch_t<bf16_t>(a, head_dim, stream);
    case SP_F16: return launch_t<f16_t>(a, head_dim, stream);
  }
  return fail(SP_EUNSUPPORTED, "paged decode: dtype %d has no kernel", (int)dtype);
}

}  // namespace sp
