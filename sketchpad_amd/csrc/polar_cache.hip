// PolarQuant compressed paged KV cache for gfx950: encode on append, decode inside attention.
//
// Semantics (reference: CompressedKvCache with KvQuantMethod::PolarQuant,
// crates/sketchpad-core/src/kv_cache.rs:437-532 and :640-727): every K/V vector is stored as
// its norm (binary16) and 4-bit direction codes n_j = round(7 x_j / |x|) clamped to [-7, 7];
// attention reads the vector back as n_j * (|x| / 7). The reference compresses on the CPU at
// every cache update and decompresses the whole sequence at every step; here the append kernel
// encodes straight into a paged pool and the decode kernel consumes the codes in place, so a
// decode step reads 2 + D/2 bytes per cached vector instead of 2D (bf16).
//
// Encoding is bit-exact with the reference: the squares are summed left to right in f32 without
// fused multiply-add, sqrt and the reciprocal are correctly rounded, codes round half away from
// zero, and the norm is converted to binary16 with round-to-nearest-even.
//
// Decode (polar_decode_kernel) follows the split-K plan of paged_decode.hip: one workgroup of
// four waves per (split, KV head, sequence), 16-token tiles, the query heads of a GQA group in
// the N = 16 columns of the MFMA tiles, per-split (m, l, acc) partials merged by
// decode_combine_kernel. Per tile and wave:
//   - K codes arrive as the A operand of S^T = K Q^T: lane (g, n) loads 16 bytes of token n's
//     code row (32 dimensions). A code word w (four bytes = eight codes) becomes four 32-bit
//     words of two 16-bit floats each by one mask-or per word: (w ^ 0x88888888) turns the two's
//     complement codes into n + 8 in 0..15, and OR-ing that into the low mantissa bits of 128.0
//     (bf16) or 1024.0 (f16) gives the float 128 + n + 8 (resp. 1024 + n + 8) exactly. The MFMA
//     then computes q . (n + B) with B = 136 (1032); the accumulator starts at -B * sum(q), so
//     it ends at q . n. Q is permuted once per workgroup to the order the unpack produces.
//   - score_j = (q . n_j) * (|k_j| / 7) * scale, online softmax in fp32.
//   - V codes arrive as the A operand of O^T = V^T P'^T from the token-quad plane: lane (g, m)
//     loads 16 bytes = 4 dimension pairs x tokens 4g..4g+3, unpacked the same way (bf16 128 + 8
//     bias); P'_j = p_j * |v_j| / 7 in bf16. One more MFMA with a ones row accumulates sum(P'),
//     and out = acc - 136 * sum(P') at the end.
// No LDS is used before the merge: every operand is loaded from HBM in the order the MFMA wants.
#include "polar_cache.hpp"

#include <math.h>

namespace sp {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef short s16x4_v __attribute__((ext_vector_type(4)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------------
// Encoding (polar_quant_compress, kv_cache.rs:437-483)
// ---------------------------------------------------------------------------------------------

// (d * 7.0).round().clamp(-7.0, 7.0) as i8: round half away from zero; a NaN stays NaN through
// the clamp and the cast maps it to 0.
__device__ __forceinline__ int polar_code(float d) {
#pragma clang fp contract(off)
  const float t = __builtin_roundf(d * 7.0f);
  if (__builtin_isnan(t)) return 0;
  return (int)fminf(fmaxf(t, -7.0f), 7.0f);
}

// Encode one row of D elements: returns the binary16 bits of |x| and hands each code byte
// (pair p: code of 2p in the high nibble, of 2p+1 in the low one; 0 past an odd D) to put(p, b).
template <typename T, typename Put>
__device__ __forceinline__ uint16_t polar_encode_row(const char* row, int D, Put&& put) {
#pragma clang fp contract(off)
  float ss = 0.0f;
  for (int j = 0; j < D; ++j) {
    const float x = Elem<T>::load(row, j);
    ss = ss + x * x;
  }
  const float mag = sqrtf(ss);
  const uint16_t bits = f32_to_f16_bits(mag);
  const int np = (D + 1) / 2;
  if (mag == 0.0f) {
    for (int p = 0; p < np; ++p) put(p, 0u);
    return bits;
  }
  const float inv = 1.0f / mag;
  for (int p = 0; p < np; ++p) {
    const int q0 = polar_code(Elem<T>::load(row, 2 * p) * inv);
    const int q1 = 2 * p + 1 < D ? polar_code(Elem<T>::load(row, 2 * p + 1) * inv) : 0;
    put(p, (uint32_t)(((q0 & 15) << 4) | (q1 & 15)));
  }
  return bits;
}

// A row of DC elements into fp32 registers with 16-byte loads (row 16-byte aligned).
template <typename T, int DC>
__device__ __forceinline__ void load_row_f32(const char* row, float (&x)[DC]) {
  constexpr int ES = Elem<T>::bytes, PER = 16 / ES;  // elements per 16-byte load
  static_assert(DC % PER == 0, "row must split into 16-byte loads");
  uint4 w[DC / PER];
#pragma unroll
  for (int i = 0; i < DC / PER; ++i) w[i] = *(const uint4*)(row + 16 * i);
#pragma unroll
  for (int i = 0; i < DC / PER; ++i)
#pragma unroll
    for (int e = 0; e < PER; ++e) x[i * PER + e] = Elem<T>::load(&w[i], e);
}

__device__ __forceinline__ int polar_nibble(uint32_t raw) {
  return raw > 7 ? (int)raw - 16 : (int)raw;
}

// One decompressed element pair (polar_quant_decompress, kv_cache.rs:486-532): code * (mag / 7)
// with the division in f32; a zero magnitude gives zeros.
__device__ __forceinline__ void polar_decode_pair(uint16_t mag_bits, uint32_t b, float& v0,
                                                  float& v1) {
  const float mag = f16_bits_to_f32(mag_bits);
  v0 = 0.0f;
  v1 = 0.0f;
  if (mag != 0.0f) {
    const float scale = mag / 7.0f;
    v0 = (float)polar_nibble((b >> 4) & 15u) * scale;
    v1 = (float)polar_nibble(b & 15u) * scale;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) polar_compress_kernel(uint8_t* out, const char* x,
                                                             int64_t n, int D) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int rec = 2 + (D + 1) / 2;
  uint8_t* o = out + i * rec;
  const uint16_t mb = polar_encode_row<T>(x + i * D * Elem<T>::bytes, D,
                                          [&](int p, uint32_t b) { o[2 + p] = (uint8_t)b; });
  o[0] = (uint8_t)(mb & 0xffu);
  o[1] = (uint8_t)(mb >> 8);
}

template <typename T>
__global__ void __launch_bounds__(256) polar_decompress_kernel(char* out, const uint8_t* recs,
                                                               int64_t n, int D) {
  const int np = (D + 1) / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * np) return;
  const int64_t i = idx / np;
  const int p = (int)(idx - i * np);
  const uint8_t* r = recs + i * (2 + np);
  float v0, v1;
  polar_decode_pair((uint16_t)(r[0] | (r[1] << 8)), r[2 + p], v0, v1);
  Elem<T>::store(out, i * D + 2 * p, v0);
  if (2 * p + 1 < D) Elem<T>::store(out, i * D + 2 * p + 1, v1);
}

// Encode on append. Generic form (DC == 0, any even head_dim): one thread per (token, KV head,
// K or V) vector with element loads. Wide form (DC = 64 / 128, 16-byte aligned rows): DC/8
// lanes per vector; every lane of the group loads the whole row with 16-byte loads and folds the
// same sum of squares (so the magnitude is the reference's left fold in every lane), then
// encodes and stores its own 8 dimensions. K codes go to the token's row of the K plane, V codes
// to the token-quad plane.
template <typename T, int DC>
__global__ void __launch_bounds__(256) polar_append_kernel(PolarAppendArgs a) {
  constexpr int LPV = DC > 0 ? DC / 8 : 1;  // lanes per vector
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = gi / LPV;
  const int part = (int)(gi - i * LPV);
  if (i >= (int64_t)a.num_tokens * a.hkv * 2) return;
  const int which = (int)(i & 1);
  const int64_t th = i >> 1;
  const int h = (int)(th % a.hkv);
  const int64_t t = th / a.hkv;
  const int32_t slot = a.slots[t];
  if (slot < 0 || (int64_t)slot >= a.num_slots) return;
  const int BS = a.block_size, D = DC > 0 ? DC : a.head_dim, HB = D / 2;
  const int blk = slot / BS, sl = slot - blk * BS;
  char* region = (which ? a.vpool : a.kpool) + (int64_t)blk * a.block_stride_b + a.layer_off_b +
                 (int64_t)h * polar_region_bytes(BS, D);
  const char* src =
      (which ? a.vnew : a.knew) + (t * a.tok_stride_e + h * a.head_stride_e) * Elem<T>::bytes;
  uint8_t* kcodes = (uint8_t*)region + (int64_t)sl * HB;
  uint8_t* vcodes = (uint8_t*)region + (int64_t)(sl >> 2) * HB * 4 + (sl & 3);
  uint16_t* mag = (uint16_t*)(region + (int64_t)BS * HB + 2 * sl);
  if constexpr (DC > 0) {
#pragma clang fp contract(off)
    float x[DC];
    load_row_f32<T, DC>(src, x);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < DC; ++j) ss = ss + x[j] * x[j];
    const float m = sqrtf(ss);
    const float inv = 1.0f / m;
    float xo[8];  // this lane's dimensions 8 part .. 8 part + 7 (a second, cached read)
    load_row_f32<T, 8>(src + 8 * part * Elem<T>::bytes, xo);
    uint32_t w = 0;  // code bytes of pairs 4 part .. 4 part + 3
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t b = m == 0.0f ? 0u
                                   : (uint32_t)(((polar_code(xo[2 * k] * inv) & 15) << 4) |
                                                (polar_code(xo[2 * k + 1] * inv) & 15));
      w |= b << (8 * k);
    }
    if (which == 0) {
      *(uint32_t*)(kcodes + 4 * part) = w;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) vcodes[4 * (4 * part + k)] = (uint8_t)(w >> (8 * k));
    }
    if (part == 0) *mag = f32_to_f16_bits(m);
  } else {
    uint32_t w = 0;
    auto put_k4 = [&](int p, uint32_t b) {  // four code bytes per 32-bit store
      w |= b << (8 * (p & 3));
      if ((p & 3) == 3) {
        *(uint32_t*)(kcodes + (p & ~3)) = w;
        w = 0;
      }
    };
    auto put_k1 = [&](int p, uint32_t b) { kcodes[p] = (uint8_t)b; };
    auto put_v = [&](int p, uint32_t b) { vcodes[4 * p] = (uint8_t)b; };
    uint16_t mb;
    if (which == 0)
      mb = (HB & 3) == 0 ? polar_encode_row<T>(src, D, put_k4) : polar_encode_row<T>(src, D, put_k1);
    else
      mb = polar_encode_row<T>(src, D, put_v);
    *mag = mb;
  }
}

// One thread per (KV head, position, pair) for decompression, per (KV head, position, record
// byte) for export; blockIdx.y selects K (0) or V (1). Positions whose block id lies outside the
// pool produce a zero record / zero values.
template <typename T, bool kExport>
__global__ void __launch_bounds__(256) polar_gather_kernel(PolarGatherArgs a) {
  const int BS = a.block_size, D = a.head_dim, HB = D / 2;
  const int per = kExport ? HB + 2 : HB;
  const int which = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.hkv * a.seq_len * per) return;
  const int e = (int)(idx % per);
  const int64_t hp = idx / per;  // h * seq_len + pos
  const int pos = (int)(hp % a.seq_len);
  const int h = (int)(hp / a.seq_len);
  const int blk = a.table[pos / BS];
  const int sl = pos - (pos / BS) * BS;
  char* out = which ? a.vout : a.kout;
  const bool ok = blk >= 0 && blk < a.num_blocks;
  const char* region = (which ? a.vpool : a.kpool) + (int64_t)(ok ? blk : 0) * a.block_stride_b +
                       a.layer_off_b + (int64_t)h * polar_region_bytes(BS, D);
  const uint16_t mb = ok ? *(const uint16_t*)(region + (int64_t)BS * HB + 2 * sl) : 0;
  auto code = [&](int p) -> uint32_t {
    if (!ok) return 0u;
    return (uint8_t)(which == 0 ? region[(int64_t)sl * HB + p]
                                : region[((int64_t)(sl >> 2) * HB + p) * 4 + (sl & 3)]);
  };
  if constexpr (kExport) {
    uint8_t* o = (uint8_t*)out + hp * (HB + 2);
    o[e] = (uint8_t)(e == 0 ? (mb & 0xffu) : e == 1 ? (mb >> 8) : code(e - 2));
  } else {
    float v0, v1;
    polar_decode_pair(mb, code(e), v0, v1);
    Elem<T>::store(out, hp * D + 2 * e, v0);
    Elem<T>::store(out, hp * D + 2 * e + 1, v1);
  }
}

// ---------------------------------------------------------------------------------------------
// Decode attention on the codes
// ---------------------------------------------------------------------------------------------
constexpr int kPTile = 16;     // tokens per tile (the plan of paged_decode.hip)
constexpr float kLazy = 8.0f;  // running-max slack of the lazy rescaling (log2 units)

template <typename T> struct PolarQk;
template <> struct PolarQk<bf16_t> {
  static constexpr uint32_t kKey = 0x43084308u;  // bf16 128.0 twice (| u gives 128 + u) | 0x8 bits
  static constexpr float kBias = 136.0f;         // 128 + 8
  __device__ __forceinline__ static f32x4_v qk(uint4 k, uint4 q, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, k),
                                                   __builtin_bit_cast(bf16x8_v, q), c, 0, 0, 0);
  }
};
template <> struct PolarQk<f16_t> {
  static constexpr uint32_t kKey = 0x64086408u;  // f16 1024.0 twice (| u gives 1024 + u) | 0x8 bits
  static constexpr float kBias = 1032.0f;        // 1024 + 8
  __device__ __forceinline__ static f32x4_v qk(uint4 k, uint4 q, f32x4_v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, k),
                                                  __builtin_bit_cast(f16x8_v, q), c, 0, 0, 0);
  }
};
constexpr uint32_t kVKey = 0x43084308u;  // V codes and P' are bf16 for every query type
constexpr float kVBias = 136.0f;

__device__ __forceinline__ f32x4_v mfma_pv(uint2 v, uint2 p, f32x4_v c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_v, v),
                                                   __builtin_bit_cast(s16x4_v, p), c, 0, 0, 0);
}

// Code word w = bytes b0..b3 (byte b: code of dimension 2p in the high nibble, 2p+1 in the low
// one) -> four words of two 16-bit floats magic + (code + 8), low half first:
//   .x = (lo b0, lo b2)   .y = (hi b0, hi b2)   .z = (lo b1, lo b3)   .w = (hi b1, hi b3)
// key = magic | 0x00080008: the masked nibble lands under the magic's zero low mantissa bits,
// and the xor both sets the magic and flips the nibble's sign bit (two's complement -> code + 8).
// Each word is one shift and one v_bitop3.
__device__ __forceinline__ uint4 polar_unpack(uint32_t w, uint32_t key) {
  uint4 r;
  r.x = (w & 0x000F000Fu) ^ key;
  r.y = ((w >> 4) & 0x000F000Fu) ^ key;
  r.z = ((w >> 8) & 0x000F000Fu) ^ key;
  r.w = ((w >> 12) & 0x000F000Fu) ^ key;
  return r;
}

typedef float f32x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {  // v_cvt_pk_bf16_f32 (RNE)
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){lo, hi}, bf16x2_v));
}

template <int NW> struct CodeWords;
template <> struct CodeWords<4> {
  using V = uint4;
  __device__ __forceinline__ static uint32_t get(const V& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
  }
};
template <> struct CodeWords<2> {
  using V = uint2;
  __device__ __forceinline__ static uint32_t get(const V& v, int i) { return i == 0 ? v.x : v.y; }
};

template <typename T, int D>
struct PolarDecodeCfg {
  static constexpr int HB = D / 2;     // code bytes per token
  static constexpr int NW = D / 32;    // code words per lane per tile, for K and for V
  static constexpr int ND = D / 16;    // 16-row output blocks (two per V code word)
  static constexpr int RB = D * 2;     // q row bytes (16-bit types)
  static constexpr int MERGE_LDS = kDecodeWaves * (2 * 16 + 16 * D) * 4;
};

template <typename T, int D>
__global__ void __launch_bounds__(64 * kDecodeWaves, 4) polar_decode_kernel(DecodeArgs a) {
  using C = PolarDecodeCfg<T, D>;
  using CW = CodeWords<C::NW>;
  using W = typename CW::V;
  constexpr int HB = C::HB, NW = C::NW, ND = C::ND, RB = C::RB;
  static_assert(NW == 2 || NW == 4, "head_dim 64 or 128");

  __shared__ __attribute__((aligned(16))) char smem[C::MERGE_LDS];

  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform(threadIdx.x >> 6);
  const int g = lane >> 4, n = lane & 15;
  const int unit = blockIdx.x, split = blockIdx.y;
  const int seq = unit / a.hkv, kvh = unit - seq * a.hkv;
  const int G = a.group;

  // Block ids of the split's tiles: lane j holds tile t_begin + j (tps <= 64), so no tile load
  // waits on a dependent block-table read. Without a window
  // t_begin = split * tps does not depend on the context length, and the table read is issued
  // together with it (one memory round trip before the first tile instead of two).
  const int32_t* table = a.block_tables + (int64_t)seq * a.max_blocks_per_seq;
  auto fetch_blocks = [&](int t0, int n_tiles, int& b0) {
    const int i0 = ((t0 + lane) * kPTile) / a.block_size;
    b0 = (lane < n_tiles && i0 < a.max_blocks_per_seq) ? table[i0] : 0;
  };
  int blk0 = 0;
  if (a.window_left < 0) fetch_blocks(split * a.tps, a.tps, blk0);

  int L = a.context_lens[seq];
  L = min(L, min(a.max_context_len, a.max_blocks_per_seq * a.block_size));
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
  const int first_tile = start_tok / kPTile, last_tile = (L - 1) / kPTile;
  const int nsplit = (last_tile - first_tile + a.tps) / a.tps;
  if (split >= nsplit) return;
  const int t_begin = first_tile + split * a.tps;
  const int t_end = min(t_begin + a.tps, last_tile + 1);
  if (a.window_left >= 0) fetch_blocks(t_begin, t_end - t_begin, blk0);

  // Q^T operand in the unpack order: for word c of lane (g, n), pairs P..P+3 with
  // P = g * HB/4 + 4c hold dimensions 2P..2P+7, and the unpacked elements are dimensions
  // 2P + {1, 5, 0, 4, 3, 7, 2, 6}. qsum = sum of head n's q (all lanes of column n).
  uint4 qv[NW];
  float qsum = 0.f;
  {
    const bool real = n < G;
    const char* qp = (const char*)a.q + ((int64_t)seq * a.hq + kvh * G + (real ? n : 0)) * RB;
#pragma unroll
    for (int c = 0; c < NW; ++c) {
      const int P = g * (HB / 4) + 4 * c;
      const uint4 x = *(const uint4*)(qp + 4 * P);  // dims 2P .. 2P+7
      uint4 r;
      r.x = (x.x >> 16) | (x.z & 0xffff0000u);       // (d1, d5)
      r.y = (x.x & 0xffffu) | (x.z << 16);           // (d0, d4)
      r.z = (x.y >> 16) | (x.w & 0xffff0000u);       // (d3, d7)
      r.w = (x.y & 0xffffu) | (x.w << 16);           // (d2, d6)
      // a negative scale is carried by q's sign (exact), so the scores scale by |scale| below
      const uint32_t flip = a.scale_log2 < 0.f ? 0x80008000u : 0u;
      r.x ^= flip;
      r.y ^= flip;
      r.z ^= flip;
      r.w ^= flip;
      qv[c] = real ? r : make_uint4(0, 0, 0, 0);
      if (real) {
        qsum += (Dot2<T>::lo(x.x) + Dot2<T>::hi(x.x)) + (Dot2<T>::lo(x.y) + Dot2<T>::hi(x.y)) +
                (Dot2<T>::lo(x.z) + Dot2<T>::hi(x.z)) + (Dot2<T>::lo(x.w) + Dot2<T>::hi(x.w));
      }
    }
  }
  qsum += xor16(qsum);
  qsum += xor32(qsum);
  if (a.scale_log2 < 0.f) qsum = -qsum;
  const float s_init = -PolarQk<T>::kBias * qsum;
  const f32x4_v s0 = {s_init, s_init, s_init, s_init};
  // score_j (log2 units) = (q . n_j) * |k_j| * ck; the 1/7 of the V side is applied at the end
  // (at least FLT_MIN, so a masked -inf score stays -inf even for a zero scale)
  const float ck = fmaxf(fabsf(a.scale_log2) * (1.0f / 7.0f), 1.17549435e-38f);
  // A operand of the sum(P') MFMA: row 0 of V^T all ones (bf16 1.0), other rows zero
  const uint2 ones_row0 = n == 0 ? make_uint2(0x3f803f80u, 0x3f803f80u) : make_uint2(0u, 0u);

  const int64_t head_off = a.layer_off_b + (int64_t)kvh * polar_region_bytes(a.block_size, D);
  const int mag_off = a.block_size * HB;
  // Each lane turns its tile's block id into the tile's code-plane and norm-plane byte offsets
  // (block 0 for an id outside the pool, whose tile is masked: bit j of okm clear), so a tile's
  // loads read their bases out of one lane instead of a scalar chain of compares, a 64-bit
  // multiply and a signed remainder per tile. Splits of PolarQuant batches span at most 64 tiles
  // (plan_decode), so lane j holds tile t_begin + j.
  int64_t coff, moff;
  uint64_t okm, fullm;
  {
    const bool ok = blk0 >= 0 && blk0 < a.num_blocks;
    const int sl0 = ((t_begin + lane) * kPTile) % a.block_size;
    const int64_t base = (int64_t)(ok ? blk0 : 0) * a.block_stride_b + head_off;
    coff = base + (int64_t)sl0 * HB;  // K codes; V token quads start at the same offset
    moff = base + mag_off + 2 * sl0;  // binary16 norms
    okm = __ballot(ok);
    // bit j of fullm: tile t_begin + j lies inside [start_tok, L) and its block in the pool, so
    // it needs no masking
    const int rel = (t_begin + lane) * kPTile - start_tok;
    fullm = __ballot(ok && rel >= 0 && rel + kPTile <= L - start_tok);
  }

  // One tile's loads: lane (g, n) holds 16 (D=64: 8) bytes of token n's K code row, 16 (8)
  // bytes of the V token-quad g, and the binary16 norms of tokens 4g..4g+3.
  struct Stage {
    W kw, vw;
    uint2 km, vm;
    bool ok, full;
  };
  // per-lane byte offsets inside a tile (the tile's base is wave-uniform: scalar address math)
  const uint32_t k_lane = n * HB + g * (HB / 4);
  const uint32_t v_lane = g * HB * 4 + n * (4 * NW);
  const uint32_t m_lane = 8 * g;
  auto readlane64 = [](int64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  auto load_tile = [&](int t, Stage& s) {
    const int ti = t - t_begin;  // < tps <= 64
    s.ok = (okm >> ti) & 1;
    s.full = (fullm >> ti) & 1;
    const int64_t c = readlane64(coff, ti), m = readlane64(moff, ti);
    const char* kt = a.kpool + c;
    const char* vt = a.vpool + c;
    const char* kmt = a.kpool + m;
    const char* vmt = a.vpool + m;
    s.kw = *(const W*)(kt + k_lane);
    s.vw = *(const W*)(vt + v_lane);
    s.km = *(const uint2*)(kmt + m_lane);
    s.vm = *(const uint2*)(vmt + m_lane);
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4_v acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  f32x4_v corr = {0.f, 0.f, 0.f, 0.f};
  const unsigned span = (unsigned)(L - start_tok);  // valid positions: start_tok + [0, span)

  auto process = [&](int t, const Stage& cur) {
    // S^T = K Q^T - B sum(q): tokens 4g..4g+3 of the tile for head n
    f32x4_v s = PolarQk<T>::qk(polar_unpack(CW::get(cur.kw, 0), PolarQk<T>::kKey), qv[0], s0);
#pragma unroll
    for (int c = 1; c < NW; ++c)
      s = PolarQk<T>::qk(polar_unpack(CW::get(cur.kw, c), PolarQk<T>::kKey), qv[c], s);

    const int rel0 = t * kPTile + 4 * g - start_tok;
    float u[4], mv[4];  // u_j = (q . n_j) |k_j| (times ck: log2 units); mv_j = |v_j|
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u[j] = s[j] * f16_bits_to_f32((uint16_t)((j < 2 ? cur.km.x : cur.km.y) >> (16 * (j & 1))));
      mv[j] = f16_bits_to_f32((uint16_t)((j < 2 ? cur.vm.x : cur.vm.y) >> (16 * (j & 1))));
    }
    if (!cur.full) {
      // a tile that straddles start_tok or L, or an invalid block: mask its tokens (score -inf,
      // |v| 0). The empty asm keeps this a branch: full tiles do no masking work.
      asm volatile("");
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool valid = cur.ok && (unsigned)(rel0 + j) < span;
        u[j] = valid ? u[j] : -INFINITY;
        mv[j] = valid ? mv[j] : 0.f;
      }
    }
    // Lazy rescaling: the running max m_run (log2 units) is raised (and acc, corr, l rescaled)
    // only when a head's tile max exceeds it by more than kLazy; otherwise the weights
    // exp2(score - m_run) stay below 2^kLazy, well inside fp32 and bf16 range. Any reference max
    // gives the same acc / l; the merge and the split combine use each wave's own m_run.
    float mt = fmaxf(fmaxf(u[0], u[1]), fmaxf(u[2], u[3]));
    mt = fmaxf(mt, xor16(mt));
    mt = fmaxf(mt, xor32(mt));
    mt *= ck;
    if (__builtin_amdgcn_ballot_w64(mt > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int i = 0; i < ND; ++i) acc[i] *= alpha;
      corr[0] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    float p[4];  // a masked token (u = -inf) gets exp2(-inf) = 0
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(fmaf(u[j], ck, -m_use));
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

    // P'^T in the token order of the V unpack: (t0, t2), (t1, t3)
    const uint2 pp = make_uint2(pack_bf16(p[0] * mv[0], p[2] * mv[2]),
                                pack_bf16(p[1] * mv[1], p[3] * mv[3]));
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint4 u = polar_unpack(CW::get(cur.vw, i), kVKey);
      acc[2 * i] = mfma_pv(make_uint2(u.x, u.z), pp, acc[2 * i]);          // dims 2p + 1
      acc[2 * i + 1] = mfma_pv(make_uint2(u.y, u.w), pp, acc[2 * i + 1]);  // dims 2p
    }
    corr = mfma_pv(ones_row0, pp, corr);
  };

  // The wave's tiles t_begin + wave + 4i through a ring of kRing register stages: a stage is
  // refilled with the tile kRing steps ahead as soon as its tile is consumed, so kRing - 1 tiles
  // stay in flight while one is computed. The refill is unconditional (past the wave's last tile
  // it reloads the tile just consumed, which is cached and never processed): loads under a
  // condition would make the compiler wait for every outstanding load before each tile.
  constexpr int kRing = 3, kStep = kDecodeWaves * kRing;
  const int t_first = t_begin + wave;
  Stage st[kRing];
#pragma unroll
  for (int r = 0; r < kRing; ++r) {
    const int tr = t_first + kDecodeWaves * r;
    load_tile(tr < t_end ? tr : t_begin, st[r]);
  }
  for (int tb = t_first; tb < t_end; tb += kStep) {
#pragma unroll
    for (int r = 0; r < kRing; ++r) {
      const int t = tb + kDecodeWaves * r;
      if (t < t_end) process(t, st[r]);
      load_tile(t + kStep < t_end ? t + kStep : (t < t_end ? t : t_begin), st[r]);
    }
  }

  // Remove the V bias (row 0 of corr, lane (0, n), holds sum(P') of head n) and apply the 1/7
  // of |v| / 7.
  const float cn = kVBias * __shfl(corr[0], n, 64);
  constexpr float kSeventh = 1.0f / 7.0f;
  l_run += xor16(l_run);
  l_run += xor32(l_run);
  __syncthreads();
  float* cm = (float*)smem;             // [waves][16]
  float* cl = cm + kDecodeWaves * 16;   // [waves][16]
  float* ca = cl + kDecodeWaves * 16;   // [waves][16][D]
  if (g == 0) {
    cm[wave * 16 + n] = m_run;
    cl[wave * 16 + n] = l_run;
  }
  // acc[2i + h] row m = 4g + r holds dimension 2 (NW m + i) + (h ? 0 : 1)
#pragma unroll
  for (int i = 0; i < NW; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pr = NW * (4 * g + r) + i;
      ca[(wave * 16 + n) * D + 2 * pr + 1] = (acc[2 * i][r] - cn) * kSeventh;
      ca[(wave * 16 + n) * D + 2 * pr] = (acc[2 * i + 1][r] - cn) * kSeventh;
    }
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

// ---------------------------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------------------------
static unsigned blocks_for(int64_t items) { return (unsigned)((items + 255) / 256); }

int launch_polar_compress(void* out, const void* x, int64_t num_vecs, int head_dim,
                          sp_dtype dtype, hipStream_t stream) {
  const dim3 grid(blocks_for(num_vecs));
  switch (dtype) {
    case SP_F32:
      hipLaunchKernelGGL(polar_compress_kernel<float>, grid, dim3(256), 0, stream, (uint8_t*)out,
                         (const char*)x, num_vecs, head_dim);
      break;
    case SP_BF16:
      hipLaunchKernelGGL(polar_compress_kernel<bf16_t>, grid, dim3(256), 0, stream,
                         (uint8_t*)out, (const char*)x, num_vecs, head_dim);
      break;
    case SP_F16:
      hipLaunchKernelGGL(polar_compress_kernel<f16_t>, grid, dim3(256), 0, stream, (uint8_t*)out,
                         (const char*)x, num_vecs, head_dim);
      break;
  }
  return check_launch("polar_compress_kernel");
}

int launch_polar_decompress(void* out, const void* records, int64_t num_vecs, int head_dim,
                            sp_dtype dtype, hipStream_t stream) {
  const dim3 grid(blocks_for(num_vecs * ((head_dim + 1) / 2)));
  switch (dtype) {
    case SP_F32:
      hipLaunchKernelGGL(polar_decompress_kernel<float>, grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim);
      break;
    case SP_BF16:
      hipLaunchKernelGGL(polar_decompress_kernel<bf16_t>, grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim);
      break;
    case SP_F16:
      hipLaunchKernelGGL(polar_decompress_kernel<f16_t>, grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim);
      break;
  }
  return check_launch("polar_decompress_kernel");
}

template <typename T>
static void append_t(const PolarAppendArgs& a, bool wide, hipStream_t stream) {
  const int64_t vecs = (int64_t)a.num_tokens * a.hkv * 2;
  if (wide && a.head_dim == 128)
    hipLaunchKernelGGL((polar_append_kernel<T, 128>), dim3(blocks_for(vecs * 16)), dim3(256), 0,
                       stream, a);
  else if (wide && a.head_dim == 64)
    hipLaunchKernelGGL((polar_append_kernel<T, 64>), dim3(blocks_for(vecs * 8)), dim3(256), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((polar_append_kernel<T, 0>), dim3(blocks_for(vecs)), dim3(256), 0, stream,
                       a);
}

int launch_polar_append(const PolarAppendArgs& a, sp_dtype dtype, hipStream_t stream) {
  const int es = dtype_size(dtype);
  const bool wide = (((uintptr_t)a.knew | (uintptr_t)a.vnew | (uintptr_t)(a.tok_stride_e * es) |
                      (uintptr_t)(a.head_stride_e * es)) & 15) == 0;
  switch (dtype) {
    case SP_F32: append_t<float>(a, wide, stream); break;
    case SP_BF16: append_t<bf16_t>(a, wide, stream); break;
    case SP_F16: append_t<f16_t>(a, wide, stream); break;
  }
  return check_launch("polar_append_kernel");
}

int launch_polar_gather(const PolarGatherArgs& a, int dtype, hipStream_t stream) {
  const int per = dtype < 0 ? a.head_dim / 2 + 2 : a.head_dim / 2;
  const dim3 grid(blocks_for((int64_t)a.hkv * a.seq_len * per), 2);
  switch (dtype) {
    case SP_F32: hipLaunchKernelGGL((polar_gather_kernel<float, false>), grid, dim3(256), 0, stream, a); break;
    case SP_BF16: hipLaunchKernelGGL((polar_gather_kernel<bf16_t, false>), grid, dim3(256), 0, stream, a); break;
    case SP_F16: hipLaunchKernelGGL((polar_gather_kernel<f16_t, false>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((polar_gather_kernel<float, true>), grid, dim3(256), 0, stream, a); break;
  }
  return check_launch("polar_gather_kernel");
}

template <typename T, int D>
static int launch_decode_typed(const DecodeArgs& a, sp_dtype dtype, hipStream_t stream) {
  const dim3 grid(a.num_seqs * a.hkv, a.max_splits);
  hipLaunchKernelGGL((polar_decode_kernel<T, D>), grid, dim3(64 * kDecodeWaves), 0, stream, a);
  if (int rc = check_launch("polar_decode_kernel")) return rc;
  return launch_decode_combine(a, dtype, D, stream);
}

int launch_polar_decode(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream) {
  // the kernel holds one tile per lane of a wave (plan_decode's PolarQuant splits: <= 64 tiles)
  if (a.tps < 1 || a.tps > 64)
    return fail(SP_EINVAL, "polar decode: %d tiles per split (at most 64)", a.tps);
  if (dtype == SP_BF16) {
    if (head_dim == 64) return launch_decode_typed<bf16_t, 64>(a, dtype, stream);
    if (head_dim == 128) return launch_decode_typed<bf16_t, 128>(a, dtype, stream);
  } else if (dtype == SP_F16) {
    if (head_dim == 64) return launch_decode_typed<f16_t, 64>(a, dtype, stream);
    if (head_dim == 128) return launch_decode_typed<f16_t, 128>(a, dtype, stream);
  }
  return fail(SP_EUNSUPPORTED, "polar decode: dtype %s / head_dim %d has no kernel",
              dtype_name(dtype), head_dim);
}

}  // namespace sp
