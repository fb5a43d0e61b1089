// Projection GEMMs for gfx950, on MFMA: y[M, N] = x[M, K] . w[N, K]^T (+ bias[N]).
//
// Semantics (reference: burn's nn::Linear as MultiHeadAttention applies it for q_proj, k_proj,
// v_proj and o_proj, crates/sketchpad-core/src/transformer.rs:196-208, :249-253): the product
// accumulates in fp32 and is rounded once to the element type; a bias is then added in fp32 and
// rounded again (matmul, then + bias). The weight is taken K-contiguous ([out, in], the layout of
// PyTorch / Hugging Face checkpoints); launch_weight_transpose turns the reference's [in, out]
// into it once.
//
// Tiling (16-bit types): a workgroup of four waves owns a BM x BN tile of y and walks K in stages
// of 32. Each stage of x (BM rows) and w (BN rows) goes global -> registers -> LDS; the next
// stage's loads are in flight while the current one is multiplied. In LDS a row is 32 elements
// = four 16-byte chunks, chunk c of row r stored at c ^ ((r >> 2) & 3), so the fragment reads
// (16 consecutive rows at one chunk per 16 lanes) are bank-conflict free. A wave computes
// C^T = w . x^T on v_mfma_f32_32x32x16: A = 32 rows of w, B = 32 rows of x, both 16 contiguous
// bytes per lane, and the accumulator hands each lane 4 consecutive output columns (one 8-byte
// store). Tiles are 128 x 128 for large M and 64 x 64 for M <= 64 (decode); when the tiles
// alone cannot fill the chip, K is split and fp32 partials [split][M][N] are summed in a fixed
// order by a second kernel (deterministic). fp32 runs a plain LDS-tiled FMA kernel.
#include "linear.hpp"

namespace sp {

typedef __bf16 ln_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 ln_f16x8 __attribute__((ext_vector_type(8)));
typedef float ln_f32x16 __attribute__((ext_vector_type(16)));
typedef float ln_f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 ln_f16x2 __attribute__((ext_vector_type(2)));

template <typename T> struct LinMfma;
template <> struct LinMfma<bf16_t> {
  __device__ __forceinline__ static ln_f32x16 mma(uint4 a, uint4 b, ln_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(ln_bf16x8, a),
                                                   __builtin_bit_cast(ln_bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((ln_f32x2){lo, hi}, bf16x2_v));
  }
  __device__ __forceinline__ static float round(float v) {
    return __uint_as_float((uint32_t)f32_to_bf16_bits(v) << 16);
  }
};
template <> struct LinMfma<f16_t> {
  __device__ __forceinline__ static ln_f32x16 mma(uint4 a, uint4 b, ln_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(ln_f16x8, a),
                                                  __builtin_bit_cast(ln_f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((ln_f32x2){lo, hi}, ln_f16x2));
  }
  __device__ __forceinline__ static float round(float v) { return (float)(_Float16)v; }
};

struct LinArgs {
  void* y;
  const char* x;
  const char* w;
  const char* bias;
  float* partials;
  int64_t M, K, N;
  int64_t k_per_split;
  int splits;
  int y_vec;  // N % 4 == 0 and y 8-byte aligned: four outputs per 8-byte store
};

constexpr int kLinStage = 32;  // K per LDS stage (two 16-deep MFMA steps)

__device__ __forceinline__ int lin_swz(int r) { return (r >> 2) & 3; }

template <typename T, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(256) linear_kernel(LinArgs a) {
  constexpr int WTM = BM / WM, WTN = BN / WN;    // wave tile (rows of x, rows of w)
  constexpr int NBM = WTM / 32, NBN = WTN / 32;  // 32 x 32 MFMA blocks per wave
  constexpr int XCH = BM * 4 / 256, WCH = BN * 4 / 256;  // 16-byte chunks per thread per stage
  static_assert(WM * WN == 4 && NBM >= 1 && NBN >= 1 && XCH >= 1 && WCH >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) char lds[2][(BM + BN) * 64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t k_begin = (int64_t)blockIdx.z * a.k_per_split;
  const int64_t k_end = min(a.K, k_begin + a.k_per_split);
  const int n_iter = (int)((k_end - k_begin + kLinStage - 1) / kLinStage);
  const int64_t M = a.M, N = a.N, K = a.K;

  uint4 xr[XCH], wr[WCH];
  auto gload = [&](int it) {
    const int64_t k0 = k_begin + (int64_t)it * kLinStage;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + 256 * i, row = c >> 2;
      const int64_t k = k0 + 8 * (c & 3);
      const bool ok = m0 + row < M && k < k_end;
      xr[i] = ok ? *(const uint4*)(a.x + ((m0 + row) * K + k) * 2) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = tid + 256 * i, row = c >> 2;
      const int64_t k = k0 + 8 * (c & 3);
      const bool ok = n0 + row < N && k < k_end;
      wr[i] = ok ? *(const uint4*)(a.w + ((n0 + row) * K + k) * 2) : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](int buf) {
    char* xs = lds[buf];
    char* ws = lds[buf] + BM * 64;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + 256 * i, row = c >> 2;
      *(uint4*)(xs + row * 64 + 16 * ((c & 3) ^ lin_swz(row))) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = tid + 256 * i, row = c >> 2;
      *(uint4*)(ws + row * 64 + 16 * ((c & 3) ^ lin_swz(row))) = wr[i];
    }
  };

  ln_f32x16 acc[NBN][NBM];
#pragma unroll
  for (int bn = 0; bn < NBN; ++bn)
#pragma unroll
    for (int bm = 0; bm < NBM; ++bm)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[bn][bm][j] = 0.f;

  if (n_iter > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  const int l32 = lane & 31;
  for (int it = 0; it < n_iter; ++it) {
    const int buf = it & 1;
    if (it + 1 < n_iter) gload(it + 1);
    const char* xs = lds[buf];
    const char* ws = lds[buf] + BM * 64;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ch = (lane >> 5) + 2 * kk;
      uint4 af[NBN], bf[NBM];
#pragma unroll
      for (int bn = 0; bn < NBN; ++bn) {
        const int r = wn * WTN + bn * 32 + l32;
        af[bn] = *(const uint4*)(ws + r * 64 + 16 * (ch ^ lin_swz(r)));
      }
#pragma unroll
      for (int bm = 0; bm < NBM; ++bm) {
        const int r = wm * WTM + bm * 32 + l32;
        bf[bm] = *(const uint4*)(xs + r * 64 + 16 * (ch ^ lin_swz(r)));
      }
#pragma unroll
      for (int bn = 0; bn < NBN; ++bn)
#pragma unroll
        for (int bm = 0; bm < NBM; ++bm)
          acc[bn][bm] = LinMfma<T>::mma(af[bn], bf[bm], acc[bn][bm]);
    }
    if (it + 1 < n_iter) lstore(buf ^ 1);
    __syncthreads();
  }

  // C^T block (bn, bm): lane holds row m = ... + l32 of y and the four consecutive columns
  // n = ... + 8 (j / 4) + 4 (lane / 32) + (j % 4).
#pragma unroll
  for (int bn = 0; bn < NBN; ++bn)
#pragma unroll
    for (int bm = 0; bm < NBM; ++bm) {
      const int64_t m = m0 + wm * WTM + bm * 32 + l32;
      if (m >= M) continue;
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int64_t nb = n0 + wn * WTN + bn * 32 + 8 * jg + 4 * (lane >> 5);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[bn][bm][4 * jg + e];
        if (a.splits > 1) {
          float* p = a.partials + ((int64_t)blockIdx.z * M + m) * N;
          if (nb + 3 < N && (N & 3) == 0) {
            *(float4*)(p + nb) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (nb + e < N) p[nb + e] = v[e];
          }
          continue;
        }
        // round the product, add the bias in fp32, round again
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (a.bias && nb + e < N) v[e] = LinMfma<T>::round(v[e]) + Elem<T>::load(a.bias, nb + e);
        char* yrow = (char*)a.y + m * N * 2;
        if (a.y_vec && nb + 3 < N) {
          *(uint2*)(yrow + nb * 2) = make_uint2(LinMfma<T>::pack(v[0], v[1]),
                                                LinMfma<T>::pack(v[2], v[3]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) Elem<T>::store(yrow, nb + e, v[e]);
        }
      }
    }
}

// ---- Large M: 256 x 256 tiles, K stages of 64 straight to LDS ------------------------------
// NW waves: two along m, NW/2 along n, each owning 128 rows of x by 256/(NW/2) rows of w in
// 32 x 32 MFMA blocks. Each stage of x (256 rows) and w (256 rows) x 64 K moves HBM -> LDS with
// global_load_lds_dwordx4 (64 KiB per workgroup, no register staging) into the other half of a
// double buffer; the loads go out one per MFMA during the first quarter of the current stage,
// so they have the rest of it to land. A row of a stage is 128 bytes = eight 16-byte chunks,
// logical chunk c stored at c ^ ((row >> 1) & 7): the operand reads (16 consecutive rows at one
// chunk) are bank-conflict free, and since each load writes 1 KiB (8 rows) contiguously, a lane
// fetches the logical chunk that lands at its position. Workgroups are numbered so that the
// ones an XCD runs together (ids i, i+8, ...) take a contiguous run of tiles, ordered in groups
// of 8 row tiles: they share x and w panels in the XCD's L2.
constexpr int kBigBK = 64;
constexpr int kBigRowB = kBigBK * 2;        // bytes of one row of a stage
constexpr int kBigTileB = 256 * kBigRowB;   // one operand's stage: 32 KiB
constexpr int kBigStageB = 2 * kBigTileB;   // x then w

__device__ __forceinline__ int big_swz(int r) { return (r >> 1) & 7; }

// Eight waves (two per SIMD) with 128 x 64 wave tiles: one wave's MFMAs cover the other's LDS
// and barrier waits (measured 1.15 PFLOP/s at 4096^3 against 0.99 for four 128 x 128 waves).
constexpr int kBigWaves = 8;

template <typename T, int NW>
__global__ void __launch_bounds__(64 * NW, 1) linear_big_kernel(LinArgs a, int tm_count, int tn_count) {
  constexpr int WGN = NW / 2;            // waves along n (two along m)
  constexpr int WTN = 256 / WGN;         // wave tile: 128 rows of x by WTN rows of w
  constexpr int NBN = WTN / 32;          // 32 x 32 blocks along n per wave
  constexpr int NLD = 64 / NW;           // 1 KiB loads per wave per stage
  constexpr int NKK = kBigBK / 16;       // MFMA k-steps per stage
  __shared__ __attribute__((aligned(1024))) char lds[2 * kBigStageB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int l32 = lane & 31, hh = lane >> 5;

  // tile order: XCD-contiguous runs, groups of 8 row tiles
  const int ntiles = tm_count * tn_count;
  const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
  const int per = ntiles >> 3, rem = ntiles & 7;
  const int nid = xcd * per + min(xcd, rem) + local;
  constexpr int GM = 8;
  const int group = nid / (GM * tn_count);
  const int first_m = group * GM;
  const int gsize = min(tm_count - first_m, GM);
  const int within = nid - group * GM * tn_count;
  const int64_t m0 = (int64_t)(first_m + within % gsize) * 256;
  const int64_t n0 = (int64_t)(within / gsize) * 256;
  const int64_t M = a.M, N = a.N, K = a.K;
  const int n_iter = (int)(K / kBigBK);
  const bool interior = m0 + 256 <= M && n0 + 256 <= N;

  // load u of this wave (g = NLD wave + u): the first half of the waves fill the x stage, the
  // second half the w stage; rows 8 (g % 32) + lane / 8, physical chunk lane % 8
  const bool is_w = wave >= NW / 2;
  const char* mat = is_w ? a.w : a.x;
  const int64_t row0 = is_w ? n0 : m0;
  const int64_t rmax = (is_w ? N : M) - 1;
  const int64_t pitch = K * 2;
  // the swizzle of row 8 g' + lane / 8 only depends on the parity of g'
  int c16[2], voff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    c16[par] = 16 * ((lane & 7) ^ big_swz(8 * par + (lane >> 3)));
    voff[par] = (int)((lane >> 3) * pitch) + c16[par];
  }
  auto issue = [&](int it, int u) __attribute__((always_inline)) {
    const int g = wave * NLD + u;  // 0 .. 63
    const int gr = g & 31;
    char* dst = lds + (it & 1) * kBigStageB + g * 1024;
    const char* sb = mat + (row0 + 8 * gr) * pitch + (int64_t)it * kBigRowB;
    if (interior) {
      lds_dma16_s(sb, voff[gr & 1], dst);
    } else {
      // rows past the end read the last row instead (valid memory; their outputs are not stored)
      const bool over = row0 + 8 * gr + (lane >> 3) > rmax;
      lds_dma16(over ? mat + rmax * pitch + (int64_t)it * kBigRowB + c16[gr & 1]
                     : sb + voff[gr & 1], dst);
    }
  };

  ln_f32x16 acc[NBN][4];
#pragma unroll
  for (int bn = 0; bn < NBN; ++bn)
#pragma unroll
    for (int bm = 0; bm < 4; ++bm)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[bn][bm][j] = 0.f;

  // operand addresses: row R = base + l32 (base a multiple of 32), logical chunk 2 kk + hh at
  // (lane part ^ 32 kk) + immediate row-block offsets
  const int lp0 = l32 * kBigRowB + 16 * (hh ^ big_swz(l32));
  const int xw = wm * 128 * kBigRowB, ww = kBigTileB + wn * WTN * kBigRowB;

#pragma unroll
  for (int u = 0; u < NLD; ++u) issue(0, u);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  for (int it = 0; it < n_iter; ++it) {
    const int bufo = (it & 1) * kBigStageB;
    const bool more = it + 1 < n_iter;
    uint4 fa[2][NBN], fb[2][4];
    auto read = [&](int kk, uint4 (&ra)[NBN], uint4 (&rb)[4]) __attribute__((always_inline)) {
      int lp = (lp0 ^ (32 * kk)) + bufo;
      asm volatile("" : "+v"(lp));
      const char* pa = lds + ww + lp;
      const char* pb2 = lds + xw + lp;
#pragma unroll
      for (int b = 0; b < NBN; ++b) ra[b] = *(const uint4*)(pa + b * 32 * kBigRowB);
#pragma unroll
      for (int b = 0; b < 4; ++b) rb[b] = *(const uint4*)(pb2 + b * 32 * kBigRowB);
    };
    read(0, fa[0], fb[0]);
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      if (kk + 1 < NKK) read(kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
      for (int j = 0; j < 4 * NBN; ++j) {
        const int bn = j >> 2, bm = j & 3;
        acc[bn][bm] = LinMfma<T>::mma(fa[kk & 1][bn], fb[kk & 1][bm], acc[bn][bm]);
        // the next stage's loads, one per MFMA from the start of the stage
        const int u = kk * 4 * NBN + j;
        if (u < NLD && more) issue(it + 1, u);
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
  }

  // C^T block (bn, bm): lane holds row m = ... + l32 of y and columns n = ... + 8 jg + 4 hh + e
#pragma unroll
  for (int bn = 0; bn < NBN; ++bn)
#pragma unroll
    for (int bm = 0; bm < 4; ++bm) {
      const int64_t m = m0 + wm * 128 + bm * 32 + l32;
      if (m >= M) continue;
      char* yrow = (char*)a.y + m * N * 2;
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int64_t nb = n0 + wn * WTN + bn * 32 + 8 * jg + 4 * hh;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[bn][bm][4 * jg + e];
          if (a.bias && nb + e < N) v[e] = LinMfma<T>::round(v[e]) + Elem<T>::load(a.bias, nb + e);
        }
        if (a.y_vec && nb + 3 < N) {
          *(uint2*)(yrow + nb * 2) = make_uint2(LinMfma<T>::pack(v[0], v[1]),
                                                LinMfma<T>::pack(v[2], v[3]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) Elem<T>::store(yrow, nb + e, v[e]);
        }
      }
    }
}

// Sum the split-K partials in split order, round, add the bias, round again.
template <typename T>
__global__ void __launch_bounds__(256) linear_reduce_kernel(LinArgs a) {
  const int64_t MN = a.M * a.N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN;
       i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int p = 0; p < a.splits; ++p) s += a.partials[p * MN + i];
    if (a.bias) s = LinMfma<T>::round(s) + Elem<T>::load(a.bias, i % a.N);
    Elem<T>::store(a.y, i, s);
  }
}

// fp32: 64 x 64 tiles, 16-deep K stages in LDS, 4 x 4 outputs per thread (FMA).
__global__ void __launch_bounds__(256) linear_f32_kernel(LinArgs a) {
  __shared__ float xs[16][65];
  __shared__ float ws[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
  const float* x = (const float*)a.x;
  const float* w = (const float*)a.w;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < a.K; k0 += 16) {
    for (int i = threadIdx.x; i < 64 * 16; i += 256) {
      const int r = i >> 4, kk = i & 15;
      const int64_t k = k0 + kk;
      xs[kk][r] = (m0 + r < a.M && k < a.K) ? x[(m0 + r) * a.K + k] : 0.f;
      ws[kk][r] = (n0 + r < a.N && k < a.K) ? w[(n0 + r) * a.K + k] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float xv[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = xs[kk][ty * 4 + i];
        wv[i] = ws[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* y = (float*)a.y;
  const float* b = (const float*)a.bias;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < a.N) y[m * a.N + n] = b ? acc[i][j] + b[n] : acc[i][j];
    }
  }
}

// dst[N, K] = src[K, N]^T through 32 x 32 LDS tiles.
template <typename T>
__global__ void __launch_bounds__(256) weight_transpose_kernel(char* dst, const char* src,
                                                               int64_t K, int64_t N) {
  __shared__ float tile[32][33];
  const int64_t k0 = (int64_t)blockIdx.y * 32, n0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8)
    if (k0 + r < K && n0 + tx < N) tile[r][tx] = Elem<T>::load(src, (k0 + r) * N + n0 + tx);
  __syncthreads();
  for (int r = ty; r < 32; r += 8)
    if (n0 + r < N && k0 + tx < K) Elem<T>::store(dst, (n0 + r) * K + k0 + tx, tile[tx][r]);
}

LinearPlan plan_linear(int64_t M, int64_t K, int64_t N, size_t max_ws) {
  LinearPlan p{};
  // 256 x 256 tiles once there are enough rows to fill them; K in whole stages of 64, lane
  // offsets of one load (7 rows) within 32 bits, and a grid within 2^31 tiles
  if (M >= 512 && K % kBigBK == 0 && K <= (1LL << 27) &&
      ((M + 255) / 256) * ((N + 255) / 256) < (1LL << 31)) {
    p.big = true;
    p.tile_m = 256;
    p.splits = 1;
    p.k_per_split = K;
    p.ws_bytes = 0;
    return p;
  }
  // decode-sized x (M <= 64): 64 x 64 tiles, twice as many as 64 x 128 for the same weight
  p.tile_m = M <= 64 ? 64 : 128;
  const int64_t tile_n = p.tile_m == 64 ? 64 : 128;
  const int64_t tiles = ((M + p.tile_m - 1) / p.tile_m) * ((N + tile_n - 1) / tile_n);
  int splits = 1;
  // split K while the tiles cannot fill the chip three times over (three resident workgroups
  // per CU), keeping >= 512 of K per split
  while (tiles * splits < 768 && K / (splits * 2) >= 512 && splits < 8 &&
         (size_t)(splits * 2) * M * N * 4 <= max_ws)
    splits *= 2;
  p.k_per_split = ((K + splits - 1) / splits + kLinStage - 1) / kLinStage * kLinStage;
  p.splits = (int)((K + p.k_per_split - 1) / p.k_per_split);
  p.ws_bytes = p.splits > 1 ? (size_t)p.splits * M * N * 4 : 0;
  return p;
}

template <typename T>
static int launch_t(const LinArgs& a0, const LinearPlan& p, hipStream_t stream) {
  LinArgs a = a0;
  a.splits = p.splits;
  a.k_per_split = p.k_per_split;
  const dim3 block(256);
  if (p.big) {
    const int tm = (int)((a.M + 255) / 256), tn = (int)((a.N + 255) / 256);
    hipLaunchKernelGGL((linear_big_kernel<T, kBigWaves>), dim3((unsigned)(tm * tn)),
                       dim3(64 * kBigWaves), 0, stream, a, tm, tn);
    return check_launch("linear_big_kernel");
  }
  if (p.tile_m == 64) {
    const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)((a.M + 63) / 64), p.splits);
    hipLaunchKernelGGL((linear_kernel<T, 64, 64, 2, 2>), grid, block, 0, stream, a);
  } else {
    const dim3 grid((unsigned)((a.N + 127) / 128), (unsigned)((a.M + 127) / 128), p.splits);
    hipLaunchKernelGGL((linear_kernel<T, 128, 128, 2, 2>), grid, block, 0, stream, a);
  }
  if (int rc = check_launch("linear_kernel")) return rc;
  if (p.splits > 1) {
    const int64_t blocks = std::min<int64_t>((a.M * a.N + 255) / 256, 65536);
    hipLaunchKernelGGL(linear_reduce_kernel<T>, dim3((unsigned)blocks), block, 0, stream, a);
    return check_launch("linear_reduce_kernel");
  }
  return SP_OK;
}

int launch_linear(void* y, const void* x, const void* w_nk, const void* bias, int64_t M,
                  int64_t K, int64_t N, sp_dtype dtype, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  LinArgs a{};
  a.y = y;
  a.x = (const char*)x;
  a.w = (const char*)w_nk;
  a.bias = (const char*)bias;
  a.partials = (float*)workspace;
  a.M = M;
  a.K = K;
  a.N = N;
  a.y_vec = N % 4 == 0 && (uintptr_t)y % 8 == 0;
  if (dtype == SP_F32) {
    a.splits = 1;
    a.k_per_split = K;
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    hipLaunchKernelGGL(linear_f32_kernel, grid, dim3(256), 0, stream, a);
    return check_launch("linear_f32_kernel");
  }
  if (K % 8 != 0)
    return fail(SP_EUNSUPPORTED, "sp_linear: K = %lld is not a multiple of 8 (16-bit types)",
                (long long)K);
  const LinearPlan p = plan_linear(M, K, N, workspace ? workspace_bytes : 0);
  if (dtype == SP_BF16) return launch_t<bf16_t>(a, p, stream);
  return launch_t<f16_t>(a, p, stream);
}

int launch_weight_transpose(void* dst, const void* src, int64_t K, int64_t N, sp_dtype dtype,
                            hipStream_t stream) {
  const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((K + 31) / 32));
  switch (dtype) {
    case SP_F32:
      hipLaunchKernelGGL(weight_transpose_kernel<float>, grid, dim3(256), 0, stream, (char*)dst,
                         (const char*)src, K, N);
      break;
    case SP_BF16:
      hipLaunchKernelGGL(weight_transpose_kernel<bf16_t>, grid, dim3(256), 0, stream, (char*)dst,
                         (const char*)src, K, N);
      break;
    case SP_F16:
      hipLaunchKernelGGL(weight_transpose_kernel<f16_t>, grid, dim3(256), 0, stream, (char*)dst,
                         (const char*)src, K, N);
      break;
  }
  return check_launch("weight_transpose_kernel");
}

}  // namespace sp
