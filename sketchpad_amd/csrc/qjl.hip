// QJL compressed-cache codec (KvQuantMethod::QJL, crates/sketchpad-core/src/kv_cache.rs:300-324,
// :371-396, :534-617): a vector of head_dim values becomes 2 + ceil(proj_dim / 8) bytes, the
// binary16 magnitude |x| then one sign bit per row k of a fixed Gaussian projection R
// [proj_dim, head_dim] (bit k, little-endian within each byte: R[k,:] . x >= 0). Decompression
// rebuilds |x| * (pi/2 / proj_dim) * R^T s, s_k = +-1.
//
// Results are the reference's bit for bit: every sum is the reference's left fold in fp32 with
// separately rounded products (fp contraction off), the magnitude is rounded once to binary16,
// and decompression adds the signed rows in k order before the one scale multiply. The
// projection matrix is generated on the host (sp_qjl_projection) from the reference's LCG.
#include "qjl.hpp"

#include <math.h>

namespace sp {

namespace {

// One wave per vector. Lane k-chunks: lane L computes rows k = L, L + 64, ...; a wave ballot of
// "dot >= 0" over 64 consecutive rows gives 8 sign bytes, written by lanes 0..7.
template <typename T>
__global__ void __launch_bounds__(64) qjl_compress_kernel(uint8_t* out, const char* x,
                                                          int64_t num_vecs, int D,
                                                          const float* proj, int P) {
#pragma clang fp contract(off)
  const int64_t vec = blockIdx.x;
  if (vec >= num_vecs) return;
  const int lane = threadIdx.x;
  const int sign_bytes = (P + 7) / 8;
  uint8_t* rec = out + vec * (int64_t)(2 + sign_bytes);
  const char* row = x + vec * (int64_t)D * Elem<T>::bytes;
  // magnitude: the reference's left fold of x * x, then sqrt, rounded once to binary16
  float ss = 0.0f;
  for (int j = 0; j < D; ++j) {
    const float v = Elem<T>::load(row, j);
    ss = ss + v * v;
  }
  const float mag = sqrtf(ss);
  if (lane == 0) {
    const uint16_t bits = f32_to_f16_bits(mag);
    rec[0] = (uint8_t)(bits & 0xff);
    rec[1] = (uint8_t)(bits >> 8);
  }
  for (int k0 = 0; k0 < P; k0 += 64) {
    const int k = k0 + lane;
    bool pos = false;
    if (k < P && mag != 0.0f) {  // a zero vector keeps all-zero sign bytes
      const float* r = proj + (int64_t)k * D;
      float dot = 0.0f;
      for (int j = 0; j < D; ++j) dot = dot + r[j] * Elem<T>::load(row, j);
      pos = dot >= 0.0f;
    }
    const uint64_t bits = __ballot(pos);
    const int b = k0 / 8 + lane;
    if (lane < 8 && b < sign_bytes) rec[2 + b] = (uint8_t)(bits >> (8 * lane));
  }
}

// One thread per output element (vector, j): sum_k s_k R[k, j] in k order, then one multiply.
template <typename T>
__global__ void __launch_bounds__(256) qjl_decompress_kernel(char* out, const uint8_t* records,
                                                             int64_t num_vecs, int D,
                                                             const float* proj, int P) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= num_vecs * D) return;
  const int64_t vec = i / D;
  const int j = (int)(i % D);
  const int sign_bytes = (P + 7) / 8;
  const uint8_t* rec = records + vec * (int64_t)(2 + sign_bytes);
  const float mag = f16_bits_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
  float acc = 0.0f;
  if (mag != 0.0f) {
    const float scale = mag * (1.57079637f / (float)P);  // FRAC_PI_2 (f32) / proj_dim
    for (int k = 0; k < P; ++k) {
      const float r = proj[(int64_t)k * D + j];
      acc = acc + (((rec[2 + k / 8] >> (k % 8)) & 1) ? r : -r);
    }
    acc = acc * scale;
  }
  Elem<T>::store(out, i, acc);
}

}  // namespace

void qjl_projection_host(float* out, int proj_dim, int head_dim, float scale) {
#pragma clang fp contract(off)
  // Numerical Recipes LCG on a 64-bit state from 42; Box-Muller pairs (cos, then sin) of
  // uniforms (state >> 11) / 2^53 rounded to f32, u1 floored at 1e-10 (kv_cache.rs:373-396)
  const uint64_t A = 1664525ull, C = 1013904223ull;
  uint64_t state = 42;
  const int64_t count = (int64_t)proj_dim * head_dim;
  const float two53 = 9007199254740992.0f;
  const float tau = 6.28318548f;  // std::f32::consts::TAU
  int64_t i = 0;
  while (i < count) {
    state = state * A + C;
    float u1 = (float)(state >> 11) / two53;
    u1 = u1 > 1e-10f ? u1 : 1e-10f;
    state = state * A + C;
    const float u2 = (float)(state >> 11) / two53;
    const float r = sqrtf(-2.0f * logf(u1)) * scale;
    const float t = tau * u2;
    out[i++] = r * cosf(t);
    if (i < count) out[i++] = r * sinf(t);
  }
}

int launch_qjl_compress(void* out, const void* x, int64_t num_vecs, int head_dim,
                        const float* proj, int proj_dim, sp_dtype dtype, hipStream_t stream) {
  if (num_vecs > 0x7fffffff) return fail(SP_EINVAL, "qjl: %lld vectors", (long long)num_vecs);
  const dim3 grid((unsigned)num_vecs);
  switch (dtype) {
    case SP_F32:
      hipLaunchKernelGGL((qjl_compress_kernel<float>), grid, dim3(64), 0, stream,
                         (uint8_t*)out, (const char*)x, num_vecs, head_dim, proj, proj_dim);
      break;
    case SP_BF16:
      hipLaunchKernelGGL((qjl_compress_kernel<bf16_t>), grid, dim3(64), 0, stream,
                         (uint8_t*)out, (const char*)x, num_vecs, head_dim, proj, proj_dim);
      break;
    case SP_F16:
      hipLaunchKernelGGL((qjl_compress_kernel<f16_t>), grid, dim3(64), 0, stream,
                         (uint8_t*)out, (const char*)x, num_vecs, head_dim, proj, proj_dim);
      break;
  }
  return check_launch("qjl_compress_kernel");
}

int launch_qjl_decompress(void* out, const void* records, int64_t num_vecs, int head_dim,
                          const float* proj, int proj_dim, sp_dtype dtype, hipStream_t stream) {
  const int64_t n = num_vecs * head_dim;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(SP_EINVAL, "qjl: %lld elements", (long long)n);
  const dim3 grid((unsigned)blocks);
  switch (dtype) {
    case SP_F32:
      hipLaunchKernelGGL((qjl_decompress_kernel<float>), grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim, proj, proj_dim);
      break;
    case SP_BF16:
      hipLaunchKernelGGL((qjl_decompress_kernel<bf16_t>), grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim, proj, proj_dim);
      break;
    case SP_F16:
      hipLaunchKernelGGL((qjl_decompress_kernel<f16_t>), grid, dim3(256), 0, stream, (char*)out,
                         (const uint8_t*)records, num_vecs, head_dim, proj, proj_dim);
      break;
  }
  return check_launch("qjl_decompress_kernel");
}

}  // namespace sp
