// Shared helpers for the gfx950 kernels and the C-ABI layer: element conversions, wavefront
// reductions, error reporting.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "sketchpad_attn.h"

namespace sp {

// ---------------------------------------------------------------------------------------------
// Error reporting (thread-local message behind sp_last_error()).
// ---------------------------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

__host__ __device__ inline int dtype_size(sp_dtype dt) {
  switch (dt) {
    case SP_F32: return 4;
    case SP_BF16: return 2;
    case SP_F16: return 2;
  }
  return 0;
}

inline const char* dtype_name(int dt) {
  switch (dt) {
    case SP_F32: return "f32";
    case SP_BF16: return "bf16";
    case SP_F16: return "f16";
  }
  return "?";
}

// ---------------------------------------------------------------------------------------------
// Element types. Storage is raw bits; arithmetic is fp32.
// ---------------------------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int bytes = 4;
  __device__ static float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  __device__ static void store(void* p, int64_t i, float v) { ((float*)p)[i] = v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int bytes = 2;
  __device__ static float load(const void* p, int64_t i) {
    return __uint_as_float(((uint32_t)((const uint16_t*)p)[i]) << 16);
  }
  __device__ static void store(void* p, int64_t i, float v) { ((uint16_t*)p)[i] = f32_to_bf16_bits(v); }
};
template <> struct Elem<f16_t> {
  static constexpr int bytes = 2;
  __device__ static float load(const void* p, int64_t i) { return f16_bits_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void store(void* p, int64_t i, float v) { ((uint16_t*)p)[i] = f32_to_f16_bits(v); }
};

// Dot product of one packed 32-bit word of two 16-bit elements with the matching word of
// another, accumulated in fp32 (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <typename T> struct Dot2;
template <> struct Dot2<bf16_t> {
  __device__ __forceinline__ static float fma(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a),
                                           __builtin_bit_cast(bf16x2_v, b), c, false);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return bf16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return bf16_hi(w); }
};
template <> struct Dot2<f16_t> {
  __device__ __forceinline__ static float fma(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a), __builtin_bit_cast(f16x2_v, b), c,
                                  false);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return f16_bits_to_f32((uint16_t)(w & 0xffffu)); }
  __device__ __forceinline__ static float hi(uint32_t w) { return f16_bits_to_f32((uint16_t)(w >> 16)); }
};

// ---------------------------------------------------------------------------------------------
// Logit soft cap (Gemma-4's attn_logit_softcap, gemma4.rs:366-369: logits = cap * tanh(logits /
// cap) on the scaled product, before the mask), in the softmax's base-2 exponent units: for a raw
// product s, with cap_in = 2 log2(e) scale / cap and cap_out = cap log2(e),
//   cap_out * tanh(s scale / cap) = cap_out - 2 cap_out / (1 + 2^(s cap_in)),
// since tanh(y) = 1 - 2 / (1 + e^(2y)). The exponential saturates cleanly: 2^(s cap_in) = inf
// gives cap_out and 0 gives -cap_out. One exponential, one reciprocal, three other ops.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float softcap_log2(float s, float cap_in, float cap_out) {
  const float r = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(s * cap_in));
  return __builtin_fmaf(-2.f * cap_out, r, cap_out);
}

// ---------------------------------------------------------------------------------------------
// Wavefront helpers (wave64).
// ---------------------------------------------------------------------------------------------
// Make LDS writes by any lane of this wave visible to later LDS reads by the same wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Value held by lane ^ 16 / lane ^ 32. v_permlane16_swap(x, x) returns (x[l & ~16], x[l | 16])
// and v_permlane32_swap(x, x) returns (x[l & ~32], x[l | 32]); the partner is the one that is not
// the lane's own value.
__device__ __forceinline__ float xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

// Workgroup barrier for data in LDS only: waits for this wave's LDS accesses, not for its global
// loads (which stay in flight across it), then meets the other waves. The memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Butterfly max / sum over aligned groups of WIDTH lanes (WIDTH a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = 1; o < WIDTH; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = 1; o < WIDTH; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): wait for every outstanding vector memory access of
// this wave (gfx9 encoding: vmcnt in bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
constexpr int kWaitVmcnt0 = 0x0F70;

typedef __attribute__((address_space(3))) void lds_void;

// global_load_lds_dwordx4: every lane copies 16 bytes from `src` to LDS at lds_dst + 16 * lane
// (lds_dst wave-uniform; the s_nop covers the M0 write -> LDS DMA wait state). Issued through inline asm so that the compiler does not guard the
// LDS reads of the other buffer with waits on these loads; completion is awaited explicitly
// (s_waitcnt vmcnt(0) + barrier) before the data is read.
__device__ __forceinline__ void lds_dma16(const char* src, char* lds_dst) {
  const unsigned m0 = (unsigned)(uintptr_t)(lds_void*)lds_dst;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
// Same with a wave-uniform base (SGPR pair) and a 32-bit per-lane byte offset.
// sbase must be wave-uniform; it is moved to SGPRs explicitly (readfirstlane) for the cases where
// the compiler keeps a uniform address in VGPRs. The compiler's hazard checks do not look inside
// inline asm, so the asm starts with s_nop 4: a VALU write of an SGPR (the readfirstlane) needs
// 5 wait states before a VMEM instruction reads that SGPR, and an M0 write 1 before LDS DMA.
__device__ __forceinline__ void lds_dma16_s(const char* sbase, int voff, char* lds_dst) {
  const unsigned m0 = (unsigned)(uintptr_t)(lds_void*)lds_dst;
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const char* s = (const char*)(uintptr_t)((hi << 32) | lo);
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(s), "{m0}"(m0)
               : "memory");
}

}  // namespace sp
