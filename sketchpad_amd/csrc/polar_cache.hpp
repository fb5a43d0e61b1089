// Launch interface of the PolarQuant compressed paged cache (polar_cache.hip).
//
// Record format (the reference's, polar_quant_compress, crates/sketchpad-core/src/kv_cache.rs:
// 437-483): a head_dim vector x becomes its norm |x| as binary16 plus one 4-bit two's-complement
// direction code per dimension, round(7 x_j / |x|) clamped to [-7, 7], two codes per byte with
// the even dimension in the high nibble.
//
// Pool layout: pool[num_blocks][num_layers][num_kv_heads] regions of block_size vectors, one
// pool for K and one for V, each region = code plane + magnitude plane:
//   K region: codes [BS][D/2]                    (token-major: a token's bytes are contiguous)
//             mags  [BS] binary16
//   V region: codes [BS/4][D/2][4]               (token quads: byte (tok, p) at
//                                                 ((tok/4)*(D/2) + p)*4 + tok%4)
//             mags  [BS] binary16
// BS * (D/2 + 2) bytes per region. The K plane lets a decode wave load the QK operand straight
// from HBM (16 contiguous bytes per lane = 32 dimensions of one token); the V plane does the same
// for the PV operand (16 bytes = 4 tokens x 4 dimension pairs). Each vector's bytes are the
// reference's record bytes; only their placement differs.
#pragma once

#include "paged_decode.hpp"
#include "sp_common.hpp"

namespace sp {

__host__ __device__ inline int64_t polar_region_bytes(int block_size, int head_dim) {
  return (int64_t)block_size * (head_dim / 2 + 2);
}

struct PolarAppendArgs {
  char* kpool;
  char* vpool;
  const char* knew;
  const char* vnew;
  int64_t tok_stride_e;   // element strides of k_new / v_new
  int64_t head_stride_e;
  const int32_t* slots;
  int64_t block_stride_b;
  int64_t layer_off_b;
  int64_t num_slots;
  int num_tokens;
  int hkv;
  int head_dim;
  int block_size;
};

struct PolarGatherArgs {
  char* kout;             // [Hkv, seq_len, D] elements, or [Hkv, seq_len, record] bytes
  char* vout;
  const char* kpool;
  const char* vpool;
  const int32_t* table;
  int64_t block_stride_b;
  int64_t layer_off_b;
  int seq_len;
  int hkv;
  int head_dim;
  int block_size;
  int num_blocks;
};

int launch_polar_compress(void* out, const void* x, int64_t num_vecs, int head_dim,
                          sp_dtype dtype, hipStream_t stream);
int launch_polar_decompress(void* out, const void* records, int64_t num_vecs, int head_dim,
                            sp_dtype dtype, hipStream_t stream);
int launch_polar_append(const PolarAppendArgs& a, sp_dtype dtype, hipStream_t stream);
// dtype < 0: export records; else decompress into that element type
int launch_polar_gather(const PolarGatherArgs& a, int dtype, hipStream_t stream);
// DecodeArgs with the polar pool strides; scale_log2 as for the plain kernel
int launch_polar_decode(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream);

}  // namespace sp
