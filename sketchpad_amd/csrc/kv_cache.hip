// Paged KV-cache append (slot-mapped scatter) and gather (block-table walk) for gfx950.
//
// Both are pure copies, so they are bit-exact for any element type: a thread moves VB bytes
// (16 when rows and pointers allow it) of one (token, head) row, consecutive threads take
// consecutive chunks of the same row, and each 16-lane group of a wave therefore reads and
// writes a contiguous 256-byte row. The roofline is HBM: read + write of the rows moved.
#include "kv_cache.hpp"

namespace sp {

template <int VB> struct VecOf;
template <> struct VecOf<16> { using T = uint4; };
template <> struct VecOf<8> { using T = uint2; };
template <> struct VecOf<4> { using T = uint32_t; };
template <> struct VecOf<2> { using T = uint16_t; };

// Scatter new rows into the pools (PagedKvCache::store_kv, paged_attention.rs:230-310).
// One work item = one VB-byte chunk of row (token t, head h), copied for both K and V.
template <int VB>
__global__ void __launch_bounds__(256) kv_append_kernel(
    char* __restrict__ kpool, char* __restrict__ vpool, const char* __restrict__ knew,
    const char* __restrict__ vnew, int64_t tok_stride_b, int64_t head_stride_b,
    const int32_t* __restrict__ slots, int num_tokens, int hkv, int row_bytes, int block_size,
    int64_t block_stride_b, int64_t layer_off_b, int64_t num_slots) {
  using V = typename VecOf<VB>::T;
  const int cpr = row_bytes / VB;  // chunks per row
  const int64_t total = (int64_t)num_tokens * hkv * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cpr);
    const int64_t th = i / cpr;
    const int h = (int)(th % hkv);
    const int t = (int)(th / hkv);
    const int32_t slot = slots[t];
    if (slot < 0 || (int64_t)slot >= num_slots) continue;
    const int blk = slot / block_size, s = slot - blk * block_size;
    const int64_t src = (int64_t)t * tok_stride_b + (int64_t)h * head_stride_b + (int64_t)c * VB;
    const int64_t dst = (int64_t)blk * block_stride_b + layer_off_b +
                        ((int64_t)h * block_size + s) * row_bytes + (int64_t)c * VB;
    const V kv = *(const V*)(knew + src);
    const V vv = *(const V*)(vnew + src);
    *(V*)(kpool + dst) = kv;
    *(V*)(vpool + dst) = vv;
  }
}

// Copy one sequence out of the pools into [Hkv, seq_len, D] (PagedKvCache::gather_kv,
// paged_attention.rs:313-378).
template <int VB>
__global__ void __launch_bounds__(256) kv_gather_kernel(
    char* __restrict__ kout, char* __restrict__ vout, const char* __restrict__ kpool,
    const char* __restrict__ vpool, const int32_t* __restrict__ table, int seq_len, int hkv,
    int row_bytes, int block_size, int64_t block_stride_b, int64_t layer_off_b, int num_blocks) {
  using V = typename VecOf<VB>::T;
  const int cpr = row_bytes / VB;
  const int64_t total = (int64_t)hkv * seq_len * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cpr);
    const int64_t ht = i / cpr;
    const int t = (int)(ht % seq_len);
    const int h = (int)(ht / seq_len);
    const int blk = table[t / block_size];
    const int s = t % block_size;
    const int64_t dst = ((int64_t)h * seq_len + t) * row_bytes + (int64_t)c * VB;
    if (blk < 0 || blk >= num_blocks) {  // never read outside the pool
      V z{};
      *(V*)(kout + dst) = z;
      *(V*)(vout + dst) = z;
      continue;
    }
    const int64_t src = (int64_t)blk * block_stride_b + layer_off_b +
                        ((int64_t)h * block_size + s) * row_bytes + (int64_t)c * VB;
    *(V*)(kout + dst) = *(const V*)(kpool + src);
    *(V*)(vout + dst) = *(const V*)(vpool + src);
  }
}

static int grid_for(int64_t items) {
  int64_t blocks = (items + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;  // grid-stride beyond this
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

static int pick_vec(int64_t align_mask) {
  if ((align_mask & 15) == 0) return 16;
  if ((align_mask & 7) == 0) return 8;
  if ((align_mask & 3) == 0) return 4;
  return 2;
}

int launch_kv_append(const KvAppendArgs& a, hipStream_t stream) {
  const int64_t mask = a.row_bytes | a.tok_stride_b | a.head_stride_b | a.block_stride_b |
                       a.layer_off_b | (int64_t)(uintptr_t)a.kpool | (int64_t)(uintptr_t)a.vpool |
                       (int64_t)(uintptr_t)a.knew | (int64_t)(uintptr_t)a.vnew;
  const int vb = pick_vec(mask);
  const int64_t items = (int64_t)a.num_tokens * a.hkv * (a.row_bytes / vb);
  const dim3 grid(grid_for(items)), block(256);
#define SP_APPEND(VB_)                                                                       \
  hipLaunchKernelGGL(kv_append_kernel<VB_>, grid, block, 0, stream, a.kpool, a.vpool, a.knew, \
                     a.vnew, a.tok_stride_b, a.head_stride_b, a.slots, a.num_tokens, a.hkv,   \
                     a.row_bytes, a.block_size, a.block_stride_b, a.layer_off_b, a.num_slots)
  switch (vb) {
    case 16: SP_APPEND(16); break;
    case 8: SP_APPEND(8); break;
    case 4: SP_APPEND(4); break;
    default: SP_APPEND(2); break;
  }
#undef SP_APPEND
  return check_launch("kv_append_kernel");
}

int launch_kv_gather(const KvGatherArgs& a, hipStream_t stream) {
  const int64_t mask = a.row_bytes | a.block_stride_b | a.layer_off_b |
                       (int64_t)(uintptr_t)a.kout | (int64_t)(uintptr_t)a.vout |
                       (int64_t)(uintptr_t)a.kpool | (int64_t)(uintptr_t)a.vpool;
  const int vb = pick_vec(mask);
  const int64_t items = (int64_t)a.hkv * a.seq_len * (a.row_bytes / vb);
  const dim3 grid(grid_for(items)), block(256);
#define SP_GATHER(VB_)                                                                         \
  hipLaunchKernelGGL(kv_gather_kernel<VB_>, grid, block, 0, stream, a.kout, a.vout, a.kpool,    \
                     a.vpool, a.table, a.seq_len, a.hkv, a.row_bytes, a.block_size,             \
                     a.block_stride_b, a.layer_off_b, a.num_blocks)
  switch (vb) {
    case 16: SP_GATHER(16); break;
    case 8: SP_GATHER(8); break;
    case 4: SP_GATHER(4); break;
    default: SP_GATHER(2); break;
  }
#undef SP_GATHER
  return check_launch("kv_gather_kernel");
}

}  // namespace sp
