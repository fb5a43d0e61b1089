// Launch interface of the QJL codec (qjl.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

// The reference's projection matrix R [proj_dim, head_dim], N(0, scale^2) from its LCG
// (host memory).
void qjl_projection_host(float* out, int proj_dim, int head_dim, float scale);
int launch_qjl_compress(void* out, const void* x, int64_t num_vecs, int head_dim,
                        const float* proj, int proj_dim, sp_dtype dtype, hipStream_t stream);
int launch_qjl_decompress(void* out, const void* records, int64_t num_vecs, int head_dim,
                          const float* proj, int proj_dim, sp_dtype dtype, hipStream_t stream);

}  // namespace sp
