// Internal launcher declarations shared by the kernel translation units and
// the C ABI layer (abi.hip). Launchers assume validated arguments.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/ringmaster_amd.h"
#include "rmx_common.h"

namespace rmx {

hipError_t launch_attn_fwd(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                           hipStream_t stream);
hipError_t launch_attn_bwd_delta(const rmx_attn_layout& L, const void* out, int out_f32,
                                 const uint16_t* dout, float* delta, int sq, hipStream_t stream);
hipError_t launch_attn_bwd(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                           hipStream_t stream);
hipError_t launch_lse_merge(float* out, float* lse, const void* blk_out, int blk_is_f32,
                            const float* blk_lse, int batch, int seq, int heads, int head_dim,
                            const int64_t* os, const int64_t* ls, const int64_t* bos,
                            const int64_t* bls, int init, hipStream_t stream);
hipError_t launch_zigzag(const void* src, void* dst, int batch, int seq, int world, int rank,
                         int64_t row_bytes, int64_t bstride, const void* pad_row, int scatter,
                         hipStream_t stream);
hipError_t launch_linear_scan_fwd(const float* a, const float* b, float* h, float* chunk_state,
                                  int batch, int L, int d, int groups, int world,
                                  hipStream_t stream);
hipError_t launch_linear_scan_bwd(const float* a, const float* h, const float* dh, float* da,
                                  float* db, int batch, int L, int d, int groups, int world,
                                  hipStream_t stream);

}  // namespace rmx
