// Block-attention backward for gfx950 using the GLOBAL (ring-merged) out/lse.
//
// Reference semantics: the explicit global-lse backward of
// ring/p2p_attn.py:243-281 and ring/varlen_blocks.py:176-200:
//   P  = exp(scale*Q K^T + mask - lse)     (lse = global, natural log)
//   dV = P^T dO;  dP = dO V^T;  delta = rowsum(dO * O_global)
//   dS = P * (dP - delta);  dQ = scale dS K;  dK = scale dS^T Q
// with the GQA fold of dK/dV over the q-head group (:193-197).
//
// Two kernels, no atomics:
//   * attn_bwd_dq   (Q-major, lane = query): S^T, dP^T, dQ^T = K^T dS^T; the
//     fp32 dq rows are owned by one workgroup.
//   * attn_bwd_dkdv (KV-major, lane = key): S, dP, dV += P^T dO,
//     dK += dS^T Q; the workgroup owns its keys and loops over every q-head
//     of the GQA group, so the fold needs no cross-workgroup reduction.
//
// This unit holds the delta kernel, the dispatch over head dims and the head-dim-256
// instantiations; the head-dim-64 and -128 ones are in attn_bwd_vf.hip, built with
// VGPR-form MFMAs (the kernels themselves: attn_bwd_kernels.h).
#include "attn_bwd_kernels.h"

namespace rmx {

// ---------------------------------------------------------------- delta
// delta = rowsum(dout * out). `out` is the bf16 output (o_* strides) or, when
// OUT_F32, the fp32 merged output (a_* strides): the fp32 form keeps the bf16
// rounding of out (up to |dout|*|out|*2^-9 per element) out of dS = P (dP - delta).
// With nlse, the same pass writes nlse = -lse log2(e) (the per-query exponent
// offset of the dK/dV kernel) at the same [b, h, s] position. Rows run query-fastest
// (row = (b, h, q)), so the 4-byte delta, lse and nlse words of neighbouring rows share
// cache lines; head-fastest rows put each word on its own line (8x the written bytes).
template <int HD, bool OUT_F32, int DT>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const rmx_attn_layout L,
                                                             const void* __restrict__ out,
                                                             const uint16_t* __restrict__ dout,
                                                             float* __restrict__ delta,
                                                             const float* __restrict__ lse,
                                                             float* __restrict__ nlse, int sq) {
  constexpr int TPR = HD / 8;  // threads per row
  const int rows = L.batch * sq * L.hq;
  const int row = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int part = threadIdx.x % TPR;
  float acc = 0.f;
  int bb = 0, q = 0, h = 0;
  if (row < rows && 8 * part >= L.head_dim) {  // columns past the head dim: nothing to add
    q = row % sq;
    h = (row / sq) % L.hq;
    bb = row / (L.hq * sq);
  } else if (row < rows) {
    q = row % sq;
    h = (row / sq) % L.hq;
    bb = row / (L.hq * sq);
    const int64_t off = bb * L.o_sb + (int64_t)q * L.o_ss + h * L.o_sh + 8 * part;
    const u32x4 b = ld16(dout + off);
    float o[8];
    if (OUT_F32) {
      const float* op = reinterpret_cast<const float*>(out) + bb * L.a_sb + (int64_t)q * L.a_ss +
                        h * L.a_sh + 8 * part;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(op);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(op + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = x0[i];
        o[4 + i] = x1[i];
      }
    } else {
      const u32x4 a = ld16(reinterpret_cast<const uint16_t*>(out) + off);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = e2f<DT>(a[i] & 0xffffu);
        o[2 * i + 1] = e2f<DT>(a[i] >> 16);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc += o[2 * i] * e2f<DT>(b[i] & 0xffffu);
      acc += o[2 * i + 1] * e2f<DT>(b[i] >> 16);
    }
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < rows && part == 0) {
    const int64_t lo = bb * L.l_sb + h * L.l_sh + q;
    delta[lo] = acc;
    if (nlse) nlse[lo] = lse[lo] * -kLog2e;
  }
}

template <int HD, int DT>
static void launch_delta_t(const rmx_attn_layout& L, const void* out, int out_f32,
                           const uint16_t* dout, float* delta, const float* lse, float* nlse,
                           int sq, int64_t rows, hipStream_t stream) {
  constexpr int RPB = 256 / (HD / 8);  // rows per block
  const int grid = (int)((rows + RPB - 1) / RPB);
  if (out_f32)
    hipLaunchKernelGGL((attn_bwd_delta_kernel<HD, true, DT>), dim3(grid), dim3(256), 0, stream, L,
                       out, dout, delta, lse, nlse, sq);
  else
    hipLaunchKernelGGL((attn_bwd_delta_kernel<HD, false, DT>), dim3(grid), dim3(256), 0, stream,
                       L, out, dout, delta, lse, nlse, sq);
}

hipError_t launch_attn_bwd_delta(const rmx_attn_layout& L, const void* out, int out_f32,
                                 const uint16_t* dout, float* delta, const float* lse, float* nlse,
                                 int sq, hipStream_t stream) {
  const int64_t rows = (int64_t)L.batch * sq * L.hq;
  if (rows == 0) return hipSuccess;
  const bool f16 = L.dtype == RMX_DTYPE_F16;
  if (L.head_dim > 128 && f16)
    launch_delta_t<256, RMX_DTYPE_F16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  else if (L.head_dim > 128)
    launch_delta_t<256, RMX_DTYPE_BF16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  else if (L.head_dim > 64 && f16)
    launch_delta_t<128, RMX_DTYPE_F16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  else if (L.head_dim > 64)
    launch_delta_t<128, RMX_DTYPE_BF16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  else if (f16)
    launch_delta_t<64, RMX_DTYPE_F16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  else
    launch_delta_t<64, RMX_DTYPE_BF16>(L, out, out_f32, dout, delta, lse, nlse, sq, rows, stream);
  return hipGetLastError();
}

// the head-dim-64 and -128 launches are instantiated in attn_bwd_vf.hip
extern template hipError_t launch_bwd_t<64, RMX_DTYPE_BF16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<64, RMX_DTYPE_BF16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<64, RMX_DTYPE_F16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<64, RMX_DTYPE_F16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<128, RMX_DTYPE_BF16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<128, RMX_DTYPE_BF16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<128, RMX_DTYPE_F16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
extern template hipError_t launch_bwd_t<128, RMX_DTYPE_F16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);

template <int DT, bool DROP>
static hipError_t launch_bwd_hd(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                                hipStream_t stream) {
  if (L.head_dim > 128) return launch_bwd_t<256, DT, DROP>(L, probs, n, stream);
  if (L.head_dim > 64) return launch_bwd_t<128, DT, DROP>(L, probs, n, stream);
  return launch_bwd_t<64, DT, DROP>(L, probs, n, stream);
}

hipError_t launch_attn_bwd(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                           hipStream_t stream) {
  const bool f16 = L.dtype == RMX_DTYPE_F16, drop = L.dropout_p > 0.f;
  if (drop)
    return f16 ? launch_bwd_hd<RMX_DTYPE_F16, true>(L, probs, n, stream)
               : launch_bwd_hd<RMX_DTYPE_BF16, true>(L, probs, n, stream);
  return f16 ? launch_bwd_hd<RMX_DTYPE_F16, false>(L, probs, n, stream)
             : launch_bwd_hd<RMX_DTYPE_BF16, false>(L, probs, n, stream);
}

}  // namespace rmx
