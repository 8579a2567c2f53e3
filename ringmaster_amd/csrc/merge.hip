// Standalone online-softmax merge (update_out_and_lse, ring/merge.py:13-31):
//   new = logaddexp(lse, blk_lse)
//   out = exp(lse - new) * out + exp(blk_lse - new) * blk_out
// out fp32 [b,s,h,d], lse fp32 [b,s,h] (the reference's [b,s,h,1]), blk_out
// bf16, fp16 or fp32 [b,s,h,d], blk_lse fp32 [b,h,s] (flash layout, transposed on
// the fly as _lse_to_bshd does). One thread owns 8 channels of one row; the
// threads of a row share the row's two lse loads through the L1. Up to 2^31
// threads the launch is one thread per 8 channels with 32-bit index math.
// HBM-bound: per element 4 (out) + 2|4 (blk) read and 4 written.
#include "rmx_fastdiv.h"
#include "rmx_kernels.h"

namespace rmx {

// Merge of the 8 channels [8 part, 8 part + 8) of row (b, s, h). BLK: RMX_BLK_*.
template <int BLK>
__device__ __forceinline__ void merge8(float* __restrict__ out, float* __restrict__ lse,
                                       const void* __restrict__ blk,
                                       const float* __restrict__ blk_lse, int b, int s, int h,
                                       int part, int64_t os0, int64_t os1, int64_t os2,
                                       int64_t ls0, int64_t ls1, int64_t ls2, int64_t bs0,
                                       int64_t bs1, int64_t bs2, int64_t bl0, int64_t bl1,
                                       int init) {
  const float lb = blk_lse[b * bl0 + h * bl1 + s];
  float* op = out + b * os0 + s * os1 + h * os2 + 8 * part;
  float* lp = lse + b * ls0 + s * ls1 + h * ls2;
  float bv[8];
  if (BLK == RMX_BLK_F32) {
    const float* bp = reinterpret_cast<const float*>(blk) + b * bs0 + s * bs1 + h * bs2 + 8 * part;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(bp);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(bp + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bv[i] = x0[i];
      bv[4 + i] = x1[i];
    }
  } else {
    const uint16_t* bp =
        reinterpret_cast<const uint16_t*>(blk) + b * bs0 + s * bs1 + h * bs2 + 8 * part;
    const u32x4 w = ld16(bp);
    constexpr int DT = BLK == RMX_BLK_F16 ? RMX_DTYPE_F16 : RMX_DTYPE_BF16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bv[2 * i] = e2f<DT>(w[i] & 0xffffu);
      bv[2 * i + 1] = e2f<DT>(w[i] >> 16);
    }
  }
  f32x4 r0, r1;
  float lnew;
  if (init) {
    lnew = lb;
    r0 = f32x4{bv[0], bv[1], bv[2], bv[3]};
    r1 = f32x4{bv[4], bv[5], bv[6], bv[7]};
  } else {
    const float la = *lp;
    const float mx = fmaxf(la, lb);
    float wa, wb;
    if (mx == kNegInf) {
      lnew = kNegInf;
      wa = 0.f;
      wb = 0.f;
    } else {
      const float mn = fminf(la, lb);
      lnew = mx + log1pf(expf(mn - mx));
      wa = expf(la - lnew);
      wb = expf(lb - lnew);
    }
    const f32x4 o0 = *reinterpret_cast<const f32x4*>(op);
    const f32x4 o1 = *reinterpret_cast<const f32x4*>(op + 4);
    r0 = o0 * wa + f32x4{bv[0], bv[1], bv[2], bv[3]} * wb;
    r1 = o1 * wa + f32x4{bv[4], bv[5], bv[6], bv[7]} * wb;
  }
  *reinterpret_cast<f32x4*>(op) = r0;
  *reinterpret_cast<f32x4*>(op + 4) = r1;
  if (part == 0) *lp = lnew;
}

// Up to 2^31 threads: one thread per 8 channels, 32-bit index arithmetic.
template <int BLK>
__global__ __launch_bounds__(256) void lse_merge_kernel32(
    float* __restrict__ out, float* __restrict__ lse, const void* __restrict__ blk,
    const float* __restrict__ blk_lse, uint32_t n, FastDiv f_tpr, FastDiv f_heads, FastDiv f_seq,
    int64_t os0, int64_t os1, int64_t os2, int64_t ls0, int64_t ls1, int64_t ls2, int64_t bs0,
    int64_t bs1, int64_t bs2, int64_t bl0, int64_t bl1, int init) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= n) return;
  const uint32_t row = fdiv(t, f_tpr);
  const uint32_t part = t - row * f_tpr.d;
  const uint32_t rs = fdiv(row, f_heads);
  const uint32_t h = row - rs * f_heads.d;
  const uint32_t b = fdiv(rs, f_seq);
  const uint32_t s = rs - b * f_seq.d;
  merge8<BLK>(out, lse, blk, blk_lse, (int)b, (int)s, (int)h, (int)part, os0, os1, os2, ls0,
                  ls1, ls2, bs0, bs1, bs2, bl0, bl1, init);
}

template <int BLK>
__global__ __launch_bounds__(256) void lse_merge_kernel(float* __restrict__ out,
                                                        float* __restrict__ lse,
                                                        const void* __restrict__ blk,
                                                        const float* __restrict__ blk_lse,
                                                        int batch, int seq, int heads, int hd,
                                                        int64_t os0, int64_t os1, int64_t os2,
                                                        int64_t ls0, int64_t ls1, int64_t ls2,
                                                        int64_t bs0, int64_t bs1, int64_t bs2,
                                                        int64_t bl0, int64_t bl1, int init) {
  const int tpr = hd / 8;
  const int64_t nthreads = (int64_t)batch * seq * heads * tpr;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < nthreads;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int part = (int)(t % tpr);
    const int64_t row = t / tpr;
    const int h = (int)(row % heads);
    const int s = (int)((row / heads) % seq);
    const int b = (int)(row / ((int64_t)heads * seq));
    merge8<BLK>(out, lse, blk, blk_lse, b, s, h, part, os0, os1, os2, ls0, ls1, ls2, bs0, bs1,
                    bs2, bl0, bl1, init);
  }
}

hipError_t launch_lse_merge(float* out, float* lse, const void* blk_out, int blk_type,
                            const float* blk_lse, int batch, int seq, int heads, int head_dim,
                            const int64_t* os, const int64_t* ls, const int64_t* bos,
                            const int64_t* bls, int init, hipStream_t stream) {
  const int64_t n = (int64_t)batch * seq * heads * (head_dim / 8);
  if (n == 0) return hipSuccess;
  if (n < (int64_t(1) << 31)) {
    const FastDiv ft = make_fastdiv((uint32_t)(head_dim / 8)), fh = make_fastdiv((uint32_t)heads),
                  fs = make_fastdiv((uint32_t)seq);
    const dim3 grid((unsigned)((n + 255) / 256));
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, out, lse, blk_out, blk_lse,
                         (uint32_t)n, ft, fh, fs, os[0], os[1], os[2], ls[0], ls[1], ls[2], bos[0],
                         bos[1], bos[2], bls[0], bls[1], init);
    };
    if (blk_type == RMX_BLK_F32)
      go(lse_merge_kernel32<RMX_BLK_F32>);
    else if (blk_type == RMX_BLK_F16)
      go(lse_merge_kernel32<RMX_BLK_F16>);
    else
      go(lse_merge_kernel32<RMX_BLK_BF16>);
    return hipGetLastError();
  }
  int64_t blocks = (n + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, out, lse, blk_out,
                       blk_lse, batch, seq, heads, head_dim, os[0], os[1], os[2], ls[0], ls[1],
                       ls[2], bos[0], bos[1], bos[2], bls[0], bls[1], init);
  };
  if (blk_type == RMX_BLK_F32)
    go(lse_merge_kernel<RMX_BLK_F32>);
  else if (blk_type == RMX_BLK_F16)
    go(lse_merge_kernel<RMX_BLK_F16>);
  else
    go(lse_merge_kernel<RMX_BLK_BF16>);
  return hipGetLastError();
}

}  // namespace rmx
