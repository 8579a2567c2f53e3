// Mamba2 CP chunk decay from dt (strategies/mamba.py:276-283): per row (rank
// shard x batch) and head,
//   e_t = softplus(dt_t + dt_bias) when dt_softplus, else dt_t
//   cum_A_t = sum_{s<=t} A e_s,   decay = exp(cum_A_{T-1})
// and the gradient of that map. softplus follows torch (beta 1, threshold 20:
// x > 20 -> x). A workgroup = 4 waves over one row and 64 consecutive heads
// (lane = head, so each step of a wave reads 64 consecutive dt values); the
// waves take consecutive quarters of the tokens and exchange their quarter sums
// through LDS between a summing pass and a writing pass.
#include "rmx_kernels.h"

namespace rmx {

struct DtArgs {
  const void* dt;        // [rows, T, H] bf16 or fp32
  int dt_f32;
  const float* bias;     // [H] or null
  const float* A;        // [H]
  int softplus;
  float* cum_A;          // fwd out [rows, T, H]
  float* e_out;          // fwd out [rows, T, H] (effective dt) or null
  const float* g_e;      // bwd in [rows, T, H] (direct gradient of e) or null
  float* decay;          // fwd out / bwd in [rows, H]
  const float* g_cum;    // bwd in [rows, T, H] or null
  const float* g_decay;  // bwd in [rows, H] or null
  float* g_dt;           // bwd out [rows, T, H] (fp32)
  float* g_A;            // bwd += [H]
  float* g_bias;         // bwd += [H] (softplus only) or null
  int rows, T, H;
};

__device__ __forceinline__ float dt_at(const DtArgs& a, int64_t i) {
  return a.dt_f32 ? reinterpret_cast<const float*>(a.dt)[i]
                  : bf2f(reinterpret_cast<const uint16_t*>(a.dt)[i]);
}
__device__ __forceinline__ float softplus_t(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float softplus_grad(float x) {  // d softplus / dx
  if (x > 20.f) return 1.f;
  const float z = expf(x);
  return z / (z + 1.f);
}

// tokens of wave w: [T w / 4, T (w + 1) / 4)
__device__ __forceinline__ void quarter(int T, int w, int& lo, int& hi) {
  lo = (int)((int64_t)T * w / 4);
  hi = (int)((int64_t)T * (w + 1) / 4);
}

__global__ __launch_bounds__(256) void mamba2_dt_cumsum_kernel(const DtArgs a) {
  __shared__ float part[4][64];
  const int hb = (a.H + 63) / 64;
  const int r = blockIdx.x / hb;
  const int h = (blockIdx.x % hb) * 64 + (threadIdx.x & 63);
  const int w = threadIdx.x >> 6;
  const bool hv = h < a.H;
  const float Ah = hv ? a.A[h] : 0.f;
  const float bh = (hv && a.bias) ? a.bias[h] : 0.f;
  int lo, hi;
  quarter(a.T, w, lo, hi);
  const int64_t base = (int64_t)r * a.T * a.H + h;
  auto e_of = [&](int t) -> float {
    const float x = dt_at(a, base + (int64_t)t * a.H);
    return a.softplus ? softplus_t(x + bh) : x;
  };
  float s = 0.f;
  if (hv) {
#pragma unroll 8
    for (int t = lo; t < hi; ++t) s += Ah * e_of(t);
  }
  part[w][threadIdx.x & 63] = s;
  __syncthreads();
  float run = 0.f;
  for (int v = 0; v < w; ++v) run += part[v][threadIdx.x & 63];
  if (hv) {
#pragma unroll 8
    for (int t = lo; t < hi; ++t) {
      const float e = e_of(t);
      run += Ah * e;
      a.cum_A[base + (int64_t)t * a.H] = run;
      if (a.e_out) a.e_out[base + (int64_t)t * a.H] = e;
    }
    if (w == 3) a.decay[(int64_t)r * a.H + h] = expf(run);
  }
}

// G_t = g_cum_t (+ g_decay decay at t = T-1);  R_s = sum_{t>=s} G_t;
// g_e_s = A R_s (+ the direct g_e_s);  g_A += sum_s R_s e_s;  g_dt_s = g_e_s softplus'(dt_s + bias)
// (or g_e_s);  g_bias += sum_s g_dt_s (softplus only).
__global__ __launch_bounds__(256) void mamba2_dt_cumsum_bwd_kernel(const DtArgs a) {
  __shared__ float part[4][64];
  __shared__ float red[2][4][64];
  const int hb = (a.H + 63) / 64;
  const int r = blockIdx.x / hb;
  const int lane = threadIdx.x & 63;
  const int h = (blockIdx.x % hb) * 64 + lane;
  const int w = threadIdx.x >> 6;
  const bool hv = h < a.H;
  const float Ah = hv ? a.A[h] : 0.f;
  const float bh = (hv && a.bias) ? a.bias[h] : 0.f;
  int lo, hi;
  quarter(a.T, w, lo, hi);
  const int64_t base = (int64_t)r * a.T * a.H + h;
  const float gd = (hv && a.g_decay) ? a.g_decay[(int64_t)r * a.H + h] * a.decay[(int64_t)r * a.H + h]
                                     : 0.f;
  auto G_of = [&](int t) -> float {
    float g = a.g_cum ? a.g_cum[base + (int64_t)t * a.H] : 0.f;
    return t == a.T - 1 ? g + gd : g;
  };
  float s = 0.f;
  if (hv) {
#pragma unroll 8
    for (int t = lo; t < hi; ++t) s += G_of(t);
  }
  part[w][lane] = s;
  __syncthreads();
  float run = 0.f;  // suffix sum of the later quarters
  for (int v = w + 1; v < 4; ++v) run += part[v][lane];
  float pa = 0.f, pb = 0.f;
  if (hv) {
#pragma unroll 8
    for (int t = hi - 1; t >= lo; --t) {
      run += G_of(t);
      const float x = dt_at(a, base + (int64_t)t * a.H);
      const float e = a.softplus ? softplus_t(x + bh) : x;
      pa += run * e;
      const float ge = Ah * run + (a.g_e ? a.g_e[base + (int64_t)t * a.H] : 0.f);
      const float gdt = a.softplus ? ge * softplus_grad(x + bh) : ge;
      pb += gdt;
      a.g_dt[base + (int64_t)t * a.H] = gdt;
    }
  }
  red[0][w][lane] = pa;
  red[1][w][lane] = pb;
  __syncthreads();
  if (w == 0 && hv) {
    const float sa = red[0][0][lane] + red[0][1][lane] + red[0][2][lane] + red[0][3][lane];
    const float sb = red[1][0][lane] + red[1][1][lane] + red[1][2][lane] + red[1][3][lane];
    atomicAdd(a.g_A + h, sa);
    if (a.softplus && a.g_bias) atomicAdd(a.g_bias + h, sb);
  }
}

hipError_t launch_mamba2_dt_cumsum(const void* dt, int dt_f32, const float* bias, const float* A,
                                   int softplus, float* cum_A, float* e, float* decay, int rows,
                                   int T, int H, hipStream_t stream) {
  DtArgs a{dt, dt_f32, bias, A, softplus, cum_A, e, nullptr, decay, nullptr, nullptr, nullptr,
           nullptr, nullptr, rows, T, H};
  const int64_t grid = (int64_t)rows * ((H + 63) / 64);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(mamba2_dt_cumsum_kernel, dim3((unsigned)grid), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_mamba2_dt_cumsum_bwd(const void* dt, int dt_f32, const float* bias,
                                       const float* A, int softplus, const float* g_cum,
                                       const float* g_e, const float* g_decay, const float* decay,
                                       float* g_dt, float* g_A, float* g_bias, int rows, int T,
                                       int H, hipStream_t stream) {
  DtArgs a{dt, dt_f32, bias, A, softplus, nullptr, nullptr, g_e, const_cast<float*>(decay),
           g_cum, g_decay, g_dt, g_A, g_bias, rows, T, H};
  const int64_t grid = (int64_t)rows * ((H + 63) / 64);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(mamba2_dt_cumsum_bwd_kernel, dim3((unsigned)grid), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace rmx
