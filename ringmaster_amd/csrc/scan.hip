// Context-parallel linear scan h_t = a_t h_{t-1} + b_t (fp32), emulated over
// `world` contiguous shards on one GPU.
//
// Reference: local_linear_scan / cp_linear_scan
// (strategies/state_passing.py:19-59). Each shard r scans its chunk from zero
// (local_h, cum_a = cumprod(a)), the (A_r = cum_a[-1], B_r = local_h[-1])
// pairs are prefix-combined in rank order (H_in = A_j H_in + B_j, :55-57) and
// the exact correction h = local_h + cum_a * H_in is applied (:59). On one GPU
// the all-gather of (A_r, B_r) becomes a register carry: a thread owns V
// channels and walks the shards in rank order, so b is read once and h written
// once (HBM-bound; the decay a is per channel group and mostly cache-resident).
//
// The backward is the exact gradient of the same map (what autograd through
// the reference's loop, cumprod and AllGatherCP computes):
//   g_t = dh_t + a_{t+1} g_{t+1};  db_t = g_t;  da_t = sum_group g_t h_{t-1}.
#include "rmx_kernels.h"

namespace rmx {

// AMODE 0: V=4 channels share one decay per step (group size % 4 == 0)
// AMODE 1: V=4 channels, elementwise decay (groups == d)
// AMODE 2: V=1, any grouping
template <int AMODE>
__global__ __launch_bounds__(256) void linear_scan_fwd_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ h,
                                                              float* __restrict__ cs, int batch,
                                                              int L, int d, int groups,
                                                              int world) {
  constexpr int V = AMODE == 2 ? 1 : 4;
  constexpr int U = 8;  // steps in flight per thread
  const int per_b = d / V;
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= (int64_t)batch * per_b) return;
  const int bb = (int)(t / per_b);
  const int c = (int)(t % per_b) * V;
  const int gs = d / groups;
  const int g = c / gs;
  const int Ls = L / world;
  const float* ap = a + (int64_t)bb * L * groups;
  const float* bp = b + (int64_t)bb * L * d + c;
  float* hp = h + (int64_t)bb * L * d + c;

  float H[V];
#pragma unroll
  for (int v = 0; v < V; ++v) H[v] = 0.f;
  for (int r = 0; r < world; ++r) {
    float loc[V], cum[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      loc[v] = 0.f;
      cum[v] = 1.f;
    }
    const int t0 = r * Ls;
    int tt = 0;
    for (; tt + U <= Ls; tt += U) {
      float bv[U][V], av[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t ts = t0 + tt + u;
        if (V == 4) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(bp + ts * d);
#pragma unroll
          for (int v = 0; v < V; ++v) bv[u][v] = x[v];
        } else {
          bv[u][0] = bp[ts * d];
        }
        if (AMODE == 1) {
          const f32x4 y = *reinterpret_cast<const f32x4*>(ap + ts * groups + c);
#pragma unroll
          for (int v = 0; v < V; ++v) av[u][v] = y[v];
        } else {
          const float s = ap[ts * groups + g];
#pragma unroll
          for (int v = 0; v < V; ++v) av[u][v] = s;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t ts = t0 + tt + u;
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          loc[v] = av[u][v] * loc[v] + bv[u][v];
          cum[v] = cum[v] * av[u][v];
          o[v] = loc[v] + cum[v] * H[v];
        }
        if (V == 4) {
          *reinterpret_cast<f32x4*>(hp + ts * d) = f32x4{o[0], o[V > 1 ? 1 : 0], o[V > 2 ? 2 : 0],
                                                          o[V > 3 ? 3 : 0]};
        } else {
          hp[ts * d] = o[0];
        }
      }
    }
    for (; tt < Ls; ++tt) {
      const int64_t ts = t0 + tt;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float av = AMODE == 1 ? ap[ts * groups + c + v] : ap[ts * groups + g];
        loc[v] = av * loc[v] + bp[ts * d + v];
        cum[v] = cum[v] * av;
        hp[ts * d + v] = loc[v] + cum[v] * H[v];
      }
    }
    if (cs) {
      float* cp = cs + ((int64_t)(r * batch + bb) * 2) * d + c;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        cp[v] = cum[v];
        cp[d + v] = loc[v];
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) H[v] = cum[v] * H[v] + loc[v];
  }
}

template <int AMODE, bool WAVE_REDUCE>
__global__ __launch_bounds__(256) void linear_scan_bwd_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ h,
                                                              const float* __restrict__ dh,
                                                              float* __restrict__ da,
                                                              float* __restrict__ db, int batch,
                                                              int L, int d, int groups) {
  constexpr int V = AMODE == 2 ? 1 : 4;
  constexpr int U = 8;
  const int per_b = d / V;
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const bool valid = t < (int64_t)batch * per_b;
  if (!WAVE_REDUCE && !valid) return;
  const int bb = valid ? (int)(t / per_b) : 0;
  const int c = valid ? (int)(t % per_b) * V : 0;
  const int gs = d / groups;
  const int g = c / gs;
  const float* ap = a + (int64_t)bb * L * groups;
  const float* hp = h + (int64_t)bb * L * d + c;
  const float* gp = dh + (int64_t)bb * L * d + c;
  float* dbp = db + (int64_t)bb * L * d + c;
  float* dap = da + (int64_t)bb * L * groups;

  float gacc[V], anext[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    gacc[v] = 0.f;
    anext[v] = 0.f;
  }
  auto emit = [&](int64_t ts, const float* gv, const float* hprev) {
    if (AMODE == 1) {
      if (valid) {
        f32x4 cur = *reinterpret_cast<const f32x4*>(dap + ts * groups + c);
#pragma unroll
        for (int v = 0; v < 4; ++v) cur[v] += gv[v] * hprev[v];
        *reinterpret_cast<f32x4*>(dap + ts * groups + c) = cur;
      }
    } else if (AMODE == 2 && gs == 1) {
      if (valid) dap[ts * groups + c] += gv[0] * hprev[0];
    } else {
      float part = 0.f;
#pragma unroll
      for (int v = 0; v < V; ++v) part += gv[v] * hprev[v];
      if (WAVE_REDUCE) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
        if ((threadIdx.x & 63) == 0 && valid) atomicAdd(dap + ts * groups + g, part);
      } else {
        atomicAdd(dap + ts * groups + g, part);
      }
    }
  };

  int ts_hi = L - 1;
  for (; ts_hi - U + 1 >= 0; ts_hi -= U) {
    float gv[U][V], hv[U][V], av[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t ts = ts_hi - u;
      if (valid) {
        if (V == 4) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(gp + ts * d);
          const f32x4 y = ts > 0 ? *reinterpret_cast<const f32x4*>(hp + (ts - 1) * d)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int v = 0; v < V; ++v) {
            gv[u][v] = x[v];
            hv[u][v] = y[v];
          }
        } else {
          gv[u][0] = gp[ts * d];
          hv[u][0] = ts > 0 ? hp[(ts - 1) * d] : 0.f;
        }
        if (AMODE == 1) {
          const f32x4 z = *reinterpret_cast<const f32x4*>(ap + ts * groups + c);
#pragma unroll
          for (int v = 0; v < V; ++v) av[u][v] = z[v];
        } else {
          const float s = ap[ts * groups + g];
#pragma unroll
          for (int v = 0; v < V; ++v) av[u][v] = s;
        }
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          gv[u][v] = 0.f;
          hv[u][v] = 0.f;
          av[u][v] = 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t ts = ts_hi - u;
      float o[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        gacc[v] = gv[u][v] + anext[v] * gacc[v];
        o[v] = gacc[v];
        anext[v] = av[u][v];
      }
      if (valid) {
        if (V == 4) {
          *reinterpret_cast<f32x4*>(dbp + ts * d) =
              f32x4{o[0], o[V > 1 ? 1 : 0], o[V > 2 ? 2 : 0], o[V > 3 ? 3 : 0]};
        } else {
          dbp[ts * d] = o[0];
        }
      }
      emit(ts, o, hv[u]);
    }
  }
  for (; ts_hi >= 0; --ts_hi) {
    const int64_t ts = ts_hi;
    float o[V], hv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float gvv = valid ? gp[ts * d + v] : 0.f;
      hv[v] = (valid && ts > 0) ? hp[(ts - 1) * d + v] : 0.f;
      const float avv = valid ? (AMODE == 1 ? ap[ts * groups + c + v] : ap[ts * groups + g]) : 0.f;
      gacc[v] = gvv + anext[v] * gacc[v];
      o[v] = gacc[v];
      anext[v] = avv;
      if (valid) dbp[ts * d + v] = o[v];
    }
    emit(ts, o, hv);
  }
}

static int scan_amode(int d, int groups) {
  const int gs = d / groups;
  if (d % 4 == 0 && gs % 4 == 0) return 0;
  if (d % 4 == 0 && gs == 1) return 1;
  return 2;
}

hipError_t launch_linear_scan_fwd(const float* a, const float* b, float* h, float* cs, int batch,
                                  int L, int d, int groups, int world, hipStream_t stream) {
  if ((int64_t)batch * L * d == 0) return hipSuccess;
  const int mode = scan_amode(d, groups);
  const int V = mode == 2 ? 1 : 4;
  const int64_t n = (int64_t)batch * (d / V);
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (mode == 0)
    hipLaunchKernelGGL(linear_scan_fwd_kernel<0>, dim3(grid), dim3(256), 0, stream, a, b, h, cs,
                       batch, L, d, groups, world);
  else if (mode == 1)
    hipLaunchKernelGGL(linear_scan_fwd_kernel<1>, dim3(grid), dim3(256), 0, stream, a, b, h, cs,
                       batch, L, d, groups, world);
  else
    hipLaunchKernelGGL(linear_scan_fwd_kernel<2>, dim3(grid), dim3(256), 0, stream, a, b, h, cs,
                       batch, L, d, groups, world);
  return hipGetLastError();
}

hipError_t launch_linear_scan_bwd(const float* a, const float* h, const float* dh, float* da,
                                  float* db, int batch, int L, int d, int groups, int world,
                                  hipStream_t stream) {
  (void)world;
  if ((int64_t)batch * L * d == 0) return hipSuccess;
  const int mode = scan_amode(d, groups);
  const int V = mode == 2 ? 1 : 4;
  const int gs = d / groups;
  const int64_t n = (int64_t)batch * (d / V);
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (mode == 0) {
    // a 64-lane wave covers 256 consecutive channels; reduce in-wave when they
    // all belong to one group
    if (gs % 256 == 0)
      hipLaunchKernelGGL((linear_scan_bwd_kernel<0, true>), dim3(grid), dim3(256), 0, stream, a, h,
                         dh, da, db, batch, L, d, groups);
    else
      hipLaunchKernelGGL((linear_scan_bwd_kernel<0, false>), dim3(grid), dim3(256), 0, stream, a,
                         h, dh, da, db, batch, L, d, groups);
  } else if (mode == 1) {
    hipLaunchKernelGGL((linear_scan_bwd_kernel<1, false>), dim3(grid), dim3(256), 0, stream, a, h,
                       dh, da, db, batch, L, d, groups);
  } else {
    hipLaunchKernelGGL((linear_scan_bwd_kernel<2, false>), dim3(grid), dim3(256), 0, stream, a, h,
                       dh, da, db, batch, L, d, groups);
  }
  return hipGetLastError();
}

}  // namespace rmx
