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
// A carried-in state h_in (nullable) is the state before token 0: H starts at
// h_in instead of zero, which is what a real rank's local chunk receives as the
// prefix of the ranks before it (the H_in of strategies/state_passing.py:55-59).
//
// The backward is the exact gradient of the same map (what autograd through
// the reference's loop, cumprod and AllGatherCP computes):
//   g_t = dh_t + a_{t+1} g_{t+1};  db_t = g_t;  da_t = sum_group g_t h_{t-1}
// with h_{-1} = h_in, and dh_in = a_0 g_0.
// When a wave's channels share one decay, da is reduced across the wave for 16
// steps at a time (and, when the workgroup shares one decay, summed per step in
// LDS and added to da once per workgroup at the end).
#include "rmx_kernels.h"
#include "scan_common.h"

namespace rmx {

// AMODE 0: the V channels of a thread share one decay per step (group size % V == 0)
// AMODE 1: elementwise decay (groups == d)
// AMODE 2: V = 1, any grouping
// V channels per thread: fewer channels per thread means more waves in flight
// (each wave waits for its block of U steps before computing it).
template <int AMODE, int V>
__global__ __launch_bounds__(256) void linear_scan_fwd_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              const float* __restrict__ hin,
                                                              float* __restrict__ h,
                                                              float* __restrict__ cs, int batch,
                                                              int L, int d, int groups,
                                                              int world) {
  // steps per block (the block's loads in flight together): 8 measured 181-182 us per
  // configs[4] forward against 194 us with 16 and 195 us with 32 (same box, back to back)
  constexpr int U = 8;
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
  for (int v = 0; v < V; ++v) H[v] = hin ? hin[(int64_t)bb * d + c + v] : 0.f;
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
        ldv<V>(bp + ts * d, bv[u]);
        if (AMODE == 1) {
          ldv<V>(ap + ts * groups + c, av[u]);
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
        stv<V>(hp + ts * d, o);
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

// WAVE_REDUCE: a wave's 64 V channels share one decay; da is reduced across
// the wave. LDS_DA (with WAVE_REDUCE): the whole workgroup's 256 V channels
// share one decay; the wave sums are accumulated per step in LDS (dynamic, L floats)
// and added to da once per workgroup at the end, so no global atomic is in
// flight during the main loop.
template <int AMODE, int V, bool WAVE_REDUCE, bool LDS_DA>
__global__ __launch_bounds__(256) void linear_scan_bwd_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ h,
                                                              const float* __restrict__ hin,
                                                              const float* __restrict__ dh,
                                                              float* __restrict__ da,
                                                              float* __restrict__ db,
                                                              float* __restrict__ dhin, int batch,
                                                              int L, int d, int groups) {
  constexpr int U = 16;
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

  extern __shared__ float sDa[];  // [L] when LDS_DA
  if (LDS_DA) {
    for (int i = threadIdx.x; i < L; i += 256) sDa[i] = 0.f;
    __syncthreads();
  }
  float gacc[V], anext[V], h0[V];  // h0: the state before token 0 (h_in or zero)
#pragma unroll
  for (int v = 0; v < V; ++v) {
    gacc[v] = 0.f;
    anext[v] = 0.f;
    h0[v] = (hin && valid) ? hin[(int64_t)bb * d + c + v] : 0.f;
  }
  auto emit = [&](int64_t ts, const float* gv, const float* hprev) {
    if (AMODE == 1) {
      if (valid) {
        float cur[V];
        ldv<V>(dap + ts * groups + c, cur);
#pragma unroll
        for (int v = 0; v < V; ++v) cur[v] += gv[v] * hprev[v];
        stv<V>(dap + ts * groups + c, cur);
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
        if ((threadIdx.x & 63) == 0 && valid) {
          if (LDS_DA)
            atomicAdd(&sDa[ts], part);
          else
            atomicAdd(dap + ts * groups + g, part);
        }
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
        ldv<V>(gp + ts * d, gv[u]);
        if (ts > 0) {
          ldv<V>(hp + (ts - 1) * d, hv[u]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) hv[u][v] = h0[v];
        }
        if (AMODE == 1) {
          ldv<V>(ap + ts * groups + c, av[u]);
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
    float part[U];  // this lane's share of da at step ts_hi - u (wave-reduced path)
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
      if (valid) stv<V>(dbp + ts * d, o);
      if (WAVE_REDUCE) {
        float pp = 0.f;
#pragma unroll
        for (int v = 0; v < V; ++v) pp += o[v] * hv[u][v];
        part[u] = pp;
      } else {
        emit(ts, o, hv[u]);
      }
    }
    if constexpr (WAVE_REDUCE) {
      static_assert(U == 16, "butterfly over 16 steps");
      int u;
      const float sum = wave_sum16(part, threadIdx.x & 63, u);
      if ((threadIdx.x & 3) == 0 && valid) {
        if (LDS_DA)
          atomicAdd(&sDa[ts_hi - u], sum);
        else
          atomicAdd(dap + (int64_t)(ts_hi - u) * groups + g, sum);
      }
    }
  }
  for (; ts_hi >= 0; --ts_hi) {
    const int64_t ts = ts_hi;
    float o[V], hv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float gvv = valid ? gp[ts * d + v] : 0.f;
      hv[v] = (valid && ts > 0) ? hp[(ts - 1) * d + v] : h0[v];
      const float avv = valid ? (AMODE == 1 ? ap[ts * groups + c + v] : ap[ts * groups + g]) : 0.f;
      gacc[v] = gvv + anext[v] * gacc[v];
      o[v] = gacc[v];
      anext[v] = avv;
      if (valid) dbp[ts * d + v] = o[v];
    }
    emit(ts, o, hv);
  }
  if (dhin && valid) {
#pragma unroll
    for (int v = 0; v < V; ++v) dhin[(int64_t)bb * d + c + v] = anext[v] * gacc[v];  // a_0 g_0
  }
  if (LDS_DA) {
    __syncthreads();
    if (valid)
      for (int i = threadIdx.x; i < L; i += 256) atomicAdd(dap + (int64_t)i * groups + g, sDa[i]);
  }
}

__global__ void scan_fill_zero_kernel(float* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

// Decay mode for V channels per thread: 0 when the V channels of a thread share one
// decay, 1 elementwise, 2 otherwise (then V = 1).
static int scan_amode(int d, int groups, int V) {
  const int gs = d / groups;
  if (d % V == 0 && gs % V == 0) return 0;
  if (d % V == 0 && gs == 1) return 1;
  return 2;
}

// Four channels per thread (16-byte accesses) where the shape allows, else two, else one.
static int scan_v(int d, int groups) {
  for (int V : {4, 2})
    if (scan_amode(d, groups, V) != 2) return V;
  return 1;
}

template <int V>
static void launch_fwd_v(int mode, unsigned grid, const float* a, const float* b, const float* hin,
                         float* h, float* cs, int batch, int L, int d, int groups, int world,
                         hipStream_t stream) {
  if (mode == 0)
    hipLaunchKernelGGL((linear_scan_fwd_kernel<0, V>), dim3(grid), dim3(256), 0, stream, a, b, hin,
                       h, cs, batch, L, d, groups, world);
  else
    hipLaunchKernelGGL((linear_scan_fwd_kernel<1, V>), dim3(grid), dim3(256), 0, stream, a, b, hin,
                       h, cs, batch, L, d, groups, world);
}

hipError_t launch_linear_scan_fwd(const float* a, const float* b, const float* hin, float* h,
                                  float* cs, int batch, int L, int d, int groups, int world,
                                  hipStream_t stream) {
  if ((int64_t)batch * L * d == 0) return hipSuccess;
  const int V = scan_v(d, groups);
  const int mode = scan_amode(d, groups, V);
  const int64_t n = (int64_t)batch * (d / V);
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (V == 4)
    launch_fwd_v<4>(mode, grid, a, b, hin, h, cs, batch, L, d, groups, world, stream);
  else if (V == 2)
    launch_fwd_v<2>(mode, grid, a, b, hin, h, cs, batch, L, d, groups, world, stream);
  else
    hipLaunchKernelGGL((linear_scan_fwd_kernel<2, 1>), dim3(grid), dim3(256), 0, stream, a, b, hin,
                       h, cs, batch, L, d, groups, world);
  return hipGetLastError();
}

// WAVE_REDUCE needs a wave's 64 V channels in one decay group, LDS_DA a workgroup's 256.
template <int V>
static void launch_bwd_v(int mode, unsigned grid, const float* a, const float* h, const float* hin,
                         const float* dh, float* da, float* db, float* dhin, int batch, int L,
                         int d, int groups, hipStream_t stream) {
  const int gs = d / groups;
  if (mode == 1)
    hipLaunchKernelGGL((linear_scan_bwd_kernel<1, V, false, false>), dim3(grid), dim3(256), 0,
                       stream, a, h, hin, dh, da, db, dhin, batch, L, d, groups);
  else if (gs % (256 * V) == 0 && L <= 16384)
    hipLaunchKernelGGL((linear_scan_bwd_kernel<0, V, true, true>), dim3(grid), dim3(256),
                       (size_t)L * sizeof(float), stream, a, h, hin, dh, da, db, dhin, batch, L, d,
                       groups);
  else if (gs % (64 * V) == 0)
    hipLaunchKernelGGL((linear_scan_bwd_kernel<0, V, true, false>), dim3(grid), dim3(256), 0,
                       stream, a, h, hin, dh, da, db, dhin, batch, L, d, groups);
  else
    hipLaunchKernelGGL((linear_scan_bwd_kernel<0, V, false, false>), dim3(grid), dim3(256), 0,
                       stream, a, h, hin, dh, da, db, dhin, batch, L, d, groups);
}

hipError_t launch_linear_scan_bwd(const float* a, const float* h, const float* hin,
                                  const float* dh, float* da, float* db, float* dhin, int batch,
                                  int L, int d, int groups, int world, hipStream_t stream) {
  (void)world;
  if ((int64_t)batch * d == 0) return hipSuccess;
  if (L == 0) {  // no token: the carried-in state gets no gradient
    if (dhin)
      hipLaunchKernelGGL(scan_fill_zero_kernel, dim3(64), dim3(256), 0, stream, dhin,
                         (int64_t)batch * d);
    return hipGetLastError();
  }
  const int V = scan_v(d, groups);
  const int mode = scan_amode(d, groups, V);
  const int64_t n = (int64_t)batch * (d / V);
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (V == 4)
    launch_bwd_v<4>(mode, grid, a, h, hin, dh, da, db, dhin, batch, L, d, groups, stream);
  else if (V == 2)
    launch_bwd_v<2>(mode, grid, a, h, hin, dh, da, db, dhin, batch, L, d, groups, stream);
  else
    hipLaunchKernelGGL((linear_scan_bwd_kernel<2, 1, false, false>), dim3(grid), dim3(256), 0,
                       stream, a, h, hin, dh, da, db, dhin, batch, L, d, groups);
  return hipGetLastError();
}

}  // namespace rmx
