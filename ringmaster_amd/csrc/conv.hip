// Depthwise causal conv1d over the P contiguous shards of one sequence, with the
// context-parallel halo of the reference's Mamba2 conv adapter (mamba.py:46-101):
// shard r's first W-1 outputs read the last W-1 tokens of shard r-1 (the
// all-gathered halo; zeros for r = 0), and for packed sequences a tap from
// another document contributes nothing (the reference splits each shard at
// document boundaries and masks the halo by document). On the global sequence:
//   z[g] = bias + sum_{i<W} w[i] x[g - (W-1) + i] [doc(g - (W-1) + i) == doc(g)]
//   y[g] = act(z[g]),  act = identity or silu
// (causal_conv1d_fn's published semantics: a depthwise conv1d with W-1 zeros of
// left padding). HBM-bound: a thread owns runs of 8 consecutive tokens of one
// (shard, batch, channel) row and reads each as a 16-byte load, with the halo tokens
// before it from the lane below (forward) or the chunks either side (backward); a
// workgroup covers consecutive runs of one row, so the row's coordinates, weights and bias
// are scalar.
#include "rmx_kernels.h"

namespace rmx {

struct ConvArgs {
  const uint16_t* x;
  const uint16_t* w;
  const uint16_t* bias;  // nullable
  const int32_t* doc;    // nullable, [batch, world * L]
  const uint16_t* dy;    // backward
  uint16_t* y;           // forward output / backward dx
  float* dw;             // backward: += dL/dw  [C, W]
  float* db;             // backward: += dL/dbias [C] (nullable)
  int world, batch, C, L, W, act;
};

__device__ __forceinline__ void load8(const uint16_t* p, float* o) {
  const u32x4 u = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(u[i] << 16);
    o[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

// sigmoid with the hardware reciprocal (1 ulp): the outputs are bf16
__device__ __forceinline__ float sigm(float z) {
  return __builtin_amdgcn_rcpf(1.f + fast_exp2(-z * kLog2e));
}
__device__ __forceinline__ float silu(float z) { return z * sigm(z); }
// d silu / dz = s (1 + z (1 - s)), s = sigmoid(z)
__device__ __forceinline__ float dsilu(float z) {
  const float s = sigm(z);
  return s * (1.f + z * (1.f - s));
}

// Row `row` = (p * batch + b) * C + c; run j covers local tokens [8j, 8j + 8).
// A workgroup covers RUNS x 256 consecutive runs of one row, thread i the runs
// base + 256 k + i (k < RUNS), so every wave load stays contiguous while each
// thread keeps RUNS runs of loads in flight; row, p, b and c are workgroup-uniform.
// (forward 4 runs per thread, backward 2: measured best of 1, 2, 4, 8 on MI355X; the
// backward holds five chunks per run)
constexpr int kConvRunsFwd = 4, kConvRunsBwd = 2;

struct ConvRun {
  int p, b, c, t0;
  int64_t rowoff;  // element offset of the row
  bool valid;
};

template <int RUNS>
__device__ __forceinline__ ConvRun conv_run(const ConvArgs& a, int k) {
  const int nr = a.L / 8;
  const int bpr = (nr + 256 * RUNS - 1) / (256 * RUNS);
  const int row = blockIdx.x / bpr;
  const int j = (blockIdx.x - row * bpr) * 256 * RUNS + 256 * k + threadIdx.x;
  ConvRun r;
  r.valid = j < nr;
  r.t0 = (r.valid ? j : 0) * 8;
  r.c = row % a.C;
  const int pb = row / a.C;
  r.b = pb % a.batch;
  r.p = pb / a.batch;
  r.rowoff = (int64_t)row * a.L;
  return r;
}

// 8 tokens of the chunk `dir` chunks away from the run (dir = -1 previous, 0
// current, +1 next), crossing into the neighbouring shard when needed; zeros
// outside the sequence. Also the document ids of those positions (outside: ids
// that match nothing). Branch-free: an outside read is redirected to the run's
// own chunk and its values are replaced by zeros. OWN: dir is 0 and the run valid, so
// the chunk is inside the shard and needs none of that (used by the forward only: the
// backward measured 2% slower with it, with fewer VALU instructions).
template <bool DOC, bool OWN = false>
__device__ __forceinline__ void chunk(const ConvArgs& a, const uint16_t* base, const ConvRun& r,
                                      int dir, float* v, int* d) {
  if (OWN && dir == 0) {  // the run's own chunk: always inside its shard
    load8(base + r.rowoff + r.t0, v);
    if (DOC) {
      const int32_t* dp = a.doc + (int64_t)r.b * a.world * a.L + (int64_t)r.p * a.L + r.t0;
      const i32x4 d0 = *reinterpret_cast<const i32x4*>(dp);
      const i32x4 d1 = *reinterpret_cast<const i32x4*>(dp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d[i] = d0[i];
        d[4 + i] = d1[i];
      }
    }
    return;
  }
  int t = r.t0 + 8 * dir, p = r.p;
  t = t < 0 ? t + a.L : (t >= a.L ? t - a.L : t);
  p = r.t0 + 8 * dir < 0 ? p - 1 : (r.t0 + 8 * dir >= a.L ? p + 1 : p);
  const bool in = p >= 0 && p < a.world;
  const int pc = in ? p : r.p, tc = in ? t : r.t0;
  // the same (batch, channel) row of shard pc starts (pc - r.p) * batch * C rows away
  load8(base + r.rowoff + (int64_t)(pc - r.p) * a.batch * a.C * a.L + tc, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = in ? v[i] : 0.f;
  if (DOC) {
    const int32_t* dp = a.doc + (int64_t)r.b * a.world * a.L + (int64_t)pc * a.L + tc;
    const i32x4 d0 = *reinterpret_cast<const i32x4*>(dp);
    const i32x4 d1 = *reinterpret_cast<const i32x4*>(dp + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = in ? d0[i] : -1 - i;
      d[4 + i] = in ? d1[i] : -5 - i;
    }
  }
}

// Forward: the W-1 tokens before a run are the last tokens of the run of the lane below
// (a wave's runs are consecutive runs of one row). They pass between lanes by shuffles;
// only the wave's first lane loads the previous chunk, issued with the run's own loads
// (one memory round trip), so every chunk is read once from the L2 instead of twice, and
// y leaves by non-temporal stores: 0.235-0.24 against 0.26-0.27 ms at configs[4]. The
// backward's form of it (the previous and next chunks of x and the next of dy shuffled,
// the wave's edge lanes loading theirs) measured 0.59 against 0.45 ms and was not kept. The
// backward's dx also leaves by non-temporal stores (0.453 -> 0.442 ms); non-temporal loads of
// x or dy measured no gain in either direction. The activation is a template flag, and the
// forward packs y with v_cvt_pk_bf16_f32 (363 -> 248 VALU instructions per thread; 0.228 ->
// 0.221 ms). The backward keeps the integer rounding (same results): with the hardware
// packing it ran 0.445 against 0.407 ms.
// v[0..7] := the previous chunk: its last W-1 tokens from the lane below, all of it from
// pv (the loaded chunk) on the wave's first lane
template <int W, bool DOC>
__device__ __forceinline__ void halo_prev(const float* pv, const int* pd, float* v, int* d) {
  const bool first = (threadIdx.x & 63) == 0;
#pragma unroll
  for (int i = 9 - W; i < 8; ++i) {
    const float x = __shfl_up(v[8 + i], 1, 64);
    v[i] = first ? pv[i] : x;
    if (DOC) {
      const int id = __shfl_up(d[8 + i], 1, 64);
      d[i] = first ? pd[i] : id;
    }
  }
}
template <int W, bool DOC, bool ACT>
__global__ __launch_bounds__(256) void causal_conv1d_fwd_kernel(const ConvArgs a) {
  constexpr int R = kConvRunsFwd;
  const bool first = (threadIdx.x & 63) == 0;
  float xv[R][16], pv[R][8];
  int dv[R][16], pd[R][8];
  ConvRun rr[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    rr[k] = conv_run<R>(a, k);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      xv[k][i] = 0.f;
      dv[k][i] = 0;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pv[k][i] = 0.f;
      pd[k][i] = 0;
    }
    if (rr[k].valid) chunk<DOC, true>(a, a.x, rr[k], 0, xv[k] + 8, dv[k] + 8);
    if (first && rr[k].valid) chunk<DOC>(a, a.x, rr[k], -1, pv[k], pd[k]);
  }
#pragma unroll
  for (int k = 0; k < R; ++k) halo_prev<W, DOC>(pv[k], pd[k], xv[k], dv[k]);
  const int c = rr[0].c;
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = bf2f(a.w[c * W + i]);
  const float bias = a.bias ? bf2f(a.bias[c]) : 0.f;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (!rr[k].valid) continue;
    float y[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float z = bias;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const int s = 8 + q - (W - 1) + i;  // tap position in xv
        const bool ok = !DOC || dv[k][s] == dv[k][8 + q];
        z += ok ? w[i] * xv[k][s] : 0.f;
      }
      y[q] = ACT ? silu(z) : z;
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = cvt_pk_bf16(y[2 * i], y[2 * i + 1]);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(a.y + rr[k].rowoff + rr[k].t0));
  }
}

// dz[g] = dy[g] act'(z[g]);  dx[g'] = sum_i w[i] dz[g' + W-1 - i] [same doc];
// dw[i] += sum_g dz[g] x[g - (W-1) + i] [same doc];  db += sum_g dz[g].
// A thread owns dx and the dw/db terms of its 8 tokens; dz of the next W-1
// tokens (next chunk, possibly the next shard's) is recomputed.
template <int W, bool DOC, bool ACT>
__global__ __launch_bounds__(256) void causal_conv1d_bwd_kernel(const ConvArgs a) {
  constexpr int R = kConvRunsBwd;
  float xv[R][24], gv[R][16];
  int dv[R][24];
  ConvRun rr[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    rr[k] = conv_run<R>(a, k);
    if (rr[k].valid) {
      chunk<DOC>(a, a.x, rr[k], -1, xv[k], dv[k]);
      chunk<DOC>(a, a.x, rr[k], 0, xv[k] + 8, dv[k] + 8);
      chunk<DOC>(a, a.x, rr[k], 1, xv[k] + 16, dv[k] + 16);
      chunk<false>(a, a.dy, rr[k], 0, gv[k], dv[k] + 8);
      chunk<false>(a, a.dy, rr[k], 1, gv[k] + 8, dv[k] + 16);
    }
  }
  const int c = rr[0].c;
  float w[W];
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = bf2f(a.w[c * W + i]);
  const float bias = a.bias ? bf2f(a.bias[c]) : 0.f;
  float pw[W], pb = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) pw[i] = 0.f;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (!rr[k].valid) continue;
    // dz of the run's 8 tokens and of the next W-1
    float dz[8 + W - 1];
#pragma unroll
    for (int q = 0; q < 8 + W - 1; ++q) {
      float z = bias;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const int s = 8 + q - (W - 1) + i;
        const bool ok = !DOC || dv[k][s] == dv[k][8 + q];
        z += ok ? w[i] * xv[k][s] : 0.f;
      }
      dz[q] = ACT ? gv[k][q] * dsilu(z) : gv[k][q];
    }
    float dx[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const int o = q + (W - 1) - i;  // output that reads token q through tap i
        const bool ok = !DOC || dv[k][8 + o] == dv[k][8 + q];
        acc += ok ? w[i] * dz[o] : 0.f;
      }
      dx[q] = acc;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      pb += dz[q];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const int s = 8 + q - (W - 1) + i;
        const bool ok = !DOC || dv[k][s] == dv[k][8 + q];
        pw[i] += ok ? dz[q] * xv[k][s] : 0.f;
      }
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf2(dx[2 * i], dx[2 * i + 1]);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(a.y + rr[k].rowoff + rr[k].t0));
  }
  // dw / db: the workgroup's runs share one channel; one atomic per wave
  // (invalid lanes hold zeros)
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    pb += __shfl_xor(pb, m, 64);
#pragma unroll
    for (int i = 0; i < W; ++i) pw[i] += __shfl_xor(pw[i], m, 64);
  }
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < W; ++i) atomicAdd(a.dw + c * W + i, pw[i]);
    if (a.db) atomicAdd(a.db + c, pb);
  }
}

static hipError_t launch_conv(const ConvArgs& a, hipStream_t stream, bool bwd) {
  const int64_t rows = (int64_t)a.world * a.batch * a.C;
  const int runs = bwd ? kConvRunsBwd : kConvRunsFwd;
  const int64_t bpr = (a.L / 8 + 256 * runs - 1) / (256 * runs);
  if (rows * bpr == 0) return hipSuccess;
  const dim3 grid((unsigned)(rows * bpr)), block(256);
  switch (a.W) {
#define RMX_CONV_GO(w, doc, act)                                                              \
  hipLaunchKernelGGL(bwd ? (causal_conv1d_bwd_kernel<w, doc, act>)                          \
                         : (causal_conv1d_fwd_kernel<w, doc, act>), grid, block, 0, stream, a)
#define RMX_CONV_CASE(w)                                                                     \
  case w:                                                                                   \
    if (a.doc && a.act)                                                                     \
      RMX_CONV_GO(w, true, true);                                                           \
    else if (a.doc)                                                                         \
      RMX_CONV_GO(w, true, false);                                                          \
    else if (a.act)                                                                         \
      RMX_CONV_GO(w, false, true);                                                          \
    else                                                                                    \
      RMX_CONV_GO(w, false, false);                                                         \
    break;
    RMX_CONV_CASE(1)
    RMX_CONV_CASE(2)
    RMX_CONV_CASE(3)
    RMX_CONV_CASE(4)
    RMX_CONV_CASE(5)
    RMX_CONV_CASE(6)
    RMX_CONV_CASE(7)
    RMX_CONV_CASE(8)
    RMX_CONV_CASE(9)
#undef RMX_CONV_CASE
#undef RMX_CONV_GO
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_causal_conv1d_cp(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                   const int32_t* doc, uint16_t* y, int world, int batch, int C,
                                   int L, int W, int act, hipStream_t stream) {
  const ConvArgs a{x, w, bias, doc, nullptr, y, nullptr, nullptr, world, batch, C, L, W, act};
  return launch_conv(a, stream, false);
}

hipError_t launch_causal_conv1d_cp_bwd(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                       const int32_t* doc, const uint16_t* dy, uint16_t* dx,
                                       float* dw, float* db, int world, int batch, int C, int L,
                                       int W, int act, hipStream_t stream) {
  const ConvArgs a{x, w, bias, doc, dy, dx, dw, db, world, batch, C, L, W, act};
  return launch_conv(a, stream, true);
}

}  // namespace rmx
