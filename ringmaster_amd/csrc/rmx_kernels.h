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
                                 const uint16_t* dout, float* delta, const float* lse, float* nlse,
                                 int sq, hipStream_t stream);
hipError_t launch_attn_bwd(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                           hipStream_t stream);
hipError_t launch_lse_merge(float* out, float* lse, const void* blk_out, int blk_type,
                            const float* blk_lse, int batch, int seq, int heads, int head_dim,
                            const int64_t* os, const int64_t* ls, const int64_t* bos,
                            const int64_t* bls, int init, hipStream_t stream);
hipError_t launch_zigzag(const void* src, void* dst, int batch, int seq, int world, int rank,
                         int64_t row_bytes, int64_t bstride, const void* pad_row, int scatter,
                         hipStream_t stream);
hipError_t launch_linear_scan_fwd(const float* a, const float* b, const float* hin, float* h,
                                  float* chunk_state, int batch, int L, int d, int groups,
                                  int world, hipStream_t stream);
hipError_t launch_linear_scan_bwd(const float* a, const float* h, const float* hin,
                                  const float* dh, float* da, float* db, float* dhin, int batch,
                                  int L, int d, int groups, int world, hipStream_t stream);
// L-parallel (chained) scan: channel tiling, chunk length and workspace layout of one shape
struct ScanChunkPlan {
  int V, amode, cw_log2, lg_log2, CT, TC, ntiles, nchunks;
  bool two_pass;  // reduce-then-rescan instead of the single pass with look-back
  size_t words_off, bytes;
};
ScanChunkPlan scan_chunk_plan(int batch, int L, int d, int groups);
hipError_t launch_linear_scan_fwd_chunked(const ScanChunkPlan& p, const float* a, const float* b,
                                          const float* hin, float* h, float* cs, void* ws,
                                          int batch, int L, int d, int groups, int world,
                                          hipStream_t stream);
// the failure word of an L-parallel scan's workspace (after a stream synchronize)
int read_linear_scan_failure(const void* ws, hipStream_t stream, hipError_t* err);
hipError_t launch_linear_scan_bwd_chunked(const ScanChunkPlan& p, const float* a, const float* h,
                                          const float* hin, const float* dh, float* da, float* db,
                                          float* dhin, void* ws, int batch, int L, int d,
                                          int groups, hipStream_t stream);

hipError_t launch_mamba2_correction(const uint16_t* out, uint16_t* y, const float* h_final,
                                    float* h_final_out, const uint16_t* C, const float* cum_A,
                                    const float* h_prev, const int32_t* seq_idx, int batch, int T,
                                    int nheads, int head_dim, int ngroups, int d_state,
                                    hipStream_t stream);
size_t mamba2_bwd_workspace(int batch, int T, int nheads, int head_dim, int d_state);
hipError_t mamba2_bwd_scratch(void** out);
hipError_t launch_mamba2_correction_bwd(const uint16_t* gy, const float* ghf, const uint16_t* C,
                                        const float* cum_A, const float* h_prev,
                                        const int32_t* seq_idx, uint16_t* gC, float* g_cumA,
                                        float* g_hprev, void* workspace, int batch, int T,
                                        int nheads, int head_dim, int ngroups, int d_state,
                                        hipStream_t stream);
hipError_t launch_mamba2_dt_cumsum(const void* dt, int dt_f32, const float* bias, const float* A,
                                   int softplus, float* cum_A, float* e, float* decay, int rows,
                                   int T, int H, hipStream_t stream);
hipError_t launch_mamba2_dt_cumsum_bwd(const void* dt, int dt_f32, const float* bias,
                                       const float* A, int softplus, const float* g_cum,
                                       const float* g_e, const float* g_decay, const float* decay,
                                       float* g_dt, float* g_A, float* g_bias, int rows, int T,
                                       int H, hipStream_t stream);
hipError_t launch_mamba2_chunk_state(const uint16_t* x, const uint16_t* B, const float* e,
                                     const float* cum_A, const int32_t* t0, float* state,
                                     int rows, int T, int H, int D, int G, int N,
                                     hipStream_t stream);
size_t mamba2_chunk_state_bwd_workspace(int rows, int H, int D, int N);
hipError_t launch_mamba2_chunk_state_bwd(const uint16_t* x, const uint16_t* B, const float* e,
                                         const float* cum_A, const int32_t* t0,
                                         const float* g_state, uint16_t* g_x, uint16_t* g_B,
                                         float* g_e, float* g_cum, int rows, int T, int H, int D,
                                         int G, int N, void* workspace, hipStream_t stream);
hipError_t launch_causal_conv1d_cp(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                   const int32_t* doc, uint16_t* y, int world, int batch, int C,
                                   int L, int W, int act, hipStream_t stream);
hipError_t launch_causal_conv1d_cp_bwd(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                       const int32_t* doc, const uint16_t* dy, uint16_t* dx,
                                       float* dw, float* db, int world, int batch, int C, int L,
                                       int W, int act, hipStream_t stream);

}  // namespace rmx

namespace rmx {

// ---------------------------------------------------------------------------
// Workgroup -> (problem, group, tile) mapping shared by the attention kernels.
// A "group" is one (batch, head) of a problem (its tiles share K/V or Q/dO) and
// every group has ntile[p] workgroups. Problems are ordered longest-workgroup
// first by the launcher. Balanced mode (every problem's group count divisible
// by 8): the dispatcher deals workgroup ids round-robin over the 8 XCDs, so
// XCD x = bid % 8 runs ids bid = 8 i + x in order of i; groups g of every
// problem with g % 8 == x are placed on XCD x (one XCD's L2 serves a group's
// shared operand, every XCD gets the same share of every problem).
struct WgMapParams {
  int nprob;
  int balanced;
  int ntile[RMX_MAX_BATCHED];
  int start[RMX_MAX_BATCHED + 1];  // balanced: per-XCD prefix; else: global prefix
  int total;                       // workgroups doing work (grid may be larger)
};

struct WgCoord {
  int p, group, tile;
  bool valid;
};

__device__ __forceinline__ WgCoord map_workgroup(const WgMapParams& m, int bid) {
  WgCoord c;
  const int i = m.balanced ? (bid >> 3) : bid;
  c.valid = m.balanced ? (i < m.start[m.nprob]) : (bid < m.total);
  int p = 0;
  while (p + 1 < m.nprob && i >= m.start[p + 1]) ++p;
  const int local = i - m.start[p];
  c.p = p;
  c.tile = local % m.ntile[p];
  c.group = m.balanced ? (local / m.ntile[p]) * 8 + (bid & 7) : local / m.ntile[p];
  return c;
}

// Host side: fill the mapping for problems already in launch order; groups[p] =
// groups of problem p, ntile[p] = workgroups per group. Returns the grid size.
inline int plan_workgroups(WgMapParams& m, int n, const int* groups, const int* ntile) {
  m.nprob = n;
  m.balanced = n > 0;
  for (int i = 0; i < n; ++i) m.balanced = m.balanced && groups[i] % 8 == 0;
  int acc = 0;
  for (int i = 0; i < n; ++i) {
    m.ntile[i] = ntile[i] > 0 ? ntile[i] : 1;
    m.start[i] = acc;
    acc += (m.balanced ? groups[i] / 8 : groups[i]) * (ntile[i] > 0 ? ntile[i] : 0);
  }
  for (int i = n; i <= RMX_MAX_BATCHED; ++i) m.start[i] = acc;
  m.total = acc;
  return m.balanced ? 8 * acc : acc;
}

// ---------------------------------------------------------------------------
// 16-bit element types of the attention kernels (RMX_DTYPE_BF16, RMX_DTYPE_F16).
// Operands travel as bf16x8 bit patterns in both cases (loads, LDS tiles, transposed
// reads and the sign flip of V are bit operations on 16-bit lanes); only the MFMA and
// the fp32 <-> 16-bit conversions (round to nearest even) depend on the type.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ f32x16 mfma32t(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  if constexpr (DT == RMX_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Two floats -> two packed 16-bit elements (lo in bits 0..15).
template <int DT>
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  if constexpr (DT == RMX_DTYPE_F16) {
    const f32x2 f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
  } else {
    return cvt_pk_bf16(lo, hi);
  }
}
template <int DT>
__device__ __forceinline__ uint16_t f2e(float f) {
  if constexpr (DT == RMX_DTYPE_F16)
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  else
    return f2bf(f);
}
template <int DT>
__device__ __forceinline__ float e2f(uint32_t bits16) {
  if constexpr (DT == RMX_DTYPE_F16)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  else
    return bf2f((uint16_t)bits16);
}
template <int DT>
__device__ __forceinline__ bf16x8 pack8t(const float* v) {
  u32x4 u;
  u[0] = cvt_pk<DT>(v[0], v[1]);
  u[1] = cvt_pk<DT>(v[2], v[3]);
  u[2] = cvt_pk<DT>(v[4], v[5]);
  u[3] = cvt_pk<DT>(v[6], v[7]);
  return __builtin_bit_cast(bf16x8, u);
}

// ---------------------------------------------------------------------------
// Attention dropout. Element (batch b, q head h, query q, key k) of a call with
// dropout is kept when
//   fmix32(bhmix ^ (q + q0) * kDropQ ^ (k + k0) * kDropK) >= threshold,
//   bhmix = fmix32(seed_lo ^ fmix32(seed_hi ^ (b * hq + h) * kDropBH)),
// with fmix32 the MurmurHash3 finalizer, threshold = floor(p 2^32) and (q0, k0) the
// problem's coordinate offsets (a ring block's place in the gathered sequence).
// Kept probabilities are scaled by 1 / (1 - p); lse is that of the undropped scores.
// Every element is its own counter, so each kernel evaluates the mask in whatever
// lane layout it holds the scores in, and the forward and both backward kernels
// agree on it bit for bit.
constexpr uint32_t kDropQ = 0x85ebca77u, kDropK = 0xc2b2ae3du, kDropBH = 0x9e3779b9u;
__device__ __forceinline__ uint32_t fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  return x;
}
__device__ __forceinline__ uint32_t drop_bhmix(const rmx_attn_layout& L, int bb, int head) {
  return fmix32(L.drop_seed_lo ^ fmix32(L.drop_seed_hi ^ (uint32_t)(bb * L.hq + head) * kDropBH));
}
// qterm = bhmix ^ (q + q0) * kDropQ, kterm = (k + k0) * kDropK
__device__ __forceinline__ bool drop_keep(uint32_t qterm, uint32_t kterm, uint32_t thr) {
  return fmix32(qterm ^ kterm) >= thr;
}

// Host side: the keep threshold floor(p 2^32) and the scale 1 / (1 - p) of dropout p.
inline void drop_params(float p, uint32_t* thr, float* scale) {
  if (!(p > 0.f)) {
    *thr = 0u;
    *scale = 1.f;
    return;
  }
  const double t = (double)p * 4294967296.0;
  *thr = t >= 4294967295.0 ? 4294967295u : (uint32_t)t;
  *scale = (float)(1.0 / (1.0 - (double)p));
}

// Host side: order[] = problem indices sorted by cost[] descending (stable).
inline void order_by_cost(int n, const long long* cost, int* order) {
  for (int i = 0; i < n; ++i) order[i] = i;
  for (int i = 1; i < n; ++i) {
    const int o = order[i];
    int j = i - 1;
    while (j >= 0 && cost[order[j]] < cost[o]) {
      order[j + 1] = order[j];
      --j;
    }
    order[j + 1] = o;
  }
}

}  // namespace rmx
