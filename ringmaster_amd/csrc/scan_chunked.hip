// Context-parallel linear scan parallel over L (fp32): the chained single-pass
// form of h_t = a_t h_{t-1} + b_t for long sequences with few channels, where a
// thread per channel walking all of L would leave most of the chip idle.
//
// Reference: local_linear_scan / cp_linear_scan (strategies/state_passing.py:19-59).
// The reference scans each shard from zero, folds the shards' affine pairs
// (A_r = prod a, B_r = the shard's zero-init state at its end) in rank order,
// H_in = A_j H_in + B_j (:55-57), and corrects h = local_h + cum_a * H_in (:59).
// This path applies that fold at four levels of the machine:
//  * thread: U consecutive tokens of V channels, scanned from zero in registers;
//  * wavefront: the token groups of a wave (lanes with the same channels) fold
//    their pairs by an inclusive scan over lanes, log2 shuffle steps;
//  * workgroup: the eight waves' totals fold through LDS into the chunk's pair;
//  * chip: chunks fold in sequence order by decoupled look-back. A workgroup
//    takes its chunk from a ticket counter, so every earlier chunk belongs to a
//    workgroup that is already running; it publishes its pair, walks back over the
//    chunks whose pair is published to the nearest one whose carried-out state is,
//    and applies those pairs to that state in order, each as fma(A, S, B) exactly
//    as the chunk's owner publishes its own state. The carried state is therefore
//    the same bits whichever chunk the walk stopped at: S_c = fma(A_c, S_{c-1}, B_c)
//    along the whole chain, and the results do not depend on timing.
// Every token's h is its thread-local state plus cum_a times the state entering
// the thread's first token: the reference's correction (:59), per thread. b is
// read once and h written once; per chunk the workspace holds one pair and one
// state per channel.
//
// The look-back wait is bounded: a chunk whose predecessor has published nothing
// after kSpinCap polls takes NaN as its carried-in state and sets the workspace's
// failure word (next to the ticket counter), so the outputs show the failure, the
// host can read it back (rmx_linear_scan_status), and every workgroup still ends.
//
// A single pass costs about 200 ns of latency per chunk of a chain, which dominates when
// few channels run over a long sequence (L = 65536, d = 256: 1024 chunks, 0.26 ms for
// 30 us of traffic). There the same per-chunk code runs as reduce-then-rescan: pass 1
// publishes each chunk's pair and stops, a fold kernel composes each channel's chain of
// pairs in 64 segments (16 channels per workgroup, the segments' maps combined in LDS)
// and publishes the state after every chunk, and pass 2 rescans every chunk from the
// state before it. The fold associates the chain differently from the
// look-back, so the two forms differ in rounding (each is deterministic); the price is
// reading a and x twice. The plan picks the form from the measured costs.
//
// The backward is the same machinery over the reversed sequence:
//   g_t = dh_t + a_{t+1} g_{t+1}   (a scan from the end with decay a_{t+1}),
//   db_t = g_t,  da_t += sum_group g_t h_{t-1} (h_{-1} = h_in),  dh_in = a_0 g_0.
#include <algorithm>

#include "rmx_kernels.h"
#include "scan_common.h"

namespace rmx {

namespace {

constexpr int kU = 16;             // tokens per thread
// waves per workgroup, token-ordered: 8 against 4 halves the chunks of a chain (and its
// look-back words and latency): 1.24 -> 0.96 / 2.00 -> 1.60 ms fwd / bwd at L = 131072, d = 4096;
// 16 spills (368 bytes in the backward) and ran the backward 2.5 ms
constexpr int kWaves = 8;
constexpr int kSpinCap = 1 << 22;  // look-back polls before giving up (about 0.3 s)

// Cross-workgroup words: a 32-bit value with a nonzero tag in the upper half, written
// and read as single 64-bit device-scope atomics. A reader that sees the tag sees the
// value of the same store, so publishing needs no fence (an agent-scope release would
// write back the whole L2 of the XCD, full of the streaming outputs) and polling no
// cache invalidation. The workspace is zeroed before every call.
struct ChunkWork {
  int* counter;     // chunk tickets in dispatch order; counter[1]: the failure word
  uint64_t* words;  // [chains * nchunks][3][CT]: A, B of the chunk's pair, state after it
  int ntiles, nchunks;
};

enum { kWordA = 0, kWordB = 1, kWordS = 2 };

__device__ __forceinline__ void put_word(uint64_t* p, float v) {
  __hip_atomic_store(p, ((uint64_t)1 << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool word_set(uint64_t w) { return (w >> 32) != 0; }
__device__ __forceinline__ float word_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

}  // namespace

// AMODE 0: a thread's V channels share one decay (group size % V == 0);
// AMODE 1: elementwise decay (groups == d), loaded as V-vectors.
// BWD: x = dh, y = db; the scan runs from the end of the sequence.
// Channel tile CT = CW * V with CW = 2^cw_log2 lanes per token group; a wave
// holds 64 / CW token groups of kU tokens. lg_log2: lanes sharing one decay
// group inside a token group (da reduction in the backward), -1 = none shared.
// PASS 0: single pass with look-back; 1: publish the chunk's pair only; 2: outputs from
// the state the fold kernel left for the previous chunk.
template <int AMODE, int V, bool BWD, int PASS>
__global__ __launch_bounds__(64 * kWaves) void linear_scan_chunked_kernel(
    const float* __restrict__ a, const float* __restrict__ x, const float* __restrict__ hin,
    const float* __restrict__ hfwd, float* __restrict__ y, float* __restrict__ da,
    float* __restrict__ dhin, ChunkWork w, int batch, int L, int d, int groups, int cw_log2,
    int lg_log2) {
  constexpr int U = kU;
  constexpr int AV = AMODE == 1 ? V : 1;
  const int CW = 1 << cw_log2, CT = CW * V, TGW = 64 >> cw_log2, TC = kWaves * TGW * U;
  __shared__ int s_ticket;
  __shared__ float s_totA[kWaves][256];
  __shared__ float s_totB[kWaves][256];
  __shared__ float s_carry[256];

  if (PASS == 0) {
    if (threadIdx.x == 0) s_ticket = atomicAdd(w.counter, 1);
    __syncthreads();
  }
  // reduce-then-rescan never polls: clear a failure word an earlier call may have left
  if (PASS == 1 && blockIdx.x == 0 && threadIdx.x == 0) w.counter[1] = 0;
  // no chunk waits for another in passes 1 and 2: the dispatch order needs no ticket
  const int ticket = PASS == 0 ? s_ticket : (int)blockIdx.x;
  const int nchains = batch * w.ntiles;
  const int chunk = ticket / nchains;
  const int chain = ticket - chunk * nchains;
  const int bb = chain / w.ntiles;
  const int tile = chain - bb * w.ntiles;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int cl = lane & (CW - 1), tgw = lane >> cw_log2;
  const int c = tile * CT + cl * V;
  const bool cv = c < d;  // V divides d: the thread's V channels are all valid or none
  const int gs = d / groups;
  const int tau0 = chunk * TC + (wv * TGW + tgw) * U;  // first token in scan order
  const int64_t row0 = (int64_t)bb * L;

  float v_[U][V];    // x, then the thread-local state
  float cm[U][AV];   // decay, then its running product
  float hp[BWD ? U : 1][V];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tau = tau0 + u;
    const int t = BWD ? L - 1 - tau : tau;
    const bool ok = cv && tau < L;
    const int ta = BWD ? t + 1 : t;  // the decay that multiplies the carried state
    if (ok) {
      ldv<V>(x + (row0 + t) * d + c, v_[u]);
      if (ta >= L) {
#pragma unroll
        for (int i = 0; i < AV; ++i) cm[u][i] = 1.f;
      } else if (AMODE == 1) {
        ldv<V>(a + (row0 + ta) * groups + c, cm[u]);
      } else {
        cm[u][0] = a[(row0 + ta) * groups + c / gs];
      }
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) v_[u][v] = 0.f;
#pragma unroll
      for (int i = 0; i < AV; ++i) cm[u][i] = 1.f;
    }
    if constexpr (BWD) {
      if (ok && t > 0) {
        ldv<V>(hfwd + (row0 + t - 1) * d + c, hp[u]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) hp[u][v] = (ok && hin) ? hin[(int64_t)bb * d + c + v] : 0.f;
      }
    }
  }

  // thread: local scan from zero; (IA, IB) = the thread's pair
  float IA[AV], IB[V];
#pragma unroll
  for (int v = 0; v < V; ++v) IB[v] = 0.f;
#pragma unroll
  for (int i = 0; i < AV; ++i) IA[i] = 1.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      IB[v] = cm[u][AMODE == 1 ? v : 0] * IB[v] + v_[u][v];
      v_[u][v] = IB[v];
    }
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      IA[i] *= cm[u][i];
      cm[u][i] = IA[i];
    }
  }

  // wavefront: inclusive scan of the pairs over the wave's token groups
  for (int o = CW; o < 64; o <<= 1) {
    float pa[AV], pb[V];
#pragma unroll
    for (int i = 0; i < AV; ++i) pa[i] = __shfl_up(IA[i], o, 64);
#pragma unroll
    for (int v = 0; v < V; ++v) pb[v] = __shfl_up(IB[v], o, 64);
    if (lane >= o) {
#pragma unroll
      for (int v = 0; v < V; ++v) IB[v] = IA[AMODE == 1 ? v : 0] * pb[v] + IB[v];
#pragma unroll
      for (int i = 0; i < AV; ++i) IA[i] *= pa[i];
    }
  }
  // exclusive pair of the thread within its wave
  float EA[AV], EB[V];
#pragma unroll
  for (int i = 0; i < AV; ++i) EA[i] = TGW > 1 ? __shfl_up(IA[i], CW, 64) : 1.f;
#pragma unroll
  for (int v = 0; v < V; ++v) EB[v] = TGW > 1 ? __shfl_up(IB[v], CW, 64) : 0.f;
  if (tgw == 0) {
#pragma unroll
    for (int i = 0; i < AV; ++i) EA[i] = 1.f;
#pragma unroll
    for (int v = 0; v < V; ++v) EB[v] = 0.f;
  }
  if (tgw == TGW - 1) {
#pragma unroll
    for (int i = 0; i < AV; ++i) s_totA[wv][cl * AV + i] = IA[i];
#pragma unroll
    for (int v = 0; v < V; ++v) s_totB[wv][cl * V + v] = IB[v];
  }
  __syncthreads();

  // workgroup: fold of the waves before this one (P) and of all four (the chunk's pair)
  float PA[AV], PB[V], CA[AV], CB[V];
#pragma unroll
  for (int i = 0; i < AV; ++i) CA[i] = 1.f;
#pragma unroll
  for (int v = 0; v < V; ++v) CB[v] = 0.f;
#pragma unroll
  for (int j = 0; j < kWaves; ++j) {
    if (j == wv) {
#pragma unroll
      for (int i = 0; i < AV; ++i) PA[i] = CA[i];
#pragma unroll
      for (int v = 0; v < V; ++v) PB[v] = CB[v];
    }
#pragma unroll
    for (int v = 0; v < V; ++v) CB[v] = s_totA[j][cl * AV + (AMODE == 1 ? v : 0)] * CB[v] + s_totB[j][cl * V + v];
#pragma unroll
    for (int i = 0; i < AV; ++i) CA[i] *= s_totA[j][cl * AV + i];
  }

  // chip: publish the chunk's pair, look back, publish the carried-out state
  const int64_t s0 = (int64_t)chain * w.nchunks;
  auto word = [&](int64_t k, int kind, int v) {
    return w.words + ((s0 + k) * 3 + kind) * CT + cl * V + v;
  };
  if (PASS == 1) {  // the chunk's pair for the fold kernel: nothing else
    if (wv == 0 && tgw == 0 && cv) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        put_word(word(chunk, kWordA, v), CA[AMODE == 1 ? v : 0]);
        put_word(word(chunk, kWordB, v), CB[v]);
      }
    }
    return;
  }
  if (PASS == 2) {  // the state after the previous chunk, from the fold kernel
    if (wv == 0 && tgw == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float X = 0.f;
        if (chunk == 0)
          X = (!BWD && hin && cv) ? hin[(int64_t)bb * d + c + v] : 0.f;
        else if (cv)
          X = word_val(get_word(word(chunk - 1, kWordS, v)));
        s_carry[cl * V + v] = X;
      }
    }
  }
  if (PASS == 0 && wv == 0) {
    if (tgw == 0 && cv) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        put_word(word(chunk, kWordA, v), CA[AMODE == 1 ? v : 0]);
        put_word(word(chunk, kWordB, v), CB[v]);
      }
    }
    float X[V] = {};  // the state entering this chunk
    if (chunk == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) X[v] = (!BWD && hin && cv) ? hin[(int64_t)bb * d + c + v] : 0.f;
    } else {
      // back to the nearest chunk whose state every lane sees (each chunk passed on the
      // way has its pair published in every lane) ...
      int j = chunk - 1;
      bool ok = true;
      for (int spins = 0;;) {
        bool st = true, pr = true;
        if (cv) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const uint64_t ws = get_word(word(j, kWordS, v));
            st = st && word_set(ws);
            X[v] = word_val(ws);
          }
        }
        if (__all(st)) break;
        if (cv && j > 0) {
#pragma unroll
          for (int v = 0; v < V; ++v)
            pr = pr && word_set(get_word(word(j, kWordA, v))) && word_set(get_word(word(j, kWordB, v)));
        }
        if (j > 0 && __all(pr)) {
          --j;
          spins = 0;
          continue;
        }
        if (++spins > kSpinCap) {  // chunk j published nothing: only if progress stopped
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      // ... then forward, applying each pair to the state exactly as its owner publishes
      // it, so the carry is the same bits whichever chunk the walk stopped at
      for (int k = j + 1; ok && k < chunk; ++k) {
#pragma unroll
        for (int v = 0; v < V; ++v)
          X[v] = __builtin_fmaf(word_val(get_word(word(k, kWordA, v))), X[v],
                                word_val(get_word(word(k, kWordB, v))));
      }
      if (!ok) {
#pragma unroll
        for (int v = 0; v < V; ++v) X[v] = __builtin_nanf("");
        if (tgw == 0) atomicOr(w.counter + 1, 1);
      }
    }
    if (tgw == 0) {
      if (cv) {
#pragma unroll
        for (int v = 0; v < V; ++v)
          put_word(word(chunk, kWordS, v), __builtin_fmaf(CA[AMODE == 1 ? v : 0], X[v], CB[v]));
      }
#pragma unroll
      for (int v = 0; v < V; ++v) s_carry[cl * V + v] = X[v];
    }
  }
  __syncthreads();

  // the state entering the thread's first token: E after P after the chunk's carry
  float Y[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = AMODE == 1 ? v : 0;
    Y[v] = EA[i] * (PA[i] * s_carry[cl * V + v] + PB[v]) + EB[v];
  }
  float part[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tau = tau0 + u;
    const int t = BWD ? L - 1 - tau : tau;
    const bool ok = cv && tau < L;
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = v_[u][v] + cm[u][AMODE == 1 ? v : 0] * Y[v];
    if (ok) stv<V>(y + (row0 + t) * d + c, o);
    if constexpr (BWD) {
      if (AMODE == 1) {
        if (ok) {
          float cur[V];
          ldv<V>(da + (row0 + t) * groups + c, cur);
#pragma unroll
          for (int v = 0; v < V; ++v) cur[v] += o[v] * hp[u][v];
          stv<V>(da + (row0 + t) * groups + c, cur);
        }
      } else {
        float p = 0.f;
#pragma unroll
        for (int v = 0; v < V; ++v) p += o[v] * hp[u][v];  // hp is zero where !ok
        part[u] = p;
      }
      if (ok && t == 0 && dhin) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float a0 = AMODE == 1 ? a[row0 * groups + c + v] : a[row0 * groups + c / gs];
          dhin[(int64_t)bb * d + c + v] = a0 * o[v];
        }
      }
    }
  }
  if constexpr (BWD && AMODE == 0) {
    // da: sum over the lanes of one decay group inside each token group, one atomic each
    if (lg_log2 == 6) {
      static_assert(U == 16, "butterfly over 16 steps");
      int u;
      const float s = wave_sum16(part, lane, u);
      const int tau = tau0 + u;  // tgw == 0: one token group per wave
      if ((lane & 3) == 0 && tau < L && cv)
        atomicAdd(da + (row0 + (L - 1 - tau)) * groups + c / gs, s);
    } else {
      for (int m = 1; m < (1 << (lg_log2 < 0 ? 0 : lg_log2)); m <<= 1) {
#pragma unroll
        for (int u = 0; u < U; ++u) part[u] += __shfl_xor(part[u], m, 64);
      }
      const int lgm = lg_log2 < 0 ? 0 : (1 << lg_log2) - 1;
      if ((cl & lgm) == 0 && cv) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int tau = tau0 + u;
          if (tau < L) atomicAdd(da + (row0 + (L - 1 - tau)) * groups + c / gs, part[u]);
        }
      }
    }
  }
}

// cs[r, b, 0/1, c] = the fold of shard r's chunk pairs (shards aligned to chunks).
__global__ void linear_scan_chunk_state_kernel(const uint64_t* __restrict__ words,
                                               float* __restrict__ cs, int batch, int d,
                                               int ntiles, int nchunks, int CT, int world,
                                               int per_shard) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= (int64_t)world * batch * d) return;
  const int c = (int)(i % d);
  const int bb = (int)((i / d) % batch);
  const int r = (int)(i / ((int64_t)d * batch));
  const int64_t chain = (int64_t)bb * ntiles + c / CT;
  float A = 1.f, B = 0.f;
  for (int k = r * per_shard; k < (r + 1) * per_shard; ++k) {
    const uint64_t* wk = words + ((chain * nchunks + k) * 3) * CT + c % CT;
    const float Ak = word_val(wk[kWordA * CT]), Bk = word_val(wk[kWordB * CT]);
    B = Ak * B + Bk;
    A *= Ak;
  }
  float* cp = cs + ((int64_t)(r * batch + bb) * 2) * d + c;
  cp[0] = A;
  cp[d] = B;
}

// Reduce-then-rescan fold: each channel's chain of chunk pairs in scan order, the state
// after chunk k published for chunk k + 1, S_{-1} = h_in (forward) or 0 (backward). A
// workgroup takes kFoldCh channels of one chain and cuts the chain into kFoldSegs
// segments; lane (s, ch) of wave w owns channel ch of segment 4 w + s, so a pair load is
// four 128-byte rows of the words. Each lane composes its segment's pairs (kFoldBatch
// loads in flight), the segments' maps meet in LDS, and each lane rescans its segment
// from the state entering it: two load round trips per kFoldBatch chunks of a segment.
constexpr int kFoldWaves = 16, kFoldSub = 4, kFoldCh = 64 / kFoldSub;
constexpr int kFoldSegs = kFoldWaves * kFoldSub, kFoldBatch = 16;

__global__ __launch_bounds__(64 * kFoldWaves) void linear_scan_chain_fold_kernel(
    uint64_t* __restrict__ words, const float* __restrict__ hin, int batch, int d, int ntiles,
    int nchunks, int CT) {
  __shared__ float s_a[kFoldSegs][kFoldCh], s_b[kFoldSegs][kFoldCh];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ch = lane % kFoldCh, g = w * kFoldSub + lane / kFoldCh;  // channel, segment
  const int ngrp = (CT + kFoldCh - 1) / kFoldCh;
  const int64_t chain = blockIdx.x / ngrp;
  const int cc = kFoldCh * (int)(blockIdx.x % ngrp) + ch;
  const int bb = (int)(chain / ntiles), tile = (int)(chain % ntiles);
  const int c = tile * CT + cc;
  const bool on = cc < CT && c < d;
  const int seg = (nchunks + kFoldSegs - 1) / kFoldSegs;
  const int k_lo = g * seg < nchunks ? g * seg : nchunks;
  const int k_hi = k_lo + seg < nchunks ? k_lo + seg : nchunks;
  uint64_t* w0 = words + (chain * nchunks * 3) * CT + (on ? cc : 0);
  auto load = [&](int k, float* A, float* B) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kFoldBatch; ++j) {
      const bool in = on && k + j < k_hi;
      const uint64_t* wk = w0 + (int64_t)(in ? k + j : 0) * 3 * CT;
      A[j] = in ? word_val(wk[kWordA * CT]) : 1.f;
      B[j] = in ? word_val(wk[kWordB * CT]) : 0.f;
    }
  };
  float PA = 1.f, PB = 0.f;  // the segment composed: x -> PA x + PB
  for (int k = k_lo; k < k_hi; k += kFoldBatch) {
    float A[kFoldBatch], B[kFoldBatch];
    load(k, A, B);
#pragma unroll
    for (int j = 0; j < kFoldBatch; ++j) {
      PB = __builtin_fmaf(A[j], PB, B[j]);
      PA *= A[j];
    }
  }
  s_a[g][ch] = PA;
  s_b[g][ch] = PB;
  __syncthreads();
  float S = on && hin ? hin[(int64_t)bb * d + c] : 0.f;
  for (int v = 0; v < g; ++v) S = __builtin_fmaf(s_a[v][ch], S, s_b[v][ch]);
  for (int k = k_lo; k < k_hi; k += kFoldBatch) {
    float A[kFoldBatch], B[kFoldBatch];
    load(k, A, B);
#pragma unroll
    for (int j = 0; j < kFoldBatch; ++j) {
      S = __builtin_fmaf(A[j], S, B[j]);
      if (on && k + j < k_hi) put_word(w0 + (int64_t)(k + j) * 3 * CT + kWordS * CT, S);
    }
  }
}

__global__ void fill_zero_u32x4_kernel(u32x4* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

ScanChunkPlan scan_chunk_plan(int batch, int L, int d, int groups) {
  ScanChunkPlan p{};
  const int gs = d / groups;
  int V = 1;
  for (int cand : {4, 2}) {
    if (d % cand == 0 && (gs % cand == 0 || gs == 1)) {
      V = cand;
      break;
    }
  }
  p.V = V;
  p.amode = gs % V == 0 ? 0 : 1;
  int cw = 1, cw_log2 = 0;
  while (cw < 64 && cw * V < d) {
    cw <<= 1;
    ++cw_log2;
  }
  p.cw_log2 = cw_log2;
  p.CT = cw * V;
  p.TC = kWaves * (64 / cw) * kU;
  p.ntiles = (d + p.CT - 1) / p.CT;
  p.nchunks = (L + p.TC - 1) / p.TC;
  // lanes of one token group that share a decay group: a power of two of them
  // (aligned, since groups start at multiples of gs) is reduced by shuffles
  const int lanes_per_group = p.amode == 0 ? gs / V : 1;
  const int lg = lanes_per_group >= cw ? cw : lanes_per_group;
  p.lg_log2 = -1;
  if (lg > 1 && (lg & (lg - 1)) == 0 && (lanes_per_group % lg == 0)) p.lg_log2 = __builtin_ctz(lg);
  const int64_t slots = (int64_t)batch * p.ntiles * p.nchunks;
  // Measured costs: the single pass takes its traffic plus about 200 ns per chunk of the
  // chain (each chunk waits for its predecessor's published state); reduce-then-rescan
  // reads the inputs twice (1.5x the forward's 8 bytes per element, at about 4.67 TB/s:
  // elems / 584 ns) plus about 20 us of fold and launches. Two passes when
  // 200 ns * nchunks > elems / 1168 ns + 20 us (both sides times 1168 below): few
  // channels over long sequences.
  const int64_t elems = (int64_t)batch * L * d;
  p.two_pass = (int64_t)p.nchunks * 233600 > elems + (int64_t)20000 * 1168;
  p.words_off = 256;  // the ticket counter and the failure word, then the words
  p.bytes = p.words_off + (size_t)slots * 3 * p.CT * 8;
  return p;
}

static ChunkWork carve(const ScanChunkPlan& p, void* ws) {
  uint8_t* base = reinterpret_cast<uint8_t*>(ws);
  return ChunkWork{reinterpret_cast<int*>(base), reinterpret_cast<uint64_t*>(base + p.words_off),
                   p.ntiles, p.nchunks};
}

template <bool BWD, int PASS>
static void launch_pass(const ScanChunkPlan& p, const float* a, const float* x, const float* hin,
                        const float* hfwd, float* y, float* da, float* dhin, const ChunkWork& w,
                        int batch, int L, int d, int groups, hipStream_t stream) {
  const unsigned grid = (unsigned)((int64_t)batch * p.ntiles * p.nchunks);
#define RMX_CHUNKED(AM, VV)                                                                      \
  hipLaunchKernelGGL((linear_scan_chunked_kernel<AM, VV, BWD, PASS>), dim3(grid), dim3(64 * kWaves), 0, \
                     stream, a, x, hin, hfwd, y, da, dhin, w, batch, L, d, groups, p.cw_log2,     \
                     p.lg_log2)
  if (p.amode == 1) {
    if (p.V == 4) RMX_CHUNKED(1, 4);
    else RMX_CHUNKED(1, 2);
  } else {
    if (p.V == 4) RMX_CHUNKED(0, 4);
    else if (p.V == 2) RMX_CHUNKED(0, 2);
    else RMX_CHUNKED(0, 1);
  }
#undef RMX_CHUNKED
}

template <bool BWD>
static hipError_t launch_chunked(const ScanChunkPlan& p, const float* a, const float* x,
                                 const float* hin, const float* hfwd, float* y, float* da,
                                 float* dhin, void* ws, int batch, int L, int d, int groups,
                                 hipStream_t stream) {
  const ChunkWork w = carve(p, ws);
  if (!p.two_pass) {
    // the ticket counter and the tags of every word start at zero (reduce-then-rescan
    // writes every word it reads first and takes no tickets)
    const int64_t n16 = (int64_t)(p.bytes / 16);
    hipLaunchKernelGGL(fill_zero_u32x4_kernel,
                       dim3((unsigned)std::min<int64_t>((n16 + 255) / 256, 2048)), dim3(256), 0,
                       stream, reinterpret_cast<u32x4*>(ws), n16);
    launch_pass<BWD, 0>(p, a, x, hin, hfwd, y, da, dhin, w, batch, L, d, groups, stream);
    return hipGetLastError();
  }
  launch_pass<BWD, 1>(p, a, x, hin, hfwd, y, da, dhin, w, batch, L, d, groups, stream);
  const int64_t nf = (int64_t)batch * p.ntiles * ((p.CT + kFoldCh - 1) / kFoldCh);
  hipLaunchKernelGGL(linear_scan_chain_fold_kernel, dim3((unsigned)nf), dim3(64 * kFoldWaves),
                     0, stream, w.words, BWD ? nullptr : hin, batch, d, p.ntiles, p.nchunks, p.CT);
  launch_pass<BWD, 2>(p, a, x, hin, hfwd, y, da, dhin, w, batch, L, d, groups, stream);
  return hipGetLastError();
}

hipError_t launch_linear_scan_fwd_chunked(const ScanChunkPlan& p, const float* a, const float* b,
                                          const float* hin, float* h, float* cs, void* ws,
                                          int batch, int L, int d, int groups, int world,
                                          hipStream_t stream) {
  hipError_t e = launch_chunked<false>(p, a, b, hin, nullptr, h, nullptr, nullptr, ws, batch, L,
                                       d, groups, stream);
  if (e != hipSuccess || !cs) return e;
  const ChunkWork w = carve(p, ws);
  const int64_t n = (int64_t)world * batch * d;
  hipLaunchKernelGGL(linear_scan_chunk_state_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, stream, w.words, cs, batch, d, p.ntiles, p.nchunks, p.CT, world,
                     (L / world) / p.TC);
  return hipGetLastError();
}

int read_linear_scan_failure(const void* ws, hipStream_t stream, hipError_t* err) {
  int flag = 0;
  *err = hipMemcpyAsync(&flag, reinterpret_cast<const int*>(ws) + 1, sizeof(int),
                        hipMemcpyDeviceToHost, stream);
  if (*err == hipSuccess) *err = hipStreamSynchronize(stream);
  return flag;
}

hipError_t launch_linear_scan_bwd_chunked(const ScanChunkPlan& p, const float* a, const float* h,
                                          const float* hin, const float* dh, float* da, float* db,
                                          float* dhin, void* ws, int batch, int L, int d,
                                          int groups, hipStream_t stream) {
  return launch_chunked<true>(p, a, dh, hin, h, db, da, dhin, ws, batch, L, d, groups, stream);
}

}  // namespace rmx
