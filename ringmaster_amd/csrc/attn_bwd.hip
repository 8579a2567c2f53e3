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
#include "rmx_kernels.h"
#include "tile_io.h"

namespace rmx {

struct BwdParams {
  rmx_attn_layout L;
  rmx_bwd_problem P[RMX_MAX_BATCHED];
  int tile_start[RMX_MAX_BATCHED + 1];
  int tiles[RMX_MAX_BATCHED];
  int nprob;
  int total;
  float scale_log2;
};

// ---------------------------------------------------------------- delta
// delta = rowsum(dout * out). `out` is the bf16 output (o_* strides) or, when
// OUT_F32, the fp32 merged output (a_* strides): the fp32 form keeps the bf16
// rounding of out (up to |dout|*|out|*2^-9 per element) out of dS = P (dP - delta).
template <int HD, bool OUT_F32>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const rmx_attn_layout L,
                                                             const void* __restrict__ out,
                                                             const uint16_t* __restrict__ dout,
                                                             float* __restrict__ delta, int sq) {
  constexpr int TPR = HD / 8;  // threads per row
  const int rows = L.batch * sq * L.hq;
  const int row = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int part = threadIdx.x % TPR;
  float acc = 0.f;
  int bb = 0, q = 0, h = 0;
  if (row < rows) {
    h = row % L.hq;
    q = (row / L.hq) % sq;
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
        o[2 * i] = __uint_as_float(a[i] << 16);
        o[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc += o[2 * i] * __uint_as_float(b[i] << 16);
      acc += o[2 * i + 1] * __uint_as_float(b[i] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < rows && part == 0) delta[bb * L.l_sb + h * L.l_sh + q] = acc;
}

template <int HD>
static void launch_delta_t(const rmx_attn_layout& L, const void* out, int out_f32,
                           const uint16_t* dout, float* delta, int sq, int64_t rows,
                           hipStream_t stream) {
  constexpr int RPB = 256 / (HD / 8);  // rows per block
  const int grid = (int)((rows + RPB - 1) / RPB);
  if (out_f32)
    hipLaunchKernelGGL((attn_bwd_delta_kernel<HD, true>), dim3(grid), dim3(256), 0, stream, L, out,
                       dout, delta, sq);
  else
    hipLaunchKernelGGL((attn_bwd_delta_kernel<HD, false>), dim3(grid), dim3(256), 0, stream, L,
                       out, dout, delta, sq);
}

hipError_t launch_attn_bwd_delta(const rmx_attn_layout& L, const void* out, int out_f32,
                                 const uint16_t* dout, float* delta, int sq, hipStream_t stream) {
  const int64_t rows = (int64_t)L.batch * sq * L.hq;
  if (rows == 0) return hipSuccess;
  if (L.head_dim == 128)
    launch_delta_t<128>(L, out, out_f32, dout, delta, sq, rows, stream);
  else
    launch_delta_t<64>(L, out, out_f32, dout, delta, sq, rows, stream);
  return hipGetLastError();
}

// ---------------------------------------------------------------- shared helpers
// Per-problem decode of the linear workgroup index.
__device__ __forceinline__ int find_problem(const BwdParams& prm, int id) {
  int p = 0;
  while (p + 1 < prm.nprob && id >= prm.tile_start[p + 1]) ++p;
  return p;
}

// Write a 4-float run of a gradient row according to the output mode.
__device__ __forceinline__ void grad_store4(int mode, float* acc, uint16_t* bf, f32x4 v) {
  if (mode == RMX_GRAD_WRITE_F32) {
    *reinterpret_cast<f32x4*>(acc) = v;
  } else if (mode == RMX_GRAD_ACC_F32) {
    *reinterpret_cast<f32x4*>(acc) = *reinterpret_cast<const f32x4*>(acc) + v;
  } else {
    if (mode == RMX_GRAD_ACC_FINAL) v += *reinterpret_cast<const f32x4*>(acc);
    u32x2 w;
    w[0] = pack_bf2(v[0], v[1]);
    w[1] = pack_bf2(v[2], v[3]);
    *reinterpret_cast<u32x2*>(bf) = w;
  }
}

// ---------------------------------------------------------------- dQ (Q-major)
template <int HD, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_bwd_dq_kernel(const BwdParams prm) {
  constexpr int BK = 64;
  constexpr int BQ = 32 * NW;
  constexpr int NKB = HD / 16;
  constexpr int NDB = HD / 32;
  constexpr int NT = NW * 64;

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BK * HD];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][BK * HD];
  __shared__ __attribute__((aligned(16))) uint16_t sKt[2][HD * BK];
  __shared__ int sKg[2][BK];
  __shared__ int sKd[2][BK];
  __shared__ int sRange[2];

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  if (id >= prm.total) return;
  const int p = find_problem(prm, id);
  const rmx_attn_layout& L = prm.L;
  const rmx_bwd_problem& P = prm.P[p];
  const int local = id - prm.tile_start[p];
  const int nqt = prm.tiles[p];
  const int qt = nqt - 1 - (local % nqt);
  const int head = (local / nqt) % L.hq;
  const int bb = local / (nqt * L.hq);
  const int kvh = head / (L.hq / L.hkv);
  const int sq = P.sq, sk = P.sk;
  const int mask = L.mask;
  const int q0 = qt * BQ;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int q = q0 + wave * 32 + l32;
  const bool qvalid = q < sq;

  bf16x8 qreg[NKB], doreg[NKB];
  {
    const int qq = qvalid ? q : 0;
    const uint16_t* qp = P.q + bb * L.q_sb + (int64_t)qq * L.q_ss + head * L.q_sh + 8 * hl;
    const uint16_t* dp = P.dout + bb * L.o_sb + (int64_t)qq * L.o_ss + head * L.o_sh + 8 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      qreg[kb] = qvalid ? __builtin_bit_cast(bf16x8, ld16(qp + 16 * kb)) : zero_bf16x8();
      doreg[kb] = qvalid ? __builtin_bit_cast(bf16x8, ld16(dp + 16 * kb)) : zero_bf16x8();
    }
  }
  const int64_t lrow = bb * L.l_sb + head * L.l_sh + (qvalid ? q : 0);
  float lse2 = qvalid ? P.lse[lrow] * kLog2e : kNegInf;
  if (lse2 == kNegInf) lse2 = __builtin_inff();  // no key attended: P == 0 everywhere
  const float dlt = qvalid ? P.delta[lrow] : 0.f;
  int qg = -2147483647, qd = -1;
  if (mask == RMX_MASK_DOC && qvalid) {
    qg = P.q_gidx[q];
    qd = P.doc[qg];
  }

  const int off = sk - sq;
  const int qlast = (q0 + BQ < sq ? q0 + BQ : sq) - 1;
  const int nkt = (sk + BK - 1) / BK;
  int kt_begin = 0, kt_end = nkt;
  int qg_first = 0, qg_last = 0, qd_first = 0, qd_last = 0;
  if (mask == RMX_MASK_CAUSAL) {
    const int kmax = qlast + off;
    kt_end = kmax < 0 ? 0 : (kmax / BK + 1 < nkt ? kmax / BK + 1 : nkt);
  } else if (mask == RMX_MASK_DOC) {
    qg_first = P.q_gidx[q0];
    qg_last = P.q_gidx[qlast];
    qd_first = P.doc[qg_first];
    qd_last = P.doc[qg_last];
    if (tid == 0) {
      sRange[0] = nkt;
      sRange[1] = -1;
    }
    __syncthreads();
    int lo = nkt, hi = -1;
    for (int t = tid; t < nkt; t += NT) {
      const int ka = t * BK, kb = (t * BK + BK < sk ? t * BK + BK : sk) - 1;
      const int kga = P.k_gidx[ka], kgb = P.k_gidx[kb];
      const int kda = P.doc[kga], kdb = P.doc[kgb];
      if (kga <= qg_last && kdb >= qd_first && kda <= qd_last) {
        lo = t < lo ? t : lo;
        hi = t > hi ? t : hi;
      }
    }
    if (lo < nkt) atomicMin(&sRange[0], lo);
    if (hi >= 0) atomicMax(&sRange[1], hi);
    __syncthreads();
    kt_begin = sRange[0];
    kt_end = sRange[1] + 1;
    if (kt_end < kt_begin) kt_end = kt_begin;
  }

  const uint16_t* kbase = P.k + bb * L.k_sb + kvh * L.k_sh;
  const uint16_t* vbase = P.v + bb * L.v_sb + kvh * L.v_sh;

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

  TileIO<HD, NT> tk, tv;
  if (kt_begin < kt_end) {
    const int k0 = kt_begin * BK;
    tk.load(kbase + (int64_t)k0 * L.k_ss, L.k_ss, sk - k0, tid);
    tv.load(vbase + (int64_t)k0 * L.v_ss, L.v_ss, sk - k0, tid);
    tk.store_rows(sK[0], tid);
    tk.store_t(sKt[0], tid);
    tv.store_rows(sV[0], tid);
    if (mask == RMX_MASK_DOC && tid < BK) {
      const int kk = k0 + tid < sk ? k0 + tid : sk - 1;
      const int g = P.k_gidx[kk];
      sKg[0][tid] = g;
      sKd[0][tid] = P.doc[g];
    }
  }
  __syncthreads();

  const float c = prm.scale_log2;
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int buf = (kt - kt_begin) & 1;
    const int k0 = kt * BK;
    const bool has_next = kt + 1 < kt_end;
    int nkg = 0, nkd = 0;
    if (has_next) {
      const int k1 = k0 + BK;
      tk.load(kbase + (int64_t)k1 * L.k_ss, L.k_ss, sk - k1, tid);
      tv.load(vbase + (int64_t)k1 * L.v_ss, L.v_ss, sk - k1, tid);
      if (mask == RMX_MASK_DOC && tid < BK) {
        const int kk = k1 + tid < sk ? k1 + tid : sk - 1;
        nkg = P.k_gidx[kk];
        nkd = P.doc[nkg];
      }
    }

    f32x16 s[2], dp[2];
    s[0] = zero16();
    s[1] = zero16();
    dp[0] = zero16();
    dp[1] = zero16();
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = sigma(l32) + 32 * mb;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const bf16x8 a = lds_row_operand(sK[buf], HD, row, 2 * kb + hl);
        s[mb] = mfma32(a, qreg[kb], s[mb]);
        const bf16x8 b = lds_row_operand(sV[buf], HD, row, 2 * kb + hl);
        dp[mb] = mfma32(b, doreg[kb], dp[mb]);
      }
    }

    bool need_mask = (k0 + BK > sk);
    if (mask == RMX_MASK_CAUSAL) need_mask |= (k0 + BK - 1 > q0 + off);
    if (mask == RMX_MASK_DOC) {
      const int kgb = sKg[buf][BK - 1];
      const int kda = sKd[buf][0], kdb = sKd[buf][BK - 1];
      need_mask |= !(kda == kdb && kda == qd_first && qd_first == qd_last && kgb <= qg_first);
    }

    bf16x8 dsb[4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(fmaf(s[mb][r], c, -lse2));
        if (need_mask) {
          const int kl = 32 * mb + sig_row(hl, r);
          const int key = k0 + kl;
          bool ok = key < sk;
          if (mask == RMX_MASK_CAUSAL) ok = ok && (key <= q + off);
          if (mask == RMX_MASK_DOC) ok = ok && (sKd[buf][kl] == qd) && (sKg[buf][kl] <= qg);
          if (!ok) pv = 0.f;
        }
        s[mb][r] = pv * (dp[mb][r] - dlt);
      }
    }
#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      const f32x16& t = s[kb2 >> 1];
      const int b8 = 8 * (kb2 & 1);
      dsb[kb2] = pack8(t[b8 + 0], t[b8 + 1], t[b8 + 2], t[b8 + 3], t[b8 + 4], t[b8 + 5], t[b8 + 6],
                       t[b8 + 7]);
    }

    // dQ^T += K^T dS^T
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const bf16x8 a = lds_t_operand(sKt[buf], d, 2 * kb2 + hl);
        acc[db] = mfma32(a, dsb[kb2], acc[db]);
      }
    }

    if (has_next) {
      tk.store_rows(sK[buf ^ 1], tid);
      tk.store_t(sKt[buf ^ 1], tid);
      tv.store_rows(sV[buf ^ 1], tid);
      if (mask == RMX_MASK_DOC && tid < BK) {
        sKg[buf ^ 1][tid] = nkg;
        sKd[buf ^ 1][tid] = nkd;
      }
    }
    __syncthreads();
  }

  if (!qvalid) return;
  const float scale = L.scale;
  float* arow = P.dq_acc ? P.dq_acc + bb * L.a_sb + (int64_t)q * L.a_ss + head * L.a_sh : nullptr;
  uint16_t* brow = P.dq ? P.dq + bb * L.o_sb + (int64_t)q * L.o_ss + head * L.o_sh : nullptr;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = 32 * db + 8 * j + 4 * hl;
      f32x4 v;
      v[0] = acc[db][4 * j + 0] * scale;
      v[1] = acc[db][4 * j + 1] * scale;
      v[2] = acc[db][4 * j + 2] * scale;
      v[3] = acc[db][4 * j + 3] * scale;
      grad_store4(P.dq_mode, arow ? arow + d0 : nullptr, brow ? brow + d0 : nullptr, v);
    }
}

// ---------------------------------------------------------------- dK, dV (KV-major)
template <int HD, int NW>
__global__ __launch_bounds__(NW * 64, 1) void attn_bwd_dkdv_kernel(const BwdParams prm) {
  constexpr int BQ = 64;          // queries per q-tile
  constexpr int BKV = 32 * NW;    // keys per workgroup
  constexpr int NKB = HD / 16;
  constexpr int NDB = HD / 32;
  constexpr int NT = NW * 64;

  __shared__ __attribute__((aligned(16))) uint16_t sQ[2][BQ * HD];
  __shared__ __attribute__((aligned(16))) uint16_t sDO[2][BQ * HD];
  __shared__ __attribute__((aligned(16))) uint16_t sQt[2][HD * BQ];
  __shared__ __attribute__((aligned(16))) uint16_t sDOt[2][HD * BQ];
  __shared__ __attribute__((aligned(16))) float sL[2][BQ];
  __shared__ __attribute__((aligned(16))) float sD[2][BQ];
  __shared__ int sQg[2][BQ];
  __shared__ int sQd[2][BQ];
  __shared__ int sRange[2];

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  if (id >= prm.total) return;
  const int p = find_problem(prm, id);
  const rmx_attn_layout& L = prm.L;
  const rmx_bwd_problem& P = prm.P[p];
  const int local = id - prm.tile_start[p];
  const int nkt = prm.tiles[p];
  const int kt = local % nkt;
  const int kvh = (local / nkt) % L.hkv;
  const int bb = local / (nkt * L.hkv);
  const int G = L.hq / L.hkv;
  const int sq = P.sq, sk = P.sk;
  const int mask = L.mask;
  const int k0 = kt * BKV;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int key = k0 + wave * 32 + l32;
  const bool kvalid = key < sk;

  bf16x8 kreg[NKB], vreg[NKB];
  {
    const int kk = kvalid ? key : 0;
    const uint16_t* kp = P.k + bb * L.k_sb + (int64_t)kk * L.k_ss + kvh * L.k_sh + 8 * hl;
    const uint16_t* vp = P.v + bb * L.v_sb + (int64_t)kk * L.v_ss + kvh * L.v_sh + 8 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      kreg[kb] = kvalid ? __builtin_bit_cast(bf16x8, ld16(kp + 16 * kb)) : zero_bf16x8();
      vreg[kb] = kvalid ? __builtin_bit_cast(bf16x8, ld16(vp + 16 * kb)) : zero_bf16x8();
    }
  }
  int kg = 2147483647, kd = -2;
  if (mask == RMX_MASK_DOC && kvalid) {
    kg = P.k_gidx[key];
    kd = P.doc[kg];
  }

  // ---- q-tile range
  const int off = sk - sq;
  const int klast = (k0 + BKV < sk ? k0 + BKV : sk) - 1;
  const int nqt = (sq + BQ - 1) / BQ;
  int qt_begin = 0, qt_end = nqt;
  int kg_first = 0, kg_last = 0, kd_first = 0, kd_last = 0;
  if (mask == RMX_MASK_CAUSAL) {
    const int qmin = k0 - off;  // first query that sees key k0
    qt_begin = qmin <= 0 ? 0 : qmin / BQ;
    if (qt_begin > nqt) qt_begin = nqt;
  } else if (mask == RMX_MASK_DOC) {
    kg_first = P.k_gidx[k0];
    kg_last = P.k_gidx[klast];
    kd_first = P.doc[kg_first];
    kd_last = P.doc[kg_last];
    if (tid == 0) {
      sRange[0] = nqt;
      sRange[1] = -1;
    }
    __syncthreads();
    int lo = nqt, hi = -1;
    for (int t = tid; t < nqt; t += NT) {
      const int qa = t * BQ, qb = (t * BQ + BQ < sq ? t * BQ + BQ : sq) - 1;
      const int qga = P.q_gidx[qa], qgb = P.q_gidx[qb];
      const int qda = P.doc[qga], qdb = P.doc[qgb];
      if (qgb >= kg_first && qdb >= kd_first && qda <= kd_last) {
        lo = t < lo ? t : lo;
        hi = t > hi ? t : hi;
      }
    }
    if (lo < nqt) atomicMin(&sRange[0], lo);
    if (hi >= 0) atomicMax(&sRange[1], hi);
    __syncthreads();
    qt_begin = sRange[0];
    qt_end = sRange[1] + 1;
    if (qt_end < qt_begin) qt_end = qt_begin;
  }
  const int nq_iter = qt_end - qt_begin;
  const int total_iter = nq_iter * G;

  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }

  TileIO<HD, NT> tq, tdo;
  float nl = 0.f, nd = 0.f;
  int nqg = 0, nqd = 0;
  auto issue_load = [&](int it) {
    const int g = it / nq_iter;
    const int qtile = qt_begin + it % nq_iter;
    const int qh = kvh * G + g;
    const int qa = qtile * BQ;
    tq.load(P.q + bb * L.q_sb + qh * L.q_sh + (int64_t)qa * L.q_ss, L.q_ss, sq - qa, tid);
    tdo.load(P.dout + bb * L.o_sb + qh * L.o_sh + (int64_t)qa * L.o_ss, L.o_ss, sq - qa, tid);
    if (tid < BQ) {
      const int qq = qa + tid;
      if (qq < sq) {
        const int64_t lr = bb * L.l_sb + qh * L.l_sh + qq;
        nl = P.lse[lr] * kLog2e;
        if (nl == kNegInf) nl = __builtin_inff();
        nd = P.delta[lr];
        if (mask == RMX_MASK_DOC) {
          nqg = P.q_gidx[qq];
          nqd = P.doc[nqg];
        }
      } else {
        nl = __builtin_inff();
        nd = 0.f;
        nqg = -2147483647;
        nqd = -1;
      }
    }
  };
  auto commit = [&](int buf) {
    tq.store_rows(sQ[buf], tid);
    tq.store_t(sQt[buf], tid);
    tdo.store_rows(sDO[buf], tid);
    tdo.store_t(sDOt[buf], tid);
    if (tid < BQ) {
      sL[buf][tid] = nl;
      sD[buf][tid] = nd;
      sQg[buf][tid] = nqg;
      sQd[buf][tid] = nqd;
    }
  };

  if (total_iter > 0) {
    issue_load(0);
    commit(0);
  }
  __syncthreads();

  const float c = prm.scale_log2;
  for (int it = 0; it < total_iter; ++it) {
    const int buf = it & 1;
    const int qa = (qt_begin + it % nq_iter) * BQ;
    const bool has_next = it + 1 < total_iter;
    if (has_next) issue_load(it + 1);

    // S = Q K^T, dP = dO V^T  (rows = queries sigma-permuted, cols = this wave's keys)
    f32x16 s[2], dp[2];
    s[0] = zero16();
    s[1] = zero16();
    dp[0] = zero16();
    dp[1] = zero16();
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = sigma(l32) + 32 * mb;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const bf16x8 a = lds_row_operand(sQ[buf], HD, row, 2 * kb + hl);
        s[mb] = mfma32(a, kreg[kb], s[mb]);
        const bf16x8 b = lds_row_operand(sDO[buf], HD, row, 2 * kb + hl);
        dp[mb] = mfma32(b, vreg[kb], dp[mb]);
      }
    }

    bool need_mask = (qa + BQ > sq) || (k0 + BKV > sk);
    if (mask == RMX_MASK_CAUSAL) need_mask |= (klast > qa + off);
    if (mask == RMX_MASK_DOC) {
      const int qga = sQg[buf][0];
      const int qda = sQd[buf][0];
      const int qlast_row = (qa + BQ < sq ? BQ : sq - qa) - 1;
      const int qdb = sQd[buf][qlast_row];
      need_mask |= !(qda == qdb && qda == kd_first && kd_first == kd_last && kg_last <= qga);
    }

    bf16x8 pt[4], dst[4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      f32x4 lv[4], dv4[4];
#pragma unroll
      for (int h8 = 0; h8 < 2; ++h8) {
        const int qb = 32 * mb + 16 * h8 + 8 * hl;
        lv[2 * h8] = *reinterpret_cast<const f32x4*>(&sL[buf][qb]);
        lv[2 * h8 + 1] = *reinterpret_cast<const f32x4*>(&sL[buf][qb + 4]);
        dv4[2 * h8] = *reinterpret_cast<const f32x4*>(&sD[buf][qb]);
        dv4[2 * h8 + 1] = *reinterpret_cast<const f32x4*>(&sD[buf][qb + 4]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float l2 = lv[r >> 2][r & 3];
        const float dl = dv4[r >> 2][r & 3];
        float pv = fast_exp2(fmaf(s[mb][r], c, -l2));
        if (need_mask) {
          const int ql = 32 * mb + sig_row(hl, r);
          const int qq = qa + ql;
          bool ok = kvalid && qq < sq;
          if (mask == RMX_MASK_CAUSAL) ok = ok && (key <= qq + off);
          if (mask == RMX_MASK_DOC) ok = ok && (sQd[buf][ql] == kd) && (kg <= sQg[buf][ql]);
          if (!ok) pv = 0.f;
        }
        s[mb][r] = pv;
        dp[mb][r] = pv * (dp[mb][r] - dl);
      }
    }
#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      const int mb = kb2 >> 1, b8 = 8 * (kb2 & 1);
      const f32x16& t = s[mb];
      pt[kb2] = pack8(t[b8 + 0], t[b8 + 1], t[b8 + 2], t[b8 + 3], t[b8 + 4], t[b8 + 5], t[b8 + 6],
                      t[b8 + 7]);
      const f32x16& u = dp[mb];
      dst[kb2] = pack8(u[b8 + 0], u[b8 + 1], u[b8 + 2], u[b8 + 3], u[b8 + 4], u[b8 + 5], u[b8 + 6],
                       u[b8 + 7]);
    }

    // dV += P^T dO, dK += dS^T Q  (rows = this wave's keys, cols = head dim)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const bf16x8 bo = lds_t_operand(sDOt[buf], d, 2 * kb2 + hl);
        dv[db] = mfma32(pt[kb2], bo, dv[db]);
        const bf16x8 bq = lds_t_operand(sQt[buf], d, 2 * kb2 + hl);
        dk[db] = mfma32(dst[kb2], bq, dk[db]);
      }
    }

    if (has_next) commit(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane (hl, d) holds rows key = k0 + 32*wave + c_row(hl, r)
  const float scale = L.scale;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 32 * db + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = k0 + wave * 32 + c_row(hl, r);
      if (kk >= sk) continue;
      const float gk = dk[db][r] * scale, gv = dv[db][r];
      const int64_t ao = bb * L.ka_sb + (int64_t)kk * L.ka_ss + kvh * L.ka_sh + d;
      const int64_t bo = bb * L.dk_sb + (int64_t)kk * L.dk_ss + kvh * L.dk_sh + d;
      const int mode = P.dkv_mode;
      if (mode == RMX_GRAD_WRITE_F32) {
        P.dk_acc[ao] = gk;
        P.dv_acc[ao] = gv;
      } else if (mode == RMX_GRAD_ACC_F32) {
        P.dk_acc[ao] += gk;
        P.dv_acc[ao] += gv;
      } else if (mode == RMX_GRAD_ACC_FINAL) {
        P.dk[bo] = f2bf(P.dk_acc[ao] + gk);
        P.dv[bo] = f2bf(P.dv_acc[ao] + gv);
      } else {
        P.dk[bo] = f2bf(gk);
        P.dv[bo] = f2bf(gv);
      }
    }
  }
}

template <int HD>
static hipError_t launch_bwd_t(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                               hipStream_t stream) {
  constexpr int NW_DQ = 4, NW_KV = 4;
  BwdParams pq, pk;
  pq.L = L;
  pk.L = L;
  pq.scale_log2 = pk.scale_log2 = L.scale * kLog2e;
  // problems with an empty side or a skipped gradient get no workgroups there
  int tq = 0, tk = 0, nq = 0, nk = 0;
  for (int i = 0; i < n; ++i) {
    const bool empty = probs[i].sq == 0 || probs[i].sk == 0;
    if (!empty && probs[i].dq_mode != RMX_GRAD_NONE) {
      pq.P[nq] = probs[i];
      pq.tiles[nq] = (probs[i].sq + 32 * NW_DQ - 1) / (32 * NW_DQ);
      pq.tile_start[nq] = tq;
      tq += L.batch * L.hq * pq.tiles[nq];
      ++nq;
    }
    if (!empty && probs[i].dkv_mode != RMX_GRAD_NONE) {
      pk.P[nk] = probs[i];
      pk.tiles[nk] = (probs[i].sk + 32 * NW_KV - 1) / (32 * NW_KV);
      pk.tile_start[nk] = tk;
      tk += L.batch * L.hkv * pk.tiles[nk];
      ++nk;
    }
  }
  for (int i = nq; i <= RMX_MAX_BATCHED; ++i) pq.tile_start[i] = tq;
  for (int i = nk; i <= RMX_MAX_BATCHED; ++i) pk.tile_start[i] = tk;
  pq.nprob = nq;
  pk.nprob = nk;
  pq.total = tq;
  pk.total = tk;
  if (tk > 0) {
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, NW_KV>), dim3((tk + 7) / 8 * 8), dim3(NW_KV * 64),
                       0, stream, pk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (tq > 0) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, NW_DQ>), dim3((tq + 7) / 8 * 8), dim3(NW_DQ * 64), 0,
                       stream, pq);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_attn_bwd(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                           hipStream_t stream) {
  if (L.head_dim == 128) return launch_bwd_t<128>(L, probs, n, stream);
  return launch_bwd_t<64>(L, probs, n, stream);
}

}  // namespace rmx
