// Block-attention forward for gfx950 with the online-softmax merge fused into
// the epilogue.
//
// Reference semantics: `math_block` (ring/kernels.py:52-78) for the block
// (out, lse), bottom-right causal (:64-67), document masks
// (ring/varlen_blocks.py:51-58,69-80, -inf lse for rows with no key), and the
// merge `update_out_and_lse` / `_merge_full` / `_merge_slice`
// (ring/merge.py:20-31, ring/zigzag.py:49-67).
//
// Formulation (per wave, 32*NB queries):
//   S^T = K Q^T   (A = K rows from LDS, sigma-permuted; B = Q held in VGPRs)
//   online softmax per lane (each lane owns one query column, the two lane
//   halves split the keys; one cross-half max per tile)
//   O^T += V^T P^T  (A = V^T from a transposed LDS tile, B = P straight from
//   the S^T accumulator registers, converted to bf16)
// so every row statistic is lane-local and P never touches LDS.
#include "rmx_kernels.h"
#include "tile_io.h"

namespace rmx {

struct FwdParams {
  rmx_attn_layout L;
  rmx_fwd_problem P[RMX_MAX_BATCHED];
  int tile_start[RMX_MAX_BATCHED + 1];
  int qtiles[RMX_MAX_BATCHED];
  int nprob;
  int total;
  float scale_log2;
};

template <int HD, int NW, int NB>
__global__ __launch_bounds__(NW * 64, 1) void attn_fwd_kernel(const FwdParams prm) {
  constexpr int BK = 64;
  constexpr int QW = 32 * NB;
  constexpr int BQ = QW * NW;
  constexpr int NKB = HD / 16;
  constexpr int NDB = HD / 32;
  constexpr int NT = NW * 64;

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BK * HD];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][HD * BK];
  __shared__ int sKg[2][BK];
  __shared__ int sKd[2][BK];
  __shared__ int sRange[2];

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  if (id >= prm.total) return;
  int p = 0;
  while (p + 1 < prm.nprob && id >= prm.tile_start[p + 1]) ++p;
  const rmx_attn_layout& L = prm.L;
  const rmx_fwd_problem& P = prm.P[p];
  const int local = id - prm.tile_start[p];
  const int nqt = prm.qtiles[p];
  const int qt = nqt - 1 - (local % nqt);  // heaviest causal tiles first
  const int head = (local / nqt) % L.hq;
  const int bb = local / (nqt * L.hq);
  const int kvh = head / (L.hq / L.hkv);
  const int sq = P.sq, sk = P.sk;
  const int mask = L.mask;
  const int q0 = qt * BQ;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[q][16kb + 8hl .. +7]
  bf16x8 qreg[NB][NKB];
  int qg[NB], qd[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int q = q0 + wave * QW + nb * 32 + l32;
    const uint16_t* qp = P.q + bb * L.q_sb + (int64_t)(q < sq ? q : 0) * L.q_ss + head * L.q_sh + 8 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      qreg[nb][kb] = q < sq ? __builtin_bit_cast(bf16x8, ld16(qp + 16 * kb)) : zero_bf16x8();
    qg[nb] = -2147483647;
    qd[nb] = -1;
    if (mask == RMX_MASK_DOC && q < sq) {
      qg[nb] = P.q_gidx[q];
      qd[nb] = P.doc[qg[nb]];
    }
  }

  // ---- key tile range
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

  f32x16 o[NB][NDB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[nb][db] = zero16();
  float m_run[NB], l_run[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = kNegInf;
    l_run[nb] = 0.f;
  }

  TileIO<HD, NT> tk, tv;
  if (kt_begin < kt_end) {
    const int k0 = kt_begin * BK;
    tk.load(kbase + (int64_t)k0 * L.k_ss, L.k_ss, sk - k0, tid);
    tv.load(vbase + (int64_t)k0 * L.v_ss, L.v_ss, sk - k0, tid);
    tk.store_rows(sK[0], tid);
    tv.store_t(sV[0], tid);
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

    // ---- S^T = K Q^T
    f32x16 s[NB][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      s[nb][0] = zero16();
      s[nb][1] = zero16();
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = sigma(l32) + 32 * mb;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const bf16x8 a = lds_row_operand(sK[buf], HD, row, 2 * kb + hl);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb][mb] = mfma32(a, qreg[nb][kb], s[nb][mb]);
      }
    }

    // ---- masking (only on tiles that need it)
    bool need_mask = (k0 + BK > sk);
    if (mask == RMX_MASK_CAUSAL) need_mask |= (k0 + BK - 1 > q0 + off);
    if (mask == RMX_MASK_DOC) {
      const int kga = sKg[buf][0], kgb = sKg[buf][BK - 1];
      const int kda = sKd[buf][0], kdb = sKd[buf][BK - 1];
      need_mask |= !(kda == kdb && kda == qd_first && qd_first == qd_last && kgb <= qg_first);
      (void)kga;
    }
    if (need_mask) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int q = q0 + wave * QW + nb * 32 + l32;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kl = 32 * mb + sig_row(hl, r);
            const int key = k0 + kl;
            bool ok = key < sk;
            if (mask == RMX_MASK_CAUSAL) ok = ok && (key <= q + off);
            if (mask == RMX_MASK_DOC) ok = ok && (sKd[buf][kl] == qd[nb]) && (sKg[buf][kl] <= qg[nb]);
            if (!ok) s[nb][mb][r] = kNegInf;
          }
      }
    }

    // ---- online softmax (log2 domain, scale folded into the exponent FMA)
    bf16x8 pb[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float mx = kNegInf;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[nb][mb][r]);
      mx = fmaxf(mx, xhalf(mx)) * c;
      const float mnew = fmaxf(m_run[nb], mx);
      const float mbase = (mnew == kNegInf) ? 0.f : mnew;
      const float alpha = fast_exp2(m_run[nb] - mbase);
      float rs = 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp2(fmaf(s[nb][mb][r], c, -mbase));
          s[nb][mb][r] = pv;
          rs += pv;
        }
      l_run[nb] = l_run[nb] * alpha + rs;
      m_run[nb] = mnew;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[nb][db] *= alpha;
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const f32x16& t = s[nb][kb2 >> 1];
        const int b8 = 8 * (kb2 & 1);
        pb[nb][kb2] = pack8(t[b8 + 0], t[b8 + 1], t[b8 + 2], t[b8 + 3], t[b8 + 4], t[b8 + 5],
                            t[b8 + 6], t[b8 + 7]);
      }
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const bf16x8 a = lds_t_operand(sV[buf], d, 2 * kb2 + hl);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[nb][db] = mfma32(a, pb[nb][kb2], o[nb][db]);
      }
    }

    if (has_next) {
      tk.store_rows(sK[buf ^ 1], tid);
      tv.store_t(sV[buf ^ 1], tid);
      if (mask == RMX_MASK_DOC && tid < BK) {
        sKg[buf ^ 1][tid] = nkg;
        sKd[buf ^ 1][tid] = nkd;
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise, lse, merge
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float lt = l_run[nb] + xhalf(l_run[nb]);
    const int q = q0 + wave * QW + nb * 32 + l32;
    if (q >= sq) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float lse_b = lt > 0.f ? (m_run[nb] + fast_log2(lt)) * kLn2 : kNegInf;
    const int64_t lrow = bb * L.l_sb + head * L.l_sh + q;
    float wa = 0.f, wb = 1.f, lnew = lse_b;
    if (P.mode == RMX_FWD_ACC_MERGE || P.mode == RMX_FWD_ACC_FINAL) {
      const float la = P.acc_lse[lrow];
      const float mx = fmaxf(la, lse_b);
      if (mx == kNegInf) {
        lnew = kNegInf;
        wa = 0.f;
        wb = 0.f;
      } else {
        const float mn = fminf(la, lse_b);
        lnew = mx + fast_log2(1.f + fast_exp2((mn - mx) * kLog2e)) * kLn2;
        wa = fast_exp2((la - lnew) * kLog2e);
        wb = fast_exp2((lse_b - lnew) * kLog2e);
      }
    }
    wb *= inv;
    float* accrow = P.acc_out ? P.acc_out + bb * L.a_sb + (int64_t)q * L.a_ss + head * L.a_sh : nullptr;
    uint16_t* orow = P.out ? P.out + bb * L.o_sb + (int64_t)q * L.o_ss + head * L.o_sh : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * db + 8 * j + 4 * hl;
        f32x4 v;
        v[0] = o[nb][db][4 * j + 0] * wb;
        v[1] = o[nb][db][4 * j + 1] * wb;
        v[2] = o[nb][db][4 * j + 2] * wb;
        v[3] = o[nb][db][4 * j + 3] * wb;
        if (P.mode == RMX_FWD_ACC_MERGE || P.mode == RMX_FWD_ACC_FINAL) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(accrow + d0);
          v += a * wa;
        }
        // every mode leaves the fp32 result in acc_out when it is given (WRITE and
        // ACC_FINAL: the final out in fp32, which the backward's delta reads)
        if (accrow) *reinterpret_cast<f32x4*>(accrow + d0) = v;
        if (P.mode == RMX_FWD_WRITE || P.mode == RMX_FWD_ACC_FINAL) {
          u32x2 w;
          w[0] = pack_bf2(v[0], v[1]);
          w[1] = pack_bf2(v[2], v[3]);
          *reinterpret_cast<u32x2*>(orow + d0) = w;
        }
      }
    if (hl == 0) {
      if (P.mode == RMX_FWD_ACC_INIT || P.mode == RMX_FWD_ACC_MERGE) {
        P.acc_lse[lrow] = lnew;
      } else if (P.lse) {
        P.lse[lrow] = lnew;
      }
    }
  }
}

template <int HD, int NW, int NB>
static hipError_t launch_fwd_t(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                               hipStream_t stream) {
  constexpr int BQ = 32 * NB * NW;
  FwdParams prm;
  prm.L = L;
  prm.nprob = n;
  prm.scale_log2 = L.scale * kLog2e;
  int tot = 0;
  for (int i = 0; i < n; ++i) {
    prm.P[i] = probs[i];
    prm.qtiles[i] = (probs[i].sq + BQ - 1) / BQ;
    prm.tile_start[i] = tot;
    tot += L.batch * L.hq * prm.qtiles[i];
  }
  for (int i = n; i <= RMX_MAX_BATCHED; ++i) prm.tile_start[i] = tot;
  prm.total = tot;
  if (tot == 0) return hipSuccess;
  const int grid = (tot + 7) / 8 * 8;
  hipLaunchKernelGGL((attn_fwd_kernel<HD, NW, NB>), dim3(grid), dim3(NW * 64), 0, stream, prm);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                           hipStream_t stream) {
  if (L.head_dim == 128) return launch_fwd_t<128, 4, 1>(L, probs, n, stream);
  return launch_fwd_t<64, 4, 1>(L, probs, n, stream);
}

}  // namespace rmx
