// Block-attention forward for gfx950 with the online-softmax merge fused into
// the epilogue.
//
// Reference semantics: `math_block` (ring/kernels.py:52-78) for the block
// (out, lse), bottom-right causal (:64-67), document masks
// (ring/varlen_blocks.py:51-58,69-80, -inf lse for rows with no key), and the
// merge `update_out_and_lse` / `_merge_full` / `_merge_slice`
// (ring/merge.py:20-31, ring/zigzag.py:49-67).
//
// Work decomposition: one workgroup = 8 waves = 256 queries of one
// (problem, batch, head); each wave owns 32 queries and walks the key tiles
// (64 keys) that the mask leaves, two waves per SIMD so one wave's softmax
// overlaps the other's MFMAs.
//
// Per key tile and wave (v_mfma_f32_32x32x16_bf16):
//   S^T = K Q^T    A = K rows from LDS (rows sigma-permuted, see rmx_common.h),
//                  B = Q held in VGPRs for the whole loop       (16 MFMAs)
//   online softmax per lane (a lane owns one query; the two lane halves split
//   the keys, one cross-half max per tile); the running max is only moved when
//   a tile raises it by more than 2^8, so the O rescale is rare
//   O^T += V^T P^T A = V^T read with ds_read_b64_tr_b16 from the row-major V
//                  tile, B = P straight from the S^T registers     (16 MFMAs)
// K/V tiles: direct global->LDS loads (buffer_load ... lds; rows past the end
// read as zeros) into three LDS buffers, issued two tiles ahead so L2/HBM
// latency stays hidden; each tile is published by a barrier that only waits for
// its own loads. The 16-byte chunks of the unpadded LDS rows are XOR-swizzled
// (swz_rows for K, swz_tr for V) so both the row reads and the transposed reads
// are bank-conflict free.
#include <type_traits>

#include "rmx_kernels.h"

namespace rmx {

struct FwdParams {
  rmx_attn_layout L;
  rmx_fwd_problem P[RMX_MAX_BATCHED];  // in launch order (longest workgroups first)
  WgMapParams map;                     // groups = (batch, q head), tiles = query tiles
  float scale_log2;
};

template <int HD>
struct FwdCfg {
  static constexpr int NW = 8;                // waves per workgroup
  static constexpr int NT = NW * 64;
  static constexpr int BQ = 32 * NW;          // queries per workgroup
  static constexpr int BK = 64;               // keys per tile
  static constexpr int MB = BK / 32;          // 32-key blocks of S^T per tile
  static constexpr int CH = HD / 8;           // 16-byte chunks per row
  static constexpr int RB = HD * 2;           // LDS row bytes (unpadded, swizzled)
  static constexpr int KT = BK * RB;          // bytes of one K (or V) tile
  static constexpr int RPK = 1024 / RB;       // rows per 1 KiB DMA instruction
  static constexpr int NDMA = KT / 1024 / NW; // DMA instructions per wave per tile (K; same for V)
  static constexpr int NKB = HD / 16;         // k-steps of S^T
  static constexpr int NDB = HD / 32;         // 32-row blocks of O^T
  static_assert(NDMA >= 1 && KT % (1024 * NW) == 0, "tile split");
};

constexpr float kRescaleSlack = 8.0f;  // log2 units: P <= 2^8 between rescales

template <int HD, int MASK>
__global__ __launch_bounds__(512, 1) void attn_fwd_kernel(const FwdParams prm) {
  using C = FwdCfg<HD>;
  constexpr int BK = C::BK, MB = C::MB, NKB = C::NKB, NDB = C::NDB, CH = C::CH, RB = C::RB;

  // three K and three V tile buffers (separate objects, so the compiler can tell
  // the buffer being read from the ones the DMA is filling)
  __shared__ __attribute__((aligned(1024))) uint8_t sK0[C::KT];
  __shared__ __attribute__((aligned(1024))) uint8_t sK1[C::KT];
  __shared__ __attribute__((aligned(1024))) uint8_t sK2[C::KT];
  __shared__ __attribute__((aligned(1024))) uint8_t sV0[C::KT];
  __shared__ __attribute__((aligned(1024))) uint8_t sV1[C::KT];
  __shared__ __attribute__((aligned(1024))) uint8_t sV2[C::KT];
  __shared__ int sKg[3][BK];
  __shared__ int sKd[3][BK];
  __shared__ int sRange[2];

  const WgCoord wc = map_workgroup(prm.map, blockIdx.x);
  if (!wc.valid) return;
  const rmx_attn_layout& L = prm.L;
  const rmx_fwd_problem& P = prm.P[wc.p];
  const int nqt = prm.map.ntile[wc.p];
  const int qt = nqt - 1 - wc.tile;  // heaviest causal tiles first
  const int head = wc.group % L.hq;
  const int bb = wc.group / L.hq;
  const int kvh = head / (L.hq / L.hkv);
  const int sq = P.sq, sk = P.sk;
  constexpr int mask = MASK;
  const int q0 = qt * C::BQ;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int qw0 = q0 + 32 * wave;  // first query of this wave
  const int q = qw0 + l32;         // this lane's query

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[q][16kb + 8hl .. +7]
  bf16x8 qreg[NKB];
  {
    const uint16_t* qb = P.q + bb * L.q_sb + head * L.q_sh;
    const i32x4 rs = make_rsrc(qb, span_bytes(sq, 2 * L.q_ss, HD * 2));
    const int off = q * (int)(2 * L.q_ss) + 16 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) qreg[kb] = __builtin_bit_cast(bf16x8, buf_load16(rs, off + 32 * kb));
  }
  int qg = -2147483647, qd = -1;
  if (mask == RMX_MASK_DOC && q < sq) {
    qg = P.q_gidx[q];
    qd = P.doc[qg];
  }

  // ---- key tile range of the workgroup
  const int off = sk - sq;
  const int qlast = (q0 + C::BQ < sq ? q0 + C::BQ : sq) - 1;
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
    for (int t = tid; t < nkt; t += C::NT) {
      const int ka = t * BK, kz = (t * BK + BK < sk ? t * BK + BK : sk) - 1;
      const int kga = P.k_gidx[ka], kgz = P.k_gidx[kz];
      const int kda = P.doc[kga], kdz = P.doc[kgz];
      if (kga <= qg_last && kdz >= qd_first && kda <= qd_last) {
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

  // last key this wave can attend (causal): tiles past it are skipped by the wave
  const int wave_qlast = (qw0 + 31 < sq ? qw0 + 31 : sq - 1);
  const int wave_kmax = mask == RMX_MASK_CAUSAL ? wave_qlast + off : 2147483647;

  // ---- K/V staging: buffer resources over this (batch, kv head)
  const int kss = (int)(2 * L.k_ss), vss = (int)(2 * L.v_ss);
  const i32x4 krs = make_rsrc(P.k + bb * L.k_sb + kvh * L.k_sh, span_bytes(sk, kss, HD * 2));
  const i32x4 vrs = make_rsrc(P.v + bb * L.v_sb + kvh * L.v_sh, span_bytes(sk, vss, HD * 2));
  auto kbuf = [&](auto b) -> uint8_t* {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return sK0;
    else if constexpr (B == 1) return sK1;
    else return sK2;
  };
  auto vbuf = [&](auto b) -> uint8_t* {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return sV0;
    else if constexpr (B == 1) return sV1;
    else return sV2;
  };
  // DMA of the K/V tile at key k0 into buffer b: instruction n of the tile fills
  // LDS bytes [1024 n, 1024 n + 1024), lane L row n*RPK + L/CH, swizzled chunk L%CH
  auto dma_tile = [&](auto b, int k0) {
    uint8_t* kd = kbuf(b);
    uint8_t* vd = vbuf(b);
#pragma unroll
    for (int i = 0; i < C::NDMA; ++i) {
      const int n = wave * C::NDMA + i;
      const int r = n * C::RPK + lane / CH, p = lane % CH;
      dma16(krs, kd + 1024 * n, (k0 + r) * kss + 16 * (p ^ swz_rows<HD>(r)));
      dma16(vrs, vd + 1024 * n, (k0 + r) * vss + 16 * (p ^ swz_tr<HD>(r)));
    }
  };
  int nkg = 0, nkd = 0;
  auto doc_load = [&](int k0) {
    if (mask == RMX_MASK_DOC && tid < BK) {
      const int kk = k0 + tid < sk ? k0 + tid : sk - 1;
      nkg = P.k_gidx[kk];
      nkd = P.doc[nkg];
    }
  };
  auto doc_store = [&](int slot) {
    if (mask == RMX_MASK_DOC && tid < BK) {
      sKg[slot][tid] = nkg;
      sKd[slot][tid] = nkd;
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;

  // per-lane LDS byte offsets of the operand reads (swizzle folded in; see
  // swz_rows / swz_tr): K rows (A of S^T) row 32mb + sigma(l32), chunk 2kb + hl
  int kaddr[NKB];
  {
    const int g = hl ^ swz_rows<HD>(sigma(l32));
    const int base = sigma(l32) * RB + 16 * g;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) kaddr[kb] = base ^ (32 * kb);
  }
  // V^T by transposed reads: key row 16kb2 + 8hl + 4t + (m >> 2), column
  // 32db + 16x + 4(m & 3), m = lane & 15, x = (lane >> 4) & 1
  int vaddr[NDB];
  {
    const int m16 = lane & 15, x16 = (lane >> 4) & 1;
    const int base = (8 * hl + (m16 >> 2)) * RB + 16 * swz_tr<HD>(m16 >> 2) + 32 * x16 +
                     16 * ((m16 & 3) >> 1) + 8 * (m16 & 1);
#pragma unroll
    for (int db = 0; db < NDB; ++db) vaddr[db] = base ^ (64 * db);
  }

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = zero16();
  float m_run = kNegInf, l_run = 0.f;
  const float c = prm.scale_log2;

  // tile j (relative to kt_begin) lives in buffer j % 3; its DMA is issued at
  // the start of tile j - 2 (tiles 0 and 1 in the prologue)
  const int ntile = kt_end - kt_begin;
  if (ntile > 0) {
    dma_tile(B0{}, kt_begin * BK);
    doc_load(kt_begin * BK);
    doc_store(0);
    if (ntile > 1) dma_tile(B1{}, (kt_begin + 1) * BK);
  }
  wait_all_loads();
  __syncthreads();

  auto tile = [&](auto b, int j) {
    constexpr int B = decltype(b)::value;  // == j % 3
    const int k0 = (kt_begin + j) * BK;
    if (j + 1 < ntile) doc_load(k0 + BK);  // key documents of the next tile
    // buffer (j + 2) % 3 held tile j - 1, released by the last barrier
    if (j + 2 < ntile) dma_tile(std::integral_constant<int, (B + 2) % 3>{}, k0 + 2 * BK);
    const uint8_t* kt_lds = kbuf(b);
    const uint8_t* vt_lds = vbuf(b);

    if (k0 <= wave_kmax) {
      bool need_mask = (k0 + BK > sk);
      if (mask == RMX_MASK_CAUSAL) need_mask |= (k0 + BK - 1 > qw0 + off);
      if (mask == RMX_MASK_DOC) {
        const int kgz = sKg[B][BK - 1];
        const int kda = sKd[B][0], kdz = sKd[B][BK - 1];
        need_mask |= !(kda == kdz && kda == qd_first && qd_first == qd_last && kgz <= qg_first);
      }

      // ---- S^T = K Q^T (A = K rows, B = Q in VGPRs); MB blocks of 32 keys
      f32x16 s[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) s[mb] = zero16();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const bf16x8 a = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const u32x4*>(kt_lds + kaddr[kb] + mb * 32 * RB));
          s[mb] = mfma32(a, qreg[kb], s[mb]);
        }
      }

      if (need_mask) {
        keep_branch();
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kl = 32 * mb + sig_row(hl, r);
            const int key = k0 + kl;
            bool ok = key < sk;
            if (mask == RMX_MASK_CAUSAL) ok &= key <= q + off;
            if (mask == RMX_MASK_DOC) {
              const int kd = sKd[B][kl], kg = sKg[B][kl];
              ok &= (kd == qd) & (kg <= qg);
            }
            s[mb][r] = ok ? s[mb][r] : kNegInf;
          }
      }

      // ---- online softmax (log2 domain, scale folded into the exponent FMA)
      // row max as a tree over the scores (short dependency chains)
      float mxp[2 * MB];
#pragma unroll
      for (int t = 0; t < 2 * MB; ++t) {
        mxp[t] = kNegInf;
#pragma unroll
        for (int r = 0; r < 8; ++r) mxp[t] = fmaxf(mxp[t], s[t >> 1][8 * (t & 1) + r]);
      }
#pragma unroll
      for (int w = MB; w >= 1; w >>= 1)
#pragma unroll
        for (int t = 0; t < w; ++t) mxp[t] = fmaxf(mxp[t], mxp[t + w]);
      float mx = fmaxf(mxp[0], xhalf(mxp[0])) * c;
      // move the running max only when this tile raises it by more than the
      // slack (or on the first finite tile); otherwise keep the stale max
      const bool raise = mx > m_run + kRescaleSlack;
      if (__any(raise)) {
        const float mnew = fmaxf(m_run, mx);
        const float alpha = (m_run == kNegInf) ? 0.f : fast_exp2(m_run - mnew);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] *= alpha;
        m_run = mnew;
      }
      const float mbase = (m_run == kNegInf) ? 0.f : m_run;
      float rsp[2 * MB];  // partial row sums (short dependency chains)
      bf16x8 pb[2 * MB];
#pragma unroll
      for (int kb2 = 0; kb2 < 2 * MB; ++kb2) {
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = fast_exp2(fmaf(s[kb2 >> 1][8 * (kb2 & 1) + i], c, -mbase));
        rsp[kb2] = ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
        pb[kb2] = pack8_hw(pv);
      }
#pragma unroll
      for (int w = MB; w >= 1; w >>= 1)
#pragma unroll
        for (int t = 0; t < w; ++t) rsp[t] += rsp[t + w];
      l_run += rsp[0];

      // ---- O^T += V^T P^T
#pragma unroll
      for (int kb2 = 0; kb2 < 2 * MB; ++kb2) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* vp = reinterpret_cast<const uint16_t*>(vt_lds + vaddr[db] + 16 * kb2 * RB);
          const bf16x8 a = join_bf16x8(lds_read_tr(vp), lds_read_tr(vp + 2 * RB));
          o[db] = mfma32(a, pb[kb2], o[db]);
        }
      }
    }

    // publish tile j + 1 (its DMA was issued a tile ago); tile j + 2's stays in flight
    if (j + 1 < ntile) doc_store((B + 1) % 3);
    if (j + 2 < ntile)
      wait_vm_barrier<2 * C::NDMA>();
    else
      wait_vm_barrier<0>();
  };
  for (int j = 0; j < ntile; j += 3) {
    tile(B0{}, j);
    if (j + 1 < ntile) tile(B1{}, j + 1);
    if (j + 2 < ntile) tile(B2{}, j + 2);
  }

  // ---- epilogue: normalise, lse, merge
  const float lt = l_run + xhalf(l_run);
  if (q >= sq) return;
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const float lse_b = lt > 0.f ? (m_run + fast_log2(lt)) * kLn2 : kNegInf;
  const int64_t lrow = bb * L.l_sb + head * L.l_sh + q;
  float wa = 0.f, wb = 1.f, lnew = lse_b;
  if (P.mode == RMX_FWD_ACC_MERGE || P.mode == RMX_FWD_ACC_FINAL) {
    const float la = P.acc_lse[lrow];
    const float mxl = fmaxf(la, lse_b);
    if (mxl == kNegInf) {
      lnew = kNegInf;
      wa = 0.f;
      wb = 0.f;
    } else {
      const float mnl = fminf(la, lse_b);
      lnew = mxl + fast_log2(1.f + fast_exp2((mnl - mxl) * kLog2e)) * kLn2;
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
      v[0] = o[db][4 * j + 0] * wb;
      v[1] = o[db][4 * j + 1] * wb;
      v[2] = o[db][4 * j + 2] * wb;
      v[3] = o[db][4 * j + 3] * wb;
      if (P.mode == RMX_FWD_ACC_MERGE || P.mode == RMX_FWD_ACC_FINAL) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(accrow + d0);
        v += a * wa;
      }
      // every mode leaves the fp32 result in acc_out when it is given (WRITE and
      // ACC_FINAL: the final out in fp32, which the backward's delta reads)
      if (accrow) *reinterpret_cast<f32x4*>(accrow + d0) = v;
      if (P.mode == RMX_FWD_WRITE || P.mode == RMX_FWD_ACC_FINAL) {
        u32x2 w;
        w[0] = cvt_pk_bf16(v[0], v[1]);
        w[1] = cvt_pk_bf16(v[2], v[3]);
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

template <int HD>
static hipError_t launch_fwd_t(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                               hipStream_t stream) {
  constexpr int BQ = FwdCfg<HD>::BQ;
  FwdParams prm;
  prm.L = L;
  prm.scale_log2 = L.scale * kLog2e;
  // longest workgroups (most key tiles) first
  long long cost[RMX_MAX_BATCHED];
  int order[RMX_MAX_BATCHED], groups[RMX_MAX_BATCHED], ntile[RMX_MAX_BATCHED];
  for (int i = 0; i < n; ++i) cost[i] = probs[i].sk;
  order_by_cost(n, cost, order);
  for (int i = 0; i < n; ++i) {
    prm.P[i] = probs[order[i]];
    groups[i] = L.batch * L.hq;
    ntile[i] = (prm.P[i].sq + BQ - 1) / BQ;
  }
  const int grid = plan_workgroups(prm.map, n, groups, ntile);
  if (grid == 0) return hipSuccess;
  if (L.mask == RMX_MASK_CAUSAL)
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_CAUSAL>), dim3(grid), dim3(FwdCfg<HD>::NT), 0,
                       stream, prm);
  else if (L.mask == RMX_MASK_DOC)
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_DOC>), dim3(grid), dim3(FwdCfg<HD>::NT), 0,
                       stream, prm);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_FULL>), dim3(grid), dim3(FwdCfg<HD>::NT), 0,
                       stream, prm);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                           hipStream_t stream) {
  if (L.head_dim == 128) return launch_fwd_t<128>(L, probs, n, stream);
  return launch_fwd_t<64>(L, probs, n, stream);
}

}  // namespace rmx
