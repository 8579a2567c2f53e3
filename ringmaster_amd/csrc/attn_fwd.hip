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
// (64 keys) that the mask leaves. At head dim 256 a workgroup is 4 waves (one per
// SIMD: the Q operand and the O accumulator alone take 192 registers) and a key tile
// 32 keys (the seven tile buffers then take 112 KiB of LDS).
//
// Each wave runs a software pipeline over the key tiles (v_mfma_f32_32x32x16_bf16);
// iteration j holds S_j = (K_j Q^T)^T (masked, its row max folded in) and does
//   region 1: S_{j+1} = K_{j+1} Q^T (A = K rows from LDS, rows sigma-permuted,
//             see rmx_common.h; B = Q in VGPRs) while the VALU computes the
//             exponentials of the first 3/4 of S_j and packs them to bf16 (P_j);
//   region 2: O^T += V_j^T P_j^T (A = V^T by ds_read_b64_tr_b16 from the
//             row-major V tile, B = P_j from registers) while the VALU finishes
//             the exponentials of S_j and takes the row max of S_{j+1};
//   then the online-softmax rescale decision for tile j + 1 (the running max
//   only moves when a tile raises it by more than 2^8, so the O rescale is
//   rare) and one workgroup barrier.
// One lane owns one query; the two lane halves split the keys. Operands are read
// from LDS three steps ahead of their MFMA, and scheduling fences keep each
// step's VALU work under its MFMAs.
// K/V tiles: direct global->LDS loads (buffer_load ... lds; rows past the end
// read as zeros) into four K and three V buffers. Iteration j issues K_{j+3}
// and V_{j+2}, which iteration j + 2 is the first to read, and its closing
// barrier waits only for the loads issued before it. The 16-byte chunks of the
// unpadded LDS rows are XOR-swizzled (swz_rows for K, swz_tr for V) so both
// the row reads and the transposed reads are bank-conflict free. The loads are
// the asm form (dma16_async, dma4_async): the kernel orders every LDS read
// after them itself.
#include <type_traits>
#include <utility>

#include "rmx_kernels.h"

namespace rmx {

struct FwdParams {
  rmx_attn_layout L;
  rmx_fwd_problem P[RMX_MAX_BATCHED];  // in launch order (longest workgroups first)
  WgMapParams map;                     // groups = (batch, q head), tiles = query tiles
  float scale_log2;
  uint32_t drop_thr;  // dropout: keep when the element's hash >= drop_thr
  float drop_scale;   // 1 / (1 - p)
};

template <int HD>
struct FwdCfg {
  static constexpr int NW = HD == 256 ? 4 : 8;  // waves per workgroup
  static constexpr int NT = NW * 64;
  static constexpr int BQ = 32 * NW;          // queries per workgroup
  static constexpr int BK = HD == 256 ? 32 : 64;  // keys per tile
  static constexpr int MB = BK / 32;          // 32-key blocks of S^T per tile
  static constexpr int CH = HD / 8;           // 16-byte chunks per row
  static constexpr int RB = HD * 2;           // LDS row bytes (unpadded, swizzled)
  static constexpr int KT = BK * RB;          // bytes of one K (or V) tile
  static constexpr int RPK = 1024 / RB;       // rows per 1 KiB DMA instruction
  static constexpr int NDMA = KT / 1024 / NW; // DMA instructions per wave per tile (K; same for V)
  static constexpr int NKB = HD / 16;         // k-steps of S^T
  static constexpr int NDB = HD / 32;         // 32-row blocks of O^T
  static constexpr int MDOC = BK < 64 ? 64 : BK;  // key metadata slots (a DMA writes 64)
  static_assert(NDMA >= 1 && KT % (1024 * NW) == 0, "tile split");
};

constexpr float kRescaleSlack = 8.0f;  // log2 units: P <= 2^8 between rescales

template <int HD, int MASK, int DT, bool DROP>
__global__ __launch_bounds__(FwdCfg<HD>::NT, 1) void attn_fwd_kernel(const FwdParams prm) {
  using C = FwdCfg<HD>;
  constexpr int BK = C::BK, MB = C::MB, NKB = C::NKB, NDB = C::NDB, CH = C::CH, RB = C::RB;
  constexpr int NDMA = C::NDMA;

  __shared__ __attribute__((aligned(1024))) uint8_t sK[4][C::KT];
  // (the fourth V buffer is for the epilogue: eight tile buffers stage the out rows)
  __shared__ __attribute__((aligned(1024))) uint8_t sV[4][C::KT];
  // RMX_MASK_DOC: global index and document of the keys of tile t, in slot t % 4
  __shared__ __attribute__((aligned(256))) int sKg[4][C::MDOC];
  __shared__ __attribute__((aligned(256))) int sKd[4][C::MDOC];
  __shared__ int sRange[2];
  __shared__ float sWa[C::NW][32];  // epilogue: weight of each row's running out

  const WgCoord wc = map_workgroup(prm.map, blockIdx.x);
  if (!wc.valid) return;
  const rmx_attn_layout& L = prm.L;
  const rmx_fwd_problem& P = prm.P[wc.p];
  const int nqt = prm.map.ntile[wc.p];
  const int qt = nqt - 1 - wc.tile;  // heaviest causal tiles first
  const int head = wc.group % L.hq;
  const int bb = wc.group / L.hq;
  // document metadata of this batch row (RMX_MASK_DOC; m_sb = 0: shared by every row)
  const int64_t moff = MASK == RMX_MASK_DOC ? bb * L.m_sb : 0;
  const int32_t* const qgid = P.q_gidx + moff;
  const int32_t* const kgid = P.k_gidx + moff;
  const int32_t* const qdoc = P.q_doc + moff;
  const int32_t* const kdoc = P.k_doc + moff;
  const int kvh = head / (L.hq / L.hkv);
  const int sq = P.sq, sk = P.sk;
  constexpr int mask = MASK;
  const int q0 = qt * C::BQ;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int qw0 = q0 + 32 * wave;  // first query of this wave
  const int q = qw0 + l32;         // this lane's query

  int qg = -2147483647, qd = -1;
  if (mask == RMX_MASK_DOC && q < sq) {
    qg = qgid[q];
    qd = qdoc[q];
  }
  const int D = L.head_dim;          // columns past D (up to HD) load as zeros
  const int wl = window_bound(P) + diag_shift<MASK>(P);  // window: q + off - key <= wl
  // this lane's lowest key: key >= q + off - wl (document masks: global index >= qlo)
  const int off = sk - sq + diag_shift<MASK>(P);  // the diagonal: key == q + off
  const int qlo = mask == RMX_MASK_DOC ? (q < sq ? clamp_i32((int64_t)qg - wl) : 2147483647)
                                       : q + off - wl;
  // dropout: this lane's query term of the mask hash, and the key offset of the problem
  uint32_t dq_term = 0, dk_off = 0;
  if constexpr (DROP) {
    dq_term = drop_bhmix(L, bb, head) ^ (uint32_t)(q + P.drop_q0) * kDropQ;
    dk_off = (uint32_t)P.drop_k0;
  }

  // ---- key tile range of the workgroup
  const int qlast = (q0 + C::BQ < sq ? q0 + C::BQ : sq) - 1;
  const int nkt = (sk + BK - 1) / BK;
  int kt_begin = 0, kt_end = nkt;
  int qg_first = 0, qg_last = 0, qd_first = 0, qd_last = 0;
  if (mask != RMX_MASK_DOC) {
    if (mask == RMX_MASK_CAUSAL) {
      const int kmax = qlast + off;
      kt_end = kmax < 0 ? 0 : (kmax / BK + 1 < nkt ? kmax / BK + 1 : nkt);
    }
    const int kmin = q0 + off - wl;  // the first query's lowest key
    kt_begin = kmin <= 0 ? 0 : (kmin / BK < nkt ? kmin / BK : nkt);
    if (kt_end < kt_begin) kt_end = kt_begin;
  } else {
    qg_first = qgid[q0];
    qg_last = qgid[qlast];
    qd_first = qdoc[q0];
    qd_last = qdoc[qlast];
    if (tid == 0) {
      sRange[0] = nkt;
      sRange[1] = -1;
    }
    __syncthreads();
    int lo = nkt, hi = -1;
    for (int t = tid; t < nkt; t += C::NT) {
      const int ka = t * BK, kz = (t * BK + BK < sk ? t * BK + BK : sk) - 1;
      const int kga = kgid[ka], kgz = kgid[kz];
      const int kda = kdoc[ka], kdz = kdoc[kz];
      if (kga <= qg_last && kdz >= qd_first && kda <= qd_last && (int64_t)kgz >= (int64_t)qg_first - wl) {
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
  const int ntile = kt_end - kt_begin;
  // no key tile: a merge into the running (out, lse) leaves it as it is
  if (ntile == 0 && P.mode == RMX_FWD_ACC_MERGE) return;
  // document bounds of this wave's 32 queries (lanes 0 and 31; rows past sq read as
  // document -1, so a tile with them takes the masked path): a tile whose keys all lie in
  // the wave's one document, at or before its first query and inside the window of its
  // last, needs no mask for this wave, whatever the rest of the workgroup's queries see
  const int wqg_first = __builtin_amdgcn_readlane(qg, 0), wqg_last = __builtin_amdgcn_readlane(qg, 31);
  const int wqd_first = __builtin_amdgcn_readlane(qd, 0), wqd_last = __builtin_amdgcn_readlane(qd, 31);

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[q][16kb + 8hl .. +7]
  bf16x8 qreg[NKB];
  if (ntile > 0) {
    const uint16_t* qb = P.q + bb * L.q_sb + head * L.q_sh;
    const i32x4 rs = make_rsrc(qb, span_bytes(sq, 2 * L.q_ss, D * 2));
    const int qo = q * (int)(2 * L.q_ss) + 16 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      qreg[kb] = __builtin_bit_cast(bf16x8, cols_below(buf_load16(rs, qo + 32 * kb), 16 * kb + 8 * hl, D));
  }

  // ---- K/V staging: buffer resources over this (batch, kv head)
  const int kss = (int)(2 * L.k_ss), vss = (int)(2 * L.v_ss);
  const i32x4 krs = make_rsrc(P.k + bb * L.k_sb + kvh * L.k_sh, span_bytes(sk, kss, D * 2));
  const i32x4 vrs = make_rsrc(P.v + bb * L.v_sb + kvh * L.v_sh, span_bytes(sk, vss, D * 2));
  const i32x4 krs0 = make_rsrc(P.k, 0u), vrs0 = make_rsrc(P.v, 0u);  // zero-length loads
  // DMA of a K (V) tile at key k0 into buffer b: instruction n of the tile fills
  // LDS bytes [1024 n, 1024 n + 1024), lane L row n*RPK + L/CH, swizzled chunk L%CH;
  // chunks of columns past D are loaded from kOutOfRange (zeros)
  auto dma_k = [&](int b, int k0) __attribute__((always_inline)) {
    const uint32_t d = lds_addr(&sK[b][0]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int n = wave * NDMA + i;
      const int r = n * C::RPK + lane / CH, ch = (lane % CH) ^ swz_rows<HD>(r);
      dma16_async(krs, d + 1024 * n, 8 * ch < D ? (k0 + r) * kss + 16 * ch : kOutOfRange);
    }
  };
  auto dma_v = [&](int b, int k0) __attribute__((always_inline)) {
    const uint32_t d = lds_addr(&sV[b][0]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int n = wave * NDMA + i;
      const int r = n * C::RPK + lane / CH, ch = (lane % CH) ^ swz_tr<HD>(r);
      dma16_async(vrs, d + 1024 * n, 8 * ch < D ? (k0 + r) * vss + 16 * ch : kOutOfRange);
    }
  };
  // instruction i of a K (V) tile's DMA through resource rs (num_records 0 past the end:
  // the buffer gets zeros and no memory is read)
  auto dma_k_part = [&](const i32x4& rs, int b, int k0, int i) __attribute__((always_inline)) {
    const int n = wave * NDMA + i;
    const int r = n * C::RPK + lane / CH, ch = (lane % CH) ^ swz_rows<HD>(r);
    dma16_async(rs, lds_addr(&sK[b][0]) + 1024 * n, 8 * ch < D ? (k0 + r) * kss + 16 * ch : kOutOfRange);
  };
  auto dma_v_part = [&](const i32x4& rs, int b, int k0, int i) __attribute__((always_inline)) {
    const int n = wave * NDMA + i;
    const int r = n * C::RPK + lane / CH, ch = (lane % CH) ^ swz_tr<HD>(r);
    dma16_async(rs, lds_addr(&sV[b][0]) + 1024 * n, 8 * ch < D ? (k0 + r) * vss + 16 * ch : kOutOfRange);
  };
  // key metadata of tile t (RMX_MASK_DOC), one dword per lane, by wave 0
  constexpr bool DOCDMA = mask == RMX_MASK_DOC;
  i32x4 kgrs = {0, 0, 0, 0}, kdrs = {0, 0, 0, 0};
  if (DOCDMA) {
    kgrs = make_rsrc(kgid, 4u * (uint32_t)sk);
    kdrs = make_rsrc(kdoc, 4u * (uint32_t)sk);
  }
  auto dma_doc = [&](int t) __attribute__((always_inline)) {
    if (DOCDMA && wave == 0) {
      const int k0 = (kt_begin + t) * BK;
      dma4_async(kgrs, lds_addr(&sKg[t & 3][0]), 4 * (k0 + lane));
      dma4_async(kdrs, lds_addr(&sKd[t & 3][0]), 4 * (k0 + lane));
    }
  };

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
  f32x16 sA[MB], sB[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    sA[mb] = zero16();
    sB[mb] = zero16();
  }
  float m_run = kNegInf, l_run = 0.f;
  const float c = prm.scale_log2;

  // ---- LDS operand reads
  auto k_op = [&](int kbi, int t, int mb) __attribute__((always_inline)) -> bf16x8 {
    return __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const u32x4*>(&sK[kbi][0] + kaddr[t] + mb * 32 * RB));
  };
  auto v_op = [&](int vbi, int kb2, int db) __attribute__((always_inline)) -> bf16x8 {
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(&sV[vbi][0] + vaddr[db] + 16 * kb2 * RB);
    return join_bf16x8(lds_read_tr(vp), lds_read_tr(vp + 2 * RB));
  };

  // ---- masking of a score tile (keys of tile t): out-of-range keys, the causal
  // diagonal, the window's lower edge and document boundaries -> -inf. A tile past
  // the wave's diagonal (or below its window) is masked whole and yields P = 0.
  auto need_mask = [&](int t) __attribute__((always_inline)) -> bool {
    const int k0 = (kt_begin + t) * BK;
    bool nm = (k0 + BK > sk);
    if (mask == RMX_MASK_CAUSAL) nm |= (k0 + BK - 1 > qw0 + off);
    if (mask != RMX_MASK_DOC) nm |= (k0 < qw0 + 31 + off - wl);
    if (mask == RMX_MASK_DOC) {
      const int ds = t & 3;
      const int kga = sKg[ds][0], kgz = sKg[ds][BK - 1];
      const int kda = sKd[ds][0], kdz = sKd[ds][BK - 1];
      nm |= !(kda == kdz && kda == wqd_first && wqd_first == wqd_last && kgz <= wqg_first &&
              (int64_t)kga >= (int64_t)wqg_last - wl);
    }
    return nm;
  };
  auto apply_mask = [&](int t, f32x16* sd) __attribute__((always_inline)) {
    const int k0 = (kt_begin + t) * BK;
    const int ds = t & 3;
    // key of (mb, r) = k0 + 8 hl + kc with the constant kc = 32 mb + 16 (r >> 3) + (r & 7):
    // compare the constants against per-lane limits (no per-element registers)
    const int kbase = k0 + 8 * hl;
    const int lim_sk = sk - kbase;      // kc < lim_sk  <=>  key < sk
    const int lim_c = q + off - kbase;  // kc <= lim_c  <=>  key <= q + off
    const int lim_w = qlo - kbase;      // kc >= lim_w  <=>  key >= q + off - wl
    const int* kgrow = &sKg[ds][8 * hl];
    const int* kdrow = &sKd[ds][8 * hl];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kc = 32 * mb + 16 * (r >> 3) + (r & 7);
        bool ok = kc < lim_sk;
        if (mask == RMX_MASK_CAUSAL) ok &= kc <= lim_c;
        if (mask != RMX_MASK_DOC) ok &= kc >= lim_w;
        if (mask == RMX_MASK_DOC) ok &= (kdrow[kc] == qd) & (kgrow[kc] <= qg) & (kgrow[kc] >= qlo);
        sd[mb][r] = ok ? sd[mb][r] : kNegInf;
      }
  };
  // row max of a score tile (log2 units, both lane halves)
  auto tile_max_part = [&](const f32x16* sd, int lo, int hi) __attribute__((always_inline)) -> float {
    float m = kNegInf;
    for (int e = lo; e < hi; ++e) m = fmaxf(m, sd[e >> 4][e & 15]);
    return m;
  };
  // online-softmax bookkeeping for a new tile whose row max (log2 units) is mx:
  // the running max only moves when the tile raises it by more than the slack
  auto rescale = [&](float mx, bool live) __attribute__((always_inline)) {
    const bool raise = live && mx > m_run + kRescaleSlack;
    if (__any(raise)) {
      const float mnew = raise ? fmaxf(m_run, mx) : m_run;
      const float alpha = (m_run == kNegInf) ? 0.f : fast_exp2(m_run - mnew);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= alpha;
      m_run = mnew;
    }
  };

  // ---- prologue: K_0, K_1, V_0 (and the metadata of tiles 0, 1) resident;
  // K_2, V_1 in flight; S_0 computed, masked and its max folded in
  if (ntile > 0) {
    dma_k(0, kt_begin * BK);
    dma_v(0, kt_begin * BK);
    dma_doc(0);
    if (ntile > 1) {
      dma_k(1, (kt_begin + 1) * BK);
      dma_doc(1);
    }
  }
  wait_all_loads();
  __syncthreads();
  // loads of iteration j: K_{j+3} into K buffer (j+3) % 4, V_{j+2} into V buffer
  // (j+2) % 3; iteration j + 2 is the first to read them. This form issues them for
  // j = -1, here; the iterations issue theirs inside region 1 (below)
  auto issue = [&](int j, int vb2) __attribute__((always_inline)) {
    if (j + 3 < ntile) {
      dma_k((j + 3) & 3, (kt_begin + j + 3) * BK);
      dma_doc(j + 3);
    }
    if (j + 2 < ntile) dma_v(vb2, (kt_begin + j + 2) * BK);
  };
  // end of iteration j: everything but the loads issued at iteration j has landed
  // (every iteration issues the same loads, zero-length past the end)
  auto barrier_wait = [&](int j) __attribute__((always_inline)) {
    if (DOCDMA && wave == 0)
      wait_vm_barrier<2 * NDMA + 2>();
    else
      wait_vm_barrier<2 * NDMA>();
  };
  issue(-1, 1);
  if (ntile > 0) {
#pragma unroll
    for (int t = 0; t < NKB; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) sA[mb] = mfma32t<DT>(k_op(0, t, mb), qreg[t], sA[mb]);
    if (need_mask(0)) {
      keep_branch();
      apply_mask(0, sA);
    }
    float mx = tile_max_part(sA, 0, 16 * MB);
    mx = fmaxf(mx, xhalf(mx)) * c;
    rescale(mx, true);
  }

  // ---- iteration j: S_j (masked, its max folded into m_run) is in sc.
  //   region 1: S_{j+1} = K_{j+1} Q^T into sn (NKB steps of MB MFMAs), with the
  //             exponentials of the first 3/4 of S_j (pairs of elements ->
  //             the 16-bit packing (v_cvt_pk_bf16_f32 for bf16) -> P_j);
  //   region 2: O += V_j^T P_j (PVS steps of two MFMAs), with the last quarter
  //             of the exponentials (ahead of the PV MFMAs that use them) and
  //             the row max of S_{j+1};
  //   then the rescale decision for tile j + 1 and the barrier.
  // Operands are read one step ahead; scheduling fences keep the steps in order
  // so each step's VALU work issues under its MFMAs.
  constexpr int PVS = (2 * MB * NDB) / 2;  // PV steps (two MFMAs each)
  constexpr int NPAIR = MB * 8;            // element pairs per lane (32 scores)
  constexpr int P1 = NPAIR * 3 / 4;        // pairs done in region 1
  // first PV step that reads the last P block (its MFMAs go over the blocks in order):
  // every pair of that block is packed before it
  constexpr int PV3 = (2 * MB - 1) * NDB / 2;
  constexpr int KD = 3, VD = 3;            // operand prefetch depth (steps) of regions 1 and 2
  static_assert(VD <= NKB && VD < PVS && 2 * MB * KD <= 15 && 4 * VD <= 15, "lgkmcnt range");
  static_assert(P1 >= 4 * (2 * MB - 1) && PV3 >= 1, "P blocks packed before their MFMAs");
  static_assert(2 * NDMA <= NKB, "a tile's loads fit the steps of region 1");
  auto pv_idx = [](int u, int v) { return 2 * u + v; };  // PV MFMA: kb2 = idx / NDB, db = idx % NDB
  auto iter = [&](int j, int vbj, f32x16* sc, f32x16* sn) __attribute__((always_inline)) {
    const int vb2 = vbj == 0 ? 2 : vbj - 1;  // (j + 2) % 3
    // this iteration's loads, K_{j+3} (and its documents) then V_{j+2}, one DMA instruction
    // per step of region 1 after the step's MFMAs (8.26-8.28 -> 8.20 ms per configs[2] ring
    // launch against all of them, behind branches, ahead of region 1)
    const bool klive = j + 3 < ntile, vlive = j + 2 < ntile;
    const i32x4 krs_j = klive ? krs : krs0, vrs_j = vlive ? vrs : vrs0;
    const int kk0 = (kt_begin + (klive ? j + 3 : 0)) * BK, vk0 = (kt_begin + (vlive ? j + 2 : 0)) * BK;
    const int kbuf = (j + 3) & 3;
    const int kbi = (j + 1) & 3;
    const bool live = j + 1 < ntile;
    const float mbase = (m_run == kNegInf) ? 0.f : m_run;
    // dropout: key term of this lane's first key of tile j (keys kd0 + 16 kb2 + 2 w + e)
    const uint32_t kd0 = DROP ? ((uint32_t)((kt_begin + j) * BK + 8 * hl) + dk_off) * kDropK : 0u;
    u32x4 pw[2 * MB];   // P_j packed to bf16, one u32x4 per 16-key block
    float rsp[2 * MB];  // partial row sums per 16-key block
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i) rsp[i] = -0.f;  // -0 + x == x: the first sums fold away
    auto pair = [&](auto pp) __attribute__((always_inline)) {
      constexpr int pi = decltype(pp)::value;  // pair index: elements 2 pi, 2 pi + 1
      constexpr int kb2 = pi / 4, w = pi % 4;
      const float x0 = fast_exp2(fmaf(sc[kb2 >> 1][8 * (kb2 & 1) + 2 * w], c, -mbase));
      const float x1 = fast_exp2(fmaf(sc[kb2 >> 1][8 * (kb2 & 1) + 2 * w + 1], c, -mbase));
      float rs = rsp[kb2] + (x0 + x1);  // the softmax normaliser: undropped
      uint32_t pk;
      if constexpr (DROP) {
        constexpr uint32_t c0 = (uint32_t)(16 * kb2 + 2 * w) * kDropK, c1 = c0 + kDropK;
        const float y0 = drop_keep(dq_term, kd0 + c0, prm.drop_thr) ? x0 * prm.drop_scale : 0.f;
        const float y1 = drop_keep(dq_term, kd0 + c1, prm.drop_thr) ? x1 * prm.drop_scale : 0.f;
        pk = cvt_pk<DT>(y0, y1);
      } else {
        pk = cvt_pk<DT>(x0, x1);
      }
      // pin the results here: otherwise the compiler sinks the exponentials to
      // their first use (after the region) and the step has no VALU work
      asm volatile("" : "+v"(rs), "+v"(pk));
      rsp[kb2] = rs;
      pw[kb2][w] = pk;
    };
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) sn[mb] = zero16();
    bf16x8 va[VD + 1][2];
    // region 1
    bf16x8 ka[KD + 1][MB];
#pragma unroll
    for (int t = 0; t < KD; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) ka[t][mb] = k_op(kbi, t, mb);
    [&]<int... T>(std::integer_sequence<int, T...>) __attribute__((always_inline)) {
      (
          [&] {
            constexpr int t = T;
            if constexpr (t + KD < NKB) {
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) ka[(t + KD) % (KD + 1)][mb] = k_op(kbi, t + KD, mb);
            }
            if constexpr (t + VD >= NKB) {  // the first V operands of region 2
              constexpr int u = t + VD - NKB;
#pragma unroll
              for (int v = 0; v < 2; ++v) va[u][v] = v_op(vbj, pv_idx(u, v) / NDB, pv_idx(u, v) % NDB);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) sn[mb] = mfma32t<DT>(ka[t % (KD + 1)][mb], qreg[t], sn[mb]);
            if constexpr (t < NDMA)
              dma_k_part(krs_j, kbuf, kk0, t);
            else if constexpr (t < 2 * NDMA)
              dma_v_part(vrs_j, vb2, vk0, t - NDMA);
            if constexpr (t == 0 && DOCDMA) {
              if (wave == 0) {
                const int b3 = (j + 3) & 3;
                dma4_async(klive ? kgrs : krs0, lds_addr(&sKg[b3][0]), 4 * (kk0 + lane));
                dma4_async(klive ? kdrs : krs0, lds_addr(&sKd[b3][0]), 4 * (kk0 + lane));
              }
            }
            [&]<int... Q>(std::integer_sequence<int, Q...>) __attribute__((always_inline)) {
              (pair(std::integral_constant<int, P1 * t / NKB + Q>{}), ...);
            }(std::make_integer_sequence<int, P1 * (t + 1) / NKB - P1 * t / NKB>{});
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, NKB>{});

    // mask S_{j+1} (rare: sequence end, causal diagonal, document boundaries)
    if (live && need_mask(j + 1)) {
      keep_branch();
      apply_mask(j + 1, sn);
    }

    // region 2
    float mpart[PVS];
    [&]<int... U>(std::integer_sequence<int, U...>) __attribute__((always_inline)) {
      (
          [&] {
            constexpr int u = U;
            if constexpr (u + VD < PVS) {
#pragma unroll
              for (int v = 0; v < 2; ++v)
                va[(u + VD) % (VD + 1)][v] = v_op(vbj, pv_idx(u + VD, v) / NDB, pv_idx(u + VD, v) % NDB);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int v = 0; v < 2; ++v) {
              const int idx = pv_idx(u, v);
              o[idx % NDB] = mfma32t<DT>(va[u % (VD + 1)][v], __builtin_bit_cast(bf16x8, pw[idx / NDB]), o[idx % NDB]);
            }
            // the remaining pairs, all before step PV3 (which starts on the last block)
            if constexpr (u < PV3) {
              [&]<int... Q>(std::integer_sequence<int, Q...>) __attribute__((always_inline)) {
                (pair(std::integral_constant<int, P1 + (NPAIR - P1) * u / PV3 + Q>{}), ...);
              }(std::make_integer_sequence<int, (NPAIR - P1) * (u + 1) / PV3 - (NPAIR - P1) * u / PV3>{});
            }
            // row max of S_{j+1}, 16 MB / PVS scores per step
            mpart[u] = tile_max_part(sn, 16 * MB * u / PVS, 16 * MB * (u + 1) / PVS);
            asm volatile("" : "+v"(mpart[u]));
            __builtin_amdgcn_sched_barrier(0);
          }(),
          ...);
    }(std::make_integer_sequence<int, PVS>{});

    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 2 * MB; ++i) rs += rsp[i];
    l_run += rs;
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < PVS; ++u) mx = fmaxf(mx, mpart[u]);
    mx = fmaxf(mx, xhalf(mx)) * c;
    rescale(mx, live);
    barrier_wait(j);
  };

  int vbj = 0;  // j % 3
  for (int j = 0; j < ntile; j += 2) {
    iter(j, vbj, sA, sB);
    vbj = vbj == 2 ? 0 : vbj + 1;
    if (j + 1 >= ntile) break;
    iter(j + 1, vbj, sB, sA);
    vbj = vbj == 2 ? 0 : vbj + 1;
  }
  wait_all_loads();  // the zero-length loads past the end

  // ---- epilogue: normalise, lse, merge. Lane (hl, l32) holds O^T of the wave's query row
  // l32, columns 32 db + 8 j + 4 hl .. + 3: stored from there, one instruction writes 32
  // (or 16) bytes of each of 32 rows and every line is assembled from partial writes, which
  // reached HBM up to 2.6 times. The rows go through LDS instead (each wave its own [32][HD]
  // fp32 region in the K/V buffers, 16-byte chunks XOR-swizzled by row) and come back as
  // whole rows per store instruction (64 / (HD / 4) rows).
  const float lt = l_run + xhalf(l_run);
  const bool qok = q < sq;
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const float lse_b = lt > 0.f ? (m_run + fast_log2(lt)) * kLn2 : kNegInf;
  const int64_t lrow = bb * L.l_sb + head * L.l_sh + (qok ? q : 0);
  const bool rd = P.mode == RMX_FWD_ACC_MERGE || P.mode == RMX_FWD_ACC_FINAL;
  float wa = 0.f, wb = 1.f, lnew = lse_b;
  if (rd && qok) {
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
  if (hl == 0 && qok) {
    if (P.mode == RMX_FWD_ACC_INIT || P.mode == RMX_FWD_ACC_MERGE) {
      P.acc_lse[lrow] = lnew;
    } else if (P.lse) {
      P.lse[lrow] = lnew;
    }
  }
  constexpr int CPR = HD / 4;   // 16-byte chunks per fp32 row
  constexpr int RPI = 64 / CPR;  // rows per store instruction
  constexpr int NI = 32 / RPI;   // store instructions per wave
  constexpr int GI = NI < 16 ? NI : 16;  // rows read back (and running out loaded) per group
  constexpr int SW = 32 * HD * 4;        // staging bytes per wave
  static_assert(SW % C::KT == 0 && C::NW * SW <= 8 * C::KT && CPR <= 64 && NI % GI == 0,
                "out staging");
  __syncthreads();  // every wave is past its reads of the last tiles and its loads have landed
  const int sb = wave * (SW / C::KT);  // first of the wave's tile buffers (K buffers, then V)
  uint8_t* const stg = sb < 4 ? &sK[sb][0] : &sV[sb - 4][0];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cw = 8 * db + 2 * j + hl;  // columns 4 cw .. 4 cw + 3
      f32x4 v;
      v[0] = o[db][4 * j + 0] * wb;
      v[1] = o[db][4 * j + 1] * wb;
      v[2] = o[db][4 * j + 2] * wb;
      v[3] = o[db][4 * j + 3] * wb;
      *reinterpret_cast<f32x4*>(stg + l32 * (HD * 4) + 16 * (cw ^ (l32 % CPR))) = v;
    }
  if (hl == 0) sWa[wave][l32] = wa;
  __syncthreads();
  // lane: chunk ch of row RPI i + lane / CPR; rows past sq and columns past D are not stored
  const int ch = lane % CPR, rr = lane / CPR;
  const bool colok = 4 * ch < D;
  float* const abase = P.acc_out ? P.acc_out + bb * L.a_sb + head * L.a_sh + 4 * ch : nullptr;
  uint16_t* const obase = P.out ? P.out + bb * L.o_sb + head * L.o_sh + 4 * ch : nullptr;
  const bool wout = P.mode == RMX_FWD_WRITE || P.mode == RMX_FWD_ACC_FINAL;
  // the merging modes read a group's running out before its first store (one wait, not
  // one memory round trip per row)
#pragma unroll
  for (int g = 0; g < NI; g += GI) {
    f32x4 v[GI], prev[GI];
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      const int row = RPI * (g + i) + rr, qq = qw0 + row;
      v[i] = *reinterpret_cast<const f32x4*>(stg + row * (HD * 4) + 16 * (ch ^ (row % CPR)));
      prev[i] = rd && colok && qq < sq ? *reinterpret_cast<const f32x4*>(abase + (int64_t)qq * L.a_ss)
                                       : f32x4{};
    }
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      const int row = RPI * (g + i) + rr, qq = qw0 + row;
      if (!colok || qq >= sq) continue;
      if (rd) v[i] += prev[i] * sWa[wave][row];
      // every mode leaves the fp32 result in acc_out when it is given (WRITE and
      // ACC_FINAL: the final out in fp32, which the backward's delta reads)
      if (abase) *reinterpret_cast<f32x4*>(abase + (int64_t)qq * L.a_ss) = v[i];
      if (wout) {
        u32x2 w;
        w[0] = cvt_pk<DT>(v[i][0], v[i][1]);
        w[1] = cvt_pk<DT>(v[i][2], v[i][3]);
        *reinterpret_cast<u32x2*>(obase + (int64_t)qq * L.o_ss) = w;
      }
    }
  }
}

template <int HD, int DT, bool DROP>
static hipError_t launch_fwd_t(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                               hipStream_t stream) {
  constexpr int BQ = FwdCfg<HD>::BQ;
  FwdParams prm;
  prm.L = L;
  prm.scale_log2 = L.scale * kLog2e;
  drop_params(L.dropout_p, &prm.drop_thr, &prm.drop_scale);
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
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_CAUSAL, DT, DROP>), dim3(grid),
                       dim3(FwdCfg<HD>::NT), 0, stream, prm);
  else if (L.mask == RMX_MASK_DOC)
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_DOC, DT, DROP>), dim3(grid),
                       dim3(FwdCfg<HD>::NT), 0, stream, prm);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<HD, RMX_MASK_FULL, DT, DROP>), dim3(grid),
                       dim3(FwdCfg<HD>::NT), 0, stream, prm);
  return hipGetLastError();
}

template <int DT, bool DROP>
static hipError_t launch_fwd_hd(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                                hipStream_t stream) {
  if (L.head_dim > 128) return launch_fwd_t<256, DT, DROP>(L, probs, n, stream);
  if (L.head_dim > 64) return launch_fwd_t<128, DT, DROP>(L, probs, n, stream);
  return launch_fwd_t<64, DT, DROP>(L, probs, n, stream);
}

hipError_t launch_attn_fwd(const rmx_attn_layout& L, const rmx_fwd_problem* probs, int n,
                           hipStream_t stream) {
  const bool f16 = L.dtype == RMX_DTYPE_F16, drop = L.dropout_p > 0.f;
  if (drop)
    return f16 ? launch_fwd_hd<RMX_DTYPE_F16, true>(L, probs, n, stream)
               : launch_fwd_hd<RMX_DTYPE_BF16, true>(L, probs, n, stream);
  return f16 ? launch_fwd_hd<RMX_DTYPE_F16, false>(L, probs, n, stream)
             : launch_fwd_hd<RMX_DTYPE_BF16, false>(L, probs, n, stream);
}

}  // namespace rmx
