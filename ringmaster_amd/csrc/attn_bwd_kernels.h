// Kernels of the block-attention backward for gfx950 (dQ, dK/dV) and their launch
// planning, shared by the units that instantiate them: attn_bwd.hip (head dim 256, where
// the MFMA results sit in the register files the compiler picks) and attn_bwd_vf.hip
// (head dims 64 and 128, built with VGPR-form MFMAs, which the register plan of their
// software-pipelined dK/dV kernel is written for).
#pragma once
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
#include <utility>

#include "rmx_kernels.h"

#ifndef RMX_DQ_NB
#define RMX_DQ_NB 2  // K/V tile buffers of the dQ kernel
#endif

namespace rmx {

struct BwdParams {
  rmx_attn_layout L;
  rmx_bwd_problem P[RMX_MAX_BATCHED];  // in launch order (longest workgroups first)
  WgMapParams map;  // dQ: groups (batch, q head) x query tiles; dK/dV: (batch, kv head) x key tiles
  float scale_log2;
  uint32_t drop_thr;  // dropout: keep when the element's hash >= drop_thr
  float drop_scale;   // 1 / (1 - p)
};

// ---------------------------------------------------------------- shared helpers
// Write a 4-float run of a gradient row according to the output mode.
template <int DT>
__device__ __forceinline__ void grad_store4(int mode, float* acc, uint16_t* bf, f32x4 v) {
  if (mode == RMX_GRAD_WRITE_F32) {
    *reinterpret_cast<f32x4*>(acc) = v;
  } else if (mode == RMX_GRAD_ACC_F32) {
    *reinterpret_cast<f32x4*>(acc) = *reinterpret_cast<const f32x4*>(acc) + v;
  } else {
    if (mode == RMX_GRAD_ACC_FINAL) v += *reinterpret_cast<const f32x4*>(acc);
    u32x2 w;
    w[0] = cvt_pk<DT>(v[0], v[1]);
    w[1] = cvt_pk<DT>(v[2], v[3]);
    *reinterpret_cast<u32x2*>(bf) = w;
  }
}

// ---------------------------------------------------------------- tiles
// Operand shapes shared by the two kernels.
template <int HD>
struct BwdTiles {
  static constexpr int CH = HD / 8;
  static constexpr int NKB = HD / 16;
  static constexpr int NDB = HD / 32;
};

// ---------------------------------------------------------------- dQ (Q-major)
// One workgroup = 8 waves x 32 queries of one (problem, batch, head). Per key
// tile (64 keys) and wave:
//   S^T  = K Q^T    A = K rows (LDS), B = Q (VGPRs)        16 MFMAs
//   dP^T = V dO^T   A = V rows (LDS), B = dO (VGPRs)       16 MFMAs
//   P = exp2(S c - lse2), dS = P (dP - delta)  (lane = query: lse/delta per lane; the
//   dP^T accumulators start at -delta, so dS is one product per element: 10.77 -> 10.47 ms
//   per configs[2] ring launch)
//   dQ^T += K^T dS^T  A = K^T by transposed reads of the K tile, B = dS^T
//                                                            16 MFMAs
// Per tile the S^T MFMAs run block by block (32 keys each), then the dP^T MFMAs; the
// exponentials of P of each S^T block issue under the MFMAs that follow it, a share per
// fenced step (operands read one step ahead), and the dS products and packs under the dQ
// MFMAs. Against S^T and dP^T interleaved with all the exponentials after them: 10.36-10.40
// -> 10.15-10.18 ms per configs[2] ring launch with the exponentials under dP^T only
// (10.50-10.59 -> 10.40-10.47 on a second box), then 10.38 -> 10.08-10.22 with them
// spread from the second S^T block on. A read-ahead ring of 2 steps measured slower.
// K/V tiles (and the key documents) arrive by LDS DMA into NB buffers, tile
// t + NB - 1 issued while tile t is computed, one barrier per tile. Rows are
// unpadded with their 16-byte chunks XOR-swizzled by swz_both, so the K row reads,
// the K transposed reads and the V row reads are all bank-conflict free. The tile
// loop is unrolled over the buffers: every operand read is then a per-lane VGPR
// (swizzle folded in) plus a compile-time offset below 64 KiB, with no address
// arithmetic in the loop. Tiles past the end are issued as zero-length loads,
// which keeps every wait count static.
// At head dim 256 a workgroup is 4 waves (one per SIMD: Q, dO and the dQ accumulator
// take 256 registers) and a key tile 32 keys, so four K/V buffers (16 KiB each) fit.
template <int HD>
struct DqCfg {
  static constexpr int NW = HD == 256 ? 4 : 8;  // waves per workgroup
  static constexpr int NT = NW * 64;
  static constexpr int BQ = 32 * NW;            // queries per workgroup
  static constexpr int BK = HD == 256 ? 32 : 64;  // keys per tile
  static constexpr int NB = HD == 256 ? 4 : RMX_DQ_NB;
  static constexpr int MDOC = BK < 64 ? 64 : BK;  // key metadata slots (a DMA writes 64)
};

template <int HD, int MASK, int DT, bool DROP>
__global__ __launch_bounds__(DqCfg<HD>::NT, 1) void attn_bwd_dq_kernel(const BwdParams prm) {
  using T = BwdTiles<HD>;
  constexpr int NW = DqCfg<HD>::NW, NT = DqCfg<HD>::NT, BQ = DqCfg<HD>::BQ, BK = DqCfg<HD>::BK;
  constexpr int MBK = BK / 32, KB2 = BK / 16;  // 32-key blocks of S^T, 16-key steps of dQ
  constexpr int CH = T::CH, NKB = T::NKB, NDB = T::NDB;
  constexpr int RB = HD * 2;              // LDS row bytes (unpadded, swizzled)
  constexpr int KT = BK * RB;             // bytes of one K (or V) tile
  constexpr int RPK = 1024 / RB;          // rows per 1 KiB DMA instruction
  constexpr int NDMA = KT / 1024 / NW;    // DMA instructions per wave, tile and operand
  constexpr int NB = DqCfg<HD>::NB;       // tile buffers
  // K tiles at [0, NB KT), V tiles after them; V rows get their own base register when
  // the last V tile would sit past the 16-bit LDS instruction offset
  constexpr bool VBASE = 2 * NB * KT - KT / 2 > 65535;
  static_assert(NDMA >= 1 && KT % (1024 * NW) == 0, "tile split");

  // K tiles, then V tiles; the epilogue stages the dQ rows here (NW x 32 x HD fp32)
  constexpr int NTB = 2 * NB > NW * 32 * HD * 4 / KT ? 2 * NB : NW * 32 * HD * 4 / KT;
  __shared__ __attribute__((aligned(1024))) uint8_t sT[NTB][KT];
  __shared__ __attribute__((aligned(256))) int sKg[NB][DqCfg<HD>::MDOC];
  __shared__ __attribute__((aligned(256))) int sKd[NB][DqCfg<HD>::MDOC];
  __shared__ int sRange[2];

  const WgCoord wc = map_workgroup(prm.map, blockIdx.x);
  if (!wc.valid) return;
  const rmx_attn_layout& L = prm.L;
  const rmx_bwd_problem& P = prm.P[wc.p];
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
  const int q0 = qt * BQ;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int qw0 = q0 + 32 * wave;
  const int q = qw0 + l32;
  const bool qvalid = q < sq;

  int qg = -2147483647, qd = -1;
  if (mask == RMX_MASK_DOC && qvalid) {
    qg = qgid[q];
    qd = qdoc[q];
  }
  // document bounds of this wave's 32 queries (lanes 0 and 31; rows past sq read as
  // document -1): the per-tile mask test is the wave's, not the workgroup's
  const int wqg_first = __builtin_amdgcn_readlane(qg, 0), wqg_last = __builtin_amdgcn_readlane(qg, 31);
  const int wqd_first = __builtin_amdgcn_readlane(qd, 0), wqd_last = __builtin_amdgcn_readlane(qd, 31);
  const int D = L.head_dim;        // columns past D (up to HD) load as zeros
  const int wl = window_bound(P) + diag_shift<MASK>(P);  // window: q + off - key <= wl
  const int off = sk - sq + diag_shift<MASK>(P);  // the diagonal: key == q + off
  // this lane's lowest key: key >= q + off - wl (document masks: global index >= qlo)
  const int qlo = mask == RMX_MASK_DOC ? (qvalid ? clamp_i32((int64_t)qg - wl) : 2147483647)
                                       : q + off - wl;
  // dropout: this lane's query term of the mask hash (the forward's)
  const uint32_t dq_term = DROP ? drop_bhmix(L, bb, head) ^ (uint32_t)(q + P.drop_q0) * kDropQ : 0u;

  const int qlast = (q0 + BQ < sq ? q0 + BQ : sq) - 1;
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
    for (int t = tid; t < nkt; t += NT) {
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
  // no key tile: an accumulated dQ keeps its value
  if (kt_end == kt_begin && P.dq_mode == RMX_GRAD_ACC_F32) return;
  bf16x8 qreg[NKB], doreg[NKB];
  {
    const i32x4 qrs = make_rsrc(P.q + bb * L.q_sb + head * L.q_sh,
                                span_bytes(sq, 2 * L.q_ss, D * 2));
    const i32x4 ors = make_rsrc(P.dout + bb * L.o_sb + head * L.o_sh,
                                span_bytes(sq, 2 * L.o_ss, D * 2));
    const int qo = q * (int)(2 * L.q_ss) + 16 * hl, oo = q * (int)(2 * L.o_ss) + 16 * hl;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int col = 16 * kb + 8 * hl;
      qreg[kb] = __builtin_bit_cast(bf16x8, cols_below(buf_load16(qrs, qo + 32 * kb), col, D));
      doreg[kb] = __builtin_bit_cast(bf16x8, cols_below(buf_load16(ors, oo + 32 * kb), col, D));
    }
  }
  const int64_t lrow = bb * L.l_sb + head * L.l_sh + (qvalid ? q : 0);
  float lse2 = qvalid ? P.lse[lrow] * kLog2e : kNegInf;
  if (lse2 == kNegInf) lse2 = __builtin_inff();  // no key attended: P == 0 everywhere
  const float dlt = qvalid ? P.delta[lrow] : 0.f;
  f32x16 ndl;  // dP^T accumulators start at -delta (lane = query): dS = P dP' needs no subtraction
#pragma unroll
  for (int i = 0; i < 16; ++i) ndl[i] = -dlt;
  const int wave_qlast = (qw0 + 31 < sq ? qw0 + 31 : sq - 1);
  const int wave_kmax = mask == RMX_MASK_CAUSAL ? wave_qlast + off : 2147483647;
  // keys below the window of every query of the wave (the first query's lowest key)
  const int wave_kmin = mask == RMX_MASK_DOC ? -2147483647 : qw0 + off - wl;

  // ---- tile loads: wave w fills 1 KiB pieces w*NDMA .. of the K and V tiles (lane L:
  // row n*RPK + L/CH, swizzled chunk L%CH); wave 0 also the tile's key documents
  const int ntile = kt_end - kt_begin;
  const int kss = (int)(2 * L.k_ss), vss = (int)(2 * L.v_ss);
  const uint8_t* const kb0 = reinterpret_cast<const uint8_t*>(P.k + bb * L.k_sb + kvh * L.k_sh);
  const uint8_t* const vb0 = reinterpret_cast<const uint8_t*>(P.v + bb * L.v_sb + kvh * L.v_sh);
  const uint32_t kspan = span_bytes(sk, kss, D * 2), vspan = span_bytes(sk, vss, D * 2);
  int vk[NDMA], vv[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int n = wave * NDMA + i;
    const int r = n * RPK + lane / CH, ch = (lane % CH) ^ swz_both<HD>(r);
    // chunks of columns past D load from kOutOfRange (zeros)
    vk[i] = 8 * ch < D ? r * kss + 16 * ch : kOutOfRange;
    vv[i] = 8 * ch < D ? r * vss + 16 * ch : kOutOfRange;
  }
  constexpr bool DOCDMA = mask == RMX_MASK_DOC;
  // loads per tile and wave: what the end-of-tile wait leaves in flight
  auto dma_tile = [&](int t) __attribute__((always_inline)) {
    const bool live = t < ntile;
    const int b = t % NB;
    const int ka = (kt_begin + (live ? t : 0)) * BK;
    if (DOCDMA && wave == 0) {
      const uint32_t n = live ? 4u * (uint32_t)(sk - ka) : 0u;
      dma4_async(make_rsrc(kgid + ka, n), lds_addr(&sKg[b][0]), 4 * lane);
      dma4_async(make_rsrc(kdoc + ka, n), lds_addr(&sKd[b][0]), 4 * lane);
    }
    const i32x4 krs = make_rsrc(kb0 + (int64_t)ka * kss, live ? kspan - (uint32_t)(ka * kss) : 0u);
    const i32x4 vrs = make_rsrc(vb0 + (int64_t)ka * vss, live ? vspan - (uint32_t)(ka * vss) : 0u);
    const uint32_t kd = lds_addr(&sT[b][0]), vd = lds_addr(&sT[NB + b][0]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int n = wave * NDMA + i;
      dma16_async(krs, kd + 1024 * n, vk[i]);
      dma16_async(vrs, vd + 1024 * n, vv[i]);
    }
  };
  // end of tile t: tile t + 1 has landed in every wave, tiles t + 2 .. t + NB - 1 stay
  // in flight
  auto tile_barrier = [&]() __attribute__((always_inline)) {
    if (DOCDMA && wave == 0)
      wait_vm_barrier<(NB - 2) * (2 * NDMA + 2)>();
    else
      wait_vm_barrier<(NB - 2) * 2 * NDMA>();
  };

  // per-lane LDS byte offsets (swizzle folded in): rows (A of S^T, dP^T): key row
  // 32 mb + sigma(l32), chunk 2 kb + hl
  int raddr[NKB], vaddr[VBASE ? NKB : 1];
  {
    const int sr = sigma(l32);
    const int base = sr * RB + 16 * (hl ^ swz_both<HD>(sr));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) raddr[kb] = base ^ (32 * kb);
    if constexpr (VBASE) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) vaddr[kb] = raddr[kb] + (int)lds_addr(&sT[NB][0]);
    }
  }
  // transposed reads (A of dQ^T = K^T): key rows 16 kb2 + 8 hl + 4 t + (m >> 2),
  // columns 32 db + 16 x + 4 (m & 3) .. + 3, m = lane & 15, x = (lane >> 4) & 1
  int taddr[2][NDB];
  {
    const int m16 = lane & 15, x16 = (lane >> 4) & 1;
    const int cc = 2 * x16 + ((m16 & 3) >> 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 8 * hl + 4 * t + (m16 >> 2);
      const int base = r * RB + 16 * (cc ^ swz_both<HD>(r)) + 8 * (m16 & 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) taddr[t][db] = base ^ (64 * db);
    }
  }
  auto tr_op = [&](const uint8_t* tile, int kb2, int db) -> bf16x8 {
    const uint8_t* p = tile + 16 * kb2 * RB;
    return join_bf16x8(lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[0][db])),
                       lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[1][db])));
  };
  auto row_op = [&](const uint8_t* tile, int kb, int mb) -> bf16x8 {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(tile + raddr[kb] + mb * 32 * RB));
  };
  // V rows of buffer b (compile-time): through the V base register when there is one
  auto vrow_op = [&](int b, int kb, int mb) -> bf16x8 {
    if constexpr (VBASE) {
      const auto* base = reinterpret_cast<const __attribute__((address_space(3))) uint8_t*>(
          (uintptr_t)(uint32_t)vaddr[kb]);
      return __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                      base + b * KT + mb * 32 * RB));
    } else {
      return row_op(&sT[NB + b][0], kb, mb);
    }
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

#pragma unroll
  for (int t = 0; t < NB - 1; ++t) dma_tile(t);
  tile_barrier();

  const float c = prm.scale_log2;
  // tile t in buffer BUF = t % NB (a compile-time constant in each unrolled copy)
  auto tile_step = [&](int t, auto bufc) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value;
    const int k0 = (kt_begin + t) * BK;
    dma_tile(t + NB - 1);  // into the buffer tile t - 1 used: every wave is past it
    const uint8_t* kt_lds = &sT[buf][0];

    if (k0 <= wave_kmax && k0 + BK > wave_kmin) {
      bool need_mask = (k0 + BK > sk);
      if (mask == RMX_MASK_CAUSAL) need_mask |= (k0 + BK - 1 > qw0 + off);
      if (mask != RMX_MASK_DOC) need_mask |= (k0 < qw0 + 31 + off - wl);
      if (mask == RMX_MASK_DOC) {
        const int kga = sKg[buf][0], kgz = sKg[buf][BK - 1];
        const int kda = sKd[buf][0], kdz = sKd[buf][BK - 1];
        need_mask |= !(kda == kdz && kda == wqd_first && wqd_first == wqd_last && kgz <= wqg_first &&
                       (int64_t)kga >= (int64_t)wqg_last - wl);
      }

      f32x16 s[MBK], dp[MBK];
#pragma unroll
      for (int mb = 0; mb < MBK; ++mb) {
        s[mb] = zero16();
        dp[mb] = DROP ? zero16() : ndl;
      }
      // S^T block by block (32 keys each), then dP^T; the exponentials of P of block mb
      // issue under the MFMAs of block mb + 1 (the last block's under dP^T), a share per
      // fenced step, pinned there (the compiler would sink them past the mask branch to
      // their use). Operands are read one step ahead.
      float pr[MBK][16];
      {
        constexpr int NSS = NKB * MBK, NST = 2 * NSS;  // S^T steps, all steps
        // step u < NSS: S^T block u / NKB, k-step u % NKB; else dP^T (kb, mb) of u - NSS
        auto op_of = [&](int u) __attribute__((always_inline)) -> bf16x8 {
          if (u < NSS) return row_op(kt_lds, u % NKB, u / NKB);
          const int w = u - NSS;
          return vrow_op(buf, w / MBK, w % MBK);
        };
        bf16x8 opr[2];
        opr[0] = op_of(0);
        [&]<int... U>(std::integer_sequence<int, U...>) __attribute__((always_inline)) {
          (
              [&] {
                constexpr int u = U;
                if constexpr (u + 1 < NST) opr[(u + 1) & 1] = op_of(u + 1);
                __builtin_amdgcn_sched_barrier(0);
                // the step's MFMA issues at raised wave priority, ahead of the other wave's
                // VALU work on the SIMD (10.14-10.60 -> 10.09-10.50 ms per configs[2] ring
                // launch on two boxes; the same around the dQ^T MFMAs, or in the forward's
                // regions, measured 4-5% slower)
                __builtin_amdgcn_s_setprio(1);
                if constexpr (u < NSS) {
                  s[u / NKB] = mfma32t<DT>(opr[u & 1], qreg[u % NKB], s[u / NKB]);
                } else {
                  constexpr int w = u - NSS;
                  dp[w % MBK] = mfma32t<DT>(opr[u & 1], doreg[w / MBK], dp[w % MBK]);
                }
                __builtin_amdgcn_s_setprio(0);
                // exponentials of block eb, spread over the steps of the next block (or dP^T)
                constexpr int eb = u < NSS ? u / NKB - 1 : MBK - 1;
                constexpr int n0 = u < NSS ? u % NKB : u - NSS, nn = u < NSS ? NKB : NSS;
                if constexpr (eb >= 0) {
#pragma unroll
                  for (int e = 16 * n0 / nn; e < 16 * (n0 + 1) / nn; ++e) {
                    pr[eb][e] = fast_exp2(fmaf(s[eb][e], c, -lse2));
                    asm volatile("" : "+v"(pr[eb][e]));
                  }
                }
                __builtin_amdgcn_sched_barrier(0);
              }(),
              ...);
        }(std::make_integer_sequence<int, NST>{});
      }

      bf16x8 dsb[KB2];
#pragma unroll
      for (int kb2 = 0; kb2 < KB2; ++kb2) {
        const int mb = kb2 >> 1, b8 = 8 * (kb2 & 1);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = pr[mb][b8 + i];
        if (need_mask) {
        keep_branch();
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int kl = 32 * mb + sig_row(hl, b8 + i);
            const int key = k0 + kl;
            bool ok = key < sk;
            if (mask == RMX_MASK_CAUSAL) ok &= key <= q + off;
            if (mask != RMX_MASK_DOC) ok &= key >= qlo;
            if (mask == RMX_MASK_DOC) {
              const int kd = sKd[buf][kl], kg = sKg[buf][kl];
              ok &= (kd == qd) & (kg <= qg) & (kg >= qlo);
            }
            v[i] = ok ? v[i] : 0.f;
          }
        }
        if constexpr (DROP) {
          // dS = P (M dP / (1 - p) - delta): dP of a dropped element is 0
          const uint32_t kd = ((uint32_t)(k0 + 8 * hl + P.drop_k0) + 16 * kb2) * kDropK;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float m = drop_keep(dq_term, kd + (uint32_t)i * kDropK, prm.drop_thr)
                                ? prm.drop_scale : 0.f;
            v[i] *= fmaf(dp[mb][b8 + i], m, -dlt);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] *= dp[mb][b8 + i];
        }
        dsb[kb2] = pack8t<DT>(v);
      }

      // dQ^T += K^T dS^T
#pragma unroll
      for (int kb2 = 0; kb2 < KB2; ++kb2)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          acc[db] = mfma32t<DT>(tr_op(kt_lds, kb2, db), dsb[kb2], acc[db]);
    }
    tile_barrier();
  };
  for (int t = 0; t < ntile; t += NB) {
    [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
      ((t + B < ntile ? tile_step(t + B, std::integral_constant<int, B>{}) : void()), ...);
    }(std::make_integer_sequence<int, NB>{});
  }
  wait_all_loads();  // the zero-length loads past the end

  // ---- epilogue. Lane (hl, l32) holds dQ^T of the wave's query row l32, columns
  // 32 db + 8 j + 4 hl .. + 3: stored from there, one instruction writes 32 bytes of each
  // of 32 rows and every 128-byte line is assembled from four partial writes, which in
  // lockstep launches reached HBM about twice. The rows go through LDS instead (each wave
  // its own [32][HD] fp32 region in the tile buffers, 16-byte chunks XOR-swizzled by row)
  // and come back as whole rows per store instruction (64 / (HD / 4) rows).
  constexpr int CPR = HD / 4;   // 16-byte chunks per fp32 row
  constexpr int RPI = 64 / CPR;  // rows per store instruction
  constexpr int NI = 32 / RPI;   // store instructions per wave
  constexpr int GI = NI < 16 ? NI : 16;  // rows read back (and prior values loaded) per group
  static_assert(NW * 32 * HD * 4 <= (int)sizeof(sT) && CPR <= 64 && NI % GI == 0, "dQ staging");
  __syncthreads();  // every wave is past its reads of the last tiles and its loads have landed
  uint8_t* const stg = &sT[0][0] + wave * (32 * HD * 4);
  const float scale = L.scale;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cw = 8 * db + 2 * j + hl;  // columns 4 cw .. 4 cw + 3
      f32x4 v;
      v[0] = acc[db][4 * j + 0] * scale;
      v[1] = acc[db][4 * j + 1] * scale;
      v[2] = acc[db][4 * j + 2] * scale;
      v[3] = acc[db][4 * j + 3] * scale;
      *reinterpret_cast<f32x4*>(stg + l32 * (HD * 4) + 16 * (cw ^ (l32 % CPR))) = v;
    }
  __syncthreads();
  // lane: chunk ch of row RPI i + lane / CPR; rows past sq and columns past D are not stored
  const int ch = lane % CPR, rr = lane / CPR;
  const bool colok = 4 * ch < D;
  float* const abase = P.dq_acc ? P.dq_acc + bb * L.a_sb + head * L.a_sh + 4 * ch : nullptr;
  uint16_t* const bbase = P.dq ? P.dq + bb * L.o_sb + head * L.o_sh + 4 * ch : nullptr;
  // the accumulating modes read a group's prior values before its first store (one wait,
  // not one memory round trip per row)
  const int mode = P.dq_mode;
  const bool rd = mode == RMX_GRAD_ACC_F32 || mode == RMX_GRAD_ACC_FINAL;
  // the prior value is added: the store is a write (f32) or a conversion (16-bit)
  const int wmode = mode == RMX_GRAD_ACC_F32 ? RMX_GRAD_WRITE_F32
                    : mode == RMX_GRAD_ACC_FINAL ? RMX_GRAD_WRITE_BF16 : mode;
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
      const int qq = qw0 + RPI * (g + i) + rr;
      if (!colok || qq >= sq) continue;
      if (rd) v[i] += prev[i];
      grad_store4<DT>(wmode, abase ? abase + (int64_t)qq * L.a_ss : nullptr,
                      bbase ? bbase + (int64_t)qq * L.o_ss : nullptr, v[i]);
    }
  }
}

// ---------------------------------------------------------------- dK, dV (KV-major, one wave per SIMD)
// One workgroup = 128 keys of one (problem, batch, kv head), 4 waves (one per
// SIMD, up to 512 registers each). Wave w owns keys k0 + 32w .. k0 + 32w + 31
// and runs all four GEMMs of a query tile (64 queries) itself, so P and dS never
// leave its registers:
//   S   = Q K^T             A = Q rows (LDS), B = K (VGPRs)
//   P   = exp2(S c + nl)    nl = -lse log2(e) per query (from the delta pass),
//                           in place in S (fp32)
//   dP' = delta - dO V^T    A = dO rows (LDS), B = -V (VGPRs); the accumulator
//                           starts at delta, read from LDS straight into it
//   dV += P^T dO            A = P^T (registers), B = dO^T (transposed LDS reads)
//   dK -= (P dP')^T Q       A = (P dP')^T, B = Q^T (transposed LDS reads)
// (dS = P (dP - delta) = -P dP'; the sign goes into the final scale of dK.)
// A tile is a software pipeline of four phases of NS = HD/8 steps, one MFMA per
// step, each step's VALU work issued under its MFMA and its LDS operand read eight
// to nine steps ahead, in pairs every other step (across phase and tile
// boundaries):
//   phase 0: dP'_j           | exponentials of S_j rows 0..31, P^T block 0
//   phase 1: dV_j            | exponentials of rows 32..63, P^T blocks 1..3,
//                              (P dP')^T block 0
//   -- barrier: tile j + 1 landed; tile j - 3's buffer takes tile j + 3
//   phase 2: dK_j            | (P dP')^T blocks 1..3, the loads of tile j + 3 (one
//                              DMA instruction per step: 15.54-15.62 -> 15.43-15.49 ms
//                              per configs[2] ring launch against all of them ahead
//                              of the phase; the dropout kernels keep that form, since
//                              ROCm 7.2's AGPR-copy MFMA rewrite crashes on them
//                              with the spread one)
//   phase 3: S_{j+1}         | (reads of nl and delta of tile j + 1)
// S_{j+1} reuses the registers of P_j (dead after phase 2). Masked tiles (rare)
// get S := -inf on their masked pairs before their exponentials, with nl clamped
// to a finite value so that a row with lse = -inf (it attends nothing) gives 0,
// not NaN.
// Q/dO tiles (with lse, delta) arrive by LDS DMA into four buffers; a tile is
// issued three barriers before it is read. Tiles past the end are issued as
// zero-length loads (they write zeros to a free buffer and touch no memory),
// which keeps every wait count static.
template <int HD>
struct DkdvCfg {
  static constexpr int NW = 4;                // waves per workgroup (one per SIMD)
  static constexpr int NT = 64 * NW;
  static constexpr int BKV = 32 * NW;         // keys per workgroup
  static constexpr int BQ = 64;               // queries per tile
  static constexpr int NBUF = 4;              // Q/dO tile buffers
  static constexpr int CH = HD / 8;           // 16-byte chunks per row
  static constexpr int RB = HD * 2;           // LDS row bytes (unpadded, swizzled)
  static constexpr int QT = BQ * RB;          // bytes of one Q (or dO) tile
  static constexpr int RPK = 1024 / RB;       // rows per 1 KiB DMA instruction
  static constexpr int NDMA = QT / 1024 / NW; // DMA instructions per wave per tile and operand
  static constexpr int NKB = HD / 16;
  static constexpr int NDB = HD / 32;
  static constexpr int NS = HD / 8;           // steps (MFMAs) per phase
  static_assert(NDMA >= 1 && QT % (1024 * NW) == 0, "tile split");
  static_assert(NS == 2 * NKB && NS == 4 * NDB, "phase shapes");
};

template <int HD, int MASK, int DT, bool DROP>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_kernel(const BwdParams prm) {
  using C = DkdvCfg<HD>;
  constexpr int BQ = C::BQ, NKB = C::NKB, NDB = C::NDB, CH = C::CH, RB = C::RB, NS = C::NS;
  constexpr int NB = C::NBUF;

  __shared__ __attribute__((aligned(1024))) uint8_t sQ[NB][C::QT];
  __shared__ __attribute__((aligned(1024))) uint8_t sO[NB][C::QT];
  // nl = -lse log2(e) and delta of each tile
  __shared__ __attribute__((aligned(512))) float sM[NB][2 * BQ];
  __shared__ int sQg[NB][BQ];
  __shared__ int sQd[NB][BQ];
  __shared__ int sRange[2];

  const WgCoord wc = map_workgroup(prm.map, blockIdx.x);
  if (!wc.valid) return;
  const rmx_attn_layout& L = prm.L;
  const rmx_bwd_problem& P = prm.P[wc.p];
  const int kvh = wc.group % L.hkv;
  const int bb = wc.group / L.hkv;
  // document metadata of this batch row (RMX_MASK_DOC; m_sb = 0: shared by every row)
  const int64_t moff = MASK == RMX_MASK_DOC ? bb * L.m_sb : 0;
  const int32_t* const qgid = P.q_gidx + moff;
  const int32_t* const kgid = P.k_gidx + moff;
  const int32_t* const qdoc = P.q_doc + moff;
  const int32_t* const kdoc = P.k_doc + moff;
  const int G = L.hq / L.hkv;
  const int sq = P.sq, sk = P.sk;
  constexpr int mask = MASK;
  const int k0 = wc.tile * C::BKV;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int kw0 = k0 + 32 * wave;  // first key of this wave
  const int key = kw0 + l32;
  const bool kvalid = key < sk;

  // ---- query-tile range of the workgroup
  const int D = L.head_dim;        // columns past D (up to HD) load as zeros
  const int wl = window_bound(P) + diag_shift<MASK>(P);  // window: q + off - key <= wl
  const int off = sk - sq + diag_shift<MASK>(P);  // the diagonal: key == q + off
  const int klast = (k0 + C::BKV < sk ? k0 + C::BKV : sk) - 1;
  const int nqt = (sq + BQ - 1) / BQ;
  int qt_begin = 0, qt_end = nqt;
  int kg_first = 0, kg_last = 0, kd_first = 0, kd_last = 0;
  if (mask != RMX_MASK_DOC) {
    if (mask == RMX_MASK_CAUSAL) {
      const int qmin = k0 - off;  // first query that sees key k0
      qt_begin = qmin <= 0 ? 0 : qmin / BQ;
      if (qt_begin > nqt) qt_begin = nqt;
    }
    const int qmax = klast + wl - off;  // last query whose window reaches key klast
    qt_end = qmax < 0 ? 0 : (qmax / BQ + 1 < nqt ? qmax / BQ + 1 : nqt);
    if (qt_end < qt_begin) qt_end = qt_begin;
  } else {
    kg_first = kgid[k0];
    kg_last = kgid[klast];
    kd_first = kdoc[k0];
    kd_last = kdoc[klast];
    if (tid == 0) {
      sRange[0] = nqt;
      sRange[1] = -1;
    }
    __syncthreads();
    int lo = nqt, hi = -1;
    for (int t = tid; t < nqt; t += C::NT) {
      const int qa = t * BQ, qz = (t * BQ + BQ < sq ? t * BQ + BQ : sq) - 1;
      const int qga = qgid[qa], qgz = qgid[qz];
      const int qda = qdoc[qa], qdz = qdoc[qz];
      if (qgz >= kg_first && qdz >= kd_first && qda <= kd_last && (int64_t)qga <= (int64_t)kg_last + wl) {
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
  const int ntile = (qt_end - qt_begin) * G;  // (q head, query tile) pairs, q head major
  // no query tile: accumulated dK and dV keep their values
  if (ntile == 0 && P.dkv_mode == RMX_GRAD_ACC_F32) return;
  const int wave_klast = (kw0 + 31 < sk ? kw0 + 31 : sk - 1);

  // ---- tile loads. Wave 0 first loads the tile's lse and delta (one dword per
  // lane; rows past the end read 0, where Q and dO rows are 0 as well, so they
  // add nothing), then every wave its share of the Q and dO rows (instruction n
  // fills LDS bytes [1024 n, 1024 n + 1024), lane L row n*RPK + L/CH, swizzled
  // chunk L%CH). Every wave issues 2*NDMA loads per tile after its metadata, so
  // a wait that leaves the last 2*NDMA loads in flight covers every earlier tile.
  struct Cursor {
    int qt, hi;
  };
  auto advance = [&](Cursor c) -> Cursor {
    if (++c.qt == qt_end) {
      c.qt = qt_begin;
      ++c.hi;
    }
    return c;
  };
  // Everything but the tile's row offset and q head is fixed per workgroup: byte bases
  // of the (batch, first q head of the group) slices, per-head strides and each lane's
  // offsets inside a tile. A tile only moves the buffer bases (scalar adds) and shrinks
  // num_records by the same amount, so rows past the end still read as zero.
  const int qss = (int)(2 * L.q_ss), oss = (int)(2 * L.o_ss);
  const uint8_t* const qb0 = reinterpret_cast<const uint8_t*>(P.q + bb * L.q_sb + (int64_t)kvh * G * L.q_sh);
  const uint8_t* const ob0 = reinterpret_cast<const uint8_t*>(P.dout + bb * L.o_sb + (int64_t)kvh * G * L.o_sh);
  const uint8_t* const nb0 = reinterpret_cast<const uint8_t*>(P.nlse + bb * L.l_sb + (int64_t)kvh * G * L.l_sh);
  const uint8_t* const db0 = reinterpret_cast<const uint8_t*>(P.delta + bb * L.l_sb + (int64_t)kvh * G * L.l_sh);
  const int qhs = (int)(2 * L.q_sh), ohs = (int)(2 * L.o_sh), lhs = (int)(4 * L.l_sh);
  const uint32_t qspan = span_bytes(sq, qss, D * 2), ospan = span_bytes(sq, oss, D * 2);
  int vq[C::NDMA], vo[C::NDMA];
#pragma unroll
  for (int i = 0; i < C::NDMA; ++i) {
    const int n = wave * C::NDMA + i;
    const int r = n * C::RPK + lane / CH, ch = (lane % CH) ^ swz_both<HD>(r);
    // chunks of columns past D load from kOutOfRange (zeros)
    vq[i] = 8 * ch < D ? r * qss + 16 * ch : kOutOfRange;
    vo[i] = 8 * ch < D ? r * oss + 16 * ch : kOutOfRange;
  }
  // part p of a tile's loads into buffer b: p = 0 also the metadata (wave 0), then the
  // wave's Q rows (p < NDMA) or dO rows; all 2 NDMA parts make the tile
  auto dma_part = [&](int b, Cursor cu, bool live, int p) __attribute__((always_inline)) {
    const int qa = cu.qt * BQ;
    const int hi = live ? cu.hi : 0;
    if (p == 0 && wave == 0) {
      const int lo = hi * lhs + 4 * qa;
      const uint32_t n = live ? 4u * (uint32_t)(sq - qa) : 0u;
      const uint32_t m = lds_addr(sM[b]);
      dma4_async(make_rsrc(nb0 + lo, n), m, 4 * lane);
      dma4_async(make_rsrc(db0 + lo, n), m + 4 * BQ, 4 * lane);
    }
    if (p < C::NDMA) {
      const i32x4 qrs = make_rsrc(qb0 + hi * qhs + qa * qss, live ? qspan - (uint32_t)(qa * qss) : 0u);
      dma16_async(qrs, lds_addr(sQ[b]) + 1024 * (wave * C::NDMA + p), vq[p]);
    } else {
      const int i = p - C::NDMA;
      const i32x4 ors = make_rsrc(ob0 + hi * ohs + qa * oss, live ? ospan - (uint32_t)(qa * oss) : 0u);
      dma16_async(ors, lds_addr(sO[b]) + 1024 * (wave * C::NDMA + i), vo[i]);
    }
  };
  auto dma_tile = [&](int b, Cursor cu, bool live) {
    const int qa = cu.qt * BQ;
    const int hi = live ? cu.hi : 0;
    if (wave == 0) {
      const int lo = hi * lhs + 4 * qa;
      const uint32_t n = live ? 4u * (uint32_t)(sq - qa) : 0u;
      const uint32_t m = lds_addr(sM[b]);
      dma4_async(make_rsrc(nb0 + lo, n), m, 4 * lane);
      dma4_async(make_rsrc(db0 + lo, n), m + 4 * BQ, 4 * lane);
    }
    const int qo = hi * qhs + qa * qss, oo = hi * ohs + qa * oss;
    const i32x4 qrs = make_rsrc(qb0 + qo, live ? qspan - (uint32_t)(qa * qss) : 0u);
    const i32x4 ors = make_rsrc(ob0 + oo, live ? ospan - (uint32_t)(qa * oss) : 0u);
    const uint32_t qd = lds_addr(sQ[b]), od = lds_addr(sO[b]);
#pragma unroll
    for (int i = 0; i < C::NDMA; ++i) {
      const int n = wave * C::NDMA + i;
      dma16_async(qrs, qd + 1024 * n, vq[i]);
      dma16_async(ors, od + 1024 * n, vo[i]);
    }
  };
  int nqg = 0, nqd = 0;
  auto doc_load = [&](Cursor cu) {
    if (mask == RMX_MASK_DOC && tid < BQ) {
      const int qq = cu.qt * BQ + tid;
      if (qq < sq) {
        nqg = qgid[qq];
        nqd = qdoc[qq];
      } else {
        nqg = -2147483647;  // rows past the end: masked
        nqd = -1;
      }
    }
  };
  auto doc_store = [&](int slot) {
    if (mask == RMX_MASK_DOC && tid < BQ) {
      sQg[slot][tid] = nqg;
      sQd[slot][tid] = nqd;
    }
  };

  // per-lane LDS byte offsets (swizzle folded in): rows (A of S, dP'): query row
  // 32 mb + sigma(l32), chunk 2 kb + hl
  int raddr[NKB];
  {
    const int sr = sigma(l32);
    const int base = sr * RB + 16 * (hl ^ swz_both<HD>(sr));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) raddr[kb] = base ^ (32 * kb);
  }
  // transposed reads (B of dV, dK): query rows 16 kb2 + 8 hl + 4 t + (m >> 2),
  // columns 32 db + 16 x + 4 (m & 3) .. + 3, m = lane & 15, x = (lane >> 4) & 1
  int taddr[2][NDB];
  {
    const int m16 = lane & 15, x16 = (lane >> 4) & 1;
    const int cc = 2 * x16 + ((m16 & 3) >> 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 8 * hl + 4 * t + (m16 >> 2);
      const int base = r * RB + 16 * (cc ^ swz_both<HD>(r)) + 8 * (m16 & 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) taddr[t][db] = base ^ (64 * db);
    }
  }
  auto tr_op = [&](const uint8_t* tile, int kb2, int db) -> bf16x8 {
    const uint8_t* p = tile + 16 * kb2 * RB;
    return join_bf16x8(lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[0][db])),
                       lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[1][db])));
  };
  auto row_op = [&](const uint8_t* tile, int kb, int mb) -> bf16x8 {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(tile + raddr[kb] + mb * 32 * RB));
  };

  // ---- K and -V of this wave's keys in registers (lane: key row, dims 16 kb + 8 hl ..)
  bf16x8 kreg[NKB], vreg[NKB];
  {
    const int kss = (int)(2 * L.k_ss), vss = (int)(2 * L.v_ss);
    const i32x4 krs = make_rsrc(P.k + bb * L.k_sb + kvh * L.k_sh, span_bytes(sk, kss, D * 2));
    const i32x4 vrs = make_rsrc(P.v + bb * L.v_sb + kvh * L.v_sh, span_bytes(sk, vss, D * 2));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int col = 16 * kb + 8 * hl;
      kreg[kb] = __builtin_bit_cast(bf16x8, cols_below(buf_load16(krs, key * kss + 16 * hl + 32 * kb), col, D));
      vreg[kb] = __builtin_bit_cast(
          bf16x8, cols_below(buf_load16(vrs, key * vss + 16 * hl + 32 * kb) ^ 0x80008000u, col, D));
    }
    // MFMA reads its A/B operands from AGPRs as well: K and -V live there, which
    // leaves the VGPRs to the fp32 tiles the VALU works on
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) asm volatile("" : "+a"(kreg[kb]), "+a"(vreg[kb]));
  }
  int kg = 2147483647, kd = -2;
  if (mask == RMX_MASK_DOC && kvalid) {
    kg = kgid[key];
    kd = kdoc[key];
  }
  // this lane's highest query: q + off <= key + wl (document masks: global index <= khi)
  const int khi = mask == RMX_MASK_DOC ? clamp_i32((int64_t)kg + wl) : key + wl - off;
  // document bounds of this wave's 32 keys (lanes 0 and 31; keys past sk read as
  // document -2): the per-tile mask test is the wave's, not the workgroup's
  const int wkg_last = __builtin_amdgcn_readlane(kg, 31);
  const int wkd_first = __builtin_amdgcn_readlane(kd, 0), wkd_last = __builtin_amdgcn_readlane(kd, 31);
  const int wkhi_first =
      mask == RMX_MASK_DOC ? clamp_i32((int64_t)__builtin_amdgcn_readlane(kg, 0) + wl) : 0;

  // dropout: the keep bits of a tile's 32 elements of this lane (bit 16 mb + r: query
  // 32 mb + sig_row(hl, r) of the tile, key `key`), hashed as the forward does
  const uint32_t dk_term = DROP ? (uint32_t)(key + P.drop_k0) * kDropK : 0u;
  const uint32_t dq_hl = (uint32_t)(8 * hl) * kDropQ;
  // bits [E0, E1) of the tile at query row qa of q head `hi` (of this kv head's group)
  auto drop_bits = [&](uint32_t& mw, int qa, int hi, auto e0c, auto e1c) __attribute__((always_inline)) {
    constexpr int E0 = decltype(e0c)::value, E1 = decltype(e1c)::value;
    const uint32_t bk = drop_bhmix(L, bb, kvh * G + hi) ^ dk_term;
    const uint32_t base = (uint32_t)(qa + P.drop_q0) * kDropQ + dq_hl;
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      (
          [&] {
            constexpr int e = E0 + E, mb = e >> 4, r = e & 15;
            constexpr uint32_t qc = (uint32_t)(32 * mb + 16 * (r >> 3) + (r & 7)) * kDropQ;
            if (drop_keep(bk, base + qc, prm.drop_thr)) mw |= 1u << e;
          }(),
          ...);
    }(std::make_integer_sequence<int, E1 - E0>{});
  };

  // per-tile metadata in the accumulator / exponent layout: element r of half mb
  // belongs to query 32 mb + sig_row(hl, r), i.e. two runs of 8 queries
  auto load_rows = [&](const float* m, f32x16* dst) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int h8 = 0; h8 < 2; ++h8) {
        const float* p = m + 32 * mb + 16 * h8 + 8 * hl;
        const f32x4 a = *reinterpret_cast<const f32x4*>(p);
        const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dst[mb][8 * h8 + i] = a[i];
          dst[mb][8 * h8 + 4 + i] = b[i];
        }
      }
  };

  // ---- masking (rare tiles: sequence end, causal diagonal, document boundaries)
  auto need_mask_of = [&](int qa, int slot) -> bool {
    bool m = (kw0 + 32 > sk);
    const int qz = (qa + BQ < sq ? BQ : sq - qa) - 1;
    if (mask == RMX_MASK_CAUSAL) m |= (wave_klast > qa + off);
    if (mask != RMX_MASK_DOC) m |= (qa + qz + off - kw0 > wl);
    if (mask == RMX_MASK_DOC) {
      const int qga = sQg[slot][0], qgz = sQg[slot][qz];
      const int qda = sQd[slot][0];
      const int qdz = sQd[slot][qz];
      m |= !(qda == qdz && qda == wkd_first && wkd_first == wkd_last && wkg_last <= qga &&
             qgz <= wkhi_first);
    }
    return m;
  };
  // S := -inf on masked pairs, nl finite (see above). The 32 elements are
  // expanded at compile time: a runtime element index would put S in scratch.
  auto apply_mask = [&](int qa, int slot, f32x16* s, f32x16* nl) __attribute__((always_inline)) {
    [&]<int... E>(std::integer_sequence<int, E...>) __attribute__((always_inline)) {
      (
          [&] {
            constexpr int mb = E >> 4, r = E & 15;
            const int ql = 32 * mb + sig_row(hl, r);
            bool ok = kvalid;
            if (mask == RMX_MASK_CAUSAL) ok &= key <= qa + ql + off;
            if (mask != RMX_MASK_DOC) ok &= qa + ql <= khi;
            if (mask == RMX_MASK_DOC)
              ok &= (sQd[slot][ql] == kd) & (kg <= sQg[slot][ql]) & (sQg[slot][ql] <= khi);
            s[mb][r] = ok ? s[mb][r] : kNegInf;
            nl[mb][r] = fminf(nl[mb][r], 3.0e38f);
          }(),
          ...);
    }(std::make_integer_sequence<int, 32>{});
  };

  // read i (0..7) of load_rows: rows 32 (i / 4) + 16 ((i / 2) % 2) + 8 hl + 4 (i % 2) .. + 3
  auto load_rows_part = [&](const float* m, f32x16* dst, int i) {
    const int mb = i >> 2, h8 = (i >> 1) & 1, hf = i & 1;
    const f32x4 a = *reinterpret_cast<const f32x4*>(m + 32 * mb + 16 * h8 + 8 * hl + 4 * hf);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[mb][8 * h8 + 4 * hf + e] = a[e];
  };

  // ---- prologue: tiles 0, 1 and 2 issued, documents of tile 0 in LDS
  Cursor cur = {qt_begin, 0};
  Cursor nx1 = advance(cur), nx2 = advance(nx1), nx3 = advance(nx2);
  dma_tile(0, cur, ntile > 0);
  dma_tile(1, nx1, ntile > 1);
  dma_tile(2, nx2, ntile > 2);
  doc_load(cur);
  doc_store(0);

  f32x16 dv[NDB], dk[NDB], s[2], dp[2], nl[2];
  // dropout: delta of the tile's rows (the dP' accumulator then starts at 0, see pack_pair)
  // and the keep bits of the current and the next tile
  f32x16 dl[DROP ? 2 : 1];
  uint32_t mw = 0, mw_next = 0;
  // register classes: S, P and dP' (read by the VALU) in VGPRs; the unit is built with
  // VGPR-form MFMAs, and the register allocator places the dV/dK accumulators
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dv[db] = zero16();
    dk[db] = zero16();
  }
  auto pin_v = [](f32x16* x) __attribute__((always_inline)) {
    asm volatile("" : "+v"(x[0]), "+v"(x[1]));
  };
  wait_all_loads();
  lds_barrier();
  const float c = prm.scale_log2;

  // operand read-ahead (steps). Reads come in pairs every other step, the later step's
  // operand first: the wait before an even step's MFMA then also covers the next step's
  // operand, so one s_waitcnt serves two MFMAs. Eight steps ahead measured 1.2% faster per
  // configs[2] launch than six (an 8-slot ring), twelve and fourteen 2-7% slower (ten
  // crashes the ROCm 7.2 device compiler).
  constexpr int KD = 8, RING = 16;
  // the ring's slots line up across tiles: a tile is 4 NS steps
  static_assert((4 * NS) % RING == 0 && KD + 2 <= RING && KD % 2 == 0,
                "operand ring size must divide the tile's steps");
  bf16x8 ops[RING];
  // LDS operand of step T of the tile in buffer b (T >= 4 NS: the next tile's)
  auto operand = [&](int b, int T) -> bf16x8 {
    const int ph = T / NS, t = T % NS;
    const int bn = (b + 1) % NB;
    if (ph == 0) return row_op(sO[b], t >> 1, t & 1);
    if (ph == 1) return tr_op(sO[b], t / NDB, t % NDB);
    if (ph == 2) return tr_op(sQ[b], t / NDB, t % NDB);
    if (ph == 3) return row_op(sQ[bn], t >> 1, t & 1);
    return row_op(sO[bn], t >> 1, t & 1);
  };

  if (ntile > 0) {
    // S_0, nl_0 and delta_0, the first operands of tile 0
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) s[mb] = zero16();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) s[mb] = mfma32t<DT>(row_op(sQ[0], kb, mb), kreg[kb], s[mb]);
    pin_v(s);
    load_rows(sM[0], nl);
    if constexpr (DROP) {
      load_rows(sM[0] + BQ, dl);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) dp[mb] = zero16();
      drop_bits(mw, cur.qt * BQ, cur.hi, std::integral_constant<int, 0>{},
                std::integral_constant<int, 32>{});
    } else {
      load_rows(sM[0] + BQ, dp);
    }
    pin_v(dp);
    if (need_mask_of(cur.qt * BQ, 0)) {
      keep_branch();
      apply_mask(cur.qt * BQ, 0, s, nl);
    }
#pragma unroll
    for (int T = 0; T < KD; ++T) ops[T] = operand(0, T);
  }

  // pack elements 2w, 2w + 1 of 8-row block blk (rows 32 (blk / 2) + sig_row(hl,
  // 8 (blk % 2) + ..)) of x (times y when given) into word w of op. With dropout
  // (keep scale m = M / (1 - p)): P^T packs P m, and (P dP')^T packs
  // P (delta + m y) with y = -dO V^T, i.e. P (delta - M dP / (1 - p))
  auto pack_pair = [&](bf16x8& op, const f32x16* x, const f32x16* y, int blk, int w) {
    const int mb = blk >> 1, r = 8 * (blk & 1) + 2 * w;
    float v0 = x[mb][r], v1 = x[mb][r + 1];
    if constexpr (DROP) {
      const int e = 16 * mb + r;
      const float m0 = (mw >> e) & 1u ? prm.drop_scale : 0.f;
      const float m1 = (mw >> (e + 1)) & 1u ? prm.drop_scale : 0.f;
      if (y) {
        v0 *= fmaf(m0, y[mb][r], dl[mb][r]);
        v1 *= fmaf(m1, y[mb][r + 1], dl[mb][r + 1]);
      } else {
        v0 *= m0;
        v1 *= m1;
      }
    } else if (y) {
      v0 *= y[mb][r];
      v1 *= y[mb][r + 1];
    }
    u32x4 u = __builtin_bit_cast(u32x4, op);
    uint32_t pk = cvt_pk<DT>(v0, v1);
    asm volatile("" : "+v"(pk));
    u[w] = pk;
    op = __builtin_bit_cast(bf16x8, u);
  };

  auto tile = [&](auto bc, int j) {
    constexpr int B = decltype(bc)::value;  // == j % NB
    constexpr int BN = (B + 1) % NB;
    if (j + 1 < ntile) doc_load(nx1);
    bf16x8 pt[4], dst[4];
    int qa_next = 0;  // first query of tile j + 1 (set at the hand-over, read in phase 3)
    Cursor dcu = nx3;  // tile j + 3: its loads issue one part per step early in phase 2
    const bool dlive = j + 3 < ntile;
    auto step = [&](auto Tc) __attribute__((always_inline)) {
      constexpr int T = decltype(Tc)::value;
      constexpr int ph = T / NS, t = T % NS;
      constexpr int NP = 4 / NDB;  // packs per step when a block is packed over NDB steps
      if constexpr (T % 2 == 0) {
        ops[(T + KD + 1) % RING] = operand(B, T + KD + 1);
        ops[(T + KD) % RING] = operand(B, T + KD);
      }
      if constexpr (ph == 3) {
        // metadata of tile j + 1 (landed at this tile's barrier): the 8 reads of
        // nl, then the 8 of delta, spread over the phase
        constexpr int RPS = 16 / NS;  // reads per step
#pragma unroll
        for (int q = 0; q < RPS; ++q) {
          const int i = RPS * t + q;
          if (i < 8)
            load_rows_part(sM[BN], nl, i);
          else
            load_rows_part(sM[BN] + BQ, DROP ? dl : dp, i - 8);
        }
        if constexpr (DROP) {
          // dP' of tile j + 1 starts at 0; its keep bits, 32 / NS per step
          if constexpr (t == 0) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) dp[mb] = zero16();
            mw_next = 0;
          }
          drop_bits(mw_next, qa_next, cur.hi, std::integral_constant<int, 32 * t / NS>{},
                    std::integral_constant<int, 32 * (t + 1) / NS>{});
        }
        if constexpr (t == NS - 1) pin_v(dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      const bf16x8 a = ops[T % RING];
      if constexpr (ph == 0) {
        dp[t & 1] = mfma32t<DT>(a, vreg[t >> 1], dp[t & 1]);
      } else if constexpr (ph == 1) {
        dv[t % NDB] = mfma32t<DT>(pt[t / NDB], a, dv[t % NDB]);
      } else if constexpr (ph == 2) {
        dk[t % NDB] = mfma32t<DT>(dst[t / NDB], a, dk[t % NDB]);
        // tile j + 3's loads (its buffer is free since the hand-over barrier), one part
        // per step under the dK MFMAs rather than all of them ahead of the first one
        if constexpr (!DROP && t < 2 * C::NDMA) dma_part((B + 3) % NB, dcu, dlive, t);
      } else {
        if constexpr (t < 2) s[t] = zero16();
        s[t & 1] = mfma32t<DT>(a, kreg[t >> 1], s[t & 1]);
        if constexpr (t == NS - 1) pin_v(s);
      }
      if constexpr (ph == 0) {
        // exponentials of rows 0..31; P^T block 0 once its rows are done
        constexpr int e0 = 16 * t / NS, e1 = 16 * (t + 1) / NS;
#pragma unroll
        for (int e = e0; e < e1; ++e) {
          float x = fast_exp2(fmaf(s[0][e], c, nl[0][e]));
          asm volatile("" : "+v"(x));
          s[0][e] = x;
        }
        if constexpr (t >= NS / 2 && t < NS / 2 + 4) pack_pair(pt[0], s, nullptr, 0, t - NS / 2);
      } else if constexpr (ph == 1) {
        // exponentials of rows 32..63 in the first half of the phase
        if constexpr (t < NS / 2) {
          constexpr int e0 = 32 * t / NS, e1 = 32 * (t + 1) / NS;
#pragma unroll
          for (int e = e0; e < e1; ++e) {
            float x = fast_exp2(fmaf(s[1][e], c, nl[1][e]));
            asm volatile("" : "+v"(x));
            s[1][e] = x;
          }
        }
        // P^T block k + 1 in steps [k NDB, (k + 1) NDB); (P dP')^T block 0 last
        constexpr int k = t / NDB;
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          const int w = NP * (t % NDB) + q;
          if constexpr (k < 3)
            pack_pair(pt[k + 1], s, nullptr, k + 1, w);
          else
            pack_pair(dst[0], s, dp, 0, w);
        }
      } else if constexpr (ph == 2) {
        // (P dP')^T block k + 1 in steps [k NDB, (k + 1) NDB)
        constexpr int k = t / NDB;
        if constexpr (k < 3) {
#pragma unroll
          for (int q = 0; q < NP; ++q) pack_pair(dst[k + 1], s, dp, k + 1, NP * (t % NDB) + q);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    [&]<int... T>(std::integer_sequence<int, T...>) __attribute__((always_inline)) {
      (step(std::integral_constant<int, T>{}), ...);
    }(std::make_integer_sequence<int, 2 * NS>{});  // phases 0, 1

    // hand-over: tile j + 1 landed (tile j + 2 may stay in flight); tile j - 3's
    // buffer (last read in phase 2 of tile j - 3) takes tile j + 3
    if (j + 1 < ntile) doc_store(BN);
    wait_vm_barrier<2 * C::NDMA>();
    if constexpr (DROP) dma_tile((B + 3) % NB, nx3, j + 3 < ntile);
    qa_next = nx1.qt * BQ;
    cur = nx1;
    nx1 = nx2;
    nx2 = nx3;
    nx3 = advance(nx3);

    [&]<int... T>(std::integer_sequence<int, T...>) __attribute__((always_inline)) {
      (step(std::integral_constant<int, 2 * NS + T>{}), ...);
    }(std::make_integer_sequence<int, 2 * NS>{});  // phases 2, 3

    if (j + 1 < ntile && need_mask_of(qa_next, BN)) {
      keep_branch();
      apply_mask(qa_next, BN, s, nl);
    }
    if constexpr (DROP) mw = mw_next;
  };
  for (int j = 0; j < ntile; j += NB) {
    tile(std::integral_constant<int, 0>{}, j);
    if (j + 1 < ntile) tile(std::integral_constant<int, 1>{}, j + 1);
    if (j + 2 < ntile) tile(std::integral_constant<int, 2>{}, j + 2);
    if (j + 3 < ntile) tile(std::integral_constant<int, 3>{}, j + 3);
  }
  wait_all_loads();  // zero-length loads issued past the end

  // ---- epilogue: lane (hl, l32) holds column d = 32 db + l32 of keys kw0 + c_row(hl, r).
  // The accumulating modes read all of the lane's prior dV and dK values before the first
  // store: element by element, each read would wait for the store before it (the compiler
  // cannot tell that they touch different elements), one memory round trip per element.
  const int mode = P.dkv_mode;
  const bool rd = mode == RMX_GRAD_ACC_F32 || mode == RMX_GRAD_ACC_FINAL;
  float prev[2][NDB][16];
  if (rd) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const float* gacc = g == 0 ? P.dv_acc : P.dk_acc;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d = 32 * db + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = kw0 + c_row(hl, r);
          const int64_t ao = bb * L.ka_sb + (int64_t)kk * L.ka_ss + kvh * L.ka_sh + d;
          prev[g][db][r] = d < D && kk < sk ? gacc[ao] : 0.f;
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float sc = g == 0 ? 1.f : -L.scale;
    float* gacc = g == 0 ? P.dv_acc : P.dk_acc;
    uint16_t* gbf = g == 0 ? P.dv : P.dk;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d = 32 * db + l32;
      if (d >= D) continue;  // columns past the head dim are not stored
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = kw0 + c_row(hl, r);
        if (kk >= sk) continue;
        const float gv = (g == 0 ? dv[db][r] : dk[db][r]) * sc;
        const int64_t ao = bb * L.ka_sb + (int64_t)kk * L.ka_ss + kvh * L.ka_sh + d;
        const int64_t bo = bb * L.dk_sb + (int64_t)kk * L.dk_ss + kvh * L.dk_sh + d;
        if (mode == RMX_GRAD_WRITE_F32) {
          gacc[ao] = gv;
        } else if (mode == RMX_GRAD_ACC_F32) {
          gacc[ao] = prev[g][db][r] + gv;
        } else if (mode == RMX_GRAD_ACC_FINAL) {
          gbf[bo] = f2e<DT>(prev[g][db][r] + gv);
        } else {
          gbf[bo] = f2e<DT>(gv);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- dK, dV at head dim 256
// The pipelined kernel above does not fit at head dim 256: its four 64-query Q/dO tile
// buffers take 256 KiB of LDS at 512-byte rows, and K, -V and a wave's dK and dV
// accumulators (32 keys x 256 columns each) take 384 registers before S and dP'.
// This form computes the same per-element math with 32-query tiles and the K block
// resident in LDS. One workgroup = 128 keys of one (problem, batch, kv head), 4 waves
// (one per SIMD); wave w owns keys k0 + 32 w .. + 31 and, per (q head, query tile):
//   S   = Q K^T          A = Q rows (LDS, rows sigma-permuted), B = K rows (LDS)
//   dP' = delta - dO V^T A = dO rows (LDS), B = -V (registers); the accumulator
//                        starts at delta (at 0 with dropout: delta enters the packs)
//   P   = exp2(S c + nl)  (masked pairs: S := -inf first, nl kept finite)
//   dV += P^T dO         A = P^T (registers), B = dO^T (transposed LDS reads)
//   dK -= (P dP')^T Q    A = (P dP')^T, B = Q^T (transposed LDS reads)
// 64 MFMAs per tile and wave, software-pipelined as the kernel above: one MFMA per step,
// the VALU work of a tile spread over the steps of the other GEMMs, LDS operands read
// ahead through a register ring (see the pipeline below). The K block arrives once by LDS
// DMA (64 KiB, rows swizzled by their index mod 16, conflict-free for reads of one chunk
// of 16 rows); Q tiles by LDS DMA into three buffers, dO tiles (+ nl, delta) into two, tile
// j + 1 in flight while tile j is computed, one barrier per tile.
template <int MASK, int DT, bool DROP>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_d256_kernel(const BwdParams prm) {
  constexpr int HD = 256, NW = 4, NT = 64 * NW, BKV = 32 * NW, BQ = 32;
  constexpr int NQB = 3, NOB = 2;  // Q tile buffers; dO tile (+ nl, delta, documents) slots
  constexpr int CH = HD / 8, RB = 2 * HD, QT = BQ * RB, RPK = 1024 / RB;
  constexpr int NDMA = QT / 1024 / NW;        // DMA instructions per wave, tile and operand
  constexpr int KDMA = BKV * RB / 1024 / NW;  // DMA instructions per wave for the K block
  constexpr int NKB = HD / 16, NDB = HD / 32;
  static_assert(NDMA >= 1 && QT % (1024 * NW) == 0 && KDMA >= 1, "tile split");

  // the Q and dO tiles, then the K block (the tiles first: their reads are a per-lane
  // address plus a compile-time offset below 64 KiB); at the end it stages dK and dV rows
  // (128 KiB)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[BKV * RB + (NQB + NOB) * QT];
  static_assert(BKV * HD * 4 <= BKV * RB + (NQB + NOB) * QT, "gradient staging");
  uint8_t(*const sQ)[QT] = reinterpret_cast<uint8_t(*)[QT]>(smem);
  uint8_t(*const sO)[QT] = reinterpret_cast<uint8_t(*)[QT]>(smem + NQB * QT);
  uint8_t* const sK = smem + (NQB + NOB) * QT;
  __shared__ __attribute__((aligned(256))) float sM[NOB][2][64];  // nl, delta (a DMA writes 64)
  __shared__ int sQg[NOB][BQ];
  __shared__ int sQd[NOB][BQ];
  __shared__ int sRange[2];

  const WgCoord wc = map_workgroup(prm.map, blockIdx.x);
  if (!wc.valid) return;
  const rmx_attn_layout& L = prm.L;
  const rmx_bwd_problem& P = prm.P[wc.p];
  const int kvh = wc.group % L.hkv;
  const int bb = wc.group / L.hkv;
  // document metadata of this batch row (RMX_MASK_DOC; m_sb = 0: shared by every row)
  const int64_t moff = MASK == RMX_MASK_DOC ? bb * L.m_sb : 0;
  const int32_t* const qgid = P.q_gidx + moff;
  const int32_t* const kgid = P.k_gidx + moff;
  const int32_t* const qdoc = P.q_doc + moff;
  const int32_t* const kdoc = P.k_doc + moff;
  const int G = L.hq / L.hkv;
  const int sq = P.sq, sk = P.sk;
  constexpr int mask = MASK;
  const int k0 = wc.tile * BKV;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int kw0 = k0 + 32 * wave;  // first key of this wave
  const int key = kw0 + l32;
  const bool kvalid = key < sk;

  // ---- query-tile range of the workgroup (as in the kernel above)
  const int D = L.head_dim;        // columns past D (up to HD) load as zeros
  const int wl = window_bound(P) + diag_shift<MASK>(P);  // window: q + off - key <= wl
  const int off = sk - sq + diag_shift<MASK>(P);  // the diagonal: key == q + off
  const int klast = (k0 + BKV < sk ? k0 + BKV : sk) - 1;
  const int nqt = (sq + BQ - 1) / BQ;
  int qt_begin = 0, qt_end = nqt;
  int kg_first = 0, kg_last = 0, kd_first = 0, kd_last = 0;
  if (mask != RMX_MASK_DOC) {
    if (mask == RMX_MASK_CAUSAL) {
      const int qmin = k0 - off;  // first query that sees key k0
      qt_begin = qmin <= 0 ? 0 : qmin / BQ;
      if (qt_begin > nqt) qt_begin = nqt;
    }
    const int qmax = klast + wl - off;  // last query whose window reaches key klast
    qt_end = qmax < 0 ? 0 : (qmax / BQ + 1 < nqt ? qmax / BQ + 1 : nqt);
    if (qt_end < qt_begin) qt_end = qt_begin;
  } else {
    kg_first = kgid[k0];
    kg_last = kgid[klast];
    kd_first = kdoc[k0];
    kd_last = kdoc[klast];
    if (tid == 0) {
      sRange[0] = nqt;
      sRange[1] = -1;
    }
    __syncthreads();
    int lo = nqt, hi = -1;
    for (int t = tid; t < nqt; t += NT) {
      const int qa = t * BQ, qz = (t * BQ + BQ < sq ? t * BQ + BQ : sq) - 1;
      const int qga = qgid[qa], qgz = qgid[qz];
      const int qda = qdoc[qa], qdz = qdoc[qz];
      if (qgz >= kg_first && qdz >= kd_first && qda <= kd_last && (int64_t)qga <= (int64_t)kg_last + wl) {
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
  const int ntile = (qt_end - qt_begin) * G;  // (q head, query tile) pairs, q head major
  // no query tile: accumulated dK and dV keep their values
  if (ntile == 0 && P.dkv_mode == RMX_GRAD_ACC_F32) return;
  const int wave_klast = (kw0 + 31 < sk ? kw0 + 31 : sk - 1);

  struct Cursor {
    int qt, hi;
  };
  auto advance = [&](Cursor c) -> Cursor {
    if (++c.qt == qt_end) {
      c.qt = qt_begin;
      ++c.hi;
    }
    return c;
  };

  // ---- tile loads: wave 0 loads the tile's nl and delta, every wave its share of the
  // Q and dO rows (instruction n fills LDS bytes [1024 n, 1024 n + 1024), lane L row
  // n*RPK + L/CH, swizzled chunk L%CH); rows past the end read as zeros
  const int qss = (int)(2 * L.q_ss), oss = (int)(2 * L.o_ss);
  const uint8_t* const qb0 = reinterpret_cast<const uint8_t*>(P.q + bb * L.q_sb + (int64_t)kvh * G * L.q_sh);
  const uint8_t* const ob0 = reinterpret_cast<const uint8_t*>(P.dout + bb * L.o_sb + (int64_t)kvh * G * L.o_sh);
  const uint8_t* const nb0 = reinterpret_cast<const uint8_t*>(P.nlse + bb * L.l_sb + (int64_t)kvh * G * L.l_sh);
  const uint8_t* const db0 = reinterpret_cast<const uint8_t*>(P.delta + bb * L.l_sb + (int64_t)kvh * G * L.l_sh);
  const int qhs = (int)(2 * L.q_sh), ohs = (int)(2 * L.o_sh), lhs = (int)(4 * L.l_sh);
  const uint32_t qspan = span_bytes(sq, qss, D * 2), ospan = span_bytes(sq, oss, D * 2);
  int vq[NDMA], vo[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int n = wave * NDMA + i;
    const int r = n * RPK + lane / CH, ch = (lane % CH) ^ swz_both<HD>(r);
    vq[i] = 8 * ch < D ? r * qss + 16 * ch : kOutOfRange;
    vo[i] = 8 * ch < D ? r * oss + 16 * ch : kOutOfRange;
  }
  // Q rows into Q buffer bq; dO rows, nl and delta into slot bo
  auto dma_tile = [&](int bq, int bo, Cursor cu) {
    const int qa = cu.qt * BQ;
    if (wave == 0) {
      const int lo = cu.hi * lhs + 4 * qa;
      const uint32_t n = 4u * (uint32_t)(sq - qa);
      dma4_async(make_rsrc(nb0 + lo, n), lds_addr(&sM[bo][0][0]), 4 * lane);
      dma4_async(make_rsrc(db0 + lo, n), lds_addr(&sM[bo][1][0]), 4 * lane);
    }
    const i32x4 qrs = make_rsrc(qb0 + cu.hi * qhs + qa * qss, qspan - (uint32_t)(qa * qss));
    const i32x4 ors = make_rsrc(ob0 + cu.hi * ohs + qa * oss, ospan - (uint32_t)(qa * oss));
    const uint32_t qd = lds_addr(&sQ[bq][0]), od = lds_addr(&sO[bo][0]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int n = wave * NDMA + i;
      dma16_async(qrs, qd + 1024 * n, vq[i]);
      dma16_async(ors, od + 1024 * n, vo[i]);
    }
  };
  int nqg = 0, nqd = 0;
  auto doc_load = [&](Cursor cu) {
    if (mask == RMX_MASK_DOC && tid < BQ) {
      const int qq = cu.qt * BQ + tid;
      if (qq < sq) {
        nqg = qgid[qq];
        nqd = qdoc[qq];
      } else {
        nqg = -2147483647;  // rows past the end: masked
        nqd = -1;
      }
    }
  };
  auto doc_store = [&](int slot) {
    if (mask == RMX_MASK_DOC && tid < BQ) {
      sQg[slot][tid] = nqg;
      sQd[slot][tid] = nqd;
    }
  };

  // ---- the K block (rows k0 .. k0 + BKV - 1) into LDS, once; -V of this wave's keys in
  // registers (lane: key row, dims 16 kb + 8 hl ..), MFMA operands from AGPRs
  {
    const int kss = (int)(2 * L.k_ss);
    const i32x4 krs = make_rsrc(P.k + bb * L.k_sb + kvh * L.k_sh, span_bytes(sk, kss, D * 2));
    const uint32_t kd = lds_addr(sK);
#pragma unroll
    for (int i = 0; i < KDMA; ++i) {
      const int n = wave * KDMA + i;
      const int r = n * RPK + lane / CH, c = (lane % CH) ^ (r & 15);
      dma16_async(krs, kd + 1024 * n, 8 * c < D ? (k0 + r) * kss + 16 * c : kOutOfRange);
    }
  }
  bf16x8 vreg[NKB];
  {
    const int vss = (int)(2 * L.v_ss);
    const i32x4 vrs = make_rsrc(P.v + bb * L.v_sb + kvh * L.v_sh, span_bytes(sk, vss, D * 2));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int col = 16 * kb + 8 * hl;
      vreg[kb] = __builtin_bit_cast(
          bf16x8, cols_below(buf_load16(vrs, key * vss + 16 * hl + 32 * kb) ^ 0x80008000u, col, D));
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) asm volatile("" : "+a"(vreg[kb]));
  }
  int kg = 2147483647, kd = -2;
  if (mask == RMX_MASK_DOC && kvalid) {
    kg = kgid[key];
    kd = kdoc[key];
  }
  // this lane's highest query: q + off <= key + wl (document masks: global index <= khi)
  const int khi = mask == RMX_MASK_DOC ? clamp_i32((int64_t)kg + wl) : key + wl - off;
  // document bounds of this wave's 32 keys (lanes 0 and 31; keys past sk read as
  // document -2): the per-tile mask test is the wave's, not the workgroup's
  const int wkg_last = __builtin_amdgcn_readlane(kg, 31);
  const int wkd_first = __builtin_amdgcn_readlane(kd, 0), wkd_last = __builtin_amdgcn_readlane(kd, 31);
  const int wkhi_first =
      mask == RMX_MASK_DOC ? clamp_i32((int64_t)__builtin_amdgcn_readlane(kg, 0) + wl) : 0;

  // per-lane LDS byte offsets, swizzle folded in. A chunk index below 16 keeps a
  // lane's offset inside a row's first 256 bytes, so the upper 8 chunk pairs of a row
  // (k-steps 8..15, d blocks 4..7) are the lower ones plus 256: compile-time offsets.
  //   raddr: Q / dO rows (A of S, dP'): query row sigma(l32), chunk 2 kb + hl
  //   kaddr: K rows (B of S): key row 32 wave + l32, chunk 2 kb + hl
  //   taddr: transposed reads (B of dV, dK): query rows 16 kb2 + 8 hl + 4 t + (m >> 2),
  //          columns 32 db + 16 x + 4 (m & 3) .. + 3, m = lane & 15, x = (lane >> 4) & 1
  int raddr[8], kaddr[8], taddr[2][4];
  {
    const int sr = sigma(l32);
    const int rbase = sr * RB + 16 * (hl ^ swz_both<HD>(sr));
    const int kr = 32 * wave + l32;
    const int kbase = kr * RB + 16 * (hl ^ (kr & 15));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      raddr[i] = rbase ^ (32 * i);
      kaddr[i] = kbase ^ (32 * i);
    }
    const int m16 = lane & 15, x16 = (lane >> 4) & 1;
    const int cc = 2 * x16 + ((m16 & 3) >> 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 8 * hl + 4 * t + (m16 >> 2);
      const int base = r * RB + 16 * (cc ^ swz_both<HD>(r)) + 8 * (m16 & 1);
#pragma unroll
      for (int db = 0; db < 4; ++db) taddr[t][db] = base ^ (64 * db);
    }
  }
  auto row_op = [&](const uint8_t* tile, int kb) -> bf16x8 {
    return __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const u32x4*>(tile + raddr[kb & 7] + 256 * (kb >> 3)));
  };
  auto k_op = [&](int kb) -> bf16x8 {
    return __builtin_bit_cast(
        bf16x8, *reinterpret_cast<const u32x4*>(sK + kaddr[kb & 7] + 256 * (kb >> 3)));
  };
  auto tr_op = [&](const uint8_t* tile, int kb2, int db) -> bf16x8 {
    const uint8_t* p = tile + 16 * kb2 * RB + 256 * (db >> 2);
    return join_bf16x8(lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[0][db & 3])),
                       lds_read_tr(reinterpret_cast<const uint16_t*>(p + taddr[1][db & 3])));
  };

  // dropout: the key term of this lane's mask hash (bit r of a tile's keep word: query
  // sig_row(hl, r) of the tile, key `key`), hashed as the forward does
  const uint32_t dk_term = DROP ? (uint32_t)(key + P.drop_k0) * kDropK : 0u;
  // per-query metadata in the accumulator layout: element r is query sig_row(hl, r)
  auto load_rows = [&](const float* m, f32x16& dst) {
#pragma unroll
    for (int h8 = 0; h8 < 2; ++h8) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(m + 16 * h8 + 8 * hl);
      const f32x4 b = *reinterpret_cast<const f32x4*>(m + 16 * h8 + 8 * hl + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dst[8 * h8 + i] = a[i];
        dst[8 * h8 + 4 + i] = b[i];
      }
    }
  };
  auto need_mask_of = [&](int qa, int slot) -> bool {
    bool m = (kw0 + 32 > sk);
    const int qz = (qa + BQ < sq ? BQ : sq - qa) - 1;
    if (mask == RMX_MASK_CAUSAL) m |= (wave_klast > qa + off);
    if (mask != RMX_MASK_DOC) m |= (qa + qz + off - kw0 > wl);
    if (mask == RMX_MASK_DOC) {
      const int qga = sQg[slot][0], qgz = sQg[slot][qz];
      const int qda = sQd[slot][0], qdz = sQd[slot][qz];
      m |= !(qda == qdz && qda == wkd_first && wkd_first == wkd_last && wkg_last <= qga &&
             qgz <= wkhi_first);
    }
    return m;
  };
  auto apply_mask = [&](int qa, int slot, f32x16& s, f32x16& nl) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ql = sig_row(hl, r);
      bool ok = kvalid;
      if (mask == RMX_MASK_CAUSAL) ok &= key <= qa + ql + off;
      if (mask != RMX_MASK_DOC) ok &= qa + ql <= khi;
      if (mask == RMX_MASK_DOC)
        ok &= (sQd[slot][ql] == kd) & (kg <= sQg[slot][ql]) & (sQg[slot][ql] <= khi);
      s[r] = ok ? s[r] : kNegInf;
      nl[r] = fminf(nl[r], 3.0e38f);
    }
  };
  // word w (elements 8 ks + 2 w, + 1) of P^T (y == nullptr) or (P dP')^T block ks. With
  // dropout (keep scale m = M / (1 - p), keep bits mwv): P m, and P (delta + m y) with
  // y = -dO V^T
  auto pack_word = [&](bf16x8& op, const f32x16& x, const f32x16* y, const f32x16& dl,
                       uint32_t mwv, int ks, int w) {
    const int r = 8 * ks + 2 * w;
    float v0 = x[r], v1 = x[r + 1];
    if constexpr (DROP) {
      const float m0 = (mwv >> r) & 1u ? prm.drop_scale : 0.f;
      const float m1 = (mwv >> (r + 1)) & 1u ? prm.drop_scale : 0.f;
      if (y) {
        v0 *= fmaf(m0, (*y)[r], dl[r]);
        v1 *= fmaf(m1, (*y)[r + 1], dl[r + 1]);
      } else {
        v0 *= m0;
        v1 *= m1;
      }
    } else if (y) {
      v0 *= (*y)[r];
      v1 *= (*y)[r + 1];
    }
    u32x4 u = __builtin_bit_cast(u32x4, op);
    uint32_t pk = cvt_pk<DT>(v0, v1);
    asm volatile("" : "+v"(pk));
    u[w] = pk;
    op = __builtin_bit_cast(bf16x8, u);
  };
  // read i (0..3) of load_rows: elements 8 (i / 2) + 4 (i % 2) .. + 3
  auto load_rows_part = [&](const float* m, f32x16& dst, int i) {
    const int h8 = i >> 1, hf = i & 1;
    const f32x4 a = *reinterpret_cast<const f32x4*>(m + 16 * h8 + 8 * hl + 4 * hf);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[8 * h8 + 4 * hf + e] = a[e];
  };
  // dropout keep bit of element r (query sig_row(hl, r) of the tile at qa, head hi)
  auto drop_bit = [&](int qa, int hi, int r) -> uint32_t {
    const uint32_t bk = drop_bhmix(L, bb, kvh * G + hi) ^ dk_term;
    const uint32_t qc = (uint32_t)(qa + P.drop_q0 + 8 * hl + 16 * (r >> 3) + (r & 7)) * kDropQ;
    return drop_keep(bk, qc, prm.drop_thr) ? 1u << r : 0u;
  };

  // ---- prologue: the K block, tiles 0 and 1 issued; tile 0's documents in LDS
  Cursor cur = {qt_begin, 0};
  Cursor nx1 = advance(cur), nx2 = advance(nx1);
  if (ntile > 0) dma_tile(0, 0, cur);
  if (ntile > 1) dma_tile(1, 1, nx1);
  doc_load(cur);
  doc_store(0);
  wait_all_loads();
  lds_barrier();

  f32x16 dv[NDB], dk[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dv[db] = zero16();
    dk[db] = zero16();
  }
  const float c = prm.scale_log2;

  // ---- the software pipeline. Tile j (Q in buffer j % 3; dO, nl, delta and documents in
  // slot j % 2) is four phases of NS = 16 steps, one MFMA per step, the VALU work of the
  // tile under the MFMAs of the phase beside it:
  //   phase 0: dP'_j  = delta - dO_j V^T       | exponentials of S_j, P^T block 0
  //   phase 1: dV    += P_j^T dO_j             | P^T block 1, (P dP')^T blocks 0 and 1
  //   -- hand-over: tile j + 1 landed in every wave; slot j % 2 takes tile j + 2's dO,
  //      nl and delta, Q buffer (j + 2) % 3 (tile j - 1's) its Q rows
  //   phase 2: dK    -= (P_j dP'_j)^T Q_j
  //   phase 3: S_j+1  = Q_j+1 K^T              | nl and delta of tile j + 1 (with dropout:
  //                                              its keep bits)
  // A tile reads F = 80 LDS operands in this order: 16 dO rows, 16 dO^T (transposed
  // reads), 16 Q^T, then a Q row and a K row per step of phase 3. They pass through a
  // RING-slot register ring: operand f sits in slot f % RING and is read when the steps
  // before have consumed f - KD + 1 of them, KD operands (at least three steps) ahead of
  // its MFMA; past the tile's end the next tile's dO rows (landed at this tile's hand-over).
  // Reading 6 operands ahead through 8 slots measured 17.9-18.0 ms per configs[1]-shaped
  // step, 8 through 10 or 16 slots 18.0-18.2, 12 through 16 slots 18.4-18.5 (same box).
  constexpr int NS = 16, F = 80, KD = 6, RING = 8;
  static_assert(NS == NKB && 2 * NDB == NS && F % RING == 0 && KD + 2 <= RING, "pipeline");
  bf16x8 ops[RING];
  f32x16 s, dp, nl, dl;
  uint32_t mw = 0, mw_next = 0;
  auto pin = [](f32x16& x) __attribute__((always_inline)) { asm volatile("" : "+v"(x)); };

  if (ntile > 0) {
    // S_0, nl_0 and delta_0, the first KD operands of tile 0
    s = zero16();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) s = mfma32t<DT>(row_op(sQ[0], kb), k_op(kb), s);
    load_rows(&sM[0][0][0], nl);
    if constexpr (DROP) {
      load_rows(&sM[0][1][0], dl);
      dp = zero16();
#pragma unroll
      for (int r = 0; r < 16; ++r) mw |= drop_bit(cur.qt * BQ, cur.hi, r);
    } else {
      load_rows(&sM[0][1][0], dp);
    }
    pin(s);
    pin(dp);
    if (need_mask_of(cur.qt * BQ, 0)) {
      keep_branch();
      apply_mask(cur.qt * BQ, 0, s, nl);
    }
#pragma unroll
    for (int f = 0; f < KD; ++f) ops[f] = row_op(sO[0], f);
  }

  auto tile = [&](auto jc, int j) {
    constexpr int JC = decltype(jc)::value;  // == j % 6
    constexpr int BQ0 = JC % NQB, BO0 = JC % NOB;              // tile j
    constexpr int BQ1 = (JC + 1) % NQB, BO1 = (JC + 1) % NOB;  // tile j + 1
    constexpr int BQ2 = (JC + 2) % NQB;                        // tile j + 2's Q
    if (j + 1 < ntile) doc_load(nx1);
    bf16x8 pt[2], dst[2];
    int qa_next = 0, hi_next = 0;  // tile j + 1 (set at the hand-over)
    // operand f of this tile (f >= F: the next tile's)
    auto operand = [&](auto fc) __attribute__((always_inline)) -> bf16x8 {
      constexpr int f = decltype(fc)::value;
      if constexpr (f < 16) return row_op(sO[BO0], f);
      else if constexpr (f < 32) return tr_op(sO[BO0], (f - 16) / NDB, (f - 16) % NDB);
      else if constexpr (f < 48) return tr_op(sQ[BQ0], (f - 32) / NDB, (f - 32) % NDB);
      else if constexpr (f < F) {
        if constexpr ((f - 48) % 2 == 0) return row_op(sQ[BQ1], (f - 48) / 2);
        else return k_op((f - 48) / 2);
      } else {
        return row_op(sO[BO1], f - F);
      }
    };
    // operands consumed through step T
    constexpr auto cons = [](int T) constexpr { return T < 0 ? 0 : (T < 48 ? T + 1 : 2 * T - 46); };
    auto step = [&](auto Tc) __attribute__((always_inline)) {
      constexpr int T = decltype(Tc)::value;
      constexpr int ph = T / NS, t = T % NS;
      [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
        ((ops[(cons(T - 1) + KD + I) % RING] =
              operand(std::integral_constant<int, cons(T - 1) + KD + I>{})),
         ...);
      }(std::make_integer_sequence<int, cons(T) - cons(T - 1)>{});
      if constexpr (ph == 3) {
        if constexpr (t < 4) {
          load_rows_part(&sM[BO1][0][0], nl, t);
        } else if constexpr (t < 8) {
          if constexpr (DROP) {
            if constexpr (t == 4) dp = zero16();
            load_rows_part(&sM[BO1][1][0], dl, t - 4);
          } else {
            load_rows_part(&sM[BO1][1][0], dp, t - 4);
          }
        }
        if constexpr (DROP) {
          if constexpr (t == 0) mw_next = 0;
          mw_next |= drop_bit(qa_next, hi_next, t);
        }
        if constexpr (t == NS - 1) pin(dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (ph == 0) {
        dp = mfma32t<DT>(ops[T % RING], vreg[t], dp);
      } else if constexpr (ph == 1) {
        dv[t % NDB] = mfma32t<DT>(pt[t / NDB], ops[T % RING], dv[t % NDB]);
      } else if constexpr (ph == 2) {
        dk[t % NDB] = mfma32t<DT>(dst[t / NDB], ops[T % RING], dk[t % NDB]);
      } else {
        constexpr int f0 = 48 + 2 * t;
        if constexpr (t == 0) s = zero16();
        s = mfma32t<DT>(ops[f0 % RING], ops[(f0 + 1) % RING], s);
        if constexpr (t == NS - 1) pin(s);
      }
      if constexpr (ph == 0) {
        // exponential of element t; P^T block 0 (elements 0..7) once they are done
        float x = fast_exp2(fmaf(s[t], c, nl[t]));
        asm volatile("" : "+v"(x));
        s[t] = x;
        if constexpr (t >= 8 && t < 12) pack_word(pt[0], s, nullptr, dl, mw, 0, t - 8);
      } else if constexpr (ph == 1) {
        // P^T block 1, then (P dP')^T blocks 0 and 1 (dP'_j complete: phase 0 ended)
        if constexpr (t < 4) pack_word(pt[1], s, nullptr, dl, mw, 1, t);
        else if constexpr (t < 8) pack_word(dst[0], s, &dp, dl, mw, 0, t - 4);
        else if constexpr (t < 12) pack_word(dst[1], s, &dp, dl, mw, 1, t - 8);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    [&]<int... T>(std::integer_sequence<int, T...>) __attribute__((always_inline)) {
      (step(std::integral_constant<int, T>{}), ...);
    }(std::make_integer_sequence<int, 2 * NS>{});  // phases 0, 1

    // hand-over: tile j + 1 has landed in every wave and this tile's dO slot (read last in
    // phase 1) and tile j - 1's Q buffer are free for tile j + 2
    if (j + 1 < ntile) doc_store(BO1);
    wait_vm_barrier<0>();
    if (j + 2 < ntile) dma_tile(BQ2, BO0, nx2);
    qa_next = nx1.qt * BQ;
    hi_next = nx1.hi;
    cur = nx1;
    nx1 = nx2;
    nx2 = advance(nx2);

    [&]<int... T>(std::integer_sequence<int, T...>) __attribute__((always_inline)) {
      (step(std::integral_constant<int, 2 * NS + T>{}), ...);
    }(std::make_integer_sequence<int, 2 * NS>{});  // phases 2, 3

    if (j + 1 < ntile && need_mask_of(qa_next, BO1)) {
      keep_branch();
      apply_mask(qa_next, BO1, s, nl);
    }
    if constexpr (DROP) mw = mw_next;
  };
  for (int j = 0; j < ntile; j += 6) {
    tile(std::integral_constant<int, 0>{}, j);
    if (j + 1 < ntile) tile(std::integral_constant<int, 1>{}, j + 1);
    if (j + 2 < ntile) tile(std::integral_constant<int, 2>{}, j + 2);
    if (j + 3 < ntile) tile(std::integral_constant<int, 3>{}, j + 3);
    if (j + 4 < ntile) tile(std::integral_constant<int, 4>{}, j + 4);
    if (j + 5 < ntile) tile(std::integral_constant<int, 5>{}, j + 5);
  }
  wait_all_loads();

  // ---- epilogue: lane (hl, l32) holds column d = 32 db + l32 of keys kw0 + c_row(hl, r).
  // Each gradient is staged through LDS as [key][d] fp32 rows (the tiles are dead) and
  // stored as 4-column runs of whole rows: one mode test per run, not per element.
  const int mode = P.dkv_mode;
  float* const stg = reinterpret_cast<float*>(smem);
  const int col = 4 * (tid & 63), rw = tid >> 6;  // columns col .. col + 3 of rows rw + 4 i
  auto store = [&](const f32x16* acc, float sc, float* gacc, uint16_t* gbf) {
    __syncthreads();  // every wave is past its last tile reads (or the previous gradient)
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        stg[(32 * wave + c_row(hl, r)) * HD + 32 * db + l32] = acc[db][r] * sc;
    __syncthreads();
    if (col >= D) return;  // columns past the head dim are not stored
    const bool vf = ((uintptr_t)gacc & 15) == 0, vb = ((uintptr_t)gbf & 7) == 0;
    auto gptr = [&](int kk) {
      return gacc ? gacc + bb * L.ka_sb + (int64_t)kk * L.ka_ss + kvh * L.ka_sh + col : nullptr;
    };
    auto bptr = [&](int kk) {
      return gbf ? gbf + bb * L.dk_sb + (int64_t)kk * L.dk_ss + kvh * L.dk_sh + col : nullptr;
    };
    if (vf && vb) {
      // the accumulating modes read the prior values of 16 of the thread's rows before
      // their first store (one wait per 16 rows, not one memory round trip per row)
      const bool rd = mode == RMX_GRAD_ACC_F32 || mode == RMX_GRAD_ACC_FINAL;
      const int wmode = mode == RMX_GRAD_ACC_F32 ? RMX_GRAD_WRITE_F32
                        : mode == RMX_GRAD_ACC_FINAL ? RMX_GRAD_WRITE_BF16 : mode;
      constexpr int RUN = 16;
#pragma unroll
      for (int i0 = 0; i0 < BKV / 4; i0 += RUN) {
        f32x4 prev[RUN];
#pragma unroll
        for (int i = 0; i < RUN; ++i) {
          const int kk = k0 + rw + 4 * (i0 + i);
          prev[i] = rd && kk < sk ? *reinterpret_cast<const f32x4*>(gptr(kk)) : f32x4{};
        }
#pragma unroll
        for (int i = 0; i < RUN; ++i) {
          const int row = rw + 4 * (i0 + i), kk = k0 + row;
          if (kk >= sk) return;
          f32x4 v = *reinterpret_cast<const f32x4*>(stg + row * HD + col);
          if (rd) v += prev[i];
          grad_store4<DT>(wmode, gptr(kk), bptr(kk), v);
        }
      }
      return;
    }
    for (int row = rw; row < BKV && k0 + row < sk; row += 4) {
      const int kk = k0 + row;
      const f32x4 v = *reinterpret_cast<const f32x4*>(stg + row * HD + col);
      float* ga = gptr(kk);
      uint16_t* gb = bptr(kk);
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // a caller pointer below vector alignment
        if (mode == RMX_GRAD_WRITE_F32) {
          ga[e] = v[e];
        } else if (mode == RMX_GRAD_ACC_F32) {
          ga[e] += v[e];
        } else if (mode == RMX_GRAD_ACC_FINAL) {
          gb[e] = f2e<DT>(ga[e] + v[e]);
        } else {
          gb[e] = f2e<DT>(v[e]);
        }
      }
    }
  };
  store(dv, 1.f, P.dv_acc, P.dv);
  store(dk, -L.scale, P.dk_acc, P.dk);
}

template <int HD, int DT, bool DROP>
hipError_t launch_bwd_t(const rmx_attn_layout& L, const rmx_bwd_problem* probs, int n,
                        hipStream_t stream) {
  constexpr int BQ_DQ = DqCfg<HD>::BQ, BKV = HD == 256 ? 128 : DkdvCfg<HD>::BKV;
  BwdParams pq, pk;
  pq.L = L;
  pk.L = L;
  pq.scale_log2 = pk.scale_log2 = L.scale * kLog2e;
  drop_params(L.dropout_p, &pq.drop_thr, &pq.drop_scale);
  pk.drop_thr = pq.drop_thr;
  pk.drop_scale = pq.drop_scale;
  // problems with an empty side or a skipped gradient get no workgroups there;
  // the others run longest workgroups first (dQ: key tiles, dK/dV: query tiles x group)
  const int G = L.hq / L.hkv;
  long long cq[RMX_MAX_BATCHED], ck[RMX_MAX_BATCHED];
  int iq[RMX_MAX_BATCHED], ik[RMX_MAX_BATCHED], nq = 0, nk = 0;
  for (int i = 0; i < n; ++i) {
    const bool empty = probs[i].sq == 0 || probs[i].sk == 0;
    if (!empty && probs[i].dq_mode != RMX_GRAD_NONE) {
      cq[nq] = probs[i].sk;
      iq[nq++] = i;
    }
    if (!empty && probs[i].dkv_mode != RMX_GRAD_NONE) {
      ck[nk] = (long long)probs[i].sq * G;
      ik[nk++] = i;
    }
  }
  int oq[RMX_MAX_BATCHED], ok[RMX_MAX_BATCHED], groups[RMX_MAX_BATCHED], ntile[RMX_MAX_BATCHED];
  order_by_cost(nq, cq, oq);
  order_by_cost(nk, ck, ok);
  for (int i = 0; i < nq; ++i) {
    pq.P[i] = probs[iq[oq[i]]];
    groups[i] = L.batch * L.hq;
    ntile[i] = (pq.P[i].sq + BQ_DQ - 1) / BQ_DQ;
  }
  const int tq = plan_workgroups(pq.map, nq, groups, ntile);
  for (int i = 0; i < nk; ++i) {
    pk.P[i] = probs[ik[ok[i]]];
    groups[i] = L.batch * L.hkv;
    ntile[i] = (pk.P[i].sk + BKV - 1) / BKV;
  }
  const int tk = plan_workgroups(pk.map, nk, groups, ntile);
  if constexpr (HD == 256) {
    if (tk > 0) {
      const dim3 grid(tk);
      if (L.mask == RMX_MASK_CAUSAL)
        hipLaunchKernelGGL((attn_bwd_dkdv_d256_kernel<RMX_MASK_CAUSAL, DT, DROP>), grid, dim3(256), 0, stream, pk);
      else if (L.mask == RMX_MASK_DOC)
        hipLaunchKernelGGL((attn_bwd_dkdv_d256_kernel<RMX_MASK_DOC, DT, DROP>), grid, dim3(256), 0, stream, pk);
      else
        hipLaunchKernelGGL((attn_bwd_dkdv_d256_kernel<RMX_MASK_FULL, DT, DROP>), grid, dim3(256), 0, stream, pk);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  } else {
    if (tk > 0) {
      const dim3 grid(tk);
      if (L.mask == RMX_MASK_CAUSAL)
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, RMX_MASK_CAUSAL, DT, DROP>), grid, dim3(DkdvCfg<HD>::NT), 0, stream, pk);
      else if (L.mask == RMX_MASK_DOC)
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, RMX_MASK_DOC, DT, DROP>), grid, dim3(DkdvCfg<HD>::NT), 0, stream, pk);
      else
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HD, RMX_MASK_FULL, DT, DROP>), grid, dim3(DkdvCfg<HD>::NT), 0, stream, pk);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  if (tq > 0) {
    const dim3 grid(tq);
    if (L.mask == RMX_MASK_CAUSAL)
      hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, RMX_MASK_CAUSAL, DT, DROP>), grid, dim3(DqCfg<HD>::NT), 0, stream, pq);
    else if (L.mask == RMX_MASK_DOC)
      hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, RMX_MASK_DOC, DT, DROP>), grid, dim3(DqCfg<HD>::NT), 0, stream, pq);
    else
      hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, RMX_MASK_FULL, DT, DROP>), grid, dim3(DqCfg<HD>::NT), 0, stream, pq);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace rmx
