// Mamba2 context-parallel output correction, backward, for gfx950.
//
// Reference: the autograd of `mamba2_cp_correction` (strategies/mamba.py:101-139),
// plain torch ops there. With e[t,h] = mask[t] * exp(cumA[t,h]) (mask = seq_idx == 0),
// S[t,h,d] = sum_n C[t,g(h),n] H_in[h,d,n] and the upstream gradients G = dL/dy
// (bf16, [B,T,H*d]) and Gs = dL/dh_final_out (fp32, may be absent):
//   dC[t,g,n]    = sum_{h in g} e[t,h] sum_d G[t,h,d] H_in[h,d,n]
//   dcumA[t,h]   = e[t,h] sum_d G[t,h,d] S[t,h,d]
//                  + [t = T-1, state updated] exp(cumA[T-1,h]) sum_{d,n} Gs H_in
//   dH_in[h,d,n] = sum_t e[t,h] G[t,h,d] C[t,g(h),n]
//                  + [state updated] exp(cumA[T-1,h]) Gs[h,d,n]
// (dout = G and dh_final = Gs pass through; the state is updated unless a batch
// row's last token starts a fresh sequence, :131). With P[t,h,n] = sum_d G[t,h,d]
// H_in[h,d,n], both dC and the sum in dcumA are contractions of P:
//   dC[t,g,n] = sum_{h in g} e[t,h] P[t,h,n],  sum_d G S = sum_n C[t,g(h),n] P[t,h,n].
// Five launches:
//  1. prep: H_in^T split into three bf16 parts hi + mid + lo ([B,H,n,d]); then e
//     transposed to [B,H,T] by a kernel of its own (64-token x 64-head tiles);
//  2. unit kernel: per head slice of 64 channels walking a token block, the block's
//     dH_in partial (G e split into bf16 hi + lo, times C) on MFMA;
//  3. dC kernel: per 256-token tile of one group, every head's P^T = H_in^T G^T on
//     MFMA (the three parts of H_in^T staged per 64-channel chunk in LDS), dC += e P
//     and dcumA = e sum_n C P (C of the tile's tokens in registers);
//  4. reduce: dH_in = sum of the block partials + the state term, and the state
//     term of dcumA.
// Every fp32 result is formed from exact bf16 x bf16 products with fp32
// accumulation (the hi/lo splits carry ~16 mantissa bits of the fp32 factors, three
// parts ~24: dcumA contracts P against C once more, and a two-part residual of 2^-18
// times that cancellation would miss 1e-4).
#include <mutex>
#include <type_traits>

#include "rmx_kernels.h"

namespace rmx {

struct MambaBwdArgs {
  const uint16_t* gy;
  const float* ghf;  // may be null: no gradient reaches h_final_out
  const uint16_t* C;
  const float* cum_A;
  const float* h_prev;
  const int32_t* seq_idx;
  uint16_t* gC;
  float* g_cumA;
  float* g_hprev;
  float* part;      // [ntb][B][H][d][n] dH_in partials of the unit kernel's token blocks
  uint16_t* ht_hi;  // [B][H][n][d]
  uint16_t* ht_mid;
  uint16_t* ht_lo;
  float* eT;        // [B][H][T]
  int batch, T, nheads, head_dim, ngroups, d_state, ntb;
};

constexpr int kMambaBwdTokensPerWg = 4096;  // unit kernel token block
constexpr int kMambaBwdCTokens = 256;       // dC kernel token tile (8 waves x 32)

// Chunk swizzle for LDS tiles read both row-wise (8 consecutive rows, one
// 16-byte chunk each) and by ds_read_b64_tr_b16 (4 consecutive rows, one
// 32-byte chunk pair each): f(row) mod 8 differs over any 8 rows and f(row) / 2
// differs over any 4 aligned rows, so both reads hit 8 distinct 16-byte bank
// slots of a 128-byte window (rows of 128 or 256 bytes).
__device__ __forceinline__ int swz_pair(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

// Transposed operand read (k = 8*hl .. 8*hl+7 <-> tile rows r0 + 8*hl + 0..7,
// column c0 + l32) from a tile with 16-byte chunks swizzled by swz_pair and
// RB-byte rows. Lane (x = (lane >> 4) & 1, m = lane & 15) addresses row
// r0 + 8*hl + 4*t + (m >> 2), columns c0 + 16x + 4(m & 3) .. + 3.
template <int RB>
__device__ __forceinline__ bf16x8 tr_read(const uint8_t* tile, int r0, int c0, int lane) {
  const int hl = lane >> 5, m = lane & 15, x = (lane >> 4) & 1;
  u32x2 part[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = r0 + 8 * hl + 4 * t + (m >> 2);
    const int col = c0 + 16 * x + 4 * (m & 3);  // element column, 8-byte aligned
    const int chunk = col >> 3;
    const uint8_t* p = tile + r * RB + 16 * (chunk ^ swz_pair(r)) + 2 * (col & 7);
    part[t] = lds_read_tr(reinterpret_cast<const uint16_t*>(p));
  }
  return join_bf16x8(part[0], part[1]);
}

__device__ __forceinline__ void split8(const float* v, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = cvt_pk_bf16(v[2 * i], v[2 * i + 1]);
    l[i] = cvt_pk_bf16(v[2 * i] - __uint_as_float(h[i] << 16),
                       v[2 * i + 1] - __uint_as_float(h[i] & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

// ---------------------------------------------------------------------------
// 1. prep: grid (H, B), 256 threads. H_in[b,h] ([d][n] fp32) -> [n][d] bf16 hi, mid, lo
// through LDS. (eT comes from its own kernel, below.)
template <int HD, int N>
__global__ __launch_bounds__(256) void mamba2_bwd_prep_kernel(const MambaBwdArgs a) {
  __shared__ float st[HD][N + 1];
  const int h = blockIdx.x, bb = blockIdx.y, tid = threadIdx.x;
  const int H = a.nheads;
  const int64_t hb = ((int64_t)bb * H + h) * HD * N;
  for (int i = tid; i < HD * N; i += 256) st[i / N][i % N] = a.h_prev[hb + i];
  __syncthreads();
  // thread -> (n, 8 consecutive d): 16-byte hi, mid and lo stores
  for (int i = tid; i < N * (HD / 8); i += 256) {
    const int n = i / (HD / 8), d0 = 8 * (i % (HD / 8));
    float v[8], r[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = st[d0 + k][n];
    bf16x8 hi, mid, lo, unused;
    split8(v, hi, mid);
    const u32x4 h4 = __builtin_bit_cast(u32x4, hi), m4 = __builtin_bit_cast(u32x4, mid);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[2 * k] = v[2 * k] - __uint_as_float(h4[k] << 16) - __uint_as_float(m4[k] << 16);
      r[2 * k + 1] = v[2 * k + 1] - __uint_as_float(h4[k] & 0xffff0000u) -
                     __uint_as_float(m4[k] & 0xffff0000u);
    }
    split8(r, lo, unused);
    *reinterpret_cast<bf16x8*>(a.ht_hi + hb + (int64_t)n * HD + d0) = hi;
    *reinterpret_cast<bf16x8*>(a.ht_mid + hb + (int64_t)n * HD + d0) = mid;
    *reinterpret_cast<bf16x8*>(a.ht_lo + hb + (int64_t)n * HD + d0) = lo;
  }
}

// 1b. eT[b,h,t] = mask * exp(cumA[b,t,h]): grid (ceil(T / 64), B), 256 threads; a tile of
// 64 tokens x 64 heads goes through LDS, so the reads take whole token rows of cum_A and
// the writes whole 256-byte runs of eT (one workgroup per head read cum_A 4 bytes per
// token, 256 bytes apart: 43 -> 27 us for both kernels at 8 x 8192 tokens x 64 heads).
__global__ __launch_bounds__(256) void mamba2_bwd_et_kernel(const MambaBwdArgs a) {
  __shared__ float st[64][65];
  const int t0 = blockIdx.x * 64, bb = blockIdx.y, tid = threadIdx.x;
  const int H = a.nheads, T = a.T;
  for (int h0 = 0; h0 < H; h0 += 64) {
    const int hn = H - h0 < 64 ? H - h0 : 64;
    for (int i = tid; i < 64 * 64; i += 256) {
      const int tt = i >> 6, hh = i & 63, t = t0 + tt;
      float v = 0.f;
      if (t < T && hh < hn) {
        const int64_t tok = (int64_t)bb * T + t;
        const bool live = !a.seq_idx || a.seq_idx[tok] == 0;
        v = live ? expf(a.cum_A[tok * H + h0 + hh]) : 0.f;
      }
      st[tt][hh] = v;
    }
    __syncthreads();
    for (int i = tid; i < 64 * 64; i += 256) {
      const int hh = i >> 6, tt = i & 63, t = t0 + tt;
      if (t < T && hh < hn) a.eT[((int64_t)bb * H + h0 + hh) * T + t] = st[tt][hh];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// 2. unit kernel. A unit is 64 channels of one head (head_dim 64: one head,
// 128: half a head); a workgroup holds 4 units of heads in one C group and
// walks kMambaBwdTokensPerWg tokens, 32 per step, with the forward's DMA rings
// (C and aux shared, G per wave, two steps ahead). Per wave and step:
//   dH^T partial (64 ch x N) += (G e)^T C  4 N/32 MFMAs per 16 tokens: A = G^T e
//       split into hi/lo (transposed reads of the G stage), B = C (transposed
//       reads of the C stage)
// The dH partial (128 fp32 per lane at N = 128) stays in registers for the
// whole walk: one wave per SIMD, accumulators in AGPRs.
template <int N>
struct MambaBwdUnitCfg {
  static constexpr int SL = 64, NDB = 2, CHC = N / 8, CHO = 8, NI = 4, NB = N / 32;
  static constexpr int ND = N / 64;            // C DMA instructions per wave and step
  static constexpr int CS = 32 * N * 2;        // C stage bytes (= ND * 4 KB)
  static constexpr int OS = 32 * SL * 2;       // G stage bytes per wave
  static constexpr int XS = 2 * 4 * 256;       // cum_A + seq_idx stage
  static constexpr int NDMA = ND + NI + 2;
  static constexpr int EW = 4 * 32 * 4;        // e of the step's tokens, per wave
  static constexpr int LDS = 3 * CS + 4 * 3 * OS + 3 * XS + EW;
};

template <int N>
__global__ __launch_bounds__(256, 1) void mamba2_bwd_unit_kernel(const MambaBwdArgs a, const int nug) {
  using F = MambaBwdUnitCfg<N>;
  constexpr int SL = F::SL, NDB = F::NDB, CHC = F::CHC, CHO = F::CHO, NI = F::NI;
  constexpr int NB = F::NB, ND = F::ND, CS = F::CS, OS = F::OS, XS = F::XS;
  __shared__ __attribute__((aligned(16))) uint8_t smem[F::LDS];
  uint8_t* const sC = smem;
  uint8_t* const sO = smem + 3 * CS;
  uint8_t* const sX = sO + 4 * 3 * OS;
  float* const sE = reinterpret_cast<float*>(sX + 3 * XS);  // [4 waves][32]

  const int ntb = a.ntb;
  int id = blockIdx.x;
  const int nwg = gridDim.x;
  if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
  const int ug = id % nug, rest = id / nug;
  const int tb = rest % ntb, bb = rest / ntb;
  const int T = a.T, H = a.nheads, HD = a.head_dim, G = a.ngroups;
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int uph = HD / SL, hpw = 4 / uph, h0 = 4 * ug / uph;
  const int unit = 4 * ug + wave, h = unit / uph, sl = unit % uph, hw = wave / uph;
  const int g = h0 / (H / G);
  const int tbeg = tb * kMambaBwdTokensPerWg;
  const int tend = tbeg + kMambaBwdTokensPerWg < T ? tbeg + kMambaBwdTokensPerWg : T;
  const int nstep = (tend - tbeg + 31) / 32;
  const int64_t HHD = (int64_t)H * HD;

  const int cstride = G * N * 2, ostride = (int)(HHD * 2);
  const uint32_t cspan = span_bytes(T, cstride, N * 2), aspan = (uint32_t)T * (uint32_t)H * 4u;
  const i32x4 rC = make_rsrc(a.C + ((int64_t)bb * T * G + g) * N, cspan);
  const i32x4 rO = make_rsrc(a.gy + (int64_t)bb * T * HHD + (int64_t)h * HD + sl * SL,
                             span_bytes(T, ostride, SL * 2));
  const i32x4 rA = make_rsrc(a.cum_A + (int64_t)bb * T * H, aspan);
  const uint32_t sspan = a.seq_idx ? (uint32_t)T * 4u : 0u;
  const i32x4 rS = make_rsrc(a.seq_idx ? (const void*)(a.seq_idx + (int64_t)bb * T) : (const void*)a.cum_A,
                             sspan);
  const uint32_t ldsC = lds_addr(sC), ldsO = lds_addr(sO + wave * 3 * OS), ldsX = lds_addr(sX);
  const int xa_tok = 8 * wave + lane / hpw, xa_head = h0 + lane % hpw;
  const bool xa_live = lane < 8 * hpw;

  auto issue = [&](int st, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int p = (i * 4 + wave) * 64 + lane, row = p / CHC, pc = p % CHC;
      dma16_async(rC, ldsC + st * CS + (i * 4 + wave) * 1024,
                  (t0 + row) * cstride + 16 * (pc ^ swz_pair(row)));
    }
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int p = 64 * k + lane, row = p / CHO, pc = p % CHO;
      dma16_async(rO, ldsO + st * OS + 1024 * k, (t0 + row) * ostride + 16 * (pc ^ swz_pair(row)));
    }
    dma4_async(rA, ldsX + st * XS + 256 * wave,
               xa_live ? (t0 + xa_tok) * (H * 4) + 4 * xa_head : (int)aspan);
    dma4_async(rS, ldsX + st * XS + 1024 + 256 * wave, lane < 8 ? (t0 + 8 * wave + lane) * 4 : (int)sspan);
  };

  f32x16 gh[NDB][NB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) gh[db][nb] = zero16();

  issue(0, tbeg);
  if (nstep > 1) issue(1, tbeg + 32);
  float* const ew = sE + 32 * wave;
  for (int s = 0; s < nstep; ++s) {
    // at the top of step s, only step s + 1's DMA was issued after step s's
    if (s + 1 < nstep)
      wait_vm_barrier<F::NDMA>();
    else
      wait_vm_barrier<0>();
    if (s + 2 < nstep) issue((s + 2) % 3, tbeg + 32 * (s + 2));
    const int st = s % 3, t0 = tbeg + 32 * s;
    const uint8_t* cst = sC + st * CS;
    const uint8_t* ost = sO + (wave * 3 + st) * OS;

    // e of token l32 (0 past the block end: those rows belong to the next block)
    const uint8_t* xst = sX + st * XS;
    const float ca = reinterpret_cast<const float*>(xst)[64 * (l32 >> 3) + (l32 & 7) * hpw + hw];
    const int sq = reinterpret_cast<const int32_t*>(xst + 1024)[64 * (l32 >> 3) + (l32 & 7)];
    const bool live = t0 + l32 < tend;
    const float e = (sq != 0 || !live) ? 0.f : expf(ca);
    if (hl == 0) ew[l32] = e;

    // dH^T += (G e)^T C over the step's 32 tokens (two k-steps of 16)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const f32x4 e0 = *reinterpret_cast<const f32x4*>(ew + 16 * kk + 8 * hl);
      const f32x4 e1 = *reinterpret_cast<const f32x4*>(ew + 16 * kk + 8 * hl + 4);
      const float e8[8] = {e0[0], e0[1], e0[2], e0[3], e1[0], e1[1], e1[2], e1[3]};
      bf16x8 gah[NDB], gal[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const u32x4 gt = __builtin_bit_cast(u32x4, tr_read<CHO * 16>(ost, 16 * kk, 32 * db, lane));
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = __uint_as_float(gt[i] << 16) * e8[2 * i];
          v[2 * i + 1] = __uint_as_float(gt[i] & 0xffff0000u) * e8[2 * i + 1];
        }
        split8(v, gah[db], gal[db]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const bf16x8 cb = tr_read<CHC * 16>(cst, 16 * kk, 32 * nb, lane);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          gh[db][nb] = mfma32(gah[db], cb, gh[db][nb]);
          gh[db][nb] = mfma32(gal[db], cb, gh[db][nb]);
        }
      }
    }
  }

  // ---- the block's dH_in partial: lane (hl, l32) reg r of (db, nb) holds
  // channel 32 db + 8 (r / 4) + 4 hl + r % 4 (A rows unpermuted), state n = 32 nb + l32
  float* dst = a.part + ((((int64_t)tb * a.batch + bb) * H + h) * HD + (int64_t)sl * SL) * N;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dst[(int64_t)(32 * db + c_row(hl, r)) * N + 32 * nb + l32] = gh[db][nb][r];
}

// ---------------------------------------------------------------------------
// 4. reduce: grid (H, B), 256 threads. dH_in = sum of the block partials
// (+ exp(cumA[T-1]) Gs when the state is updated), and the state's term of
// dcumA[T-1] = exp(cumA[T-1]) sum Gs H_in (added after the dC kernel).
template <int HD, int N>
__global__ __launch_bounds__(256) void mamba2_bwd_reduce_kernel(const MambaBwdArgs a) {
  __shared__ float red[4];
  const int h = blockIdx.x, bb = blockIdx.y, tid = threadIdx.x;
  const int H = a.nheads, T = a.T;
  bool fresh_last = false;
  if (a.seq_idx)
    for (int b2 = 0; b2 < a.batch; ++b2) fresh_last |= a.seq_idx[(int64_t)b2 * T + T - 1] != 0;
  const bool upd = a.ghf && !fresh_last;
  const float el = upd ? expf(a.cum_A[((int64_t)bb * T + T - 1) * H + h]) : 0.f;
  const int64_t hb = ((int64_t)bb * H + h) * HD * N;
  const int64_t pstride = (int64_t)a.batch * H * HD * N;
  float dot = 0.f;
  for (int i = 4 * tid; i < HD * N; i += 4 * 256) {
    f32x4 s = *reinterpret_cast<const f32x4*>(a.part + hb + i);
    for (int k = 1; k < a.ntb; ++k) s += *reinterpret_cast<const f32x4*>(a.part + k * pstride + hb + i);
    if (upd) {
      const f32x4 gs = *reinterpret_cast<const f32x4*>(a.ghf + hb + i);
      const f32x4 hp = *reinterpret_cast<const f32x4*>(a.h_prev + hb + i);
      s += el * gs;
      dot += gs[0] * hp[0] + gs[1] * hp[1] + gs[2] * hp[2] + gs[3] * hp[3];
    }
    *reinterpret_cast<f32x4*>(a.g_hprev + hb + i) = s;
  }
  if (upd) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = dot;
    __syncthreads();
    if (tid == 0) a.g_cumA[((int64_t)bb * T + T - 1) * H + h] += el * (red[0] + red[1] + red[2] + red[3]);
  }
}

// ---------------------------------------------------------------------------
// 3. dC kernel: one workgroup = 8 waves (two per SIMD) x 32 tokens of one (batch,
// group); the contraction runs over the group's (head, channel) pairs in chunks of 64
// channels (one head at head_dim 64, half a head at 128). Per chunk and wave:
//   P^T (N x 32 tok) = H_in^T G^T   A = H_in^T rows (hi, mid and lo, LDS, sigma-
//                                    permuted), B = G rows (LDS)   3 N/32 MFMAs per
//                                    k-step of 16 channels
//   dC^T += e P^T                   (lane = token: one e per lane and chunk)
//   q    += sum_n C P               (C of the lane's token and rows, registers)
// and after a head's last chunk dcumA[t,h] = e q (both lane halves' rows). The next
// chunk's H_in^T (shared) and G (per wave) tiles load by DMA during the current one,
// its e (from the transposed eT rows) into registers.
template <int N>
struct MambaBwdCCfg {
  static constexpr int NW = 8;                 // waves, 32 tokens each
  static constexpr int NB = N / 32, CH = 8;    // 64 channels = 8 chunks per row
  static constexpr int HS = 3 * N * 128;       // H_in^T chunk stage: hi, mid, lo, N rows x 128 B
  static constexpr int GS = 32 * 128;          // G chunk stage per wave: 32 tokens x 128 B
  static constexpr int NDH = HS / (1024 * NW); // H DMA instructions per wave
  static constexpr int LDS = 2 * HS + NW * 2 * GS;
  static_assert(HS % (1024 * NW) == 0 && (N * CH / 64) % NW == 0,
                "a plane is whole DMA instructions of every wave");
};

template <int N>
__global__ __launch_bounds__(512, 1) void mamba2_bwd_c_kernel(const MambaBwdArgs a, const int ntt) {
  using F = MambaBwdCCfg<N>;
  constexpr int NW = F::NW, NB = F::NB, CH = F::CH, HS = F::HS, GS = F::GS, NDH = F::NDH;
  __shared__ __attribute__((aligned(16))) uint8_t smem[F::LDS];
  uint8_t* const sH = smem;                 // [2][HS]: hi [N][64], mid, lo
  uint8_t* const sG = smem + 2 * HS;        // [NW waves][2][GS]

  int id = blockIdx.x;
  const int nwg = gridDim.x;
  if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
  const int tt = id % ntt, rest = id / ntt;
  const int g = rest % a.ngroups, bb = rest / a.ngroups;
  const int T = a.T, H = a.nheads, HD = a.head_dim;
  const int hpg = H / a.ngroups, cph = HD / 64, nchunk = hpg * cph;
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = tt * kMambaBwdCTokens;
  const int t = t0 + 32 * wave + l32;  // this lane's token
  const int64_t HHD = (int64_t)H * HD;
  const int ostride = (int)(HHD * 2);

  const i32x4 rG = make_rsrc(a.gy + (int64_t)bb * T * HHD, span_bytes(T, ostride, (int)(HHD * 2)));
  const uint32_t ldsH = lds_addr(sH), ldsG = lds_addr(sG + wave * 2 * GS);
  // chunk j: head hg = g * hpg + j / cph, channels 64 (j % cph) .. + 63
  auto issue = [&](int st, int j) __attribute__((always_inline)) {
    const int hg = g * hpg + j / cph, c0 = 64 * (j % cph);
    const int64_t ho = ((int64_t)bb * H + hg) * N * HD + c0;
    const i32x4 rh = make_rsrc(a.ht_hi + ho, span_bytes(N, HD * 2, 128));
    const i32x4 rm = make_rsrc(a.ht_mid + ho, span_bytes(N, HD * 2, 128));
    const i32x4 rl = make_rsrc(a.ht_lo + ho, span_bytes(N, HD * 2, 128));
#pragma unroll
    for (int i = 0; i < NDH; ++i) {
      const int n = i * NW + wave;                 // 1 KB DMA instruction of the stage
      const int plane = n * 64 / (N * CH);         // one plane per instruction
      const int q = n * 64 + lane - plane * N * CH, row = q / CH, pc = q % CH;
      const int off = row * (HD * 2) + 16 * (pc ^ swz_row(row));
      dma16_async(plane == 0 ? rh : (plane == 1 ? rm : rl), ldsH + st * HS + n * 1024, off);
    }
    // g_y with the non-temporal policy: its last reader (0.463 -> 0.450 ms per backward at
    // 8 x 8192 tokens x 64 heads; the same in the unit kernel, an earlier reader, was slower)
#pragma unroll
    for (int k = 0; k < GS / 1024; ++k) {
      const int p = 64 * k + lane, row = p / CH, pc = p % CH;
      dma16_async_nt(rG, ldsG + st * GS + 1024 * k,
                     (t0 + 32 * wave + row) * ostride + 2 * (hg * HD + c0) + 16 * (pc ^ (row & 7)));
    }
  };
  // e of the lane's token for the head of chunk j (0 past the sequence end)
  auto load_e = [&](int j) __attribute__((always_inline)) -> float {
    const float* et = a.eT + ((int64_t)bb * H + g * hpg + j / cph) * T;
    return t < T ? et[t] : 0.f;
  };

  // C of the lane's P rows n = 32 nb + 16 half + 8 hl .. + 7
  u32x4 cv[NB][2];
  {
    const uint16_t* crow = a.C + (((int64_t)bb * T + (t < T ? t : 0)) * a.ngroups + g) * N + 8 * hl;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int half = 0; half < 2; ++half)
        cv[nb][half] = t < T ? *reinterpret_cast<const u32x4*>(crow + 32 * nb + 16 * half) : u32x4{};
  }

  f32x16 acc[NB];  // dC^T: [n block]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = zero16();
  float q = 0.f;

  issue(0, 0);
  float ecur = load_e(0), enext = 0.f;
  const int arow = sigma(l32);
  for (int j = 0; j < nchunk; ++j) {
    wait_vm_barrier<0>();
    if (j + 1 < nchunk) {
      issue((j + 1) & 1, j + 1);
      enext = load_e(j + 1);
    }
    const uint8_t* hst = sH + (j & 1) * HS;
    const uint8_t* gst = sG + (wave * 2 + (j & 1)) * GS;
    f32x16 p[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) p[nb] = zero16();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 gb =
          *reinterpret_cast<const bf16x8*>(gst + l32 * 128 + 16 * ((2 * ks + hl) ^ (l32 & 7)));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int row = 32 * nb + arow;
        const int off = row * 128 + 16 * ((2 * ks + hl) ^ swz_row(row));
#pragma unroll
        for (int part = 0; part < 3; ++part)
          p[nb] = mfma32(*reinterpret_cast<const bf16x8*>(hst + part * N * 128 + off), gb, p[nb]);
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      acc[nb] += ecur * p[nb];
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t c2 = cv[nb][half][w];
          q = fmaf(__uint_as_float(c2 << 16), p[nb][8 * half + 2 * w], q);
          q = fmaf(__uint_as_float(c2 & 0xffff0000u), p[nb][8 * half + 2 * w + 1], q);
        }
    }
    if (j % cph == cph - 1) {  // the head's last chunk: dcumA of its tokens
      const float tot = q + xhalf(q);
      if (hl == 0 && t < T) a.g_cumA[((int64_t)bb * T + t) * H + g * hpg + j / cph] = ecur * tot;
      q = 0.f;
    }
    ecur = enext;
  }

  // dC[b, t, g, n]: lane (hl, l32) reg r of nb = token 32 wave + l32,
  // n = 32 nb + 16 (r / 8) + 8 hl + r % 8 (sigma-permuted A rows)
  if (t < T) {
    uint16_t* dst = a.gC + (((int64_t)bb * T + t) * a.ngroups + g) * N + 8 * hl;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = acc[nb][8 * half + i];
        *reinterpret_cast<bf16x8*>(dst + 32 * nb + 16 * half) = pack8_hw(v);
      }
  }
}

// ---------------------------------------------------------------------------
// Workspace of the allocation-free entry point (rmx_mamba2_cp_correction_bwd_noalloc):
// a file-scope device array, one per GPU the library runs on, held until the process
// ends. In host code `scratch` names a host-side stand-in, not device memory: host code
// only ever uses the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[RMX_MAMBA2_BWD_SCRATCH_MAX];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` per device
}  // namespace

// The current device's copy of `scratch`, looked up once per device (with that device
// current) and kept for the rest of the process.
hipError_t mamba2_bwd_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

size_t mamba2_bwd_workspace(int batch, int T, int nheads, int head_dim, int d_state) {
  const size_t state = (size_t)batch * nheads * head_dim * d_state;
  const size_t ntb = (size_t)((T + kMambaBwdTokensPerWg - 1) / kMambaBwdTokensPerWg);
  return ntb * state * 4 + 3 * state * 2 + (size_t)batch * nheads * T * 4 + 256;
}

hipError_t launch_mamba2_correction_bwd(const uint16_t* gy, const float* ghf, const uint16_t* C,
                                        const float* cum_A, const float* h_prev,
                                        const int32_t* seq_idx, uint16_t* gC, float* g_cumA,
                                        float* g_hprev, void* workspace, int batch, int T,
                                        int nheads, int head_dim, int ngroups, int d_state,
                                        hipStream_t stream) {
  const size_t state = (size_t)batch * nheads * head_dim * d_state;
  const int ntb = (T + kMambaBwdTokensPerWg - 1) / kMambaBwdTokensPerWg;
  uint8_t* ws = reinterpret_cast<uint8_t*>(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  MambaBwdArgs a{gy, ghf, C, cum_A, h_prev, seq_idx, gC, g_cumA, g_hprev,
                 reinterpret_cast<float*>(ws),
                 reinterpret_cast<uint16_t*>(ws + ntb * state * 4),
                 reinterpret_cast<uint16_t*>(ws + ntb * state * 4 + state * 2),
                 reinterpret_cast<uint16_t*>(ws + ntb * state * 4 + state * 4),
                 reinterpret_cast<float*>(ws + ntb * state * 4 + state * 6),
                 batch, T, nheads, head_dim, ngroups, d_state, ntb};
  const int uph = head_dim / 64, nug = nheads * uph / 4;
  const int ntt = (T + kMambaBwdCTokens - 1) / kMambaBwdCTokens;
  auto run = [&](auto hd, auto n) {
    constexpr int HDc = decltype(hd)::value, Nc = decltype(n)::value;
    hipLaunchKernelGGL((mamba2_bwd_prep_kernel<HDc, Nc>), dim3(nheads, batch), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(mamba2_bwd_et_kernel, dim3((unsigned)((T + 63) / 64), batch), dim3(256), 0,
                       stream, a);
    hipLaunchKernelGGL((mamba2_bwd_unit_kernel<Nc>), dim3((unsigned)(nug * ntb * batch)), dim3(256), 0,
                       stream, a, nug);
    // the dC kernel writes dcumA, to which the reduce then adds the state term
    hipLaunchKernelGGL((mamba2_bwd_c_kernel<Nc>), dim3((unsigned)(ntt * ngroups * batch)),
                       dim3(64 * MambaBwdCCfg<Nc>::NW), 0, stream, a, ntt);
    hipLaunchKernelGGL((mamba2_bwd_reduce_kernel<HDc, Nc>), dim3(nheads, batch), dim3(256), 0, stream, a);
    return hipGetLastError();
  };
  if (head_dim == 64)
    return d_state == 64 ? run(std::integral_constant<int, 64>{}, std::integral_constant<int, 64>{})
                         : run(std::integral_constant<int, 64>{}, std::integral_constant<int, 128>{});
  return d_state == 64 ? run(std::integral_constant<int, 128>{}, std::integral_constant<int, 64>{})
                       : run(std::integral_constant<int, 128>{}, std::integral_constant<int, 128>{});
}

}  // namespace rmx
