// Mamba2 context-parallel output correction for gfx950.
//
// Reference: `mamba2_cp_correction` (strategies/mamba.py:101-139). A rank whose
// shard starts with a carried-in SSM state H_in (= h_prev, the exact prefix of
// the earlier ranks' chunk states, :68-98) adds its analytic contribution:
//   y[b,t,h,:] = out[b,t,h,:] + bf16( e^{cumA[b,t,h]} * sum_n C[b,t,g(h),n] H_in[b,h,:,n] )
//   h_final[b,h] += e^{cumA[b,T-1,h]} * H_in[b,h]
// with g(h) = h / (nheads / ngroups) (repeat_interleave, :121); tokens whose
// seq_idx != 0 (a packed sequence that starts fresh on this rank) get no
// correction (:124-126), and no state is updated when the last token of any
// batch row is such a token (the batch-wide test of :131-135). The bf16
// rounding of the correction before the add mirrors `delta_y.to(out.dtype)`
// followed by the bf16 add (:128-129).
//
// Per head the correction is a (T x d_state) x (d_state x head_dim) product, so
// it runs on MFMA (v_mfma_f32_32x32x16_bf16) as dY^T = H_in C^T: A = H_in rows
// (head_dim x d_state, staged in LDS once per workgroup as bf16 hi + lo parts,
// so the product carries about 16 mantissa bits; C is bf16 and exact), B = C^T
// (a lane holds one token's C row). The A rows are sigma-permuted (rmx_common.h),
// so a lane ends up holding two runs of 8 consecutive head_dim channels of ONE
// token: its slice of out / y moves as 16-byte accesses, and e^{cumA} and
// seq_idx are one value per lane. One workgroup = 4 waves walks 1024 tokens of
// one (batch, head), 32 tokens per wave and step. The kernel is HBM-bound on
// reading `out` and writing `y` (4 bytes per element).
#include <algorithm>
#include <type_traits>

#include "rmx_kernels.h"

namespace rmx {

struct MambaCorrArgs {
  const uint16_t* out;
  uint16_t* y;
  const float* h_final;
  float* h_final_out;
  const uint16_t* C;
  const float* cum_A;
  const float* h_prev;
  const int32_t* seq_idx;
  int batch, T, nheads, head_dim, ngroups, d_state;
};

constexpr int kMambaTokensPerWg = 1024;

template <int HD, int N>
__global__ __launch_bounds__(256) void mamba2_correction_kernel(const MambaCorrArgs a) {
  constexpr int NDB = HD / 32;  // 32-row blocks of dY^T (head_dim channels)
  constexpr int NS = N / 16;    // k-steps
  constexpr int CHR = N / 8;    // 16-byte chunks per H row
  // 16-byte chunks of an LDS row are XOR-swizzled by (row & 7) when a row has a
  // multiple of 8 chunks, so the A-operand reads of 32 rows spread over the banks
  constexpr int SWM = CHR % 8 == 0 ? 7 : 0;
  __shared__ __attribute__((aligned(16))) uint16_t shi[HD * N];
  __shared__ __attribute__((aligned(16))) uint16_t slo[HD * N];
  // heads vary fastest over the grid, so the workgroups running together read
  // and write whole token rows of out / y (all heads), not 128-byte pieces
  const int h = blockIdx.x, tb = blockIdx.y, bb = blockIdx.z;
  const int T = a.T, H = a.nheads;
  const int g = h / (H / a.ngroups);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int64_t hbase = ((int64_t)bb * H + h) * HD * N;

  // ---- the state update, once per (batch, head), by the first token block
  if (tb == 0) {
    // the reference tests seq_idx[:, -1].any() over the whole batch (:131)
    bool fresh_last = false;
    if (a.seq_idx)
      for (int b2 = 0; b2 < (int)gridDim.z; ++b2)
        fresh_last |= a.seq_idx[(int64_t)b2 * T + T - 1] != 0;
    const float e = fresh_last ? 0.f : expf(a.cum_A[((int64_t)bb * T + T - 1) * H + h]);
    for (int i = 4 * tid; i < HD * N; i += 4 * 256) {
      const f32x4 hf = *reinterpret_cast<const f32x4*>(a.h_final + hbase + i);
      const f32x4 hp = *reinterpret_cast<const f32x4*>(a.h_prev + hbase + i);
      *reinterpret_cast<f32x4*>(a.h_final_out + hbase + i) = hf + hp * e;
    }
  }

  // ---- H_in -> LDS as bf16 hi and lo planes, [HD][N] each
  for (int c = tid; c < HD * CHR; c += 256) {
    const int row = c / CHR, ch = c % CHR;
    const float* src = a.h_prev + hbase + (int64_t)row * N + 8 * ch;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(src);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(src + 4);
    const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    float hv[8], lv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hv[i] = bf2f(f2bf(xv[i]));
      lv[i] = xv[i] - hv[i];
    }
    const int off = row * N + 8 * (ch ^ (row & SWM));
    *reinterpret_cast<bf16x8*>(shi + off) = pack8_hw(hv);
    *reinterpret_cast<bf16x8*>(slo + off) = pack8_hw(lv);
  }
  __syncthreads();

  // ---- token tiles: the C row, out slice and e^{cumA} of tile i + 1 load while
  // tile i runs its MFMAs and epilogue
  const int arow = sigma(l32);  // A operand: H row sigma(l32) + 32 db, k = 16 ks + 8 hl ..
  const int64_t HDt = (int64_t)H * HD;
  const int tbeg = tb * kMambaTokensPerWg;
  const int tend = tbeg + kMambaTokensPerWg < T ? tbeg + kMambaTokensPerWg : T;
  struct Tile {
    bf16x8 c[NS];         // this lane's token: C[t, g, 16 ks + 8 hl .. + 7]
    u32x4 o[NDB][2];      // out[t, h, 32 db + 16 half + 8 hl .. + 7]
    float e;              // e^{cumA[t, h]} (0 for a fresh packed sequence)
  };
  auto load = [&](int t0, Tile& tl) {
    const int t = t0 + l32 < tend ? t0 + l32 : tend - 1;
    const int64_t tok = (int64_t)bb * T + t;
    const uint16_t* crow = a.C + (tok * a.ngroups + g) * N + 8 * hl;
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) tl.c[ks] = __builtin_bit_cast(bf16x8, ld16(crow + 16 * ks));
    const uint16_t* orow = a.out + tok * HDt + (int64_t)h * HD + 8 * hl;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) tl.o[db][half] = ld16(orow + 32 * db + 16 * half);
    tl.e = a.cum_A[tok * H + h];
    if (a.seq_idx && a.seq_idx[tok] != 0) tl.e = kNegInf;  // e^{-inf} = 0: no correction
  };
  auto compute = [&](int t0, const Tile& tl) {
    // re-read the H operands from LDS every tile: hoisted out of the loop they
    // would hold 4*NS*NDB*2 registers and leave one wave per SIMD, too few loads
    // in flight for an HBM-bound kernel
    asm volatile("" ::: "memory");
    f32x16 acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = zero16();
#pragma unroll
    for (int ks = 0; ks < NS; ++ks)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int row = arow + 32 * db;
        const int off = row * N + 8 * ((2 * ks + hl) ^ (row & SWM));
        acc[db] = mfma32(*reinterpret_cast<const bf16x8*>(shi + off), tl.c[ks], acc[db]);
        acc[db] = mfma32(*reinterpret_cast<const bf16x8*>(slo + off), tl.c[ks], acc[db]);
      }
    const int t = t0 + l32;
    if (t >= tend) return;
    const float e = expf(tl.e);
    uint16_t* yrow = a.y + ((int64_t)bb * T + t) * HDt + (int64_t)h * HD + 8 * hl;
    // lane (hl, l32), reg r of block db: channel 32 db + 16 (r / 8) + 8 hl + r % 8
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const u32x4 ov = tl.o[db][half];
        u32x4 yv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dy0 = bf2f(f2bf(acc[db][8 * half + 2 * i] * e));
          const float dy1 = bf2f(f2bf(acc[db][8 * half + 2 * i + 1] * e));
          const float o0 = __uint_as_float(ov[i] << 16), o1 = __uint_as_float(ov[i] & 0xffff0000u);
          yv[i] = pack_bf2(o0 + dy0, o1 + dy1);
        }
        st16(yrow + 32 * db + 16 * half, yv);
      }
  };
  // two tile buffers used alternately (a copy of in-flight loads would wait for them)
  int t0 = tbeg + 32 * wave;
  if (t0 >= tend) return;
  Tile ta, tb2;
  load(t0, ta);
  while (true) {
    const bool more1 = t0 + 128 < tend;
    if (more1) load(t0 + 128, tb2);
    compute(t0, ta);
    if (!more1) break;
    t0 += 128;
    const bool more2 = t0 + 128 < tend;
    if (more2) load(t0 + 128, ta);
    compute(t0, tb2);
    if (!more2) break;
    t0 += 128;
  }
}

// ---------------------------------------------------------------------------
// Streaming variant for d_state <= 128 (the production Mamba2 shapes). A
// "unit" is SL = min(head_dim, 64) channels of one head; a workgroup holds 4
// units of heads that share one C group and walks kMambaFastTokensPerWg tokens,
// 32 per step. Per wave:
//  * H_in of its unit lives in registers for the whole walk, as the MFMA A
//    operands (bf16 hi + lo, 2 * NDB * NS * 4 VGPRs). It is read once with
//    coalesced 16-byte loads, split into hi + lo and transposed through LDS into
//    the operand layout (a direct operand-layout load would touch 32 cache lines
//    per instruction);
//  * the step's C rows, cum_A values (of the workgroup's heads) and seq_idx
//    values are shared by the 4 waves, its out rows are its own; all arrive by
//    LDS DMA two steps ahead, in 3-stage rings, and every wave issues the same
//    number of DMA instructions per step, so the vmcnt budget is static;
//  * dY^T = H_in C^T runs on MFMA with sigma-permuted A rows, so a lane holds
//    runs of 8 consecutive channels of one token; out + dY is formed in place in
//    the out stage (same 16-byte slots), then re-read row-wise and stored as
//    full 128-byte lines through a buffer resource that drops rows past the
//    range end. out is read and y written with the non-temporal cache policy
//    (each byte is touched once): 0.215 -> 0.203 ms at 8 x 8192 tokens x 64 heads.
// Workgroups are renumbered so that consecutive logical ids land on the same
// XCD, unit groups fastest: the workgroups running together on an XCD cover
// whole token rows of out / y (every head) for a few token blocks of one batch
// row, so their HBM traffic spreads over all channels, each C tile is fetched
// once and re-read from that XCD's L2, and so is each unit's H_in. 2048 tokens
// per workgroup amortise the H_in prologue (and at configs[4] give exactly two
// resident workgroups per CU).
constexpr int kMambaFastTokensPerWg = 2048;

// 16-byte chunk swizzle for LDS rows of CH chunks. A ds_read/write_b128 is
// served 8 lanes at a time from one 128-byte bank window, so the 8 rows that 8
// consecutive lanes touch (one logical chunk each) must land in 8 distinct
// 16-byte bank slots: (row * CH + (c ^ swz(row))) mod 8 distinct over 8 rows.
template <int CH>
__device__ __forceinline__ int swz_chunks(int row) {
  constexpr int RP = CH >= 8 ? 1 : 8 / CH;  // rows sharing one 128-byte window
  return (row / RP) & (CH - 1);
}

template <int SL, int N>
struct MambaFastCfg {
  static constexpr int NDB = SL / 32;              // 32-channel blocks per unit
  static constexpr int NS = N / 16;                // MFMA k-steps over d_state
  static constexpr int CHC = N / 8;                // 16-byte chunks per C row (and per H row in bf16)
  static constexpr int CHO = SL / 8;               // 16-byte chunks per out row of a unit
  static constexpr int NI = SL / 16;               // out DMA / y store instructions per step
  static constexpr int ND = N >= 64 ? N / 64 : 1;  // C DMA instructions per wave and step
  static constexpr int CS = ND * 4 * 1024;         // C stage bytes (rows past 32 are padding)
  static constexpr int OS = 32 * SL * 2;           // out stage bytes per wave
  static constexpr int XS = 2 * 4 * 256;           // cum_A + seq_idx stage: one 256-byte DMA per wave each
  static constexpr int NDMA = ND + NI + 2;         // DMA instructions per wave and step
  static constexpr int RING = 3 * CS + 4 * 3 * OS + 3 * XS;
  static constexpr int HSCR = 4 * 32 * N * 4;      // H_in transpose: 32 rows x N (bf16 hi + lo) per wave
  static constexpr int LDS = RING > HSCR ? RING : HSCR;
};

template <int SL, int N>
__global__ __launch_bounds__(256, 2) void mamba2_correction_stream_kernel(const MambaCorrArgs a,
                                                                          const int ntb,
                                                                          const int nug) {
  using F = MambaFastCfg<SL, N>;
  constexpr int NDB = F::NDB, NS = F::NS, CHC = F::CHC, CHO = F::CHO, NI = F::NI, ND = F::ND;
  constexpr int CS = F::CS, OS = F::OS, XS = F::XS;
  __shared__ __attribute__((aligned(16))) uint8_t smem[F::LDS];
  uint8_t* const sC = smem;                       // [3][CS]
  uint8_t* const sO = smem + 3 * CS;              // [4 waves][3][OS]
  uint8_t* const sX = sO + 4 * 3 * OS;            // [3][XS]: cum_A [4][256 B], seq_idx [4][256 B]

  int id = blockIdx.x;
  const int nwg = gridDim.x;
  if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
  const int ug = id % nug, rest = id / nug;
  const int tb = rest % ntb, bb = rest / ntb;
  const int T = a.T, H = a.nheads, HD = a.head_dim, G = a.ngroups;
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: resources stay in SGPRs
  const int uph = HD / SL;             // units per head
  const int hpw = 4 / uph;             // heads per workgroup
  const int h0 = 4 * ug / uph;         // first head of the workgroup
  const int unit = 4 * ug + wave, h = unit / uph, sl = unit % uph;
  const int g = h0 / (H / G);          // one C group for the whole workgroup
  const int tbeg = tb * kMambaFastTokensPerWg;
  const int tend = tbeg + kMambaFastTokensPerWg < T ? tbeg + kMambaFastTokensPerWg : T;
  const int nstep = (tend - tbeg + 31) / 32;
  const int64_t HHD = (int64_t)H * HD;
  const int64_t hbase = (((int64_t)bb * H + h) * HD + (int64_t)sl * SL) * N;  // unit's rows of [HD][N]

  // ---- H_in -> registers (and, in the first token block, the state update).
  // Per 32-row block: coalesced fp32 loads -> bf16 hi/lo rows in this wave's LDS
  // scratch ([32][N] each, 16-byte chunks swizzled) -> A operands (db, ks) =
  // rows 32 db + sigma(l32), k = 16 ks + 8 hl .. + 7.
  float e_last = 0.f;
  if (tb == 0) {
    bool fresh_last = false;  // seq_idx[:, -1].any() over the whole batch (:131)
    if (a.seq_idx)
      for (int b2 = 0; b2 < a.batch; ++b2) fresh_last |= a.seq_idx[(int64_t)b2 * T + T - 1] != 0;
    e_last = fresh_last ? 0.f : expf(a.cum_A[((int64_t)bb * T + T - 1) * H + h]);
  }
  bf16x8 ahi[NDB][NS], alo[NDB][NS];
  {
    uint16_t* const shi = reinterpret_cast<uint16_t*>(smem + wave * (32 * N * 4));
    uint16_t* const slo = shi + 32 * N;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int64_t blk = hbase + (int64_t)32 * db * N;
      // 32 rows x N fp32 = N/8 loads of 1 KB per wave, all issued before any use
      f32x4 xs[N / 8];
#pragma unroll
      for (int q = 0; q < N / 8; ++q)
        xs[q] = *reinterpret_cast<const f32x4*>(a.h_prev + blk + 4 * (64 * q + lane));
      if (tb == 0) {
        f32x4 hf[N / 8];
#pragma unroll
        for (int q = 0; q < N / 8; ++q)
          hf[q] = *reinterpret_cast<const f32x4*>(a.h_final + blk + 4 * (64 * q + lane));
#pragma unroll
        for (int q = 0; q < N / 8; ++q)
          *reinterpret_cast<f32x4*>(a.h_final_out + blk + 4 * (64 * q + lane)) = hf[q] + xs[q] * e_last;
      }
#pragma unroll
      for (int q = 0; q < N / 8; ++q) {
        const int p = 64 * q + lane, row = p / (N / 4), n0 = 4 * (p % (N / 4));
        const f32x4 x = xs[q];
        u32x2 hi, lo;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          // hardware round-to-nearest-even; lo = the exact remainder, rounded
          hi[i] = cvt_pk_bf16(x[2 * i], x[2 * i + 1]);
          lo[i] = cvt_pk_bf16(x[2 * i] - __uint_as_float(hi[i] << 16),
                              x[2 * i + 1] - __uint_as_float(hi[i] & 0xffff0000u));
        }
        const int off = row * N + 8 * ((n0 >> 3) ^ (swz_row(row) & (CHC - 1))) + (n0 & 4);
        *reinterpret_cast<u32x2*>(shi + off) = hi;
        *reinterpret_cast<u32x2*>(slo + off) = lo;
      }
      const int arow = sigma(l32);
#pragma unroll
      for (int ks = 0; ks < NS; ++ks) {
        const int off = arow * N + 8 * ((2 * ks + hl) ^ (swz_row(arow) & (CHC - 1)));
        ahi[db][ks] = *reinterpret_cast<const bf16x8*>(shi + off);
        alo[db][ks] = *reinterpret_cast<const bf16x8*>(slo + off);
      }
    }
  }
  lds_barrier();  // every wave's scratch reads are done before the rings' DMA lands there

  // ---- buffer resources (offsets at or past num_records read zeros / drop stores)
  const int cstride = G * N * 2, ostride = (int)(HHD * 2);
  const uint32_t cspan = span_bytes(T, cstride, N * 2), aspan = (uint32_t)T * (uint32_t)H * 4u;
  const i32x4 rC = make_rsrc(a.C + ((int64_t)bb * T * G + g) * N, cspan);
  const i32x4 rO = make_rsrc(a.out + (int64_t)bb * T * HHD + (int64_t)h * HD + sl * SL,
                             span_bytes(T, ostride, SL * 2));
  const i32x4 rY = make_rsrc(a.y + ((int64_t)bb * T + tbeg) * HHD + (int64_t)h * HD + sl * SL,
                             span_bytes(tend - tbeg, ostride, SL * 2));
  const i32x4 rA = make_rsrc(a.cum_A + (int64_t)bb * T * H, aspan);
  const uint32_t sspan = a.seq_idx ? (uint32_t)T * 4u : 0u;
  const i32x4 rS = make_rsrc(a.seq_idx ? (const void*)(a.seq_idx + (int64_t)bb * T) : (const void*)a.cum_A,
                             sspan);
  const uint32_t ldsC = lds_addr(sC), ldsO = lds_addr(sO + wave * 3 * OS), ldsX = lds_addr(sX);
  // cum_A / seq_idx: wave w fetches tokens 8 w .. 8 w + 7 of the step; lane L
  // of the cum_A DMA holds (token 8 w + L / hpw, head h0 + L % hpw)
  const int xa_tok = 8 * wave + lane / hpw, xa_head = h0 + lane % hpw;
  const bool xa_live = lane < 8 * hpw;

  auto issue = [&](int st, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int p = (i * 4 + wave) * 64 + lane, row = p / CHC, pc = p % CHC;
      const int off = row < 32 ? (t0 + row) * cstride + 16 * (pc ^ swz_chunks<CHC>(row)) : (int)cspan;
      dma16_async(rC, ldsC + st * CS + (i * 4 + wave) * 1024, off);
    }
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int p = 64 * k + lane, row = p / CHO, pc = p % CHO;
      dma16_async_nt(rO, ldsO + st * OS + 1024 * k,
                     (t0 + row) * ostride + 16 * (pc ^ swz_chunks<CHO>(row)));
    }
    dma4_async(rA, ldsX + st * XS + 256 * wave,
               xa_live ? (t0 + xa_tok) * (H * 4) + 4 * xa_head : (int)aspan);
    dma4_async(rS, ldsX + st * XS + 1024 + 256 * wave, lane < 8 ? (t0 + 8 * wave + lane) * 4 : (int)sspan);
  };

  issue(0, tbeg);
  if (nstep > 1) issue(1, tbeg + 32);
  // vmcnt budget at the top of step s: everything issued after step s's DMA may
  // stay in flight (the y stores of steps s-2 and s-1, the DMA of step s+1)
  constexpr int K0 = F::NDMA, K1 = F::NDMA + NI, KS = F::NDMA + 2 * NI;
  const int hw = wave / uph;  // this unit's head within the workgroup
  for (int s = 0; s < nstep; ++s) {
    if (s >= 2 && s + 1 < nstep)
      wait_vm_barrier<KS>();
    else if (s == 1 && nstep > 2)
      wait_vm_barrier<K1>();
    else if (s == 0 && nstep > 1)
      wait_vm_barrier<K0>();
    else
      wait_vm_barrier<0>();
    if (s + 2 < nstep) issue((s + 2) % 3, tbeg + 32 * (s + 2));
    const int st = s % 3;

    const uint8_t* cst = sC + st * CS + l32 * (CHC * 16);
    f32x16 acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = zero16();
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(cst + 16 * ((2 * ks + hl) ^ swz_chunks<CHC>(l32)));
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = mfma32(ahi[db][ks], b, acc[db]);
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = mfma32(alo[db][ks], b, acc[db]);
    }
    const uint8_t* xst = sX + st * XS;
    const float ca = reinterpret_cast<const float*>(xst)[64 * (l32 >> 3) + (l32 & 7) * hpw + hw];
    const int sq = reinterpret_cast<const int32_t*>(xst + 1024)[64 * (l32 >> 3) + (l32 & 7)];
    const float e = sq != 0 ? 0.f : expf(ca);

    // out + bf16(dY) in place: lane (hl, l32), reg r of block db holds channel
    // 32 db + 16 (r / 8) + 8 hl + r % 8 of token l32 = logical chunk 4 db + 2 (r / 8) + hl
    uint8_t* ost = sO + (wave * 3 + st) * OS;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int c = 4 * db + 2 * half + hl;
        u32x4* slot = reinterpret_cast<u32x4*>(ost + 16 * (l32 * CHO + (c ^ swz_chunks<CHO>(l32))));
        const u32x4 ov = *slot;
        u32x4 yv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // bf16(out + bf16(dy)), both roundings to nearest even
          const uint32_t dy = cvt_pk_bf16(acc[db][8 * half + 2 * i] * e, acc[db][8 * half + 2 * i + 1] * e);
          yv[i] = cvt_pk_bf16(__uint_as_float(ov[i] << 16) + __uint_as_float(dy << 16),
                              __uint_as_float(ov[i] & 0xffff0000u) + __uint_as_float(dy & 0xffff0000u));
        }
        *slot = yv;
      }
    // y rows back out as full 128-byte lines (rows past the range end are dropped)
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int p = 64 * k + lane, row = p / CHO, pc = p % CHO;
      const u32x4 yv = *reinterpret_cast<const u32x4*>(ost + 16 * p);
      buf_store16_nt(rY, (32 * s + row) * ostride + 16 * (pc ^ swz_chunks<CHO>(row)), yv);
    }
  }
}

hipError_t launch_mamba2_correction(const uint16_t* out, uint16_t* y, const float* h_final,
                                    float* h_final_out, const uint16_t* C, const float* cum_A,
                                    const float* h_prev, const int32_t* seq_idx, int batch, int T,
                                    int nheads, int head_dim, int ngroups, int d_state,
                                    hipStream_t stream) {
  MambaCorrArgs a{out, y, h_final, h_final_out, C, cum_A, h_prev, seq_idx,
                  batch, T, nheads, head_dim, ngroups, d_state};
  // streaming kernel: 4 units (SL channels of a head) per workgroup, all in one C group,
  // and every buffer offset (up to two 32-token steps past T) within int32
  const int SL = head_dim == 32 ? 32 : 64, uph = head_dim / SL;
  const int units = nheads * uph, heads_per_wg = 4 / uph;
  const int64_t row_bytes = std::max<int64_t>({(int64_t)nheads * head_dim * 2,
                                              (int64_t)ngroups * d_state * 2, (int64_t)nheads * 4});
  if (d_state <= 128 && units % 4 == 0 && (nheads / ngroups) % heads_per_wg == 0 &&
      ((int64_t)T + 64) * row_bytes < ((int64_t)1 << 31)) {
    const int ntb = (T + kMambaFastTokensPerWg - 1) / kMambaFastTokensPerWg, nug = units / 4;
    const dim3 sgrid((unsigned)((int64_t)nug * ntb * batch));
    auto go = [&](auto sl, auto n) {
      constexpr int S = decltype(sl)::value, NN = decltype(n)::value;
      hipLaunchKernelGGL((mamba2_correction_stream_kernel<S, NN>), sgrid, dim3(256), 0, stream, a, ntb,
                         nug);
    };
    auto by_n = [&](auto sl) {
      switch (d_state) {
        case 16: go(sl, std::integral_constant<int, 16>{}); break;
        case 32: go(sl, std::integral_constant<int, 32>{}); break;
        case 64: go(sl, std::integral_constant<int, 64>{}); break;
        default: go(sl, std::integral_constant<int, 128>{}); break;
      }
    };
    if (SL == 32)
      by_n(std::integral_constant<int, 32>{});
    else
      by_n(std::integral_constant<int, 64>{});
    return hipGetLastError();
  }
  const dim3 grid(nheads, (T + kMambaTokensPerWg - 1) / kMambaTokensPerWg, batch);
  auto go = [&](auto hd, auto n) {
    constexpr int HD = decltype(hd)::value, N = decltype(n)::value;
    if constexpr (HD * N <= 32768)
      hipLaunchKernelGGL((mamba2_correction_kernel<HD, N>), grid, dim3(256), 0, stream, a);
  };
  auto by_n = [&](auto hd) {
    switch (d_state) {
      case 16: go(hd, std::integral_constant<int, 16>{}); break;
      case 32: go(hd, std::integral_constant<int, 32>{}); break;
      case 64: go(hd, std::integral_constant<int, 64>{}); break;
      case 128: go(hd, std::integral_constant<int, 128>{}); break;
      default: go(hd, std::integral_constant<int, 256>{}); break;
    }
  };
  if (head_dim == 32)
    by_n(std::integral_constant<int, 32>{});
  else if (head_dim == 64)
    by_n(std::integral_constant<int, 64>{});
  else
    by_n(std::integral_constant<int, 128>{});
  return hipGetLastError();
}

}  // namespace rmx
