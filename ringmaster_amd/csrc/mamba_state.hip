// Mamba2 per-shard final SSM state from x, B and dt: the final_states that
// mamba-ssm's mamba_chunk_scan_combined returns for a zero initial state, which
// the reference's CP scan wrapper all-gathers and carries across ranks
// (mamba.py:113-141,160-172; strategies/mamba.py:250-300). Per row (rank shard x
// batch) and head h of group g,
//   S[h] = sum_{t0 <= t < T} w_t x_t (x) B_t,   w_t = exp(cum_A_{T-1} - cum_A_t) e_t
// with e the effective dt (after bias and softplus) and cum_A = cumsum(A e), both
// from rmx_mamba2_dt_cumsum; t0 is the first token of the row's last document (0
// when unpacked), since the scan restarts its state at every document start. The
// closed form is the SSD recurrence h_t = exp(A e_t) h_{t-1} + e_t x_t (x) B_t
// unrolled. The weight scales x in fp32 and the product is rounded to bf16 before
// the MFMA (mamba-ssm's chunk-state kernel scales B instead: the two differ by the
// bf16 rounding of one factor of each product); sums are fp32.
//
// Forward: a workgroup = 4 waves over one (row, pair of heads (or one head), token
// half). Each stage stages 64 tokens of w*x and of B in LDS (rows padded so the
// transposed reads are free of bank conflicts); both MFMA operands are token-major,
// so they come from ds_read_b64_tr_b16 (S = (wX)^T B: M = head dim, N = state,
// K = tokens). Each wave owns D*N/4096 of the 32x32 output tiles of each head, all in
// one row block. Two heads read 256 contiguous bytes of a token's x row where one
// head reads 128 at the token stride (a strided copy of 128-byte rows runs at half
// the HBM rate of one of 512-byte rows), and share each B operand read. x is read
// with the non-temporal cache policy (each byte once): 0.166 -> 0.155 ms at 8 x 8192
// tokens x 64 heads.
//
// Backward (given G = dL/dS fp32): a workgroup = 8 waves x 32 tokens of one
// (row, group); it loops over the group's heads, staging G_h in LDS as bf16:
//   U   = B G_h^T            (MFMA M = head dim, N = tokens, K = state)
//   g_x = w U,  g_w = <x, U>,  g_e = g_w exp(cum_A_{T-1} - cum_A_t),
//   g_cum_A_t = -g_w w_t  (the t = T-1 entry is replaced by the caller with
//   sum_{t<T-1} g_w w, the dependence of every weight on cum_A_{T-1})
//   g_B += G_h^T (w x)       (MFMA M = state, N = tokens, K = head dim), summed
//   over the group's heads in registers and written once.
// Each wave stages its 32 tokens' g_x rows of a head in LDS and writes them as
// whole rows (a store of 8-byte pieces of 32 rows 8 KiB apart was the kernel's
// main cost), and reads e / cum_A 32 bytes (8 heads) per token at a time into an
// LDS table (4-byte reads per head fetched each 128-byte line again and again).
// g_x leaves by non-temporal stores (0.318 -> 0.307 ms at 8 x 8192 tokens x 64 heads);
// non-temporal x loads measured slower here (0.343 ms).
#include "rmx_kernels.h"

namespace rmx {

struct StateArgs {
  const uint16_t* x;      // [rows, T, H, D] bf16
  const uint16_t* B;      // [rows, T, G, N] bf16
  const float* e;         // [rows, T, H]
  const float* cum_A;     // [rows, T, H]
  const int32_t* t0;      // [rows] or null
  float* state;           // fwd out [rows, H, D, N]
  const float* g_state;   // bwd in [rows, H, D, N]
  uint16_t* g_x;          // bwd out [rows, T, H, D] bf16
  uint16_t* g_B;          // bwd out [rows, T, G, N] bf16
  float* g_e;             // bwd out [rows, T, H]
  float* g_cum;           // bwd out [rows, T, H]
  int rows, T, H, G;
  int split;              // fwd: workgroups per (row, head) over the tokens
};

// LDS row stride (bytes) of a tile of `row_bytes` rows: a stride of 16 banks
// (mod 64) puts the 8 reads of 8 bytes that 32 lanes of a transposed read make
// (4 rows x 2 column halves) on disjoint banks.
template <int ROW_BYTES>
constexpr int padded_stride() {
  static_assert(ROW_BYTES == 128 || ROW_BYTES == 256, "rows of 64 or 128 bf16");
  return ROW_BYTES + 64;
}

// Transposed operand (8 tokens x column l32 of a 32-column block) of a row-major
// bf16 LDS tile whose rows are tokens: rows r0 .. r0+7, columns c0 .. c0+31.
template <int STRIDE>
__device__ __forceinline__ bf16x8 tr_tokens(const uint8_t* tile, int r0, int c0, int lane) {
  const int j = lane & 15, half = (lane >> 4) & 1;
  const int row = r0 + 8 * (lane >> 5) + (j >> 2);
  const uint8_t* p = tile + row * STRIDE + 2 * (c0 + 16 * half + 4 * (j & 3));
  return join_bf16x8(lds_read_tr(reinterpret_cast<const uint16_t*>(p)),
                     lds_read_tr(reinterpret_cast<const uint16_t*>(p + 4 * STRIDE)));
}

// The same operand from a tile of unpadded RB-byte rows whose 16-byte chunk p of
// row r sits at p ^ swz_both<RB / 2>(r), the swizzle that keeps both the 16-byte
// row reads of 16 consecutive rows and these transposed reads free of conflicts.
template <int RB>
__device__ __forceinline__ bf16x8 tr_tokens_swz(const uint8_t* tile, int r0, int c0, int lane) {
  const int j = lane & 15, half = (lane >> 4) & 1;
  const int row = r0 + 8 * (lane >> 5) + (j >> 2);
  const int col = c0 + 16 * half + 4 * (j & 3);
  const int p = col >> 3, sub = 2 * (col & 7);
  const uint8_t* p0 = tile + row * RB + 16 * (p ^ swz_both<RB / 2>(row)) + sub;
  const uint8_t* p1 = tile + (row + 4) * RB + 16 * (p ^ swz_both<RB / 2>(row + 4)) + sub;
  return join_bf16x8(lds_read_tr(reinterpret_cast<const uint16_t*>(p0)),
                     lds_read_tr(reinterpret_cast<const uint16_t*>(p1)));
}

__device__ __forceinline__ u32x4 scale_bf16x8(const u32x4& v, float w) {
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = cvt_pk_bf16(__uint_as_float(v[i] << 16) * w, __uint_as_float(v[i] & 0xffff0000u) * w);
  return o;
}

// ---------------------------------------------------------------- forward
template <int D, int N, int HPW>
__global__ __launch_bounds__(256) void mamba2_chunk_state_kernel(const StateArgs a) {
  constexpr int TK = 64;                                // tokens per stage
  constexpr int XS = padded_stride<2 * D>(), BS = padded_stride<2 * N>();
  constexpr int NBN = N / 32;                           // 32-wide state blocks
  constexpr int TPW = (D / 32) * NBN / 4;               // output tiles per wave and head
  constexpr int XR = HPW * D / 8;                       // 16-B chunks of a token's x row
  constexpr int XCH = TK * XR / 256, BCH = TK * N / 8 / 256;  // 16-B chunks per thread
  static_assert(TPW >= 1 && NBN % TPW == 0 && XCH >= 1 && BCH >= 1, "tile split");
  // HPW consecutive heads of one group per workgroup: a token's x row of those heads is
  // HPW * 2D contiguous bytes (rows of 128 bytes at the token stride read at half the
  // rate of 512-byte ones), and one B operand read serves every head
  __shared__ __attribute__((aligned(16))) uint8_t sX[HPW][TK * XS];
  __shared__ __attribute__((aligned(16))) uint8_t sB[TK * BS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups go to the 8 XCDs round-robin. Give each XCD a contiguous run of
  // (row, split, head) ordinals, head fastest, so the heads that read the same B
  // rows run together on one XCD and find them in its L2.
  const int nwg = gridDim.x;
  const int k = (nwg % 8 == 0) ? (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8)
                               : (int)blockIdx.x;
  const int nhb = a.H / HPW;
  const int h = (k % nhb) * HPW;  // first head of the workgroup
  const int split = (k / nhb) % a.split;
  const int row = k / (nhb * a.split);
  const int g = h / (a.H / a.G);
  const int T = a.T;
  // tokens of this workgroup: whole stages, the last split takes the remainder
  const int nst = (T + TK - 1) / TK;
  const int st_lo = (int)((int64_t)nst * split / a.split);
  const int st_hi = (int)((int64_t)nst * (split + 1) / a.split);
  const int t0 = a.t0 ? a.t0[row] : 0;
  const int st_begin = st_lo > t0 / TK ? st_lo : t0 / TK;

  const int64_t th = (int64_t)row * T * a.H + h;  // (row, t = 0, h) in [rows, T, H]
  float cl[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) cl[j] = a.cum_A[th + (int64_t)(T - 1) * a.H + j];
  const i32x4 xrs = make_rsrc(a.x + (int64_t)row * T * a.H * D, (uint32_t)T * a.H * D * 2);
  const i32x4 brs = make_rsrc(a.B + (int64_t)row * T * a.G * N, (uint32_t)T * a.G * N * 2);

  // One stage of loads in flight (the next stage's registers fill while this one
  // computes); the weights are formed at the store, so issuing loads never waits,
  // and the small register set lets four workgroups share a CU.
  struct Regs {
    u32x4 x[XCH], b[BCH];
    float e[XCH], c[XCH];
  };
  Regs rg;
  auto load = [&](int st, Regs& r) __attribute__((always_inline)) {
    const int tb = st * TK;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + 256 * i, t = tb + c / XR, j = (c % XR) / (D / 8);
      r.x[i] = buf_load16_nt(xrs, ((t * a.H + h) * D + 8 * (c % XR)) * 2);  // read once
      const int64_t o = th + (int64_t)(t < T ? t : T - 1) * a.H + j;
      r.e[i] = a.e[o];
      r.c[i] = a.cum_A[o];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i, t = tb + c / (N / 8);
      r.b[i] = buf_load16(brs, ((t * a.G + g) * N + 8 * (c % (N / 8))) * 2);
    }
  };
  auto store = [&](int st, const Regs& r) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + 256 * i, t = st * TK + c / XR, j = (c % XR) / (D / 8);
      // XR is a power of two and c % XR a multiple of D / 8 per head: j is wave-uniform
      // only when XR >= 64; the head's cum_A at T-1 is picked per lane
      float clj = cl[0];
#pragma unroll
      for (int jj = 1; jj < HPW; ++jj) clj = j == jj ? cl[jj] : clj;
      const float w = (t >= t0 && t < T) ? r.e[i] * expf(clj - r.c[i]) : 0.f;
      st16(sX[j] + (c / XR) * XS + 16 * (c % (D / 8)), scale_bf16x8(r.x[i], w));
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i;
      st16(sB + (c / (N / 8)) * BS + 16 * (c % (N / 8)), r.b[i]);
    }
  };

  const int mb = (wave * TPW) / NBN, nb0 = (wave * TPW) % NBN;
  f32x16 acc[HPW][TPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j)
#pragma unroll
    for (int i = 0; i < TPW; ++i) acc[j][i] = zero16();
  auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < TK / 16; ++ks) {
      bf16x8 av[HPW];
#pragma unroll
      for (int j = 0; j < HPW; ++j) av[j] = tr_tokens<XS>(sX[j], 16 * ks, 32 * mb, lane);
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const bf16x8 bv = tr_tokens<BS>(sB, 16 * ks, 32 * (nb0 + i), lane);
#pragma unroll
        for (int j = 0; j < HPW; ++j) acc[j][i] = mfma32(av[j], bv, acc[j][i]);
      }
    }
  };
  if (st_begin < st_hi) load(st_begin, rg);
  for (int st = st_begin; st < st_hi; ++st) {
    __syncthreads();  // the previous stage's reads are done
    store(st, rg);
    __syncthreads();
    if (st + 1 < st_hi) load(st + 1, rg);
    compute();
  }

  // lane (hl, l32), reg r: d = 32 mb + c_row(hl, r), n = 32 nb + l32
  const int hl = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    float* out = a.state + ((int64_t)row * a.H + h + j) * D * N;
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float* p = out + (32 * mb + c_row(hl, r)) * N + 32 * (nb0 + i) + l32;
        if (a.split == 1)
          *p = acc[j][i][r];
        else
          atomicAdd(p, acc[j][i][r]);  // two splits onto zero: exact in either order
      }
  }
}

__global__ void zero_f32_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------- backward
template <int D, int N>
__global__ __launch_bounds__(512) void mamba2_chunk_state_bwd_kernel(const StateArgs a) {
  constexpr int NW = 8, NT = 64 * NW, BT = 32 * NW;  // 32 tokens per wave
  constexpr int GS = 2 * N;                          // LDS row bytes of G (bf16, swizzled)
  constexpr int NMD = D / 32, NKN = N / 16;          // GEMM 1 (U): M blocks, k-steps
  constexpr int NMN = N / 32, NKD = D / 16;          // GEMM 2 (g_B): M blocks, k-steps
  constexpr int GCH = D * N / 8 / NT;                // 8-float chunks of G per thread
  static_assert(GCH >= 1, "G split");
  __shared__ __attribute__((aligned(16))) uint8_t sG[2][D * GS];
  // g_e (lane half 0) and g_cum_A (half 1) of 8 consecutive heads per token, so
  // that each token's row of those [rows, T, H] arrays is written 32 bytes at a time
  __shared__ __attribute__((aligned(16))) float sE[2][BT][8];
  // each wave's g_x rows of one head (32 tokens x D bf16), staged so that they leave as
  // whole rows: rows of 2D + 8 bytes keep the 8-byte writes of 32 rows on distinct banks
  constexpr int XS = 2 * D + 8;
  __shared__ __attribute__((aligned(16))) uint8_t sX[NW][32 * XS];
  // e (columns 0..7) and cum_A (8..15) of 8 consecutive heads per token, loaded 32 bytes
  // per token row instead of 4 bytes per head (a 17-float row keeps 32 tokens' reads of
  // one column on distinct banks); each wave reads only its own tokens' rows. Shapes whose
  // tiles leave no room for the table load 4 bytes per head.
  constexpr bool kEC = 2 * D * GS + 2 * BT * 8 * 4 + NW * 32 * XS + BT * 17 * 4 <= 163840;
  __shared__ float sEC[kEC ? BT : 1][17];

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nbt = (a.T + BT - 1) / BT;
  const int bt = blockIdx.x % nbt;
  const int rg = blockIdx.x / nbt;
  const int g = rg % a.G, row = rg / a.G;
  const int T = a.T, H = a.H, hpg = H / a.G;
  const int t = bt * BT + 32 * wave + l32;  // this lane's token
  const bool tv = t < T;
  const int t0 = a.t0 ? a.t0[row] : 0;
  const bool live = tv && t >= t0;

  // B rows of this lane's token as the B operand of U (k = state n = 16 kb + 8 hl ..)
  bf16x8 bop[NKN];
  {
    const i32x4 brs = make_rsrc(a.B + (int64_t)row * T * a.G * N, (uint32_t)T * a.G * N * 2);
#pragma unroll
    for (int kb = 0; kb < NKN; ++kb)
      bop[kb] = __builtin_bit_cast(bf16x8, buf_load16(brs, ((t * a.G + g) * N + 16 * kb + 8 * hl) * 2));
  }
  const i32x4 xrs = make_rsrc(a.x + (int64_t)row * T * H * D, (uint32_t)T * H * D * 2);

  f32x16 gb[NMN];
#pragma unroll
  for (int i = 0; i < NMN; ++i) gb[i] = zero16();

  // G_h (fp32 [D][N]) -> bf16 LDS rows, through registers one head ahead
  f32x4 gr[GCH][2];
  auto load_g = [&](int h) {
    const float* gp = a.g_state + ((int64_t)row * H + h) * D * N;
#pragma unroll
    for (int i = 0; i < GCH; ++i) {
      const int c = tid + NT * i;
      gr[i][0] = *reinterpret_cast<const f32x4*>(gp + 8 * c);
      gr[i][1] = *reinterpret_cast<const f32x4*>(gp + 8 * c + 4);
    }
  };
  auto store_g = [&](int buf) {
#pragma unroll
    for (int i = 0; i < GCH; ++i) {
      const int c = tid + NT * i, d = c / (N / 8), n8 = c % (N / 8);
      u32x4 u;
      u[0] = cvt_pk_bf16(gr[i][0][0], gr[i][0][1]);
      u[1] = cvt_pk_bf16(gr[i][0][2], gr[i][0][3]);
      u[2] = cvt_pk_bf16(gr[i][1][0], gr[i][1][1]);
      u[3] = cvt_pk_bf16(gr[i][1][2], gr[i][1][3]);
      st16(sG[buf] + d * GS + 16 * (n8 ^ swz_both<N>(d)), u);
    }
  };

  // per-head operands of this lane's token, loaded one head ahead: x[t, h, 16 kb +
  // 8 hl .. +7] (the B operand layout of g_B), e, cum_A at t and at T-1
  struct HeadRegs {
    u32x4 x[NKD];
    float e, c, cl;
  };
  HeadRegs hr[2];
  // e / cum_A by 8-head groups when the group's heads are 8-aligned rows of 32 bytes
  const bool ec8 = kEC && ((H | hpg | g * hpg) & 7) == 0;
  // a group's values (e for lane half 0, cum_A for half 1: 32 bytes of this lane's token
  // row) go straight to the wave's table, so no registers stay live across heads
  float* ecrow = sEC[kEC ? 32 * wave + l32 : 0];
  auto load_ec = [&](int h0) __attribute__((always_inline)) {
    const float* src = (hl ? a.cum_A : a.e) + ((int64_t)row * T + (tv ? t : 0)) * H + h0;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(src);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ecrow[8 * hl + i] = v0[i];
      ecrow[8 * hl + 4 + i] = v1[i];
    }
  };
  auto load_h = [&](int h, HeadRegs& r) __attribute__((always_inline)) {
    const int xo = (t * H + h) * D;
#pragma unroll
    for (int kb = 0; kb < NKD; ++kb) r.x[kb] = buf_load16(xrs, (xo + 16 * kb + 8 * hl) * 2);
    const int64_t th = (int64_t)row * T * H + h;
    if (!ec8) {
      r.e = a.e[th + (int64_t)(tv ? t : 0) * H];
      r.c = a.cum_A[th + (int64_t)(tv ? t : 0) * H];
    }
    r.cl = a.cum_A[th + (int64_t)(T - 1) * H];
  };

  auto head = [&](int hi, const HeadRegs& cur, HeadRegs& nxt) __attribute__((always_inline)) {
    const int h = g * hpg + hi, buf = hi & 1;
    store_g(buf);
    // G_h visible, and every wave's LDS reads of buffer buf from two heads ago are done.
    // Only LDS is waited for: the g_x / g_e stores of earlier heads stay in flight
    // (__syncthreads would wait for them, one store latency per head).
    lds_barrier();
    if (hi + 1 < hpg) {
      load_g(h + 1);
      load_h(h + 1, nxt);
    }
    const uint8_t* sg = sG[buf];
    float ce = cur.e, cc = cur.c;
    if (ec8) {
      if ((hi & 7) == 0) load_ec(h);  // a new group: its values to the wave's table
      asm volatile("" ::: "memory");  // the table rows are this wave's own: LDS order suffices
      ce = ecrow[hi & 7];
      cc = ecrow[8 + (hi & 7)];
    }
    const float dec = live ? expf(cur.cl - cc) : 0.f;
    const float w = live ? dec * ce : 0.f;

    // U^T (d x tokens) = G_h B^T: A = G rows (LDS), B = this lane's B row
    f32x16 u[NMD];
#pragma unroll
    for (int m = 0; m < NMD; ++m) {
      u[m] = zero16();
#pragma unroll
      for (int kb = 0; kb < NKN; ++kb) {
        const int gr = 32 * m + l32;
        const bf16x8 ga = __builtin_bit_cast(
            bf16x8, ld16(sg + gr * GS + 16 * ((2 * kb + hl) ^ swz_both<N>(gr))));
        u[m] = mfma32(ga, bop[kb], u[m]);
      }
    }
    // x in the C layout of U (lane half hl: d = 8 blk + 4 hl .. +3, blk = 4 m + q):
    // 8-wide block 2 kb + hl is this lane's, the other half-blocks come from the
    // partner lane (l ^ 32), which holds block 2 kb + (1 - hl)
    u32x2 xc[D / 8];
#pragma unroll
    for (int kb = 0; kb < NKD; ++kb) {
      const u32x4 own = cur.x[kb];
      const uint32_t s0 = hl ? own[0] : own[2], s1 = hl ? own[1] : own[3];
      const uint32_t r0 = (uint32_t)__shfl_xor((int)s0, 32, 64);
      const uint32_t r1 = (uint32_t)__shfl_xor((int)s1, 32, 64);
      xc[2 * kb][0] = hl ? r0 : own[0];
      xc[2 * kb][1] = hl ? r1 : own[1];
      xc[2 * kb + 1][0] = hl ? own[2] : r0;
      xc[2 * kb + 1][1] = hl ? own[3] : r1;
    }
    // lane (hl, l32) holds U[token t][d = 32 m + c_row(hl, r)]: g_x, g_w. The wave's
    // g_x rows go to its LDS strip first (8 bytes per lane and piece) ...
    float gw = 0.f;
    uint8_t* xs = sX[wave];
#pragma unroll
    for (int m = 0; m < NMD; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x2 xv = xc[4 * m + q];
        const float x0 = __uint_as_float(xv[0] << 16), x1 = __uint_as_float(xv[0] & 0xffff0000u);
        const float x2 = __uint_as_float(xv[1] << 16), x3 = __uint_as_float(xv[1] & 0xffff0000u);
        gw += x0 * u[m][4 * q] + x1 * u[m][4 * q + 1] + x2 * u[m][4 * q + 2] + x3 * u[m][4 * q + 3];
        u32x2 sv;
        sv[0] = cvt_pk_bf16(w * u[m][4 * q], w * u[m][4 * q + 1]);
        sv[1] = cvt_pk_bf16(w * u[m][4 * q + 2], w * u[m][4 * q + 3]);
        *reinterpret_cast<u32x2*>(xs + l32 * XS + 2 * (32 * m + 8 * q + 4 * hl)) = sv;
      }
    // ... and leave it as whole rows: LPR lanes per token row, 16 bytes each (the strip
    // is this wave's own, and a wave's LDS operations complete in order)
    {
      constexpr int LPR = 2 * D / 16, RPI = 64 / LPR;
      asm volatile("" ::: "memory");
      // the wave's rows of head h: tokens past T fall outside num_records and are dropped
      const int tw = bt * BT + 32 * wave;
      const int nrows = T - tw < 32 ? T - tw : 32;
      const i32x4 grs = make_rsrc(a.g_x + ((int64_t)row * T + tw) * H * D + (int64_t)h * D,
                                  nrows > 0 ? (uint32_t)((nrows - 1) * H * D + D) * 2u : 0u);
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int rr = RPI * i + lane / LPR;
        const uint8_t* src = xs + rr * XS + 16 * (lane % LPR);
        u32x4 v;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(src);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 8);
        v[0] = lo[0];
        v[1] = lo[1];
        v[2] = hi[0];
        v[3] = hi[1];
        buf_store16_nt(grs, (rr * H * D + 8 * (lane % LPR)) * 2, v);
      }
    }
    gw += xhalf(gw);
    // each wave stages only its own tokens' strip: no barrier, LDS order suffices
    float* strip = &sE[hl][32 * wave + l32][0];
    strip[hi & 7] = hl ? -gw * w : gw * dec;
    if ((hi & 7) == 7 || hi == hpg - 1) {
      const int h0 = h - (hi & 7), cnt = (hi & 7) + 1;
      if (tv) {
        float* dst = (hl ? a.g_cum : a.g_e) + (int64_t)row * T * H + (int64_t)t * H + h0;
        if (cnt == 8 && ((H | h0) & 3) == 0) {  // 16-byte aligned rows
          *reinterpret_cast<f32x4*>(dst) = *reinterpret_cast<const f32x4*>(strip);
          *reinterpret_cast<f32x4*>(dst + 4) = *reinterpret_cast<const f32x4*>(strip + 4);
        } else {
          for (int j = 0; j < cnt; ++j) dst[j] = strip[j];
        }
      }
    }

    // g_B^T (state x tokens) += G_h^T (w x)^T: A = G^T by transposed reads, B = w x
#pragma unroll
    for (int m = 0; m < NMN; ++m)
#pragma unroll
      for (int kb = 0; kb < NKD; ++kb)
        gb[m] = mfma32(tr_tokens_swz<GS>(sg, 16 * kb, 32 * m, lane),
                       __builtin_bit_cast(bf16x8, scale_bf16x8(cur.x[kb], w)), gb[m]);
  };

  load_g(g * hpg);
  load_h(g * hpg, hr[0]);
  for (int hi = 0; hi < hpg; hi += 2) {
    head(hi, hr[0], hr[1]);
    if (hi + 1 < hpg) head(hi + 1, hr[1], hr[0]);
  }

  // lane (hl, l32) holds g_B[token t][n = 32 m + c_row(hl, r)]
  if (tv) {
    uint16_t* gbp = a.g_B + ((int64_t)row * T * a.G + (int64_t)t * a.G + g) * N;
#pragma unroll
    for (int m = 0; m < NMN; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x2 s;
        s[0] = cvt_pk_bf16(gb[m][4 * q], gb[m][4 * q + 1]);
        s[1] = cvt_pk_bf16(gb[m][4 * q + 2], gb[m][4 * q + 3]);
        *reinterpret_cast<u32x2*>(gbp + 32 * m + 8 * q + 4 * hl) = s;
      }
  }
}

// ---------------------------------------------------------------- backward, two heads per step
// The backward above moves a token's x and g_x row of ONE head (128 bytes at the
// token stride) per step; a strided copy of such rows runs at half the HBM rate of
// one of 256-byte rows. This form moves two adjacent heads per step: a workgroup =
// 8 waves = 4 token waves (32 tokens each, 128 tokens) x 2 head slots, step i doing
// head 2i of the group in slot 0 and 2i + 1 in slot 1, the same math per (token,
// head) as above. G arrives as bf16 rows [rows, H, D, N] (g_state_bf16_kernel fills
// a caller workspace) by LDS DMA one step ahead, so no registers carry it. A step:
//   wait for everything this wave issued (G of this step, its x rows, the previous
//   step's stores) and barrier; store the previous step's g_x rows (staged in the
//   wave's LDS strip) and the g_e / g_cum_A strips of an 8-head group the previous
//   step finished; load the step's e / cum_A table; DMA the next step's G, load its
//   x rows; compute.
// Workgroups walk the heads from different 8-head groups (a rotation by a multiple of four
// steps, when the group holds an even number of such groups): with every workgroup on the
// same head pair, the ones running together read and write the same 256-byte column of
// their token rows (8 KiB apart), which HBM serves at about 3.4 TB/s; rotated, 323 us
// against 376-390 us per configs[4] call.
// Each slot sums its own heads' g_B in registers; the two sums meet in LDS at the end.
template <int D, int N>
__global__ __launch_bounds__(512) void mamba2_chunk_state_bwd2_kernel(const StateArgs a,
                                                                       const uint16_t* gws) {
  constexpr int NW = 8, BT = 128;                 // 4 token waves x 2 head slots
  constexpr int GS = 2 * N, GT = D * GS;          // a G_h tile: D rows of N bf16, swizzled
  constexpr int NMD = D / 32, NKN = N / 16;       // GEMM 1 (U): M blocks, k-steps
  constexpr int NMN = N / 32, NKD = D / 16;       // GEMM 2 (g_B): M blocks, k-steps
  constexpr int PPW = GT / 1024 / 4;              // 1 KiB DMA pieces per wave and step
  constexpr int XS = 2 * D + 8;
  static_assert(PPW >= 1 && GT % 4096 == 0, "G tile split");
  static_assert(2 * 2 * GT >= BT * N * 4, "g_B meeting place");
  __shared__ __attribute__((aligned(1024))) uint8_t sG[2][2][GT];  // [step parity][slot]
  __shared__ __attribute__((aligned(16))) float sE[2][2][BT][8];   // [group parity][e, cum][token][head]
  __shared__ __attribute__((aligned(16))) uint8_t sX[NW][32 * XS];
  __shared__ float sEC[NW * 32][17];

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tw = wave & 3, hs = wave >> 2;  // token wave, head slot
  const int nbt = (a.T + BT - 1) / BT;
  const int bt = blockIdx.x % nbt;
  const int rg = blockIdx.x / nbt;
  const int g = rg % a.G, row = rg / a.G;
  const int T = a.T, H = a.H, hpg = H / a.G;
  const int nstep = (hpg + 1) / 2;
  // workgroups start at different 8-head groups (rotation by 4 steps), so the ones running
  // together read and write different 256-byte pieces of the token rows
  const bool rotate = (hpg & 7) == 0 && ((hpg >> 3) & 1) == 0 && ((H | hpg | g * hpg) & 7) == 0;
  const int rot = rotate ? 4 * (int)(blockIdx.x % (unsigned)(nstep / 4)) : 0;
  auto pr = [&](int i) { return i + rot < nstep ? i + rot : i + rot - nstep; };
  const int tb = bt * BT + 32 * tw;  // first token of this wave
  const int t = tb + l32;            // this lane's token
  const bool tv = t < T;
  const int t0 = a.t0 ? a.t0[row] : 0;
  const bool live = tv && t >= t0;

  bf16x8 bop[NKN];
  {
    const i32x4 brs = make_rsrc(a.B + (int64_t)row * T * a.G * N, (uint32_t)T * a.G * N * 2);
#pragma unroll
    for (int kb = 0; kb < NKN; ++kb)
      bop[kb] = __builtin_bit_cast(bf16x8, buf_load16(brs, ((t * a.G + g) * N + 16 * kb + 8 * hl) * 2));
  }
  const i32x4 xrs = make_rsrc(a.x + (int64_t)row * T * H * D, (uint32_t)T * H * D * 2);
  f32x16 gb[NMN];
#pragma unroll
  for (int i = 0; i < NMN; ++i) gb[i] = zero16();

  // G DMA: the 4 waves of slot s fill its tile, wave piece (tw PPW + j); lane L of piece p
  // writes LDS bytes 1024 p + 16 L (row d, chunk position c) from global chunk c ^ swz(d)
  int goff[PPW];
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    const int byte = 1024 * (tw * PPW + j) + 16 * lane;
    const int d = byte / GS, c = (byte % GS) / 16;
    goff[j] = d * GS + 16 * (c ^ swz_both<N>(d));
  }
  auto dma_g = [&](int i, int buf) __attribute__((always_inline)) {
    const int hh = 2 * i + hs;  // this slot's head of step pair i (none past the group)
    const bool on = hh < hpg;
    const uint16_t* base = gws + ((int64_t)row * H + g * hpg + (on ? hh : 0)) * D * N;
    const i32x4 rs = make_rsrc(base, on ? (uint32_t)GT : 0u);
    const uint32_t dst = lds_addr(&sG[buf][hs][0]);
#pragma unroll
    for (int j = 0; j < PPW; ++j) dma16_async(rs, dst + 1024 * (tw * PPW + j), goff[j]);
  };

  struct HeadRegs {
    u32x4 x[NKD];
    float e, c, cl;
  };
  HeadRegs hr[2];
  const bool ec8 = ((H | hpg | g * hpg) & 7) == 0;
  float* ecrow = sEC[32 * wave + l32];
  auto load_ec = [&](int h0) __attribute__((always_inline)) {
    const float* src = (hl ? a.cum_A : a.e) + ((int64_t)row * T + (tv ? t : 0)) * H + h0;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(src);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ecrow[8 * hl + i] = v0[i];
      ecrow[8 * hl + 4 + i] = v1[i];
    }
  };
  auto load_h = [&](int h, HeadRegs& r) __attribute__((always_inline)) {
    const int xo = (t * H + h) * D;
#pragma unroll
    for (int kb = 0; kb < NKD; ++kb) r.x[kb] = buf_load16(xrs, (xo + 16 * kb + 8 * hl) * 2);
    const int64_t th = (int64_t)row * T * H + h;
    if (!ec8) {
      r.e = a.e[th + (int64_t)(tv ? t : 0) * H];
      r.c = a.cum_A[th + (int64_t)(tv ? t : 0) * H];
    }
    r.cl = a.cum_A[th + (int64_t)(T - 1) * H];
  };
  // this wave's g_x rows of head h, staged in its LDS strip, as whole rows: tokens past T
  // fall outside num_records and are dropped
  auto store_gx = [&](int h) __attribute__((always_inline)) {
    constexpr int LPR = 2 * D / 16, RPI = 64 / LPR;
    const int nrows = T - tb < 32 ? T - tb : 32;
    const i32x4 grs = make_rsrc(a.g_x + ((int64_t)row * T + tb) * H * D + (int64_t)h * D,
                                nrows > 0 ? (uint32_t)((nrows - 1) * H * D + D) * 2u : 0u);
    const uint8_t* xs = sX[wave];
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int rr = RPI * i + lane / LPR;
      const uint8_t* src = xs + rr * XS + 16 * (lane % LPR);
      const u32x2 lo = *reinterpret_cast<const u32x2*>(src);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 8);
      u32x4 v;
      v[0] = lo[0];
      v[1] = lo[1];
      v[2] = hi[0];
      v[3] = hi[1];
      buf_store16_nt(grs, (rr * H * D + 8 * (lane % LPR)) * 2, v);
    }
  };
  // g_e (lane half 0) / g_cum_A (half 1) of the 8-head group k (heads 8k .. 8k + cnt - 1
  // of the group), both slots' columns, stored by slot 0
  auto store_strip = [&](int k, int cnt) __attribute__((always_inline)) {
    if (hs != 0 || !tv) return;
    const float* strip = &sE[k & 1][hl][32 * tw + l32][0];
    const int h0 = g * hpg + 8 * k;
    float* dst = (hl ? a.g_cum : a.g_e) + (int64_t)row * T * H + (int64_t)t * H + h0;
    if (cnt == 8 && ((H | h0) & 3) == 0) {  // 16-byte aligned rows
      *reinterpret_cast<f32x4*>(dst) = *reinterpret_cast<const f32x4*>(strip);
      *reinterpret_cast<f32x4*>(dst + 4) = *reinterpret_cast<const f32x4*>(strip + 4);
    } else {
      for (int j = 0; j < cnt; ++j) dst[j] = strip[j];
    }
  };

  auto step = [&](int i, const HeadRegs& cur, HeadRegs& nxt) __attribute__((always_inline)) {
    const int pi = pr(i), buf = i & 1, hh = 2 * pi + hs, h = g * hpg + hh;
    const bool on = hh < hpg;
    wait_vm_barrier<0>();
    if (i > 0) {
      const int hp = 2 * pr(i - 1) + hs;  // the previous step's head
      if (hp < hpg) store_gx(g * hpg + hp);
      if (((2 * pi) & 7) == 0) store_strip(pr(i - 1) / 4, 8);
    }
    float ce = cur.e, cc = cur.c;
    if (ec8 && ((2 * pi) & 7) == 0) load_ec(g * hpg + 2 * pi);
    if (i + 1 < nstep) {
      const int pn = pr(i + 1);
      dma_g(pn, buf ^ 1);
      if (2 * pn + hs < hpg) load_h(g * hpg + 2 * pn + hs, nxt);
    }
    if (!on) return;
    if (ec8) {
      asm volatile("" ::: "memory");  // the table rows are this wave's own: LDS order suffices
      ce = ecrow[hh & 7];
      cc = ecrow[8 + (hh & 7)];
    }
    const uint8_t* sg = sG[buf][hs];
    const float dec = live ? expf(cur.cl - cc) : 0.f;
    const float w = live ? dec * ce : 0.f;

    // U^T (d x tokens) = G_h B^T: A = G rows (LDS), B = this lane's B row
    f32x16 u[NMD];
#pragma unroll
    for (int m = 0; m < NMD; ++m) {
      u[m] = zero16();
#pragma unroll
      for (int kb = 0; kb < NKN; ++kb) {
        const int gr = 32 * m + l32;
        const bf16x8 ga = __builtin_bit_cast(
            bf16x8, ld16(sg + gr * GS + 16 * ((2 * kb + hl) ^ swz_both<N>(gr))));
        u[m] = mfma32(ga, bop[kb], u[m]);
      }
    }
    // x in the C layout of U (see the backward above)
    u32x2 xc[D / 8];
#pragma unroll
    for (int kb = 0; kb < NKD; ++kb) {
      const u32x4 own = cur.x[kb];
      const uint32_t s0 = hl ? own[0] : own[2], s1 = hl ? own[1] : own[3];
      const uint32_t r0 = (uint32_t)__shfl_xor((int)s0, 32, 64);
      const uint32_t r1 = (uint32_t)__shfl_xor((int)s1, 32, 64);
      xc[2 * kb][0] = hl ? r0 : own[0];
      xc[2 * kb][1] = hl ? r1 : own[1];
      xc[2 * kb + 1][0] = hl ? own[2] : r0;
      xc[2 * kb + 1][1] = hl ? own[3] : r1;
    }
    float gw = 0.f;
    uint8_t* xs = sX[wave];
#pragma unroll
    for (int m = 0; m < NMD; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x2 xv = xc[4 * m + q];
        const float x0 = __uint_as_float(xv[0] << 16), x1 = __uint_as_float(xv[0] & 0xffff0000u);
        const float x2 = __uint_as_float(xv[1] << 16), x3 = __uint_as_float(xv[1] & 0xffff0000u);
        gw += x0 * u[m][4 * q] + x1 * u[m][4 * q + 1] + x2 * u[m][4 * q + 2] + x3 * u[m][4 * q + 3];
        u32x2 sv;
        sv[0] = cvt_pk_bf16(w * u[m][4 * q], w * u[m][4 * q + 1]);
        sv[1] = cvt_pk_bf16(w * u[m][4 * q + 2], w * u[m][4 * q + 3]);
        *reinterpret_cast<u32x2*>(xs + l32 * XS + 2 * (32 * m + 8 * q + 4 * hl)) = sv;
      }
    gw += xhalf(gw);
    sE[(hh >> 3) & 1][hl][32 * tw + l32][hh & 7] = hl ? -gw * w : gw * dec;

    // g_B^T (state x tokens) += G_h^T (w x)^T: A = G^T by transposed reads, B = w x
#pragma unroll
    for (int m = 0; m < NMN; ++m)
#pragma unroll
      for (int kb = 0; kb < NKD; ++kb)
        gb[m] = mfma32(tr_tokens_swz<GS>(sg, 16 * kb, 32 * m, lane),
                       __builtin_bit_cast(bf16x8, scale_bf16x8(cur.x[kb], w)), gb[m]);
  };

  dma_g(pr(0), 0);
  if (2 * pr(0) + hs < hpg) load_h(g * hpg + 2 * pr(0) + hs, hr[0]);
  for (int i = 0; i < nstep; i += 2) {
    step(i, hr[0], hr[1]);
    if (i + 1 < nstep) step(i + 1, hr[1], hr[0]);
  }
  // the last step's g_x rows and the last (possibly partial) group's strips
  wait_vm_barrier<0>();
  {
    const int hh = 2 * pr(nstep - 1) + hs;
    if (hh < hpg) store_gx(g * hpg + hh);
    const int k = pr(nstep - 1) / 4;
    store_strip(k, rot ? 8 : hpg - 8 * k);
  }
  // g_B: slot 1's sums meet slot 0's in LDS (transposed, [n][token], conflict-free)
  float* sgb = reinterpret_cast<float*>(&sG[0][0][0]);
  if (hs == 1) {
#pragma unroll
    for (int m = 0; m < NMN; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) sgb[(32 * m + c_row(hl, r)) * BT + 32 * tw + l32] = gb[m][r];
  }
  lds_barrier();
  if (hs == 0 && tv) {
    uint16_t* gbp = a.g_B + ((int64_t)row * T * a.G + (int64_t)t * a.G + g) * N;
#pragma unroll
    for (int m = 0; m < NMN; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int n = 32 * m + 8 * q + 4 * hl + k;
          v[k] = gb[m][4 * q + k] + sgb[n * BT + 32 * tw + l32];
        }
        u32x2 st;
        st[0] = cvt_pk_bf16(v[0], v[1]);
        st[1] = cvt_pk_bf16(v[2], v[3]);
        *reinterpret_cast<u32x2*>(gbp + 32 * m + 8 * q + 4 * hl) = st;
      }
  }
}

// G = dL/dS (fp32) -> bf16 rows of the same layout, for the two-head backward's DMA
__global__ void g_state_bf16_kernel(const float* __restrict__ g, uint16_t* __restrict__ o,
                                    int64_t n8) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const f32x4 a = *reinterpret_cast<const f32x4*>(g + 8 * i);
  const f32x4 b = *reinterpret_cast<const f32x4*>(g + 8 * i + 4);
  u32x4 u;
  u[0] = cvt_pk_bf16(a[0], a[1]);
  u[1] = cvt_pk_bf16(a[2], a[3]);
  u[2] = cvt_pk_bf16(b[0], b[1]);
  u[3] = cvt_pk_bf16(b[2], b[3]);
  *reinterpret_cast<u32x4*>(o + 8 * i) = u;
}

size_t mamba2_chunk_state_bwd_workspace(int rows, int H, int D, int N) {
  // the two-head form runs where its LDS fits: head_dim 64 (d_state 64 or 128)
  if (D != 64) return 0;
  return (size_t)rows * H * D * N * 2;
}

// ---------------------------------------------------------------- launchers
template <int D, int N>
static void launch_fwd_dn(const StateArgs& a, hipStream_t stream) {
  // two heads per workgroup where that keeps three workgroups per CU (at configs[4]:
  // 163 us against 205 us for one head; four heads per workgroup fit one workgroup per
  // CU and ran 216 us)
  if (D * N <= 64 * 128 && (a.H / a.G) % 2 == 0) {
    hipLaunchKernelGGL((mamba2_chunk_state_kernel<D, N, 2>),
                       dim3((unsigned)(a.rows * (a.H / 2) * a.split)), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((mamba2_chunk_state_kernel<D, N, 1>),
                       dim3((unsigned)(a.rows * a.H * a.split)), dim3(256), 0, stream, a);
  }
}
template <int D, int N>
static void launch_bwd_dn(const StateArgs& a, hipStream_t stream) {
  const int nbt = (a.T + 255) / 256;
  hipLaunchKernelGGL((mamba2_chunk_state_bwd_kernel<D, N>), dim3((unsigned)(a.rows * a.G * nbt)),
                     dim3(512), 0, stream, a);
}

#define RMX_STATE_DISPATCH(FN, D, N, A, S)         \
  if ((D) == 64 && (N) == 64) FN<64, 64>(A, S);    \
  else if ((D) == 64 && (N) == 128) FN<64, 128>(A, S); \
  else if ((D) == 128 && (N) == 64) FN<128, 64>(A, S); \
  else FN<128, 128>(A, S);

hipError_t launch_mamba2_chunk_state(const uint16_t* x, const uint16_t* B, const float* e,
                                     const float* cum_A, const int32_t* t0, float* state,
                                     int rows, int T, int H, int D, int G, int N,
                                     hipStream_t stream) {
  StateArgs a{};
  a.x = x;
  a.B = B;
  a.e = e;
  a.cum_A = cum_A;
  a.t0 = t0;
  a.state = state;
  a.rows = rows;
  a.T = T;
  a.H = H;
  a.G = G;
  // a second workgroup per (row, head) when fewer than 4 per CU would run
  a.split = ((int64_t)rows * H < 1024 && T >= 1024) ? 2 : 1;
  if (a.split == 2 || T == 0) {  // atomically summed halves / the empty shard's zero state
    const int64_t n = (int64_t)rows * H * D * N;
    hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       state, n);
    if (T == 0) return hipGetLastError();
  }
  RMX_STATE_DISPATCH(launch_fwd_dn, D, N, a, stream)
  return hipGetLastError();
}

hipError_t launch_mamba2_chunk_state_bwd(const uint16_t* x, const uint16_t* B, const float* e,
                                         const float* cum_A, const int32_t* t0,
                                         const float* g_state, uint16_t* g_x, uint16_t* g_B,
                                         float* g_e, float* g_cum, int rows, int T, int H, int D,
                                         int G, int N, void* workspace, hipStream_t stream) {
  StateArgs a{};
  a.x = x;
  a.B = B;
  a.e = e;
  a.cum_A = cum_A;
  a.t0 = t0;
  a.g_state = g_state;
  a.g_x = g_x;
  a.g_B = g_B;
  a.g_e = g_e;
  a.g_cum = g_cum;
  a.rows = rows;
  a.T = T;
  a.H = H;
  a.G = G;
  a.split = 1;
  if (workspace && mamba2_chunk_state_bwd_workspace(rows, H, D, N) > 0) {
    uint16_t* gws = static_cast<uint16_t*>(workspace);
    const int64_t n8 = (int64_t)rows * H * D * N / 8;
    hipLaunchKernelGGL(g_state_bf16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                       stream, g_state, gws, n8);
    const unsigned grid = (unsigned)(rows * G * ((T + 127) / 128));
    if (N == 128)
      hipLaunchKernelGGL((mamba2_chunk_state_bwd2_kernel<64, 128>), dim3(grid), dim3(512), 0,
                         stream, a, gws);
    else
      hipLaunchKernelGGL((mamba2_chunk_state_bwd2_kernel<64, 64>), dim3(grid), dim3(512), 0,
                         stream, a, gws);
    return hipGetLastError();
  }
  RMX_STATE_DISPATCH(launch_bwd_dn, D, N, a, stream)
  return hipGetLastError();
}

}  // namespace rmx
