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
  int T, nheads, head_dim, ngroups, d_state;
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

hipError_t launch_mamba2_correction(const uint16_t* out, uint16_t* y, const float* h_final,
                                    float* h_final_out, const uint16_t* C, const float* cum_A,
                                    const float* h_prev, const int32_t* seq_idx, int batch, int T,
                                    int nheads, int head_dim, int ngroups, int d_state,
                                    hipStream_t stream) {
  MambaCorrArgs a{out, y, h_final, h_final_out, C, cum_A, h_prev, seq_idx,
                  T, nheads, head_dim, ngroups, d_state};
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
