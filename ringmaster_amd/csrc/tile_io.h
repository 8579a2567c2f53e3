// Global -> register -> LDS staging of 64-row bf16 tiles for the attention
// kernels. A tile is 64 rows (keys or queries) x HD head-dim values taken from
// a [seq, head, dim] tensor with a contiguous dim axis.
//
// Work split: item = (row quad kq, 16-byte chunk o); a thread loads the chunk o
// of rows 4kq..4kq+3 (four 16-byte loads; the 16 lanes of one row quad read one
// contiguous 256-byte row segment per load). From those registers it can write
//   * a row tile  [64][HD]  (chunk XOR-swizzled by swz_row), and/or
//   * a transposed tile [HD][64] (row d holds 64 consecutive tokens, chunk
//     XOR-swizzled by swz_t), 8-byte writes of 4 tokens for one d.
#pragma once
#include "rmx_common.h"

namespace rmx {

__device__ __forceinline__ int swz_tt(int d) { return (d & 7) ^ ((d >> 3) & 7); }

template <int HD, int NT>
struct TileIO {
  static constexpr int CH = HD / 8;
  static constexpr int ITEMS = 16 * CH;
  static constexpr int PER = (ITEMS + NT - 1) / NT;
  u32x4 r[PER][4];

  // base: element pointer of row 0 of this tile's (batch, head); stride: seq stride.
  __device__ __forceinline__ void load(const uint16_t* __restrict__ base, int64_t stride,
                                       int nvalid, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int item = tid + i * NT;
      if (ITEMS % NT == 0 || item < ITEMS) {
        const int kq = item / CH, o = item % CH;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 4 * kq + j;
          if (row < nvalid) {
            r[i][j] = ld16(base + (int64_t)row * stride + 8 * o);
          } else {
            r[i][j] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store_rows(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int item = tid + i * NT;
      if (ITEMS % NT == 0 || item < ITEMS) {
        const int kq = item / CH, o = item % CH;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 4 * kq + j;
          *reinterpret_cast<u32x4*>(lds + row * HD + 8 * (o ^ swz_row(row))) = r[i][j];
        }
      }
    }
  }

  __device__ __forceinline__ void store_t(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int item = tid + i * NT;
      if (ITEMS % NT == 0 || item < ITEMS) {
        const int kq = item / CH, o = item % CH;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 8 * o + e;
          const uint32_t w0 = r[i][0][e >> 1], w1 = r[i][1][e >> 1];
          const uint32_t w2 = r[i][2][e >> 1], w3 = r[i][3][e >> 1];
          u32x2 v;
          if (e & 1) {
            v[0] = (w0 >> 16) | (w1 & 0xffff0000u);
            v[1] = (w2 >> 16) | (w3 & 0xffff0000u);
          } else {
            v[0] = (w0 & 0xffffu) | (w1 << 16);
            v[1] = (w2 & 0xffffu) | (w3 << 16);
          }
          const int chunk = (kq >> 1) ^ swz_tt(d);
          *reinterpret_cast<u32x2*>(lds + d * 64 + 8 * chunk + 4 * (kq & 1)) = v;
        }
      }
    }
  }
};

// 16-byte LDS operand reads.
__device__ __forceinline__ bf16x8 lds_row_operand(const uint16_t* tile, int HD, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                        tile + row * HD + 8 * (chunk ^ swz_row(row))));
}
__device__ __forceinline__ bf16x8 lds_t_operand(const uint16_t* tile, int d, int chunk) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                        tile + d * 64 + 8 * (chunk ^ swz_tt(d))));
}

}  // namespace rmx
