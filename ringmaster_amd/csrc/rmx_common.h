// Shared device helpers for the gfx950 (CDNA4) kernels of ringmaster_amd.
//
// MFMA conventions used throughout (v_mfma_f32_32x32x16_bf16, one wave of 64
// lanes, lane = 32*hl + l32):
//   A operand (32 rows x 16 k): lane holds row l32, 8 k-values;
//   B operand (16 k x 32 cols): lane holds col l32, 8 k-values;
//   C/D (32 x 32 fp32, 16 regs): lane holds col l32, reg r holds row
//       8*(r/4) + 4*hl + (r%4).
// The k-order inside an operand only has to agree between A and B, so every
// kernel feeds element i of lane-half hl with k = 8*hl + i.
//
// A C/D tile whose rows were produced from A-rows permuted by sigma (swap of
// index bits 2 and 3) holds, in lane (hl, l32), reg r, the logical row
//   16*(r/8) + 8*hl + (r%8),
// i.e. regs 0..7 and 8..15 are two runs of 8 consecutive rows. That is exactly
// the k-layout of the next MFMA's operand, so softmax probabilities and dS
// feed the second GEMM straight from registers with no LDS round trip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ringmaster_amd.h"

namespace rmx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// sigma: swap bits 2 and 3 of a row index (an involution on 0..31).
__device__ __forceinline__ int sigma(int m) {
  return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Logical row/col held by register r of lane-half hl in a sigma-permuted C tile.
__device__ __forceinline__ int sig_row(int hl, int r) { return 16 * (r >> 3) + 8 * hl + (r & 7); }
// Row held by register r of lane-half hl in a plain C tile.
__device__ __forceinline__ int c_row(int hl, int r) { return 8 * (r >> 2) + 4 * hl + (r & 3); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// Pack 8 floats to a bf16x8 operand.
__device__ __forceinline__ bf16x8 pack8(float v0, float v1, float v2, float v3, float v4, float v5,
                                        float v6, float v7) {
  u32x4 u;
  u[0] = pack_bf2(v0, v1);
  u[1] = pack_bf2(v2, v3);
  u[2] = pack_bf2(v4, v5);
  u[3] = pack_bf2(v6, v7);
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  u32x4 u = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8, u);
}

// LDS tiles of bf16 rows, 16-byte chunks XOR-swizzled by row so that the
// 8-lane groups of a ds_read_b128 hit distinct bank quads.
//  * "row" tiles ([rows][dim], read by sigma-permuted A operands):
//    swizzle f(row) = (row & 3) | ((row >> 1) & 4)  (rows r and r^12 differ).
//  * "t" tiles ([dim][keys], read by rows d = l32): swizzle g(row) = row & 7.
__device__ __forceinline__ int swz_row(int row) { return (row & 3) | ((row >> 1) & 4); }
__device__ __forceinline__ int swz_t(int row) { return row & 7; }

// 16-byte global load/store helpers (bf16x8 / u32x4 bit patterns).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// An empty volatile asm statement: a block containing it cannot be speculated,
// so the compiler keeps a rarely taken branch (the masked-tile path) a branch
// instead of if-converting it into per-element selects on every tile.
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

// Wait for every outstanding memory operation of the wave. Issued once before a
// main loop whose body reads registers filled by loads issued before it: the
// waitcnt pass cannot tell those loads from the loop's own prefetches, and
// would otherwise wait for the prefetches at the first use in every iteration.
__device__ __forceinline__ void wait_all_loads() { __builtin_amdgcn_s_waitcnt(0); }

// Cross-half exchange: value held by lane l ^ 32.
__device__ __forceinline__ float xhalf(float v) { return __shfl_xor(v, 32, 64); }

// ---------------------------------------------------------------------------
// Sliding windows and head dims below the kernel's.
// A problem's window bounds pos_q - pos_k by window_bound(P). kWinMax stands for
// "no window": the host keeps sq and sk below 2^27 (every (batch, head) slice
// spans less than 2 GiB), so no pair is further apart than that and the bound
// arithmetic (positions, offsets and bounds added) stays inside int32.
constexpr int kWinMax = 1 << 29;
template <class Prob>
__device__ __forceinline__ int window_bound(const Prob& P) {
  if (!P.has_window) return kWinMax;
  const int w = P.window_left;
  return w > kWinMax ? kWinMax : (w < -kWinMax ? -kWinMax : w);
}
// A right-bounded window (RMX_MASK_CAUSAL with window_right = R: pos_k - pos_q <= R) is
// the causal mask with its diagonal moved R keys to the right. The kernels take positions
// relative to that diagonal: off = sk - sq + R and the left bound wl + R, so every causal
// and window test (key <= q + off, q + off - key <= wl) reads as for R = 0. The host keeps
// R in [0, 2^28], so the shifted bounds stay inside int32 with kWinMax.
template <int MASK, class Prob>
__device__ __forceinline__ int diag_shift(const Prob& P) {
  return MASK == RMX_MASK_CAUSAL ? P.window_right : 0;
}
__device__ __forceinline__ int clamp_i32(int64_t v) {
  return v > 2147483647 ? 2147483647 : (v < -2147483647 ? -2147483647 : (int)v);
}
// A buffer offset past every num_records (the host keeps them below 2^31): loads
// from it return zeros, LDS DMA from it writes zeros.
constexpr int kOutOfRange = (int)0x80000000u;
// A 16-byte chunk of 8 columns starting at col: kept when col < D, zeros otherwise.
__device__ __forceinline__ u32x4 cols_below(u32x4 v, int col, int D) {
  if (col >= D) v = u32x4{0u, 0u, 0u, 0u};
  return v;
}


}  // namespace rmx

namespace rmx {

// ---------------------------------------------------------------------------
// Buffer-resource loads. A raw buffer (stride 0) returns zeros for any 16-byte
// access whose offset lies at or past num_records, so tiles that run over the
// end of a sequence need no branches and can never read out of bounds.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__device__ u32x4 llvm_raw_buffer_load_v4(i32x4 rsrc, int voffset, int soffset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

// Word 3 = 0x00020000: 32-bit data format, no swizzle/stride (gfx9 family).
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t num_bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = (int32_t)(uint32_t)a;
  r[1] = (int32_t)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = (int32_t)num_bytes;
  r[3] = 0x00020000;
  return r;
}

__device__ __forceinline__ u32x4 buf_load16(const i32x4& rsrc, int byte_off) {
  return llvm_raw_buffer_load_v4(rsrc, byte_off, 0, 0);
}
// Non-temporal form (cache policy NT), for data the grid reads once.
__device__ __forceinline__ u32x4 buf_load16_nt(const i32x4& rsrc, int byte_off) {
  return llvm_raw_buffer_load_v4(rsrc, byte_off, 0, 2);
}

// Stores at or past num_records are dropped by the hardware, so a tile's rows
// past the end of its range need no branch (and every wave issues the same
// number of stores, which keeps vmcnt accounting static).
__device__ void llvm_raw_buffer_store_v4(u32x4 data, i32x4 rsrc, int voffset, int soffset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.store.v4i32");
__device__ __forceinline__ void buf_store16(const i32x4& rsrc, int byte_off, const u32x4& v) {
  llvm_raw_buffer_store_v4(v, rsrc, byte_off, 0, 0);
}
// Non-temporal form (cache policy NT) for data written once and not read back by
// this kernel: whole 128-byte lines stream out without displacing reused lines.
// A store that covers only part of a line is slower in this form.
__device__ __forceinline__ void buf_store16_nt(const i32x4& rsrc, int byte_off, const u32x4& v) {
  llvm_raw_buffer_store_v4(v, rsrc, byte_off, 0, 2);
}

// Bytes a buffer over `rows` rows of `row_bytes` at stride `stride_bytes` must cover.
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t stride_bytes, int row_bytes) {
  return rows <= 0 ? 0u : (uint32_t)((int64_t)(rows - 1) * stride_bytes + row_bytes);
}

// ---------------------------------------------------------------------------
// ds_read_b64_tr_b16 (gfx950): inside each 16-lane group, lane j receives, as
// element i (0..3), the 16-bit element (j % 4) of the 8-byte chunk addressed by
// lane 4*i + j/4. With lane 4*i + q pointing at row (r0 + i), columns
// (c0 + 4q .. c0 + 4q + 3) of a row-major tile, lane j gets column c0 + j of
// rows r0 .. r0 + 3: a 4 x 16 -> 16 x 4 transpose.
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  const bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (__attribute__((address_space(3))) bf16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ bf16x8 join_bf16x8(const u32x2& lo, const u32x2& hi) {
  u32x4 u;
  u[0] = lo[0];
  u[1] = lo[1];
  u[2] = hi[0];
  u[3] = hi[1];
  return __builtin_bit_cast(bf16x8, u);
}

// Hardware round-to-nearest-even packing of two floats (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

__device__ __forceinline__ bf16x8 pack8_hw(const float* v) {
  u32x4 u;
  u[0] = cvt_pk_bf16(v[0], v[1]);
  u[1] = cvt_pk_bf16(v[2], v[3]);
  u[2] = cvt_pk_bf16(v[4], v[5]);
  u[3] = cvt_pk_bf16(v[6], v[7]);
  return __builtin_bit_cast(bf16x8, u);
}

}  // namespace rmx

namespace rmx {

// ---------------------------------------------------------------------------
// Direct global -> LDS loads (buffer_load_dwordx4 ... lds). Lane L of the wave
// writes the 16 bytes at voffset of the buffer to LDS address lds + 16*L
// (lds must be wave-uniform); offsets at or past num_records write zeros.
// Completion is counted by vmcnt.
__device__ void llvm_raw_buffer_load_lds(i32x4 rsrc, __attribute__((address_space(3))) uint32_t* lds,
                                         int size, int voffset, int soffset, int offset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

__device__ __forceinline__ void dma16(const i32x4& rsrc, void* lds, int byte_off) {
  llvm_raw_buffer_load_lds(rsrc, (__attribute__((address_space(3))) uint32_t*)lds, 16, byte_off, 0,
                           0, 0);
}
// The same loads written as inline asm (LDS byte address in M0, set by the
// compiler through the {m0} operand). The compiler does not see these as LDS
// writes, so it inserts no waits for them at later LDS reads (its alias
// tracking of LDS DMA falls back to waiting for every outstanding DMA when a
// kernel has more DMA targets than it can tell apart); the kernel orders them
// itself with wait_vm_barrier. Loads the compiler cannot see only make its own
// vmcnt waits stricter, never weaker. The s_nop covers the M0 -> LDS DMA hazard.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16_async(const i32x4& rsrc, uint32_t lds, int byte_off) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(byte_off), "s"(rsrc),
               "{m0}"(lds)
               : "memory");
}
// Non-temporal form, for operands read once by the whole grid (a streamed input).
__device__ __forceinline__ void dma16_async_nt(const i32x4& rsrc, uint32_t lds, int byte_off) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds" ::"v"(byte_off), "s"(rsrc),
               "{m0}"(lds)
               : "memory");
}
// One dword per lane: lane L writes LDS address lds + 4*L.
__device__ __forceinline__ void dma4_async(const i32x4& rsrc, uint32_t lds, int byte_off) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(byte_off), "s"(rsrc),
               "{m0}"(lds)
               : "memory");
}

// Workgroup barrier that first waits until at most VM vector-memory operations
// (LDS DMA included) of this wave are outstanding and all its LDS operations are
// done. Unlike __syncthreads() it does not wait for every outstanding load, so
// LDS DMA issued for later tiles stays in flight across it. The wait is the
// s_waitcnt builtin, not inline asm, so that the compiler's own wait insertion
// knows which loads it has retired (it would otherwise wait for LDS DMA again
// before the next reads); the empty asm statements keep memory accesses from
// moving across the barrier. Encoding (gfx9): vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[15:14].
template <int VM>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | ((VM >> 4) << 14));  // vmcnt(VM) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Workgroup barrier after this wave's LDS operations only (vector-memory loads,
// LDS DMA included, stay in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// XOR swizzles of the 16-byte chunks of unpadded LDS rows (HD bf16 per row). A row
// of 128 or 256 elements starts at bank 0 (256 or 512 bytes), and a chunk's banks
// depend on its index mod 16 only, so both use the same swizzles (values below 16:
// bit 4 of a 256-element row's chunk index is kept).
// Row reads (16 bytes of 16 consecutive rows, rows permuted by sigma):
template <int HD>
__device__ __forceinline__ int swz_rows(int r) {
  return HD >= 128 ? sigma(r & 15) : ((r >> 1) & 7);
}
// Transposed reads (ds_read_b64_tr_b16 over 4 consecutive rows, 64 bytes each):
template <int HD>
__device__ __forceinline__ int swz_tr(int r) {
  return HD >= 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
}
// Both kinds of read on the same tile:
template <int HD>
__device__ __forceinline__ int swz_both(int r) {
  return HD >= 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

}  // namespace rmx
