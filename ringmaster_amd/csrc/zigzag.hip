// Zigzag (head_tail) shard / unshard as a coalesced row gather / scatter.
//
// Reference: head_tail_indices (balancers.py:18-29), _zigzag_gidx
// (ring/zigzag.py:40-46) and _zigzag_shard (shard.py:150-176, pad to a
// multiple of 2*world per shard.py:34-36): rank r holds chunks r and
// 2*world-1-r of the padded sequence, early chunk first. The inverse scatter
// is the position-id scatter of tests/test_zigzag_shard.py:39-43.
//
// A token is an opaque row of row_bytes bytes; the kernel moves rows in the
// widest unit (16/8/4/1 bytes) that divides row_bytes and every base address,
// so consecutive lanes touch consecutive bytes of a row (full 64-byte HBM
// bursts). Up to 2^31 units, one unit per thread with 32-bit index arithmetic
// (multiply-high division); beyond, a grid-stride loop with 64-bit indices.
// Padding rows are copied from a caller-provided pad row (zeros when NULL).
#include "rmx_fastdiv.h"
#include "rmx_kernels.h"

namespace rmx {

template <typename U>
__global__ __launch_bounds__(256) void zigzag_kernel32(const char* __restrict__ src,
                                                       char* __restrict__ dst, int seq, int world,
                                                       int rank, uint32_t nunits, uint32_t half,
                                                       FastDiv f_upr, FastDiv f_local,
                                                       FastDiv f_batch, int64_t row_bytes,
                                                       int64_t bstride,
                                                       const char* __restrict__ pad_row,
                                                       int scatter) {
  const uint32_t u = blockIdx.x * 256u + threadIdx.x;
  if (u >= nunits) return;
  const uint32_t row = fdiv(u, f_upr);  // shard row (rank-major over all ranks when rank < 0)
  const uint32_t col = u - row * f_upr.d;
  const uint32_t rb = fdiv(row, f_local);
  const uint32_t i = row - rb * f_local.d;  // position inside the rank's shard
  const uint32_t rr = fdiv(rb, f_batch);
  const uint32_t b = rb - rr * f_batch.d;
  const int64_t r = rank < 0 ? (int64_t)rr : rank;
  const int64_t g = i < half ? r * half + i : (2 * world - 1 - r) * half + (i - half);
  const int64_t shard_off = (int64_t)row * row_bytes;
  const int64_t full_off = (int64_t)b * bstride + g * row_bytes;
  // the destination streams past the caches (non-temporal stores)
  if (scatter) {
    if (g < seq)
      __builtin_nontemporal_store(reinterpret_cast<const U*>(src + shard_off)[col],
                                  reinterpret_cast<U*>(dst + full_off) + col);
  } else {
    U v;
    __builtin_memset(&v, 0, sizeof(U));
    if (g < seq) {
      v = reinterpret_cast<const U*>(src + full_off)[col];
    } else if (pad_row) {
      v = reinterpret_cast<const U*>(pad_row)[col];
    }
    __builtin_nontemporal_store(v, reinterpret_cast<U*>(dst + shard_off) + col);
  }
}

template <typename U>
__global__ __launch_bounds__(256) void zigzag_kernel(const char* __restrict__ src,
                                                     char* __restrict__ dst, int batch, int seq,
                                                     int world, int rank, int64_t upr,
                                                     int64_t row_bytes,
                                                     int64_t bstride,
                                                     const char* __restrict__ pad_row,
                                                     int scatter) {
  const int64_t total_padded = ((int64_t)seq + 2 * world - 1) / (2 * world) * (2 * world);
  const int64_t half = total_padded / (2 * world);
  const int64_t local = 2 * half;
  const int64_t nrows = (int64_t)(rank < 0 ? world : 1) * batch * local;
  const int64_t nunits = nrows * upr;
  U zero;
  __builtin_memset(&zero, 0, sizeof(U));
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < nunits;
       u += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = u / upr;
    const int64_t col = u - row * upr;
    const int64_t i = row % local;
    const int64_t b = (row / local) % batch;
    const int64_t r = rank < 0 ? row / (local * batch) : rank;
    const int64_t g = i < half ? r * half + i : (2 * world - 1 - r) * half + (i - half);
    const int64_t shard_off = row * row_bytes;
    const int64_t full_off = b * bstride + g * row_bytes;
    if (scatter) {
      if (g < seq)
        reinterpret_cast<U*>(dst + full_off)[col] = reinterpret_cast<const U*>(src + shard_off)[col];
    } else {
      U v = zero;
      if (g < seq) {
        v = reinterpret_cast<const U*>(src + full_off)[col];
      } else if (pad_row) {
        v = reinterpret_cast<const U*>(pad_row)[col];
      }
      reinterpret_cast<U*>(dst + shard_off)[col] = v;
    }
  }
}

typedef u32x4 U16;  // 16- and 8-byte units (vector types, so stores can be non-temporal)
typedef u32x2 U8;

hipError_t launch_zigzag(const void* src, void* dst, int batch, int seq, int world, int rank,
                         int64_t row_bytes, int64_t bstride, const void* pad_row, int scatter,
                         hipStream_t stream) {
  const int64_t total_padded = ((int64_t)seq + 2 * world - 1) / (2 * world) * (2 * world);
  const int64_t nrows = (rank < 0 ? total_padded : total_padded / world) * batch;
  if (nrows == 0 || row_bytes == 0) return hipSuccess;
  const uintptr_t al = (uintptr_t)src | (uintptr_t)dst | (uintptr_t)row_bytes | (uintptr_t)bstride |
                       (uintptr_t)pad_row;
  const int unit = (al % 16 == 0) ? 16 : (al % 8 == 0) ? 8 : (al % 4 == 0) ? 4 : 1;
  const int64_t upr = row_bytes / unit;
  const int64_t nunits = nrows * upr;
  if (nunits < (int64_t(1) << 31)) {
    const int64_t half = total_padded / (2 * world);
    const FastDiv fu = make_fastdiv((uint32_t)upr), fl = make_fastdiv((uint32_t)(2 * half)),
                  fb = make_fastdiv((uint32_t)batch);
    const dim3 grid((unsigned)((nunits + 255) / 256));
    const char* s = reinterpret_cast<const char*>(src);
    const char* pr = reinterpret_cast<const char*>(pad_row);
    char* d = reinterpret_cast<char*>(dst);
    const uint32_t nu = (uint32_t)nunits, hf = (uint32_t)half;
    switch (unit) {
      case 16:
        hipLaunchKernelGGL(zigzag_kernel32<U16>, grid, dim3(256), 0, stream, s, d, seq, world, rank,
                           nu, hf, fu, fl, fb, row_bytes, bstride, pr, scatter);
        break;
      case 8:
        hipLaunchKernelGGL(zigzag_kernel32<U8>, grid, dim3(256), 0, stream, s, d, seq, world, rank,
                           nu, hf, fu, fl, fb, row_bytes, bstride, pr, scatter);
        break;
      case 4:
        hipLaunchKernelGGL(zigzag_kernel32<uint32_t>, grid, dim3(256), 0, stream, s, d, seq, world,
                           rank, nu, hf, fu, fl, fb, row_bytes, bstride, pr, scatter);
        break;
      default:
        hipLaunchKernelGGL(zigzag_kernel32<uint8_t>, grid, dim3(256), 0, stream, s, d, seq, world,
                           rank, nu, hf, fu, fl, fb, row_bytes, bstride, pr, scatter);
        break;
    }
    return hipGetLastError();
  }
  int64_t blocks = (nunits + 255) / 256;
  if (blocks > 256 * 128) blocks = 256 * 128;
  const char* s = reinterpret_cast<const char*>(src);
  const char* pr = reinterpret_cast<const char*>(pad_row);
  char* d = reinterpret_cast<char*>(dst);
  switch (unit) {
    case 16:
      hipLaunchKernelGGL(zigzag_kernel<U16>, dim3((unsigned)blocks), dim3(256), 0, stream, s, d,
                         batch, seq, world, rank, upr, row_bytes, bstride, pr, scatter);
      break;
    case 8:
      hipLaunchKernelGGL(zigzag_kernel<U8>, dim3((unsigned)blocks), dim3(256), 0, stream, s, d,
                         batch, seq, world, rank, upr, row_bytes, bstride, pr, scatter);
      break;
    case 4:
      hipLaunchKernelGGL(zigzag_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, stream, s,
                         d, batch, seq, world, rank, upr, row_bytes, bstride, pr, scatter);
      break;
    default:
      hipLaunchKernelGGL(zigzag_kernel<uint8_t>, dim3((unsigned)blocks), dim3(256), 0, stream, s,
                         d, batch, seq, world, rank, upr, row_bytes, bstride, pr, scatter);
      break;
  }
  return hipGetLastError();
}

}  // namespace rmx
