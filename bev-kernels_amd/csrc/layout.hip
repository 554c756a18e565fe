// Layout changes for gfx950: dst[b][c][r] = src[b][r][c] (the last two dimensions
// swapped), used to go between the NCHW module API and the NHWC kernels.
//
// 64 x 64 tiles through LDS: a 256-thread block reads 64 rows of the source tile with
// 4-element vector loads (whole rows of 64 elements per 16 threads), keeps the tile in LDS
// as 32-bit words (pitch 65, so the transposed reads hit 64 different banks), and writes
// 64 rows of the destination tile the same way. Every HBM byte is read once and written
// once with full-row accesses on both sides.
#include "bevk_common.h"
#include "bevk_launch.h"

namespace bevk {
namespace {

constexpr int kTile = 64;
constexpr int kTBlock = 256;

template <typename E, bool VEC>
__global__ void __launch_bounds__(kTBlock) transpose_kernel(const E *__restrict__ src,
                                                            E *__restrict__ dst, int R, int C) {
  __shared__ uint32_t tile[kTile][kTile + 1];
  const int b = blockIdx.z;
  const int r0 = blockIdx.y * kTile, c0 = blockIdx.x * kTile;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const E *s = src + (int64_t)b * R * C;
  E *d = dst + (int64_t)b * R * C;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty + 16 * i, c = c0 + 4 * tx;
    E v[4];
    if (VEC && r < R && c + 3 < C) {
      const Vec<E, 4> w = *reinterpret_cast<const Vec<E, 4> *>(s + (int64_t)r * C + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = w.v[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (r < R && c + e < C) ? s[(int64_t)r * C + c + e] : E(0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[ty + 16 * i][4 * tx + e] = (uint32_t)v[e];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + ty + 16 * i, r = r0 + 4 * tx;  // destination row c, columns r..r+3
    Vec<E, 4> w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w.v[e] = (E)tile[4 * tx + e][ty + 16 * i];
    if (c >= C) continue;
    if (VEC && r + 3 < R) {
      *reinterpret_cast<Vec<E, 4> *>(d + (int64_t)c * R + r) = w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r + e < R) d[(int64_t)c * R + r + e] = w.v[e];
    }
  }
}

template <typename E>
hipError_t launch_t(const void *src, void *dst, int batch, int rows, int cols,
                    hipStream_t stream) {
  const bool vec = rows % 4 == 0 && cols % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(src) % (4 * sizeof(E))) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst) % (4 * sizeof(E))) == 0;
  dim3 grid((cols + kTile - 1) / kTile, (rows + kTile - 1) / kTile, batch);
  if (vec)
    hipLaunchKernelGGL((transpose_kernel<E, true>), grid, dim3(kTBlock), 0, stream,
                       static_cast<const E *>(src), static_cast<E *>(dst), rows, cols);
  else
    hipLaunchKernelGGL((transpose_kernel<E, false>), grid, dim3(kTBlock), 0, stream,
                       static_cast<const E *>(src), static_cast<E *>(dst), rows, cols);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_transpose(int elem_bytes, const void *src, void *dst, int batch, int rows,
                            int cols, hipStream_t stream) {
  if (batch == 0 || rows == 0 || cols == 0) return hipSuccess;
  if (elem_bytes == 4) return launch_t<uint32_t>(src, dst, batch, rows, cols, stream);
  if (elem_bytes == 2) return launch_t<uint16_t>(src, dst, batch, rows, cols, stream);
  return hipErrorInvalidValue;
}

}  // namespace bevk
