// Reductions shared by the scan backwards: per-channel partial sums of every
// (time chunk, batch row) reduced to one value per state column, in a fixed
// order in fp64 (no atomics), and a graph-safe zero fill.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_device.hpp"

namespace ossm {
namespace {

// The partials form, for each sum j, a matrix of R = n_chunks * B rows
// (chunk c, batch row b) by P columns (state column p): address
// (c * NS + j) * nc + b * P + p.  Column sums in two passes:
//   pass 1: block (column tile of 64, row group g) sums rows r = g*4 + w + k*4G
//           (w = wave) in fp64, four rows in flight per lane, waves combined
//           through LDS -> colsum[g][j][p];
//   pass 2 (per model): one wave per column, lane g holding row group g,
//           adds them by a butterfly over the wave, then the model's chain rule.
// Fixed order everywhere (no atomics).
constexpr int kRowGroups = kWave;
constexpr int kColsumRows = 4;  // rows per lane per round (independent loads)

template <int NS, class PT = float>
__global__ __launch_bounds__(256) void osc_colsum_kernel(const PT* __restrict__ partials,
                                                         double* __restrict__ colsum, int P,
                                                         int B, int n_chunks) {
  __shared__ double s_red[4][NS][kWave];
  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int p = blockIdx.x * kWave + lane;
  const int pc = min(p, P - 1);
  const int g = blockIdx.y;
  const size_t nc = static_cast<size_t>(B) * P;
  const int R = n_chunks * B;
  constexpr int kStride = kRowGroups * 4;
  double acc[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) acc[j] = 0.0;
  for (int r0 = g * 4 + w; r0 < R; r0 += kStride * kColsumRows) {
    PT v[kColsumRows][NS];
#pragma unroll
    for (int u = 0; u < kColsumRows; ++u) {
      const int r = min(r0 + u * kStride, R - 1);
      const int c = r / B, b = r - c * B;
      const PT* src = partials + static_cast<size_t>(c) * NS * nc + static_cast<size_t>(b) * P + pc;
#pragma unroll
      for (int j = 0; j < NS; ++j) v[u][j] = src[j * nc];
    }
#pragma unroll
    for (int u = 0; u < kColsumRows; ++u)
      if (r0 + u * kStride < R) {
#pragma unroll
        for (int j = 0; j < NS; ++j) acc[j] += static_cast<double>(v[u][j]);
      }
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) s_red[w][j][lane] = acc[j];
  __syncthreads();
  if (w == 0 && p < P) {
#pragma unroll
    for (int j = 0; j < NS; ++j)
      colsum[(static_cast<size_t>(g) * NS + j) * P + p] =
          ((s_red[0][j][lane] + s_red[1][j][lane]) + s_red[2][j][lane]) + s_red[3][j][lane];
  }
}

// Launches pass 1 over `partials` ([n_chunks][NS][B * P]) into `colsum`
// ([kRowGroups][NS][P]).
template <int NS, class PT>
int launch_colsum(const PT* partials, double* colsum, int64_t P, int64_t B, int64_t n_chunks,
                  hipStream_t stream) {
  hipLaunchKernelGGL((osc_colsum_kernel<NS, PT>),
                     dim3(static_cast<unsigned>((P + kWave - 1) / kWave), kRowGroups), dim3(256), 0,
                     stream, partials, colsum, static_cast<int>(P), static_cast<int>(B),
                     static_cast<int>(n_chunks));
  return launch_check("osc_colsum_kernel");
}

// Zero-fill used where the reference returns zero gradients (empty scans);
// a kernel rather than hipMemsetAsync so the call can sit in a captured graph.
__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// n floats (all-zero bits, so also n / 2 doubles).
int fill_zero(float* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return OSSM_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
  return launch_check("fill_zero_kernel");
}

}  // namespace
}  // namespace ossm
