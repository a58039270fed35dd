// Reductions shared by the scan backwards: per-channel partial sums of every
// (time chunk, batch row) reduced to one value per state column (fixed-order
// fp64 sums per row group, row groups combined with float atomics), and a
// graph-safe zero fill.
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
// (c * NS + j) * nc + b * P + p.  Column sums in one launch: block (column
// tile of 64, row group g) sums rows r = g*4 + w + k*4G (w = wave) in fp64,
// four rows in flight per lane, waves combined through LDS in a fixed order,
// then calls Epi::add(p, S) with its row group's NS sums.  Every epilogue here
// is linear in the sums (parameter gradients = a per-column Jacobian times
// them), so each row group applies it to its own share and adds the result to
// the zero-initialised outputs with one hardware float atomic per output: the
// 64-way combine is the only unordered step.  (Finishing a column inside one
// launch without atomics costs a cross-block handoff, measured no cheaper than
// a second launch: 20 us with a fetch-add counter and tagged fp64 row-group
// sums, 68 us with a compare-and-swap counter, 77 us with an acq_rel counter
// whose release writes back an L2 still dirty with the scan's output rows.)
constexpr int kRowGroups = kWave;
constexpr int kColsumRows = 4;  // rows per lane per round (independent loads)

template <int NS, class PT, class Epi>
__global__ __launch_bounds__(256) void column_sum_kernel(const PT* __restrict__ partials, int P,
                                                         int B, int n_chunks, Epi epi) {
  __shared__ double s_red[4][NS][kWave];
  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int p = blockIdx.x * kWave + lane;
  const int pc = min(p, P - 1);
  const int g = blockIdx.y;
  const size_t nc = static_cast<size_t>(B) * P;
  const int R = n_chunks * B;
  constexpr int kStride = kRowGroups * 4;
  if (g * 4 >= R) return;  // an empty row group adds nothing
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
    double S[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j)
      S[j] = ((s_red[0][j][lane] + s_red[1][j][lane]) + s_red[2][j][lane]) + s_red[3][j][lane];
    epi.add(p, S);
  }
}

// Column sums of `partials` ([n_chunks][NS][B * P]) added into Epi's outputs,
// which must hold zeros when the kernel starts.
template <int NS, class PT, class Epi>
int launch_column_sums(const PT* partials, int64_t P, int64_t B, int64_t n_chunks, const Epi& epi,
                       hipStream_t stream) {
  hipLaunchKernelGGL((column_sum_kernel<NS, PT, Epi>),
                     dim3(static_cast<unsigned>((P + kWave - 1) / kWave), kRowGroups), dim3(256), 0,
                     stream, partials, static_cast<int>(P), static_cast<int>(B),
                     static_cast<int>(n_chunks), epi);
  return launch_check("column_sum_kernel");
}

// Output accumulation for the epilogues: one hardware float atomic add.
__device__ __forceinline__ void atomic_put(float* dst, double v) {
  unsafeAtomicAdd(dst, static_cast<float>(v));
}
__device__ __forceinline__ void atomic_put(double* dst, double v) { unsafeAtomicAdd(dst, v); }

// Up to three output arrays a backward scan kernel clears before the column
// sums add into them (the workgroup with the first ticket does it; the
// column-sum launch runs after the scan kernel has finished).
struct ZeroFill {
  float* p[3];
  int n[3];  // floats per array
};

__device__ __forceinline__ void zero_fill_block(const ZeroFill& z) {
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if (z.p[k] != nullptr)
      for (int i = threadIdx.x; i < z.n[k]; i += blockDim.x) z.p[k][i] = 0.f;
}

// The same zero-fill for outputs that the launch's own workgroups then add
// into (one launch, no column-sum kernel): the workgroup of order 0 writes
// the zeros through to memory with agent-scope stores, waits until they have
// all completed, and then publishes the launch's tag in sync.flag.  A
// workgroup adds its share only after it has read that tag
// (wait_outputs_zeroed), so no add can land before a zero.  The order-0
// workgroup is the first to start, so the wait is over long before any
// workgroup reaches its adds.
__device__ __forceinline__ void zero_fill_publish(const ZeroFill& z, const LaunchSync& sync) {
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if (z.p[k] != nullptr)
      for (int i = threadIdx.x; i < z.n[k]; i += blockDim.x)
        __hip_atomic_store(reinterpret_cast<unsigned int*>(z.p[k]) + i, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // every zero of this thread is in memory
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(sync.flag, static_cast<unsigned long long>(sync.tag), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Waits (bounded) until this launch's outputs are zeroed; false after a
// spin that gave up (kErrSpinTimeout raised: the caller adds NaN instead).
__device__ __forceinline__ bool wait_outputs_zeroed(const LaunchSync& sync) {
  uint32_t spins = 0;
  while (__hip_atomic_load(sync.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
         static_cast<unsigned long long>(sync.tag)) {
    if (++spins > kSpinLimit) {
      __hip_atomic_fetch_or(sync.err, kErrSpinTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return true;
}

// Zero-fill used where the reference returns zero gradients (empty scans).
// A kernel rather than hipMemsetAsync: memset nodes are not trusted inside
// graphs on this platform, and a caller may capture the surrounding work.
__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// n floats (all-zero bits, so also n / 2 doubles).
[[maybe_unused]] int fill_zero(float* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return OSSM_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
  return launch_check("fill_zero_kernel");
}

}  // namespace
}  // namespace ossm
