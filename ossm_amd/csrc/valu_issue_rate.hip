// VALU issue-rate microbenchmark for gfx950: the cycle costs behind the VALU
// floors of the selective-scan kernels.  A standalone program (built next to
// the library as _lib/valu_issue_rate, run by `python bench.py --issue-rate`);
// it is not part of libossm_scan.so.
//
// Part 1, throughput: every lane runs 8 independent chains (no dependency
// stall) of one operation kind; grids of 1, 2, 4 and 8 workgroups of 256
// threads per CU put that many waves on each SIMD.  Printed: SIMD cycles per
// wave-instruction at 2.4 GHz.  Part 2, a single wave's issue rate against the
// number of independent chains (1, 2, 4, 8) at one and two waves per SIMD.
//
// Every thread writes at most one float of a 1024-float buffer (only when a
// sum that cannot occur appears, so the compiler keeps the loops); the loops
// have fixed trip counts.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

constexpr int kThreads = 256;  // four waves: one per SIMD of a CU
constexpr double kClock = 2.4e9;

#define CHECK(x)                                                            \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));          \
      std::exit(1);                                                         \
    }                                                                       \
  } while (0)

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

enum Kind { kFma = 0, kMulExp = 1, kExp = 2, kDppAdd = 3, kSwapAdd = 4 };
const char* kKindName[] = {"v_fma_f32", "v_mul_f32 + v_exp_f32", "v_exp_f32", "v_add_f32 (row DPP)",
                           "v_permlane32_swap + v_add_f32"};
// wave-instructions per chain step
constexpr int kInstrPerOp[] = {1, 2, 1, 1, 2};

template <int KIND, int ILP>
__global__ __launch_bounds__(kThreads) void issue_kernel(float* out, int iters, float c) {
  float x[ILP];
#pragma unroll
  for (int j = 0; j < ILP; ++j) x[j] = static_cast<float>(threadIdx.x) * 1e-3f + static_cast<float>(j) * 0.1f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 16 / ILP; ++r) {
#pragma unroll
      for (int j = 0; j < ILP; ++j) {
        if constexpr (KIND == kFma) {
          x[j] = fmaf(x[j], c, 0.5f);
        } else if constexpr (KIND == kMulExp) {
          x[j] = __builtin_amdgcn_exp2f(x[j] * c);
        } else if constexpr (KIND == kExp) {
          x[j] = __builtin_amdgcn_exp2f(x[j]);
        } else if constexpr (KIND == kDppAdd) {
          x[j] += dpp<0x141>(x[j]);  // row_half_mirror
        } else {
          const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[j]), __float_as_uint(c), false, false);
          x[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
        }
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < ILP; ++j) s += x[j];
  if (s == 1234.5f) out[threadIdx.x] = s;
}

// Average ms of one launch of `blocks` workgroups, over 5 timed launches after one untimed.
template <int KIND, int ILP>
float time_launch(float* out, int blocks, int iters) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  issue_kernel<KIND, ILP><<<blocks, kThreads>>>(out, iters, 0.999f);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(a));
  for (int r = 0; r < 5; ++r) issue_kernel<KIND, ILP><<<blocks, kThreads>>>(out, iters, 0.999f);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return ms / 5.f;
}

// cycles per wave-instruction: per SIMD (all its waves together) and per wave
template <int KIND, int ILP>
void report(float* out, int ncu, int waves_per_simd, int iters, const char* part) {
  const float ms = time_launch<KIND, ILP>(out, ncu * waves_per_simd, iters);
  const double instr_per_wave = static_cast<double>(iters) * 16 * kInstrPerOp[KIND];
  const double cycles = ms * 1e-3 * kClock;
  std::printf("%s | %-30s | chains %d | waves/SIMD %d | %.2f cycles per wave-instruction per SIMD | %.2f per wave\n",
              part, kKindName[KIND], ILP, waves_per_simd, cycles / (instr_per_wave * waves_per_simd),
              cycles / instr_per_wave);
}

template <int KIND>
void part1(float* out, int ncu) {
  for (int w = 1; w <= 8; w *= 2) report<KIND, 8>(out, ncu, w, 4096, "throughput");
}

template <int KIND>
void part2(float* out, int ncu) {
  for (int w = 1; w <= 2; ++w) {
    report<KIND, 1>(out, ncu, w, 2048, "single-wave");
    report<KIND, 2>(out, ncu, w, 2048, "single-wave");
    report<KIND, 4>(out, ncu, w, 2048, "single-wave");
    report<KIND, 8>(out, ncu, w, 2048, "single-wave");
  }
}

}  // namespace

int main() {
  int ncu = 0;
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
  float* out = nullptr;
  CHECK(hipMalloc(&out, 1024 * sizeof(float)));
  std::printf("CUs %d, cycles at %.1f GHz\n", ncu, kClock * 1e-9);
  part1<kFma>(out, ncu);
  part1<kMulExp>(out, ncu);
  part1<kExp>(out, ncu);
  part2<kFma>(out, ncu);
  part2<kDppAdd>(out, ncu);
  part2<kExp>(out, ncu);
  part2<kSwapAdd>(out, ncu);
  CHECK(hipFree(out));
  return 0;
}
