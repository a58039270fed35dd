// The Mamba mixer's causal depthwise convolution + SiLU on gfx950, forward and
// backward, in the mixer's own [B, L, D] layout (mambarec.py:143-150 runs it
// as transpose -> pad -> Conv1d -> SiLU -> transpose):
//
//   pre[b,t,d] = bias[d] + sum_{k<K} w[d,k] x[b, t-K+1+k, d]      (x = 0 before t = 0)
//   out[b,t,d] = pre * sigmoid(pre)
//
// x is [B, L, D] with row stride ld_x (the x half of in_proj's [B, L, 2D]
// output is such a view), out dense [B, L, D]; w [D, K] (Conv1d's [D, 1, K]),
// bias [D] or null.  Backward, with dpre = dout * silu'(pre):
//   dx[t] = sum_k w[k] dpre[t+K-1-k],  dw[d,k] = sum_{b,t} dpre[b,t,d] x[b,t-K+1+k,d],
//   dbias[d] = sum_{b,t} dpre[b,t,d].
//
// Memory-bound elementwise work: a thread owns 4 channels (16-byte runs along
// d, so a wave moves 1 KiB per step) and a span of steps, keeping the K-1
// previous inputs in registers.  The weight and bias gradients are per-thread
// partial sums over its span, written per (batch row, span) and added by a
// second kernel in a fixed order in fp64 (deterministic).

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"

namespace ossm {
namespace {

constexpr int kConvThreads = 256;
constexpr int kFwdSpan = 16;   // steps per thread, forward
constexpr int kBwdTile = 8;    // steps per register tile, backward
constexpr int kBwdSpan = 128;  // steps per thread, backward (kBwdSpan / kBwdTile tiles)
constexpr int kMaxK = 8;

struct ConvArgs {
  const float* x;     // [B, L, D], row stride ld_x
  const float* w;     // [D, K]
  const float* bias;  // [D] or null
  const float* dout;  // backward: [B, L, D] dense
  float* out;         // forward: [B, L, D] dense; backward: dx [B, L, D] dense
  float* partials;    // backward: [B * n_spans][K + 1][D]
  int B, L, D, ld_x;
};

__device__ __forceinline__ float sigm(float p) { return 1.f / (1.f + __expf(-p)); }

// C channels per thread (4 with 16-byte moves, else 1), as a fixed-size vector.
template <int C>
struct Vec {
  float v[C];
};

template <int C>
__device__ __forceinline__ Vec<C> load_vec(const float* p) {
  Vec<C> r;
  if constexpr (C == 4) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    r.v[0] = q.x; r.v[1] = q.y; r.v[2] = q.z; r.v[3] = q.w;
  } else {
    r.v[0] = *p;
  }
  return r;
}

template <int C>
__device__ __forceinline__ void store_vec(float* p, const Vec<C>& r) {
  if constexpr (C == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
  } else {
    *p = r.v[0];
  }
}

template <int C>
__device__ __forceinline__ Vec<C> zero_vec() {
  Vec<C> r;
#pragma unroll
  for (int e = 0; e < C; ++e) r.v[e] = 0.f;
  return r;
}

// x[b, t, d..] or zeros outside [0, L)
template <int C>
__device__ __forceinline__ Vec<C> x_at(const ConvArgs& a, size_t xb, int t, int d) {
  if (t < 0 || t >= a.L) return zero_vec<C>();
  return load_vec<C>(a.x + xb + static_cast<size_t>(t) * a.ld_x + d);
}

template <int K, int C>
__device__ __forceinline__ void load_weights(const ConvArgs& a, int d, float (&w)[K][C],
                                             float (&bias)[C]) {
#pragma unroll
  for (int e = 0; e < C; ++e) {
#pragma unroll
    for (int k = 0; k < K; ++k) w[k][e] = a.w[static_cast<size_t>(d + e) * K + k];
    bias[e] = a.bias != nullptr ? a.bias[d + e] : 0.f;
  }
}

// grid (channel groups, spans of kFwdSpan steps, batch)
template <int K, int C>
__global__ __launch_bounds__(kConvThreads) void conv_silu_fwd_kernel(ConvArgs a) {
  const int d = (blockIdx.x * kConvThreads + threadIdx.x) * C;
  if (d >= a.D) return;  // no barriers below
  const int b = blockIdx.z, t0 = blockIdx.y * kFwdSpan;
  const size_t xb = static_cast<size_t>(b) * a.L * a.ld_x;
  const size_t ob = static_cast<size_t>(b) * a.L * a.D;
  float w[K][C], bias[C];
  load_weights<K, C>(a, d, w, bias);
  // inputs t0-K+1 .. t0+kFwdSpan-1, all loaded before any is used
  Vec<C> xs[kFwdSpan + K - 1];
#pragma unroll
  for (int i = 0; i < kFwdSpan + K - 1; ++i) xs[i] = x_at<C>(a, xb, t0 - K + 1 + i, d);
#pragma unroll
  for (int i = 0; i < kFwdSpan; ++i) {
    const int t = t0 + i;
    if (t >= a.L) break;
    Vec<C> y;
#pragma unroll
    for (int e = 0; e < C; ++e) {
      float p = bias[e];
#pragma unroll
      for (int k = 0; k < K; ++k) p = fmaf(w[k][e], xs[i + k].v[e], p);
      y.v[e] = p * sigm(p);
    }
    store_vec<C>(a.out + ob + static_cast<size_t>(t) * a.D + d, y);
  }
}

// grid (channel groups, spans of kBwdSpan steps, batch)
template <int K, int C>
__global__ __launch_bounds__(kConvThreads) void conv_silu_bwd_kernel(ConvArgs a) {
  const int d = (blockIdx.x * kConvThreads + threadIdx.x) * C;
  if (d >= a.D) return;  // no barriers below
  const int b = blockIdx.z, span = blockIdx.y;
  const size_t xb = static_cast<size_t>(b) * a.L * a.ld_x;
  const size_t ob = static_cast<size_t>(b) * a.L * a.D;
  float w[K][C], bias[C];
  load_weights<K, C>(a, d, w, bias);
  float gw[K][C], gb[C];
#pragma unroll
  for (int e = 0; e < C; ++e) {
    gb[e] = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) gw[k][e] = 0.f;
  }
  constexpr int NX = kBwdTile + 2 * (K - 1);  // inputs for pre over the tile and its K-1 successors
  constexpr int NP = kBwdTile + K - 1;        // dpre over the tile and its K-1 successors
  for (int t0 = span * kBwdSpan; t0 < min(a.L, (span + 1) * kBwdSpan); t0 += kBwdTile) {
    Vec<C> xs[NX], dp[NP];
#pragma unroll
    for (int i = 0; i < NX; ++i) xs[i] = x_at<C>(a, xb, t0 - K + 1 + i, d);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int t = t0 + i;
      const Vec<C> go = t < a.L ? load_vec<C>(a.dout + ob + static_cast<size_t>(t) * a.D + d) : zero_vec<C>();
#pragma unroll
      for (int e = 0; e < C; ++e) {
        float p = bias[e];
#pragma unroll
        for (int k = 0; k < K; ++k) p = fmaf(w[k][e], xs[i + k].v[e], p);
        const float s = sigm(p);
        dp[i].v[e] = t < a.L ? go.v[e] * (s * (1.f + p * (1.f - s))) : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < kBwdTile; ++i) {
      const int t = t0 + i;
      if (t >= a.L) break;
      Vec<C> gx;
#pragma unroll
      for (int e = 0; e < C; ++e) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) s = fmaf(w[k][e], dp[i + K - 1 - k].v[e], s);
        gx.v[e] = s;
        gb[e] += dp[i].v[e];
#pragma unroll
        for (int k = 0; k < K; ++k) gw[k][e] = fmaf(dp[i].v[e], xs[i + k].v[e], gw[k][e]);
      }
      store_vec<C>(a.out + ob + static_cast<size_t>(t) * a.D + d, gx);
    }
  }
  // partials row (b, span): [K + 1][D]
  const int n_spans = gridDim.y;
  float* prow = a.partials + (static_cast<size_t>(b) * n_spans + span) * (K + 1) * a.D;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    Vec<C> v;
#pragma unroll
    for (int e = 0; e < C; ++e) v.v[e] = gw[k][e];
    store_vec<C>(prow + static_cast<size_t>(k) * a.D + d, v);
  }
  Vec<C> v;
#pragma unroll
  for (int e = 0; e < C; ++e) v.v[e] = gb[e];
  store_vec<C>(prow + static_cast<size_t>(K) * a.D + d, v);
}

// grad_w[d, k] (j < K) and grad_bias[d] (j = K): the R partial rows added in
// row order in fp64.  One thread per (j, d).
__global__ void conv_param_sum_kernel(const float* __restrict__ partials, int R, int KP1, int D,
                                      float* __restrict__ grad_w, float* __restrict__ grad_bias) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(KP1) * D) return;
  const int j = static_cast<int>(i / D), d = static_cast<int>(i - static_cast<int64_t>(j) * D);
  const size_t stride = static_cast<size_t>(KP1) * D;
  double s = 0.0;
  for (int r = 0; r < R; ++r) s += static_cast<double>(partials[r * stride + i]);
  if (j < KP1 - 1) {
    grad_w[static_cast<size_t>(d) * (KP1 - 1) + j] = static_cast<float>(s);
  } else if (grad_bias != nullptr) {
    grad_bias[d] = static_cast<float>(s);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_conv(int64_t B, int64_t L, int64_t D, int64_t K, int64_t ld_x, const char* what) {
  if (B < 0 || L < 0 || D < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (K < 1 || K > kMaxK)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": kernel width 1.." +
                                               std::to_string(kMaxK) + " supported, got " +
                                               std::to_string(K));
  if (ld_x < D) return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": ld_x < D");
  if (B > 65535 || L > int64_t(65535) * kFwdSpan || D > INT_MAX / 8 || ld_x > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds launch limits");
  return OSSM_OK;
}

template <int K>
int launch_fwd(const ConvArgs& a, bool vec, hipStream_t stream) {
  const int C = vec ? 4 : 1;
  const int64_t groups = (a.D / C + kConvThreads - 1) / kConvThreads;
  const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>((a.L + kFwdSpan - 1) / kFwdSpan),
                  static_cast<unsigned>(a.B));
  if (vec)
    hipLaunchKernelGGL((conv_silu_fwd_kernel<K, 4>), grid, dim3(kConvThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((conv_silu_fwd_kernel<K, 1>), grid, dim3(kConvThreads), 0, stream, a);
  return launch_check("conv_silu_fwd_kernel");
}

template <int K>
int launch_bwd(const ConvArgs& a, bool vec, int n_spans, hipStream_t stream) {
  const int C = vec ? 4 : 1;
  const int64_t groups = (a.D / C + kConvThreads - 1) / kConvThreads;
  const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(n_spans),
                  static_cast<unsigned>(a.B));
  if (vec)
    hipLaunchKernelGGL((conv_silu_bwd_kernel<K, 4>), grid, dim3(kConvThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((conv_silu_bwd_kernel<K, 1>), grid, dim3(kConvThreads), 0, stream, a);
  return launch_check("conv_silu_bwd_kernel");
}

template <template <int> class F, class... Args>
int by_width(int K, Args&&... args) {
  switch (K) {
    case 1: return F<1>::run(args...);
    case 2: return F<2>::run(args...);
    case 3: return F<3>::run(args...);
    case 4: return F<4>::run(args...);
    case 5: return F<5>::run(args...);
    case 6: return F<6>::run(args...);
    case 7: return F<7>::run(args...);
    default: return F<8>::run(args...);
  }
}

template <int K>
struct FwdLaunch {
  static int run(const ConvArgs& a, bool vec, hipStream_t s) { return launch_fwd<K>(a, vec, s); }
};
template <int K>
struct BwdLaunch {
  static int run(const ConvArgs& a, bool vec, int n, hipStream_t s) { return launch_bwd<K>(a, vec, n, s); }
};

__global__ void conv_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

int zero(float* p, int64_t n, hipStream_t stream) {
  if (p == nullptr || n <= 0) return OSSM_OK;
  hipLaunchKernelGGL(conv_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, p, n);
  return launch_check("conv_zero_kernel");
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_mamba_conv_forward(const float* x, int64_t ld_x, const float* weight, const float* bias,
                            float* out, int64_t batch, int64_t length, int64_t dim, int64_t width,
                            ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_conv(batch, length, dim, width, ld_x, "mamba_conv_forward")) return rc;
  if (batch == 0 || length == 0 || dim == 0) return OSSM_OK;
  if (!x || !weight || !out)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "mamba_conv_forward: null pointer");
  ConvArgs a{x, weight, bias, nullptr, out, nullptr, static_cast<int>(batch),
             static_cast<int>(length), static_cast<int>(dim), static_cast<int>(ld_x)};
  const bool vec = dim % 4 == 0 && ld_x % 4 == 0 && aligned16(x) && aligned16(out);
  return by_width<FwdLaunch>(static_cast<int>(width), a, vec, static_cast<hipStream_t>(stream_v));
}

int ossm_mamba_conv_backward(const float* x, int64_t ld_x, const float* weight, const float* bias,
                             const float* grad_out, float* grad_x, float* grad_weight,
                             float* grad_bias, int64_t batch, int64_t length, int64_t dim,
                             int64_t width, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_conv(batch, length, dim, width, ld_x, "mamba_conv_backward")) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  if (dim > 0 && (batch == 0 || length == 0)) {
    if (!grad_weight) return set_error(OSSM_ERR_INVALID_ARGUMENT, "mamba_conv_backward: null pointer");
    if (int rc = zero(grad_weight, dim * width, stream)) return rc;
    return zero(grad_bias, dim, stream);
  }
  if (batch == 0 || length == 0 || dim == 0) return OSSM_OK;
  if (!x || !weight || !grad_out || !grad_x || !grad_weight)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "mamba_conv_backward: null pointer");
  const int n_spans = static_cast<int>((length + kBwdSpan - 1) / kBwdSpan);
  const int64_t R = batch * n_spans;
  void* ws = nullptr;
  if (int rc = acquire_workspace(stream, static_cast<size_t>(R * (width + 1) * dim) * sizeof(float), &ws))
    return rc;
  ConvArgs a{x, weight, bias, grad_out, grad_x, static_cast<float*>(ws), static_cast<int>(batch),
             static_cast<int>(length), static_cast<int>(dim), static_cast<int>(ld_x)};
  const bool vec = dim % 4 == 0 && ld_x % 4 == 0 && aligned16(x) && aligned16(grad_out) &&
                   aligned16(grad_x) && aligned16(ws);
  if (int rc = by_width<BwdLaunch>(static_cast<int>(width), a, vec, n_spans, stream)) return rc;
  const int64_t n = (width + 1) * dim;
  hipLaunchKernelGGL(conv_param_sum_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, static_cast<const float*>(ws), static_cast<int>(R),
                     static_cast<int>(width + 1), static_cast<int>(dim), grad_weight, grad_bias);
  return launch_check("conv_param_sum_kernel");
}

}  // extern "C"
