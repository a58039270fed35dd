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
// Memory-bound elementwise work: a thread owns 2 channels in the forward
// (8-byte runs along d, so a wave moves 512 bytes per step), 1 in the
// backward, and a span of steps, loading all of
// the span's inputs (and the K-1 before it) before the first is used; the
// backward walks its span in tiles that share the overlapping inputs and
// pre-activation gradients through registers.  Threads are
// numbered channel group fastest, then span, then batch row, so narrow D still
// fills whole waves.  The weight and bias gradients are per-thread partial
// sums over its span, written per (batch row, span) and reduced over those
// rows by the column-sum kernel shared with the scans (fp64 per row group,
// row groups combined with float atomics).

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_reduce.hpp"

namespace ossm {
namespace {

constexpr int kConvThreads = 256;
constexpr int kFwdSpan = 16;   // steps per thread, forward
constexpr int kBwdTile = 8;    // steps per register tile, backward
constexpr int kBwdSpan = 32;   // steps per thread, backward (kBwdSpan / kBwdTile tiles)
constexpr int kMaxK = 8;

struct ConvArgs {
  const float* x;     // [B, L, D], row stride ld_x
  const float* w;     // [D, K]
  const float* bias;  // [D] or null
  const float* dout;  // backward: [B, L, D] dense
  float* out;         // forward: [B, L, D] dense; backward: dx [B, L, D] dense
  float* partials;    // backward: [B * n_spans][K + 1][D]
  float* grad_w;      // backward: zeroed by the first workgroup (the column sums add into it)
  float* grad_bias;
  int B, L, D, ld_x;
  int n_spans;
};

// The thread's (batch row, span, first channel) in the flat numbering; false
// past the end.
template <int C>
__device__ __forceinline__ bool conv_pos(const ConvArgs& a, int& b, int& span, int& d) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kConvThreads + threadIdx.x;
  const int Q = a.D / C;
  const int64_t rest = gid / Q;
  if (rest >= static_cast<int64_t>(a.B) * a.n_spans) return false;
  d = static_cast<int>(gid - rest * Q) * C;
  span = static_cast<int>(rest % a.n_spans);
  b = static_cast<int>(rest / a.n_spans);
  return true;
}

__device__ __forceinline__ float sigm(float p) { return 1.f / (1.f + __expf(-p)); }

// C channels per thread (2 with 8-byte moves, else 1), as a fixed-size vector.
template <int C>
struct Vec {
  float v[C];
};

template <int C>
__device__ __forceinline__ Vec<C> load_vec(const float* p) {
  Vec<C> r;
  if constexpr (C == 2) {
    const float2 q = *reinterpret_cast<const float2*>(p);
    r.v[0] = q.x; r.v[1] = q.y;
  } else {
    r.v[0] = *p;
  }
  return r;
}

template <int C>
__device__ __forceinline__ void store_vec(float* p, const Vec<C>& r) {
  if constexpr (C == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(r.v[0], r.v[1]);
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

// one thread per (batch row, span of kFwdSpan steps, C channels)
template <int K, int C>
__global__ __launch_bounds__(kConvThreads) void conv_silu_fwd_kernel(ConvArgs a) {
  int b, span, d;
  if (!conv_pos<C>(a, b, span, d)) return;  // no barriers below
  const int t0 = span * kFwdSpan;
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

// one thread per (batch row, span of kBwdSpan steps, C channels)
template <int K, int C>
__global__ __launch_bounds__(kConvThreads) void conv_silu_bwd_kernel(ConvArgs a) {
  if (blockIdx.x == 0) {  // the column sums that follow add into zeroed outputs
    for (int i = threadIdx.x; i < a.D * K; i += kConvThreads) a.grad_w[i] = 0.f;
    if (a.grad_bias != nullptr)
      for (int i = threadIdx.x; i < a.D; i += kConvThreads) a.grad_bias[i] = 0.f;
  }
  int b, span, d;
  if (!conv_pos<C>(a, b, span, d)) return;  // no barriers below
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
  // One sliding window over the span: xs[i] = x at ts - K + 1 + i, dp[i] =
  // dpre at ts + i.  Each tile loads its new inputs and forms its new dpre;
  // the K - 1 values of each it shares with the previous tile stay in
  // registers (the loops are unrolled, so the indices are fixed).
  const int ts = span * kBwdSpan;
  constexpr int NX = kBwdSpan + 2 * (K - 1);
  constexpr int NP = kBwdSpan + K - 1;
  Vec<C> xs[NX], dp[NP];
#pragma unroll
  for (int tile = 0; tile < kBwdSpan / kBwdTile; ++tile) {
    const int base = tile * kBwdTile;
    if (ts + base >= a.L) break;
    constexpr int kShareX = 2 * (K - 1), kShareP = K - 1;
#pragma unroll
    for (int i = (tile == 0 ? 0 : base + kShareX); i < base + kBwdTile + kShareX; ++i)
      xs[i] = x_at<C>(a, xb, ts - K + 1 + i, d);
#pragma unroll
    for (int i = (tile == 0 ? 0 : base + kShareP); i < base + kBwdTile + kShareP; ++i) {
      const int t = ts + i;
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
    for (int j = 0; j < kBwdTile; ++j) {
      const int i = base + j;
      const int t = ts + i;
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
  float* prow = a.partials + (static_cast<size_t>(b) * a.n_spans + span) * (K + 1) * a.D;
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

// Column-sum epilogue: S[k] for k < K is grad_w[d, k], S[K] grad_bias[d].
template <int K>
struct ConvEpilogue {
  float* grad_w;
  float* grad_bias;
  __device__ void add(int d, const double* S) const {
#pragma unroll
    for (int k = 0; k < K; ++k) atomic_put(grad_w + static_cast<size_t>(d) * K + k, S[k]);
    if (grad_bias != nullptr) atomic_put(grad_bias + d, S[K]);
  }
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_conv(int64_t B, int64_t L, int64_t D, int64_t K, int64_t ld_x, const char* what) {
  if (B < 0 || L < 0 || D < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (K < 1 || K > kMaxK)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": kernel width 1.." +
                                               std::to_string(kMaxK) + " supported, got " +
                                               std::to_string(K));
  if (ld_x < D) return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": ld_x < D");
  if (B > 65535 || L > INT_MAX / 2 || D > INT_MAX / 8 || ld_x > INT_MAX || B * L * D > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds launch limits");
  return OSSM_OK;
}

dim3 flat_grid(const ConvArgs& a, int C) {
  const int64_t threads = static_cast<int64_t>(a.B) * a.n_spans * (a.D / C);
  return dim3(static_cast<unsigned>((threads + kConvThreads - 1) / kConvThreads));
}

// The forward takes 2 channels per thread (8-byte moves; a wave still covers
// 512 contiguous bytes of a row), the backward one: its windows of inputs,
// upstream gradients, weights and weight sums grow with the channels (at K = 4:
// 189 VGPRs and two waves per SIMD with 4 channels, 100 and four with 2, 64
// and eight with 1), and this latency-bound kernel needs the waves (C4's
// shape: 182, 154 and 142 us with its column sums); the forward, lighter,
// measured best with 2 (84, 77 and 86 us).
template <int K>
int launch_fwd(const ConvArgs& a, bool vec, hipStream_t stream) {
  const dim3 grid = flat_grid(a, vec ? 2 : 1);
  if (vec)
    hipLaunchKernelGGL((conv_silu_fwd_kernel<K, 2>), grid, dim3(kConvThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((conv_silu_fwd_kernel<K, 1>), grid, dim3(kConvThreads), 0, stream, a);
  return launch_check("conv_silu_fwd_kernel");
}

template <int K>
int launch_bwd(const ConvArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((conv_silu_bwd_kernel<K, 1>), flat_grid(a, 1), dim3(kConvThreads), 0, stream, a);
  if (int rc = launch_check("conv_silu_bwd_kernel")) return rc;
  return launch_column_sums<K + 1>(static_cast<const float*>(a.partials), a.D, 1,
                                   static_cast<int64_t>(a.B) * a.n_spans,
                                   ConvEpilogue<K>{a.grad_w, a.grad_bias}, stream);
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
  static int run(const ConvArgs& a, hipStream_t s) { return launch_bwd<K>(a, s); }
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
  ConvArgs a{x, weight, bias, nullptr, out, nullptr, nullptr, nullptr, static_cast<int>(batch),
             static_cast<int>(length), static_cast<int>(dim), static_cast<int>(ld_x),
             static_cast<int>((length + kFwdSpan - 1) / kFwdSpan)};
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
  StreamCall call(stream);
  if (call.status()) return call.status();
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
  if (int rc = acquire_workspace(call, static_cast<size_t>(R * (width + 1) * dim) * sizeof(float), &ws))
    return rc;
  ConvArgs a{x, weight, bias, grad_out, grad_x, static_cast<float*>(ws), grad_weight, grad_bias,
             static_cast<int>(batch), static_cast<int>(length), static_cast<int>(dim),
             static_cast<int>(ld_x), n_spans};
  return by_width<BwdLaunch>(static_cast<int>(width), a, stream);
}

}  // extern "C"
