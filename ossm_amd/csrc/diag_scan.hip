// Diagonal complex scans on gfx950 (LRU, S5): x_t = lambda_p * x_{t-1} + b_t
// for every channel (b, p), forward and a native backward, in fp32 (complex64)
// and fp64 (complex128).
//
// Reference: the forward kernels lru_scan.cpp:10-58 and s5_scan.cpp:10-66 (one
// loop, two names; CUDA lru_scan_cuda.cu:33-74 runs one thread per channel),
// and the backward, which the reference runs as a Python loop over time
// (lru.py:52-80, s5.py:137-165):
//   g_t = grad_t + conj(lambda) g_{t+1},   grad_b_t = g_t,
//   grad_lambda_p = sum_{t, b} g_t conj(x_{t-1})   (x_{-1} = 0).
//
// Decomposition (the oscillator scans' skeleton, with a complex scalar as the
// transition): one wave = 64 consecutive channels of the [L, B*P] complex
// tensor (one 512-byte row per step in fp32), a workgroup of W waves owns a
// time chunk of W*T steps, wave w the T steps from w*T.
//   forward:  per-lane aggregate of its T inputs from a zero state, waves
//             combined through LDS with lambda^T, chunk carries handed over
//             by decoupled look-back (tagged records, launch-ticket order),
//             then each wave re-runs its steps from its carry and stores.
//             HBM: read b once, write x once (16 B per state-step in fp32).
//   backward: the same scan in reverse time with conj(lambda); the final pass
//             stores grad_b and accumulates g_t conj(x_{t-1}) per lane from the
//             saved states.  HBM: read grad + states, write grad_b (24 B per
//             state-step).  Each workgroup adds its chunk's per-channel sums
//             into grad_lambda[P] with one hardware float atomic per
//             component, after the launch's order-0 workgroup has zeroed
//             grad_lambda and published its tag (zero_fill_publish): one
//             launch, no partials (a second, column-sum launch cost ~5 us plus
//             the gap between launches at config 2's shape).
//
// Records carry a complex value as 32-bit payload words, each in a 64-bit word
// with the launch tag in its high half (2 words in fp32, 4 in fp64: a double
// is split into its two halves, each tagged), so a reader that sees this
// launch's tag in every word has the complete value.

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_device.hpp"
#include "scan_reduce.hpp"

namespace ossm {
namespace {

// ---- complex scalars ---------------------------------------------------------
template <class R>
struct CxOf;
template <>
struct CxOf<float> {
  using V = float2;
  static constexpr int kWords = 2;  // 32-bit payload words of one record
};
template <>
struct CxOf<double> {
  using V = double2;
  static constexpr int kWords = 4;
};
template <class R>
using Cx = typename CxOf<R>::V;

template <class V>
struct RealOf;
template <>
struct RealOf<float2> {
  using R = float;
};
template <>
struct RealOf<double2> {
  using R = double;
};

__device__ __forceinline__ float2 cx(float re, float im) { return make_float2(re, im); }
__device__ __forceinline__ double2 cx(double re, double im) { return make_double2(re, im); }

template <class V>
__device__ __forceinline__ V cx_zero() {
  using R = typename RealOf<V>::R;
  return cx(R(0), R(0));
}
template <class V>
__device__ __forceinline__ V cx_one() {
  using R = typename RealOf<V>::R;
  return cx(R(1), R(0));
}
template <class V>
__device__ __forceinline__ V cx_add(V a, V b) {
  using R = typename RealOf<V>::R;
  return cx(R(a.x) + R(b.x), R(a.y) + R(b.y));
}
template <class V>
__device__ __forceinline__ V cx_mul(V a, V b) {
  using R = typename RealOf<V>::R;
  const R ar = a.x, ai = a.y, br = b.x, bi = b.y;
  return cx(ar * br - ai * bi, ar * bi + ai * br);
}
template <class V>
__device__ __forceinline__ V cx_conj(V a) {
  using R = typename RealOf<V>::R;
  return cx(R(a.x), -R(a.y));
}
// l * s + b, rounded as the reference's GPU step (lru_scan_cuda.cu:60-65):
// fma(l.re, s.re, -l.im * s.im) + b.re and fma(l.re, s.im, l.im * s.re) + b.im.
template <class V>
__device__ __forceinline__ V cx_step(V l, V s, V b) {
  using R = typename RealOf<V>::R;
  const R lr = l.x, li = l.y, sr = s.x, si = s.y;
  return cx(fma(lr, sr, -(li * si)) + R(b.x), fma(lr, si, li * sr) + R(b.y));
}
// acc + g * conj(x)
template <class V>
__device__ __forceinline__ V cx_acc_conj(V acc, V g, V x) {
  using R = typename RealOf<V>::R;
  const R gr = g.x, gi = g.y, xr = x.x, xi = x.y;
  return cx(R(acc.x) + (gr * xr + gi * xi), R(acc.y) + (gi * xr - gr * xi));
}

// l^n for n >= 1 by binary powering in fp64, rounded once (once per lane).
template <class V>
__device__ __forceinline__ V cx_pow(V l, int n) {
  using R = typename RealOf<V>::R;
  double br = R(l.x), bi = R(l.y), rr = 1.0, ri = 0.0;
  while (n > 0) {
    if (n & 1) {
      const double t = rr * br - ri * bi;
      ri = rr * bi + ri * br;
      rr = t;
    }
    n >>= 1;
    if (n) {
      const double t = br * br - bi * bi;
      bi = 2.0 * br * bi;
      br = t;
    }
  }
  return cx(static_cast<R>(rr), static_cast<R>(ri));
}

// ---- tagged records ------------------------------------------------------------
// rec[((chunk * 2 + kind) * NW + k) * nc + ch], kind kRecAgg / kRecInc.
template <class V>
constexpr int kRecWords = CxOf<typename RealOf<V>::R>::kWords;

template <class V>
__device__ __forceinline__ size_t drec_index(int chunk, int kind, int k, int nc, int ch) {
  return ((size_t(chunk) * 2 + kind) * kRecWords<V> + k) * size_t(nc) + ch;
}

__device__ __forceinline__ void to_words(float2 v, uint32_t (&w)[2]) {
  w[0] = __float_as_uint(static_cast<float>(v.x));
  w[1] = __float_as_uint(static_cast<float>(v.y));
}
__device__ __forceinline__ void to_words(double2 v, uint32_t (&w)[4]) {
  const unsigned long long a = __builtin_bit_cast(unsigned long long, static_cast<double>(v.x));
  const unsigned long long b = __builtin_bit_cast(unsigned long long, static_cast<double>(v.y));
  w[0] = static_cast<uint32_t>(a);
  w[1] = static_cast<uint32_t>(a >> 32);
  w[2] = static_cast<uint32_t>(b);
  w[3] = static_cast<uint32_t>(b >> 32);
}
__device__ __forceinline__ float2 from_words(const uint32_t (&w)[2]) {
  return make_float2(__uint_as_float(w[0]), __uint_as_float(w[1]));
}
__device__ __forceinline__ double2 from_words(const uint32_t (&w)[4]) {
  const unsigned long long a = (static_cast<unsigned long long>(w[1]) << 32) | w[0];
  const unsigned long long b = (static_cast<unsigned long long>(w[3]) << 32) | w[2];
  return make_double2(__builtin_bit_cast(double, a), __builtin_bit_cast(double, b));
}

template <class V>
__device__ __forceinline__ void drec_publish(unsigned long long* rec, int chunk, int kind, int nc,
                                             int ch, V v, unsigned int tag) {
  constexpr int NW = kRecWords<V>;
  uint32_t w[NW];
  to_words(v, w);
  const unsigned long long t = static_cast<unsigned long long>(tag) << 32;
#pragma unroll
  for (int k = 0; k < NW; ++k)
    __hip_atomic_store(rec + drec_index<V>(chunk, kind, k, nc, ch), t | w[k], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

template <class V>
__device__ __forceinline__ void drec_fetch(const unsigned long long* rec, int chunk, int kind,
                                           int nc, int ch, unsigned long long (&w)[kRecWords<V>]) {
#pragma unroll
  for (int k = 0; k < kRecWords<V>; ++k)
    w[k] = __hip_atomic_load(rec + drec_index<V>(chunk, kind, k, nc, ch), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

template <class V>
__device__ __forceinline__ bool drec_decode(const unsigned long long (&w)[kRecWords<V>],
                                            unsigned int tag, V* v) {
  constexpr int NW = kRecWords<V>;
  bool ok = true;
  uint32_t p[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    ok = ok && (static_cast<unsigned int>(w[k] >> 32) == tag);
    p[k] = static_cast<uint32_t>(w[k]);
  }
  *v = from_words(p);
  return ok;
}

// Carry into chunk c for one channel, walking predecessors c - dir, c - 2 dir,
// ... and composing their aggregates with lam_c (the chunk transition) until
// an inclusive prefix is found.  Every predecessor drew an earlier ticket, so
// it is resident and publishes its aggregate without waiting: the walk ends.
// The spin is still bounded; giving up raises kErrSpinTimeout and returns a
// NaN carry, as does a poisoned launch.
template <class V>
__device__ V diag_lookback(unsigned long long* rec, int c, int dir, int n_chunks, int nc, int ch,
                           V lam_c, const LaunchSync& sync) {
  using R = typename RealOf<V>::R;
  const V nan_carry = cx(R(__builtin_nan("")), R(__builtin_nan("")));
  if (sync.poison) return nan_carry;
  V acc = cx_zero<V>();
  V pw = cx_one<V>();
  int j = c - dir;
  uint32_t spins = 0;
  while (j >= 0 && j < n_chunks) {
    unsigned long long wi[kRecWords<V>], wa[kRecWords<V>];
    drec_fetch<V>(rec, j, kRecInc, nc, ch, wi);
    drec_fetch<V>(rec, j, kRecAgg, nc, ch, wa);
    V v;
    if (drec_decode<V>(wi, sync.tag, &v)) return cx_add(acc, cx_mul(pw, v));
    if (drec_decode<V>(wa, sync.tag, &v)) {
      acc = cx_add(acc, cx_mul(pw, v));
      pw = cx_mul(pw, lam_c);
      j -= dir;
      continue;
    }
    if (++spins > kSpinLimit) {
      __hip_atomic_fetch_or(sync.err, kErrSpinTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return nan_carry;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return acc;
}

// The channel's eigenvalue (lanes past the last channel read the last one).
template <class R>
__device__ __forceinline__ Cx<R> lane_lambda(const R* lam_re, const R* lam_im, int g, unsigned lc,
                                             int P) {
  const unsigned p = (static_cast<unsigned>(g) * kWave + lc) % static_cast<unsigned>(P);
  return cx(lam_re[p], lam_im[p]);
}

// ============================================================================
// Forward
// ============================================================================
template <class R, int T, int W>
__global__ __launch_bounds__(W * kWave) void diag_forward_kernel(
    const R* __restrict__ lam_re, const R* __restrict__ lam_im, int P,
    const Cx<R>* __restrict__ in, Cx<R>* __restrict__ out, int L, int nc, int n_groups,
    int n_chunks, unsigned long long* __restrict__ rec, LaunchSync sync) {
  using V = Cx<R>;
  __shared__ V s_agg[W][kWave];
  __shared__ V s_carry[kWave];
  __shared__ int s_ticket;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int ticket = launch_order(sync, n_groups * n_chunks, &s_ticket);
  const int c = ticket / n_groups;
  const int g = ticket - c * n_groups;
  const int ch = g * kWave + lane;
  const bool active = ch < nc;
  const unsigned lc = clamped_lane(g, nc);
  const V lam = lane_lambda(lam_re, lam_im, g, lc, P);
  const long long t0 = static_cast<long long>(c) * (T * W) + static_cast<long long>(w) * T;

  // clamped in-range loads (steps past L and inactive lanes are never stored)
  V x[T];
#pragma unroll
  for (int i = 0; i < T; ++i) x[i] = group_row(in, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[lc];

  // 1. sub-chunk aggregate from a zero state
  const bool full = t0 + T <= L;
  V e = cx_zero<V>();
  if (full) {
#pragma unroll
    for (int i = 0; i < T; ++i) e = cx_step(lam, e, x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < T; ++i)
      if (t0 + i < L) e = cx_step(lam, e, x[i]);
  }
  s_agg[w][lane] = e;
  const V lam_t = cx_pow(lam, T);
  __syncthreads();

  // 2. chunk aggregate (published by wave 1), look-back by wave 0: a wave's
  // loads complete in issue order behind its own stores
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    V E = cx_zero<V>();
#pragma unroll
    for (int v = 0; v < W; ++v) E = cx_step(lam_t, E, s_agg[v][lane]);
    const bool scan = active && n_chunks > 1;
    if (w == kPub && scan && c > 0) drec_publish(rec, c, kRecAgg, nc, ch, E, sync.tag);
    if (w == 0) {
      V carry = cx_zero<V>();
      if (scan) {
        if (c == 0) {
          drec_publish(rec, c, kRecInc, nc, ch, E, sync.tag);
        } else {
          const V lam_c = cx_pow(lam, T * W);
          carry = diag_lookback(rec, c, +1, n_chunks, nc, ch, lam_c, sync);
          if (c + 1 < n_chunks) drec_publish(rec, c, kRecInc, nc, ch, cx_step(lam_c, carry, E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }
  __syncthreads();

  // 3. own carry, re-run, store
  V s = s_carry[lane];
  for (int v = 0; v < w; ++v) s = cx_step(lam_t, s, s_agg[v][lane]);
  if (active) {
    if (full) {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        s = cx_step(lam, s, x[i]);
        stream_store(&group_row(out, t0 + i, nc, g)[lane], s);
      }
    } else {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        if (t0 + i < L) {
          s = cx_step(lam, s, x[i]);
          stream_store(&group_row(out, t0 + i, nc, g)[lane], s);
        }
      }
    }
  }
}

// ============================================================================
// Backward
// ============================================================================
// One workgroup per (chunk, channel group), chunks handed out last-first.
// grad_lambda: [P] complex as (re, im); each (chunk, channel) adds its sum of
// g_t conj(x_{t-1}) into it.
template <class R, int T, int W>
__global__ __launch_bounds__(W * kWave) void diag_backward_kernel(
    const R* __restrict__ lam_re, const R* __restrict__ lam_im, int P, const Cx<R>* states,
    const Cx<R>* __restrict__ gout, Cx<R>* __restrict__ gin, R* __restrict__ grad_lambda,
    ZeroFill zero, int L, int nc, int n_groups, int n_chunks, unsigned long long* __restrict__ rec,
    LaunchSync sync) {
  using V = Cx<R>;
  __shared__ V s_agg[W][kWave];
  __shared__ V s_carry[kWave];
  __shared__ V s_sum[W][kWave];
  __shared__ int s_ticket;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int ticket = launch_order(sync, n_groups * n_chunks, &s_ticket);
  if (ticket == 0) zero_fill_publish(zero, sync);  // grad_lambda
  const int cr = ticket / n_groups;
  const int g = ticket - cr * n_groups;
  const int c = n_chunks - 1 - cr;
  const int ch = g * kWave + lane;
  const bool active = ch < nc;
  const unsigned lc = clamped_lane(g, nc);
  const V lamc = cx_conj(lane_lambda(lam_re, lam_im, g, lc, P));
  const long long t0 = static_cast<long long>(c) * (T * W) + static_cast<long long>(w) * T;

  // Issue order = order of use: the saved states x_{t-1} first, then the
  // upstream gradient last step first, as the reverse sweeps consume it.
  V sp[T], go[T];
#pragma unroll
  for (int i = 0; i < T; ++i)
    sp[i] = group_row(states, max(min(t0 + i - 1, static_cast<long long>(L - 1)), 0ll), nc, g)[lc];
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = T - 1; i >= 0; --i)
    go[i] = group_row(gout, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[lc];
  if (t0 == 0) sp[0] = cx_zero<V>();  // x_{-1} = 0

  // 1. reverse aggregate from a zero carry: m = conj(lambda) g_{t0}
  const bool full = t0 + T <= L;
  V m = cx_zero<V>();
  if (full) {
#pragma unroll
    for (int i = T - 1; i >= 0; --i) m = cx_mul(lamc, cx_add(m, go[i]));
  } else {
#pragma unroll
    for (int i = T - 1; i >= 0; --i)
      if (t0 + i < L) m = cx_mul(lamc, cx_add(m, go[i]));
  }
  s_agg[w][lane] = m;
  const V lam_t = cx_pow(lamc, T);
  __syncthreads();

  // 2. chunk aggregate over waves W-1 .. 0, look-back over later chunks
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    V E = cx_zero<V>();
#pragma unroll
    for (int v = W - 1; v >= 0; --v) E = cx_step(lam_t, E, s_agg[v][lane]);
    const bool scan = active && n_chunks > 1;
    if (w == kPub && scan && c < n_chunks - 1) drec_publish(rec, c, kRecAgg, nc, ch, E, sync.tag);
    if (w == 0) {
      V carry = cx_zero<V>();
      if (scan) {
        if (c == n_chunks - 1) {
          drec_publish(rec, c, kRecInc, nc, ch, E, sync.tag);
        } else {
          const V lam_c = cx_pow(lamc, T * W);
          carry = diag_lookback(rec, c, -1, n_chunks, nc, ch, lam_c, sync);
          if (c > 0) drec_publish(rec, c, kRecInc, nc, ch, cx_step(lam_c, carry, E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }
  __syncthreads();

  // 3. the wave's carry through the later waves, then the final reverse pass
  V y = s_carry[lane];
  for (int v = W - 1; v > w; --v) y = cx_step(lam_t, y, s_agg[v][lane]);
  V acc = cx_zero<V>();
  if (active) {
    if (full) {
#pragma unroll
      for (int i = T - 1; i >= 0; --i) {
        const V gt = cx_add(go[i], y);
        stream_store(&group_row(gin, t0 + i, nc, g)[lane], gt);
        acc = cx_acc_conj(acc, gt, sp[i]);
        y = cx_mul(lamc, gt);
      }
    } else {
#pragma unroll
      for (int i = T - 1; i >= 0; --i) {
        if (t0 + i < L) {
          const V gt = cx_add(go[i], y);
          stream_store(&group_row(gin, t0 + i, nc, g)[lane], gt);
          acc = cx_acc_conj(acc, gt, sp[i]);
          y = cx_mul(lamc, gt);
        }
      }
    }
  }
  s_sum[w][lane] = acc;
  __syncthreads();
  // the chunk's share of grad_lambda[p], summed over the waves in a fixed
  // order; NaN if the zeroed outputs were never seen (a bounded wait that gave
  // up, kErrSpinTimeout raised)
  if (w == 0 && active) {
    V v = s_sum[0][lane];
#pragma unroll
    for (int u = 1; u < W; ++u) v = cx_add(v, s_sum[u][lane]);
    if (!wait_outputs_zeroed(sync)) v = cx(R(__builtin_nan("")), R(__builtin_nan("")));
    const int p = ch % P;
    atomic_put(grad_lambda + 2 * p, static_cast<double>(v.x));
    atomic_put(grad_lambda + 2 * p + 1, static_cast<double>(v.y));
  }
}

// ============================================================================
// Host side
// ============================================================================
struct DiagTile {
  int T, W;
};

// "TxW" from the environment, else the default.
DiagTile diag_tile(const char* env, DiagTile dflt) {
  const char* s = std::getenv(env);
  if (!s) return dflt;
  int t = 0, w = 0;
  if (std::sscanf(s, "%dx%d", &t, &w) != 2) return dflt;
  return {t, w};
}

// Instantiated (T, W) tiles per precision.
#define OSSM_DIAG_TILES_F32(X) X(16, 8) X(32, 4) X(16, 4) X(8, 8) X(32, 8) X(16, 16) X(8, 16) X(32, 16)
#define OSSM_DIAG_TILES_F64(X) X(8, 8) X(16, 4) X(16, 8) X(8, 4)

template <class R>
struct DiagDefaults;
template <>
struct DiagDefaults<float> {
  // forward 32 x 16 measured best at config 2's shape after the non-temporal stores
  // (40.4 vs 44.0 us for 16 x 16).  Backward (parameter gradient added in the
  // kernel, so every chunk is one float-atomic share of each output): 16 x 16
  // (256-step chunks, half the shares) for 128 to 2048 workgroups of that tile,
  // else 16 x 8 (bwd_tile).  Measured (events, us; 16 x 8 / 16 x 16) at
  // [L, B, P]: [1024, 8, 64] 10.4 / 11.8 (32 workgroups); [4096, 8, 128]
  // 29.6 / 20.9; [1024, 32, 128] 28.1 / 20.6; [4096, 32, 128] 76.2 / 70.7;
  // [16384, 8, 512] 270 / 275 (4096 workgroups); [65536, 4, 256] 287 / 288.
  static constexpr DiagTile kFwd{32, 16}, kBwd{16, 8}, kBwdWide{16, 16};
  static constexpr const char* kEnvFwd = "OSSM_DIAG_TILE_FWD";
  static constexpr const char* kEnvBwd = "OSSM_DIAG_TILE_BWD";
};
template <>
struct DiagDefaults<double> {
  // backward 16 x 8 at every measured shape ([1024, 8, 64] 11.5 us, [4096, 8, 128] 37.3,
  // [1024, 32, 128] 34.2, [4096, 32, 128] 140.0; 8 x 8: 12.4, 45.2, 44.3, 147.4)
  static constexpr DiagTile kFwd{8, 8}, kBwd{16, 8}, kBwdWide{16, 8};
  static constexpr const char* kEnvFwd = "OSSM_DIAG_TILE_FWD_F64";
  static constexpr const char* kEnvBwd = "OSSM_DIAG_TILE_BWD_F64";
};

// The backward's tile: the environment's, else kBwdWide when that tile gives
// 128 to 2048 workgroups, else kBwd.
template <class R>
DiagTile bwd_tile(int64_t L, int64_t nc) {
  static const DiagTile env = diag_tile(DiagDefaults<R>::kEnvBwd, DiagTile{0, 0});
  if (env.T > 0) return env;
  constexpr DiagTile wide = DiagDefaults<R>::kBwdWide;
  const int64_t span = int64_t(wide.T) * wide.W;
  const int64_t n_wg = (L + span - 1) / span * ((nc + kWave - 1) / kWave);
  return n_wg >= 128 && n_wg <= 2048 ? wide : DiagDefaults<R>::kBwd;
}

int check_diag_sizes(int64_t L, int64_t B, int64_t P, const char* what) {
  if (L < 0 || B < 0 || P < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (L > INT_MAX || B * P > INT_MAX / 2 || P > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  return OSSM_OK;
}

template <class R>
int diag_forward_impl(const R* lam_re, const R* lam_im, const void* b_seq, void* out, int64_t L,
                      int64_t B, int64_t P, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  static const DiagTile tile = diag_tile(DiagDefaults<R>::kEnvFwd, DiagDefaults<R>::kFwd);
  const int64_t nc = B * P;
  const int64_t CL = int64_t(tile.T) * tile.W;
  const int64_t n_chunks = (L + CL - 1) / CL;
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  const int64_t total = n_chunks * n_groups;
  if (total > INT_MAX) return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  const size_t rec_bytes = static_cast<size_t>(n_chunks) * 2 * CxOf<R>::kWords * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  if (int rc = acquire_scratch(call, rec_bytes, total, &payload, &sync)) return rc;
  bool launched = false;
#define OSSM_LAUNCH_DIAG_FWD(TT, WW)                                                              \
  if (!launched && tile.T == TT && tile.W == WW) {                                                \
    hipLaunchKernelGGL((diag_forward_kernel<R, TT, WW>), dim3(static_cast<unsigned>(total)),      \
                       dim3(WW * kWave), 0, stream, lam_re, lam_im, static_cast<int>(P),          \
                       static_cast<const Cx<R>*>(b_seq), static_cast<Cx<R>*>(out),                \
                       static_cast<int>(L), static_cast<int>(nc), static_cast<int>(n_groups),     \
                       static_cast<int>(n_chunks), static_cast<unsigned long long*>(payload), sync); \
    launched = true;                                                                              \
  }
  if constexpr (std::is_same_v<R, float>) {
    OSSM_DIAG_TILES_F32(OSSM_LAUNCH_DIAG_FWD)
  } else {
    OSSM_DIAG_TILES_F64(OSSM_LAUNCH_DIAG_FWD)
  }
#undef OSSM_LAUNCH_DIAG_FWD
  if (!launched) return set_error(OSSM_ERR_UNSUPPORTED, std::string(DiagDefaults<R>::kEnvFwd) + " names no built tile");
  if (int rc = launch_check("diag_forward_kernel")) return rc;
  return OSSM_OK;
}

template <class R>
int diag_backward_impl(const R* lam_re, const R* lam_im, const void* states, const void* gout,
                       R* grad_lambda, void* grad_b, int64_t L, int64_t B, int64_t P,
                       hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const int64_t nc = B * P;
  const DiagTile tile = bwd_tile<R>(L, nc);
  const int64_t CL = int64_t(tile.T) * tile.W;
  const int64_t n_chunks = (L + CL - 1) / CL;
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  const int64_t total = n_chunks * n_groups;
  if (total > INT_MAX) return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  const size_t rec_bytes = static_cast<size_t>(n_chunks) * 2 * CxOf<R>::kWords * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  if (int rc = acquire_scratch(call, rec_bytes, total, &payload, &sync)) return rc;
  const ZeroFill zero{{reinterpret_cast<float*>(grad_lambda), nullptr, nullptr},
                      {static_cast<int>(2 * P * (sizeof(R) / sizeof(float))), 0, 0}};
  bool launched = false;
#define OSSM_LAUNCH_DIAG_BWD(TT, WW)                                                              \
  if (!launched && tile.T == TT && tile.W == WW) {                                                \
    hipLaunchKernelGGL((diag_backward_kernel<R, TT, WW>), dim3(static_cast<unsigned>(total)),     \
                       dim3(WW * kWave), 0, stream, lam_re, lam_im, static_cast<int>(P),          \
                       static_cast<const Cx<R>*>(states), static_cast<const Cx<R>*>(gout),        \
                       static_cast<Cx<R>*>(grad_b), grad_lambda, zero, static_cast<int>(L),       \
                       static_cast<int>(nc), static_cast<int>(n_groups),                          \
                       static_cast<int>(n_chunks), static_cast<unsigned long long*>(payload), sync); \
    launched = true;                                                                              \
  }
  if constexpr (std::is_same_v<R, float>) {
    OSSM_DIAG_TILES_F32(OSSM_LAUNCH_DIAG_BWD)
  } else {
    OSSM_DIAG_TILES_F64(OSSM_LAUNCH_DIAG_BWD)
  }
#undef OSSM_LAUNCH_DIAG_BWD
  if (!launched) return set_error(OSSM_ERR_UNSUPPORTED, std::string(DiagDefaults<R>::kEnvBwd) + " names no built tile");
  return launch_check("diag_backward_kernel");
}

template <class R>
int diag_forward_entry(const R* lam_re, const R* lam_im, const void* b_seq, void* out, int64_t L,
                       int64_t B, int64_t P, ossm_stream_t stream, const char* what) {
  clear_error();
  if (int rc = check_diag_sizes(L, B, P, what)) return rc;
  if (L == 0 || B == 0 || P == 0) return OSSM_OK;
  if (!lam_re || !lam_im || !b_seq || !out)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  return diag_forward_impl<R>(lam_re, lam_im, b_seq, out, L, B, P, static_cast<hipStream_t>(stream));
}

template <class R>
int diag_backward_entry(const R* lam_re, const R* lam_im, const void* states, const void* gout,
                        void* grad_lambda, void* grad_b, int64_t L, int64_t B, int64_t P,
                        ossm_stream_t stream_v, const char* what) {
  clear_error();
  if (int rc = check_diag_sizes(L, B, P, what)) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  if (P > 0 && (L == 0 || B == 0)) {
    // nothing to scan: grad_lambda is zero (lru.py:57-58)
    if (!grad_lambda) return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
    return fill_zero(static_cast<float*>(grad_lambda), 2 * P * int64_t(sizeof(R) / sizeof(float)), stream);
  }
  if (L == 0 || B == 0 || P == 0) return OSSM_OK;
  if (!lam_re || !lam_im || !states || !gout || !grad_lambda || !grad_b)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  return diag_backward_impl<R>(lam_re, lam_im, states, gout, static_cast<R*>(grad_lambda), grad_b,
                               L, B, P, stream);
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_diag_scan_forward(const float* lambda_real, const float* lambda_imag, const void* b_seq,
                           void* out, int64_t length, int64_t batch, int64_t state,
                           ossm_stream_t stream) {
  return diag_forward_entry<float>(lambda_real, lambda_imag, b_seq, out, length, batch, state,
                                   stream, "diag_scan_forward");
}

int ossm_diag_scan_backward(const float* lambda_real, const float* lambda_imag, const void* states,
                            const void* grad_output, void* grad_lambda, void* grad_b,
                            int64_t length, int64_t batch, int64_t state, ossm_stream_t stream) {
  return diag_backward_entry<float>(lambda_real, lambda_imag, states, grad_output, grad_lambda,
                                    grad_b, length, batch, state, stream, "diag_scan_backward");
}

int ossm_diag_scan_forward_f64(const double* lambda_real, const double* lambda_imag,
                               const void* b_seq, void* out, int64_t length, int64_t batch,
                               int64_t state, ossm_stream_t stream) {
  return diag_forward_entry<double>(lambda_real, lambda_imag, b_seq, out, length, batch, state,
                                    stream, "diag_scan_forward_f64");
}

int ossm_diag_scan_backward_f64(const double* lambda_real, const double* lambda_imag,
                                const void* states, const void* grad_output, void* grad_lambda,
                                void* grad_b, int64_t length, int64_t batch, int64_t state,
                                ossm_stream_t stream) {
  return diag_backward_entry<double>(lambda_real, lambda_imag, states, grad_output, grad_lambda,
                                     grad_b, length, batch, state, stream, "diag_scan_backward_f64");
}

}  // extern "C"
