// Selective D-LinOSS scans on gfx950: the D-LinOSS recurrence with
// per-step (time- and batch-varying) parameters, forward and backward, for
// the four discretisations imex1, imex2, im and ex.
//
// Recurrence (sdlinoss_<v>.cpp forward kernels; the bridge's fallback
// restates it in _sdlinoss_scan.py:150-197).  Per step, with
// dt = clamp(step, 1e-6, 1):
//   comb = -a x + bu,  tmpw = alpha w + dt^2 comb,  w' = tmpw / S,  x' = x + w'
//   imex1: alpha = 1,         S = max(1 + dt g, 1e-6)
//   imex2: alpha = 1 - dt g,  S = max(1 + dt^2 a, 1e-6)
//   im:    alpha = 1,         S = max(1 + dt g + dt^2 a, 1e-6)
//   ex:    alpha = 1 - dt g,  S = 1
// i.e. (w, x) -> M_t (w, x) + f_t bu with the real 2x2
//   M_t = [[c0, c1], [c0, 1 + c1]],  f_t = (c2, c2),
//   c0 = alpha / S,  c1 = -dt^2 a / S,  c2 = dt^2 / S.
//
// Parameters a, g, step are [La, Ba, M] with La in {1, L} and Ba in {1, B}
// (broadcast over time and/or batch, as normalize_param_view_cpu allows,
// sdlinoss_cpu_utils.h:11-72).  bu is [L, B, M] complex64 and the states
// [L, B, M, 2] complex64 (component 0 = w, 1 = x), channel ch = b M + m
// contiguous: one wave = 64 consecutive channels.
//
// Both directions are the chunked scan of the oscillator kernels with the
// chunk transition no longer a matrix power: each lane composes its
// sub-chunk's matrices while it scans, workgroups combine (matrix, vector)
// aggregates through LDS, and the look-back records carry both.
//
// Backward: the adjoint lambda_t = (0, g_t) + M_{t+1}^T lambda_{t+1} in
// reverse time; the states s_{t-1} are rebuilt from states[t0 - 1] at each
// sub-chunk start into LDS; the per-step gradients of a, g and step follow
// the reference's chain rule (sdlinoss_<v>.cpp backward kernels) and are
// written per element; parameters broadcast over time or batch are then
// summed over those axes by a two-pass column reduction in a fixed order.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_device.hpp"
#include "sdl_model.hpp"

namespace ossm {
namespace {

// M_t * P for a 2x2 P (rows of M_t: (c0, c1), (c0, 1 + c1))
template <int V>
__device__ __forceinline__ RMat sdl_mat_left(const SdlCoef<V>& k, RMat p) {
  const float a = fmaf(k.c0, p.a, k.c1 * p.c);
  const float b = fmaf(k.c0, p.b, k.c1 * p.d);
  return {a, b, a + p.c, b + p.d};
}

// M_t^T * P (rows of M_t^T: (c0, c0), (c1, 1 + c1))
template <int V>
__device__ __forceinline__ RMat sdl_matT_left(const SdlCoef<V>& k, RMat p) {
  const float sa = p.a + p.c, sb = p.b + p.d;
  return {k.c0 * sa, k.c0 * sb, fmaf(k.c1, sa, p.c), fmaf(k.c1, sb, p.d)};
}

// M_t^T applied to an adjoint (lw, lx): (c0 (lw + lx), lx + c1 (lw + lx))
template <int V>
__device__ __forceinline__ float4 sdl_matT_apply(const SdlCoef<V>& k, float4 l) {
  const float sr = l.x + l.z, si = l.y + l.w;
  return make_float4(k.c0 * sr, k.c0 * si, fmaf(k.c1, sr, l.z), fmaf(k.c1, si, l.w));
}

__device__ __forceinline__ float4 rmat_pack(RMat m) { return make_float4(m.a, m.b, m.c, m.d); }
__device__ __forceinline__ RMat rmat_unpack(float4 v) { return {v.x, v.y, v.z, v.w}; }

// ---- look-back with per-chunk matrices ---------------------------------------
// Records per (chunk, channel): kind 0 = aggregate vector, 1 = inclusive
// prefix, 2 = aggregate matrix; four tagged 64-bit words each (the protocol
// of scan_device.hpp: a word written once per launch, valid when it carries
// this launch's tag).
constexpr int kTvKinds = 3;
constexpr int kTvAgg = 0, kTvInc = 1, kTvMat = 2;

__device__ __forceinline__ size_t tv_index(int chunk, int kind, int k, int nc, int ch) {
  return ((size_t(chunk) * kTvKinds + kind) * 4 + k) * size_t(nc) + ch;
}

__device__ __forceinline__ void tv_publish(unsigned long long* rec, int chunk, int kind, int nc,
                                           int ch, float4 v, unsigned int tag) {
  const unsigned long long t = static_cast<unsigned long long>(tag) << 32;
  const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k)
    __hip_atomic_store(rec + tv_index(chunk, kind, k, nc, ch), t | __float_as_uint(vals[k]),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void tv_fetch(const unsigned long long* rec, int chunk, int kind, int nc,
                                         int ch, unsigned long long (&w)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = __hip_atomic_load(rec + tv_index(chunk, kind, k, nc, ch), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Carry into chunk c for one channel, walking predecessors c - dir, ...:
// acc + P * (inclusive of j), where each aggregate (E_j, K_j) passed over
// adds P E_j to acc and turns P into P K_j.  Bounded spin and NaN carry as in
// lookback().
__device__ float4 lookback_tv(unsigned long long* rec, int c, int dir, int n_chunks, int nc,
                              int ch, const LaunchSync& sync) {
  if (sync.poison) return f4nan();
  float4 acc = f4zero();
  RMat P = {1.f, 0.f, 0.f, 1.f};
  int j = c - dir;
  uint32_t spins = 0;
  while (j >= 0 && j < n_chunks) {
    unsigned long long wi[4], wa[4], wm[4];
    tv_fetch(rec, j, kTvInc, nc, ch, wi);
    tv_fetch(rec, j, kTvAgg, nc, ch, wa);
    tv_fetch(rec, j, kTvMat, nc, ch, wm);
    float4 v, e, km;
    if (rec_decode(wi, sync.tag, &v)) return f4add(acc, mat_apply(P, v));
    const bool ea = rec_decode(wa, sync.tag, &e);
    const bool em = rec_decode(wm, sync.tag, &km);
    if (ea && em) {
      acc = f4add(acc, mat_apply(P, e));
      P = mat_mul(P, rmat_unpack(km));
      j -= dir;
      continue;
    }
    if (++spins > kSpinLimit) {
      __hip_atomic_fetch_or(sync.err, kErrSpinTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return f4nan();
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return acc;
}

// ---- addressing ---------------------------------------------------------------
template <class E>
__device__ __forceinline__ E* row_of(E* base, long long t, int nc, int g) {
  return base + static_cast<size_t>(t) * nc + static_cast<size_t>(g) * kWave;
}

// Per-lane indices of one workgroup's channel group: lanes past the last
// channel are clamped onto it (their loads stay in bounds; nothing of theirs
// is stored).
struct LaneIdx {
  unsigned lc;  // lane offset within the group, clamped
  int pch;      // index of the lane's channel within a parameter row of B*M
  int pm;       // index of the lane's oscillator m within a parameter row of M
};

__device__ __forceinline__ LaneIdx lane_idx(int g, int nc, int M) {
  LaneIdx r;
  r.lc = static_cast<unsigned>(min(static_cast<int>(threadIdx.x & (kWave - 1)), nc - 1 - g * kWave));
  r.pch = g * kWave + static_cast<int>(r.lc);
  r.pm = r.pch % M;
  return r;
}

__device__ __forceinline__ float param_at(const ParamView& v, long long t, const LaneIdx& li) {
  return v.p[static_cast<size_t>(t * v.t_stride) + (v.by_channel ? li.pch : li.pm)];
}

// The parameters of steps t0 .. t0 + T - 1 (clamped rows); TB: broadcast over
// time, one read each.
template <int T, bool TB>
__device__ __forceinline__ void load_params(const SdlParams& prm, long long t0, int L,
                                            const LaneIdx& li, float (&pa)[T], float (&pg)[T],
                                            float (&ps)[T]) {
  if constexpr (TB) {
    const float a = param_at(prm.a, 0, li), g = param_at(prm.g, 0, li), s = param_at(prm.s, 0, li);
#pragma unroll
    for (int i = 0; i < T; ++i) {
      pa[i] = a;
      pg[i] = g;
      ps[i] = s;
    }
  } else {
#pragma unroll
    for (int i = 0; i < T; ++i) {
      const long long t = min(t0 + i, static_cast<long long>(L - 1));
      pa[i] = param_at(prm.a, t, li);
      pg[i] = param_at(prm.g, t, li);
      ps[i] = param_at(prm.s, t, li);
    }
  }
}

// ============================================================================
// Forward
// ============================================================================
// One workgroup = one time chunk of W*T steps for 64 channels; wave w owns
// steps [t0, t0 + T).  Workgroups take chunks first-first in ticket order.
// TB: all three parameters broadcast over time (time stride 0): they are
// read once and every per-step coefficient is the same value, which the
// compiler then computes once.
// PERSIST: as the oscillatory forward's persistent launch (ticket order, a
// grid of fewer workgroups than chunks, workgroup b taking ceil((total - b) /
// grid) chunks and drawing the next ticket while it stores the current one).
template <int V, int T, int W, bool TB, bool PERSIST>
__global__ __launch_bounds__(W * kWave) void sdl_forward_kernel(
    SdlParams prm, const float2* __restrict__ bu, float4* __restrict__ out, int L, int nc,
    int n_groups, int n_chunks, unsigned long long* __restrict__ rec, LaunchSync sync) {
  __shared__ float4 s_e[W][kWave];
  __shared__ float4 s_m[W][kWave];
  __shared__ float4 s_carry[kWave];
  __shared__ int s_ticket;
  __shared__ unsigned int s_tag;
  __shared__ int s_poison;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int total = n_groups * n_chunks;
  int order;
  int left = 1;
  if constexpr (PERSIST) {
    left = (total - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) /
           static_cast<int>(gridDim.x);
    if (threadIdx.x == 0) {
      unsigned int tag = 0;
      int poison = 0;
      s_ticket = draw_ticket(sync, total, &tag, &poison);
      s_tag = tag;
      s_poison = poison;
    }
    __syncthreads();
    sync.tag = __builtin_amdgcn_readfirstlane(s_tag);
    sync.poison = __builtin_amdgcn_readfirstlane(s_poison);
    order = __builtin_amdgcn_readfirstlane(s_ticket);
  } else {
    order = launch_order(sync, total, &s_ticket);
  }
  for (;;) {
  const int ticket = order;
  const int c = ticket / n_groups;
  const int g = ticket - c * n_groups;
  const int ch = g * kWave + lane;
  const bool active = ch < nc;
  const long long t0 = static_cast<long long>(c) * (T * W) + static_cast<long long>(w) * T;
  const LaneIdx li = lane_idx(g, nc, prm.M);

  // loads (clamped rows): parameters, then bu
  float pa[T], pg[T], ps[T];
  float2 x[T];
  load_params<T, TB>(prm, t0, L, li, pa, pg, ps);
#pragma unroll
  for (int i = 0; i < T; ++i) x[i] = row_of(bu, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[li.lc];

  // 1. sub-chunk aggregate from a zero state, composing the matrices
  const bool full = t0 + T <= L;
  SdlCoef<V> k[T];
  float4 e = f4zero();
  RMat Mc = {1.f, 0.f, 0.f, 1.f};
#pragma unroll
  for (int i = 0; i < T; ++i) {
    k[i] = sdl_coef<V>(pa[i], pg[i], ps[i]);
    if (full || t0 + i < L) {
      e = sdl_step<V>(k[i], e, x[i]);
      Mc = sdl_mat_left<V>(k[i], Mc);
    }
  }
  s_e[w][lane] = e;
  s_m[w][lane] = rmat_pack(Mc);
  __syncthreads();

  // 2. chunk aggregate, look-back (wave 0), aggregate published by wave 1
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    float4 E = f4zero();
    RMat Mch = {1.f, 0.f, 0.f, 1.f};
#pragma unroll
    for (int v = 0; v < W; ++v) {
      const RMat Mv = rmat_unpack(s_m[v][lane]);
      E = f4add(mat_apply(Mv, E), s_e[v][lane]);
      Mch = mat_mul(Mv, Mch);
    }
    const bool scan = active && n_chunks > 1;
    if (w == kPub && scan && c > 0) {
      tv_publish(rec, c, kTvAgg, nc, ch, E, sync.tag);
      tv_publish(rec, c, kTvMat, nc, ch, rmat_pack(Mch), sync.tag);
    }
    if (w == 0) {
      float4 carry = f4zero();
      if (scan) {
        if (c == 0) {
          tv_publish(rec, c, kTvInc, nc, ch, E, sync.tag);
        } else {
          carry = lookback_tv(rec, c, +1, n_chunks, nc, ch, sync);
          if (c + 1 < n_chunks)
            tv_publish(rec, c, kTvInc, nc, ch, f4add(mat_apply(Mch, carry), E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }
  __syncthreads();

  // 3. own carry through the earlier waves, then re-run and store
  int next = 0, next_poison = 0;
  if constexpr (PERSIST) {
    if (threadIdx.x == 0 && left > 1) {
      unsigned int tag = 0;
      next = draw_ticket(sync, total, &tag, &next_poison);
    }
  }
  float4 s = s_carry[lane];
  for (int v = 0; v < w; ++v) s = f4add(mat_apply(rmat_unpack(s_m[v][lane]), s), s_e[v][lane]);
  if (active) {
    if (full) {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        s = sdl_step<V>(k[i], s, x[i]);
        stream_store(&row_of(out, t0 + i, nc, g)[lane], s);
      }
    } else {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        if (t0 + i < L) {
          s = sdl_step<V>(k[i], s, x[i]);
          stream_store(&row_of(out, t0 + i, nc, g)[lane], s);
        }
      }
    }
  }
  if constexpr (!PERSIST) break;
  if (--left == 0) break;
  // every wave is past its reads of s_e, s_m and s_carry before the next
  // chunk writes them
  if (threadIdx.x == 0) {
    s_ticket = next;
    s_poison = next_poison;
  }
  __syncthreads();
  sync.poison = __builtin_amdgcn_readfirstlane(s_poison);
  order = __builtin_amdgcn_readfirstlane(s_ticket);
  }
}

// ============================================================================
// Backward
// ============================================================================
// Per-step gradients, given the adjoint lam = (lw, lx) of the new state, the
// previous state sp = (w_prev, x_prev), bu and the raw parameters; returns
// the adjoint carried to the previous step (M_t^T lam).  The arithmetic
// follows the reference backward kernels: sdlinoss_imex1.cpp:186-220,
// sdlinoss_imex2.cpp:178-221, sdlinoss_im.cpp:176-225, sdlinoss_ex.cpp:163-189.
template <int V>
__device__ __forceinline__ float4 sdl_grad_step(float a, float g, float step_raw, float inv,
                                                float4 sp, float2 bu, float4 lam, float2& gbu,
                                                float& ga, float& gg, float& gs) {
  const float dt = sdl_dt(step_raw);
  const float dt2 = dt * dt;
  const float alpha = sdl_alpha<V>(dt, g);
  // gradient w.r.t. the new w, through both components (x' = x + w')
  const float gwr = lam.x + lam.z, gwi = lam.y + lam.w;
  const float combr = fmaf(-a, sp.z, bu.x), combi = fmaf(-a, sp.w, bu.y);
  float gdt = 0.f, gA = 0.f, gG = 0.f;
  float gtr = gwr, gti = gwi;  // gradient w.r.t. tmpw
  if constexpr (V != OSSM_DLINOSS_EX) {
    const float s_raw = sdl_s_raw<V>(dt, g, a);
    const float tmpr = fmaf(alpha, sp.x, dt2 * combr), tmpi = fmaf(alpha, sp.y, dt2 * combi);
    gtr = gwr * inv;
    gti = gwi * inv;
    const float gS = -(gwr * tmpr + gwi * tmpi) * (inv * inv) * (s_raw > kClampMin ? 1.f : 0.f);
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      gdt = gS * g;
      gG = gS * dt;
    } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
      gdt = gS * (2.f * dt * a);
      gA = gS * dt2;
    } else {
      gdt = gS * (g + 2.f * dt * a);
      gA = gS * dt2;
      gG = gS * dt;
    }
  }
  // tmpw = alpha w_prev + dt^2 (-a x_prev + bu)
  if constexpr (V == OSSM_DLINOSS_IMEX2 || V == OSSM_DLINOSS_EX) {
    gdt += gtr * (-g * sp.x + 2.f * dt * combr) + gti * (-g * sp.y + 2.f * dt * combi);
    gG += gtr * (-dt * sp.x) + gti * (-dt * sp.y);
  } else {
    gdt += gtr * (2.f * dt * combr) + gti * (2.f * dt * combi);
  }
  gA += gtr * (-dt2 * sp.z) + gti * (-dt2 * sp.w);
  gbu = make_float2(gtr * dt2, gti * dt2);
  ga = gA;
  gg = gG;
  gs = (step_raw > kDtMin && step_raw < kDtMax) ? gdt : 0.f;
  // carry to the previous step: d/dw_prev = alpha gt, d/dx_prev = lx - dt^2 a gt
  return make_float4(alpha * gtr, alpha * gti, fmaf(-dt2 * a, gtr, lam.z), fmaf(-dt2 * a, gti, lam.w));
}

// Destinations of the parameter gradients.  Bit p of `tsum` (p = 0 a, 1 g,
// 2 step) set: the parameter is broadcast over time, so each workgroup writes
// its chunk's sum over time (row c of a [n_chunks, B*M] partials array);
// clear: per-element gradients ([L, B*M]).
struct SdlGradOut {
  float* p[3];
  int tsum;
};

template <int V, int T, int W, bool TB>
__global__ __launch_bounds__(W * kWave) void sdl_backward_kernel(
    SdlParams prm, const float2* __restrict__ bu, const float4* states,
    const float2* __restrict__ gout, float2* __restrict__ gin, SdlGradOut go_prm, int L, int nc,
    int n_groups, int n_chunks, unsigned long long* __restrict__ rec, LaunchSync sync) {
  __shared__ float4 s_e[W][kWave];
  __shared__ float4 s_k[W][kWave];
  __shared__ float4 s_carry[kWave];
  __shared__ float4 s_sp[W][T][kWave];  // recomputed s_{t-1}
  __shared__ float s_psum[3][W][kWave];  // per-wave sums over time (broadcast parameters)
  __shared__ int s_ticket;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int ticket = launch_order(sync, n_groups * n_chunks, &s_ticket);
  // chunks are handed out last-first
  const int cr = ticket / n_groups;
  const int g = ticket - cr * n_groups;
  const int c = n_chunks - 1 - cr;
  const int ch = g * kWave + lane;
  const bool active = ch < nc;
  const long long t0 = static_cast<long long>(c) * (T * W) + static_cast<long long>(w) * T;
  const LaneIdx li = lane_idx(g, nc, prm.M);

  // loads in order of use: checkpoint, parameters and bu (forward
  // recompute), upstream gradient last step first (reverse sweep)
  const float4 ck = row_of(states, max(min(t0 - 1, static_cast<long long>(L - 1)), 0ll), nc, g)[li.lc];
  asm volatile("" ::: "memory");
  float pa[T], pg[T], ps[T];
  float2 x[T], go[T];
  load_params<T, TB>(prm, t0, L, li, pa, pg, ps);
#pragma unroll
  for (int i = 0; i < T; ++i) x[i] = row_of(bu, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[li.lc];
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = T - 1; i >= 0; --i) go[i] = row_of(gout, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[li.lc];

  const bool full = t0 + T <= L;
  auto live = [&](int i) { return full || t0 + i < L; };

  // recompute s_{t-1} into LDS (1/S of every step kept for the later
  // passes); reverse aggregate (e, K) of the sub-chunk
  float inv[T];
  {
    float4 s = t0 >= 1 ? ck : f4zero();
#pragma unroll
    for (int i = 0; i < T; ++i) {
      inv[i] = sdl_inv_of<V>(pa[i], pg[i], ps[i]);
      s_sp[w][i][lane] = s;
      if (live(i)) s = sdl_step<V>(sdl_coef_inv<V>(pa[i], pg[i], ps[i], inv[i]), s, x[i]);
    }
  }
  float4 e = f4zero();
  RMat K = {1.f, 0.f, 0.f, 1.f};
#pragma unroll
  for (int i = T - 1; i >= 0; --i) {
    if (live(i)) {
      const SdlCoef<V> k = sdl_coef_inv<V>(pa[i], pg[i], ps[i], inv[i]);
      e = sdl_matT_apply<V>(k, make_float4(e.x, e.y, e.z + go[i].x, e.w + go[i].y));
      K = sdl_matT_left<V>(k, K);
    }
  }
  s_e[w][lane] = e;
  s_k[w][lane] = rmat_pack(K);
  __syncthreads();

  // chunk aggregate over waves W-1 .. 0; look-back over later chunks
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    float4 E = f4zero();
    RMat Kch = {1.f, 0.f, 0.f, 1.f};
#pragma unroll
    for (int v = W - 1; v >= 0; --v) {
      const RMat Kv = rmat_unpack(s_k[v][lane]);
      E = f4add(mat_apply(Kv, E), s_e[v][lane]);
      Kch = mat_mul(Kv, Kch);
    }
    const bool scan = active && n_chunks > 1;
    if (w == kPub && scan && c < n_chunks - 1) {
      tv_publish(rec, c, kTvAgg, nc, ch, E, sync.tag);
      tv_publish(rec, c, kTvMat, nc, ch, rmat_pack(Kch), sync.tag);
    }
    if (w == 0) {
      float4 carry = f4zero();
      if (scan) {
        if (c == n_chunks - 1) {
          tv_publish(rec, c, kTvInc, nc, ch, E, sync.tag);
        } else {
          carry = lookback_tv(rec, c, -1, n_chunks, nc, ch, sync);
          if (c > 0) tv_publish(rec, c, kTvInc, nc, ch, f4add(mat_apply(Kch, carry), E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }
  __syncthreads();

  // the wave's carry: the chunk carry through the later waves' sub-chunks
  float4 rho = s_carry[lane];
  for (int v = W - 1; v > w; --v) rho = f4add(mat_apply(rmat_unpack(s_k[v][lane]), rho), s_e[v][lane]);

  // final reverse pass: per-step gradients (per element, or summed over the
  // sub-chunk for parameters broadcast over time)
  float psum[3] = {0.f, 0.f, 0.f};
  bool by_sums = false;
  if constexpr (TB) {
    // every parameter constant over time and every gradient summed over it:
    // the step keeps only the adjoint, grad_bu and the three contractions
    // (sdl_param_grads_of_sums), about a third of sdl_grad_step's work
    if (go_prm.tsum == 7) {
      by_sums = true;
      if (active) {
        const SdlCoef<V> k = sdl_coef_inv<V>(pa[0], pg[0], ps[0], inv[0]);
        float px = 0.f, pz = 0.f, pb = 0.f;
#pragma unroll
        for (int i = T - 1; i >= 0; --i) {
          if (live(i)) {
            const float lzr = rho.z + go[i].x, lzi = rho.w + go[i].y;
            const float gwr = rho.x + lzr, gwi = rho.y + lzi;
            const float4 sp = s_sp[w][i][lane];
            px = fmaf(gwr, sp.x, fmaf(gwi, sp.y, px));
            pz = fmaf(gwr, sp.z, fmaf(gwi, sp.w, pz));
            pb = fmaf(gwr, x[i].x, fmaf(gwi, x[i].y, pb));
            stream_store(&row_of(gin, t0 + i, nc, g)[lane], make_float2(k.c2 * gwr, k.c2 * gwi));
            rho = make_float4(k.c0 * gwr, k.c0 * gwi, fmaf(k.c1, gwr, lzr), fmaf(k.c1, gwi, lzi));
          }
        }
        sdl_param_grads_of_sums<V>(pa[0], pg[0], ps[0], inv[0], px, pz, pb, psum[0], psum[1], psum[2]);
      }
    }
  }
  if (!by_sums && active) {
#pragma unroll
    for (int i = T - 1; i >= 0; --i) {
      if (live(i)) {
        const long long t = t0 + i;
        const float4 lam = make_float4(rho.x, rho.y, rho.z + go[i].x, rho.w + go[i].y);
        float2 gbu;
        float gp[3];
        rho = sdl_grad_step<V>(pa[i], pg[i], ps[i], inv[i], s_sp[w][i][lane], x[i], lam, gbu,
                               gp[0], gp[1], gp[2]);
        stream_store(&row_of(gin, t, nc, g)[lane], gbu);
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          if (go_prm.tsum & (1 << p)) psum[p] += gp[p];
          else stream_store(&row_of(go_prm.p[p], t, nc, g)[lane], gp[p]);
        }
      }
    }
  }
  if (go_prm.tsum != 0) {
#pragma unroll
    for (int p = 0; p < 3; ++p) s_psum[p][w][lane] = psum[p];
    __syncthreads();
    if (w == 0 && active) {
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        if (!(go_prm.tsum & (1 << p))) continue;
        float v = 0.f;
        for (int u = 0; u < W; ++u) v += s_psum[p][u][lane];
        row_of(go_prm.p[p], c, nc, g)[lane] = v;
      }
    }
  }
}

// ============================================================================
// Sums over broadcast axes: out[n][c] = sum_r in[n][r][c], in fp64, fixed
// order.  Pass 1: block (64-column tile, row group q) sums rows
// r = q*4 + wave + k*4G; pass 2 adds the G row groups.  Short reductions
// (sdl_colsum_direct) take one launch instead.
// ============================================================================
constexpr int kSumGroups = 32;

// One reduction: out[n][c] = sum_r in[n][r][c] for n < nb, r < R, c < C.
struct ColSum {
  const float* in;
  float* out;
  double* part;  // [nb][kSumGroups][C]
  int nb, R, C, col_tiles;
};

// Up to three reductions per launch (one per parameter), selected by blockIdx.z.
struct ColSums {
  ColSum s[3];
};

// grid: x = n * col_tiles + column tile (up to the largest reduction), y = row group q
__global__ __launch_bounds__(256) void sdl_colsum_pass1(ColSums all) {
  const ColSum& cs = all.s[blockIdx.z];
  const float* in = cs.in;
  double* part = cs.part;
  const int R = cs.R, C = cs.C, col_tiles = cs.col_tiles;
  if (blockIdx.x >= static_cast<unsigned>(cs.nb * col_tiles)) return;  // uniform per block
  __shared__ double s_red[4][kWave];
  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int n = blockIdx.x / col_tiles;
  const int col = (blockIdx.x - n * col_tiles) * kWave + lane;
  const int q = blockIdx.y;
  const int cc = min(col, C - 1);
  const float* src = in + static_cast<size_t>(n) * R * C + cc;
  double acc = 0.0;
  constexpr int kStride = kSumGroups * 4;
  for (int r0 = q * 4 + w; r0 < R; r0 += kStride * 4) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = src[static_cast<size_t>(min(r0 + u * kStride, R - 1)) * C];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (r0 + u * kStride < R) acc += static_cast<double>(v[u]);
  }
  s_red[w][lane] = acc;
  __syncthreads();
  if (w == 0 && col < C)
    part[(static_cast<size_t>(n) * kSumGroups + q) * C + col] =
        ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
}

__global__ __launch_bounds__(256) void sdl_colsum_pass2(ColSums all) {
  const ColSum& cs = all.s[blockIdx.z];
  const double* part = cs.part;
  float* out = cs.out;
  const int C = cs.C, nb = cs.nb;
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<long long>(nb) * C) return;
  const int n = static_cast<int>(i / C), col = static_cast<int>(i - static_cast<long long>(n) * C);
  double s = 0.0;
#pragma unroll 8
  for (int q = 0; q < kSumGroups; ++q) s += part[(static_cast<size_t>(n) * kSumGroups + q) * C + col];
  out[i] = static_cast<float>(s);
}

// One launch for short reductions (R <= kDirectRows): a thread per output,
// its rows in order in fp64, eight loads in flight.
constexpr int kDirectRows = 256;
__global__ __launch_bounds__(256) void sdl_colsum_direct(ColSums all) {
  const ColSum& cs = all.s[blockIdx.z];
  const int C = cs.C, R = cs.R;
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<long long>(cs.nb) * C) return;
  const int n = static_cast<int>(i / C), col = static_cast<int>(i - static_cast<long long>(n) * C);
  const float* src = cs.in + static_cast<size_t>(n) * R * C + col;
  double s = 0.0;
  for (int r0 = 0; r0 < R; r0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[static_cast<size_t>(min(r0 + u, R - 1)) * C];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (r0 + u < R) s += static_cast<double>(v[u]);
  }
  cs.out[i] = static_cast<float>(s);
}

__global__ void sdl_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ============================================================================
// Host side
// ============================================================================
struct ParamShape {
  const float* p;
  int64_t la, ba;  // leading dims of [La, Ba, M]
};

int check_param(const ParamShape& s, int64_t L, int64_t B, const char* what, const char* name) {
  if (s.p == nullptr) return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null " + name);
  if (!(s.la == 1 || s.la == L) || !(s.ba == 1 || s.ba == B))
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     std::string(name) + " must have shape (L,B,M) with optional singleton L/B axes");
  return OSSM_OK;
}

ParamView view_of(const ParamShape& s, int64_t L, int64_t B, int64_t M) {
  ParamView v;
  v.p = s.p;
  v.t_stride = (s.la == 1 && L > 1) ? 0 : s.ba * M;
  v.by_channel = (s.ba == B) ? 1 : 0;
  return v;
}

// Runs the `n` reductions of `all`: in one launch when every one sums at
// most kDirectRows rows, else in two.
int launch_colsums(const ColSums& all, int n, hipStream_t stream) {
  if (n == 0) return OSSM_OK;
  int64_t max_blocks = 0, max_out = 0, max_rows = 0;
  for (int k = 0; k < n; ++k) {
    max_blocks = std::max<int64_t>(max_blocks, static_cast<int64_t>(all.s[k].nb) * all.s[k].col_tiles);
    max_out = std::max<int64_t>(max_out, static_cast<int64_t>(all.s[k].nb) * all.s[k].C);
    max_rows = std::max<int64_t>(max_rows, all.s[k].R);
  }
  if (max_blocks > INT_MAX || (max_out + 255) / 256 > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "gradient reduction too large");
  if (max_rows <= kDirectRows) {
    hipLaunchKernelGGL(sdl_colsum_direct, dim3(static_cast<unsigned>((max_out + 255) / 256), 1, n),
                       dim3(256), 0, stream, all);
    return launch_check("sdl_colsum_direct");
  }
  hipLaunchKernelGGL(sdl_colsum_pass1, dim3(static_cast<unsigned>(max_blocks), kSumGroups, n),
                     dim3(256), 0, stream, all);
  if (int rc = launch_check("sdl_colsum_pass1")) return rc;
  hipLaunchKernelGGL(sdl_colsum_pass2, dim3(static_cast<unsigned>((max_out + 255) / 256), 1, n),
                     dim3(256), 0, stream, all);
  return launch_check("sdl_colsum_pass2");
}

int fill_zero_f(float* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return OSSM_OK;
  hipLaunchKernelGGL(sdl_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, p, n);
  return launch_check("sdl_zero_kernel");
}

// Tiles (T steps per lane, W waves): defaults, and the instantiated choices
// for OSSM_SDL_TILE_FWD / OSSM_SDL_TILE_BWD ("TxW").
struct TileTW {
  int T, W;
};
#define OSSM_SDL_FWD_TILES(X) X(8, 16) X(16, 8) X(8, 8) X(16, 4) X(4, 16)
#define OSSM_SDL_BWD_TILES(X) X(8, 8) X(8, 4) X(4, 8) X(4, 16) X(16, 4) X(16, 8)

TileTW sdl_tile(const char* env, TileTW dflt) {
  const char* e = std::getenv(env);
  TileTW t{0, 0};
  if (e == nullptr || std::sscanf(e, "%dx%d", &t.T, &t.W) != 2) return dflt;
  return t;
}

template <int V, int T, int W>
int sdl_forward_tw(const SdlParams& prm, const void* bu, void* states, int64_t L, int64_t nc,
                   hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const int64_t n_chunks = (L + T * W - 1) / (T * W);
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  if (n_chunks * n_groups > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  const size_t rec_bytes = static_cast<size_t>(n_chunks) * kTvKinds * 4 * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  const int64_t total = n_chunks * n_groups;
  if (int rc = acquire_scratch(call, rec_bytes, total, &payload, &sync)) return rc;
  const bool tb = prm.a.t_stride == 0 && prm.g.t_stride == 0 && prm.s.t_stride == 0;
  // persistent (per-step parameters, ticket order) when the grid has more
  // chunks than the device holds workgroups at once
  static const int64_t cap = [] {
    int dev = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&sdl_forward_kernel<V, T, W, false, true>),
            W * kWave, 0) != hipSuccess) {
      (void)hipGetLastError();
      return int64_t(0);
    }
    return int64_t(per_cu) * device_cu_count(dev);
  }();
  const char* pe = std::getenv("OSSM_OSC_PERSIST");
  const bool persist = !tb && sync.use_ticket && cap > 0 && total > cap &&
                       !(pe != nullptr && std::string(pe) == "0");
  const auto kern = persist ? sdl_forward_kernel<V, T, W, false, true>
                            : (tb ? sdl_forward_kernel<V, T, W, true, false>
                                  : sdl_forward_kernel<V, T, W, false, false>);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(persist ? cap : total)),
                     dim3(W * kWave), 0, stream, prm, static_cast<const float2*>(bu),
                     static_cast<float4*>(states), static_cast<int>(L), static_cast<int>(nc),
                     static_cast<int>(n_groups), static_cast<int>(n_chunks),
                     static_cast<unsigned long long*>(payload), sync);
  if (int rc = launch_check("sdl_forward_kernel")) return rc;
  return OSSM_OK;
}

template <int V>
int sdl_forward_v(const SdlParams& prm, const void* bu, void* states, int64_t L, int64_t nc,
                  hipStream_t stream) {
  static const TileTW tile = sdl_tile("OSSM_SDL_TILE_FWD", TileTW{8, 16});
#define OSSM_SDL_FWD_CASE(TT, WW) \
  if (tile.T == TT && tile.W == WW) return sdl_forward_tw<V, TT, WW>(prm, bu, states, L, nc, stream);
  OSSM_SDL_FWD_TILES(OSSM_SDL_FWD_CASE)
#undef OSSM_SDL_FWD_CASE
  return set_error(OSSM_ERR_UNSUPPORTED, "OSSM_SDL_TILE_FWD names no built tile");
}

template <int V, int T, int W>
int sdl_backward_tw(const SdlParams& prm, const ParamShape (&shapes)[3], const void* bu,
                    const void* states, const void* gout, float* const (&grads)[3], void* gbu,
                    int64_t L, int64_t B, int64_t M, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const int64_t nc = B * M;
  const int64_t n_chunks = (L + T * W - 1) / (T * W);
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  if (n_chunks * n_groups > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  // Where each parameter's gradient goes: straight to the output (full
  // shape), per-chunk sums over time [n_chunks, B*M] (broadcast over time,
  // summed over the chunks and, if also broadcast over batch, the batch rows
  // afterwards), or per element [L, B*M] (broadcast over batch only, summed
  // over the batch rows afterwards).
  SdlGradOut dst{};
  size_t ws_floats = 0;
  size_t offs[3] = {0, 0, 0};
  int64_t max_out = 0;  // the largest reduction output (batches x columns)
  for (int p = 0; p < 3; ++p) {
    const bool rt = shapes[p].la == 1 && L > 1, rb = shapes[p].ba == 1 && B > 1;
    if (rt) dst.tsum |= 1 << p;
    if (rt || rb) {
      offs[p] = ws_floats;
      ws_floats += static_cast<size_t>(rt ? n_chunks : L) * nc;
      max_out = std::max<int64_t>(max_out, rt ? (rb ? M : nc) : L * M);
    }
  }
  double* part = nullptr;
  float* bufs = nullptr;
  if (ws_floats > 0) {
    const size_t buf_bytes = (ws_floats * sizeof(float) + 255) & ~static_cast<size_t>(255);
    const size_t part_bytes = 3 * static_cast<size_t>(kSumGroups) * max_out * sizeof(double);
    void* ws = nullptr;
    if (int rc = acquire_workspace(call, buf_bytes + part_bytes, &ws)) return rc;
    bufs = static_cast<float*>(ws);
    part = reinterpret_cast<double*>(static_cast<char*>(ws) + buf_bytes);
  }
  bool staged[3];
  for (int p = 0; p < 3; ++p) {
    staged[p] = (shapes[p].la == 1 && L > 1) || (shapes[p].ba == 1 && B > 1);
    dst.p[p] = staged[p] ? bufs + offs[p] : grads[p];
  }

  const size_t rec_bytes = static_cast<size_t>(n_chunks) * kTvKinds * 4 * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  const int64_t total = n_chunks * n_groups;
  if (int rc = acquire_scratch(call, rec_bytes, total, &payload, &sync)) return rc;
  const bool tb = prm.a.t_stride == 0 && prm.g.t_stride == 0 && prm.s.t_stride == 0;
  hipLaunchKernelGGL((tb ? sdl_backward_kernel<V, T, W, true> : sdl_backward_kernel<V, T, W, false>),
                     dim3(static_cast<unsigned>(total)),
                     dim3(W * kWave), 0, stream, prm, static_cast<const float2*>(bu),
                     static_cast<const float4*>(states), static_cast<const float2*>(gout),
                     static_cast<float2*>(gbu), dst, static_cast<int>(L), static_cast<int>(nc),
                     static_cast<int>(n_groups), static_cast<int>(n_chunks),
                     static_cast<unsigned long long*>(payload), sync);
  if (int rc = launch_check("sdl_backward_kernel")) return rc;
  ColSums sums{};
  int n_sums = 0;
  for (int p = 0; p < 3; ++p) {
    if (!staged[p]) continue;
    const bool rt = shapes[p].la == 1 && L > 1, rb = shapes[p].ba == 1 && B > 1;
    ColSum& cs = sums.s[n_sums];
    cs.in = dst.p[p];
    cs.out = grads[p];
    cs.part = part + static_cast<size_t>(n_sums) * kSumGroups * max_out;
    if (rt && rb) {  // [n_chunks, B, M] -> [M]
      cs.nb = 1; cs.R = static_cast<int>(n_chunks * B); cs.C = static_cast<int>(M);
    } else if (rt) {  // [n_chunks, B*M] -> [B*M]
      cs.nb = 1; cs.R = static_cast<int>(n_chunks); cs.C = static_cast<int>(nc);
    } else {  // [L, B, M] -> [L, M]
      cs.nb = static_cast<int>(L); cs.R = static_cast<int>(B); cs.C = static_cast<int>(M);
    }
    cs.col_tiles = (cs.C + kWave - 1) / kWave;
    ++n_sums;
  }
  return launch_colsums(sums, n_sums, stream);
}

template <int V>
int sdl_backward_v(const SdlParams& prm, const ParamShape (&shapes)[3], const void* bu,
                   const void* states, const void* gout, float* const (&grads)[3], void* gbu,
                   int64_t L, int64_t B, int64_t M, hipStream_t stream) {
  // Parameters broadcast over time run 8 waves of 16 steps (128-step chunks,
  // one workgroup per CU: 109 vs 116 us at config 2's shape), per-step
  // parameters 4 waves (the 8-wave tile is no faster for them).
  static const TileTW forced = sdl_tile("OSSM_SDL_TILE_BWD", TileTW{0, 0});
  const bool tb = prm.a.t_stride == 0 && prm.g.t_stride == 0 && prm.s.t_stride == 0;
  const TileTW tile = forced.T != 0 ? forced : (tb ? TileTW{16, 8} : TileTW{16, 4});
#define OSSM_SDL_BWD_CASE(TT, WW)                                                            \
  if (tile.T == TT && tile.W == WW)                                                          \
    return sdl_backward_tw<V, TT, WW>(prm, shapes, bu, states, gout, grads, gbu, L, B, M, stream);
  OSSM_SDL_BWD_TILES(OSSM_SDL_BWD_CASE)
#undef OSSM_SDL_BWD_CASE
  return set_error(OSSM_ERR_UNSUPPORTED, "OSSM_SDL_TILE_BWD names no built tile");
}

// Parameters all constant over time run on the oscillatory-scan kernels
// (sdl_tb_forward / sdl_tb_backward: chunk transitions as matrix powers, the
// D-LinOSS kernels' tiles) unless OSSM_SDL_TB_OSC=0 (read per call: tests
// run both).
bool tb_on_osc(const SdlParams& prm) {
  const char* e = std::getenv("OSSM_SDL_TB_OSC");
  const bool off = e != nullptr && std::string(e) == "0";
  return !off && prm.a.t_stride == 0 && prm.g.t_stride == 0 && prm.s.t_stride == 0;
}

// The backward with parameters constant over time on the oscillatory-scan
// kernels, in one launch: each chunk adds its share of the parameter
// gradients into grads (zeroed by the launch) with float atomics.
int sdl_backward_tb_osc(int variant, const SdlParams& prm, const void* bu, const void* states,
                        const void* gout, float* const (&grads)[3], void* gbu, int64_t L, int64_t B,
                        int64_t M, hipStream_t stream) {
  return sdl_tb_backward(variant, prm, bu, states, gout, gbu, grads, L, B * M, stream);
}

int check_sdl(int variant, int64_t L, int64_t B, int64_t M, const char* what) {
  if (variant < 0 || variant > 3)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown selective D-LinOSS variant code");
  if (L < 0 || B < 0 || M < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (L > INT_MAX / 2 || B * M > INT_MAX / 2 || L * B * M > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  return OSSM_OK;
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_sdlinoss_forward(int variant, const float* A, int64_t a_len, int64_t a_batch,
                          const float* G, int64_t g_len, int64_t g_batch, const float* step,
                          int64_t s_len, int64_t s_batch, const void* bu, void* states,
                          int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sdl(variant, length, batch, ssm, "sdlinoss_forward")) return rc;
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  const ParamShape shapes[3] = {{A, a_len, a_batch}, {G, g_len, g_batch}, {step, s_len, s_batch}};
  const char* names[3] = {"A", "G", "step"};
  for (int p = 0; p < 3; ++p)
    if (int rc = check_param(shapes[p], length, batch, "sdlinoss_forward", names[p])) return rc;
  if (!bu || !states) return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_forward: null pointer");
  const SdlParams prm{view_of(shapes[0], length, batch, ssm), view_of(shapes[1], length, batch, ssm),
                      view_of(shapes[2], length, batch, ssm), static_cast<int>(ssm)};
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const int64_t nc = batch * ssm;
  if (tb_on_osc(prm)) return sdl_tb_forward(variant, prm, bu, states, length, nc, stream);
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return sdl_forward_v<OSSM_DLINOSS_IMEX1>(prm, bu, states, length, nc, stream);
    case OSSM_DLINOSS_IMEX2: return sdl_forward_v<OSSM_DLINOSS_IMEX2>(prm, bu, states, length, nc, stream);
    case OSSM_DLINOSS_IM: return sdl_forward_v<OSSM_DLINOSS_IM>(prm, bu, states, length, nc, stream);
    default: return sdl_forward_v<OSSM_DLINOSS_EX>(prm, bu, states, length, nc, stream);
  }
}

int ossm_sdlinoss_backward(int variant, const float* A, int64_t a_len, int64_t a_batch,
                           const float* G, int64_t g_len, int64_t g_batch, const float* step,
                           int64_t s_len, int64_t s_batch, const void* bu, const void* states,
                           const void* grad_output, float* grad_A, float* grad_G,
                           float* grad_step, void* grad_bu, int64_t length, int64_t batch,
                           int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sdl(variant, length, batch, ssm, "sdlinoss_backward")) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const ParamShape shapes[3] = {{A, a_len, a_batch}, {G, g_len, g_batch}, {step, s_len, s_batch}};
  float* const grads[3] = {grad_A, grad_G, grad_step};
  if (length == 0 || batch == 0 || ssm == 0) {
    // nothing to scan: zero parameter gradients (the reference's zeros_like)
    for (int p = 0; p < 3; ++p) {
      if (grads[p] == nullptr) return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_backward: null pointer");
      if (int rc = fill_zero_f(grads[p], shapes[p].la * shapes[p].ba * ssm, stream)) return rc;
    }
    return OSSM_OK;
  }
  const char* names[3] = {"A", "G", "step"};
  for (int p = 0; p < 3; ++p)
    if (int rc = check_param(shapes[p], length, batch, "sdlinoss_backward", names[p])) return rc;
  if (!bu || !states || !grad_output || !grad_A || !grad_G || !grad_step || !grad_bu)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_backward: null pointer");
  const SdlParams prm{view_of(shapes[0], length, batch, ssm), view_of(shapes[1], length, batch, ssm),
                      view_of(shapes[2], length, batch, ssm), static_cast<int>(ssm)};
  if (tb_on_osc(prm))
    return sdl_backward_tb_osc(variant, prm, bu, states, grad_output, grads, grad_bu, length, batch,
                               ssm, stream);
  switch (variant) {
#define OSSM_SDL_BWD(V)                                                                          \
  case V:                                                                                        \
    return sdl_backward_v<V>(prm, shapes, bu, states, grad_output, grads, grad_bu, length, batch, \
                             ssm, stream);
    OSSM_SDL_BWD(OSSM_DLINOSS_IMEX1)
    OSSM_SDL_BWD(OSSM_DLINOSS_IMEX2)
    OSSM_SDL_BWD(OSSM_DLINOSS_IM)
    default:
      return sdl_backward_v<OSSM_DLINOSS_EX>(prm, shapes, bu, states, grad_output, grads, grad_bu,
                                             length, batch, ssm, stream);
#undef OSSM_SDL_BWD
  }
}

}  // extern "C"
