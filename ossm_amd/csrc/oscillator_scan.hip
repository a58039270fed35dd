// Oscillatory 2x2 scans on gfx950: D-LinOSS (imex1, imex2, im, ex) and the
// generic complex LinOSS scan, forward and backward.
//
// Layout and parallel decomposition
//   The reference tensors are [L, B, P(, 2)] with the (b, p) channel index
//   contiguous, so one wave = 64 consecutive channels and every per-step load
//   or store is one coalesced row (512 B of bu, 1 KiB of states).  A
//   workgroup of W waves owns one time chunk of W*T steps for its 64
//   channels; wave w owns the sub-chunk of T steps starting at w*T.
//
// Forward (one pass over HBM: read bu once, write states once)
//   1. each lane keeps its T inputs in registers and scans them from a zero
//      state -> sub-chunk aggregate e_w;
//   2. wave 0 combines the W aggregates through LDS with M^T (the sub-chunk
//      transition) into the chunk aggregate, publishes it, and looks back over
//      earlier chunks' records for the carry into the chunk (decoupled
//      look-back, workgroups ordered by a launch ticket);
//   3. every wave rebuilds its own carry from the LDS aggregates and re-runs
//      its T steps from it, storing the states.
//
// Backward (reverse time; reads bu + grad once, states only at chunk starts,
// writes grad_bu once)
//   The adjoint mu_t = M^T mu_{t+1} + (0, g_t) is the same chunked scan run
//   backwards with the transposed transition.  States s_{t-1} needed by the
//   parameter gradients are recomputed in registers from one checkpoint per
//   chunk, the state before its first step, and the waves' forward summaries
//   exchanged through LDS, instead of reading the whole trajectory.  Per-lane sums of
//   <mu_i, s_j,t-1> and <mu_i, bu_t> are added over the workgroup's waves;
//   each variant's chain rule is linear in them, so wave 0 applies it to its
//   chunk's per-channel sums and adds the result into grad a, g, dt with
//   float atomics, after the launch's order-0 workgroup has zeroed those
//   outputs and published its tag (zero_fill_publish, scan_reduce.hpp).  (A
//   separate column-sum launch with fixed-order fp64 row-group sums cost
//   4.4 us plus a launch gap at config 2; a last-workgroup-done reduction
//   inside the scan kernel was measured 3x slower: each agent-scope release
//   fence writes back the XCD's L2, dirty with the workgroup's grad_bu rows.)

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_device.hpp"
#include "scan_reduce.hpp"
#include "dlinoss_model.hpp"
#include "sdl_model.hpp"

namespace ossm {
namespace {

// ============================================================================
// Models: what one step of each recurrence does.
// ============================================================================

// Generic complex LinOSS: s_t = M s_{t-1} + b_t (linoss_scan.cpp:48-66).
struct Linoss {
  using In = float4;    // b_t (both components)
  using GIn = float4;   // grad of s_t
  using GOut = float4;  // grad of b_t
  using Mat = CMat;
  using Coef = CMat;
  static constexpr int kSums = 8;
  // The bridge keeps (M, states) but not b_seq (linoss.py:79), so the
  // backward reads s_{t-1} from the saved trajectory.
  static constexpr bool kRecompute = false;

  struct Params {
    const float2* m11;
    const float2* m12;
    const float2* m21;
    const float2* m22;
    int P;
    int nc;  // channels B * P: the row length of the backward's partials
  };

  using Raw = CMat;
  static __device__ __forceinline__ Raw load_raw(const Params& prm, int ch) {
    const int p = ch % prm.P;
    return {prm.m11[p], prm.m12[p], prm.m21[p], prm.m22[p]};
  }
  static __device__ __forceinline__ Coef coef_of(const Raw& r) { return r; }
  static __device__ __forceinline__ Coef coef(const Params& prm, int ch) { return load_raw(prm, ch); }
  static __device__ __forceinline__ float4 step(const Coef& m, float4 s, float4 b) {
    return f4add(mat_apply(m, s), b);
  }
  static __device__ __forceinline__ Mat matrix(const Coef& m) { return m; }
  static __device__ __forceinline__ float4 mu(float4 carry, float4 go) { return f4add(carry, go); }
  // grad_next = M^H g (linoss.py:144-146)
  static __device__ __forceinline__ float4 rev_carry(const Coef& m, float4 g) {
    return mat_apply(mat_adjoint(m), g);
  }
  static __device__ __forceinline__ float4 grad_input(const Coef&, float4 g) { return g; }
  // grad_M_ij += g_i * conj(s_j,t-1)  (linoss.py:129-133)
  static __device__ __forceinline__ void accumulate(float* acc, float4 g, float4 sp, float4) {
    acc[0] += g.x * sp.x + g.y * sp.y;  acc[1] += g.y * sp.x - g.x * sp.y;  // m11
    acc[2] += g.x * sp.z + g.y * sp.w;  acc[3] += g.y * sp.z - g.x * sp.w;  // m12
    acc[4] += g.z * sp.x + g.w * sp.y;  acc[5] += g.w * sp.x - g.z * sp.y;  // m21
    acc[6] += g.z * sp.z + g.w * sp.w;  acc[7] += g.w * sp.z - g.z * sp.w;  // m22
  }

  // grad_m [P, 2, 2] complex = the summed products themselves, each chunk's
  // share added with float atomics by the whole wave (kWaveEpilogue): the
  // wave's 64 channels x 8 sums go through LDS so that each atomic instruction
  // covers 64 consecutive floats of grad_m (two cache lines) instead of 64
  // lanes 32 bytes apart (16).  Issued lane by lane they queued in the memory
  // system: a copy of the kernel without them ran 154 us against 234 us at
  // [4096, 32, 128] (1024 shares per output), 13.7 against 22.9 us at config
  // 1's shape.  `active`: the lane's channel is below nc.
  static constexpr int kOutsPerColumn = 8;
  static constexpr bool kWaveEpilogue = true;
  // The 16 x 16 forward is at the 128-VGPR cap of a 16-wave workgroup (two
  // complex inputs per step): 9 registers spill one chunk per workgroup, 29
  // in the persistent loop (config 2's shape 94 -> 123 us), so it keeps one
  // workgroup per chunk.
  static constexpr bool kPersistForward = false;
  static __device__ void epilogue_wave(const Params& prm, int ch, const double* S, float* grad_m) {
    __shared__ float s_t[8 * kWave];
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) s_t[lane * 8 + j] = static_cast<float>(S[j]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int c0 = ch - lane;  // the wave's first channel
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int f = j * kWave + lane;  // sum f & 7 of the wave's channel f >> 3
      const int c = c0 + (f >> 3);
      if (c < prm.nc) atomic_put(grad_m + 8 * (c % prm.P) + (f & 7), static_cast<double>(s_t[f]));
    }
  }
};

// Selective D-LinOSS (sdlinoss_<v>.cpp) with A, G and step constant over time:
// per channel one set of coefficients, w' = c0 w + c1 x + c2 bu and x' = x + w'
// (the imex1 D-LinOSS step's shape, with (c0, c1, c2) = (alpha, -a dt^2, dt^2) / S
// of the variant; sdl_coef).  The parameter-gradient sums are the three
// contractions of the new w's gradient gw = mu_w + mu_x with w_{t-1}, x_{t-1}
// and bu_t, mapped to (dA, dG, dstep) by sdl_param_grads_of_sums (linear in the
// sums) and added per chunk into the parameter's gradient element (its batch
// row's, or the shared one of a parameter broadcast over the batch) with one
// float atomic each.
template <int V>
struct SdlTb {
  using In = float2;    // bu_t
  using GIn = float2;   // grad of x_t
  using GOut = float2;  // grad of bu_t
  using Mat = RMat;
  using Coef = SdlCoef<V>;
  static constexpr int kSums = 3;
  static constexpr bool kRecompute = true;

  struct Params {
    SdlParams v;
    int P;  // M (the oscillators per batch row)
    int nc;
  };
  struct Raw {
    float a, g, s;
  };
  static __device__ __forceinline__ int at(const ParamView& pv, int ch, int M) {
    return pv.by_channel ? ch : ch % M;
  }
  static __device__ __forceinline__ Raw load_raw(const Params& prm, int ch) {
    return {prm.v.a.p[at(prm.v.a, ch, prm.P)], prm.v.g.p[at(prm.v.g, ch, prm.P)],
            prm.v.s.p[at(prm.v.s, ch, prm.P)]};
  }
  static __device__ __forceinline__ Coef coef_of(const Raw& r) { return sdl_coef<V>(r.a, r.g, r.s); }
  static __device__ __forceinline__ Coef coef(const Params& prm, int ch) { return coef_of(load_raw(prm, ch)); }
  static __device__ __forceinline__ float4 step(const Coef& k, float4 s, float2 bu) {
    return sdl_step<V>(k, s, bu);
  }
  static __device__ __forceinline__ Mat matrix(const Coef& k) { return {k.c0, k.c1, k.c0, 1.f + k.c1}; }
  static __device__ __forceinline__ float4 mu(float4 carry, float2 go) {
    return make_float4(carry.x, carry.y, carry.z + go.x, carry.w + go.y);
  }
  // carry to t-1 = M^T mu: (c0 gw, mu_x + c1 gw), gw = mu_w + mu_x
  static __device__ __forceinline__ float4 rev_carry(const Coef& k, float4 m) {
    const float gr = m.x + m.z, gi = m.y + m.w;
    return make_float4(k.c0 * gr, k.c0 * gi, fmaf(k.c1, gr, m.z), fmaf(k.c1, gi, m.w));
  }
  static __device__ __forceinline__ float2 grad_input(const Coef& k, float4 m) {
    return make_float2(k.c2 * (m.x + m.z), k.c2 * (m.y + m.w));
  }
  static __device__ __forceinline__ void accumulate(float* acc, float4 m, float4 sp, float2 bu) {
    const float gr = m.x + m.z, gi = m.y + m.w;
    acc[0] = fmaf(gr, sp.x, fmaf(gi, sp.y, acc[0]));  // gw . w_{t-1}
    acc[1] = fmaf(gr, sp.z, fmaf(gi, sp.w, acc[1]));  // gw . x_{t-1}
    acc[2] = fmaf(gr, bu.x, fmaf(gi, bu.y, acc[2]));  // gw . bu_t
  }
  static constexpr int kOutsPerColumn = 0;
  static constexpr bool kWaveEpilogue = false;
  static constexpr bool kPersistForward = true;  // no spills either way (105 VGPRs)
  static __device__ void epilogue(const Params& prm, int ch, int /*chunk*/, const double* S, float* pa,
                                  float* pg, float* ps) {
    const Raw r = load_raw(prm, ch);
    float ga, gg, gs;
    sdl_param_grads_of_sums<V>(r.a, r.g, r.s, sdl_inv_of<V>(r.a, r.g, r.s), static_cast<float>(S[0]),
                               static_cast<float>(S[1]), static_cast<float>(S[2]), ga, gg, gs);
    atomic_put(pa + at(prm.v.a, ch, prm.P), ga);
    atomic_put(pg + at(prm.v.g, ch, prm.P), gg);
    atomic_put(ps + at(prm.v.s, ch, prm.P), gs);
  }
};

// ============================================================================
// Forward kernel
// ============================================================================
// PERSIST (ticket order, a grid of fewer workgroups than chunks): workgroup b
// takes ceil((total - b) / grid) chunks one after the other, so the launch
// still draws exactly `total` tickets (the protocol of launch_order,
// out-of-range tickets included), and draws each next ticket while it
// stores the current chunk: the atomic's round trip and the start of a new
// workgroup leave the path from one chunk to the next.  A workgroup holding
// a drawn ticket is running and takes that chunk next without waiting on
// anything, so every look-back still ends.
template <class Model, int T, int W, int OCC, bool PERSIST>
__global__ __launch_bounds__(W * kWave, OCC) void osc_forward_kernel(
    typename Model::Params prm, const typename Model::In* __restrict__ in,
    float4* __restrict__ out, int L, int nc, int n_groups, int n_chunks,
    unsigned long long* __restrict__ rec, LaunchSync sync) {
  __shared__ float4 s_agg[W][kWave];
  __shared__ float4 s_carry[kWave];
  __shared__ int s_ticket;
  __shared__ unsigned int s_tag;
  __shared__ int s_poison;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int total = n_groups * n_chunks;
  int order;
  int left = 1;  // chunks this workgroup still takes, the current one included
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
  const auto k = Model::coef(prm, active ? ch : 0);
  const long long t0 = static_cast<long long>(c) * (T * W) + static_cast<long long>(w) * T;

  // Clamped in-range addresses and no selects on the loaded values: the
  // aggregate below consumes the steps as they arrive instead of waiting for
  // all T loads (steps past L and inactive lanes are never used).
  typename Model::In x[T];
  const unsigned lc = clamped_lane(g, nc);
#pragma unroll
  for (int i = 0; i < T; ++i) x[i] = group_row(in, min(t0 + i, static_cast<long long>(L - 1)), nc, g)[lc];

  // 1. sub-chunk aggregate from a zero state (FULL: all T steps in range)
  const bool full = t0 + T <= L;
  float4 e = f4zero();
  if (full) {
#pragma unroll
    for (int i = 0; i < T; ++i) e = Model::step(k, e, x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < T; ++i)
      if (t0 + i < L) e = Model::step(k, e, x[i]);
  }
  s_agg[w][lane] = e;
  const typename Model::Mat MT = mat_pow(Model::matrix(k), T);
  __syncthreads();

  // 2. chunk aggregate, look-back, inclusive prefix.  The aggregate is
  // published by wave 1 while wave 0 walks back: a wave's loads complete in
  // issue order behind its own stores, so a look-back issued after the
  // publishing store would first wait for that store to reach memory.
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    float4 E = f4zero();
#pragma unroll
    for (int v = 0; v < W; ++v) E = f4add(mat_apply(MT, E), s_agg[v][lane]);
    const bool scan = active && n_chunks > 1;
    if (w == kPub && scan && c > 0) rec_publish(rec, c, kRecAgg, nc, ch, E, sync.tag);
    if (w == 0) {
      float4 carry = f4zero();
      if (scan) {
        const typename Model::Mat MC = mat_pow(Model::matrix(k), T * W);
        if (c == 0) {
          rec_publish(rec, c, kRecInc, nc, ch, E, sync.tag);
        } else {
          carry = lookback(rec, c, +1, n_chunks, nc, ch, MC, sync);
          if (c + 1 < n_chunks) rec_publish(rec, c, kRecInc, nc, ch, f4add(mat_apply(MC, carry), E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }
  __syncthreads();

  // 3. own carry, then re-run the sub-chunk and store (PERSIST: the next
  // ticket is drawn first, its round trip overlapping the stores)
  int next = 0, next_poison = 0;
  if constexpr (PERSIST) {
    if (threadIdx.x == 0 && left > 1) {
      unsigned int tag = 0;
      next = draw_ticket(sync, total, &tag, &next_poison);
    }
  }
  float4 s = s_carry[lane];
  for (int v = 0; v < w; ++v) s = f4add(mat_apply(MT, s), s_agg[v][lane]);
  if (active) {
    if (full) {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        s = Model::step(k, s, x[i]);
        stream_store(&group_row(out, t0 + i, nc, g)[lane], s);
      }
    } else {
#pragma unroll
      for (int i = 0; i < T; ++i) {
        const long long t = t0 + i;
        if (t < L) {
          s = Model::step(k, s, x[i]);
          stream_store(&group_row(out, t, nc, g)[lane], s);
        }
      }
    }
  }
  if constexpr (!PERSIST) break;
  if (--left == 0) break;
  // every wave is past its reads of s_agg and s_carry before the next chunk
  // writes them
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
// Backward kernel
// ============================================================================
// One workgroup's inputs for one chunk, loaded ahead of its use.  Loads use
// clamped in-range addresses and no branches; out-of-range steps are masked
// where the values are consumed.
template <class Model, int T>
struct BwdBuf {
  typename Model::In x[Model::kRecompute ? T : 1];  // bu_t (recomputing models)
  float4 sp[Model::kRecompute ? 1 : T];             // s_{t-1} read from states (LinOSS)
  typename Model::GIn go[T];
  float4 ck;  // states at the chunk's start, then the wave's s_{t0-1} (recomputing models)
  typename Model::Raw raw;                          // the channel's oscillator parameters
};

struct BwdTicket {
  int c, g, ch;
  bool active;
  long long t0;  // first step of this wave's sub-chunk
};

template <int T, int W>
__device__ __forceinline__ BwdTicket bwd_ticket(int ticket, int n_groups, int n_chunks, int nc) {
  BwdTicket k;
  const int cr = ticket / n_groups;  // chunks are handed out last-first
  k.g = ticket - cr * n_groups;
  k.c = n_chunks - 1 - cr;
  k.ch = k.g * kWave + (threadIdx.x & (kWave - 1));
  k.active = k.ch < nc;
  k.t0 = static_cast<long long>(k.c) * (T * W) + static_cast<long long>(wave_id()) * T;
  return k;
}

template <class Model, int T, int W>
__device__ __forceinline__ void bwd_load(BwdBuf<Model, T>& b, const BwdTicket& k,
                                         const typename Model::Params& prm,
                                         const typename Model::In* __restrict__ in,
                                         const float4* states,
                                         const typename Model::GIn* __restrict__ gout, int L,
                                         int nc) {
  // Issue order = order of use (loads complete in order): parameters and the
  // checkpoint, then the forward recompute's inputs, then the upstream
  // gradient last step first, as the reverse sweep consumes it.
  const unsigned lc = clamped_lane(k.g, nc);
  b.raw = Model::load_raw(prm, k.g * kWave + static_cast<int>(lc));
  if constexpr (Model::kRecompute)
    b.ck = group_row(states, max(min(static_cast<long long>(k.c) * (T * W) - 1,
                                     static_cast<long long>(L - 1)), 0ll), nc, k.g)[lc];
  asm volatile("" ::: "memory");  // keep the issue order: the compiler would sink these
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if constexpr (Model::kRecompute)
      b.x[i] = group_row(in, min(k.t0 + i, static_cast<long long>(L - 1)), nc, k.g)[lc];
    else
      b.sp[i] = group_row(states, max(min(k.t0 + i - 1, static_cast<long long>(L - 1)), 0ll), nc, k.g)[lc];
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = T - 1; i >= 0; --i)
    b.go[i] = group_row(gout, min(k.t0 + i, static_cast<long long>(L - 1)), nc, k.g)[lc];
}

// First part of one chunk: reverse aggregate, look-back for the carry from
// later chunks.  Returns the carry into the wave's sub-chunk (the adjoint
// after its last step) and sets KT = (M^T)^T.  For recomputing models the
// states s_{t-1} are rebuilt from one checkpoint per chunk, the state before
// its first step: wave 0 runs its sub-chunk from it, the other waves first run
// theirs from a zero state, and each wave v passes its result (wave 0: its end
// state; the others: the sub-chunk's effect on a zero state) to the later
// waves through slot kLink of its LDS staging region, from which wave w folds
// its own first state s_{t0-1} = M^T (...(M^T e_0 + f_1)...) + f_{w-1}.  The
// states are staged in H segments of T/H steps (S slots per wave) just before
// the final pass reads them (bwd_back): with H = 1 the front stages all of
// them; with H = 2 it only runs to the middle of the sub-chunk (s_mid) and the
// back recomputes each half in turn, halving the LDS footprint for one extra
// half sweep.  SS = 2 (H = 1 only) stages every other state, s_{t-1} of the
// even steps; the back rebuilds an odd step's from the even one before it with
// one forward step, for half the LDS.  Slot kLink is read by the later waves
// between the two barriers, so a staged state that belongs there waits in a
// register until after the second.  All waves call it together.
template <class Model, int T, int W, int S, int H, int SS>
__device__ __forceinline__ float4 bwd_front(
    BwdBuf<Model, T>& b, const BwdTicket& k, int L, int nc, int n_chunks,
    unsigned long long* __restrict__ rec, const LaunchSync& sync, float4 (*s_agg)[kWave],
    float4* s_carry, float4 (*s_sp)[S][kWave], typename Model::Mat& KT, float4& s_mid) {
  static_assert(H == 1 || H == 2, "one or two staging segments");
  constexpr int kLink = S - 1;
  constexpr bool kLinkStaged = H == 1 && kLink < T / SS;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const auto cf = Model::coef_of(b.raw);
  float4 held = f4zero();

  // The forward recurrence over the sub-chunk from s.  MODE 0 runs it only
  // for its result; 1 also stages (H = 1: s_{t-1} of every SS-th step; H = 2:
  // s_mid); 2 stages and stops where staging ends.  Steps at or past L are
  // never used (every use below is guarded), and lanes past the last channel
  // only feed values that are never stored, so the loaded buffers need no
  // masking.  FULL: the whole sub-chunk is in range (uniform), so the step
  // loops run without guards.
  auto forward = [&](auto full_tag, auto mode_tag, float4 s) -> float4 {
    constexpr bool FULL = decltype(full_tag)::value;
    constexpr int MODE = decltype(mode_tag)::value;
    constexpr int N = MODE == 2 && H == 2 ? T / 2 : T;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if constexpr (MODE != 0 && H == 1) {
        if (i % SS == 0) {
          if (i / SS == kLink)
            held = s;
          else
            s_sp[w][i / SS][lane] = s;
        }
      }
      if constexpr (MODE == 1 && H == 2) {
        if (i == T / 2) s_mid = s;
      }
      if (FULL || k.t0 + i < L) s = Model::step(cf, s, b.x[i]);
    }
    if constexpr (MODE == 2 && H == 2) s_mid = s;
    return s;
  };
  using Summary = std::integral_constant<int, 0>;
  using StageAll = std::integral_constant<int, 1>;
  using Stage = std::integral_constant<int, 2>;
  const float4 start0 = k.c > 0 ? b.ck : f4zero();

  auto sweep = [&](auto full_tag) -> float4 {
    constexpr bool FULL = decltype(full_tag)::value;
    auto live = [&](int i) { return FULL || k.t0 + i < L; };
    if constexpr (Model::kRecompute) {
      const float4 link =
          w == 0 ? forward(full_tag, StageAll{}, start0) : forward(full_tag, Summary{}, f4zero());
      s_sp[w][kLink][lane] = link;
    } else {
      if (k.t0 == 0) b.sp[0] = f4zero();  // s_{-1} = 0
    }
    // 1. reverse aggregate of the sub-chunk from a zero carry
    float4 m = f4zero();
#pragma unroll
    for (int i = T - 1; i >= 0; --i)
      if (live(i)) m = Model::rev_carry(cf, Model::mu(m, b.go[i]));
    return m;
  };
  const bool full = k.t0 + T <= L;
  const float4 m = full ? sweep(std::true_type{}) : sweep(std::false_type{});
  s_agg[w][lane] = m;
  KT = mat_pow(mat_adjoint(Model::matrix(cf)), T);
  typename Model::Mat KC{};
  if (w == 0 && n_chunks > 1) KC = mat_pow(mat_adjoint(Model::matrix(cf)), T * W);
  __syncthreads();

  // 2. chunk aggregate (waves W-1 .. 0), look-back over later chunks; the
  // aggregate is published by wave 1 so that wave 0's look-back loads do not
  // queue behind the publishing stores (a wave's memory operations complete
  // in issue order)
  constexpr int kPub = W > 1 ? 1 : 0;
  if (w == 0 || w == kPub) {
    float4 E = f4zero();
#pragma unroll
    for (int v = W - 1; v >= 0; --v) E = f4add(mat_apply(KT, E), s_agg[v][lane]);
    const bool scan = k.active && n_chunks > 1;
    if (w == kPub && scan && k.c < n_chunks - 1) rec_publish(rec, k.c, kRecAgg, nc, k.ch, E, sync.tag);
    if (w == 0) {
      float4 carry = f4zero();
      if (scan) {
        if (k.c == n_chunks - 1) {
          rec_publish(rec, k.c, kRecInc, nc, k.ch, E, sync.tag);
        } else {
          carry = lookback(rec, k.c, -1, n_chunks, nc, k.ch, KC, sync);
          if (k.c > 0) rec_publish(rec, k.c, kRecInc, nc, k.ch, f4add(mat_apply(KC, carry), E), sync.tag);
        }
      }
      s_carry[lane] = carry;
    }
  }

  // 3. the other waves' first states, and their staging, while wave 0 walks back
  if constexpr (Model::kRecompute) {
    if (w > 0) {
      const typename Model::Mat MT = mat_pow(Model::matrix(cf), T);
      float4 s = s_sp[0][kLink][lane];
      for (int v = 1; v < w; ++v) s = f4add(mat_apply(MT, s), s_sp[v][kLink][lane]);
      b.ck = s;
      if (full)
        forward(std::true_type{}, Stage{}, s);
      else
        forward(std::false_type{}, Stage{}, s);
    } else {
      b.ck = start0;
    }
  }
  __syncthreads();
  if constexpr (Model::kRecompute && kLinkStaged) s_sp[w][kLink][lane] = held;

  // the wave's own carry: the chunk carry through the later waves' sub-chunks
  float4 y = s_carry[lane];
  for (int v = W - 1; v > w; --v) y = f4add(mat_apply(KT, y), s_agg[v][lane]);
  return y;
}

// Second part: the final reverse pass (grad of the inputs and the parameter
// sums) from carry y, then the chunk's share of the parameter gradients.
// `sp_lds` is the wave's own S = T/H staging slots (see bwd_front); `s_sums`
// holds each wave's NS sums, which wave 0 adds after a barrier.  The
// variant's chain rule is linear in the sums, so wave 0 applies it to the
// chunk's per-channel sums and adds the result into the outputs `zero` names
// (zeroed by the launch's order-0 workgroup, zero_fill_publish).
template <class Model, int T, int W, int H, int SS>
__device__ __forceinline__ void bwd_back(BwdBuf<Model, T>& b, const BwdTicket& k, float4 y,
                                         float4 s_mid, float4* sp_lds,
                                         typename Model::GOut* __restrict__ gin,
                                         const typename Model::Params& prm, const ZeroFill& zero,
                                         const LaunchSync& sync, int L, int nc, float* s_sums,
                                         int sums_stride) {
  constexpr int NS = Model::kSums;
  constexpr int Q = T / H;  // steps per staged segment
  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const auto cf = Model::coef_of(b.raw);
  float acc[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) acc[j] = 0.f;
  auto sweep = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    auto live = [&](int i) { return FULL || k.t0 + i < L; };
#pragma unroll
    for (int h = H - 1; h >= 0; --h) {
      if constexpr (Model::kRecompute && H > 1) {
        // stage segment h: s_{t-1} for its Q steps, from its first state
        float4 s = h == 0 ? b.ck : s_mid;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          sp_lds[q * kWave + lane] = s;
          if (live(h * Q + q)) s = Model::step(cf, s, b.x[h * Q + q]);
        }
      }
#pragma unroll
      for (int q = Q - 1; q >= 0; --q) {
        const int i = h * Q + q;
        if (live(i)) {
          const float4 mu = Model::mu(y, b.go[i]);
          stream_store(&group_row(gin, k.t0 + i, nc, k.g)[lane], Model::grad_input(cf, mu));
          if constexpr (Model::kRecompute && SS == 2) {
            const float4 se = sp_lds[(i / 2) * kWave + lane];  // s_{t-1} of the even step
            Model::accumulate(acc, mu, (i & 1) ? Model::step(cf, se, b.x[i - 1]) : se, b.x[i]);
          } else if constexpr (Model::kRecompute)
            Model::accumulate(acc, mu, sp_lds[(H > 1 ? q : i) * kWave + lane], b.x[i]);
          else
            Model::accumulate(acc, mu, b.sp[i], b.x[0]);
          y = Model::rev_carry(cf, mu);
        }
      }
    }
  };
  if (k.active) {
    if (k.t0 + T <= L)
      sweep(std::true_type{});
    else
      sweep(std::false_type{});
  }
  float* mine = s_sums + w * sums_stride;
#pragma unroll
  for (int j = 0; j < NS; ++j) mine[j * kWave + lane] = acc[j];
  __syncthreads();

  // this chunk's share of the parameter gradients (one channel per lane)
  if (w == 0) {
    double S[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      float v = 0.f;
      for (int u = 0; u < W; ++u) v += s_sums[u * sums_stride + j * kWave + lane];
      S[j] = v;
    }
    if (!wait_outputs_zeroed(sync)) {
#pragma unroll
      for (int j = 0; j < NS; ++j) S[j] = __builtin_nan("");
    }
    if constexpr (Model::kWaveEpilogue)
      Model::epilogue_wave(prm, k.ch, S, zero.p[0]);
    else if (k.active)
      Model::epilogue(prm, k.ch, k.c, S, zero.p[0], zero.p[1], zero.p[2]);
  }
}

// One workgroup per (chunk, channel group), chunks handed out last-first in
// launch-ticket order (so every chunk a look-back waits on is resident).
template <class Model, int T, int W, int OCC, int H, int SS>
__global__ __launch_bounds__(W * kWave, OCC) void osc_backward_kernel(
    typename Model::Params prm, const typename Model::In* __restrict__ in,
    const float4* states, const typename Model::GIn* __restrict__ gout,
    typename Model::GOut* __restrict__ gin, ZeroFill zero, int L, int nc, int n_groups,
    int n_chunks, unsigned long long* __restrict__ rec, LaunchSync sync) {
  constexpr int NS = Model::kSums;
  __shared__ float4 s_agg[W][kWave];
  __shared__ float4 s_carry[kWave];
  // per wave: its T / H staged states s_{t-1}, later its NS partial sums
  static_assert(SS == 1 || (SS == 2 && H == 1 && T % 2 == 0), "every other state: one segment");
  constexpr int kStage = Model::kRecompute ? T / H / SS : 0;
  constexpr int kSlots = kStage > (NS + 3) / 4 ? kStage : (NS + 3) / 4;
  __shared__ float4 s_sp[W][kSlots][kWave];
  __shared__ int s_ticket;
  const int ticket = launch_order(sync, n_groups * n_chunks, &s_ticket);
  if (ticket == 0) zero_fill_publish(zero, sync);  // the parameter-gradient outputs
  const BwdTicket k = bwd_ticket<T, W>(ticket, n_groups, n_chunks, nc);
  BwdBuf<Model, T> b;
  bwd_load<Model, T, W>(b, k, prm, in, states, gout, L, nc);
  typename Model::Mat KT;
  float4 s_mid = f4zero();
  const float4 y = bwd_front<Model, T, W, kSlots, H, SS>(b, k, L, nc, n_chunks, rec, sync, s_agg,
                                                         s_carry, s_sp, KT, s_mid);
  // the per-wave sums go into the wave's own s_{t-1} region, which only the
  // wave itself reads before this point
  bwd_back<Model, T, W, H, SS>(b, k, y, s_mid, &s_sp[wave_id()][0][0], gin, prm, zero, sync, L,
                               nc, reinterpret_cast<float*>(&s_sp[0][0][0]), kSlots * kWave * 4);
}

// T steps per lane, W waves per workgroup, OCC = minimum waves per SIMD the
// register allocation must allow (__launch_bounds__' second argument).
// H (backward only) = staging segments of the recomputed states, S (backward
// only) = 1, or 2 to stage every other state.
struct Tile {
  int T, W, O, H, S;
};

// "TxWxO", "TxWxOxH" or "TxWxOxHxS" (H and S default to 1).
Tile parse_tile(const char* env, Tile dflt) {
  const char* s = std::getenv(env);
  if (!s) return dflt;
  int t = 0, w = 0, o = 0, h = 1, st = 1;
  const int n = std::sscanf(s, "%dx%dx%dx%dx%d", &t, &w, &o, &h, &st);
  if (n < 3) return dflt;
  return {t, w, o, h, st};
}

// Instantiated tiles (T, W, OCC).
#define OSSM_FWD_TILES(X) \
  X(16, 8, 1) X(16, 16, 1) X(16, 8, 4) X(8, 8, 4) X(16, 4, 4) X(8, 16, 4) X(32, 4, 2)
// Backward tiles (T, W, OCC, H, S): H = staging segments of the recomputed
// states, S = 2 stages every other one.
#define OSSM_BWD_TILES(X)                                                                     \
  X(16, 8, 1, 1, 1) X(16, 8, 4, 2, 1) X(16, 8, 2, 2, 1) X(16, 4, 1, 1, 1) X(8, 8, 1, 1, 1)    \
  X(8, 8, 4, 2, 1) X(32, 4, 1, 1, 1) X(32, 4, 2, 2, 1) X(8, 16, 1, 1, 1) X(16, 8, 4, 1, 2)   \
  X(16, 8, 1, 1, 2) X(16, 16, 1, 1, 2)

// Launch geometry of a forward scan: the tile, the chunk grid and the bytes
// of look-back records it needs (two 4-word records per chunk and channel).
struct FwdPlan {
  Tile tile;
  int64_t n_chunks, n_groups, total;
  size_t rec_bytes;
};

// Without OSSM_OSC_TILE_FWD: 16 steps x 16 waves (256-step chunks, half the
// look-back records and depth of 128-step ones), unless that leaves fewer
// than 128 workgroups; then 16 x 8.  Measured (imex1, events, us; 16x8,
// 8x16 at four waves per SIMD, 16x16) at [L, B, P]: [1024, 8, 64] 8.8, 9.0,
// 9.7 (32 workgroups at 256 steps); [4096, 8, 128] 23.4, 22.0, 19.6;
// [1024, 32, 128] 21.0, 18.9, 18.2; [8192, 16, 64] 39.1, 37.5, 34.4;
// [4096, 16, 128] 37.7, 35.5, 33.3; [4096, 32, 128] 66.1, 63.1, 62.8;
// [2048, 32, 256] 66.0, 62.7, 61.9; [16384, 8, 128] 70.1, 68.8, 64.2;
// [4096, 64, 128] 139.6, 146.7, 129.0; [65536, 4, 256] 285.5, 309.6, 278.6.
FwdPlan fwd_plan_with(int64_t L, int64_t nc, Tile tile) {
  FwdPlan pl;
  pl.tile = tile;
  const int64_t CL = int64_t(tile.T) * tile.W;
  pl.n_groups = (nc + kWave - 1) / kWave;
  pl.n_chunks = (L + CL - 1) / CL;
  pl.total = pl.n_chunks * pl.n_groups;
  pl.rec_bytes = static_cast<size_t>(pl.n_chunks) * 2 * 4 * nc * sizeof(unsigned long long);
  return pl;
}

FwdPlan fwd_plan(int64_t L, int64_t nc) {
  static const Tile env_tile = parse_tile("OSSM_OSC_TILE_FWD", Tile{0, 0, 0, 1, 1});
  if (env_tile.T > 0) return fwd_plan_with(L, nc, env_tile);
  const bool wide = (L + 255) / 256 * ((nc + kWave - 1) / kWave) >= 128;
  return fwd_plan_with(L, nc, wide ? Tile{16, 16, 1, 1, 1} : Tile{16, 8, 1, 1, 1});
}

// Enqueues the forward kernel of plan `pl` with look-back records at
// `payload` and launch bookkeeping `sync`; `tm` (when set) are events the
// launch records as its own start and end.  The caller undoes its ticket
// reservation when this returns an error (nothing was launched).
// Workgroups of a persistent forward with tile (TT, WW, OO): as many as the
// device holds at once (0 when the occupancy query fails: no persistent launch).
template <class Model, int TT, int WW, int OO>
int64_t forward_persist_grid() {
  static const int64_t cap = [] {
    int dev = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&osc_forward_kernel<Model, TT, WW, OO, true>),
            WW * kWave, 0) != hipSuccess) {
      (void)hipGetLastError();
      return int64_t(0);
    }
    return int64_t(per_cu) * device_cu_count(dev);
  }();
  return cap;
}

// OSSM_OSC_PERSIST=0 (read per call) launches one workgroup per chunk always.
bool forward_persist_enabled() {
  const char* e = std::getenv("OSSM_OSC_PERSIST");
  return e == nullptr || std::string(e) != "0";
}

template <class Model>
int enqueue_forward(const FwdPlan& pl, const typename Model::Params& prm, const void* in, void* out,
                    int64_t L, int64_t nc, hipStream_t stream, void* payload, const LaunchSync& sync,
                    const LaunchTiming& tm = LaunchTiming{}) {
  const Tile& tile = pl.tile;
  bool launched = false;
#define OSSM_FWD_ARGS                                                                         \
  prm, static_cast<const typename Model::In*>(in), static_cast<float4*>(out),                 \
      static_cast<int>(L), static_cast<int>(nc), static_cast<int>(pl.n_groups),               \
      static_cast<int>(pl.n_chunks), static_cast<unsigned long long*>(payload), sync
#define OSSM_FWD_LAUNCH_ONE(TT, WW, OO, PP, NWG)                                              \
  {                                                                                           \
    const dim3 grid(static_cast<unsigned>(NWG));                                              \
    if (tm.start != nullptr)                                                                  \
      hipExtLaunchKernelGGL((osc_forward_kernel<Model, TT, WW, OO, PP>), grid,                \
                            dim3(WW * kWave), 0, stream, tm.start, tm.stop, 0, OSSM_FWD_ARGS); \
    else                                                                                      \
      hipLaunchKernelGGL((osc_forward_kernel<Model, TT, WW, OO, PP>), grid, dim3(WW * kWave), \
                         0, stream, OSSM_FWD_ARGS);                                           \
  }
  // the default tiles (16 x 16 and 16 x 8) run persistent in ticket order
  // when the grid has more chunks than the device holds workgroups at once
  // (models whose persistent loop spills excepted: Model::kPersistForward)
#define OSSM_LAUNCH_FWD(TT, WW, OO)                                                           \
  if (!launched && tile.T == TT && tile.W == WW && tile.O == OO) {                            \
    bool persist = false;                                                                     \
    if constexpr (Model::kPersistForward && TT == 16 && OO == 1 && (WW == 16 || WW == 8)) {   \
      const int64_t cap = forward_persist_grid<Model, TT, WW, OO>();                          \
      persist = sync.use_ticket && cap > 0 && pl.total > cap && forward_persist_enabled();     \
      if (persist) OSSM_FWD_LAUNCH_ONE(TT, WW, OO, true, cap)                                 \
    }                                                                                         \
    if (!persist) OSSM_FWD_LAUNCH_ONE(TT, WW, OO, false, pl.total)                            \
    launched = true;                                                                          \
  }
  OSSM_FWD_TILES(OSSM_LAUNCH_FWD)
#undef OSSM_LAUNCH_FWD
#undef OSSM_FWD_LAUNCH_ONE
#undef OSSM_FWD_ARGS
  if (!launched) return set_error(OSSM_ERR_UNSUPPORTED, "OSSM_OSC_TILE_FWD names no built tile");
  return launch_check("osc_forward_kernel");
}

template <class Model>
int launch_forward(const typename Model::Params& prm, const void* in, void* out, int64_t L,
                   int64_t nc, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const FwdPlan pl = fwd_plan(L, nc);
  if (pl.total > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  LaunchTiming tm;
  if (int rc = take_launch_timing(call, &tm)) return rc;
  void* payload = nullptr;
  LaunchSync sync{};
  if (int rc = acquire_scratch(call, pl.rec_bytes, pl.total, &payload, &sync)) return rc;
  if (int rc = enqueue_forward<Model>(pl, prm, in, out, L, nc, stream, payload, sync, tm)) return rc;
  return OSSM_OK;
}

// The backward's tile for L steps of nc channels (see launch_backward).
Tile bwd_tile(int64_t L, int64_t nc, bool recompute) {
  // Without OSSM_OSC_TILE_BWD: 16 x 16 (256-step chunks, one 16-wave workgroup
  // per CU, 145 KiB of LDS) for 128..2047 workgroups at that chunk length, else
  // 16 x 8.  Measured (imex1, events, us, 16x8 vs 16x16) at [L, B, P]:
  // [1024, 8, 64] 12.9 vs 15.5 (32 workgroups); [4096, 8, 128] 29.6 vs 24.1;
  // [1024, 32, 128] 26.7 vs 22.8; [8192, 16, 64] 46.8 vs 43.7; [4096, 16, 128]
  // 46.5 vs 42.9; [16384, 4, 256] 84.5 vs 78.3; [4096, 32, 128] 78.6 vs 76.6;
  // [2048, 32, 256] 79.5 vs 71.2; [16384, 8, 128] 84.1 vs 78.2; [4096, 64, 128]
  // 155.1 vs 164.7 (2048 workgroups).  Sixteen waves cap a lane at 128 VGPRs:
  // imex1 and ex fit (no spills); imex2 and im spill 6 and 2 registers and still
  // gain (config 2: 90.5 -> 81.8 and 86.9 -> 80.4 us); the LinOSS backward, which
  // holds every s_{t-1} it reads, spills 75 and keeps 16 x 8.
  static const Tile env_tile = parse_tile("OSSM_OSC_TILE_BWD", Tile{0, 0, 0, 1, 1});
  const int64_t wgs256 = (L + 255) / 256 * ((nc + kWave - 1) / kWave);
  return env_tile.T > 0 ? env_tile
         : recompute && wgs256 >= 128 && wgs256 < 2048 ? Tile{16, 16, 1, 1, 2}
                                                        : Tile{16, 8, 1, 1, 2};
}

// Backward launch: one kernel.  It computes grad_in; its order-0 workgroup
// zeroes the arrays `zero` names and every workgroup hands its chunk's
// per-channel sums to Model::epilogue (D-LinOSS, selective D-LinOSS with
// constant parameters: the chain rule applied to the chunk's share, one float
// atomic per output and channel; LinOSS: the whole wave's shares at once,
// Model::epilogue_wave).  A column-sum launch after the scan cost 4.4 us plus
// the launch gap at config 2, where the scan takes ~73 us.  nc = B * P
// channels.
template <class Model>
int launch_backward(const typename Model::Params& prm, const void* in, const void* states,
                    const void* gout, void* gin, const ZeroFill& zero, int64_t L, int64_t B,
                    int64_t P, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const int64_t nc = B * P;
  const Tile tile = bwd_tile(L, nc, Model::kRecompute);
  const int64_t CL = int64_t(tile.T) * tile.W;
  const int64_t n_chunks = (L + CL - 1) / CL;
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  if (n_chunks * n_groups > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  const size_t rec_bytes = static_cast<size_t>(n_chunks) * 2 * 4 * nc * sizeof(unsigned long long);
  const int64_t total = n_chunks * n_groups;
  LaunchTiming tm;
  if (int rc = take_launch_timing(call, &tm)) return rc;
  void* payload = nullptr;
  LaunchSync sync{};
  if (int rc = acquire_scratch(call, rec_bytes, total, &payload, &sync)) return rc;
  const dim3 grid(static_cast<unsigned>(total));
  bool launched = false;
#define OSSM_BWD_ARGS                                                                            \
  prm, static_cast<const typename Model::In*>(in), static_cast<const float4*>(states),           \
      static_cast<const typename Model::GIn*>(gout), static_cast<typename Model::GOut*>(gin),    \
      zero, static_cast<int>(L), static_cast<int>(nc), static_cast<int>(n_groups),               \
      static_cast<int>(n_chunks), static_cast<unsigned long long*>(payload), sync
#define OSSM_LAUNCH_BWD(TT, WW, OO, HH, SS)                                                      \
  if (!launched && tile.T == TT && tile.W == WW && tile.O == OO && tile.H == HH &&               \
      tile.S == SS) {                                                                            \
    if (tm.start != nullptr)                                                                     \
      hipExtLaunchKernelGGL((osc_backward_kernel<Model, TT, WW, OO, HH, SS>), grid,              \
                            dim3(WW * kWave), 0, stream, tm.start, tm.stop, 0, OSSM_BWD_ARGS);   \
    else                                                                                         \
      hipLaunchKernelGGL((osc_backward_kernel<Model, TT, WW, OO, HH, SS>), grid,                 \
                         dim3(WW * kWave), 0, stream, OSSM_BWD_ARGS);                            \
    if (int rc = launch_check("osc_backward_kernel")) return rc;                                 \
    launched = true;                                                                             \
  }
  OSSM_BWD_TILES(OSSM_LAUNCH_BWD)
#undef OSSM_LAUNCH_BWD
#undef OSSM_BWD_ARGS
  if (!launched) return set_error(OSSM_ERR_UNSUPPORTED, "OSSM_OSC_TILE_BWD names no built tile");
  return OSSM_OK;
}

int check_sizes(int64_t L, int64_t B, int64_t P, const char* what) {
  if (L < 0 || B < 0 || P < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (L > INT_MAX || B * P > INT_MAX / 2 || P > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  return OSSM_OK;
}

template <int V>
int dlinoss_forward_v(const float* a, const float* g, const float* dt, const void* bu, void* states,
                      int64_t L, int64_t B, int64_t P, hipStream_t stream) {
  typename Dlinoss<V>::Params prm{a, g, dt, static_cast<int>(P)};
  return launch_forward<Dlinoss<V>>(prm, bu, states, L, B * P, stream);
}

template <int V>
int dlinoss_backward_v(const float* a, const float* g, const float* dt, const void* bu,
                       const void* states, const void* gout, float* ga, float* gg, float* gs,
                       void* gbu, int64_t L, int64_t B, int64_t P, hipStream_t stream) {
  typename Dlinoss<V>::Params prm{a, g, dt, static_cast<int>(P)};
  const int n = static_cast<int>(Dlinoss<V>::kOutsPerColumn * P);
  return launch_backward<Dlinoss<V>>(prm, bu, states, gout, gbu, ZeroFill{{ga, gg, gs}, {n, n, n}},
                                     L, B, P, stream);
}

template <int V>
int sdl_tb_forward_v(const SdlParams& v, const void* bu, void* states, int64_t L, int64_t nc,
                     hipStream_t stream) {
  const typename SdlTb<V>::Params prm{v, v.M, static_cast<int>(nc)};
  return launch_forward<SdlTb<V>>(prm, bu, states, L, nc, stream);
}

template <int V>
int sdl_tb_backward_v(const SdlParams& v, const void* bu, const void* states, const void* gout,
                      void* gbu, float* const (&grads)[3], int64_t L, int64_t nc, hipStream_t stream) {
  const typename SdlTb<V>::Params prm{v, v.M, static_cast<int>(nc)};
  // zeroed by the launch's order-0 workgroup before any chunk adds its share
  auto n_of = [&](const ParamView& pv) { return static_cast<int>(pv.by_channel ? nc : v.M); };
  return launch_backward<SdlTb<V>>(prm, bu, states, gout, gbu,
                                   ZeroFill{{grads[0], grads[1], grads[2]}, {n_of(v.a), n_of(v.g), n_of(v.s)}},
                                   L, nc / v.M, v.M, stream);
}

}  // namespace


int sdl_tb_forward(int variant, const SdlParams& prm, const void* bu, void* states, int64_t L,
                   int64_t nc, hipStream_t stream) {
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return sdl_tb_forward_v<OSSM_DLINOSS_IMEX1>(prm, bu, states, L, nc, stream);
    case OSSM_DLINOSS_IMEX2: return sdl_tb_forward_v<OSSM_DLINOSS_IMEX2>(prm, bu, states, L, nc, stream);
    case OSSM_DLINOSS_IM: return sdl_tb_forward_v<OSSM_DLINOSS_IM>(prm, bu, states, L, nc, stream);
    default: return sdl_tb_forward_v<OSSM_DLINOSS_EX>(prm, bu, states, L, nc, stream);
  }
}

int sdl_tb_backward(int variant, const SdlParams& prm, const void* bu, const void* states,
                    const void* gout, void* gbu, float* const (&grads)[3], int64_t L, int64_t nc,
                    hipStream_t stream) {
  switch (variant) {
    case OSSM_DLINOSS_IMEX1:
      return sdl_tb_backward_v<OSSM_DLINOSS_IMEX1>(prm, bu, states, gout, gbu, grads, L, nc, stream);
    case OSSM_DLINOSS_IMEX2:
      return sdl_tb_backward_v<OSSM_DLINOSS_IMEX2>(prm, bu, states, gout, gbu, grads, L, nc, stream);
    case OSSM_DLINOSS_IM:
      return sdl_tb_backward_v<OSSM_DLINOSS_IM>(prm, bu, states, gout, gbu, grads, L, nc, stream);
    default:
      return sdl_tb_backward_v<OSSM_DLINOSS_EX>(prm, bu, states, gout, gbu, grads, L, nc, stream);
  }
}

// ---- allocation-free D-LinOSS forward ------------------------------------------
// ossm_dlinoss_forward_noalloc keeps its look-back records in this array: a
// 256-byte header (the launch-ticket counter at kHdrTicket, the error bits at
// kHdrErr) and kNoAllocRecordBytes of tagged records.  Device memory is
// zero at load, which is the state the protocol starts from (tag 0 is never a
// launch's tag, and a launch starts with the ticket counter at a multiple of
// 2^32).  The launch's order and tag come from that counter on the device,
// so the call can be captured into a HIP graph and replayed.  Each GPU
// holds its own copy until the process ends; its address on a device comes
// from hipGetSymbolAddress, taken once per device on that device's first
// call.  The array is per process and per GPU: every call of this process on
// a GPU shares that GPU's copy (another process has a copy of its own).
// Records are tagged per launch, so nothing needs clearing between calls, but
// calls of this process that overlap on one GPU (several streams or threads)
// race.
constexpr size_t kNoAllocRecordBytes = size_t(16) << 20;
// 64 bytes of records per channel and 128-step chunk: half a byte per state-step.
constexpr int64_t kNoAllocStateSteps = int64_t(kNoAllocRecordBytes) * 2;
static __device__ __align__(256) unsigned char scratch[kHdrBytes + kNoAllocRecordBytes];

constexpr int kNoAllocMaxDevices = 64;
struct NoAllocDevice {
  std::mutex mu;                        // held from bookkeeping through the launch
  char* ptr = nullptr;                  // device address of `scratch` on this device
  unsigned int epoch = 0;               // counter of the dispatch-order tags (next_dispatch_tag)
};
NoAllocDevice g_noalloc[kNoAllocMaxDevices];

// The address of `scratch` on device `dev` (current), looked up once.
// Called with g_noalloc[dev].mu held.
int noalloc_address(int dev) {
  NoAllocDevice& s = g_noalloc[dev];
  if (s.ptr != nullptr) return OSSM_OK;
  void* p = nullptr;
  if (int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
    return rc;
  s.ptr = static_cast<char*>(p);
  return OSSM_OK;
}

uint32_t noalloc_error_bits(int dev) {
  if (dev < 0 || dev >= kNoAllocMaxDevices) return 0;
  NoAllocDevice& s = g_noalloc[dev];
  std::lock_guard<std::mutex> hold(s.mu);
  if (s.ptr == nullptr) return 0;  // the allocation-free path never ran here
  // the array is shared by every stream of the device: drain them all
  if (hipDeviceSynchronize() != hipSuccess) return 0xffffffffu;
  uint32_t bits = 0;
  unsigned long long t = 0;
  if (hipMemcpy(&bits, s.ptr + kHdrErr, sizeof(bits), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&t, s.ptr + kHdrTicket, sizeof(t), hipMemcpyDeviceToHost) != hipSuccess)
    return 0xffffffffu;
  if ((t & (kEpochSpan - 1)) != 0) {  // a launch that did not run to its end: realign
    t = (t | (kEpochSpan - 1)) + 1;
    (void)hipMemcpy(s.ptr + kHdrTicket, &t, sizeof(t), hipMemcpyHostToDevice);
  }
  if (bits != 0) {
    const uint32_t zero = 0;
    (void)hipMemcpy(s.ptr + kHdrErr, &zero, sizeof(zero), hipMemcpyHostToDevice);
  }
  return bits;
}

namespace {

template <int V>
int dlinoss_forward_noalloc_v(const FwdPlan& pl, const float* a, const float* g, const float* dt,
                              const void* bu, void* states, int64_t L, int64_t B, int64_t P,
                              hipStream_t stream, void* payload, const LaunchSync& sync) {
  typename Dlinoss<V>::Params prm{a, g, dt, static_cast<int>(P)};
  return enqueue_forward<Dlinoss<V>>(pl, prm, bu, states, L, B * P, stream, payload, sync);
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_dlinoss_forward_noalloc(int variant, const float* a_diag, const float* g_diag,
                                 const float* step, const void* bu, void* states, int64_t length,
                                 int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sizes(length, batch, ssm, "dlinoss_forward_noalloc")) return rc;
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!a_diag || !g_diag || !step || !bu || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_forward_noalloc: null pointer");
  if (variant < OSSM_DLINOSS_IMEX1 || variant > OSSM_DLINOSS_EX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  // Always 128-step chunks (16 x 8), whatever ossm_dlinoss_forward would pick,
  // so that the records take the half byte per state-step the limit is stated in.
  const FwdPlan pl = fwd_plan_with(length, batch * ssm, Tile{16, 8, 1, 1, 1});
  if (pl.total > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "problem too large for one launch grid");
  if (length * batch * ssm > kNoAllocStateSteps || pl.rec_bytes > kNoAllocRecordBytes)
    return set_error(OSSM_ERR_UNSUPPORTED,
                     "dlinoss_forward_noalloc: " + std::to_string(length * batch * ssm) +
                         " state-steps need " + std::to_string(pl.rec_bytes) +
                         " bytes of look-back records; the fixed " +
                         std::to_string(kNoAllocRecordBytes) +
                         "-byte scratch serves at most 33,554,432 state-steps per call (half a "
                         "byte each); use ossm_dlinoss_forward");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev >= kNoAllocMaxDevices)
    return set_error(OSSM_ERR_UNSUPPORTED, "dlinoss_forward_noalloc: device index above 63");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const hipError_t ce = hipStreamIsCapturing(stream, &cap);
  if (ce != hipSuccess) {
    (void)hipGetLastError();
    return set_error(OSSM_ERR_HIP, std::string("hipStreamIsCapturing: ") + hipGetErrorString(ce));
  }
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (capturing && cap != hipStreamCaptureStatusActive)
    return set_error(OSSM_ERR_UNSUPPORTED,
                     "dlinoss_forward_noalloc: the stream's graph capture was invalidated");
  bool by_ticket = true;
  if (int rc = choose_scan_order(dev, capturing, pl.total, &by_ticket)) return rc;
  NoAllocDevice& s = g_noalloc[dev];
  std::lock_guard<std::mutex> hold(s.mu);
  if (capturing && s.ptr == nullptr)
    return set_error(OSSM_ERR_UNSUPPORTED,
                     "dlinoss_forward_noalloc: call it once eagerly on this device before capturing "
                     "it (the first call looks up the fixed array's address)");
  if (int rc = noalloc_address(dev)) return rc;
  LaunchSync sync{};
  sync.ticket = reinterpret_cast<unsigned long long*>(s.ptr + kHdrTicket);
  sync.err = reinterpret_cast<unsigned int*>(s.ptr + kHdrErr);
  sync.flag = reinterpret_cast<unsigned long long*>(s.ptr + kHdrFlag);
  sync.use_ticket = by_ticket ? 1 : 0;
  sync.poison = 0;
  sync.tag = by_ticket ? 0 : next_dispatch_tag(s.epoch);  // ticket order: drawn on the device
  void* payload = s.ptr + kHdrBytes;
  int rc = OSSM_OK;
  switch (variant) {
    case OSSM_DLINOSS_IMEX1:
      rc = dlinoss_forward_noalloc_v<OSSM_DLINOSS_IMEX1>(pl, a_diag, g_diag, step, bu, states, length, batch, ssm, stream, payload, sync);
      break;
    case OSSM_DLINOSS_IMEX2:
      rc = dlinoss_forward_noalloc_v<OSSM_DLINOSS_IMEX2>(pl, a_diag, g_diag, step, bu, states, length, batch, ssm, stream, payload, sync);
      break;
    case OSSM_DLINOSS_IM:
      rc = dlinoss_forward_noalloc_v<OSSM_DLINOSS_IM>(pl, a_diag, g_diag, step, bu, states, length, batch, ssm, stream, payload, sync);
      break;
    default:
      rc = dlinoss_forward_noalloc_v<OSSM_DLINOSS_EX>(pl, a_diag, g_diag, step, bu, states, length, batch, ssm, stream, payload, sync);
      break;
  }
  return rc;
}

int ossm_dlinoss_forward(int variant, const float* a_diag, const float* g_diag, const float* step,
                         const void* bu, void* states, int64_t length, int64_t batch, int64_t ssm,
                         ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sizes(length, batch, ssm, "dlinoss_forward")) return rc;
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!a_diag || !g_diag || !step || !bu || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_forward: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  switch (variant) {
    case OSSM_DLINOSS_IMEX1:
      return dlinoss_forward_v<OSSM_DLINOSS_IMEX1>(a_diag, g_diag, step, bu, states, length, batch, ssm, stream);
    case OSSM_DLINOSS_IMEX2:
      return dlinoss_forward_v<OSSM_DLINOSS_IMEX2>(a_diag, g_diag, step, bu, states, length, batch, ssm, stream);
    case OSSM_DLINOSS_IM:
      return dlinoss_forward_v<OSSM_DLINOSS_IM>(a_diag, g_diag, step, bu, states, length, batch, ssm, stream);
    case OSSM_DLINOSS_EX:
      return dlinoss_forward_v<OSSM_DLINOSS_EX>(a_diag, g_diag, step, bu, states, length, batch, ssm, stream);
    default:
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  }
}

int ossm_dlinoss_backward(int variant, const float* a_diag, const float* g_diag, const float* step,
                          const void* bu, const void* states, const void* grad_output,
                          float* grad_a, float* grad_g, float* grad_step, void* grad_bu,
                          int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sizes(length, batch, ssm, "dlinoss_backward")) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  if (ssm > 0 && (length == 0 || batch == 0)) {
    // reference: zero gradients when there is nothing to scan (dlinoss_imex1.cpp:366-375)
    if (!grad_a || !grad_g || !grad_step)
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_backward: null pointer");
    for (float* p : {grad_a, grad_g, grad_step})
      if (int rc = fill_zero(p, ssm, stream)) return rc;
    return OSSM_OK;
  }
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!a_diag || !g_diag || !step || !bu || !states || !grad_output || !grad_a || !grad_g ||
      !grad_step || !grad_bu)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_backward: null pointer");
  switch (variant) {
#define OSSM_BWD_CASE(V)                                                                       \
  case V:                                                                                      \
    return dlinoss_backward_v<V>(a_diag, g_diag, step, bu, states, grad_output, grad_a, grad_g, \
                                 grad_step, grad_bu, length, batch, ssm, stream);
    OSSM_BWD_CASE(OSSM_DLINOSS_IMEX1)
    OSSM_BWD_CASE(OSSM_DLINOSS_IMEX2)
    OSSM_BWD_CASE(OSSM_DLINOSS_IM)
    OSSM_BWD_CASE(OSSM_DLINOSS_EX)
#undef OSSM_BWD_CASE
    default:
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  }
}

int ossm_linoss_forward(const void* m11, const void* m12, const void* m21, const void* m22,
                        const void* b_seq, void* states, int64_t length, int64_t batch, int64_t ssm,
                        ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sizes(length, batch, ssm, "linoss_forward")) return rc;
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!m11 || !m12 || !m21 || !m22 || !b_seq || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_forward: null pointer");
  Linoss::Params prm{static_cast<const float2*>(m11), static_cast<const float2*>(m12),
                     static_cast<const float2*>(m21), static_cast<const float2*>(m22),
                     static_cast<int>(ssm), static_cast<int>(batch * ssm)};
  return launch_forward<Linoss>(prm, b_seq, states, length, batch * ssm,
                                static_cast<hipStream_t>(stream_v));
}

int ossm_linoss_backward(const void* m11, const void* m12, const void* m21, const void* m22,
                         const void* states, const void* grad_output, void* grad_m, void* grad_b,
                         int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_sizes(length, batch, ssm, "linoss_backward")) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  if (ssm > 0 && (length == 0 || batch == 0)) {
    if (!grad_m) return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_backward: null pointer");
    return fill_zero(static_cast<float*>(grad_m), 8 * ssm, stream);
  }
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!m11 || !m12 || !m21 || !m22 || !states || !grad_output || !grad_m || !grad_b)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_backward: null pointer");
  Linoss::Params prm{static_cast<const float2*>(m11), static_cast<const float2*>(m12),
                     static_cast<const float2*>(m21), static_cast<const float2*>(m22),
                     static_cast<int>(ssm), static_cast<int>(batch * ssm)};
  const int n = static_cast<int>(Linoss::kOutsPerColumn * ssm);
  return launch_backward<Linoss>(prm, nullptr, states, grad_output, grad_b,
                                 ZeroFill{{static_cast<float*>(grad_m), nullptr, nullptr}, {n, 0, 0}},
                                 length, batch, ssm, stream);
}

}  // extern "C"
