// Device helpers for the chunked linear-recurrence scans on gfx950:
// 2x2 transition algebra on complex 2-vectors, and the decoupled look-back
// protocol that hands chunk carries from one workgroup to the next.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "runtime.hpp"

namespace ossm {

constexpr int kWave = 64;

// A state is a complex 2-vector packed as float4 (s0.re, s0.im, s1.re, s1.im),
// the [.., 2] complex64 layout of the reference's states tensors.
__device__ __forceinline__ float4 f4add(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 f4zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
// The carry of a chunk whose predecessors could not be read (a bounded wait
// that gave up, an out-of-range ticket): NaN, so that every output computed
// from it is NaN rather than a plausible wrong value.
__device__ __forceinline__ float4 f4nan() {
  const float q = __builtin_nanf("");
  return make_float4(q, q, q, q);
}

// ---- real 2x2 transition [[a, b], [c, d]] (D-LinOSS) -----------------------
struct RMat {
  float a, b, c, d;
};
__device__ __forceinline__ RMat mat_identity(RMat) { return {1.f, 0.f, 0.f, 1.f}; }
__device__ __forceinline__ RMat mat_mul(RMat p, RMat q) {
  return {p.a * q.a + p.b * q.c, p.a * q.b + p.b * q.d, p.c * q.a + p.d * q.c,
          p.c * q.b + p.d * q.d};
}
__device__ __forceinline__ RMat mat_adjoint(RMat p) { return {p.a, p.c, p.b, p.d}; }
__device__ __forceinline__ float4 mat_apply(RMat m, float4 s) {
  return make_float4(m.a * s.x + m.b * s.z, m.a * s.y + m.b * s.w, m.c * s.x + m.d * s.z,
                     m.c * s.y + m.d * s.w);
}

// ---- complex 2x2 transition (LinOSS) ----------------------------------------
struct CMat {
  float2 a, b, c, d;
};
__device__ __forceinline__ float2 cmul(float2 p, float2 q) {
  return make_float2(p.x * q.x - p.y * q.y, p.x * q.y + p.y * q.x);
}
__device__ __forceinline__ float2 cadd(float2 p, float2 q) { return make_float2(p.x + q.x, p.y + q.y); }
__device__ __forceinline__ float2 cconj(float2 p) { return make_float2(p.x, -p.y); }
__device__ __forceinline__ CMat mat_identity(CMat) {
  return {make_float2(1.f, 0.f), make_float2(0.f, 0.f), make_float2(0.f, 0.f), make_float2(1.f, 0.f)};
}
__device__ __forceinline__ CMat mat_mul(CMat p, CMat q) {
  return {cadd(cmul(p.a, q.a), cmul(p.b, q.c)), cadd(cmul(p.a, q.b), cmul(p.b, q.d)),
          cadd(cmul(p.c, q.a), cmul(p.d, q.c)), cadd(cmul(p.c, q.b), cmul(p.d, q.d))};
}
__device__ __forceinline__ CMat mat_adjoint(CMat p) {  // conjugate transpose
  return {cconj(p.a), cconj(p.c), cconj(p.b), cconj(p.d)};
}
__device__ __forceinline__ float4 mat_apply(CMat m, float4 s) {
  const float2 s0 = make_float2(s.x, s.y), s1 = make_float2(s.z, s.w);
  const float2 n0 = cadd(cmul(m.a, s0), cmul(m.b, s1));
  const float2 n1 = cadd(cmul(m.c, s0), cmul(m.d, s1));
  return make_float4(n0.x, n0.y, n1.x, n1.y);
}

// ---- fp64 twins, used only to raise a transition to a power ------------------
// A chunk transition M^n composed in fp32 by repeated squaring loses ~log2(n)
// roundings per entry, and non-normal M (LinOSS) amplifies that through
// cancellation.  The powers are computed once per lane, so they are formed in
// fp64 and rounded to fp32 once.
struct RMatD {
  double a, b, c, d;
};
struct CMatD {
  double ar, ai, br, bi, cr, ci, dr, di;
};
__device__ __forceinline__ RMatD widen(RMat m) { return {m.a, m.b, m.c, m.d}; }
__device__ __forceinline__ RMat narrow(RMatD m) {
  return {static_cast<float>(m.a), static_cast<float>(m.b), static_cast<float>(m.c),
          static_cast<float>(m.d)};
}
__device__ __forceinline__ RMatD mat_identity(RMatD) { return {1.0, 0.0, 0.0, 1.0}; }
__device__ __forceinline__ RMatD mat_mul(RMatD p, RMatD q) {
  return {p.a * q.a + p.b * q.c, p.a * q.b + p.b * q.d, p.c * q.a + p.d * q.c,
          p.c * q.b + p.d * q.d};
}
__device__ __forceinline__ CMatD widen(CMat m) {
  return {m.a.x, m.a.y, m.b.x, m.b.y, m.c.x, m.c.y, m.d.x, m.d.y};
}
__device__ __forceinline__ CMat narrow(CMatD m) {
  return {make_float2(static_cast<float>(m.ar), static_cast<float>(m.ai)),
          make_float2(static_cast<float>(m.br), static_cast<float>(m.bi)),
          make_float2(static_cast<float>(m.cr), static_cast<float>(m.ci)),
          make_float2(static_cast<float>(m.dr), static_cast<float>(m.di))};
}
__device__ __forceinline__ CMatD mat_identity(CMatD) { return {1, 0, 0, 0, 0, 0, 1, 0}; }
__device__ __forceinline__ CMatD mat_mul(CMatD p, CMatD q) {
  // (p q)_ij = sum_k p_ik q_kj with complex entries a b / c d
  CMatD r;
  r.ar = p.ar * q.ar - p.ai * q.ai + p.br * q.cr - p.bi * q.ci;
  r.ai = p.ar * q.ai + p.ai * q.ar + p.br * q.ci + p.bi * q.cr;
  r.br = p.ar * q.br - p.ai * q.bi + p.br * q.dr - p.bi * q.di;
  r.bi = p.ar * q.bi + p.ai * q.br + p.br * q.di + p.bi * q.dr;
  r.cr = p.cr * q.ar - p.ci * q.ai + p.dr * q.cr - p.di * q.ci;
  r.ci = p.cr * q.ai + p.ci * q.ar + p.dr * q.ci + p.di * q.cr;
  r.dr = p.cr * q.br - p.ci * q.bi + p.dr * q.dr - p.di * q.di;
  r.di = p.cr * q.bi + p.ci * q.br + p.dr * q.di + p.di * q.dr;
  return r;
}

// m^n for n >= 1 by binary powering in fp64, rounded to fp32 once.
template <class Mat>
__device__ __forceinline__ Mat mat_pow(Mat m, int n) {
  auto b = widen(m);
  auto r = mat_identity(b);
  while (n > 0) {
    if (n & 1) r = mat_mul(r, b);
    n >>= 1;
    if (n) b = mat_mul(b, b);
  }
  return narrow(r);
}

// ---- decoupled look-back ----------------------------------------------------
//
// Each (chunk, channel) owns two records, an aggregate (the chunk's effect on
// a zero carry) and an inclusive prefix (the true state at the chunk's end),
// each four 64-bit words: high half = launch tag, low half = float bits.  A
// word is written once per launch with one 64-bit atomic store, so a reader
// that sees this launch's tag in all four words has the complete value; no
// fence, flag or clearing pass is needed, and records of earlier launches
// (older tags) are simply not ready.
//
// Records layout: rec[((chunk * 2 + kind) * 4 + k) * nc + ch], kind 0 =
// aggregate, 1 = inclusive.  Lanes of a wave touch consecutive channels, so
// every record access is one coalesced 512-byte row per word.
constexpr int kRecAgg = 0;
constexpr int kRecInc = 1;
constexpr uint32_t kSpinLimit = 1u << 22;  // ~ a few hundred ms of polling

__device__ __forceinline__ size_t rec_index(int chunk, int kind, int k, int nc, int ch) {
  return ((size_t(chunk) * 2 + kind) * 4 + k) * size_t(nc) + ch;
}

__device__ __forceinline__ void rec_publish(unsigned long long* rec, int chunk, int kind,
                                            int nc, int ch, float4 v, unsigned int tag) {
  const unsigned long long t = static_cast<unsigned long long>(tag) << 32;
  const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const unsigned long long w = t | __float_as_uint(vals[k]);
    __hip_atomic_store(rec + rec_index(chunk, kind, k, nc, ch), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Loads the four words of one record without waiting for them.
__device__ __forceinline__ void rec_fetch(const unsigned long long* rec, int chunk, int kind, int nc,
                                          int ch, unsigned long long (&w)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = __hip_atomic_load(rec + rec_index(chunk, kind, k, nc, ch), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Whether all four words carry this launch's tag; the value in *v.
__device__ __forceinline__ bool rec_decode(const unsigned long long (&w)[4], unsigned int tag,
                                           float4* v) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < 4; ++k) ok = ok && (static_cast<unsigned int>(w[k] >> 32) == tag);
  *v = make_float4(__uint_as_float(static_cast<unsigned int>(w[0])),
                   __uint_as_float(static_cast<unsigned int>(w[1])),
                   __uint_as_float(static_cast<unsigned int>(w[2])),
                   __uint_as_float(static_cast<unsigned int>(w[3])));
  return ok;
}

// Predecessor records fetched per round trip of the look-back.  Records live
// in memory shared by all XCDs, so each read is a full memory round trip;
// fetching both records of kLookbackWindow predecessors at once turns a walk
// over k chunks from 2k round trips into about k / kLookbackWindow.
#ifndef OSSM_LOOKBACK_WINDOW
#define OSSM_LOOKBACK_WINDOW 1
#endif
constexpr int kLookbackWindow = OSSM_LOOKBACK_WINDOW;

// Carry into chunk `c` for one channel: walks predecessors c - dir, c - 2 dir,
// ... (dir = +1 forward in time, -1 for reverse scans), composing aggregates
// with `step_mat` (the chunk transition) until an inclusive prefix is found.
// Every predecessor drew an earlier ticket, so it is resident and publishes
// its aggregate without waiting on anything: the walk always ends.  The spin
// is still bounded; giving up raises kErrSpinTimeout and returns a NaN carry
// instead of hanging.  A poisoned launch (out-of-range ticket) returns NaN
// without walking.
template <class Mat>
__device__ float4 lookback(unsigned long long* rec, int c, int dir, int n_chunks, int nc, int ch,
                           Mat step_mat, const LaunchSync& sync) {
  constexpr int K = kLookbackWindow;
  if (sync.poison) return f4nan();
  float4 acc = f4zero();
  Mat pw = mat_identity(step_mat);
  int j = c - dir;  // next predecessor to fold in
  uint32_t spins = 0;
  while (j >= 0 && j < n_chunks) {
    unsigned long long wi[K][4], wa[K][4];
#pragma unroll
    for (int q = 0; q < K; ++q) {
      const int jj = min(max(j - q * dir, 0), n_chunks - 1);  // in range; unused past the end
      rec_fetch(rec, jj, kRecInc, nc, ch, wi[q]);
      rec_fetch(rec, jj, kRecAgg, nc, ch, wa[q]);
    }
    bool moved = false, done = false;
#pragma unroll
    for (int q = 0; q < K; ++q) {
      if (done || !(j >= 0 && j < n_chunks)) break;
      float4 v;
      if (rec_decode(wi[q], sync.tag, &v)) {
        acc = f4add(acc, mat_apply(pw, v));
        done = true;
      } else if (rec_decode(wa[q], sync.tag, &v)) {
        acc = f4add(acc, mat_apply(pw, v));
        pw = mat_mul(pw, step_mat);
        j -= dir;
        moved = true;
      } else {
        break;  // not published yet: fetch again from j
      }
    }
    if (done) return acc;
    if (!moved) {
      if (++spins > kSpinLimit) {
        __hip_atomic_fetch_or(sync.err, kErrSpinTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return f4nan();
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  return acc;
}

// The order in which this workgroup's chunk is scheduled.  A chunk only waits
// on chunks of smaller order, so if the workgroup of the smallest unfinished
// order is always resident, every look-back ends.
//
// Ticket order (default, sync.use_ticket): a global atomic counter drawn at
// workgroup start guarantees that under any dispatch order, at the price of
// one serialised atomic per workgroup (~10 us per 2048 workgroups measured
// on a streaming kernel of the same shape).  The ticket also gives the
// launch's record tag (see LaunchSync), written into sync.tag.
//
// Dispatch order (sync.use_ticket == 0, which the host chooses for grids of at
// most a quarter as many workgroups as CUs; see choose_scan_order): the
// workgroup index, no atomic.  On an idle device such a grid is resident at
// once, so nothing waits on a chunk that is not running.  Otherwise (other
// work on the device, or a larger grid under OSSM_SCAN_ORDER=dispatch) it
// relies on each XCD dispatching its share of the grid in increasing index
// order, and a wait that still outlasts the bounded spin gives NaN carries
// and an error bit.
//
// A ticket whose order is out of range means the counter was out of step
// (a launch on this scratch that did not run to its end): the workgroup
// raises kErrBadTicket, takes order (rel mod total) — the orders a
// misaligned launch never draws are exactly those the out-of-range tickets
// map to — and marks the launch poisoned, so its look-backs return NaN and
// every output that depends on a carry is NaN.
// One ticket draw by the calling thread: the chunk order it gives, the
// launch's record tag in *tag and, for an out-of-range ticket (see
// launch_order), 1 in *poison.  The draw of the launch's last order moves the
// counter to the next epoch.
__device__ __forceinline__ int draw_ticket(const LaunchSync& sync, int total, unsigned int* tag,
                                           int* poison) {
  const unsigned long long t =
      __hip_atomic_fetch_add(sync.ticket, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned long long rel = t & (kEpochSpan - 1);
  const unsigned long long epoch = t >> 32;
  *poison = 0;
  if (rel >= static_cast<unsigned long long>(total)) {
    __hip_atomic_fetch_or(sync.err, kErrBadTicket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    rel %= static_cast<unsigned long long>(total);
    *poison = 1;
  } else if (rel == static_cast<unsigned long long>(total - 1)) {
    // the launch's last ticket: the next launch starts at the next epoch
    __hip_atomic_fetch_add(sync.ticket, kEpochSpan - static_cast<unsigned long long>(total),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // 1 .. 2^31 - 1: never 0 (never-written memory) nor a dispatch-order tag
  *tag = static_cast<unsigned int>(epoch % (kDispatchTagBase - 1u)) + 1u;
  return static_cast<int>(rel);
}

__device__ __forceinline__ int launch_order(LaunchSync& sync, int total, int* s_slot) {
  if (!sync.use_ticket) return static_cast<int>(blockIdx.x);
  __shared__ unsigned int s_tag;
  __shared__ int s_poison;
  if (threadIdx.x == 0) {
    unsigned int tag = 0;
    int poison = 0;
    *s_slot = draw_ticket(sync, total, &tag, &poison);
    s_tag = tag;
    s_poison = poison;
  }
  __syncthreads();
  // uniform across the workgroup: keep them (and what derives from them) scalar
  sync.tag = __builtin_amdgcn_readfirstlane(s_tag);
  sync.poison = __builtin_amdgcn_readfirstlane(s_poison);
  return __builtin_amdgcn_readfirstlane(*s_slot);
}

// Index of the calling wave in its workgroup, as a scalar value.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
}

// Row t of a [L, nc] tensor, from the first channel of channel group g.  t,
// nc and g are uniform across the wave, so the pointer is a scalar and each
// lane adds only its 32-bit lane offset.
template <class E>
__device__ __forceinline__ E* group_row(E* base, long long t, int nc, int g) {
  return base + static_cast<size_t>(t) * nc + static_cast<size_t>(g) * kWave;
}

// Store of a streamed output (written once, read by a later launch) with the
// non-temporal hint, so it does not displace lines this launch still reads
// from the caches.  E is a float vector type (float, float2, float4) or a
// struct of floats of the same size.  Measured at config 2's shape: the
// D-LinOSS forward 79.8 -> 66.0 us, its backward 93.4 -> 89.5 us.
template <class E>
__device__ __forceinline__ void stream_store(E* p, const E& v) {
  static_assert(sizeof(E) % 4 == 0 && sizeof(E) <= 16, "float vector of 1-4 lanes");
  typedef float V __attribute__((ext_vector_type(sizeof(E) / 4)));
  V bits;
  __builtin_memcpy(&bits, &v, sizeof(E));
  __builtin_nontemporal_store(bits, reinterpret_cast<V*>(p));
}

// The lane's offset within its group, clamped onto the group's last channel
// for lanes past the end (their loads stay in bounds; results are unused).
__device__ __forceinline__ unsigned clamped_lane(int g, int nc) {
  return static_cast<unsigned>(min(static_cast<int>(threadIdx.x & (kWave - 1)), nc - 1 - g * kWave));
}

}  // namespace ossm
