// Selective (Mamba-style) scan on gfx950, forward and backward, fp32.
//
//   h_t[n] = exp(dt_t A[d,n]) h_{t-1}[n] + dt_t B_t[n] u_t,   y_t = sum_n C_t[n] h_t[n],
//   out_t  = y_t * silu(z_t)   (out = y without a gate)
// per (batch b, channel d), tensors u, dt, z, out [B,D,L]; A [D,N]; B, C [B,L,N].
//
// Parallel decomposition
//   A workgroup owns one batch row b and 64 (forward: 64 or 32) consecutive
//   channels d and walks the sequence (or one time segment of it); up to 16
//   states run per launch ("pass"), 4 (forward: 4 or 2) per lane in
//   registers; larger N runs ceil(N/16) passes that accumulate y (forward) and
//   du/ddt (backward) in the output tensors.  Time is processed in tiles
//   staged through LDS: u, dt (and the gated upstream gradient) are loaded with
//   coalesced row reads and read back per channel.
//   Forward: lane = (channel, state group) with 4 states per lane (16
//   channels per wave, 64 per workgroup) or, when that leaves the SIMDs short
//   of waves, 2 (8 channels per wave, 32 per workgroup); a wave holds all 16
//   states of its channels and y is summed over the states inside the wave
//   (cross-row swaps and DPP), with no LDS round trip.
//   Backward: lane = channel and wave w carries states 4w .. 4w + 3, so the
//   sums over channels (dB, dC) finish inside a wave and the sums over states
//   (du, ddt) across the waves through LDS; or, when 64-channel workgroups
//   would leave the device short of them, 32 channels per workgroup with 2
//   states per lane (selective_bwd2_kernel: half the registers, three
//   workgroups per CU instead of two).
//
// Transcendentals: exp(dt A) = exp2(dt * (A log2 e)) with A log2 e formed once
//   per lane, so each state-step costs one v_exp_f32.
//
// Checkpoints (chunk_states [B, D, n_chunks, 2N], n_chunks = ceil(L/32)):
//   row c holds h after step 32c+15 (first N) and after step 32c+31 (last N);
//   a checkpoint past the end holds h after the last step.  The backward
//   restarts every 16-step tile from the checkpoint before it, so it re-runs
//   the forward recurrence for one tile in registers instead of reading a
//   stored trajectory.
//
// Backward (reverse time, 16-step tiles)
//   gacc_t = gy_t C_t + exp(dt_{t+1} A) gacc_{t+1},   gy = gout * silu(z)
//   du_t  = dt_t sum_n gacc B_t,   ddt_t = sum_n gacc (A e^{dt A} h_{t-1} + B_t u_t)
//   dA    = sum_{b,t} gacc dt e^{dt A} h_{t-1},   dz = gout * y * silu'(z) (y = raw_out)
//   dB_t  = sum_d gacc dt u,   dC_t = sum_d gy h_t
// A tile is done in two 8-step halves, the later one first: the forward is
// re-run from the checkpoint over the whole tile once (the first half's
// trajectory kept for later, the second half's held while the adjoint runs
// over it in reverse).  The 2-states-per-lane kernel stages 32-step tiles and
// starts each 16-step half from its own checkpoint.
// Time split: with fewer (batch row, 64-channel) rows than twice the CUs the
// grid's z dimension cuts each row's tiles into 2 or 4 segments; a segment
// first carries the adjoint from the end of the sequence through the later
// segments' tiles (adjoint only: no recompute, no sums), with the main loop's
// per-step arithmetic, so the carry is bitwise the one the later segments
// reach.  The forward splits the same way when there are fewer rows than CUs,
// re-running h only over the earlier segments' tiles.
// dB/dC are sums over channels: each wave reduces its 64 lanes with the
// gfx950 cross-row swaps (v_permlane32_swap / v_permlane16_swap) and row DPP,
// and writes one partial per 64-channel tile; dA partials are per batch row.
// A finishing kernel adds the partials in a fixed order (deterministic).
//
// Reference semantics: selective_scan_cpu.cpp:78-166 (forward) and :168-360
// (backward); the drop-in entry points are selective_scan_cuda[_backward]
// (selective_scan_cuda.cu:253-393).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <climits>
#include <initializer_list>
#include <cstdint>
#include <string>
#include <type_traits>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"

namespace ossm {
namespace {

constexpr int kWave = 64;
constexpr int kNpw = 4;                      // states per lane
constexpr int kMaxWaves = 4;                 // waves per workgroup
constexpr int kPassStates = kNpw * kMaxWaves;  // states per launch
constexpr int kCkpt = 16;                    // checkpoint stride (steps)
constexpr int kChunk = 2 * kCkpt;            // chunk_states row = two checkpoints
constexpr int kFwdTile = 32;                 // forward LDS tile (steps)
constexpr int kBwdTile = kCkpt;              // backward LDS tile (steps)
constexpr float kLog2e = 1.4426950408889634f;
// Workgroups per compute unit the time split aims for (forward, backward).
#ifndef OSSM_SEL_FWD_WG_PER_CU
#define OSSM_SEL_FWD_WG_PER_CU 1
#endif
#ifndef OSSM_SEL_BWD_WG_PER_CU
#define OSSM_SEL_BWD_WG_PER_CU 2
#endif
constexpr int kFwdWgPerCu = OSSM_SEL_FWD_WG_PER_CU;
constexpr int kBwdWgPerCu = OSSM_SEL_BWD_WG_PER_CU;
constexpr int kBwd2WgPerCu = 3;  // the 2-states-per-lane backward

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 1 / (1 + e^-z) with the hardware reciprocal (1 ulp) instead of an IEEE
// division sequence: the gate is evaluated for every output element.
__device__ __forceinline__ float sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.f + fast_exp2(-z * kLog2e));
}

// Issue priority from the share of a workgroup's tiles still to run: waves of
// the workgroups sharing a SIMD are otherwise issued oldest first, so the
// first workgroup on a CU finishes well before the last and the CU's final
// stretch runs one or two waves per SIMD.  With the wave that is behind (more
// tiles left) ahead in the arbitration the workgroups resynchronise each time
// they cross a level: priority 3 while more than half the tiles are left, 2
// above a quarter, 1 above an eighth, 0 for the last eighth (finer at the end,
// where a lead turns into idle SIMD time).  remaining in 1..total.
__device__ __forceinline__ void balance_priority(int remaining, int total) {
  const int r8 = 8 * remaining;
  if (r8 > 4 * total) {
    __builtin_amdgcn_s_setprio(3);
  } else if (r8 > 2 * total) {
    __builtin_amdgcn_s_setprio(2);
  } else if (r8 > total) {
    __builtin_amdgcn_s_setprio(1);
  } else {
    __builtin_amdgcn_s_setprio(0);
  }
}

// ---- cross-lane helpers -------------------------------------------------------
// permlane32 swap: lanes 32..63 of a trade places with lanes 0..31 of b.
__device__ __forceinline__ void swap32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// permlane16 swap: odd 16-lane rows of a trade places with even rows of b.
__device__ __forceinline__ void swap16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
// Transposing stage between the two halves of each 16-lane row: the low half
// returns p + p of the lane 8 above, the high half q + q of the lane 8 below
// (each half keeps one value and sends the other: two selects and one
// row_ror:8 add).
__device__ __forceinline__ float transpose_ror8(float p, float q) {
  const bool hi = (threadIdx.x & 8) != 0;
  const float keep = hi ? q : p, send = hi ? p : q;
  return keep + dpp<0x128>(send);
}
// Sums v[0..7] over all 64 lanes; every lane of half-row k (lanes 8k..8k+7)
// receives the total of v[k].  Two transposing stages across rows
// (permlane32 / permlane16 swaps), a third between the two halves of each row
// (transpose_ror8), then an 8-lane all-reduce.
__device__ __forceinline__ float reduce8(const float (&v)[8]) {
  float a0 = v[0], a1 = v[1], a2 = v[2], a3 = v[3];
  float b0 = v[4], b1 = v[5], b2 = v[6], b3 = v[7];
  swap32(a0, b0);
  swap32(a1, b1);
  swap32(a2, b2);
  swap32(a3, b3);
  // lanes 0..31 now hold 2-lane sums of v0..v3, lanes 32..63 of v4..v7
  float s0 = a0 + b0, s1 = a1 + b1, s2 = a2 + b2, s3 = a3 + b3;
  swap16(s0, s2);
  swap16(s1, s3);
  // row r: p = 4-lane sums of v[2r], q of v[2r + 1]
  const float p = s0 + s2, q = s1 + s3;
  float r = transpose_ror8(p, q);
  r += dpp<0x141>(r);  // row_half_mirror
  r += dpp<0x4E>(r);   // quad_perm [2,3,0,1]
  r += dpp<0xB1>(r);   // quad_perm [1,0,3,2]
  return r;
}

__device__ __forceinline__ void unpack(float4 v, float (&o)[4]) {
  o[0] = v.x;
  o[1] = v.y;
  o[2] = v.z;
  o[3] = v.w;
}
__device__ __forceinline__ void unpack(float2 v, float (&o)[2]) {
  o[0] = v.x;
  o[1] = v.y;
}

// ---- element types -----------------------------------------------------------
// The row tensors (u, dt, z, out, grads) and B/C are fp32 or bf16 in HBM; the
// recurrence, its state and every sum run in fp32.  bf16 is stored as its
// 16 bits; conversions are exact widening and round-to-nearest-even narrowing
// (gfx950's v_cvt_pk_bf16_f32, two values per instruction, NaN kept quiet).
using bf16_t = uint16_t;
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
// lo in bits 0..15, hi in bits 16..31
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  const f32x2_v f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_v));
}
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return static_cast<bf16_t>(f32x2_to_bf16x2(f, 0.f));
}

template <class E>
struct Elem;

template <>
struct Elem<float> {
  static __device__ __forceinline__ float4 load4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
  }
  static __device__ __forceinline__ float load1(const float* p) { return *p; }
  static __device__ __forceinline__ void store4(float* p, float4 v) {
    *reinterpret_cast<float4*>(p) = v;
  }
  static __device__ __forceinline__ void store1(float* p, float v) { *p = v; }
};

template <>
struct Elem<bf16_t> {
  static __device__ __forceinline__ float4 load4(const bf16_t* p) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
  }
  static __device__ __forceinline__ float load1(const bf16_t* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ void store4(bf16_t* p, float4 v) {
    uint2 w;
    w.x = f32x2_to_bf16x2(v.x, v.y);
    w.y = f32x2_to_bf16x2(v.z, v.w);
    *reinterpret_cast<uint2*>(p) = w;
  }
  static __device__ __forceinline__ void store1(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// ---- tile staging -----------------------------------------------------------
// Every launch runs kThreads threads.  A tile of a [.., L] tensor is ROWS rows
// (channels d0..d0+ROWS-1: 64, or 32 for the forward with 2 states per lane)
// x TT steps; thread i owns the float4 column groups
// q = i + k * kThreads of it, so its global loads are 16-byte row segments,
// consecutive threads covering a row.  Loads go to registers first and are
// written to LDS one tile later: the next tile's HBM reads overlap this
// tile's recurrence.
constexpr int kThreads = kMaxWaves * kWave;

template <int TT, int ROWS = kWave>
struct RowRegs {
  static constexpr int kQ = ROWS * TT / 4 / kThreads;
  static_assert(kQ >= 1, "a tile has at least one float4 per thread");
  float4 v[kQ];
};

template <int TT>
__device__ __forceinline__ void tile_pos(int k, int& row, int& c) {
  constexpr int C4 = TT / 4;
  const int q = threadIdx.x + k * kThreads;
  row = q / C4;
  c = (q - row * C4) * 4;
}

// Loads the thread's share of rows d0.. columns t0..  VEC: rows are 16-byte
// aligned (float4 loads).  Out-of-range elements read a clamped in-range
// address, so the loads carry no branches and all stay in flight together;
// they are zeroed when the tile is written to LDS (store_rows), not here, so
// that nothing waits on the loads before then.
template <int TT, bool VEC, class E, int ROWS>
__device__ __forceinline__ void load_rows(RowRegs<TT, ROWS>& r, const E* __restrict__ g,
                                          size_t row0, int d0, int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT, ROWS>::kQ; ++k) {
    int row, c;
    tile_pos<TT>(k, row, c);
    const int t = t0 + c;
    const size_t base = row0 + static_cast<size_t>(min(d0 + row, D - 1)) * L;
    if constexpr (VEC) {
      r.v[k] = Elem<E>::load4(g + base + min(t, L - 4));
    } else {
      r.v[k].x = Elem<E>::load1(g + base + min(t, L - 1));
      r.v[k].y = Elem<E>::load1(g + base + min(t + 1, L - 1));
      r.v[k].z = Elem<E>::load1(g + base + min(t + 2, L - 1));
      r.v[k].w = Elem<E>::load1(g + base + min(t + 3, L - 1));
    }
  }
}

// The loaded element (k, e) of a row tile is inside the tensor.
template <int TT>
__device__ __forceinline__ bool row_ok(int k, int e, int d0, int D, int t0, int L) {
  int row, c;
  tile_pos<TT>(k, row, c);
  return d0 + row < D && t0 + c + e < L;
}

template <int TT, int ROWS>
__device__ __forceinline__ float4 masked(const RowRegs<TT, ROWS>& r, int k, int d0, int D, int t0,
                                         int L) {
  const float4 v = r.v[k];
  return make_float4(row_ok<TT>(k, 0, d0, D, t0, L) ? v.x : 0.f,
                     row_ok<TT>(k, 1, d0, D, t0, L) ? v.y : 0.f,
                     row_ok<TT>(k, 2, d0, D, t0, L) ? v.z : 0.f,
                     row_ok<TT>(k, 3, d0, D, t0, L) ? v.w : 0.f);
}

template <int TT, int RS, int ROWS>
__device__ __forceinline__ void store_rows(float* __restrict__ s, const RowRegs<TT, ROWS>& r, int d0,
                                           int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT, ROWS>::kQ; ++k) {
    int row, c;
    tile_pos<TT>(k, row, c);
    const float4 v = masked<TT>(r, k, d0, D, t0, L);
    float* p = s + row * RS + c;
    p[0] = v.x;
    p[1] = v.y;
    p[2] = v.z;
    p[3] = v.w;
  }
}

// Stores 4 consecutive steps of one row of a [.., L] tensor.
template <bool VEC, class E>
__device__ __forceinline__ void store_row4(E* __restrict__ g, size_t off, int t, int L,
                                           float4 v) {
  if constexpr (VEC) {
    Elem<E>::store4(g + off, v);
  } else {
    Elem<E>::store1(g + off, v.x);
    if (t + 1 < L) Elem<E>::store1(g + off + 1, v.y);
    if (t + 2 < L) Elem<E>::store1(g + off + 2, v.z);
    if (t + 3 < L) Elem<E>::store1(g + off + 3, v.w);
  }
}

// ---- [B, L, D] tensors (the Mamba mixer's layout: channels contiguous) -----
// The same 64-channel x TT-step tile, loaded as 16-byte runs along the
// channels: thread i owns groups q = i + k * kThreads, step q / 16, channels
// 4 (q % 16) .. +3; written to LDS transposed (s[channel * RS + step]), the
// layout the kernels read.  `base` is the tensor's (b, 0, 0), `ld` its row
// stride (elements per step).  VEC: D % 4 == 0, ld % 4 == 0, 16-byte base.
template <int TT>
__device__ __forceinline__ void tile_pos_bld(int k, int& step, int& c4) {
  const int q = threadIdx.x + k * kThreads;
  step = q >> 4;
  c4 = (q & 15) * 4;
}

template <int TT, bool VEC, class E>
__device__ __forceinline__ void load_cols(RowRegs<TT>& r, const E* __restrict__ g, size_t base,
                                          int ld, int d0, int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
    int step, c4;
    tile_pos_bld<TT>(k, step, c4);
    const E* row = g + base + static_cast<size_t>(min(t0 + step, L - 1)) * ld;
    if constexpr (VEC) {
      r.v[k] = Elem<E>::load4(row + min(d0 + c4, D - 4));
    } else {
      r.v[k].x = Elem<E>::load1(row + min(d0 + c4, D - 1));
      r.v[k].y = Elem<E>::load1(row + min(d0 + c4 + 1, D - 1));
      r.v[k].z = Elem<E>::load1(row + min(d0 + c4 + 2, D - 1));
      r.v[k].w = Elem<E>::load1(row + min(d0 + c4 + 3, D - 1));
    }
  }
}

template <int TT>
__device__ __forceinline__ bool col_ok(int k, int e, int d0, int D, int t0, int L) {
  int step, c4;
  tile_pos_bld<TT>(k, step, c4);
  return d0 + c4 + e < D && t0 + step < L;
}

template <int TT>
__device__ __forceinline__ float4 masked_cols(const RowRegs<TT>& r, int k, int d0, int D, int t0,
                                              int L) {
  const float4 v = r.v[k];
  return make_float4(col_ok<TT>(k, 0, d0, D, t0, L) ? v.x : 0.f,
                     col_ok<TT>(k, 1, d0, D, t0, L) ? v.y : 0.f,
                     col_ok<TT>(k, 2, d0, D, t0, L) ? v.z : 0.f,
                     col_ok<TT>(k, 3, d0, D, t0, L) ? v.w : 0.f);
}

__device__ __forceinline__ void put_col4(float* __restrict__ s, int RS, int c4, int step, float4 v) {
  s[c4 * RS + step] = v.x;
  s[(c4 + 1) * RS + step] = v.y;
  s[(c4 + 2) * RS + step] = v.z;
  s[(c4 + 3) * RS + step] = v.w;
}

template <int TT, int RS>
__device__ __forceinline__ void store_cols(float* __restrict__ s, const RowRegs<TT>& r, int d0,
                                           int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
    int step, c4;
    tile_pos_bld<TT>(k, step, c4);
    put_col4(s, RS, c4, step, masked_cols<TT>(r, k, d0, D, t0, L));
  }
}

// softplus(x) = log(1 + e^x), and x itself above 20 (torch's default threshold,
// F.softplus as mambarec.py:155 applies it), as max(x, 0) + log1p(e) with
// e = e^-|x| <= 1: below e = 1/64 by the series e - e^2/2 + e^3/3 - e^4/4
// (truncation < e^5/5, 2e-10 relative), above it by the hardware log of 1 + e
// (rounding of 1 + e costs < 2^-24 / e relative, < 4e-6).
__device__ __forceinline__ float softplus(float x) {
  if (x > 20.f) return x;
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float l = e < 0.015625f ? e * (1.f - e * (0.5f - e * (1.f / 3.f - 0.25f * e)))
                                : __builtin_amdgcn_logf(1.f + e) * 0.69314718055994531f;
  return fmaxf(x, 0.f) + l;
}

// d softplus(x) / dx = sigmoid(x) = 1 - e^-s with s = softplus(x) >= 0: below
// s = 1/64 by the series s - s^2/2 + s^3/6 - s^4/24 (no cancellation), above
// it as 1 - e^-s.
__device__ __forceinline__ float sigmoid_of_softplus(float s) {
  return s < 0.015625f ? s * (1.f - s * (0.5f - s * (1.f / 6.f - s * (1.f / 24.f))))
                       : 1.f - fast_exp2(-s * kLog2e);
}

// dt = softplus(dt_pre + bias[d]) staged like store_cols (bias may be null).
template <int TT, int RS>
__device__ __forceinline__ void store_cols_softplus(float* __restrict__ s, const RowRegs<TT>& r,
                                                    const float* __restrict__ bias, int d0, int D,
                                                    int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
    int step, c4;
    tile_pos_bld<TT>(k, step, c4);
    const float4 v = r.v[k];
    const float x[4] = {v.x, v.y, v.z, v.w};
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = min(d0 + c4 + e, D - 1);
      o[e] = col_ok<TT>(k, e, d0, D, t0, L) ? softplus(x[e] + (bias != nullptr ? bias[d] : 0.f)) : 0.f;
    }
    put_col4(s, RS, c4, step, make_float4(o[0], o[1], o[2], o[3]));
  }
}

// B or C rows t0..t0+TT-1, states n_base..n_base+15 (zero outside the
// tensor, so padded states contribute nothing); LDS layout s[t * 16 + j].
template <int TT>
struct StateRegs {
  static constexpr int kQ = TT * kPassStates / kThreads;
  float v[kQ];
};

// `ld` is the row stride (N for a dense [B, L, N] tensor; wider for a view
// into a projection's output).
template <int TT, class E>
__device__ __forceinline__ void load_states(StateRegs<TT>& r, const E* __restrict__ g,
                                            size_t base, int ld, int t0, int L, int N, int n_base) {
#pragma unroll
  for (int k = 0; k < StateRegs<TT>::kQ; ++k) {
    const int e = threadIdx.x + k * kThreads;
    const int t = e / kPassStates, j = e - t * kPassStates;
    r.v[k] = Elem<E>::load1(g + base + static_cast<size_t>(min(t0 + t, L - 1)) * ld +
                            min(n_base + j, N - 1));
  }
}

template <int TT>
__device__ __forceinline__ void store_states(float* __restrict__ s, const StateRegs<TT>& r, int t0,
                                             int L, int N, int n_base) {
#pragma unroll
  for (int k = 0; k < StateRegs<TT>::kQ; ++k) {
    const int e = threadIdx.x + k * kThreads;
    const int t = e / kPassStates, j = e - t * kPassStates;
    s[e] = (t0 + t < L && n_base + j < N) ? r.v[k] : 0.f;
  }
}

// ---- forward ------------------------------------------------------------------
template <class E>
struct FwdArgs {
  const E* u;
  const E* dt;
  const float* A;
  const E* Bm;
  const E* Cm;
  const E* z;        // may be null
  E* out;
  E* raw;            // y before the gate, written by the last pass; may be null
  float* acc;        // fp32 y summed over the passes before the last; null for one pass
  float* ckpt;       // chunk_states, may be null
  int D, L, N, n_base, n_chunks;
  int first, last, vec;
  int ld_bc;         // row stride of B and C
  // [B, L, D] layout only: row strides of u, dt and z (out, raw, acc: D), and
  // dt given before its softplus, with an optional per-channel bias
  int ld_u, ld_dt, ld_z;
  const float* dt_bias;
  // [B, D, L] only: per-channel skip D (the extended API): the last pass adds
  // D u to y before raw_out and the gate; null for the reference's scan
  const float* dskip;
};

// (dt_t, u_t) pairs of a [.., L] row tile: s[row * RS2 + 2t].
template <int TT, int RS2, int ROWS>
__device__ __forceinline__ void store_rows_dtu(float* __restrict__ s, const RowRegs<TT, ROWS>& dt,
                                               const RowRegs<TT, ROWS>& u, int d0, int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT, ROWS>::kQ; ++k) {
    int row, c;
    tile_pos<TT>(k, row, c);
    const float4 a = masked<TT>(dt, k, d0, D, t0, L);
    const float4 b = masked<TT>(u, k, d0, D, t0, L);
    float* p = s + row * RS2 + 2 * c;
    *reinterpret_cast<float2*>(p) = make_float2(a.x, b.x);
    *reinterpret_cast<float2*>(p + 2) = make_float2(a.y, b.y);
    *reinterpret_cast<float2*>(p + 4) = make_float2(a.z, b.z);
    *reinterpret_cast<float2*>(p + 6) = make_float2(a.w, b.w);
  }
}

// The same from a [B, L, D] tile, dt through its softplus (as
// store_cols_softplus).
template <int TT, int RS2>
__device__ __forceinline__ void store_cols_dtu(float* __restrict__ s, const RowRegs<TT>& dt,
                                               const RowRegs<TT>& u, const float* __restrict__ bias,
                                               int d0, int D, int t0, int L) {
#pragma unroll
  for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
    int step, c4;
    tile_pos_bld<TT>(k, step, c4);
    const float4 v = dt.v[k];
    const float x[4] = {v.x, v.y, v.z, v.w};
    const float4 uu = masked_cols<TT>(u, k, d0, D, t0, L);
    const float uv[4] = {uu.x, uu.y, uu.z, uu.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = min(d0 + c4 + e, D - 1);
      const float sp = col_ok<TT>(k, e, d0, D, t0, L) ? softplus(x[e] + (bias != nullptr ? bias[d] : 0.f)) : 0.f;
      *reinterpret_cast<float2*>(s + (c4 + e) * RS2 + 2 * step) = make_float2(sp, uv[e]);
    }
  }
}

// B and C rows of a tile per state group of NPW: s[(t * groups + group) * 2 NPW
// + (state % NPW)] = B, + NPW = C (the groups of a step contiguous, so the
// lanes of a wave reading one step touch distinct banks); zero outside the
// tensor.
template <int TT, int NPW>
__device__ __forceinline__ void store_bc(float* __restrict__ s, const StateRegs<TT>& B,
                                         const StateRegs<TT>& C, int t0, int L, int N, int n_base) {
#pragma unroll
  for (int k = 0; k < StateRegs<TT>::kQ; ++k) {
    const int e = threadIdx.x + k * kThreads;
    const int t = e / kPassStates, j = e - t * kPassStates;
    const bool ok = t0 + t < L && n_base + j < N;
    float* q = s + (t * (kPassStates / NPW) + j / NPW) * 2 * NPW + (j % NPW);
    q[0] = ok ? B.v[k] : 0.f;
    q[NPW] = ok ? C.v[k] : 0.f;
  }
}

// The forward's lane layout for NPW states per lane: lane = (channel
// c = lane % CW, state group g = lane / CW), GR = 16 / NPW groups, so a wave
// holds all 16 states of CW = 64 / GR channels and a workgroup 4 CW channels.
// After the y reduction a lane holds SEG = 32 / GR output steps of its channel:
//   NPW = 4: steps 4g..4g+3 and 16+4g..16+4g+3 (the four lanes of a channel
//            cover 16 contiguous steps, 64 bytes of fp32, per 4-step access);
//   NPW = 2: steps 4g..4g+3 (the eight lanes of a channel cover the tile's 32
//            steps, 128 bytes).
// NPW = 2 has twice the waves for the same work (at BASELINE config 4, 768
// workgroups on 256 CUs instead of 384) for a third reduction stage and twice
// the per-lane dt / u reads per state.
template <int NPW>
struct FwdLayout {
  static_assert(NPW == 4 || NPW == 2, "4 or 2 states per lane");
  static constexpr int kGroups = kPassStates / NPW;
  static constexpr int kWaveCh = kWave / kGroups;
  static constexpr int kRows = kMaxWaves * kWaveCh;
  static constexpr int kSeg = kFwdTile / kGroups;
  static __device__ __forceinline__ int step(int g, int k) {
    if constexpr (NPW == 4) return (k < 4 ? 0 : 12) + 4 * g + k;
    else return 4 * g + k;
  }
};

// vec: N % 4 == 0 and chunk_states 16-byte aligned, so a lane whose NPW
// states all lie below N stores them with one 16-byte (8-byte) store (the
// lanes of a channel: 64 contiguous bytes); lanes past N store nothing.
template <int NPW>
__device__ __forceinline__ void write_ckpt(float* ckpt, size_t lane_row, int slot, int N, int n0,
                                           const float (&h)[NPW], bool vec) {
  const int c = slot >> 1, half = slot & 1;
  float* p = ckpt + lane_row + static_cast<size_t>(c) * 2 * N + half * N;
  if (vec && n0 + NPW <= N) {
    if constexpr (NPW == 4) {
      *reinterpret_cast<float4*>(p + n0) = make_float4(h[0], h[1], h[2], h[3]);
    } else {
      *reinterpret_cast<float2*>(p + n0) = make_float2(h[0], h[1]);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NPW; ++j)
    if (n0 + j < N) p[n0 + j] = h[j];
}

template <int ROWS>
struct FwdTile {
  RowRegs<kFwdTile, ROWS> u, dt;
  StateRegs<kFwdTile> B, C;
};

// row0: (b, 0, 0) of the [B, D, L] tensors; with BLD, bl0 = b * L is the
// first row of batch b and each tensor adds its own row stride.
template <class E, bool VEC, bool BLD, int ROWS>
__device__ __forceinline__ void fwd_prefetch(FwdTile<ROWS>& f, const FwdArgs<E>& a, size_t row0,
                                             size_t bc0, int d0, int t0) {
  if constexpr (BLD) {
    load_cols<kFwdTile, VEC>(f.u, a.u, row0 * a.ld_u, a.ld_u, d0, a.D, t0, a.L);
    load_cols<kFwdTile, VEC>(f.dt, a.dt, row0 * a.ld_dt, a.ld_dt, d0, a.D, t0, a.L);
  } else {
    load_rows<kFwdTile, VEC>(f.u, a.u, row0, d0, a.D, t0, a.L);
    load_rows<kFwdTile, VEC>(f.dt, a.dt, row0, d0, a.D, t0, a.L);
  }
  load_states<kFwdTile>(f.B, a.Bm, bc0, a.ld_bc, t0, a.L, a.N, a.n_base);
  load_states<kFwdTile>(f.C, a.Cm, bc0, a.ld_bc, t0, a.L, a.N, a.n_base);
}

// The lane's SEG steps of one row of a [.., L] tensor in tile t0, as 4-step
// pieces; reads past the end use clamped in-range addresses (values unused).
template <int NPW, bool VEC, class E>
__device__ __forceinline__ void load_seg(float (&v)[FwdLayout<NPW>::kSeg], const E* __restrict__ g,
                                         size_t row, int t0, int grp, int L) {
#pragma unroll
  for (int q = 0; q < FwdLayout<NPW>::kSeg / 4; ++q) {
    const int t = t0 + FwdLayout<NPW>::step(grp, 4 * q);
    if constexpr (VEC) {
      const float4 x = Elem<E>::load4(g + row + min(t, L - 4));
      v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * q + k] = Elem<E>::load1(g + row + min(t + k, L - 1));
    }
  }
}

// Stores the lane's SEG steps of tile t0 that lie before L.
template <int NPW, bool VEC, class E>
__device__ __forceinline__ void store_seg(E* __restrict__ g, size_t row, int t0, int grp, int L,
                                          const float (&v)[FwdLayout<NPW>::kSeg]) {
#pragma unroll
  for (int q = 0; q < FwdLayout<NPW>::kSeg / 4; ++q) {
    const int t = t0 + FwdLayout<NPW>::step(grp, 4 * q);
    if constexpr (VEC) {  // L % 4 == 0, so a group of 4 is all in or all out
      if (t < L) Elem<E>::store4(g + row + t, make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]));
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (t + k < L) Elem<E>::store1(g + row + t + k, v[4 * q + k]);
    }
  }
}

// Sums y over the state groups of each channel: lane (c, g) enters with its
// group's partial y for steps 0..31 of the tile and leaves with the full y of
// its steps FwdLayout<NPW>::step(g, 0..SEG-1).
//   NPW = 4: permlane32 swaps pair groups g and g ^ 2 (the lower half keeps
//   steps 0..7 and 16..23, the upper half 8..15 and 24..31), permlane16 swaps
//   pair g and g ^ 1.
//   NPW = 2: permlane32 pairs g and g ^ 4 (the lower half keeps steps 0..15),
//   permlane16 pairs g and g ^ 2 (even 16-lane rows keep the lower 8 of their
//   16), and a row_ror:8 DPP pairs g and g ^ 1 (lanes l and l ^ 8): each keeps
//   its 4 steps and sends the partner the other 4.
template <int NPW>
__device__ __forceinline__ void reduce_groups(float (&yv)[kFwdTile],
                                              float (&out)[FwdLayout<NPW>::kSeg], int g) {
  if constexpr (NPW == 4) {
    float s1[kFwdTile / 2];
#pragma unroll
    for (int k = 0; k < kFwdTile / 2; ++k) {
      const int i = k < 8 ? k : k + 8;
      float lo = yv[i], hi = yv[i + 8];
      swap32(lo, hi);
      s1[k] = lo + hi;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = j < 4 ? j : j + 4;
      float lo = s1[k], hi = s1[k + 4];
      swap16(lo, hi);
      out[j] = lo + hi;
    }
  } else {
    float s1[16], s2[8];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      float lo = yv[k], hi = yv[k + 16];
      swap32(lo, hi);
      s1[k] = lo + hi;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float lo = s1[k], hi = s1[k + 8];
      swap16(lo, hi);
      s2[k] = lo + hi;
    }
    const bool odd = (g & 1) != 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float keep = odd ? s2[k + 4] : s2[k];
      const float send = odd ? s2[k] : s2[k + 4];
      out[k] = keep + dpp<0x128>(send);  // row_ror:8
    }
  }
}

// GATED kernels multiply by silu(z) in the last pass; VEC: L % 4 == 0 and
// u/dt/z/out rows 16-byte aligned.  NPW: states per lane (FwdLayout); the
// [B, L, D] layout (BLD) runs 4.
template <class E, bool VEC, bool GATED, bool BLD, int NPW>
__global__ __launch_bounds__(kThreads) void selective_fwd_kernel(FwdArgs<E> a) {
  using LY = FwdLayout<NPW>;
  constexpr int TT = kFwdTile;
  constexpr int ROWS = LY::kRows, CW = LY::kWaveCh, SEG = LY::kSeg;
  static_assert(TT == 32, "reduce_groups assumes 32-step tiles");
  static_assert(!BLD || NPW == 4, "the [B, L, D] layout stages 64 channels");
  // dt and u interleaved, (dt_t, u_t) at [row * RS2 + 2t]: one 8-byte read per
  // step (rows of 66 floats: the wave's rows on distinct banks)
  constexpr int RS2 = 2 * TT + 2;
  __shared__ __align__(8) float s_dtu[ROWS * RS2];
  // B and C of each state group interleaved: (B of its NPW states, C of them)
  // at [(t * groups + group) * 2 NPW], one or two 16-byte reads per step
  __shared__ __align__(16) float s_BC[kPassStates * TT * 2];
  // BLD: the tile's y, [step][channel], stored to HBM as rows of channels
  constexpr int YS = kWave + 4;  // row stride (floats): 16-byte rows, banks staggered
  __shared__ __align__(16) float s_y[BLD ? TT * YS : 1];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int c = lane & (CW - 1), g = lane / CW;
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * ROWS;
  const int r = w * CW + c;  // the lane's channel row in the workgroup's tile
  const int d = d0 + r;
  const bool dvalid = d < a.D;
  const int n0 = a.n_base + g * NPW;  // first state of this lane
  const float Dskip = (!BLD && a.dskip != nullptr && dvalid) ? a.dskip[d] : 0.f;

  float A2[NPW], h[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    A2[j] = (dvalid && n0 + j < a.N) ? a.A[static_cast<size_t>(d) * a.N + n0 + j] * kLog2e : 0.f;
    h[j] = 0.f;
  }
  // BDL: row0 = (b, 0, 0) of [B,D,L]; BLD: row0 = b * L, the first row of batch b
  const size_t row0 = BLD ? static_cast<size_t>(b) * a.L : static_cast<size_t>(b) * a.D * a.L;
  const size_t bc0 = static_cast<size_t>(b) * a.L * a.ld_bc;  // (b, 0, 0) of B and C
  const size_t ck_row = (static_cast<size_t>(b) * a.D + (dvalid ? d : 0)) * a.n_chunks * 2 * a.N;
  const int dc = dvalid ? d : a.D - 1;
  const size_t my_row = row0 + static_cast<size_t>(dc) * a.L;  // [.., L] row of d (BDL)
  const bool ck = a.ckpt != nullptr && dvalid;
  const bool ck4 = a.N % 4 == 0 && (reinterpret_cast<uintptr_t>(a.ckpt) & 15) == 0;
  // [B, D, L] only: the gate and the outputs of the lane's SEG steps of tile t0
  auto load_gate = [&](float (&zv)[SEG], int t0) { load_seg<NPW, VEC>(zv, a.z, my_row, t0, g, a.L); };
  auto put_seg = [&](auto* dst, int t0, const float (&v)[SEG]) {
    store_seg<NPW, VEC>(dst, my_row, t0, g, a.L, v);
  };
  // this lane's NPW states of B and of C at step i of a staged tile
  using SV = std::conditional_t<NPW == 4, float4, float2>;
  struct BCv {
    SV b, c;
  };
  auto bc_vals = [&](const float* grp, int i) {
    const float* p = grp + i * 2 * kPassStates;
    if constexpr (NPW == 4) {
      return BCv{*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
    } else {
      const float4 v = *reinterpret_cast<const float4*>(p);
      return BCv{make_float2(v.x, v.y), make_float2(v.z, v.w)};
    }
  };

  // Time split: gridDim.z segments of consecutive tiles; segment s scans
  // tiles [s n / S, (s + 1) n / S) after re-running h alone over the tiles
  // before them (no outputs, the same per-step arithmetic, so the state it
  // reaches is bitwise the one the earlier segments compute).
  const int n_tiles = (a.L + TT - 1) / TT;
  const int n_seg = static_cast<int>(gridDim.z), seg = static_cast<int>(blockIdx.z);
  const int t_lo = (seg * n_tiles / n_seg) * TT;
  const int t_hi = min(a.L, ((seg + 1) * n_tiles / n_seg) * TT);

  FwdTile<ROWS> nxt;
  float zn[SEG];  // the gate of the lane's output segment, one tile ahead
  fwd_prefetch<E, VEC, BLD>(nxt, a, row0, bc0, d0, 0);
  for (int t0 = 0; t0 < t_lo; t0 += TT) {
    // h only over the earlier segment's tiles
    __syncthreads();
    if constexpr (BLD) {
      store_cols_dtu<TT, RS2>(s_dtu, nxt.dt, nxt.u, a.dt_bias, d0, a.D, t0, a.L);
    } else {
      store_rows_dtu<TT, RS2>(s_dtu, nxt.dt, nxt.u, d0, a.D, t0, a.L);
    }
    store_bc<TT, NPW>(s_BC, nxt.B, nxt.C, t0, a.L, a.N, a.n_base);
    __syncthreads();
    fwd_prefetch<E, VEC, BLD>(nxt, a, row0, bc0, d0, t0 + TT);
    const float* dturow = s_dtu + r * RS2;
    const float* BCgrp = s_BC + g * 2 * NPW;
#pragma unroll 8
    for (int i = 0; i < TT; ++i) {
      const float2 du = *reinterpret_cast<const float2*>(dturow + 2 * i);
      const float dtv = du.x;
      const float dtu = dtv * du.y;
      float Bv[NPW];
      unpack(bc_vals(BCgrp, i).b, Bv);
#pragma unroll
      for (int j = 0; j < NPW; ++j) h[j] = fmaf(fast_exp2(dtv * A2[j]), h[j], dtu * Bv[j]);
    }
  }
  if constexpr (GATED && !BLD) load_gate(zn, t_lo);
  for (int t0 = t_lo; t0 < t_hi; t0 += TT) {
    balance_priority((t_hi - t0 + TT - 1) / TT, (t_hi - t_lo + TT - 1) / TT);
    __syncthreads();  // the previous tile's LDS readers are done
    if constexpr (BLD) {
      store_cols_dtu<TT, RS2>(s_dtu, nxt.dt, nxt.u, a.dt_bias, d0, a.D, t0, a.L);
    } else {
      store_rows_dtu<TT, RS2>(s_dtu, nxt.dt, nxt.u, d0, a.D, t0, a.L);
    }
    store_bc<TT, NPW>(s_BC, nxt.B, nxt.C, t0, a.L, a.N, a.n_base);
    float zt[SEG];
#pragma unroll
    for (int k = 0; k < SEG; ++k) zt[k] = zn[k];
    __syncthreads();
    if (t0 + TT < t_hi) {
      fwd_prefetch<E, VEC, BLD>(nxt, a, row0, bc0, d0, t0 + TT);
      if constexpr (GATED && !BLD) load_gate(zn, t0 + TT);
    }
    // BLD: this tile's gate, for the row stores after the step loop
    RowRegs<TT> zq;
    if constexpr (GATED && BLD) load_cols<TT, VEC>(zq, a.z, row0 * a.ld_z, a.ld_z, d0, a.D, t0, a.L);

    // Every tile runs all TT steps: past L the staged dt, u, B and C are zero,
    // so h stays at the last step's state and y is zero there; the checkpoint
    // slots of the last tile then hold that final state, as their layout says.
    float yv[TT];  // this lane's y partial (its NPW states) per step
    float hck[TT / kCkpt][NPW];  // h after steps 15 and 31, checkpointed after the loop
    auto step = [&](int i, float dtv, float uv, SV Bt, SV Ct) {
      const float dtu = dtv * uv;
      float Bv[NPW], Cv[NPW];
      unpack(Bt, Bv);
      unpack(Ct, Cv);
      float y = 0.f;
#pragma unroll
      for (int j = 0; j < NPW; ++j) {
        const float dA = fast_exp2(dtv * A2[j]);
        h[j] = fmaf(dA, h[j], dtu * Bv[j]);
        y = fmaf(Cv[j], h[j], y);
      }
      // pin y here: left alone, the compiler sinks these FMAs to the reduction
      // after the loop and keeps every step's h and C alive (256 VGPRs)
      asm volatile("" : "+v"(y));
      yv[i] = y;
      if ((i + 1) % kCkpt == 0) {
#pragma unroll
        for (int j = 0; j < NPW; ++j) hck[i / kCkpt][j] = h[j];
      }
    };
    const float* dturow = s_dtu + r * RS2;
    const float* BCgrp = s_BC + g * 2 * NPW;
    {
      // Software-pipelined: the LDS operands of the next kGroup steps are read
      // before this group is computed, so a read's latency is covered by a
      // group of steps; a compiler fence per group keeps the compiler from
      // hoisting every step's reads to the top (256 VGPRs without it).
      constexpr int kGroup = 4;
      float pdt[2][kGroup], pu[2][kGroup];
      SV pB[2][kGroup], pC[2][kGroup];
      auto fetch = [&](int buf, int gr) {
#pragma unroll
        for (int q = 0; q < kGroup; ++q) {
          const int i = gr * kGroup + q;
          const float2 du = *reinterpret_cast<const float2*>(dturow + 2 * i);
          pdt[buf][q] = du.x;
          pu[buf][q] = du.y;
          const BCv bc = bc_vals(BCgrp, i);
          pB[buf][q] = bc.b;
          pC[buf][q] = bc.c;
        }
      };
      fetch(0, 0);
#pragma unroll
      for (int gr = 0; gr < TT / kGroup; ++gr) {
        const int cur = gr & 1;
        if (gr + 1 < TT / kGroup) fetch(cur ^ 1, gr + 1);
#pragma unroll
        for (int q = 0; q < kGroup; ++q)
          step(gr * kGroup + q, pdt[cur][q], pu[cur][q], pB[cur][q], pC[cur][q]);
        asm volatile("" ::: "memory");
      }
    }
    if (ck) {
#pragma unroll
      for (int q = 0; q < TT / kCkpt; ++q) write_ckpt<NPW>(a.ckpt, ck_row, t0 / kCkpt + q, a.N, n0, hck[q], ck4);
    }

    // y over the state groups (within the wave), then this lane's SEG outputs;
    // with a skip D, u of those steps is read first, behind the reduction
    float uskip[BLD ? 1 : SEG];
    if constexpr (!BLD) {
      if (a.last && a.dskip != nullptr) {
#pragma unroll
        for (int k = 0; k < SEG; ++k) uskip[k] = dturow[2 * LY::step(g, k) + 1];
      }
    }
    float y[SEG];
    reduce_groups<NPW>(yv, y, g);
    if constexpr (BLD) {
      // through LDS, so that rows of 64 channels leave as 16-byte runs
#pragma unroll
      for (int k = 0; k < SEG; ++k) s_y[LY::step(g, k) * YS + r] = y[k];
      __syncthreads();
#pragma unroll
      for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
        int step, c4;
        tile_pos_bld<TT>(k, step, c4);
        const int t = t0 + step, dd = d0 + c4;
        if (t >= a.L || dd >= a.D) continue;
        const int ne = min(4, a.D - dd);
        const float4 v4 = *reinterpret_cast<const float4*>(s_y + step * YS + c4);
        float v[4] = {v4.x, v4.y, v4.z, v4.w};
        const size_t gi = (row0 + t) * a.D + dd;
        if (!a.first) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (e < ne) v[e] += a.acc[gi + e];
        }
        auto put = [&](auto* dst) {
          if constexpr (VEC) {
            Elem<std::remove_pointer_t<decltype(dst)>>::store4(dst + gi, make_float4(v[0], v[1], v[2], v[3]));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < ne) Elem<std::remove_pointer_t<decltype(dst)>>::store1(dst + gi + e, v[e]);
          }
        };
        if (a.last) {
          if (a.raw != nullptr) put(a.raw);
          if constexpr (GATED) {
            const float4 zz = zq.v[k];
            const float zv[4] = {zz.x, zz.y, zz.z, zz.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= zv[e] * sigmoid(zv[e]);
          }
          put(a.out);
        } else {
          put(a.acc);
        }
      }
    } else if (dvalid) {
      if (!a.first) {
        float prev[SEG];
        load_seg<NPW, VEC>(prev, a.acc, my_row, t0, g, a.L);
#pragma unroll
        for (int k = 0; k < SEG; ++k) y[k] += prev[k];
      }
      if (a.last) {
        if (a.dskip != nullptr) {  // + D u, u of this tile as staged
#pragma unroll
          for (int k = 0; k < SEG; ++k) y[k] = fmaf(Dskip, uskip[k], y[k]);
        }
        if (a.raw != nullptr) put_seg(a.raw, t0, y);
        if constexpr (GATED) {
#pragma unroll
          for (int k = 0; k < SEG; ++k) y[k] *= zt[k] * sigmoid(zt[k]);
        }
        put_seg(a.out, t0, y);
      } else {
        put_seg(a.acc, t0, y);
      }
    }
  }
}

// ---- backward -----------------------------------------------------------------
template <class E>
struct BwdArgs {
  const E* gout;
  const E* u;
  const E* dt;
  const float* A;
  const E* Bm;
  const E* Cm;
  const E* z;          // may be null
  const E* raw;        // y from the forward; needed when z is given
  const float* ckpt;
  E* du;               // written by the last pass
  E* ddt;
  E* dz;               // written by the first pass when z is given
  float* du_acc;       // fp32 du / ddt summed over the passes before the last
  float* ddt_acc;
  float* part_dB;      // [n_dtiles, B, L, N]
  float* part_dC;
  float* part_dA;      // [time segments * B, D, N]
  int Bsz, D, L, N, n_base, n_chunks;
  int first, last, vec;
  int ld_bc;           // row stride of B and C
  // [B, L, D] layout only: row strides of u, dt and z (gout, raw, du, ddt, dz:
  // D); dt is given before its softplus and ddt is returned w.r.t. it
  int ld_u, ld_dt, ld_z;
  const float* dt_bias;
  // SKIP kernels ([B, D, L] only): the skip D of the forward; the first pass
  // adds D gy to du and writes the (segment, batch row) partials of
  // dD = sum_t gy u into part_dD [time segments * B, D]
  const float* dskip;
  float* part_dD;
};

struct BwdTile {
  RowRegs<kBwdTile> u, dt, go, z, raw;
  StateRegs<kBwdTile> B, C;
  float h0[kNpw];  // state after the step before the tile (this lane, this wave's states), unmasked
};

template <class E, bool VEC, bool GATED, bool BLD>
__device__ __forceinline__ void bwd_prefetch(BwdTile& f, const BwdArgs<E>& a, size_t row0, size_t bc0,
                                             size_t ck_row, int d0, bool dvalid, int n0, int tile) {
  const int t0 = tile * kBwdTile;
  if constexpr (BLD) {
    load_cols<kBwdTile, VEC>(f.u, a.u, row0 * a.ld_u, a.ld_u, d0, a.D, t0, a.L);
    load_cols<kBwdTile, VEC>(f.dt, a.dt, row0 * a.ld_dt, a.ld_dt, d0, a.D, t0, a.L);
    load_cols<kBwdTile, VEC>(f.go, a.gout, row0 * a.D, a.D, d0, a.D, t0, a.L);
    if constexpr (GATED) {
      load_cols<kBwdTile, VEC>(f.z, a.z, row0 * a.ld_z, a.ld_z, d0, a.D, t0, a.L);
      load_cols<kBwdTile, VEC>(f.raw, a.raw, row0 * a.D, a.D, d0, a.D, t0, a.L);
    }
  } else {
    load_rows<kBwdTile, VEC>(f.u, a.u, row0, d0, a.D, t0, a.L);
    load_rows<kBwdTile, VEC>(f.dt, a.dt, row0, d0, a.D, t0, a.L);
    load_rows<kBwdTile, VEC>(f.go, a.gout, row0, d0, a.D, t0, a.L);
    if constexpr (GATED) {
      load_rows<kBwdTile, VEC>(f.z, a.z, row0, d0, a.D, t0, a.L);
      load_rows<kBwdTile, VEC>(f.raw, a.raw, row0, d0, a.D, t0, a.L);
    }
  }
  load_states<kBwdTile>(f.B, a.Bm, bc0, a.ld_bc, t0, a.L, a.N, a.n_base);
  load_states<kBwdTile>(f.C, a.Cm, bc0, a.ld_bc, t0, a.L, a.N, a.n_base);
  // state after step t0 - 1 = checkpoint slot tile - 1 (zero before the start)
  const int slot = max(tile - 1, 0);
  const float* p = a.ckpt + ck_row + static_cast<size_t>(slot >> 1) * 2 * a.N + (slot & 1) * a.N;
  if (a.N % 4 == 0 && n0 + kNpw <= a.N && (reinterpret_cast<uintptr_t>(a.ckpt) & 15) == 0) {
    const float4 v = *reinterpret_cast<const float4*>(p + n0);
    f.h0[0] = v.x;
    f.h0[1] = v.y;
    f.h0[2] = v.z;
    f.h0[3] = v.w;
    return;
  }
#pragma unroll
  for (int j = 0; j < kNpw; ++j) {
    f.h0[j] = p[min(n0 + j, a.N - 1)];  // masked where it is consumed
  }
}

// What the adjoint-only pass of the time split reads per tile: dt, the
// upstream gradient and the gate (for gy), and C.
struct AdjTile {
  RowRegs<kBwdTile> dt, go, z;
  StateRegs<kBwdTile> C;
};

template <class E, bool VEC, bool GATED, bool BLD>
__device__ __forceinline__ void adj_prefetch(AdjTile& f, const BwdArgs<E>& a, size_t row0, size_t bc0,
                                             int d0, int tile) {
  const int t0 = tile * kBwdTile;
  if constexpr (BLD) {
    load_cols<kBwdTile, VEC>(f.dt, a.dt, row0 * a.ld_dt, a.ld_dt, d0, a.D, t0, a.L);
    load_cols<kBwdTile, VEC>(f.go, a.gout, row0 * a.D, a.D, d0, a.D, t0, a.L);
    if constexpr (GATED) load_cols<kBwdTile, VEC>(f.z, a.z, row0 * a.ld_z, a.ld_z, d0, a.D, t0, a.L);
  } else {
    load_rows<kBwdTile, VEC>(f.dt, a.dt, row0, d0, a.D, t0, a.L);
    load_rows<kBwdTile, VEC>(f.go, a.gout, row0, d0, a.D, t0, a.L);
    if constexpr (GATED) load_rows<kBwdTile, VEC>(f.z, a.z, row0, d0, a.D, t0, a.L);
  }
  load_states<kBwdTile>(f.C, a.Cm, bc0, a.ld_bc, t0, a.L, a.N, a.n_base);
}

template <class E, bool VEC, bool GATED, bool BLD, bool SKIP>
__global__ __launch_bounds__(kThreads) void selective_bwd_kernel(BwdArgs<E> a) {
  static_assert(!BLD || std::is_same_v<E, float>, "the [B, L, D] layout is fp32");
  static_assert(!(BLD && SKIP), "the skip D is for the [B, D, L] layout");
  constexpr int TT = kBwdTile;
  constexpr int HT = TT / 2;  // steps whose trajectory is held in registers at once
  constexpr int RS = TT + 1;
  __shared__ float s_u[kWave * RS];
  __shared__ float s_dt[kWave * RS];
  __shared__ float s_gy[kWave * RS];
  __shared__ __align__(16) float s_B[TT * kPassStates];
  __shared__ __align__(16) float s_C[TT * kPassStates];
  // per-wave du / ddt partials, [wave][channel][step], rows of DS = 16 floats
  // with the four 4-step groups of channel c rotated by (c >> 2) & 3
  // (du_col): a lane writes 4 steps of its channel as one 16-byte store and
  // the finish reads 4 steps of a channel with one 16-byte load, and both
  // touch 16 distinct 16-byte bank groups per quarter-wave
  constexpr int DS = TT;
  static_assert(TT == 16, "du_col rotates four 4-step groups");
  auto du_col = [](int c, int step) { return ((((step >> 2) + (c >> 2)) & 3) << 2) | (step & 3); };
  __shared__ __align__(16) float s_du[kMaxWaves * kWave * DS];
  __shared__ __align__(16) float s_ddt[kMaxWaves * kWave * DS];
  // SKIP: the skip D of the workgroup's channels, and each thread's running
  // sum of gy u over the steps it stages (dD)
  __shared__ float s_dsk[SKIP ? kWave : 1];
  __shared__ float s_dsum[SKIP ? kThreads : 1];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kWave;
  if constexpr (SKIP) {
    if (threadIdx.x < kWave) s_dsk[threadIdx.x] = d0 + static_cast<int>(threadIdx.x) < a.D ? a.dskip[d0 + threadIdx.x] : 0.f;
    s_dsum[threadIdx.x] = 0.f;  // read back by this thread only; s_dsk after the loop's first barrier
  }
  const int d = d0 + lane;
  const bool dvalid = d < a.D;
  const int n0 = a.n_base + w * kNpw;
  const int nw = min(kMaxWaves, (a.N - a.n_base + kNpw - 1) / kNpw);
  const bool wave_active = w < nw;

  float A2[kNpw], Af[kNpw], gs[kNpw], gA[kNpw];
#pragma unroll
  for (int j = 0; j < kNpw; ++j) {
    Af[j] = (dvalid && n0 + j < a.N) ? a.A[static_cast<size_t>(d) * a.N + n0 + j] : 0.f;
    A2[j] = Af[j] * kLog2e;
    gs[j] = 0.f;
    gA[j] = 0.f;
  }
  // BDL: row0 = (b, 0, 0) of [B,D,L]; BLD: row0 = b * L, the first row of batch b
  const size_t row0 = BLD ? static_cast<size_t>(b) * a.L : static_cast<size_t>(b) * a.D * a.L;
  const size_t bc0 = static_cast<size_t>(b) * a.L * a.ld_bc;
  const size_t ck_row = (static_cast<size_t>(b) * a.D + (dvalid ? d : 0)) * a.n_chunks * 2 * a.N;
  const size_t part0 = (static_cast<size_t>(blockIdx.x) * a.Bsz + b) * a.L * a.N;
  const int n_tiles = (a.L + TT - 1) / TT;
  // Time split: gridDim.z segments of consecutive tiles; segment s runs tiles
  // [s n / S, (s + 1) n / S) after an adjoint-only pass over the tiles after
  // them that carries gs from the end of the sequence with the main loop's
  // per-step arithmetic (so the carry is bitwise the one the later segments
  // reach).
  const int n_seg = static_cast<int>(gridDim.z), seg = static_cast<int>(blockIdx.z);
  const int tile_lo = seg * n_tiles / n_seg;
  const int tile_hi = (seg + 1) * n_tiles / n_seg;
  if (tile_hi < n_tiles) {
    AdjTile p;
    adj_prefetch<E, VEC, GATED, BLD>(p, a, row0, bc0, d0, n_tiles - 1);
    for (int tile = n_tiles - 1; tile >= tile_hi; --tile) {
      const int t0 = tile * TT;
      __syncthreads();
      if constexpr (BLD) {
        store_cols_softplus<TT, RS>(s_dt, p.dt, a.dt_bias, d0, a.D, t0, a.L);
      } else {
        store_rows<TT, RS>(s_dt, p.dt, d0, a.D, t0, a.L);
      }
      store_states<TT>(s_C, p.C, t0, a.L, a.N, a.n_base);
#pragma unroll
      for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
        float4 gy;
        if constexpr (BLD) gy = masked_cols<TT>(p.go, k, d0, a.D, t0, a.L);
        else gy = masked<TT>(p.go, k, d0, a.D, t0, a.L);
        if constexpr (GATED) {
          const float4 zz = p.z.v[k];
          gy = make_float4(gy.x * zz.x * sigmoid(zz.x), gy.y * zz.y * sigmoid(zz.y),
                           gy.z * zz.z * sigmoid(zz.z), gy.w * zz.w * sigmoid(zz.w));
        }
        if constexpr (BLD) {
          int step, c4;
          tile_pos_bld<TT>(k, step, c4);
          put_col4(s_gy, RS, c4, step, gy);
        } else {
          int rr, cc;
          tile_pos<TT>(k, rr, cc);
          float* q = s_gy + rr * RS + cc;
          q[0] = gy.x;
          q[1] = gy.y;
          q[2] = gy.z;
          q[3] = gy.w;
        }
      }
      __syncthreads();
      if (tile > tile_hi) adj_prefetch<E, VEC, GATED, BLD>(p, a, row0, bc0, d0, tile - 1);
      if (wave_active) {
        const float* dtrow = s_dt + lane * RS;
        const float* gyrow = s_gy + lane * RS;
        const float* Ccol = s_C + w * kNpw;
#pragma unroll 4
        for (int i = TT - 1; i >= 0; --i) {
          const float gy = gyrow[i], dtv = dtrow[i];
          const float4 Ct = *reinterpret_cast<const float4*>(Ccol + i * kPassStates);
          const float Cv[4] = {Ct.x, Ct.y, Ct.z, Ct.w};
#pragma unroll
          for (int j = 0; j < kNpw; ++j) gs[j] = fmaf(gy, Cv[j], gs[j]) * fast_exp2(dtv * A2[j]);
        }
      }
    }
  }

  // du / ddt of the tile at ft0, summed over the waves (states) from their
  // LDS partials and accumulated over passes
  auto finish_dudt = [&](const int ft0) {
    const int t0 = ft0;
    if constexpr (BLD) {
      // 4 channels at one step per thread; ddt is taken through the softplus:
      // d softplus(x) / dx = sigmoid(x), from softplus(x) staged in s_dt
#pragma unroll
      for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
        int step, c4;
        tile_pos_bld<TT>(k, step, c4);
        const int dd = d0 + c4, t = t0 + step;
        if (dd >= a.D || t >= a.L) continue;
        float su[4] = {0.f, 0.f, 0.f, 0.f}, sd[4] = {0.f, 0.f, 0.f, 0.f};
        for (int v = 0; v < nw; ++v) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            su[e] += s_du[(v * kWave + c4 + e) * DS + du_col(c4 + e, step)];
            sd[e] += s_ddt[(v * kWave + c4 + e) * DS + du_col(c4 + e, step)];
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) sd[e] *= sigmoid_of_softplus(s_dt[(c4 + e) * RS + step]);
        const size_t gi = (row0 + t) * a.D + dd;
        const int ne = min(4, a.D - dd);
        if (!a.first) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (e < ne) {
              su[e] += a.du_acc[gi + e];
              sd[e] += a.ddt_acc[gi + e];
            }
        }
        E* du = a.last ? a.du : reinterpret_cast<E*>(a.du_acc);
        E* ddt = a.last ? a.ddt : reinterpret_cast<E*>(a.ddt_acc);
        if (VEC) {
          Elem<E>::store4(du + gi, make_float4(su[0], su[1], su[2], su[3]));
          Elem<E>::store4(ddt + gi, make_float4(sd[0], sd[1], sd[2], sd[3]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (e < ne) {
              Elem<E>::store1(du + gi + e, su[e]);
              Elem<E>::store1(ddt + gi + e, sd[e]);
            }
        }
      }
    } else {
#pragma unroll
    for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
      int r, c;
      tile_pos<TT>(k, r, c);
      const int dd = d0 + r, t = t0 + c;
      if (dd >= a.D || t >= a.L) continue;
      float4 su = make_float4(0.f, 0.f, 0.f, 0.f), sd = su;
      for (int v = 0; v < nw; ++v) {
        const float4 pu = *reinterpret_cast<const float4*>(s_du + (v * kWave + r) * DS + du_col(r, c));
        const float4 pd = *reinterpret_cast<const float4*>(s_ddt + (v * kWave + r) * DS + du_col(r, c));
        su.x += pu.x;
        su.y += pu.y;
        su.z += pu.z;
        su.w += pu.w;
        sd.x += pd.x;
        sd.y += pd.y;
        sd.z += pd.z;
        sd.w += pd.w;
      }
      if constexpr (SKIP) {
        if (a.first) {  // + D gy (the tile's gy is still staged)
          const float* gq = s_gy + r * RS + c;
          const float Dd = s_dsk[r];
          su.x = fmaf(Dd, gq[0], su.x);
          su.y = fmaf(Dd, gq[1], su.y);
          su.z = fmaf(Dd, gq[2], su.z);
          su.w = fmaf(Dd, gq[3], su.w);
        }
      }
      const size_t gi = row0 + static_cast<size_t>(dd) * a.L + t;
      if (!a.first) {
        su.x += a.du_acc[gi];
        sd.x += a.ddt_acc[gi];
        if (t + 1 < a.L) { su.y += a.du_acc[gi + 1]; sd.y += a.ddt_acc[gi + 1]; }
        if (t + 2 < a.L) { su.z += a.du_acc[gi + 2]; sd.z += a.ddt_acc[gi + 2]; }
        if (t + 3 < a.L) { su.w += a.du_acc[gi + 3]; sd.w += a.ddt_acc[gi + 3]; }
      }
      if (a.last) {
        store_row4<VEC>(a.du, gi, t, a.L, su);
        store_row4<VEC>(a.ddt, gi, t, a.L, sd);
      } else {
        store_row4<VEC>(a.du_acc, gi, t, a.L, su);
        store_row4<VEC>(a.ddt_acc, gi, t, a.L, sd);
      }
    }
    }
  };

  BwdTile nxt;
  int prev_t0 = -1;  // [B, D, L]: the tile whose du / ddt are still to be finished
  bwd_prefetch<E, VEC, GATED, BLD>(nxt, a, row0, bc0, ck_row, d0, dvalid, n0, tile_hi - 1);
  for (int tile = tile_hi - 1; tile >= tile_lo; --tile) {
    const int t0 = tile * TT;
    const int nsteps = min(TT, a.L - t0);
    balance_priority(tile - tile_lo + 1, tile_hi - tile_lo);
    __syncthreads();  // the previous tile's LDS readers are done
    if constexpr (SKIP) {
      // the previous tile is finished while its gy is still staged.
      // No barrier before the staging below: a thread's finish reads only
      // the s_gy slots that the same thread stages (tile_pos), and the
      // LDS partials, which nothing writes before the next barrier.
      if (prev_t0 >= 0) finish_dudt(prev_t0);
    }
    float4 dz_v = make_float4(0.f, 0.f, 0.f, 0.f);
    size_t dz_off = 0;
    int dz_t = 0;
    bool dz_ok = false;
    if constexpr (BLD) {
      store_cols<TT, RS>(s_u, nxt.u, d0, a.D, t0, a.L);
      store_cols_softplus<TT, RS>(s_dt, nxt.dt, a.dt_bias, d0, a.D, t0, a.L);
    } else {
      store_rows<TT, RS>(s_u, nxt.u, d0, a.D, t0, a.L);
      store_rows<TT, RS>(s_dt, nxt.dt, d0, a.D, t0, a.L);
    }
    store_states<TT>(s_B, nxt.B, t0, a.L, a.N, a.n_base);
    store_states<TT>(s_C, nxt.C, t0, a.L, a.N, a.n_base);
    // gated upstream gradient into LDS; the first pass also writes dz
    if constexpr (BLD) {
#pragma unroll
      for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
        int step, c4;
        tile_pos_bld<TT>(k, step, c4);
        float4 gy = masked_cols<TT>(nxt.go, k, d0, a.D, t0, a.L);
        if constexpr (GATED) {
          const float4 zz = nxt.z.v[k], go = gy;
          const float4 sg = make_float4(sigmoid(zz.x), sigmoid(zz.y), sigmoid(zz.z), sigmoid(zz.w));
          gy = make_float4(go.x * zz.x * sg.x, go.y * zz.y * sg.y, go.z * zz.z * sg.z,
                           go.w * zz.w * sg.w);
          const int dd = d0 + c4, t = t0 + step;
          if (a.first && t < a.L && dd < a.D) {
            const float4 y = nxt.raw.v[k];
            const float dzv[4] = {go.x * y.x * (sg.x * (1.f + zz.x * (1.f - sg.x))),
                                  go.y * y.y * (sg.y * (1.f + zz.y * (1.f - sg.y))),
                                  go.z * y.z * (sg.z * (1.f + zz.z * (1.f - sg.z))),
                                  go.w * y.w * (sg.w * (1.f + zz.w * (1.f - sg.w)))};
            E* dst = a.dz + (row0 + t) * a.D + dd;
            if constexpr (VEC) {
              Elem<E>::store4(dst, make_float4(dzv[0], dzv[1], dzv[2], dzv[3]));
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (dd + e < a.D) Elem<E>::store1(dst + e, dzv[e]);
            }
          }
        }
        put_col4(s_gy, RS, c4, step, gy);
      }
    } else {
    static_assert(RowRegs<TT>::kQ == 1, "one deferred dz store per thread");
#pragma unroll
    for (int k = 0; k < RowRegs<TT>::kQ; ++k) {
      int r, c;
      tile_pos<TT>(k, r, c);
      float4 gy = masked<TT>(nxt.go, k, d0, a.D, t0, a.L);
      if constexpr (GATED) {
        const float4 zz = nxt.z.v[k], go = gy;
        const float4 sg = make_float4(sigmoid(zz.x), sigmoid(zz.y), sigmoid(zz.z), sigmoid(zz.w));
        gy = make_float4(go.x * zz.x * sg.x, go.y * zz.y * sg.y, go.z * zz.z * sg.z,
                         go.w * zz.w * sg.w);
        const int dd = d0 + r, t = t0 + c;
        if (a.first && dd < a.D && t < a.L) {
          const float4 y = nxt.raw.v[k];
          const float4 dzv = make_float4(go.x * y.x * (sg.x * (1.f + zz.x * (1.f - sg.x))),
                                         go.y * y.y * (sg.y * (1.f + zz.y * (1.f - sg.y))),
                                         go.z * y.z * (sg.z * (1.f + zz.z * (1.f - sg.z))),
                                         go.w * y.w * (sg.w * (1.f + zz.w * (1.f - sg.w))));
          dz_v = dzv;  // stored after the next tile's loads are issued
          dz_off = row0 + static_cast<size_t>(dd) * a.L + t;
          dz_t = t;
          dz_ok = true;
        }
      }
      float* p = s_gy + r * RS + c;
      p[0] = gy.x;
      p[1] = gy.y;
      p[2] = gy.z;
      p[3] = gy.w;
      if constexpr (SKIP) {
        if (a.first) {  // gy u of the staged steps into this thread's dD sum
          const float4 uu = masked<TT>(nxt.u, k, d0, a.D, t0, a.L);
          s_dsum[threadIdx.x] =
              fmaf(gy.x, uu.x, fmaf(gy.y, uu.y, fmaf(gy.z, uu.z, fmaf(gy.w, uu.w, s_dsum[threadIdx.x]))));
        }
      }
    }
    }
    float h0[kNpw];
#pragma unroll
    for (int j = 0; j < kNpw; ++j) h0[j] = (tile > 0 && dvalid && n0 + j < a.N) ? nxt.h0[j] : 0.f;
    if constexpr (BLD) {
      __syncthreads();
      if (tile > tile_lo) bwd_prefetch<E, VEC, GATED, BLD>(nxt, a, row0, bc0, ck_row, d0, dvalid, n0, tile - 1);
    } else {
      // the next tile's loads go out before this interval's stores (dz, and
      // du / ddt of the previous tile, whose LDS partials this barrier
      // interval still holds)
      if (tile > tile_lo) bwd_prefetch<E, VEC, GATED, BLD>(nxt, a, row0, bc0, ck_row, d0, dvalid, n0, tile - 1);
      if (dz_ok) store_row4<VEC>(a.dz, dz_off, dz_t, a.L, dz_v);
      if (!SKIP && prev_t0 >= 0) finish_dudt(prev_t0);
      __syncthreads();
    }

    if (wave_active) {
      const float* dtrow = s_dt + lane * RS;
      const float* urow = s_u + lane * RS;
      const float* gyrow = s_gy + lane * RS;
      const float* Bcol = s_B + w * kNpw;
      const float* Ccol = s_C + w * kNpw;
      float* durow = s_du + (w * kWave + lane) * DS;
      float* ddtrow = s_ddt + (w * kWave + lane) * DS;
      // keep[h]: this lane's share of the dB / dC tile partials of steps
      // 8h .. 8h + 7 (see reduce8 for which lane holds which total)
      float keep[2] = {0.f, 0.f};

      // The forward over steps s0 .. s0 + HT - 1 of the tile from the state
      // before step s0, into registers: the state after each step and its
      // exp(dt A).  Steps past L were staged as zeros, so they leave h
      // unchanged and contribute exact zeros below.  Each step's LDS operands
      // are read one step ahead; the empty asm with a memory clobber after
      // every step keeps the compiler from hoisting all of them to the top
      // (registers).
      auto forward_half = [&](auto s0_tag, const float (&hst)[kNpw], float (&hs)[HT][kNpw],
                              float (&dAs)[HT][kNpw]) {
        constexpr int s0 = decltype(s0_tag)::value;
        float h[kNpw];
#pragma unroll
        for (int j = 0; j < kNpw; ++j) h[j] = hst[j];
        float ndt = dtrow[s0], nu = urow[s0];
        float4 nB = *reinterpret_cast<const float4*>(Bcol + s0 * kPassStates);
#pragma unroll
        for (int i = 0; i < HT; ++i) {
          const float dtv = ndt, uv = nu;
          const float Bv[4] = {nB.x, nB.y, nB.z, nB.w};
          if (i + 1 < HT) {
            ndt = dtrow[s0 + i + 1];
            nu = urow[s0 + i + 1];
            nB = *reinterpret_cast<const float4*>(Bcol + (s0 + i + 1) * kPassStates);
          }
          const float dtu = dtv * uv;
#pragma unroll
          for (int j = 0; j < kNpw; ++j) {
            const float dA = fast_exp2(dtv * A2[j]);
            h[j] = fmaf(dA, h[j], dtu * Bv[j]);
            hs[i][j] = h[j];
            dAs[i][j] = dA;
          }
          asm volatile("" ::: "memory");
        }
      };
      // The adjoint over the same steps in reverse, from the trajectory the
      // forward above left (hst = the state before step s0).
      auto adjoint_half = [&](auto s0_tag, const float (&hst)[kNpw], const float (&hs)[HT][kNpw],
                              const float (&dAs)[HT][kNpw]) {
        constexpr int s0 = decltype(s0_tag)::value;
        constexpr int il = HT - 1;
        float ngy = gyrow[s0 + il], ndt = dtrow[s0 + il], nu = urow[s0 + il];
        float4 nB = *reinterpret_cast<const float4*>(Bcol + (s0 + il) * kPassStates);
        float4 nC = *reinterpret_cast<const float4*>(Ccol + (s0 + il) * kPassStates);
        float du4[4], dd4[4];  // the current group of 4 steps, written together
#pragma unroll
        for (int i = il; i >= 0; --i) {
          const float gy = ngy, dtv = ndt, uv = nu;
          const float Bv[4] = {nB.x, nB.y, nB.z, nB.w};
          const float Cv[4] = {nC.x, nC.y, nC.z, nC.w};
          if (i > 0) {
            ngy = gyrow[s0 + i - 1];
            ndt = dtrow[s0 + i - 1];
            nu = urow[s0 + i - 1];
            nB = *reinterpret_cast<const float4*>(Bcol + (s0 + i - 1) * kPassStates);
            nC = *reinterpret_cast<const float4*>(Ccol + (s0 + i - 1) * kPassStates);
          }
          const float dtu = dtv * uv;
          float S1 = 0.f, S2 = 0.f;
          float v[8];
#pragma unroll
          for (int j = 0; j < kNpw; ++j) {
            const float hprev = i > 0 ? hs[i > 0 ? i - 1 : 0][j] : hst[j];
            const float gacc = fmaf(gy, Cv[j], gs[j]);
            const float gsn = gacc * dAs[i][j];
            const float q = gsn * hprev;
            gA[j] = fmaf(dtv, q, gA[j]);
            S2 = fmaf(Af[j], q, S2);
            S1 = fmaf(gacc, Bv[j], S1);
            v[j] = gacc * dtu;         // dB contribution
            v[4 + j] = gy * hs[i][j];  // dC contribution
            gs[j] = gsn;
          }
          du4[i & 3] = dtv * S1;
          dd4[i & 3] = fmaf(uv, S1, S2);
          if ((i & 3) == 0) {
            *reinterpret_cast<float4*>(durow + du_col(lane, s0 + i)) = make_float4(du4[0], du4[1], du4[2], du4[3]);
            *reinterpret_cast<float4*>(ddtrow + du_col(lane, s0 + i)) = make_float4(dd4[0], dd4[1], dd4[2], dd4[3]);
          }
          const float o = reduce8(v);
          if ((lane & 7) == i) keep[s0 / HT] = o;
          asm volatile("" ::: "memory");
        }
      };

      // The second half first (from the state after step HT - 1), then the
      // first, whose trajectory the forward over it kept.  A tile that ends
      // within its first half skips the second: all padding.  The [B, L, D]
      // kernels (more registers for their column staging) keep only the first
      // half's exponentials across the second half and re-run its states.
      float hs0[HT][kNpw], dA0[HT][kNpw];
      forward_half(std::integral_constant<int, 0>{}, h0, hs0, dA0);
      if (nsteps > HT) {
        float hs1[HT][kNpw], dA1[HT][kNpw];
        forward_half(std::integral_constant<int, HT>{}, hs0[HT - 1], hs1, dA1);
        adjoint_half(std::integral_constant<int, HT>{}, hs0[HT - 1], hs1, dA1);
        if constexpr (BLD) {
          float h[kNpw];
#pragma unroll
          for (int j = 0; j < kNpw; ++j) h[j] = h0[j];
#pragma unroll
          for (int i = 0; i < HT; ++i) {
            const float dtu = dtrow[i] * urow[i];
            const float4 Bt = *reinterpret_cast<const float4*>(Bcol + i * kPassStates);
            const float Bv[4] = {Bt.x, Bt.y, Bt.z, Bt.w};
#pragma unroll
            for (int j = 0; j < kNpw; ++j) {
              h[j] = fmaf(dA0[i][j], h[j], dtu * Bv[j]);
              hs0[i][j] = h[j];
            }
          }
        }
      }
      adjoint_half(std::integral_constant<int, 0>{}, h0, hs0, dA0);

      // lane l holds the tile partial of step t0 + 8h + (l & 7) in keep[h]:
      // dB[n0 + k] for k = (l >> 3) & 7 < 4, dC[n0 + k - 4] for the rest
      const int k = (lane >> 3) & 7, c8 = lane & 7;
      const int nn = n0 + (k & 3);
      if (nn < a.N) {
        float* dst = (k < 4 ? a.part_dB : a.part_dC) + part0 + nn;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = 8 * h + c8;
          if (c < nsteps) dst[static_cast<size_t>(t0 + c) * a.N] = keep[h];
        }
      }
    }
    if constexpr (BLD) {
      __syncthreads();
      finish_dudt(t0);
    } else {
      prev_t0 = t0;  // finished while the next tile is staged
    }
  }
  if constexpr (!BLD) {
    __syncthreads();
    finish_dudt(prev_t0);
  }
  if constexpr (SKIP) {
    if (a.first) {
      // over the 4 threads (one quad) that staged each channel row
      float dsum = s_dsum[threadIdx.x];
      dsum += dpp<0xB1>(dsum);  // quad_perm [1,0,3,2]
      dsum += dpp<0x4E>(dsum);  // quad_perm [2,3,0,1]
      int r, c;
      tile_pos<TT>(0, r, c);
      if (c == 0 && d0 + r < a.D)
        a.part_dD[(static_cast<size_t>(seg) * a.Bsz + b) * a.D + d0 + r] = dsum;
    }
  }

  if (dvalid && wave_active) {
    // one row of partials per (segment, batch row)
    const size_t prow = static_cast<size_t>(seg) * a.Bsz + b;
#pragma unroll
    for (int j = 0; j < kNpw; ++j)
      if (n0 + j < a.N) a.part_dA[(prow * a.D + d) * a.N + n0 + j] = gA[j];
  }
}

// ---- backward, 2 states per lane ---------------------------------------------
// lane = (channel c = lane % 32, state pair: wave w holds states 4w..4w+3,
// lanes 0..31 the first two, lanes 32..63 the other two), so a workgroup holds
// 32 channels x 16 states with half the registers per lane of the kernel
// above: three workgroups fit on a compute unit instead of two.  Tiles of 32
// steps are staged; each 16-step half starts from the checkpoint the forward
// wrote for it (after step 15 of the tile, or before the tile), is re-run
// forward into registers and then walked backward, so no step is recomputed.
// dB / dC are summed over the 32 channels of a pair (reduce4_32); du / ddt
// over the two pairs of a wave with a permlane32 swap and over the four waves
// through LDS.
constexpr int kB2Rows = 32;       // channels per workgroup
constexpr int kB2Tile = kChunk;   // staged steps (two checkpoint intervals)
constexpr int kB2Half = kCkpt;    // steps whose trajectory is held in registers

// Sums v[0..3] over the 32 channel lanes of each pair (lanes with the same
// lane / 32): lanes of row r = lane / 16 receive, in their low half (lane % 16
// < 8), the total of v[r & 1] and, in their high half, of v[2 + (r & 1)].
__device__ __forceinline__ float reduce4_32(const float (&v)[4]) {
  float a0 = v[0], a1 = v[1], b0 = v[2], b1 = v[3];
  swap16(a0, a1);
  swap16(b0, b1);
  // even rows: 2-lane sums (channels c, c + 16) of v[0] / v[2], odd rows of v[1] / v[3]
  float r = transpose_ror8(a0 + a1, b0 + b1);
  r += dpp<0x141>(r);  // row_half_mirror
  r += dpp<0x4E>(r);   // quad_perm [2,3,0,1]
  r += dpp<0xB1>(r);   // quad_perm [1,0,3,2]
  return r;
}

struct BwdTile2 {
  float4 u, dt, go, z, raw;  // this thread's 4 steps of one channel row
  float B[2], C[2];          // StateRegs of the tile
  float h0[2];               // this lane's two states before the tile, unmasked
  float hm[2];               // and after its step kB2Half - 1
};

// Addressing of the 2-states-per-lane backward: every global access is a
// workgroup-uniform base (scalar registers) plus a 32-bit lane offset, so the
// loop-invariant part of an address costs one VGPR instead of two.  The host
// takes this kernel only when every offset fits (bwd2_offsets_fit).
template <bool VEC, class E>
__device__ __forceinline__ float4 b2_load_row(const E* __restrict__ base, uint32_t roff, int t, int L) {
  if constexpr (VEC) {
    return Elem<E>::load4(base + (roff + static_cast<uint32_t>(min(t, L - 4))));
  } else {
    return make_float4(Elem<E>::load1(base + (roff + static_cast<uint32_t>(min(t, L - 1)))),
                       Elem<E>::load1(base + (roff + static_cast<uint32_t>(min(t + 1, L - 1)))),
                       Elem<E>::load1(base + (roff + static_cast<uint32_t>(min(t + 2, L - 1)))),
                       Elem<E>::load1(base + (roff + static_cast<uint32_t>(min(t + 3, L - 1)))));
  }
}

// B or C of steps t0.. (rows of stride ld from `base` = the batch row's first)
template <class E>
__device__ __forceinline__ void b2_load_states(float (&v)[2], const E* __restrict__ base, int ld, int t0,
                                               int L, int N, int n_base) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = threadIdx.x + k * kThreads;
    const int t = e / kPassStates, j = e - t * kPassStates;
    v[k] = Elem<E>::load1(base + static_cast<uint32_t>(min(t0 + t, L - 1) * ld + min(n_base + j, N - 1)));
  }
}

__device__ __forceinline__ void b2_load_pair(float (&h)[2], const float* __restrict__ base, uint32_t off,
                                             int n0, int N, bool vec2) {
  if (vec2) {
    const float2 v = *reinterpret_cast<const float2*>(base + (off + static_cast<uint32_t>(n0)));
    h[0] = v.x;
    h[1] = v.y;
  } else {
    h[0] = base[off + static_cast<uint32_t>(min(n0, N - 1))];  // masked where they are consumed
    h[1] = base[off + static_cast<uint32_t>(min(n0 + 1, N - 1))];
  }
}

// Workgroup-uniform bases of the 2-states-per-lane backward.
template <class E>
struct Bwd2Bases {
  const E *u, *dt, *go, *z, *raw;  // (b, d0, 0) of the [B, D, L] tensors
  const E *Bm, *Cm;                // (b, 0, 0) of B and C
  const float* ck;                 // chunk_states of (b, d0)
};

template <class E, bool VEC, bool GATED>
__device__ __forceinline__ void bwd2_prefetch(BwdTile2& f, const BwdArgs<E>& a, const Bwd2Bases<E>& g,
                                              uint32_t roff, int cc, uint32_t ckoff, int n0, bool vec2,
                                              int tile) {
  const int t0 = tile * kB2Tile;
  f.u = b2_load_row<VEC>(g.u, roff, t0 + cc, a.L);
  f.dt = b2_load_row<VEC>(g.dt, roff, t0 + cc, a.L);
  f.go = b2_load_row<VEC>(g.go, roff, t0 + cc, a.L);
  if constexpr (GATED) {
    f.z = b2_load_row<VEC>(g.z, roff, t0 + cc, a.L);
    f.raw = b2_load_row<VEC>(g.raw, roff, t0 + cc, a.L);
  }
  b2_load_states(f.B, g.Bm, a.ld_bc, t0, a.L, a.N, a.n_base);
  b2_load_states(f.C, g.Cm, a.ld_bc, t0, a.L, a.N, a.n_base);
  // chunk_states row k holds h after steps 32k + 15 and 32k + 31
  b2_load_pair(f.h0, g.ck, ckoff + static_cast<uint32_t>(max(tile - 1, 0) * 2 * a.N + a.N), n0, a.N, vec2);
  b2_load_pair(f.hm, g.ck, ckoff + static_cast<uint32_t>(tile * 2 * a.N), n0, a.N, vec2);
}

struct AdjTile2 {
  float4 dt, go, z;
  float C[2];
};

template <class E, bool VEC, bool GATED>
__device__ __forceinline__ void adj2_prefetch(AdjTile2& f, const BwdArgs<E>& a, const Bwd2Bases<E>& g,
                                              uint32_t roff, int cc, int tile) {
  const int t0 = tile * kB2Tile;
  f.dt = b2_load_row<VEC>(g.dt, roff, t0 + cc, a.L);
  f.go = b2_load_row<VEC>(g.go, roff, t0 + cc, a.L);
  if constexpr (GATED) f.z = b2_load_row<VEC>(g.z, roff, t0 + cc, a.L);
  b2_load_states(f.C, g.Cm, a.ld_bc, t0, a.L, a.N, a.n_base);
}

// A staged float4 of (row r, steps t..t+3), zero outside the tensor.
__device__ __forceinline__ float4 b2_mask(float4 v, bool row_ok, int t, int L) {
  return make_float4(row_ok && t < L ? v.x : 0.f, row_ok && t + 1 < L ? v.y : 0.f,
                     row_ok && t + 2 < L ? v.z : 0.f, row_ok && t + 3 < L ? v.w : 0.f);
}
__device__ __forceinline__ void b2_put(float* p, float4 v) {
  p[0] = v.x;
  p[1] = v.y;
  p[2] = v.z;
  p[3] = v.w;
}
// (dt_t, u_t) pairs of steps cs..cs+3 of one channel row.
__device__ __forceinline__ void b2_put_dtu(float* p, float4 dt, float4 u) {
  *reinterpret_cast<float2*>(p) = make_float2(dt.x, u.x);
  *reinterpret_cast<float2*>(p + 2) = make_float2(dt.y, u.y);
  *reinterpret_cast<float2*>(p + 4) = make_float2(dt.z, u.z);
  *reinterpret_cast<float2*>(p + 6) = make_float2(dt.w, u.w);
}
// B (when given) and C of the tile per state pair: s[(t * 8 + pair) * 4 +
// (state & 1)] = B, + 2 = C (the pairs of a step contiguous: a wave's two pairs
// on distinct banks); zero outside the tensor.
__device__ __forceinline__ void b2_store_bc(float* __restrict__ s, const float* B, const float (&C)[2], int t0,
                                            int L, int N, int n_base) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = threadIdx.x + k * kThreads;
    const int t = e / kPassStates, j = e - t * kPassStates;
    const bool ok = t0 + t < L && n_base + j < N;
    float* q = s + (t * (kPassStates / 2) + (j >> 1)) * 4 + (j & 1);
    if (B != nullptr) q[0] = ok ? B[k] : 0.f;
    q[2] = ok ? C[k] : 0.f;
  }
}

template <class E, bool VEC, bool GATED, bool SKIP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
void selective_bwd2_kernel(BwdArgs<E> a) {
  constexpr int TT = kB2Tile;
  constexpr int HT = kB2Half;
  constexpr int RS = TT + 1;
  constexpr int ROWS = kB2Rows;
  static_assert(ROWS * TT == 4 * kThreads, "one float4 of each row tensor per thread");
  // dt and u interleaved, (dt_t, u_t) at [c * RS2 + 2t]: one 8-byte read per
  // step; rows of 66 floats put the 32 channels' reads on distinct banks
  constexpr int RS2 = 2 * TT + 2;
  __shared__ __align__(16) float s_dtu[ROWS * RS2];
  __shared__ float s_gy[ROWS * RS];
  // B and C of each state pair interleaved, (B_n, B_n+1, C_n, C_n+1) at
  // [(t * 8 + pair) * 4]: one 16-byte read per step
  __shared__ __align__(16) float s_BC[kPassStates / 2 * TT * 4];
  // per-wave du / ddt partials (sums over the wave's four states),
  // [wave][channel][step], with the eight 4-step groups of channel c permuted
  // by XOR with (c >> 1) & 7 (du_col): 16-byte stores by 32 consecutive
  // channels and the finish's 16-byte reads both touch 16 distinct 16-byte
  // bank groups per quarter-wave
  auto du_col = [](int c, int step) { return ((((step >> 2) ^ (c >> 1)) & 7) << 2) | (step & 3); };
  __shared__ __align__(16) float s_du[kMaxWaves * ROWS * TT];
  __shared__ __align__(16) float s_ddt[kMaxWaves * ROWS * TT];

  // SKIP: the skip D of the workgroup's channels, and each thread's running
  // sum of gy u over the steps it stages (dD)
  __shared__ float s_dsk[SKIP ? ROWS : 1];
  __shared__ float s_dsum[SKIP ? kThreads : 1];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int c = lane & (ROWS - 1);
  const int hi = lane >> 5;
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * ROWS;
  const bool dvalid = d0 + c < a.D;
  if constexpr (SKIP) {
    if (threadIdx.x < ROWS) s_dsk[threadIdx.x] = d0 + static_cast<int>(threadIdx.x) < a.D ? a.dskip[d0 + threadIdx.x] : 0.f;
    s_dsum[threadIdx.x] = 0.f;  // read back by this thread only; s_dsk after the loop's first barrier
  }
  const int n0 = a.n_base + 4 * w + 2 * hi;  // this lane's states n0, n0 + 1
  const int nw = min(kMaxWaves, (a.N - a.n_base + 3) / 4);
  const bool wave_active = w < nw;
  const bool vec2 = a.N % 2 == 0 && n0 + 2 <= a.N && (reinterpret_cast<uintptr_t>(a.ckpt) & 7) == 0;
  // staging position of this thread: channel row rs, steps cs..cs+3
  const int rs = static_cast<int>(threadIdx.x) >> 3, cs = (static_cast<int>(threadIdx.x) & 7) * 4;
  const bool rs_ok = d0 + rs < a.D;
  const uint32_t roff = static_cast<uint32_t>(min(d0 + rs, a.D - 1) - d0) * static_cast<uint32_t>(a.L);

  float A2[2], Af[2], gs[2], gA[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    Af[j] = (dvalid && n0 + j < a.N) ? a.A[static_cast<size_t>(d0 + c) * a.N + n0 + j] : 0.f;
    A2[j] = Af[j] * kLog2e;
    gs[j] = 0.f;
    gA[j] = 0.f;
  }
  const size_t rowbase = (static_cast<size_t>(b) * a.D + d0) * a.L;
  Bwd2Bases<E> g;
  g.u = a.u + rowbase;
  g.dt = a.dt + rowbase;
  g.go = a.gout + rowbase;
  g.z = GATED ? a.z + rowbase : nullptr;
  g.raw = GATED ? a.raw + rowbase : nullptr;
  g.Bm = a.Bm + static_cast<size_t>(b) * a.L * a.ld_bc;
  g.Cm = a.Cm + static_cast<size_t>(b) * a.L * a.ld_bc;
  g.ck = a.ckpt + (static_cast<size_t>(b) * a.D + d0) * a.n_chunks * 2 * a.N;
  const uint32_t ckoff = static_cast<uint32_t>(dvalid ? c : 0) * static_cast<uint32_t>(a.n_chunks * 2 * a.N);
  const int n_tiles = (a.L + TT - 1) / TT;
  // time split as in selective_bwd_kernel: segment s runs tiles
  // [s n / S, (s + 1) n / S) after an adjoint-only pass over the later tiles
  const int n_seg = static_cast<int>(gridDim.z), seg = static_cast<int>(blockIdx.z);
  const int tile_lo = seg * n_tiles / n_seg;
  const int tile_hi = (seg + 1) * n_tiles / n_seg;
  if (tile_hi < n_tiles) {
    AdjTile2 p;
    adj2_prefetch<E, VEC, GATED>(p, a, g, roff, cs, n_tiles - 1);
    for (int tile = n_tiles - 1; tile >= tile_hi; --tile) {
      const int t0 = tile * TT;
      __syncthreads();
      b2_put_dtu(s_dtu + rs * RS2 + 2 * cs, b2_mask(p.dt, rs_ok, t0 + cs, a.L), make_float4(0.f, 0.f, 0.f, 0.f));
      b2_store_bc(s_BC, nullptr, p.C, t0, a.L, a.N, a.n_base);
      float4 gy = b2_mask(p.go, rs_ok, t0 + cs, a.L);
      if constexpr (GATED) {
        const float4 zz = p.z;
        gy = make_float4(gy.x * zz.x * sigmoid(zz.x), gy.y * zz.y * sigmoid(zz.y),
                         gy.z * zz.z * sigmoid(zz.z), gy.w * zz.w * sigmoid(zz.w));
      }
      b2_put(s_gy + rs * RS + cs, gy);
      __syncthreads();
      if (tile > tile_hi) adj2_prefetch<E, VEC, GATED>(p, a, g, roff, cs, tile - 1);
      if (wave_active) {
        const float* dturow = s_dtu + c * RS2;
        const float* gyrow = s_gy + c * RS;
        const float* BCrow = s_BC + (2 * w + hi) * 4;
#pragma unroll 4
        for (int i = TT - 1; i >= 0; --i) {
          const float gy = gyrow[i], dtv = dturow[2 * i];
          const float2 Ct = *reinterpret_cast<const float2*>(BCrow + 32 * i + 2);
          const float Cv[2] = {Ct.x, Ct.y};
#pragma unroll
          for (int j = 0; j < 2; ++j) gs[j] = fmaf(gy, Cv[j], gs[j]) * fast_exp2(dtv * A2[j]);
        }
      }
    }
  }

  // du / ddt of the tile at t0, summed over the waves from their LDS partials
  // and accumulated over passes: thread = (channel rs, steps cs..cs+3)
  // dgy: D gy of those steps (the skip's share of du), zero without a skip
  auto finish_dudt = [&](const int t0, const float4 dgy) {
    const int t = t0 + cs;
    if (!rs_ok || t >= a.L) return;
    float4 su = make_float4(0.f, 0.f, 0.f, 0.f), sd = su;
    for (int v = 0; v < nw; ++v) {
      const float4 pu = *reinterpret_cast<const float4*>(s_du + (v * ROWS + rs) * TT + du_col(rs, cs));
      const float4 pd = *reinterpret_cast<const float4*>(s_ddt + (v * ROWS + rs) * TT + du_col(rs, cs));
      su.x += pu.x;
      su.y += pu.y;
      su.z += pu.z;
      su.w += pu.w;
      sd.x += pd.x;
      sd.y += pd.y;
      sd.z += pd.z;
      sd.w += pd.w;
    }
    if constexpr (SKIP) {
      su.x += dgy.x;
      su.y += dgy.y;
      su.z += dgy.z;
      su.w += dgy.w;
    }
    const uint32_t off = roff + static_cast<uint32_t>(t);
    if (!a.first) {
      const float* pu = a.du_acc + rowbase;
      const float* pd = a.ddt_acc + rowbase;
      su.x += pu[off];
      sd.x += pd[off];
      if (t + 1 < a.L) { su.y += pu[off + 1]; sd.y += pd[off + 1]; }
      if (t + 2 < a.L) { su.z += pu[off + 2]; sd.z += pd[off + 2]; }
      if (t + 3 < a.L) { su.w += pu[off + 3]; sd.w += pd[off + 3]; }
    }
    if (a.last) {
      store_row4<VEC>(a.du + rowbase, off, t, a.L, su);
      store_row4<VEC>(a.ddt + rowbase, off, t, a.L, sd);
    } else {
      store_row4<VEC>(a.du_acc + rowbase, off, t, a.L, su);
      store_row4<VEC>(a.ddt_acc + rowbase, off, t, a.L, sd);
    }
  };

  // D gy of this thread's staged steps of tile t0 (staged now), SKIP first pass only
  auto skip_dgy = [&](const int t0) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (SKIP) {
      if (a.first && t0 >= 0) {
        const float* gq = s_gy + rs * RS + cs;
        const float Dd = s_dsk[rs];
        v = make_float4(Dd * gq[0], Dd * gq[1], Dd * gq[2], Dd * gq[3]);
      }
    }
    return v;
  };

  BwdTile2 nxt;
  int prev_t0 = -1;  // the tile whose du / ddt are still to be finished
  bwd2_prefetch<E, VEC, GATED>(nxt, a, g, roff, cs, ckoff, n0, vec2, tile_hi - 1);
  for (int tile = tile_hi - 1; tile >= tile_lo; --tile) {
    const int t0 = tile * TT;
    const int nsteps = min(TT, a.L - t0);
    balance_priority(tile - tile_lo + 1, tile_hi - tile_lo);
    __syncthreads();  // the previous tile's LDS readers are done
    // SKIP: D gy of the previous tile, read before the staging below replaces
    // its gy (a thread reads only the s_gy slots that it stages itself)
    const float4 dgy_prev = skip_dgy(prev_t0);
    b2_put_dtu(s_dtu + rs * RS2 + 2 * cs, b2_mask(nxt.dt, rs_ok, t0 + cs, a.L),
               b2_mask(nxt.u, rs_ok, t0 + cs, a.L));
    b2_store_bc(s_BC, nxt.B, nxt.C, t0, a.L, a.N, a.n_base);
    // gated upstream gradient into LDS; the first pass also writes dz
    float4 dz_v = make_float4(0.f, 0.f, 0.f, 0.f);
    bool dz_ok = false;
    {
      float4 gy = b2_mask(nxt.go, rs_ok, t0 + cs, a.L);
      if constexpr (GATED) {
        const float4 zz = nxt.z, go = gy;
        const float4 sg = make_float4(sigmoid(zz.x), sigmoid(zz.y), sigmoid(zz.z), sigmoid(zz.w));
        gy = make_float4(go.x * zz.x * sg.x, go.y * zz.y * sg.y, go.z * zz.z * sg.z, go.w * zz.w * sg.w);
        if (a.first && rs_ok && t0 + cs < a.L) {
          const float4 y = nxt.raw;
          dz_v = make_float4(go.x * y.x * (sg.x * (1.f + zz.x * (1.f - sg.x))),
                             go.y * y.y * (sg.y * (1.f + zz.y * (1.f - sg.y))),
                             go.z * y.z * (sg.z * (1.f + zz.z * (1.f - sg.z))),
                             go.w * y.w * (sg.w * (1.f + zz.w * (1.f - sg.w))));
          dz_ok = true;
        }
      }
      b2_put(s_gy + rs * RS + cs, gy);
      if constexpr (SKIP) {
        if (a.first) {  // gy u of the staged steps into this thread's dD sum
          const float4 uu = b2_mask(nxt.u, rs_ok, t0 + cs, a.L);
          s_dsum[threadIdx.x] =
              fmaf(gy.x, uu.x, fmaf(gy.y, uu.y, fmaf(gy.z, uu.z, fmaf(gy.w, uu.w, s_dsum[threadIdx.x]))));
        }
      }
    }
    float h0[2], hm[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bool ok = dvalid && n0 + j < a.N;
      h0[j] = (tile > 0 && ok) ? nxt.h0[j] : 0.f;
      hm[j] = ok ? nxt.hm[j] : 0.f;
    }
    // the next tile's loads go out before this interval's stores (dz, and
    // du / ddt of the previous tile, whose LDS partials this barrier interval
    // still holds)
    if (tile > tile_lo) bwd2_prefetch<E, VEC, GATED>(nxt, a, g, roff, cs, ckoff, n0, vec2, tile - 1);
    if (dz_ok) store_row4<VEC>(a.dz + rowbase, roff + static_cast<uint32_t>(t0 + cs), t0 + cs, a.L, dz_v);
    if (prev_t0 >= 0) finish_dudt(prev_t0, dgy_prev);
    __syncthreads();

    if (wave_active) {
      const float* dturow = s_dtu + c * RS2;
      const float* gyrow = s_gy + c * RS;
      const float* BCrow = s_BC + (2 * w + hi) * 4;  // this lane's state pair
      float* durow = (hi ? s_ddt : s_du) + (w * ROWS + c) * TT;
      const int du_rot = (c >> 1) & 7;  // du_col(c, 4 G) = (G ^ du_rot) << 2
      // keep[m]: this lane's share of the dB / dC tile partials of steps
      // 8m .. 8m + 7 (see reduce4_32 for which lane holds which total)
      float keep[4] = {0.f, 0.f, 0.f, 0.f};

      // forward over steps s0 .. s0 + HT - 1 from the state before s0: the
      // state after each step and its exp(dt A), in registers; operands read
      // one step ahead, the empty asm keeping the reads from being hoisted
      auto forward_half = [&](auto s0_tag, const float (&hst)[2], float (&hs)[HT][2], float (&dAs)[HT][2]) {
        constexpr int s0 = decltype(s0_tag)::value;
        float h[2] = {hst[0], hst[1]};
        float2 ndu = *reinterpret_cast<const float2*>(dturow + 2 * s0);
        float2 nB = *reinterpret_cast<const float2*>(BCrow + 32 * s0);
#pragma unroll
        for (int i = 0; i < HT; ++i) {
          const float dtv = ndu.x, uv = ndu.y;
          const float Bv[2] = {nB.x, nB.y};
          if (i + 1 < HT) {
            ndu = *reinterpret_cast<const float2*>(dturow + 2 * (s0 + i + 1));
            nB = *reinterpret_cast<const float2*>(BCrow + 32 * (s0 + i + 1));
          }
          const float dtu = dtv * uv;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float dA = fast_exp2(dtv * A2[j]);
            h[j] = fmaf(dA, h[j], dtu * Bv[j]);
            hs[i][j] = h[j];
            dAs[i][j] = dA;
          }
          asm volatile("" ::: "memory");
        }
      };
      // the adjoint over the same steps in reverse
      auto adjoint_half = [&](auto s0_tag, const float (&hst)[2], const float (&hs)[HT][2],
                              const float (&dAs)[HT][2]) {
        constexpr int s0 = decltype(s0_tag)::value;
        constexpr int il = HT - 1;
        float ngy = gyrow[s0 + il];
        float2 ndu = *reinterpret_cast<const float2*>(dturow + 2 * (s0 + il));
        float4 nBC = *reinterpret_cast<const float4*>(BCrow + 32 * (s0 + il));
        float du4[4], dd4[4];
#pragma unroll
        for (int i = il; i >= 0; --i) {
          const float gy = ngy, dtv = ndu.x, uv = ndu.y;
          const float Bv[2] = {nBC.x, nBC.y};
          const float Cv[2] = {nBC.z, nBC.w};
          if (i > 0) {
            ngy = gyrow[s0 + i - 1];
            ndu = *reinterpret_cast<const float2*>(dturow + 2 * (s0 + i - 1));
            nBC = *reinterpret_cast<const float4*>(BCrow + 32 * (s0 + i - 1));
          }
          const float dtu = dtv * uv;
          float S1 = 0.f, S2 = 0.f;
          float v[4];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float hprev = i > 0 ? hs[i > 0 ? i - 1 : 0][j] : hst[j];
            const float gacc = fmaf(gy, Cv[j], gs[j]);
            const float gsn = gacc * dAs[i][j];
            const float q = gsn * hprev;
            gA[j] = fmaf(dtv, q, gA[j]);
            S2 = fmaf(Af[j], q, S2);
            S1 = fmaf(gacc, Bv[j], S1);
            v[j] = gacc * dtu;         // dB contribution
            v[2 + j] = gy * hs[i][j];  // dC contribution
            gs[j] = gsn;
          }
          du4[i & 3] = dtv * S1;
          dd4[i & 3] = fmaf(uv, S1, S2);
          if ((i & 3) == 0) {
            // over the wave's two pairs: lanes 0..31 keep du, 32..63 ddt
            float x[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              float pu = du4[k], pd = dd4[k];
              swap32(pu, pd);
              x[k] = pu + pd;
            }
            // the column formed here, not hoisted: eight loop-invariant
            // addresses would be held across the tile (and spilled)
            int rot = du_rot;
            asm volatile("" : "+v"(rot));
            *reinterpret_cast<float4*>(durow + ((((s0 + i) >> 2) ^ rot) << 2)) =
                make_float4(x[0], x[1], x[2], x[3]);
          }
          const float o = reduce4_32(v);
          if ((lane & 7) == (i & 7)) keep[s0 / 8 + (i >> 3)] = o;
          asm volatile("" ::: "memory");
        }
      };

      // the second half first (from the checkpoint after step HT - 1), then
      // the first; a tile that ends within its first half skips the second
      if (nsteps > HT) {
        float hs[HT][2], dAs[HT][2];
        forward_half(std::integral_constant<int, HT>{}, hm, hs, dAs);
        adjoint_half(std::integral_constant<int, HT>{}, hm, hs, dAs);
      }
      {
        float hs[HT][2], dAs[HT][2];
        forward_half(std::integral_constant<int, 0>{}, h0, hs, dAs);
        adjoint_half(std::integral_constant<int, 0>{}, h0, hs, dAs);
      }

      // lane l holds in keep[m] the tile partial of step t0 + 8m + (l & 7):
      // dB (low half of its row) or dC (high half) of state n_base + 4w + l / 16
      const int n = a.n_base + 4 * w + (lane >> 4), c8 = lane & 7;
      if (n < a.N) {
        float* dst = (((lane >> 3) & 1) ? a.part_dC : a.part_dB) +
                     (static_cast<size_t>(blockIdx.x) * a.Bsz + b) * a.L * a.N;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int st = 8 * m + c8;
          if (st < nsteps) dst[static_cast<uint32_t>((t0 + st) * a.N + n)] = keep[m];
        }
      }
    }
    prev_t0 = t0;  // finished while the next tile is staged
  }
  __syncthreads();
  finish_dudt(prev_t0, skip_dgy(prev_t0));
  if constexpr (SKIP) {
    if (a.first) {
      // over the 8 threads (half a row of 16 lanes) that staged each channel row
      float dsum = s_dsum[threadIdx.x];
      dsum += dpp<0xB1>(dsum);   // quad_perm [1,0,3,2]
      dsum += dpp<0x4E>(dsum);   // quad_perm [2,3,0,1]
      dsum += dpp<0x141>(dsum);  // row_half_mirror
      if (cs == 0 && rs_ok) a.part_dD[(static_cast<size_t>(seg) * a.Bsz + b) * a.D + d0 + rs] = dsum;
    }
  }

  if (dvalid && wave_active) {
    float* dst = a.part_dA + ((static_cast<size_t>(seg) * a.Bsz + b) * a.D + d0) * a.N;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (n0 + j < a.N) dst[static_cast<uint32_t>(c * a.N + n0 + j)] = gA[j];
  }
}

// Adds the partials in a fixed order.  Blocks [0, n_bc_blocks): dB and dC,
// summed over the channel tiles, kFinVec consecutive elements per thread when
// `vec` (16-byte loads; n_bln % 4 == 0 and 16-byte aligned outputs), else one.
// The next n_dA_blocks blocks: dA, kFinCols columns per block, each column
// summed over `rows` partial rows (batch rows x time segments) by kFinGroups
// row groups (eight loads in flight each) and then over the groups in order
// through LDS.  The remaining blocks: dD (the skip's gradient, n_d columns)
// from part_dD the same way.
constexpr int kFinThreads = 256;
constexpr int kFinCols = 16;
constexpr int kFinGroups = kFinThreads / kFinCols;
constexpr int kFinVec = 4;

template <class E>
__global__ __launch_bounds__(kFinThreads) void selective_finish_kernel(
    const float* __restrict__ part_dB, const float* __restrict__ part_dC,
    const float* __restrict__ part_dA, E* __restrict__ dB, E* __restrict__ dC,
    float* __restrict__ dA, int64_t n_bln, int n_dtiles, int64_t n_dn, int rows, int n_bc_blocks,
    int vec, int n_dA_blocks, const float* __restrict__ part_dD, float* __restrict__ dD, int n_d) {
  if (static_cast<int>(blockIdx.x) < n_bc_blocks) {
    // tiles added in ascending order; the loads of 8 tiles are issued before
    // any of them is added (the sum stays the same, bit for bit)
    constexpr int kBatch = 8;
    if (vec) {
      const int64_t i = (static_cast<int64_t>(blockIdx.x) * kFinThreads + threadIdx.x) * kFinVec;
      if (i >= n_bln) return;
      float4 sb = make_float4(0.f, 0.f, 0.f, 0.f), sc = sb;
      auto add = [](float4& s, float4 v) {
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
      };
      int k = 0;
      for (; k + kBatch <= n_dtiles; k += kBatch) {
        float4 vb[kBatch], vc[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
          vb[q] = *reinterpret_cast<const float4*>(part_dB + static_cast<size_t>(k + q) * n_bln + i);
          vc[q] = *reinterpret_cast<const float4*>(part_dC + static_cast<size_t>(k + q) * n_bln + i);
        }
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
          add(sb, vb[q]);
          add(sc, vc[q]);
        }
      }
      for (; k < n_dtiles; ++k) {
        add(sb, *reinterpret_cast<const float4*>(part_dB + static_cast<size_t>(k) * n_bln + i));
        add(sc, *reinterpret_cast<const float4*>(part_dC + static_cast<size_t>(k) * n_bln + i));
      }
      Elem<E>::store4(dB + i, sb);
      Elem<E>::store4(dC + i, sc);
      return;
    }
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kFinThreads + threadIdx.x;
    if (i >= n_bln) return;
    float sb = 0.f, sc = 0.f;
    int k = 0;
    for (; k + kBatch <= n_dtiles; k += kBatch) {
      float vb[kBatch], vc[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        vb[q] = part_dB[static_cast<size_t>(k + q) * n_bln + i];
        vc[q] = part_dC[static_cast<size_t>(k + q) * n_bln + i];
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        sb += vb[q];
        sc += vc[q];
      }
    }
    for (; k < n_dtiles; ++k) {
      sb += part_dB[static_cast<size_t>(k) * n_bln + i];
      sc += part_dC[static_cast<size_t>(k) * n_bln + i];
    }
    Elem<E>::store1(dB + i, sb);
    Elem<E>::store1(dC + i, sc);
    return;
  }
  __shared__ float s_part[kFinGroups][kFinCols];
  const bool skip_cols = static_cast<int>(blockIdx.x) >= n_bc_blocks + n_dA_blocks;
  const float* __restrict__ part = skip_cols ? part_dD : part_dA;
  float* __restrict__ out = skip_cols ? dD : dA;
  const int64_t n_cols = skip_cols ? n_d : n_dn;
  const int c = threadIdx.x % kFinCols, grp = threadIdx.x / kFinCols;
  const int first_block = skip_cols ? n_bc_blocks + n_dA_blocks : n_bc_blocks;
  const int64_t col = static_cast<int64_t>(static_cast<int>(blockIdx.x) - first_block) * kFinCols + c;
  const int64_t cc = col < n_cols ? col : n_cols - 1;
  float s = 0.f;
  constexpr int kBatch = 8;
  int r = grp;
  for (; r + (kBatch - 1) * kFinGroups < rows; r += kBatch * kFinGroups) {
    float v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) v[q] = part[static_cast<size_t>(r + q * kFinGroups) * n_cols + cc];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) s += v[q];
  }
  for (; r < rows; r += kFinGroups) s += part[static_cast<size_t>(r) * n_cols + cc];
  s_part[grp][c] = s;
  __syncthreads();
  if (grp == 0 && col < n_cols) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < kFinGroups; ++q) t += s_part[q][c];
    out[col] = t;
  }
}

template <class E>
__global__ void selective_zero_kernel(E* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) Elem<E>::store1(p + i, 0.f);
}

int check_selective(int64_t Bsz, int64_t D, int64_t L, int64_t N, const char* what) {
  if (Bsz < 0 || D < 0 || L < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (N <= 0) return set_error(OSSM_ERR_INVALID_ARGUMENT, "state dimension must be positive");
  if (N > 256)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "state dimension exceeds supported maximum (256)");
  if (L > INT_MAX / 2 || D > INT_MAX / 2 || Bsz > 65535)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds launch limits");
  return OSSM_OK;
}

int64_t num_chunks(int64_t L) { return L <= 0 ? 0 : (L + kChunk - 1) / kChunk; }

// Rows of [.., L] tensors move four elements at a time when L % 4 == 0 and
// every row tensor starts aligned to four elements (null pointers pass).
bool rows_vectorizable(int64_t L, size_t elem_bytes, std::initializer_list<const void*> ptrs) {
  if (L % 4 != 0) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % (4 * elem_bytes) != 0) return false;
  return true;
}

template <class E>
int zero_fill(E* p, int64_t n, hipStream_t stream) {
  if (p == nullptr || n <= 0) return OSSM_OK;
  hipLaunchKernelGGL(selective_zero_kernel<E>, dim3(static_cast<unsigned>((n + 255) / 256)),
                     dim3(256), 0, stream, p, n);
  return launch_check("selective_zero_kernel");
}

// The Mamba mixer's layout: u, dt, z and the outputs as [B, L, D] (row
// strides below; outputs dense), dt before its softplus (plus an optional
// per-channel bias), B and C as [B, L, N] views with row stride ld_bc.
struct MambaLayout {
  int64_t ld_u, ld_dt, ld_z, ld_bc;
  const float* dt_bias;
};

bool aligned_to(const void* p, size_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; }

// 16-byte moves along the channels: D and every row stride a multiple of 4
// and every tensor 16-byte aligned (null pointers pass).
bool cols_vectorizable(int64_t D, const MambaLayout& ml, std::initializer_list<const void*> ptrs) {
  if (D % 4 != 0 || ml.ld_u % 4 != 0 || ml.ld_dt % 4 != 0 || ml.ld_z % 4 != 0) return false;
  for (const void* p : ptrs)
    if (!aligned_to(p, 16)) return false;
  return true;
}

// Time segments per (batch row, channel tile), 1, 2 or 4: the fewest that
// give at least `want` workgroups per compute unit, with every segment at
// least two tiles long.  OSSM_SEL_SPLIT=1|2|4 overrides.  Segment s re-runs
// the recurrence of the other segments it depends on (h only forward, the
// adjoint only backward) before its own tiles.
int time_segments(int64_t n_wg, int64_t L, int tile, int want) {
  static const int forced = [] {
    const char* v = std::getenv("OSSM_SEL_SPLIT");
    return v == nullptr ? 0 : std::atoi(v);
  }();
  const int64_t n_tiles = (L + tile - 1) / tile;
  int n_cu = 0;
  if (forced == 1 || forced == 2 || forced == 4) {
    n_cu = 1;
  } else {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n_cu <= 0)
      return 1;
  }
  int s = 1;
  while (s < 4 && n_tiles >= 4 * s &&
         (forced ? s < forced : n_wg * s < static_cast<int64_t>(want) * n_cu))
    s *= 2;
  return s;
}

// The 2-states-per-lane backward addresses everything as a workgroup base
// plus a 32-bit (int) offset.
bool bwd2_offsets_fit(int64_t L, int64_t N, int64_t ld_bc) {
  const int64_t lim = INT_MAX;
  return kB2Rows * L < lim && L * std::max(N, ld_bc) < lim &&
         kB2Rows * num_chunks(L) * 2 * N < lim;
}

// States per lane of the [B, D, L] backward for `rows64` (batch row,
// 64-channel) rows: 4 (two 64-channel workgroups per compute unit) while that
// fills the device without a time split, 2 below (32-channel workgroups,
// three per compute unit: twice the workgroups at 1.5x the occupancy).
// OSSM_SEL_BWD_NPW=2|4 overrides.
int bwd_states_per_lane(int64_t rows64) {
  const char* env = std::getenv("OSSM_SEL_BWD_NPW");  // read per call: tests switch it
  const int forced = env == nullptr ? 0 : std::atoi(env);
  if (forced == 2 || forced == 4) return forced;
  int dev = 0, n_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
    return 4;
  return rows64 < static_cast<int64_t>(kBwdWgPerCu) * n_cu ? 2 : 4;
}

// States per lane of the [B, D, L] forward for `rows64` (batch row, 64-channel)
// rows: 2 while 64-channel workgroups would give fewer than kFwdNpw2Below
// waves per SIMD (OSSM_SEL_FWD_NPW=2|4 overrides).
#ifndef OSSM_SEL_FWD_NPW2_BELOW
#define OSSM_SEL_FWD_NPW2_BELOW 4
#endif
int fwd_states_per_lane(int64_t rows64) {
  const char* env = std::getenv("OSSM_SEL_FWD_NPW");  // read per call: tests switch it
  const int forced = env == nullptr ? 0 : std::atoi(env);
  if (forced == 2 || forced == 4) return forced;
  int dev = 0, n_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n_cu <= 0)
    return 4;
  // kMaxWaves waves per workgroup over 4 SIMDs per CU
  return rows64 * kMaxWaves < static_cast<int64_t>(OSSM_SEL_FWD_NPW2_BELOW) * 4 * n_cu ? 2 : 4;
}

// E = float: the fp32 API of the reference.  E = bf16_t: the same scan with
// bf16 rows, B and C in HBM (A, chunk_states and dA stay fp32).  ml: the
// [B, L, D] layout (fp32 only); null for the reference's [B, D, L].  dskip:
// the extended API's per-channel skip D ([B, D, L] only), null for none.
template <class E>
int selective_forward_impl(const E* u, const E* dt, const float* A, const E* Bm, const E* Cm,
                           const E* gate, E* out, E* raw_out, float* chunk_states, int64_t batch,
                           int64_t dim, int64_t length, int64_t dstate, hipStream_t stream,
                           const char* what, const MambaLayout* ml = nullptr,
                           const float* dskip = nullptr) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  clear_error();
  if (int rc = check_selective(batch, dim, length, dstate, what)) return rc;
  if (batch == 0 || dim == 0 || length == 0) return OSSM_OK;
  if (!u || !dt || !A || !Bm || !Cm || !out)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  if (dskip != nullptr && ml != nullptr)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": the skip D is for the [B, D, L] layout");
  const int n_pass = static_cast<int>((dstate + kPassStates - 1) / kPassStates);
  FwdArgs<E> a{};
  a.dskip = dskip;
  a.u = u;
  a.dt = dt;
  a.A = A;
  a.Bm = Bm;
  a.Cm = Cm;
  a.z = gate;
  a.out = out;
  a.raw = raw_out;
  a.acc = nullptr;
  if (n_pass > 1) {
    if constexpr (std::is_same_v<E, float>) {
      a.acc = raw_out != nullptr ? raw_out : out;  // summed in place, then overwritten
    } else {
      void* ws = nullptr;
      if (int rc = acquire_workspace(call, static_cast<size_t>(batch * dim * length) * sizeof(float), &ws))
        return rc;
      a.acc = static_cast<float*>(ws);
    }
  }
  a.ckpt = chunk_states;
  a.D = static_cast<int>(dim);
  a.L = static_cast<int>(length);
  a.N = static_cast<int>(dstate);
  a.n_chunks = static_cast<int>(num_chunks(length));
  a.ld_bc = static_cast<int>(dstate);
  if (ml != nullptr) {
    a.ld_bc = static_cast<int>(ml->ld_bc);
    a.ld_u = static_cast<int>(ml->ld_u);
    a.ld_dt = static_cast<int>(ml->ld_dt);
    a.ld_z = static_cast<int>(ml->ld_z);
    a.dt_bias = ml->dt_bias;
    a.vec = cols_vectorizable(dim, *ml, {u, dt, gate, out, raw_out}) ? 1 : 0;
  } else {
    a.vec = rows_vectorizable(length, sizeof(E), {u, dt, gate, out, raw_out}) ? 1 : 0;
  }
  // states per lane: 2 (32-channel workgroups) when 64-channel workgroups
  // would leave the SIMDs short of waves, else 4; the [B, L, D] layout runs 4
  const int npw = ml != nullptr ? 4 : fwd_states_per_lane(((dim + kWave - 1) / kWave) * batch);
  const int rows = npw == 4 ? FwdLayout<4>::kRows : FwdLayout<2>::kRows;
  const int64_t n_dtiles = (dim + rows - 1) / rows;
  const int n_seg = time_segments(n_dtiles * batch, length, kFwdTile, kFwdWgPerCu);
  const dim3 grid(static_cast<unsigned>(n_dtiles), static_cast<unsigned>(batch),
                  static_cast<unsigned>(n_seg));
  for (int p = 0; p < n_pass; ++p) {
    a.n_base = p * kPassStates;
    a.first = p == 0;
    a.last = p == n_pass - 1;
    using K = void (*)(FwdArgs<E>);
    K kern;
    if (ml != nullptr) {
      if constexpr (std::is_same_v<E, float>) {
        kern = a.vec ? (gate ? selective_fwd_kernel<E, true, true, true, 4> : selective_fwd_kernel<E, true, false, true, 4>)
                     : (gate ? selective_fwd_kernel<E, false, true, true, 4> : selective_fwd_kernel<E, false, false, true, 4>);
      } else {
        return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": the [B, L, D] layout is fp32");
      }
    } else if (npw == 4) {
      kern = a.vec ? (gate ? selective_fwd_kernel<E, true, true, false, 4> : selective_fwd_kernel<E, true, false, false, 4>)
                   : (gate ? selective_fwd_kernel<E, false, true, false, 4> : selective_fwd_kernel<E, false, false, false, 4>);
    } else {
      kern = a.vec ? (gate ? selective_fwd_kernel<E, true, true, false, 2> : selective_fwd_kernel<E, true, false, false, 2>)
                   : (gate ? selective_fwd_kernel<E, false, true, false, 2> : selective_fwd_kernel<E, false, false, false, 2>);
    }
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, stream, a);
    if (int rc = launch_check("selective_fwd_kernel")) return rc;
  }
  return OSSM_OK;
}

template <class E>
int selective_backward_impl(const E* grad_out, const E* u, const E* dt, const float* A,
                            const E* Bm, const E* Cm, const E* gate, const float* chunk_states,
                            const E* raw_out, E* du, E* ddt, float* dA, E* dB, E* dC, E* dgate,
                            int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                            hipStream_t stream, const char* what,
                            const MambaLayout* ml = nullptr, const float* dskip = nullptr,
                            float* dD = nullptr) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  clear_error();
  if (int rc = check_selective(batch, dim, length, dstate, what)) return rc;
  if ((dskip == nullptr) != (dD == nullptr))
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": give the skip D and dD together");
  if (dskip != nullptr && ml != nullptr)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": the skip D is for the [B, D, L] layout");
  if (batch == 0 || dim == 0 || length == 0) {
    // nothing to scan: every gradient is zero (dA still has D*N entries)
    if (int rc = zero_fill(dD, dim, stream)) return rc;
    if (int rc = zero_fill(dA, dim * dstate, stream)) return rc;
    if (int rc = zero_fill(dB, batch * length * dstate, stream)) return rc;
    if (int rc = zero_fill(dC, batch * length * dstate, stream)) return rc;
    return OSSM_OK;
  }
  if (!grad_out || !u || !dt || !A || !Bm || !Cm || !chunk_states || !du || !ddt || !dA || !dB ||
      !dC)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  if (gate != nullptr && (raw_out == nullptr || dgate == nullptr))
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     std::string(what) + ": a gated scan needs raw_outputs and dgate");
  const int n_pass = static_cast<int>((dstate + kPassStates - 1) / kPassStates);
  // [B, D, L]: 2 states per lane (32-channel workgroups) or 4 (64-channel)
  const bool npw2 = ml == nullptr && bwd2_offsets_fit(length, dstate, dstate) &&
                    bwd_states_per_lane(batch * ((dim + kWave - 1) / kWave)) == 2;
  const int64_t wg_rows = npw2 ? kB2Rows : kWave;
  const int64_t n_dtiles = (dim + wg_rows - 1) / wg_rows;
  const int64_t n_bln = batch * length * dstate;
  const int64_t n_dn = dim * dstate;
  const int64_t n_rows = batch * dim * length;
  const bool staged = !std::is_same_v<E, float> && n_pass > 1;  // fp32 du/ddt between passes
  const int n_seg = npw2 ? time_segments(n_dtiles * batch, length, kB2Tile, kBwd2WgPerCu)
                         : time_segments(n_dtiles * batch, length, kBwdTile, kBwdWgPerCu);
  const int64_t dA_rows = n_seg * batch;  // dA partial rows: (segment, batch row)
  const size_t part_floats = static_cast<size_t>(2 * n_dtiles * n_bln + dA_rows * n_dn) +
                            (staged ? 2 * n_rows : 0) + (dskip ? dA_rows * dim : 0);
  void* ws = nullptr;
  if (int rc = acquire_workspace(call, part_floats * sizeof(float), &ws)) return rc;
  float* part_dB = static_cast<float*>(ws);
  float* part_dC = part_dB + n_dtiles * n_bln;
  float* part_dA = part_dC + n_dtiles * n_bln;
  // after part_dA and the staged fp32 du / ddt
  float* part_dD = dskip ? part_dA + dA_rows * n_dn + (staged ? 2 * n_rows : 0) : nullptr;

  BwdArgs<E> a{};
  a.gout = grad_out;
  a.u = u;
  a.dt = dt;
  a.A = A;
  a.Bm = Bm;
  a.Cm = Cm;
  a.z = gate;
  a.raw = raw_out;
  a.ckpt = chunk_states;
  a.du = du;
  a.ddt = ddt;
  a.dz = dgate;
  if constexpr (std::is_same_v<E, float>) {
    a.du_acc = du;  // summed in place
    a.ddt_acc = ddt;
  } else {
    a.du_acc = staged ? part_dA + dA_rows * n_dn : nullptr;
    a.ddt_acc = staged ? a.du_acc + n_rows : nullptr;
  }
  a.part_dB = part_dB;
  a.part_dC = part_dC;
  a.part_dA = part_dA;
  a.dskip = dskip;
  a.part_dD = part_dD;
  a.Bsz = static_cast<int>(batch);
  a.D = static_cast<int>(dim);
  a.L = static_cast<int>(length);
  a.N = static_cast<int>(dstate);
  a.n_chunks = static_cast<int>(num_chunks(length));
  // the staged fp32 sums sit at a 16-byte multiple only when n_bln and B*D*N are
  // multiples of 4; otherwise the rows go element by element
  const bool staged_aligned = !staged || (n_bln % 4 == 0 && (dA_rows * n_dn) % 4 == 0);
  a.ld_bc = static_cast<int>(dstate);
  if (ml != nullptr) {
    a.ld_bc = static_cast<int>(ml->ld_bc);
    a.ld_u = static_cast<int>(ml->ld_u);
    a.ld_dt = static_cast<int>(ml->ld_dt);
    a.ld_z = static_cast<int>(ml->ld_z);
    a.dt_bias = ml->dt_bias;
    a.vec = cols_vectorizable(dim, *ml, {grad_out, u, dt, gate, raw_out, du, ddt, dgate}) ? 1 : 0;
  } else {
    a.vec = staged_aligned &&
                    rows_vectorizable(length, sizeof(E), {grad_out, u, dt, gate, raw_out, du, ddt, dgate})
                ? 1
                : 0;
  }
  const dim3 grid(static_cast<unsigned>(n_dtiles), static_cast<unsigned>(batch),
                  static_cast<unsigned>(n_seg));
  for (int p = 0; p < n_pass; ++p) {
    a.n_base = p * kPassStates;
    a.first = p == 0;
    a.last = p == n_pass - 1;
    using K = void (*)(BwdArgs<E>);
    K kern;
    if (npw2 && dskip != nullptr) {
      kern = a.vec ? (gate ? selective_bwd2_kernel<E, true, true, true> : selective_bwd2_kernel<E, true, false, true>)
                   : (gate ? selective_bwd2_kernel<E, false, true, true> : selective_bwd2_kernel<E, false, false, true>);
    } else if (npw2) {
      kern = a.vec ? (gate ? selective_bwd2_kernel<E, true, true, false> : selective_bwd2_kernel<E, true, false, false>)
                   : (gate ? selective_bwd2_kernel<E, false, true, false> : selective_bwd2_kernel<E, false, false, false>);
    } else if (ml != nullptr) {
      if constexpr (std::is_same_v<E, float>) {
        kern = a.vec ? (gate ? selective_bwd_kernel<E, true, true, true, false> : selective_bwd_kernel<E, true, false, true, false>)
                     : (gate ? selective_bwd_kernel<E, false, true, true, false> : selective_bwd_kernel<E, false, false, true, false>);
      } else {
        return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": the [B, L, D] layout is fp32");
      }
    } else if (dskip != nullptr) {
      kern = a.vec ? (gate ? selective_bwd_kernel<E, true, true, false, true> : selective_bwd_kernel<E, true, false, false, true>)
                   : (gate ? selective_bwd_kernel<E, false, true, false, true> : selective_bwd_kernel<E, false, false, false, true>);
    } else {
      kern = a.vec ? (gate ? selective_bwd_kernel<E, true, true, false, false> : selective_bwd_kernel<E, true, false, false, false>)
                   : (gate ? selective_bwd_kernel<E, false, true, false, false> : selective_bwd_kernel<E, false, false, false, false>);
    }
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, stream, a);
    if (int rc = launch_check("selective_bwd_kernel")) return rc;
  }
  const int fin_vec = n_bln % kFinVec == 0 && aligned_to(dB, kFinVec * sizeof(E)) &&
                      aligned_to(dC, kFinVec * sizeof(E));
  const int64_t per_block = static_cast<int64_t>(kFinThreads) * (fin_vec ? kFinVec : 1);
  const int64_t n_bc_blocks = (n_bln + per_block - 1) / per_block;
  const int64_t n_dA_blocks = (n_dn + kFinCols - 1) / kFinCols;
  const int64_t n_dD_blocks = dskip ? (dim + kFinCols - 1) / kFinCols : 0;
  hipLaunchKernelGGL(selective_finish_kernel<E>,
                     dim3(static_cast<unsigned>(n_bc_blocks + n_dA_blocks + n_dD_blocks)),
                     dim3(kFinThreads), 0, stream, part_dB, part_dC, part_dA, dB, dC, dA, n_bln,
                     static_cast<int>(n_dtiles), n_dn, static_cast<int>(dA_rows),
                     static_cast<int>(n_bc_blocks), fin_vec, static_cast<int>(n_dA_blocks), part_dD,
                     dD, static_cast<int>(dim));
  if (int rc = launch_check("selective_finish_kernel")) return rc;
  if (gate == nullptr && dgate != nullptr) return zero_fill(dgate, n_rows, stream);
  return OSSM_OK;
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int64_t ossm_selective_num_chunks(int64_t length) { return ossm::num_chunks(length); }

int ossm_selective_forward(const float* u, const float* dt, const float* A, const float* Bm,
                           const float* Cm, const float* gate, float* out, float* raw_out,
                           float* chunk_states, int64_t batch, int64_t dim, int64_t length,
                           int64_t dstate, ossm_stream_t stream) {
  return selective_forward_impl<float>(u, dt, A, Bm, Cm, gate, out, raw_out, chunk_states, batch,
                                       dim, length, dstate, static_cast<hipStream_t>(stream),
                                       "selective_forward");
}

int ossm_selective_backward(const float* grad_out, const float* u, const float* dt, const float* A,
                            const float* Bm, const float* Cm, const float* gate,
                            const float* chunk_states, const float* raw_out, float* du, float* ddt,
                            float* dA, float* dB, float* dC, float* dgate, int64_t batch,
                            int64_t dim, int64_t length, int64_t dstate, ossm_stream_t stream) {
  return selective_backward_impl<float>(grad_out, u, dt, A, Bm, Cm, gate, chunk_states, raw_out, du,
                                        ddt, dA, dB, dC, dgate, batch, dim, length, dstate,
                                        static_cast<hipStream_t>(stream), "selective_backward");
}

// Row strides of the [B, L, D] layout: at least D (and N for B and C).
static int check_mamba_strides(int64_t D, int64_t N, int64_t ld_u, int64_t ld_dt, int64_t ld_z,
                               bool gated, int64_t ld_bc, const char* what) {
  if (ld_u < D || ld_dt < D || (gated && ld_z < D) || ld_bc < N || ld_u > INT_MAX ||
      ld_dt > INT_MAX || ld_z > INT_MAX || ld_bc > INT_MAX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     std::string(what) + ": row strides must be at least the row length");
  return OSSM_OK;
}

int ossm_selective_mamba_forward(const float* u, int64_t ld_u, const float* dt, int64_t ld_dt,
                                 const float* dt_bias, const float* A, const float* Bm,
                                 const float* Cm, int64_t ld_bc, const float* gate, int64_t ld_z,
                                 float* out, float* raw_out, float* chunk_states, int64_t batch,
                                 int64_t dim, int64_t length, int64_t dstate, ossm_stream_t stream) {
  const char* what = "selective_mamba_forward";
  clear_error();
  if (dstate > 0)
    if (int rc = check_mamba_strides(dim, dstate, ld_u, ld_dt, ld_z, gate != nullptr, ld_bc, what))
      return rc;
  const MambaLayout ml{ld_u, ld_dt, gate != nullptr ? ld_z : dim, ld_bc, dt_bias};
  return selective_forward_impl<float>(u, dt, A, Bm, Cm, gate, out, raw_out, chunk_states, batch,
                                       dim, length, dstate, static_cast<hipStream_t>(stream), what,
                                       &ml);
}

int ossm_selective_mamba_backward(const float* grad_out, const float* u, int64_t ld_u,
                                  const float* dt, int64_t ld_dt, const float* dt_bias,
                                  const float* A, const float* Bm, const float* Cm, int64_t ld_bc,
                                  const float* gate, int64_t ld_z, const float* chunk_states,
                                  const float* raw_out, float* du, float* ddt, float* dA,
                                  float* dB, float* dC, float* dgate, int64_t batch, int64_t dim,
                                  int64_t length, int64_t dstate, ossm_stream_t stream) {
  const char* what = "selective_mamba_backward";
  clear_error();
  if (dstate > 0)
    if (int rc = check_mamba_strides(dim, dstate, ld_u, ld_dt, ld_z, gate != nullptr, ld_bc, what))
      return rc;
  const MambaLayout ml{ld_u, ld_dt, gate != nullptr ? ld_z : dim, ld_bc, dt_bias};
  return selective_backward_impl<float>(grad_out, u, dt, A, Bm, Cm, gate, chunk_states, raw_out,
                                        du, ddt, dA, dB, dC, dgate, batch, dim, length, dstate,
                                        static_cast<hipStream_t>(stream), what, &ml);
}

int ossm_selective_forward_bf16(const void* u, const void* dt, const float* A, const void* Bm,
                                const void* Cm, const void* gate, void* out, void* raw_out,
                                float* chunk_states, int64_t batch, int64_t dim, int64_t length,
                                int64_t dstate, ossm_stream_t stream) {
  using E = bf16_t;
  return selective_forward_impl<E>(
      static_cast<const E*>(u), static_cast<const E*>(dt), A, static_cast<const E*>(Bm),
      static_cast<const E*>(Cm), static_cast<const E*>(gate), static_cast<E*>(out),
      static_cast<E*>(raw_out), chunk_states, batch, dim, length, dstate,
      static_cast<hipStream_t>(stream), "selective_forward_bf16");
}

int ossm_selective_backward_bf16(const void* grad_out, const void* u, const void* dt,
                                 const float* A, const void* Bm, const void* Cm, const void* gate,
                                 const float* chunk_states, const void* raw_out, void* du,
                                 void* ddt, float* dA, void* dB, void* dC, void* dgate,
                                 int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                                 ossm_stream_t stream) {
  using E = bf16_t;
  return selective_backward_impl<E>(
      static_cast<const E*>(grad_out), static_cast<const E*>(u), static_cast<const E*>(dt), A,
      static_cast<const E*>(Bm), static_cast<const E*>(Cm), static_cast<const E*>(gate),
      chunk_states, static_cast<const E*>(raw_out), static_cast<E*>(du), static_cast<E*>(ddt), dA,
      static_cast<E*>(dB), static_cast<E*>(dC), static_cast<E*>(dgate), batch, dim, length, dstate,
      static_cast<hipStream_t>(stream), "selective_backward_bf16");
}

int ossm_selective_forward_skip(int elem, const void* u, const void* dt, const float* A,
                                const void* Bm, const void* Cm, const float* d_skip,
                                const void* gate, void* out, void* raw_out, float* chunk_states,
                                int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                                ossm_stream_t stream) {
  const char* what = "selective_forward_skip";
  clear_error();
  if (d_skip == nullptr) return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null skip D");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (elem == OSSM_ELEM_F32) {
    using E = float;
    return selective_forward_impl<E>(
        static_cast<const E*>(u), static_cast<const E*>(dt), A, static_cast<const E*>(Bm),
        static_cast<const E*>(Cm), static_cast<const E*>(gate), static_cast<E*>(out),
        static_cast<E*>(raw_out), chunk_states, batch, dim, length, dstate, st, what, nullptr, d_skip);
  }
  if (elem == OSSM_ELEM_BF16) {
    using E = bf16_t;
    return selective_forward_impl<E>(
        static_cast<const E*>(u), static_cast<const E*>(dt), A, static_cast<const E*>(Bm),
        static_cast<const E*>(Cm), static_cast<const E*>(gate), static_cast<E*>(out),
        static_cast<E*>(raw_out), chunk_states, batch, dim, length, dstate, st, what, nullptr, d_skip);
  }
  return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": unknown element type");
}

int ossm_selective_backward_skip(int elem, const void* grad_out, const void* u, const void* dt,
                                 const float* A, const void* Bm, const void* Cm,
                                 const float* d_skip, const void* gate, const float* chunk_states,
                                 const void* raw_out, void* du, void* ddt, float* dA, void* dB,
                                 void* dC, float* dD, void* dgate, int64_t batch, int64_t dim,
                                 int64_t length, int64_t dstate, ossm_stream_t stream) {
  const char* what = "selective_backward_skip";
  clear_error();
  if (d_skip == nullptr || dD == nullptr)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null skip D or dD");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (elem == OSSM_ELEM_F32) {
    using E = float;
    return selective_backward_impl<E>(
        static_cast<const E*>(grad_out), static_cast<const E*>(u), static_cast<const E*>(dt), A,
        static_cast<const E*>(Bm), static_cast<const E*>(Cm), static_cast<const E*>(gate),
        chunk_states, static_cast<const E*>(raw_out), static_cast<E*>(du), static_cast<E*>(ddt), dA,
        static_cast<E*>(dB), static_cast<E*>(dC), static_cast<E*>(dgate), batch, dim, length, dstate,
        st, what, nullptr, d_skip, dD);
  }
  if (elem == OSSM_ELEM_BF16) {
    using E = bf16_t;
    return selective_backward_impl<E>(
        static_cast<const E*>(grad_out), static_cast<const E*>(u), static_cast<const E*>(dt), A,
        static_cast<const E*>(Bm), static_cast<const E*>(Cm), static_cast<const E*>(gate),
        chunk_states, static_cast<const E*>(raw_out), static_cast<E*>(du), static_cast<E*>(ddt), dA,
        static_cast<E*>(dB), static_cast<E*>(dC), static_cast<E*>(dgate), batch, dim, length, dstate,
        st, what, nullptr, d_skip, dD);
  }
  return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": unknown element type");
}

}  // extern "C"
