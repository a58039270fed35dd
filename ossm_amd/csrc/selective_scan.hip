// Selective (Mamba-style) scan on gfx950, forward and backward, fp32.
//
//   h_t[n] = exp(dt_t A[d,n]) h_{t-1}[n] + dt_t B_t[n] u_t,   y_t = sum_n C_t[n] h_t[n],
//   out_t  = y_t * silu(z_t)   (out = y without a gate)
// per (batch b, channel d), tensors u, dt, z, out [B,D,L]; A [D,N]; B, C [B,L,N].
//
// Parallel decomposition
//   A workgroup owns one batch row b and 64 consecutive channels d (one lane
//   per channel) and walks the whole sequence; its waves split the states:
//   wave w carries states n_base + 4w .. n_base + 4w + 3 in registers, so the
//   B/C values a wave needs at a step are the same for all its lanes (LDS
//   broadcast reads).  Up to 16 states run per launch ("pass"); larger N runs
//   ceil(N/16) passes that accumulate y (forward) and du/ddt (backward) in the
//   output tensors.  Time is processed in tiles staged through LDS: u, dt (and
//   the gated upstream gradient) are loaded with coalesced row reads and read
//   back by lane = channel.  The sum over states (y, du, ddt) is finished
//   across the waves through LDS.
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
#include <climits>
#include <cstdint>
#include <string>

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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoid(float z) { return 1.f / (1.f + __expf(-z)); }

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
// Sum over the 16 lanes of each row, result in every lane of the row.
__device__ __forceinline__ float row_allreduce(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  return v;
}
// Sums v[0..7] over all 64 lanes; lanes of row r (= lane / 16) receive the
// totals of v[2r] and v[2r+1].
__device__ __forceinline__ void reduce8(const float (&v)[8], float& o0, float& o1) {
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
  // row 0: (v0, v1), row 1: (v2, v3), row 2: (v4, v5), row 3: (v6, v7), 4-lane sums
  o0 = row_allreduce(s0 + s2);
  o1 = row_allreduce(s1 + s3);
}

// ---- tile staging -----------------------------------------------------------
// Stages rows d0..d0+63 of a [.., L] tensor, columns t0..t0+TT-1, into LDS
// s[r * RS + c] (zero outside the tensor).  `vec` = rows are 16-byte aligned
// (L % 4 == 0), then the loads are float4.
template <int TT, int RS>
__device__ __forceinline__ void stage_rows(float* __restrict__ s, const float* __restrict__ g,
                                           size_t row0, int d0, int D, int t0, int L, bool vec) {
  if (vec) {
    constexpr int C4 = TT / 4;
    for (int i = threadIdx.x; i < kWave * C4; i += blockDim.x) {
      const int r = i / C4, c = (i - r * C4) * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (d0 + r < D && t0 + c < L)
        v = *reinterpret_cast<const float4*>(g + row0 + static_cast<size_t>(d0 + r) * L + t0 + c);
      float* p = s + r * RS + c;
      p[0] = v.x;
      p[1] = v.y;
      p[2] = v.z;
      p[3] = v.w;
    }
  } else {
    for (int i = threadIdx.x; i < kWave * TT; i += blockDim.x) {
      const int r = i / TT, c = i - r * TT;
      float v = 0.f;
      if (d0 + r < D && t0 + c < L) v = g[row0 + static_cast<size_t>(d0 + r) * L + t0 + c];
      s[r * RS + c] = v;
    }
  }
}

// Stages B or C rows t0..t0+TT-1, states n_base..n_base+15, into s[t * 16 + j]
// (zero outside the tensor, so padded states contribute nothing).
template <int TT>
__device__ __forceinline__ void stage_states(float* __restrict__ s, const float* __restrict__ g,
                                             size_t base, int t0, int L, int N, int n_base) {
  for (int i = threadIdx.x; i < TT * kPassStates; i += blockDim.x) {
    const int t = i / kPassStates, j = i - t * kPassStates;
    float v = 0.f;
    if (t0 + t < L && n_base + j < N) v = g[base + static_cast<size_t>(t0 + t) * N + n_base + j];
    s[i] = v;
  }
}

// ---- forward ------------------------------------------------------------------
struct FwdArgs {
  const float* u;
  const float* dt;
  const float* A;
  const float* Bm;
  const float* Cm;
  const float* z;    // may be null
  float* out;
  float* acc;        // y accumulator across passes (raw_out, or out when raw_out is null)
  float* ckpt;       // chunk_states, may be null
  int D, L, N, n_base, n_chunks;
  int first, last, vec;
};

__device__ __forceinline__ void write_ckpt(float* ckpt, size_t lane_row, int slot, int N,
                                           int n0, const float (&h)[kNpw]) {
  const int c = slot >> 1, half = slot & 1;
  float* p = ckpt + lane_row + static_cast<size_t>(c) * 2 * N + half * N;
#pragma unroll
  for (int j = 0; j < kNpw; ++j)
    if (n0 + j < N) p[n0 + j] = h[j];
}

__global__ __launch_bounds__(kMaxWaves * kWave) void selective_fwd_kernel(FwdArgs a) {
  constexpr int TT = kFwdTile;
  constexpr int RS = TT + 1;  // odd row stride: lane-per-row accesses hit distinct banks
  __shared__ float s_u[kWave * RS];
  __shared__ float s_dt[kWave * RS];
  __shared__ __align__(16) float s_B[TT * kPassStates];
  __shared__ __align__(16) float s_C[TT * kPassStates];
  __shared__ float s_y[kMaxWaves * kWave * RS];

  const int nw = blockDim.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kWave;
  const int d = d0 + lane;
  const bool dvalid = d < a.D;
  const int n0 = a.n_base + w * kNpw;  // first state of this wave

  float A2[kNpw], h[kNpw];
#pragma unroll
  for (int j = 0; j < kNpw; ++j) {
    A2[j] = (dvalid && n0 + j < a.N) ? a.A[static_cast<size_t>(d) * a.N + n0 + j] * kLog2e : 0.f;
    h[j] = 0.f;
  }
  const size_t row0 = static_cast<size_t>(b) * a.D * a.L;     // (b, 0, 0) in [B,D,L]
  const size_t bc0 = static_cast<size_t>(b) * a.L * a.N;      // (b, 0, 0) in [B,L,N]
  const size_t ck_row = (static_cast<size_t>(b) * a.D + (dvalid ? d : 0)) * a.n_chunks * 2 * a.N;
  const int n_slots = (a.L + kCkpt - 1) / kCkpt;

  for (int t0 = 0; t0 < a.L; t0 += TT) {
    __syncthreads();
    stage_rows<TT, RS>(s_u, a.u, row0, d0, a.D, t0, a.L, a.vec);
    stage_rows<TT, RS>(s_dt, a.dt, row0, d0, a.D, t0, a.L, a.vec);
    stage_states<TT>(s_B, a.Bm, bc0, t0, a.L, a.N, a.n_base);
    stage_states<TT>(s_C, a.Cm, bc0, t0, a.L, a.N, a.n_base);
    __syncthreads();

    const int nsteps = min(TT, a.L - t0);
    float* yrow = s_y + (w * kWave + lane) * RS;
#pragma unroll
    for (int i = 0; i < TT; ++i) {
      if (i < nsteps) {
        const float dtv = s_dt[lane * RS + i];
        const float dtu = dtv * s_u[lane * RS + i];
        const float4 Bt = *reinterpret_cast<const float4*>(s_B + i * kPassStates + w * kNpw);
        const float4 Ct = *reinterpret_cast<const float4*>(s_C + i * kPassStates + w * kNpw);
        const float Bv[4] = {Bt.x, Bt.y, Bt.z, Bt.w};
        const float Cv[4] = {Ct.x, Ct.y, Ct.z, Ct.w};
        float y = 0.f;
#pragma unroll
        for (int j = 0; j < kNpw; ++j) {
          const float dA = fast_exp2(dtv * A2[j]);
          h[j] = fmaf(dA, h[j], dtu * Bv[j]);
          y = fmaf(Cv[j], h[j], y);
        }
        yrow[i] = y;
        if (a.ckpt != nullptr && dvalid) {
          const int t = t0 + i;
          if ((t + 1) % kCkpt == 0 || t + 1 == a.L) {
            const int slot = t / kCkpt;
            write_ckpt(a.ckpt, ck_row, slot, a.N, n0, h);
            // an odd number of slots leaves the last row's second half: final h
            if (t + 1 == a.L && (n_slots & 1)) write_ckpt(a.ckpt, ck_row, slot + 1, a.N, n0, h);
          }
        }
      }
    }
    __syncthreads();

    // finish y over the waves (states), gate, store
    for (int i = threadIdx.x; i < kWave * TT; i += blockDim.x) {
      const int r = i / TT, c = i - r * TT;
      const int dd = d0 + r, t = t0 + c;
      if (dd >= a.D || t >= a.L) continue;
      float y = 0.f;
      for (int v = 0; v < nw; ++v) y += s_y[(v * kWave + r) * RS + c];
      const size_t gi = row0 + static_cast<size_t>(dd) * a.L + t;
      if (!a.first) y += a.acc[gi];
      if (a.last) {
        if (a.acc != a.out) a.acc[gi] = y;
        float o = y;
        if (a.z != nullptr) {
          const float zz = a.z[gi];
          o = y * (zz * sigmoid(zz));
        }
        a.out[gi] = o;
      } else {
        a.acc[gi] = y;
      }
    }
  }
}

// ---- backward -----------------------------------------------------------------
struct BwdArgs {
  const float* gout;
  const float* u;
  const float* dt;
  const float* A;
  const float* Bm;
  const float* Cm;
  const float* z;      // may be null
  const float* raw;    // y from the forward; needed when z is given
  const float* ckpt;
  float* du;
  float* ddt;
  float* dz;           // written by the first pass when z is given
  float* part_dB;      // [n_dtiles, B, L, N]
  float* part_dC;
  float* part_dA;      // [B, D, N]
  int Bsz, D, L, N, n_base, n_chunks;
  int first, vec;
};

__global__ __launch_bounds__(kMaxWaves * kWave) void selective_bwd_kernel(BwdArgs a) {
  constexpr int TT = kBwdTile;
  constexpr int RS = TT + 1;
  __shared__ float s_u[kWave * RS];
  __shared__ float s_dt[kWave * RS];
  __shared__ float s_gy[kWave * RS];
  __shared__ __align__(16) float s_B[TT * kPassStates];
  __shared__ __align__(16) float s_C[TT * kPassStates];
  __shared__ float s_du[kMaxWaves * kWave * RS];
  __shared__ float s_ddt[kMaxWaves * kWave * RS];

  const int nw = blockDim.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kWave;
  const int d = d0 + lane;
  const bool dvalid = d < a.D;
  const int n0 = a.n_base + w * kNpw;

  float A2[kNpw], Af[kNpw], gs[kNpw], gA[kNpw];
#pragma unroll
  for (int j = 0; j < kNpw; ++j) {
    Af[j] = (dvalid && n0 + j < a.N) ? a.A[static_cast<size_t>(d) * a.N + n0 + j] : 0.f;
    A2[j] = Af[j] * kLog2e;
    gs[j] = 0.f;
    gA[j] = 0.f;
  }
  const size_t row0 = static_cast<size_t>(b) * a.D * a.L;
  const size_t bc0 = static_cast<size_t>(b) * a.L * a.N;
  const size_t ck_row = (static_cast<size_t>(b) * a.D + (dvalid ? d : 0)) * a.n_chunks * 2 * a.N;
  const size_t part0 = (static_cast<size_t>(blockIdx.x) * a.Bsz + b) * a.L * a.N;
  const int n_tiles = (a.L + TT - 1) / TT;

  for (int tile = n_tiles - 1; tile >= 0; --tile) {
    const int t0 = tile * TT;
    const int nsteps = min(TT, a.L - t0);
    __syncthreads();
    stage_rows<TT, RS>(s_u, a.u, row0, d0, a.D, t0, a.L, a.vec);
    stage_rows<TT, RS>(s_dt, a.dt, row0, d0, a.D, t0, a.L, a.vec);
    stage_states<TT>(s_B, a.Bm, bc0, t0, a.L, a.N, a.n_base);
    stage_states<TT>(s_C, a.Cm, bc0, t0, a.L, a.N, a.n_base);
    // gated upstream gradient; the first pass also writes dz
    for (int i = threadIdx.x; i < kWave * TT; i += blockDim.x) {
      const int r = i / TT, c = i - r * TT;
      const int dd = d0 + r, t = t0 + c;
      float gy = 0.f;
      if (dd < a.D && t < a.L) {
        const size_t gi = row0 + static_cast<size_t>(dd) * a.L + t;
        const float go = a.gout[gi];
        gy = go;
        if (a.z != nullptr) {
          const float zz = a.z[gi];
          const float sg = sigmoid(zz);
          gy = go * (zz * sg);
          if (a.first) a.dz[gi] = go * a.raw[gi] * (sg * (1.f + zz * (1.f - sg)));
        }
      }
      s_gy[r * RS + c] = gy;
    }
    __syncthreads();

    // state after step t0 - 1 (checkpoint slot tile - 1)
    float h0[kNpw];
#pragma unroll
    for (int j = 0; j < kNpw; ++j) h0[j] = 0.f;
    if (tile > 0 && dvalid) {
      const int slot = tile - 1;
      const float* p = a.ckpt + ck_row + static_cast<size_t>(slot >> 1) * 2 * a.N + (slot & 1) * a.N;
#pragma unroll
      for (int j = 0; j < kNpw; ++j)
        if (n0 + j < a.N) h0[j] = p[n0 + j];
    }

    // re-run the tile forward in registers
    float hs[TT][kNpw], dAs[TT][kNpw];
    {
      float h[kNpw];
#pragma unroll
      for (int j = 0; j < kNpw; ++j) h[j] = h0[j];
#pragma unroll
      for (int i = 0; i < TT; ++i) {
        if (i < nsteps) {
          const float dtv = s_dt[lane * RS + i];
          const float dtu = dtv * s_u[lane * RS + i];
          const float4 Bt = *reinterpret_cast<const float4*>(s_B + i * kPassStates + w * kNpw);
          const float Bv[4] = {Bt.x, Bt.y, Bt.z, Bt.w};
#pragma unroll
          for (int j = 0; j < kNpw; ++j) {
            const float dA = fast_exp2(dtv * A2[j]);
            h[j] = fmaf(dA, h[j], dtu * Bv[j]);
            hs[i][j] = h[j];
            dAs[i][j] = dA;
          }
        } else {
#pragma unroll
          for (int j = 0; j < kNpw; ++j) {
            hs[i][j] = 0.f;
            dAs[i][j] = 0.f;
          }
        }
      }
    }

    // reverse sweep
    float keep0 = 0.f, keep1 = 0.f;
    float* durow = s_du + (w * kWave + lane) * RS;
    float* ddtrow = s_ddt + (w * kWave + lane) * RS;
#pragma unroll
    for (int i = TT - 1; i >= 0; --i) {
      if (i < nsteps) {
        const float gy = s_gy[lane * RS + i];
        const float dtv = s_dt[lane * RS + i];
        const float uv = s_u[lane * RS + i];
        const float dtu = dtv * uv;
        const float4 Bt = *reinterpret_cast<const float4*>(s_B + i * kPassStates + w * kNpw);
        const float4 Ct = *reinterpret_cast<const float4*>(s_C + i * kPassStates + w * kNpw);
        const float Bv[4] = {Bt.x, Bt.y, Bt.z, Bt.w};
        const float Cv[4] = {Ct.x, Ct.y, Ct.z, Ct.w};
        float S1 = 0.f, S2 = 0.f;
        float v[8];
#pragma unroll
        for (int j = 0; j < kNpw; ++j) {
          const float hprev = i > 0 ? hs[i > 0 ? i - 1 : 0][j] : h0[j];
          const float gacc = fmaf(gy, Cv[j], gs[j]);
          const float gsn = gacc * dAs[i][j];
          const float q = gsn * hprev;
          gA[j] = fmaf(dtv, q, gA[j]);
          S2 = fmaf(Af[j], q, S2);
          S1 = fmaf(gacc, Bv[j], S1);
          v[j] = gacc * dtu;          // dB contribution
          v[4 + j] = gy * hs[i][j];   // dC contribution
          gs[j] = gsn;
        }
        durow[i] = dtv * S1;
        ddtrow[i] = fmaf(uv, S1, S2);
        float o0, o1;
        reduce8(v, o0, o1);
        if ((lane & 15) == i) {
          keep0 = o0;
          keep1 = o1;
        }
      }
    }
    // lane (row r, column c) holds the tile-partials of step t0 + c:
    // r = 0: dB[n0], dB[n0+1]; r = 1: dB[n0+2], dB[n0+3]; r = 2, 3: same for dC
    {
      const int r = lane >> 4, c = lane & 15;
      if (c < nsteps) {
        float* dst = (r < 2 ? a.part_dB : a.part_dC) + part0 + static_cast<size_t>(t0 + c) * a.N;
        const int nn = n0 + 2 * (r & 1);
        if (nn < a.N) dst[nn] = keep0;
        if (nn + 1 < a.N) dst[nn + 1] = keep1;
      }
    }
    __syncthreads();

    // finish du / ddt over the waves (states), accumulate over passes
    for (int i = threadIdx.x; i < kWave * TT; i += blockDim.x) {
      const int r = i / TT, c = i - r * TT;
      const int dd = d0 + r, t = t0 + c;
      if (dd >= a.D || t >= a.L) continue;
      float su = 0.f, sd = 0.f;
      for (int v = 0; v < nw; ++v) {
        su += s_du[(v * kWave + r) * RS + c];
        sd += s_ddt[(v * kWave + r) * RS + c];
      }
      const size_t gi = row0 + static_cast<size_t>(dd) * a.L + t;
      if (!a.first) {
        su += a.du[gi];
        sd += a.ddt[gi];
      }
      a.du[gi] = su;
      a.ddt[gi] = sd;
    }
  }

  if (dvalid) {
#pragma unroll
    for (int j = 0; j < kNpw; ++j)
      if (n0 + j < a.N) a.part_dA[(static_cast<size_t>(b) * a.D + d) * a.N + n0 + j] = gA[j];
  }
}

// Adds the per-tile partials in a fixed order: dB, dC over channel tiles,
// dA over batch rows.
__global__ void selective_finish_kernel(const float* __restrict__ part_dB,
                                        const float* __restrict__ part_dC,
                                        const float* __restrict__ part_dA, float* __restrict__ dB,
                                        float* __restrict__ dC, float* __restrict__ dA,
                                        int64_t n_bln, int n_dtiles, int64_t n_dn, int Bsz) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n_bln) {
    float sb = 0.f, sc = 0.f;
    for (int k = 0; k < n_dtiles; ++k) {
      sb += part_dB[static_cast<size_t>(k) * n_bln + i];
      sc += part_dC[static_cast<size_t>(k) * n_bln + i];
    }
    dB[i] = sb;
    dC[i] = sc;
  }
  if (i < n_dn) {
    float s = 0.f;
    for (int bb = 0; bb < Bsz; ++bb) s += part_dA[static_cast<size_t>(bb) * n_dn + i];
    dA[i] = s;
  }
}

__global__ void selective_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
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

// Rows of [.., L] can be staged with float4 loads when every row start is
// 16-byte aligned.
bool rows_vectorizable(int64_t L, const float* p, const float* q) {
  return L % 4 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(q) % 16 == 0;
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int64_t ossm_selective_num_chunks(int64_t length) { return ossm::num_chunks(length); }

int ossm_selective_forward(const float* u, const float* dt, const float* A, const float* Bm,
                           const float* Cm, const float* gate, float* out, float* raw_out,
                           float* chunk_states, int64_t batch, int64_t dim, int64_t length,
                           int64_t dstate, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_selective(batch, dim, length, dstate, "selective_forward")) return rc;
  if (batch == 0 || dim == 0 || length == 0) return OSSM_OK;
  if (!u || !dt || !A || !Bm || !Cm || !out)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "selective_forward: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  FwdArgs a{};
  a.u = u;
  a.dt = dt;
  a.A = A;
  a.Bm = Bm;
  a.Cm = Cm;
  a.z = gate;
  a.out = out;
  a.acc = raw_out != nullptr ? raw_out : out;
  a.ckpt = chunk_states;
  a.D = static_cast<int>(dim);
  a.L = static_cast<int>(length);
  a.N = static_cast<int>(dstate);
  a.n_chunks = static_cast<int>(num_chunks(length));
  a.vec = rows_vectorizable(length, u, dt) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>((dim + kWave - 1) / kWave), static_cast<unsigned>(batch));
  const int n_pass = static_cast<int>((dstate + kPassStates - 1) / kPassStates);
  for (int p = 0; p < n_pass; ++p) {
    a.n_base = p * kPassStates;
    a.first = p == 0;
    a.last = p == n_pass - 1;
    const int states = static_cast<int>(std::min<int64_t>(kPassStates, dstate - a.n_base));
    const int waves = (states + kNpw - 1) / kNpw;
    hipLaunchKernelGGL(selective_fwd_kernel, grid, dim3(waves * kWave), 0, stream, a);
    if (int rc = launch_check("selective_fwd_kernel")) return rc;
  }
  return OSSM_OK;
}

int ossm_selective_backward(const float* grad_out, const float* u, const float* dt, const float* A,
                            const float* Bm, const float* Cm, const float* gate,
                            const float* chunk_states, const float* raw_out, float* du, float* ddt,
                            float* dA, float* dB, float* dC, float* dgate, int64_t batch,
                            int64_t dim, int64_t length, int64_t dstate, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_selective(batch, dim, length, dstate, "selective_backward")) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  auto zero = [&](float* p, int64_t n) -> int {
    if (p == nullptr || n <= 0) return OSSM_OK;
    hipLaunchKernelGGL(selective_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
                       dim3(256), 0, stream, p, n);
    return launch_check("selective_zero_kernel");
  };
  if (batch == 0 || dim == 0 || length == 0) {
    // nothing to scan: every gradient is zero (dA still has D*N entries)
    if (int rc = zero(dA, dim * dstate)) return rc;
    if (int rc = zero(dB, batch * length * dstate)) return rc;
    if (int rc = zero(dC, batch * length * dstate)) return rc;
    return OSSM_OK;
  }
  if (!grad_out || !u || !dt || !A || !Bm || !Cm || !chunk_states || !du || !ddt || !dA || !dB ||
      !dC)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "selective_backward: null pointer");
  if (gate != nullptr && (raw_out == nullptr || dgate == nullptr))
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     "selective_backward: a gated scan needs raw_outputs and dgate");
  const int64_t n_dtiles = (dim + kWave - 1) / kWave;
  const int64_t n_bln = batch * length * dstate;
  const int64_t n_dn = dim * dstate;
  const size_t part_bytes = (static_cast<size_t>(2 * n_dtiles * n_bln) + batch * n_dn) * sizeof(float);
  void* ws = nullptr;
  if (int rc = acquire_workspace(stream, part_bytes, &ws)) return rc;
  float* part_dB = static_cast<float*>(ws);
  float* part_dC = part_dB + n_dtiles * n_bln;
  float* part_dA = part_dC + n_dtiles * n_bln;

  BwdArgs a{};
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
  a.part_dB = part_dB;
  a.part_dC = part_dC;
  a.part_dA = part_dA;
  a.Bsz = static_cast<int>(batch);
  a.D = static_cast<int>(dim);
  a.L = static_cast<int>(length);
  a.N = static_cast<int>(dstate);
  a.n_chunks = static_cast<int>(num_chunks(length));
  a.vec = rows_vectorizable(length, u, dt) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(n_dtiles), static_cast<unsigned>(batch));
  const int n_pass = static_cast<int>((dstate + kPassStates - 1) / kPassStates);
  for (int p = 0; p < n_pass; ++p) {
    a.n_base = p * kPassStates;
    a.first = p == 0;
    const int states = static_cast<int>(std::min<int64_t>(kPassStates, dstate - a.n_base));
    const int waves = (states + kNpw - 1) / kNpw;
    hipLaunchKernelGGL(selective_bwd_kernel, grid, dim3(waves * kWave), 0, stream, a);
    if (int rc = launch_check("selective_bwd_kernel")) return rc;
  }
  const int64_t n_fin = n_bln > n_dn ? n_bln : n_dn;
  hipLaunchKernelGGL(selective_finish_kernel, dim3(static_cast<unsigned>((n_fin + 255) / 256)),
                     dim3(256), 0, stream, part_dB, part_dC, part_dA, dB, dC, dA, n_bln,
                     static_cast<int>(n_dtiles), n_dn, static_cast<int>(batch));
  if (int rc = launch_check("selective_finish_kernel")) return rc;
  if (gate == nullptr && dgate != nullptr) return zero(dgate, batch * dim * length);
  return OSSM_OK;
}

}  // extern "C"
