// Fused D-LinOSS layer forward on gfx950: the in-projection, the D-LinOSS scan
// and the out-projection with the D skip in one kernel (DampedLinOSSLayer.forward,
// dlinoss.py:184-247, after the parameter projection of dlinoss.py:249-264):
//
//   bu[b,t,p] = sum_h u[b,t,h] (B[p,h,0] + i B[p,h,1])
//   s_t       = M s_{t-1} + f bu_t       (per variant, s_{-1} = 0; x = s1)
//   y[b,t,h]  = sum_p (Re x[b,t,p] C[h,p,0] - Im x[b,t,p] C[h,p,1]) + D[h] u[b,t,h]
//
// u, y [B,L,H] fp32 row-major; B [P,H,2]; C [H,P,2]; D [H]; a, g, dt [P]
// (already projected).  The unfused layer moves bu and the states through HBM
// several times (GEMM outputs, complex assembly, two permutes, the scan's
// [L,B,P,2] states); here only u is read and y written: 8 bytes per (t, h).
//
// Decomposition: one workgroup (4 waves) per (batch row b, 32-step chunk).
//   1. The chunk's u rows (contiguous in HBM) are staged in LDS.
//   2. In-projection on the matrix cores, v_mfma_f32_32x32x2f32 (fp32 products
//      and sums, no reduced precision): the 32 x 2P result (re and im planes)
//      waits in the accumulators until every wave has read u, then replaces
//      u in LDS (one buffer: four workgroups share a CU at H, P <= 128).
//      Wave w owns oscillator groups w, w+4, ... of 32; its lanes read the
//      weights straight from HBM/L2 (every workgroup reads the same B, so it
//      stays in L2).
//   3. One lane per oscillator scans the 32 steps from a zero state; the
//      chunk aggregate goes through the decoupled look-back of the oscillatory
//      scans (tagged records, launch tickets, chunk transition M^32 formed in
//      fp64) for the carry; the lane re-runs the chunk from the carry and
//      overwrites the projection with x (imaginary part negated).
//   4. Out-projection on the matrix cores (K = the oscillators, the two
//      components as the MFMA's two k slots), plus D u (u read again, from
//      L2), stored as y rows.
//
// MFMA operand layout (v_mfma_f32_32x32x2f32, 64 lanes): lane l supplies
// A[m = l % 32][k = l / 32] and B[k = l / 32][n = l % 32]; accumulator register
// r of lane l holds D[m = 8 (r / 4) + 4 (l / 32) + r % 4][n = l % 32].  The two
// k slots of one instruction take h (or the component) from the two lane
// halves; the sum over k is order-free in the math, so the in-projection gives
// lane half j the h range [j H'/2, (j+1) H'/2) and reads both operands as
// 16-byte runs along h.
//
// Limits: hidden and ssm sizes up to 256 (LDS of one workgroup: 32 rows of u,
// or of the projection's 2 x 32, padded to multiples of 32).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <string>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"
#include "scan_device.hpp"
#include "dlinoss_model.hpp"

namespace ossm {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kLc = 32;            // time steps per chunk = MFMA tile rows
constexpr int kLayerWaves = 4;
constexpr int kLayerThreads = kLayerWaves * kWave;
constexpr int kLayerMax = 256;     // largest hidden / ssm size
// oscillator groups of 32 per wave in the backward's bu projection (Pp / 32
// groups over kLayerWaves waves)
constexpr int kBwdGroups = kLayerMax / 32 / kLayerWaves;
// Weight groups (of 4 k-steps) loaded ahead in the projection loops.  It
// divides every trip count (Hp / 8 and Pp / 4 with Hp, Pp multiples of 32),
// so the unrolled loop bodies have no tail branches and the prefetches are
// unconditional (the last groups reload a clamped in-range group, unused):
// the compiler then keeps them in flight instead of waiting for each.
constexpr int kAhead = 4;

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int round32(int n) { return (n + 31) & ~31; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct LayerArgs {
  const float* u;   // [B, L, H]
  const float* Bw;  // [P, H, 2]
  const float* Cw;  // [H, P, 2]
  const float* Dw;  // [H]
  const float* a;
  const float* g;
  const float* dt;
  float* y;         // [B, L, H]
  float4* carries;  // [B, n_chunks, P]: state entering each chunk (for the backward); may be null
  int Bsz, L, H, P, n_chunks;
};

// Row m of the accumulator register r (see the layout above).
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// Weight loads are branch-free and unmasked: an element outside the tensor
// reads a clamped in-range address, so the loads of the projection loops stay
// unconditional and in flight together.  The matching mask_* zeroes those
// elements where a loop consumes them, a prefetch distance after the load
// (a select at load time needs the data, so each iteration would wait for its
// own loads).
__device__ __forceinline__ float zero_unless(bool ok, float v) { return ok ? v : 0.f; }

// In-projection weights of oscillator p for h = h0 .. h0 + 3, as
// (re h0, im h0, re h0+1, im h0+1) and (re h0+2, ..): B[p, h, 0..1].
// VEC: H % 4 == 0 and B 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ void load_bw(const float* __restrict__ Bw, int H, int P, int p, int h0,
                                        float4 (&w)[2]) {
  const float* row = Bw + static_cast<size_t>(min(p, P - 1)) * H * 2;
  if (VEC) {
    const float4* src = reinterpret_cast<const float4*>(row + min(h0, H - 4) * 2);
    w[0] = src[0];
    w[1] = src[1];
  } else {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = row[min(h0 + (j >> 1), H - 1) * 2 + (j & 1)];
    w[0] = make_float4(v[0], v[1], v[2], v[3]);
    w[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}
__device__ __forceinline__ void mask_bw(int H, int P, int p, int h0, float4 (&w)[2]) {
  const bool k0 = p < P && h0 < H, k1 = p < P && h0 + 1 < H;
  const bool k2 = p < P && h0 + 2 < H, k3 = p < P && h0 + 3 < H;
  w[0] = make_float4(zero_unless(k0, w[0].x), zero_unless(k0, w[0].y), zero_unless(k1, w[0].z),
                     zero_unless(k1, w[0].w));
  w[1] = make_float4(zero_unless(k2, w[1].x), zero_unless(k2, w[1].y), zero_unless(k3, w[1].z),
                     zero_unless(k3, w[1].w));
}

// Out-projection weights of output column h for oscillators p0, p0 + 1:
// (re p0, im p0, re p0+1, im p0+1) = C[h, p0 .. p0+1, 0..1].
// VEC: P % 4 == 0 (p0 even) and C 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ float4 load_cw(const float* __restrict__ Cw, int H, int P, int h, int p0) {
  const float* row = Cw + static_cast<size_t>(min(h, H - 1)) * P * 2;
  if (VEC) return *reinterpret_cast<const float4*>(row + min(p0, P - 2) * 2);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = row[min(p0 + (j >> 1), P - 1) * 2 + (j & 1)];
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 mask_cw(int H, int P, int h, int p0, float4 w) {
  const bool k0 = h < H && p0 < P, k1 = h < H && p0 + 1 < P;
  return make_float4(zero_unless(k0, w.x), zero_unless(k0, w.y), zero_unless(k1, w.z), zero_unless(k1, w.w));
}

// Rows t0 .. t0 + nt - 1 of a [B, L, H] tensor to LDS [kLc][HS], zero-padded,
// in two halves, so that a chunk's rows can be loaded early and written to
// LDS when their phase begins: the thread's share is the float4
// groups e = threadIdx.x + k * kLayerThreads, k < Hp / 32 (kLc x Hp / 4
// groups over the workgroup), all loaded before any is waited on.  Rows past
// nt and columns past H read a clamped in-range address and are zeroed when
// written to LDS.
// SK: float4 groups per thread held (Hp / 32 at most; kLayerMax / 32 covers
// every supported size).
template <int SK = kLayerMax / 32>
struct RowStage {
  float4 v[SK];
};

template <bool VEC, int SK>
__device__ __forceinline__ void stage_load(RowStage<SK>& r, const float* __restrict__ src, size_t row0,
                                           int nt, int H, int Hp) {
  const int q4 = Hp / 4, n = Hp / 32;
#pragma unroll
  for (int k = 0; k < SK; ++k) {
    if (k >= n) break;  // uniform
    const int e = threadIdx.x + k * kLayerThreads;
    const int t = min(e / q4, nt - 1), h = (e - (e / q4) * q4) * 4;
    const float* p = src + row0 + static_cast<size_t>(t) * H;
    if (VEC) {
      r.v[k] = *reinterpret_cast<const float4*>(p + min(h, H - 4));
    } else {
      r.v[k] = make_float4(p[min(h, H - 1)], p[min(h + 1, H - 1)], p[min(h + 2, H - 1)],
                           p[min(h + 3, H - 1)]);
    }
  }
}

template <int SK>
__device__ __forceinline__ void stage_store(const RowStage<SK>& r, float* __restrict__ dst, int nt, int H,
                                            int Hp, int HS) {
  const int q4 = Hp / 4, n = Hp / 32;
#pragma unroll
  for (int k = 0; k < SK; ++k) {
    if (k >= n) break;  // uniform
    const int e = threadIdx.x + k * kLayerThreads;
    const int t = e / q4, h = (e - t * q4) * 4;
    const float4 v = r.v[k];
    const bool row = t < nt;
    *reinterpret_cast<float4*>(dst + t * HS + h) =
        make_float4(row && h < H ? v.x : 0.f, row && h + 1 < H ? v.y : 0.f,
                    row && h + 2 < H ? v.z : 0.f, row && h + 3 < H ? v.w : 0.f);
  }
}

// SMALL: Hp, Pp <= 128 (one oscillator group per wave, four row groups per
// thread): the registers are sized for that, so that four workgroups share a CU.
// PAD: H or P is not a multiple of 32, so the projections' padded rows and
// columns read clamped weights that mask_* zeroes; without padding every weight
// is in range and the loops consume the loads as they are (a select on a loaded
// value is where the compiler puts the wait for it).
template <int V, bool VEC, bool SMALL, bool PAD>
__global__ __launch_bounds__(kLayerThreads) __attribute__((amdgpu_waves_per_eu(SMALL ? 4 : 1)))
void dlinoss_layer_fwd_kernel(
    LayerArgs A, unsigned long long* __restrict__ rec, LaunchSync sync) {
  using Model = Dlinoss<V>;
  constexpr int NG = SMALL ? 1 : kBwdGroups;           // oscillator groups per wave
  constexpr int SK = SMALL ? 128 / 32 : kLayerMax / 32;  // staged float4 per thread
  constexpr int AH = SMALL ? 2 : kAhead;                  // weight groups loaded ahead
  extern __shared__ __align__(16) float smem[];
  __shared__ int s_ticket;

  const int Hp = round32(A.H), Pp = round32(A.P);
  const int HS = Hp + 4, XS = 2 * Pp + 4;  // row strides (floats): 16-byte rows, banks staggered
  float* sU = smem;  // [kLc][HS]     u rows of the chunk, until the in-projection has read them
  float* sX = smem;  // [kLc][Pp][2]  then bu (re, im), then (x.re, -x.im)
  float4* s_agg = reinterpret_cast<float4*>(smem + kLc * max(HS, XS));  // [P] chunk aggregates

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int ticket = launch_order(sync, A.Bsz * A.n_chunks, &s_ticket);
  const int c = ticket / A.Bsz;  // every chunk-(c-1) workgroup holds an earlier ticket
  const int b = ticket - c * A.Bsz;
  const int t0 = c * kLc;
  const int nt = min(kLc, A.L - t0);
  const size_t row0 = (static_cast<size_t>(b) * A.L + t0) * A.H;  // u / y row t0 of batch b

  // 1. u rows t0 .. t0 + nt - 1 (contiguous) -> LDS, zero-padded to 32 x Hp
  {
    RowStage<SK> st;
    stage_load<VEC>(st, A.u, row0, nt, A.H, Hp);
    stage_store(st, sU, nt, A.H, Hp, HS);
  }
  __syncthreads();

  // 2. in-projection: for oscillator group pg (32 oscillators) the wave forms
  //    the re and im 32 x 32 tiles, K = Hp split over the two lane halves;
  //    held in the accumulators until every wave has read u, then written
  //    to sX over it
  {
    const int half = lane >> 5, m = lane & 31;
    const int hh = Hp / 2;        // h per lane half (a multiple of 16)
    const int ng = hh / 4;        // groups of 4 k-steps (a multiple of 4)
    const float* arow = sU + m * HS + half * hh;
    floatx16 acc_re[NG], acc_im[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int pg = w + i * kLayerWaves;
      if (pg >= Pp / 32) break;  // uniform
      const int p = pg * 32 + m;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_re[i][r] = acc_im[i][r] = 0.f;
      float4 wb[AH][2];
#pragma unroll
      for (int j = 0; j < AH; ++j) load_bw<VEC>(A.Bw, A.H, A.P, p, half * hh + 4 * j, wb[j]);
      // A operand one group ahead: its LDS read overlaps this group's MFMAs
      float4 an = *reinterpret_cast<const float4*>(arow);
      for (int q0 = 0; q0 < ng; q0 += AH) {
#pragma unroll
        for (int j = 0; j < AH; ++j) {
          const int q = q0 + j;
          float4 av = an;
          an = *reinterpret_cast<const float4*>(arow + 4 * min(q + 1, ng - 1));
          float4 wq[2] = {wb[j][0], wb[j][1]};
          if constexpr (PAD) mask_bw(A.H, A.P, p, half * hh + 4 * q, wq);
          const float4 w0 = wq[0], w1 = wq[1];
          load_bw<VEC>(A.Bw, A.H, A.P, p, half * hh + 4 * min(q + AH, ng - 1), wb[j]);
          asm volatile("" ::: "memory");  // the prefetch stays here, not next to its use
          // and the MFMAs below it, after the next group's LDS read
          asm volatile("" : "+v"(av.x), "+v"(av.y), "+v"(av.z), "+v"(av.w));
          acc_re[i] = mfma32(av.x, w0.x, acc_re[i]);
          acc_im[i] = mfma32(av.x, w0.y, acc_im[i]);
          acc_re[i] = mfma32(av.y, w0.z, acc_re[i]);
          acc_im[i] = mfma32(av.y, w0.w, acc_im[i]);
          acc_re[i] = mfma32(av.z, w1.x, acc_re[i]);
          acc_im[i] = mfma32(av.z, w1.y, acc_im[i]);
          acc_re[i] = mfma32(av.w, w1.z, acc_re[i]);
          acc_im[i] = mfma32(av.w, w1.w, acc_im[i]);
          __builtin_amdgcn_sched_barrier(0);  // groups stay in program order (prefetch distance)
        }
      }
    }
    __syncthreads();  // u is read: sX may overwrite it
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int pg = w + i * kLayerWaves;
      if (pg >= Pp / 32) break;  // uniform
      const int p = pg * 32 + m;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = acc_row(r, lane);
        *reinterpret_cast<float2*>(sX + t * XS + 2 * p) = make_float2(acc_re[i][r], acc_im[i][r]);
      }
    }
  }
  __syncthreads();

  // 3. the scan, one thread per oscillator
  const int p = threadIdx.x;
  const bool osc = p < A.P;
  const int nc = A.Bsz * A.P;
  const int ch = b * A.P + p;
  const bool scan = A.n_chunks > 1;
  typename Model::Coef k{};
  if (osc) k = Model::coef_of({A.a[p], A.g[p], A.dt[p]});
  // All 32 steps run: rows past L hold zeros (zero u rows), which only the
  // last chunk has; its aggregate is never read and its rows past L never stored.
  const float2* bu_col = reinterpret_cast<const float2*>(sX) + p;
  const int xs2 = XS / 2;
  float4 e = f4zero();
  if (osc) {
#pragma unroll
    for (int t = 0; t < kLc; ++t) e = Model::step(k, e, bu_col[t * xs2]);
    s_agg[p] = e;
  }
  // The aggregate is published by a wave that does not then walk back when
  // there is one (P <= 128: waves 2 and 3): a wave's loads complete in issue
  // order behind its own stores.
  const bool split_pub = A.P <= 2 * kWave;
  if (scan && c > 0) {
    if (split_pub) {
      __syncthreads();
      const int q = threadIdx.x - 2 * kWave;
      if (q >= 0 && q < A.P) rec_publish(rec, c, kRecAgg, nc, b * A.P + q, s_agg[q], sync.tag);
    } else if (osc) {
      rec_publish(rec, c, kRecAgg, nc, ch, e, sync.tag);
    }
  }
  if (osc) {
    float4 s = f4zero();
    if (scan) {
      const RMat MC = mat_pow(Model::matrix(k), kLc);
      if (c == 0) {
        rec_publish(rec, c, kRecInc, nc, ch, e, sync.tag);
      } else {
        s = lookback(rec, c, +1, A.n_chunks, nc, ch, MC, sync);
        if (c + 1 < A.n_chunks) rec_publish(rec, c, kRecInc, nc, ch, f4add(mat_apply(MC, s), e), sync.tag);
      }
    }
    if (A.carries != nullptr) A.carries[(static_cast<size_t>(b) * A.n_chunks + c) * A.P + p] = s;
    float2* x_col = reinterpret_cast<float2*>(sX) + p;
#pragma unroll
    for (int t = 0; t < kLc; ++t) {
      s = Model::step(k, s, x_col[t * xs2]);
      x_col[t * xs2] = make_float2(s.z, -s.w);
    }
  }
  __syncthreads();

  // 4. out-projection + D skip: wave w owns output column groups w, w+4, ...
  //    Group q covers oscillators 4q .. 4q+3; lane half kk takes 4q + 2kk and
  //    4q + 2kk + 1, so A (x.re, -x.im of two oscillators, from LDS) and B
  //    (C[h, p, re], C[h, p, im] of the same two) are matching 16-byte runs.
  {
    const int kk = lane >> 5, m = lane & 31;
    const int ng = Pp / 4;  // groups of 4 oscillators (a multiple of 8)
    const float* arow = sX + m * XS + 4 * kk;
    for (int hg = w; hg < Hp / 32; hg += kLayerWaves) {
      const int h = hg * 32 + m;
      floatx16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
      // u for the D skip (LDS holds x now), loaded before the MFMA loop
      // (clamped in range; the chunk's rows were just read, so L2 serves them)
      float uv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        uv[r] = A.u[row0 + static_cast<size_t>(min(acc_row(r, lane), nt - 1)) * A.H + min(h, A.H - 1)];
      float4 cb[AH];
#pragma unroll
      for (int j = 0; j < AH; ++j) cb[j] = load_cw<VEC>(A.Cw, A.H, A.P, h, 4 * j + 2 * kk);
      // A operand one group ahead: its LDS read overlaps this group's MFMAs
      float4 an = *reinterpret_cast<const float4*>(arow);
      for (int q0 = 0; q0 < ng; q0 += AH) {
#pragma unroll
        for (int j = 0; j < AH; ++j) {
          const int q = q0 + j;
          float4 av = an;
          an = *reinterpret_cast<const float4*>(arow + 8 * min(q + 1, ng - 1));
          const float4 cv = PAD ? mask_cw(A.H, A.P, h, 4 * q + 2 * kk, cb[j]) : cb[j];
          cb[j] = load_cw<VEC>(A.Cw, A.H, A.P, h, 4 * min(q + AH, ng - 1) + 2 * kk);
          asm volatile("" ::: "memory");  // the prefetch stays here, not next to its use
          // and the MFMAs below it, after the next group's LDS read
          asm volatile("" : "+v"(av.x), "+v"(av.y), "+v"(av.z), "+v"(av.w));
          acc = mfma32(av.x, cv.x, acc);
          acc = mfma32(av.y, cv.y, acc);
          acc = mfma32(av.z, cv.z, acc);
          acc = mfma32(av.w, cv.w, acc);
          __builtin_amdgcn_sched_barrier(0);  // groups stay in program order (prefetch distance)
        }
      }
      if (h < A.H) {
        const float dh = A.Dw[h];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(r, lane);
          if (t < nt) A.y[row0 + static_cast<size_t>(t) * A.H + h] = acc[r] + uv[r] * dh;
        }
      }
    }
  }
}

// ============================================================================
// Backward.  For y = Re(x C^T) + D u with x the states driven by bu = u B^T:
//   g_x   = gy (C_re - i C_im)                          (complex gradient of x)
//   mu_t  = M^T mu_{t+1} + (0, g_x,t),  grad_bu_t = f^T mu_t   (the scan adjoint)
//   grad_u = Re(grad_bu) B_re + Im(grad_bu) B_im + D gy
//   sums of <mu, s_{t-1}>, <mu, bu> -> grad a, g, dt  (the scan's chain rule)
// One workgroup per (batch row, 32-step chunk), chunks in reverse time order:
//   1. gy rows -> LDS; g_x on the matrix cores (K = H) -> LDS (re, im pairs);
//   2. u rows -> LDS (over gy); bu on the matrix cores -> LDS;
//   3. one lane per oscillator re-runs the forward over the chunk from the
//      carry the forward saved, keeping the 32 states s_{t-1} in registers and
//      writing x (re, -im) for the weight gradient of C; the adjoint runs from
//      zero over the chunk, its aggregate goes through the look-back (reverse,
//      transition (M^T)^32), then it re-runs from the carry: grad_bu over g_x
//      in LDS, the parameter sums per lane (partials for the column sums);
//   4. grad_u on the matrix cores (K = the oscillators, the components as k
//      slots, as the forward's out-projection) plus D gy; grad_bu rows stored.
// grad_B = grad_bu^T u and grad_C = gy^T x' are sums over all (b, t): plain
// GEMMs over the stored grad_bu and x' (the caller runs them).
// ============================================================================
struct LayerBwdArgs {
  const float* u;        // [B, L, H]
  const float* gy;       // [B, L, H]
  const float* Bw;       // [P, H, 2]
  const float* Cw;       // [H, P, 2]
  const float* Dw;       // [H]
  const float* a;
  const float* g;
  const float* dt;
  const float4* carries; // [B, n_chunks, P] from the forward
  float* grad_u;         // [B, L, H]
  float2* grad_bu;       // [B, L, P] (re, im)
  float2* xq;            // [B, L, P] (x.re, -x.im)
  float* partials;       // [n_chunks][NS][B * P]
  ZeroFill zero;         // grad a, g, dt, cleared by the first workgroup
  int Bsz, L, H, P, n_chunks;
};

// Weights of the g_x projection for oscillator p and h = h0 .. h0 + 3:
// (re h0, im h0, re h0+1, im h0+1), (.. h0+2, h0+3) of (C_re, C_im)[h, p].
template <bool VEC>
__device__ __forceinline__ void load_cw_pair(const float* __restrict__ Cw, int H, int P, int h0, int p,
                                             float4 (&w)[2]) {
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float* q = Cw + (static_cast<size_t>(min(h0 + j, H - 1)) * P + min(p, P - 1)) * 2;
    if (VEC) {
      const float2 c = *reinterpret_cast<const float2*>(q);
      v[2 * j] = c.x;
      v[2 * j + 1] = c.y;
    } else {
      v[2 * j] = q[0];
      v[2 * j + 1] = q[1];
    }
  }
  w[0] = make_float4(v[0], v[1], v[2], v[3]);
  w[1] = make_float4(v[4], v[5], v[6], v[7]);
}
// zero outside the tensor: the same pattern as mask_bw with the roles of h and p
__device__ __forceinline__ void mask_cw_pair(int H, int P, int h0, int p, float4 (&w)[2]) {
  mask_bw(H, P, p, h0, w);
}

// (B_re, B_im)[p0, h], (B_re, B_im)[p0 + 1, h].
__device__ __forceinline__ float4 load_bw_pair(const float* __restrict__ Bw, int H, int P, int h, int p0) {
  float v[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float2 b = *reinterpret_cast<const float2*>(
        Bw + (static_cast<size_t>(min(p0 + j, P - 1)) * H + min(h, H - 1)) * 2);
    v[2 * j] = b.x;
    v[2 * j + 1] = b.y;
  }
  return make_float4(v[0], v[1], v[2], v[3]);
}
// zero outside the tensor: mask_cw's pattern (column h, oscillators p0, p0 + 1)
__device__ __forceinline__ float4 mask_bw_pair(int H, int P, int h, int p0, float4 w) {
  return mask_cw(H, P, h, p0, w);
}

// PAD: as for the forward (H or P not a multiple of 32: weights masked where used).
template <int V, bool VEC, bool PAD>
__global__ __launch_bounds__(kLayerThreads) void dlinoss_layer_bwd_kernel(
    LayerBwdArgs A, unsigned long long* __restrict__ rec, LaunchSync sync) {
  using Model = Dlinoss<V>;
  constexpr int NS = Model::kSums;
  extern __shared__ __align__(16) float smem[];
  __shared__ int s_ticket;

  const int Hp = round32(A.H), Pp = round32(A.P);
  const int HS = Hp + 4, XS = 2 * Pp + 4;
  float* sA = smem;                   // [kLc][HS]   gy rows, then u rows
  float* sX = smem;                   // [kLc][Pp][2] bu, over sA once u is read
  float* sG = smem + kLc * max(HS, XS);  // [kLc][Pp][2] g_x, then grad_bu
  float4* s_agg = reinterpret_cast<float4*>(sG + kLc * XS);  // [P]

  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int ticket = launch_order(sync, A.Bsz * A.n_chunks, &s_ticket);
  if (ticket == 0) zero_fill_block(A.zero);
  const int cr = ticket / A.Bsz;     // chunks in reverse time order
  const int c = A.n_chunks - 1 - cr;
  const int b = ticket - cr * A.Bsz;
  const int t0 = c * kLc;
  const int nt = min(kLc, A.L - t0);
  const size_t row0 = (static_cast<size_t>(b) * A.L + t0) * A.H;
  const size_t prow0 = (static_cast<size_t>(b) * A.L + t0) * A.P;  // grad_bu / xq rows
  const int half = lane >> 5, m = lane & 31;
  const int hh = Hp / 2, ng1 = hh / 4;

  // Every HBM read the chunk needs before its last phase goes out now: the
  // gy and u rows (to LDS at phases 1 and 2) and the carry entering the
  // chunk (phase 3).
  RowStage<> st_gy, st_u;
  stage_load<VEC>(st_gy, A.gy, row0, nt, A.H, Hp);
  stage_load<VEC>(st_u, A.u, row0, nt, A.H, Hp);
  const int p = threadIdx.x;
  const bool osc = p < A.P;
  const float4 carry_in = A.carries[(static_cast<size_t>(b) * A.n_chunks + c) * A.P + min(p, A.P - 1)];

  // 1. gy -> LDS; g_x = gy (C_re - i C_im) on the matrix cores -> sG
  stage_store(st_gy, sA, nt, A.H, Hp, HS);
  __syncthreads();
  {
    const float* arow = sA + m * HS + half * hh;
    for (int pg = w; pg < Pp / 32; pg += kLayerWaves) {
      const int p = pg * 32 + m;
      floatx16 acc_re, acc_im;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_re[r] = acc_im[r] = 0.f;
      float4 wb[kAhead][2];
#pragma unroll
      for (int j = 0; j < kAhead; ++j) load_cw_pair<VEC>(A.Cw, A.H, A.P, half * hh + 4 * j, p, wb[j]);
      // A operand one group ahead: its LDS read overlaps this group's MFMAs
      float4 an = *reinterpret_cast<const float4*>(arow);
      for (int q0 = 0; q0 < ng1; q0 += kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
          const int q = q0 + j;
          float4 av = an;
          an = *reinterpret_cast<const float4*>(arow + 4 * min(q + 1, ng1 - 1));
          float4 wq[2] = {wb[j][0], wb[j][1]};
          if constexpr (PAD) mask_cw_pair(A.H, A.P, half * hh + 4 * q, p, wq);
          const float4 w0 = wq[0], w1 = wq[1];
          load_cw_pair<VEC>(A.Cw, A.H, A.P, half * hh + 4 * min(q + kAhead, ng1 - 1), p, wb[j]);
          asm volatile("" ::: "memory");  // the prefetch stays here, not next to its use
          // and the MFMAs below it, after the next group's LDS read
          asm volatile("" : "+v"(av.x), "+v"(av.y), "+v"(av.z), "+v"(av.w));
          acc_re = mfma32(av.x, w0.x, acc_re);
          acc_im = mfma32(av.x, w0.y, acc_im);
          acc_re = mfma32(av.y, w0.z, acc_re);
          acc_im = mfma32(av.y, w0.w, acc_im);
          acc_re = mfma32(av.z, w1.x, acc_re);
          acc_im = mfma32(av.z, w1.y, acc_im);
          acc_re = mfma32(av.w, w1.z, acc_re);
          acc_im = mfma32(av.w, w1.w, acc_im);
          __builtin_amdgcn_sched_barrier(0);  // groups stay in program order (prefetch distance)
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = acc_row(r, lane);
        *reinterpret_cast<float2*>(sG + t * XS + 2 * p) = make_float2(acc_re[r], -acc_im[r]);
      }
    }
  }
  __syncthreads();

  // 2. u -> LDS (over gy); bu on the matrix cores, held in the accumulators
  //    until every wave has read u, then written to sX over it
  stage_store(st_u, sA, nt, A.H, Hp, HS);
  __syncthreads();
  {
    const float* arow = sA + m * HS + half * hh;
    floatx16 acc_re[kBwdGroups], acc_im[kBwdGroups];
#pragma unroll
    for (int i = 0; i < kBwdGroups; ++i) {
      const int pg = w + i * kLayerWaves;
      if (pg >= Pp / 32) break;  // uniform
      const int p = pg * 32 + m;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_re[i][r] = acc_im[i][r] = 0.f;
      float4 wb[kAhead][2];
#pragma unroll
      for (int j = 0; j < kAhead; ++j) load_bw<VEC>(A.Bw, A.H, A.P, p, half * hh + 4 * j, wb[j]);
      // A operand one group ahead: its LDS read overlaps this group's MFMAs
      float4 an = *reinterpret_cast<const float4*>(arow);
      for (int q0 = 0; q0 < ng1; q0 += kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
          const int q = q0 + j;
          float4 av = an;
          an = *reinterpret_cast<const float4*>(arow + 4 * min(q + 1, ng1 - 1));
          float4 wq[2] = {wb[j][0], wb[j][1]};
          if constexpr (PAD) mask_bw(A.H, A.P, p, half * hh + 4 * q, wq);
          const float4 w0 = wq[0], w1 = wq[1];
          load_bw<VEC>(A.Bw, A.H, A.P, p, half * hh + 4 * min(q + kAhead, ng1 - 1), wb[j]);
          asm volatile("" ::: "memory");  // the prefetch stays here, not next to its use
          // and the MFMAs below it, after the next group's LDS read
          asm volatile("" : "+v"(av.x), "+v"(av.y), "+v"(av.z), "+v"(av.w));
          acc_re[i] = mfma32(av.x, w0.x, acc_re[i]);
          acc_im[i] = mfma32(av.x, w0.y, acc_im[i]);
          acc_re[i] = mfma32(av.y, w0.z, acc_re[i]);
          acc_im[i] = mfma32(av.y, w0.w, acc_im[i]);
          acc_re[i] = mfma32(av.z, w1.x, acc_re[i]);
          acc_im[i] = mfma32(av.z, w1.y, acc_im[i]);
          acc_re[i] = mfma32(av.w, w1.z, acc_re[i]);
          acc_im[i] = mfma32(av.w, w1.w, acc_im[i]);
          __builtin_amdgcn_sched_barrier(0);  // groups stay in program order (prefetch distance)
        }
      }
    }
    __syncthreads();  // u is read: sX may overwrite it
#pragma unroll
    for (int i = 0; i < kBwdGroups; ++i) {
      const int pg = w + i * kLayerWaves;
      if (pg >= Pp / 32) break;  // uniform
      const int p = pg * 32 + m;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = acc_row(r, lane);
        *reinterpret_cast<float2*>(sX + t * XS + 2 * p) = make_float2(acc_re[i][r], acc_im[i][r]);
      }
    }
  }
  __syncthreads();

  // 3. states, adjoint, grad_bu, parameter sums: one thread per oscillator
  const int nc = A.Bsz * A.P;
  const int ch = b * A.P + p;
  const bool scan = A.n_chunks > 1;
  const float2* bu_col = reinterpret_cast<const float2*>(sX) + p;
  float2* g_col = reinterpret_cast<float2*>(sG) + p;
  const int xs2 = XS / 2;
  typename Model::Coef k{};
  float4 sp[kLc];  // state before step t of the chunk
  float4 e = f4zero();
  if (osc) {
    k = Model::coef_of({A.a[p], A.g[p], A.dt[p]});
    float4 s = carry_in;
#pragma unroll
    for (int t = 0; t < kLc; ++t) {
      sp[t] = s;
      s = Model::step(k, s, bu_col[t * xs2]);
      if (t < nt) A.xq[prow0 + static_cast<size_t>(t) * A.P + p] = make_float2(s.z, -s.w);
    }
    // adjoint from zero over the chunk (rows past L carry zero gradients)
#pragma unroll
    for (int t = kLc - 1; t >= 0; --t) e = Model::rev_carry(k, Model::mu(e, g_col[t * xs2]));
    s_agg[p] = e;
  }
  const bool split_pub = A.P <= 2 * kWave;
  if (scan && c < A.n_chunks - 1) {
    if (split_pub) {
      __syncthreads();
      const int q = threadIdx.x - 2 * kWave;
      if (q >= 0 && q < A.P) rec_publish(rec, c, kRecAgg, nc, b * A.P + q, s_agg[q], sync.tag);
    } else if (osc) {
      rec_publish(rec, c, kRecAgg, nc, ch, e, sync.tag);
    }
  }
  if (osc) {
    float4 carry = f4zero();
    if (scan) {
      const RMat KC = mat_pow(mat_adjoint(Model::matrix(k)), kLc);
      if (c == A.n_chunks - 1) {
        rec_publish(rec, c, kRecInc, nc, ch, e, sync.tag);
      } else {
        carry = lookback(rec, c, -1, A.n_chunks, nc, ch, KC, sync);
        if (c > 0) rec_publish(rec, c, kRecInc, nc, ch, f4add(mat_apply(KC, carry), e), sync.tag);
      }
    }
    float acc[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[j] = 0.f;
    float4 mcar = carry;
#pragma unroll
    for (int t = kLc - 1; t >= 0; --t) {
      const float4 mu = Model::mu(mcar, g_col[t * xs2]);
      const float2 gb = Model::grad_input(k, mu);
      Model::accumulate(acc, mu, sp[t], bu_col[t * xs2]);
      g_col[t * xs2] = gb;
      mcar = Model::rev_carry(k, mu);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j)
      A.partials[(static_cast<size_t>(c) * NS + j) * nc + ch] = acc[j];
  }
  __syncthreads();

  // 4. grad_bu rows out; grad_u = grad_bu (B_re, B_im) + D gy on the matrix cores
  {
    const int q2 = A.P;  // float2 per row
    for (int e2 = threadIdx.x; e2 < kLc * q2; e2 += kLayerThreads) {
      const int t = e2 / q2, pp = e2 - t * q2;
      if (t < nt) A.grad_bu[prow0 + static_cast<size_t>(t) * A.P + pp] = reinterpret_cast<const float2*>(sG)[t * xs2 + pp];
    }
  }
  {
    const int kk = lane >> 5;
    const int ng = Pp / 4;
    const float* arow = sG + m * XS + 4 * kk;
    for (int hg = w; hg < Hp / 32; hg += kLayerWaves) {
      const int h = hg * 32 + m;
      floatx16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
      // gy for the D skip, loaded before the MFMA loop (clamped in range)
      float gyv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        gyv[r] = A.gy[row0 + static_cast<size_t>(min(acc_row(r, lane), nt - 1)) * A.H + min(h, A.H - 1)];
      float4 cb[kAhead];
#pragma unroll
      for (int j = 0; j < kAhead; ++j) cb[j] = load_bw_pair(A.Bw, A.H, A.P, h, 4 * j + 2 * kk);
      // A operand one group ahead: its LDS read overlaps this group's MFMAs
      float4 an = *reinterpret_cast<const float4*>(arow);
      for (int q0 = 0; q0 < ng; q0 += kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
          const int q = q0 + j;
          float4 av = an;
          an = *reinterpret_cast<const float4*>(arow + 8 * min(q + 1, ng - 1));
          const float4 cv = PAD ? mask_bw_pair(A.H, A.P, h, 4 * q + 2 * kk, cb[j]) : cb[j];
          cb[j] = load_bw_pair(A.Bw, A.H, A.P, h, 4 * min(q + kAhead, ng - 1) + 2 * kk);
          asm volatile("" ::: "memory");  // the prefetch stays here, not next to its use
          // and the MFMAs below it, after the next group's LDS read
          asm volatile("" : "+v"(av.x), "+v"(av.y), "+v"(av.z), "+v"(av.w));
          acc = mfma32(av.x, cv.x, acc);
          acc = mfma32(av.y, cv.y, acc);
          acc = mfma32(av.z, cv.z, acc);
          acc = mfma32(av.w, cv.w, acc);
          __builtin_amdgcn_sched_barrier(0);  // groups stay in program order (prefetch distance)
        }
      }
      if (h < A.H) {
        const float dh = A.Dw[h];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = acc_row(r, lane);
          if (t < nt) A.grad_u[row0 + static_cast<size_t>(t) * A.H + h] = acc[r] + gyv[r] * dh;
        }
      }
    }
  }
}

template <class Model>
struct LayerParamEpilogue {
  typename Model::Params prm;
  float *ga, *gg, *gs;
  __device__ void add(int p, const double* S) const { Model::epilogue(prm, p, 0, S, ga, gg, gs); }
};

size_t layer_bwd_lds_bytes(int64_t H, int64_t P) {
  const int64_t Hp = (H + 31) / 32 * 32, Pp = (P + 31) / 32 * 32;
  return static_cast<size_t>(kLc * std::max(Hp + 4, 2 * Pp + 4) + kLc * (2 * Pp + 4) + 4 * P) *
         sizeof(float);
}

constexpr size_t kMaxLds = 160 * 1024;

template <int V>
int launch_layer_bwd(LayerBwdArgs args, float* ga, float* gg, float* gs, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  using Model = Dlinoss<V>;
  constexpr int NS = Model::kSums;
  const int64_t n_wg = static_cast<int64_t>(args.Bsz) * args.n_chunks;
  const int64_t nc = static_cast<int64_t>(args.Bsz) * args.P;
  const size_t rec_bytes = static_cast<size_t>(args.n_chunks) * 2 * 4 * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  void* ws = nullptr;
  if (int rc = acquire_workspace(call, static_cast<size_t>(args.n_chunks) * NS * nc * sizeof(float), &ws))
    return rc;
  args.partials = static_cast<float*>(ws);
  args.zero = ZeroFill{{ga, gg, gs}, {args.P, args.P, args.P}};
  const bool vec = args.H % 4 == 0 && args.P % 4 == 0 && aligned16(args.u) && aligned16(args.gy) &&
                   aligned16(args.Bw) && aligned16(args.Cw);
  const bool pad = args.H % 32 != 0 || args.P % 32 != 0;
  auto kern = vec ? (pad ? dlinoss_layer_bwd_kernel<V, true, true> : dlinoss_layer_bwd_kernel<V, true, false>)
                  : (pad ? dlinoss_layer_bwd_kernel<V, false, true> : dlinoss_layer_bwd_kernel<V, false, false>);
  const size_t lds = layer_bwd_lds_bytes(args.H, args.P);
  // before the ticket reservation: a failure here leaves nothing reserved
  if (int rc = hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds)),
                         "hipFuncSetAttribute"))
    return rc;
  if (int rc = acquire_scratch(call, rec_bytes, n_wg, &payload, &sync)) return rc;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(n_wg)), dim3(kLayerThreads), lds, stream, args,
                     static_cast<unsigned long long*>(payload), sync);
  if (int rc = launch_check("dlinoss_layer_bwd_kernel")) return rc;
  if (args.P == 0) return OSSM_OK;
  const typename Model::Params prm{args.a, args.g, args.dt, args.P};
  return launch_column_sums<NS>(static_cast<const float*>(ws), args.P, args.Bsz, args.n_chunks,
                                LayerParamEpilogue<Model>{prm, ga, gg, gs}, stream);
}

size_t layer_lds_bytes(int64_t H, int64_t P) {
  const int64_t Hp = (H + 31) / 32 * 32, Pp = (P + 31) / 32 * 32;
  return static_cast<size_t>(kLc * std::max(Hp + 4, 2 * Pp + 4) + 4 * P) * sizeof(float);
}


template <int V>
int launch_layer(const LayerArgs& args, hipStream_t stream) {
  StreamCall call(stream);
  if (call.status()) return call.status();
  const int64_t n_wg = static_cast<int64_t>(args.Bsz) * args.n_chunks;
  const int64_t nc = static_cast<int64_t>(args.Bsz) * args.P;
  const size_t rec_bytes = static_cast<size_t>(args.n_chunks) * 2 * 4 * nc * sizeof(unsigned long long);
  void* payload = nullptr;
  LaunchSync sync{};
  const bool vec = args.H % 4 == 0 && args.P % 4 == 0 && aligned16(args.u) && aligned16(args.Bw) &&
                   aligned16(args.Cw);
  const bool small = args.H <= 128 && args.P <= 128;
  const bool pad = args.H % 32 != 0 || args.P % 32 != 0;
  using K = void (*)(LayerArgs, unsigned long long*, LaunchSync);
  const K kern =
      vec ? (small ? (pad ? dlinoss_layer_fwd_kernel<V, true, true, true> : dlinoss_layer_fwd_kernel<V, true, true, false>)
                   : (pad ? dlinoss_layer_fwd_kernel<V, true, false, true> : dlinoss_layer_fwd_kernel<V, true, false, false>))
          : (small ? (pad ? dlinoss_layer_fwd_kernel<V, false, true, true> : dlinoss_layer_fwd_kernel<V, false, true, false>)
                   : (pad ? dlinoss_layer_fwd_kernel<V, false, false, true> : dlinoss_layer_fwd_kernel<V, false, false, false>));
  const size_t lds = layer_lds_bytes(args.H, args.P);
  // before the ticket reservation: a failure here leaves nothing reserved
  if (int rc = hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds)),
                         "hipFuncSetAttribute"))
    return rc;
  if (int rc = acquire_scratch(call, rec_bytes, n_wg, &payload, &sync)) return rc;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(n_wg)), dim3(kLayerThreads), lds, stream, args,
                     static_cast<unsigned long long*>(payload), sync);
  return launch_check("dlinoss_layer_fwd_kernel");
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_dlinoss_layer_forward(int variant, const float* inputs, const float* B, const float* C,
                               const float* D, const float* a_diag, const float* g_diag,
                               const float* step, float* outputs, void* carries, int64_t batch,
                               int64_t length, int64_t hidden, int64_t ssm,
                               ossm_stream_t stream_v) {
  clear_error();
  const char* what = "dlinoss_layer_forward";
  if (batch < 0 || length < 0 || hidden < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (variant < OSSM_DLINOSS_IMEX1 || variant > OSSM_DLINOSS_EX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": unknown variant");
  if (hidden > kLayerMax || ssm > kLayerMax)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": hidden_dim and ssm_size up to " +
                                               std::to_string(kLayerMax) + " are supported, got " +
                                               std::to_string(hidden) + " and " + std::to_string(ssm));
  if (batch == 0 || length == 0 || hidden == 0) return OSSM_OK;
  const int64_t n_chunks = (length + kLc - 1) / kLc;
  if (length > INT_MAX || batch * n_chunks > INT_MAX || batch * length * hidden > (int64_t(1) << 62) ||
      batch * ssm > INT_MAX / 8)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  if (!inputs || !D || !outputs || (ssm > 0 && (!B || !C || !a_diag || !g_diag || !step)))
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  LayerArgs args{inputs, B, C, D, a_diag, g_diag, step, outputs, static_cast<float4*>(carries),
                 static_cast<int>(batch), static_cast<int>(length), static_cast<int>(hidden),
                 static_cast<int>(ssm), static_cast<int>(n_chunks)};
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return launch_layer<OSSM_DLINOSS_IMEX1>(args, stream);
    case OSSM_DLINOSS_IMEX2: return launch_layer<OSSM_DLINOSS_IMEX2>(args, stream);
    case OSSM_DLINOSS_IM: return launch_layer<OSSM_DLINOSS_IM>(args, stream);
    default: return launch_layer<OSSM_DLINOSS_EX>(args, stream);
  }
}

int ossm_dlinoss_layer_backward(int variant, const float* inputs, const float* grad_output,
                                const float* B, const float* C, const float* D,
                                const float* a_diag, const float* g_diag, const float* step,
                                const void* carries, float* grad_inputs, void* grad_bu,
                                void* x_conj, float* grad_a, float* grad_g, float* grad_step,
                                int64_t batch, int64_t length, int64_t hidden, int64_t ssm,
                                ossm_stream_t stream_v) {
  clear_error();
  const char* what = "dlinoss_layer_backward";
  if (batch < 0 || length < 0 || hidden < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (variant < OSSM_DLINOSS_IMEX1 || variant > OSSM_DLINOSS_EX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": unknown variant");
  if (hidden > kLayerMax || ssm > kLayerMax || layer_bwd_lds_bytes(hidden, ssm) > kMaxLds)
    return set_error(OSSM_ERR_UNSUPPORTED,
                     std::string(what) + ": hidden_dim " + std::to_string(hidden) + " and ssm_size " +
                         std::to_string(ssm) + " exceed one workgroup's LDS");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  if (ssm > 0 && (!grad_a || !grad_g || !grad_step))
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  if (batch == 0 || length == 0 || hidden == 0) {
    // no terms: zero parameter gradients (grad_inputs, grad_bu, x_conj are empty
    // or, with hidden == 0, hold no dependence on the scan)
    for (float* p : {grad_a, grad_g, grad_step})
      if (int rc = fill_zero(p, ssm, stream)) return rc;
    if (hidden == 0 && batch > 0 && length > 0 && ssm > 0) {
      if (int rc = fill_zero(static_cast<float*>(grad_bu), 2 * batch * length * ssm, stream)) return rc;
      if (int rc = fill_zero(static_cast<float*>(x_conj), 2 * batch * length * ssm, stream)) return rc;
    }
    return OSSM_OK;
  }
  const int64_t n_chunks = (length + kLc - 1) / kLc;
  if (length > INT_MAX || batch * n_chunks > INT_MAX || batch * ssm > INT_MAX / 8)
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  if (!inputs || !grad_output || !D || !grad_inputs ||
      (ssm > 0 && (!B || !C || !a_diag || !g_diag || !step || !carries || !grad_bu || !x_conj)))
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  LayerBwdArgs args{inputs, grad_output, B, C, D, a_diag, g_diag, step,
                    static_cast<const float4*>(carries), grad_inputs,
                    static_cast<float2*>(grad_bu), static_cast<float2*>(x_conj), nullptr,
                    ZeroFill{}, static_cast<int>(batch), static_cast<int>(length),
                    static_cast<int>(hidden), static_cast<int>(ssm), static_cast<int>(n_chunks)};
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return launch_layer_bwd<OSSM_DLINOSS_IMEX1>(args, grad_a, grad_g, grad_step, stream);
    case OSSM_DLINOSS_IMEX2: return launch_layer_bwd<OSSM_DLINOSS_IMEX2>(args, grad_a, grad_g, grad_step, stream);
    case OSSM_DLINOSS_IM: return launch_layer_bwd<OSSM_DLINOSS_IM>(args, grad_a, grad_g, grad_step, stream);
    default: return launch_layer_bwd<OSSM_DLINOSS_EX>(args, grad_a, grad_g, grad_step, stream);
  }
}

}  // extern "C"
