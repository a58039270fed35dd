// The complex128 scans on gfx950 that the reference's device kernels dispatch
// besides complex64: D-LinOSS (dlinoss_imex1_cuda.cu:196, 234, and the imex2 /
// im / ex siblings), selective D-LinOSS (sdlinoss_imex1_cuda.cu:232, 271, and
// siblings) and the LinOSS scan (linoss_scan_cuda.cu:139).
// fp64 is the accuracy path, not the hot one: one lane per channel walks the
// sequence, forward in time for the states and in reverse for the adjoint, and
// consecutive lanes own consecutive channels, so every load and store of a
// wave is one contiguous run.
//
// Selective D-LinOSS: recurrence and chain rule of the complex64 kernels
// (sdlinoss_<v>.cpp forward kernels, backward kernels sdlinoss_imex1.cpp:186-220,
// sdlinoss_imex2.cpp:178-221, sdlinoss_im.cpp:176-225,
// sdlinoss_ex.cpp:163-189), in double, with the division by S kept as a
// division:
//   dt = clamp(step, 1e-6, 1), comb = -a x + bu, tmpw = alpha w + dt^2 comb,
//   w' = tmpw / S, x' = x + w'.
// Parameter gradients broadcast over time are summed over time in the lane
// (sequential, fixed order); those broadcast over batch rows are summed over
// the rows afterwards by one lane per output element, also in a fixed order.
//
// LinOSS: s_t = M s_{t-1} + b_t with a complex 2x2 M per oscillator
// (linoss_scan.cpp:11-96); backward g_t = grad_t + M^H g_{t+1}, grad_b_t = g_t,
// grad_M_ij = sum over (b, t) of g_i,t conj(s_j,t-1) (linoss.py:83-151), summed
// over time in the lane and over batch rows afterwards.

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "../../include/ossm_scan.h"
#include "runtime.hpp"

namespace ossm {
namespace {

constexpr double kDtMin64 = 1e-6;
constexpr double kDtMax64 = 1.0;
constexpr double kClampMin64 = 1e-6;
constexpr int kBlock64 = 256;

// One parameter [La, Ba, M]: element (t, channel ch = b M + m) at
// p[t * t_stride + (by_channel ? ch : m)].
struct View64 {
  const double* p;
  long long t_stride;
  int by_channel;
};

struct Params64 {
  View64 v[3];  // a, g, step
  int M;
};

__device__ __forceinline__ double at64(const View64& v, int t, int ch, int m) {
  return v.p[static_cast<size_t>(t) * v.t_stride + (v.by_channel ? ch : m)];
}

template <int V>
__device__ __forceinline__ double alpha64(double dt, double g) {
  if constexpr (V == OSSM_DLINOSS_IMEX2 || V == OSSM_DLINOSS_EX) return 1.0 - dt * g;
  else return 1.0;
}

template <int V>
__device__ __forceinline__ double s_raw64(double dt, double g, double a) {
  if constexpr (V == OSSM_DLINOSS_IMEX1) return 1.0 + dt * g;
  else if constexpr (V == OSSM_DLINOSS_IMEX2) return 1.0 + dt * dt * a;
  else if constexpr (V == OSSM_DLINOSS_IM) return 1.0 + dt * g + dt * dt * a;
  else return 1.0;
}

__device__ __forceinline__ double dt64(double step_raw) {
  return fmin(fmax(step_raw, kDtMin64), kDtMax64);
}

// ---- forward: states[t] = (w_t, x_t) ------------------------------------------
template <int V>
__global__ __launch_bounds__(kBlock64) void sdl64_forward_kernel(Params64 prm,
                                                                 const double2* __restrict__ bu,
                                                                 double2* __restrict__ states,
                                                                 int L, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int m = ch % prm.M;
  double wr = 0.0, wi = 0.0, xr = 0.0, xi = 0.0;
  // unrolled so that the loads of several steps are in flight at once
#pragma unroll 8
  for (int t = 0; t < L; ++t) {
    const double a = at64(prm.v[0], t, ch, m), g = at64(prm.v[1], t, ch, m);
    const double dt = dt64(at64(prm.v[2], t, ch, m));
    const double dt2 = dt * dt, alpha = alpha64<V>(dt, g);
    const double2 b = bu[static_cast<size_t>(t) * nc + ch];
    double tr = alpha * wr + dt2 * (-a * xr + b.x);
    double ti = alpha * wi + dt2 * (-a * xi + b.y);
    if constexpr (V != OSSM_DLINOSS_EX) {
      const double S = fmax(s_raw64<V>(dt, g, a), kClampMin64);
      tr /= S;
      ti /= S;
    }
    wr = tr;
    wi = ti;
    xr += wr;
    xi += wi;
    double2* out = states + 2 * (static_cast<size_t>(t) * nc + ch);
    out[0] = make_double2(wr, wi);
    out[1] = make_double2(xr, xi);
  }
}

// ---- backward -------------------------------------------------------------------
// Where parameter p's gradient goes (mode[p]): 0 = per element at
// out[t * nc + ch] (full shape); 1 = summed over time, written at out[ch];
// 2 = per element, to be summed over the batch rows afterwards.
struct Grads64 {
  double* out[3];
  int mode[3];
};

template <int V>
__global__ __launch_bounds__(kBlock64) void sdl64_backward_kernel(
    Params64 prm, const double2* __restrict__ bu, const double2* __restrict__ states,
    const double2* __restrict__ gout, double2* __restrict__ gin, Grads64 dst, int L, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int m = ch % prm.M;
  // adjoint of the state after step t: (lw, lx); the upstream gradient
  // enters through x
  double lwr = 0.0, lwi = 0.0, lxr = 0.0, lxi = 0.0;
  double tsum[3] = {0.0, 0.0, 0.0};
  for (int t = L - 1; t >= 0; --t) {
    const size_t e = static_cast<size_t>(t) * nc + ch;
    const double2 go = gout[e];
    lxr += go.x;
    lxi += go.y;
    double2 wp = make_double2(0.0, 0.0), xp = make_double2(0.0, 0.0);
    if (t > 0) {
      wp = states[2 * (e - nc)];
      xp = states[2 * (e - nc) + 1];
    }
    const double2 b = bu[e];
    const double a = at64(prm.v[0], t, ch, m), g = at64(prm.v[1], t, ch, m);
    const double step_raw = at64(prm.v[2], t, ch, m);
    const double dt = dt64(step_raw), dt2 = dt * dt, alpha = alpha64<V>(dt, g);
    // gradient w.r.t. the new w, through both components (x' = x + w')
    const double gwr = lwr + lxr, gwi = lwi + lxi;
    const double combr = -a * xp.x + b.x, combi = -a * xp.y + b.y;
    double gdt = 0.0, gA = 0.0, gG = 0.0;
    double gtr = gwr, gti = gwi;  // gradient w.r.t. tmpw
    if constexpr (V != OSSM_DLINOSS_EX) {
      const double s_raw = s_raw64<V>(dt, g, a);
      const double S = fmax(s_raw, kClampMin64);
      const double tmpr = alpha * wp.x + dt2 * combr, tmpi = alpha * wp.y + dt2 * combi;
      gtr = gwr / S;
      gti = gwi / S;
      const double gS = s_raw > kClampMin64 ? -(gwr * tmpr + gwi * tmpi) / (S * S) : 0.0;
      if constexpr (V == OSSM_DLINOSS_IMEX1) {
        gdt = gS * g;
        gG = gS * dt;
      } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
        gdt = gS * (2.0 * dt * a);
        gA = gS * dt2;
      } else {
        gdt = gS * (g + 2.0 * dt * a);
        gA = gS * dt2;
        gG = gS * dt;
      }
    }
    // tmpw = alpha w_prev + dt^2 (-a x_prev + bu)
    if constexpr (V == OSSM_DLINOSS_IMEX2 || V == OSSM_DLINOSS_EX) {
      gdt += gtr * (-g * wp.x + 2.0 * dt * combr) + gti * (-g * wp.y + 2.0 * dt * combi);
      gG += gtr * (-dt * wp.x) + gti * (-dt * wp.y);
    } else {
      gdt += gtr * (2.0 * dt * combr) + gti * (2.0 * dt * combi);
    }
    gA += gtr * (-dt2 * xp.x) + gti * (-dt2 * xp.y);
    gin[e] = make_double2(gtr * dt2, gti * dt2);
    const double gp[3] = {gA, gG, (step_raw > kDtMin64 && step_raw < kDtMax64) ? gdt : 0.0};
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      if (dst.mode[p] == 1) tsum[p] += gp[p];
      else dst.out[p][e] = gp[p];
    }
    // carry to the previous state: d/dw_prev = alpha gt, d/dx_prev = lx - dt^2 a gt
    lwr = alpha * gtr;
    lwi = alpha * gti;
    lxr -= dt2 * a * gtr;
    lxi -= dt2 * a * gti;
  }
#pragma unroll
  for (int p = 0; p < 3; ++p)
    if (dst.mode[p] == 1) dst.out[p][ch] = tsum[p];
}

// out[n * C + c] = sum_{r < R} in[(n R + r) C + c], one lane per output, rows in order.
__global__ __launch_bounds__(kBlock64) void sdl64_rows_sum_kernel(const double* __restrict__ in,
                                                                  double* __restrict__ out,
                                                                  long long n_out, int R, int C) {
  const long long i = static_cast<long long>(blockIdx.x) * kBlock64 + threadIdx.x;
  if (i >= n_out) return;
  const long long n = i / C, c = i - n * C;
  const double* src = in + static_cast<size_t>(n) * R * C + c;
  double s = 0.0;
  for (int r = 0; r < R; ++r) s += src[static_cast<size_t>(r) * C];
  out[i] = s;
}

__global__ __launch_bounds__(kBlock64) void sdl64_zero_kernel(double* __restrict__ p, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * kBlock64 + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

// ---- LinOSS ---------------------------------------------------------------------
__device__ __forceinline__ double2 cmul(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
// conj(a) * b
__device__ __forceinline__ double2 cmulc(double2 a, double2 b) {
  return make_double2(a.x * b.x + a.y * b.y, a.x * b.y - a.y * b.x);
}
__device__ __forceinline__ double2 cadd(double2 a, double2 b) { return make_double2(a.x + b.x, a.y + b.y); }

struct Lin64 {
  const double2* m[4];  // m11, m12, m21, m22, [P] each
  int P;
};

// states [L, nc, 2] and b [L, nc, 2], channel ch = b P + p
__global__ __launch_bounds__(kBlock64) void lin64_forward_kernel(Lin64 mp,
                                                                 const double2* __restrict__ b,
                                                                 double2* __restrict__ states,
                                                                 int L, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int p = ch % mp.P;
  const double2 m11 = mp.m[0][p], m12 = mp.m[1][p], m21 = mp.m[2][p], m22 = mp.m[3][p];
  double2 s0 = make_double2(0.0, 0.0), s1 = s0;
#pragma unroll 8
  for (int t = 0; t < L; ++t) {
    const size_t e = 2 * (static_cast<size_t>(t) * nc + ch);
    const double2 n0 = cadd(cadd(cmul(m11, s0), cmul(m12, s1)), b[e]);
    const double2 n1 = cadd(cadd(cmul(m21, s0), cmul(m22, s1)), b[e + 1]);
    s0 = n0;
    s1 = n1;
    states[e] = s0;
    states[e + 1] = s1;
  }
}

// grad_b [L, nc, 2]; per-channel sums of g_i conj(s_j,t-1) into part[ch][4]
// (i, j row-major), summed over batch rows afterwards
__global__ __launch_bounds__(kBlock64) void lin64_backward_kernel(
    Lin64 mp, const double2* __restrict__ states, const double2* __restrict__ gout,
    double2* __restrict__ gb, double2* __restrict__ part, int L, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int p = ch % mp.P;
  const double2 m11 = mp.m[0][p], m12 = mp.m[1][p], m21 = mp.m[2][p], m22 = mp.m[3][p];
  double2 g0 = make_double2(0.0, 0.0), g1 = g0;  // adjoint of s_{t+1}, then of s_t
  double2 acc[4] = {g0, g0, g0, g0};
  for (int t = L - 1; t >= 0; --t) {
    const size_t e = 2 * (static_cast<size_t>(t) * nc + ch);
    // g_t = grad_t + M^H g_{t+1}
    const double2 h0 = cadd(gout[e], cadd(cmulc(m11, g0), cmulc(m21, g1)));
    const double2 h1 = cadd(gout[e + 1], cadd(cmulc(m12, g0), cmulc(m22, g1)));
    g0 = h0;
    g1 = h1;
    gb[e] = g0;
    gb[e + 1] = g1;
    if (t > 0) {
      const size_t q = e - 2 * static_cast<size_t>(nc);
      const double2 sp0 = states[q], sp1 = states[q + 1];
      // g_i conj(s_j) = conj(conj(g_i) s_j)
      const double2 a00 = cmulc(g0, sp0), a01 = cmulc(g0, sp1), a10 = cmulc(g1, sp0), a11 = cmulc(g1, sp1);
      acc[0] = cadd(acc[0], make_double2(a00.x, -a00.y));
      acc[1] = cadd(acc[1], make_double2(a01.x, -a01.y));
      acc[2] = cadd(acc[2], make_double2(a10.x, -a10.y));
      acc[3] = cadd(acc[3], make_double2(a11.x, -a11.y));
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) part[4 * static_cast<size_t>(ch) + k] = acc[k];
}

// ---- D-LinOSS (time-invariant parameters) ----------------------------------------
// The four variants' coefficient tables, adjoint and chain rule in double, as
// the reference's device kernels run them for complex128 (one thread per
// channel, dlinoss_imex1_cuda.cu:23-172 and siblings):
//   new0 = c0 s0 + c1 s1 + c2 bu ;  new1 = c3 s0 + c4 s1 + c5 bu
// except imex1 (new1 = new0 + s1) and ex (new1 = c3 s0 + s1); tables
// dlinoss_imex1.cpp:32-48, dlinoss_imex2.cpp:35-47, dlinoss_im.cpp:34-50,
// dlinoss_ex.cpp:33-42.  No clamp on dt (the reference applies none).
struct Coef64 {
  double c0, c1, c2, c3, c4, c5;
};

struct DlParams64 {
  const double* a;
  const double* g;
  const double* dt;
  int P;
};

template <int V>
__device__ __forceinline__ Coef64 dl64_coef(double alpha, double gamma, double sigma) {
  if constexpr (V == OSSM_DLINOSS_IMEX1) {
    const double inv = 1.0 / (1.0 + sigma * gamma);
    const double s2i = sigma * sigma * inv;
    return {inv, -alpha * s2i, s2i, 0.0, 0.0, 0.0};
  } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
    const double s2 = sigma * sigma;
    return {1.0 - sigma * gamma, -sigma * alpha, sigma, sigma - s2 * gamma, 1.0 - s2 * alpha, s2};
  } else if constexpr (V == OSSM_DLINOSS_IM) {
    const double s2 = sigma * sigma;
    const double inv = 1.0 / (1.0 + sigma * gamma + s2 * alpha);
    const double si = sigma * inv;
    return {inv, -alpha * si, si, si, (1.0 + sigma * gamma) * inv, s2 * inv};
  } else {
    return {1.0 - sigma * gamma, -sigma * alpha, sigma, sigma, 0.0, 0.0};
  }
}

// Sums per channel the chain rule reads (G_ij = sum <mu_i, s_j,t-1>, F_i =
// sum <mu_i, bu_t>, real inner products of complex numbers), in the
// combinations each variant needs:
//   imex1: G00 + G10, G01 + G11, F0 + F1     ex: G00, G01, F0 + G10
//   im:    G00, G01, G11, F0 + G10, F1       imex2: G00, G01, G10, G11, F0, F1
template <int V>
struct DlSums64 {
  static constexpr int kN =
      (V == OSSM_DLINOSS_IMEX1 || V == OSSM_DLINOSS_EX) ? 3 : (V == OSSM_DLINOSS_IM ? 5 : 6);
};

template <int V>
__global__ __launch_bounds__(kBlock64) void dl64_forward_kernel(DlParams64 prm,
                                                                const double2* __restrict__ bu,
                                                                double2* __restrict__ states,
                                                                int L, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int p = ch % prm.P;
  const Coef64 k = dl64_coef<V>(prm.a[p], prm.g[p], prm.dt[p]);
  double s0r = 0.0, s0i = 0.0, s1r = 0.0, s1i = 0.0;
#pragma unroll 8
  for (int t = 0; t < L; ++t) {
    const size_t e = static_cast<size_t>(t) * nc + ch;
    const double2 b = bu[e];
    const double n0r = s0r * k.c0 + s1r * k.c1 + b.x * k.c2;
    const double n0i = s0i * k.c0 + s1i * k.c1 + b.y * k.c2;
    double n1r, n1i;
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      n1r = n0r + s1r;
      n1i = n0i + s1i;
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      n1r = s0r * k.c3 + s1r;
      n1i = s0i * k.c3 + s1i;
    } else {
      n1r = s0r * k.c3 + s1r * k.c4 + b.x * k.c5;
      n1i = s0i * k.c3 + s1i * k.c4 + b.y * k.c5;
    }
    s0r = n0r;
    s0i = n0i;
    s1r = n1r;
    s1i = n1i;
    states[2 * e] = make_double2(s0r, s0i);
    states[2 * e + 1] = make_double2(s1r, s1i);
  }
}

// Reverse adjoint per channel: mu_t = carry + (0, grad_out_t) (the upstream
// gradient enters through x); grad_bu_t = f^T mu_t; carry to t-1 = M^T mu_t
// (dlinoss_imex1.cpp:200-208, dlinoss_imex2.cpp:222-230, dlinoss_im.cpp:229-237,
// dlinoss_ex.cpp:189-197).  Writes the channel's sums to part[ch * kN + i].
template <int V>
__global__ __launch_bounds__(kBlock64) void dl64_backward_kernel(
    DlParams64 prm, const double2* __restrict__ bu, const double2* __restrict__ states,
    const double2* __restrict__ gout, double2* __restrict__ gin, double* __restrict__ part, int L,
    int nc) {
  constexpr int NS = DlSums64<V>::kN;
  const int ch = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const int p = ch % prm.P;
  const Coef64 k = dl64_coef<V>(prm.a[p], prm.g[p], prm.dt[p]);
  double c0r = 0.0, c0i = 0.0, c1r = 0.0, c1i = 0.0;  // carry: gradient w.r.t. s_t
  double acc[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) acc[i] = 0.0;
  for (int t = L - 1; t >= 0; --t) {
    const size_t e = static_cast<size_t>(t) * nc + ch;
    const double2 go = gout[e], b = bu[e];
    const double m0r = c0r, m0i = c0i, m1r = c1r + go.x, m1i = c1i + go.y;
    double2 sp0 = make_double2(0.0, 0.0), sp1 = sp0;  // s_{t-1} (zero before the first step)
    if (t > 0) {
      sp0 = states[2 * (e - nc)];
      sp1 = states[2 * (e - nc) + 1];
    }
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      const double tr = m0r + m1r, ti = m0i + m1i;
      acc[0] += tr * sp0.x + ti * sp0.y;
      acc[1] += tr * sp1.x + ti * sp1.y;
      acc[2] += tr * b.x + ti * b.y;
      gin[e] = make_double2(tr * k.c2, ti * k.c2);
      c0r = tr * k.c0;
      c0i = ti * k.c0;
      c1r = m1r + tr * k.c1;
      c1i = m1i + ti * k.c1;
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      acc[0] += m0r * sp0.x + m0i * sp0.y;
      acc[1] += m0r * sp1.x + m0i * sp1.y;
      acc[2] += m0r * b.x + m0i * b.y + m1r * sp0.x + m1i * sp0.y;
      gin[e] = make_double2(m0r * k.c2, m0i * k.c2);
      c0r = m0r * k.c0 + m1r * k.c3;
      c0i = m0i * k.c0 + m1i * k.c3;
      c1r = m0r * k.c1 + m1r;
      c1i = m0i * k.c1 + m1i;
    } else {
      if constexpr (V == OSSM_DLINOSS_IM) {
        acc[0] += m0r * sp0.x + m0i * sp0.y;
        acc[1] += m0r * sp1.x + m0i * sp1.y;
        acc[2] += m1r * sp1.x + m1i * sp1.y;
        acc[3] += m0r * b.x + m0i * b.y + m1r * sp0.x + m1i * sp0.y;
        acc[4] += m1r * b.x + m1i * b.y;
      } else {
        acc[0] += m0r * sp0.x + m0i * sp0.y;
        acc[1] += m0r * sp1.x + m0i * sp1.y;
        acc[2] += m1r * sp0.x + m1i * sp0.y;
        acc[3] += m1r * sp1.x + m1i * sp1.y;
        acc[4] += m0r * b.x + m0i * b.y;
        acc[5] += m1r * b.x + m1i * b.y;
      }
      gin[e] = make_double2(m0r * k.c2 + m1r * k.c5, m0i * k.c2 + m1i * k.c5);
      c0r = m0r * k.c0 + m1r * k.c3;
      c0i = m0i * k.c0 + m1i * k.c3;
      c1r = m0r * k.c1 + m1r * k.c4;
      c1i = m0i * k.c1 + m1i * k.c4;
    }
  }
#pragma unroll
  for (int i = 0; i < NS; ++i) part[static_cast<size_t>(ch) * NS + i] = acc[i];
}

// One lane per oscillator p: the channel sums of the B batch rows added in
// row order, then the chain rule to (a, g, dt) — imex1 dlinoss_imex1.cpp:219-232,
// im dlinoss_im.cpp:236-263, imex2 / ex by differentiating the coefficient
// tables (the terms the reference accumulates per step).
template <int V>
__global__ __launch_bounds__(kBlock64) void dl64_param_kernel(DlParams64 prm,
                                                              const double* __restrict__ part,
                                                              double* __restrict__ grad_a,
                                                              double* __restrict__ grad_g,
                                                              double* __restrict__ grad_step,
                                                              int B) {
  constexpr int NS = DlSums64<V>::kN;
  const int p = static_cast<int>(blockIdx.x) * kBlock64 + static_cast<int>(threadIdx.x);
  if (p >= prm.P) return;
  double S[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) S[i] = 0.0;
  for (int b = 0; b < B; ++b) {
    const double* src = part + (static_cast<size_t>(b) * prm.P + p) * NS;
#pragma unroll
    for (int i = 0; i < NS; ++i) S[i] += src[i];
  }
  const double a = prm.a[p], g = prm.g[p], dt = prm.dt[p];
  double ga, gg, gs;
  if constexpr (V == OSSM_DLINOSS_IMEX1) {
    const double inv = 1.0 / (1.0 + dt * g);
    const double s2i = dt * dt * inv;
    const double gs2i = S[2] - a * S[1];
    ga = -s2i * S[1];
    const double inv_total = S[0] + gs2i * dt * dt;
    gs = gs2i * (2.0 * dt * inv) - inv_total * g * inv * inv;
    gg = -inv_total * dt * inv * inv;
  } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
    ga = -dt * S[1] - dt * dt * S[3];
    gg = -dt * S[0] - dt * dt * S[2];
    gs = -g * S[0] - a * S[1] + (1.0 - 2.0 * dt * g) * S[2] - 2.0 * dt * a * S[3] + S[4] +
         2.0 * dt * S[5];
  } else if constexpr (V == OSSM_DLINOSS_IM) {
    const double inv = 1.0 / (1.0 + dt * g + dt * dt * a);
    const double si = dt * inv;
    const double gsi = S[3] - a * S[1];
    double ginv = S[0] + S[2] * (1.0 + dt * g);
    const double gt = S[2] * inv;
    ga = -si * S[1];
    gg = gt * dt;
    gs = gt * g + gsi * inv + S[4] * (2.0 * dt * inv);
    ginv += gsi * dt + S[4] * dt * dt;
    const double gden = -ginv * inv * inv;
    ga += gden * dt * dt;
    gg += gden * dt;
    gs += gden * (g + 2.0 * dt * a);
  } else {
    ga = -dt * S[1];
    gg = -dt * S[0];
    gs = -g * S[0] - a * S[1] + S[2];
  }
  grad_a[p] = ga;
  grad_g[p] = gg;
  grad_step[p] = gs;
}

unsigned blocks_for(long long n) { return static_cast<unsigned>((n + kBlock64 - 1) / kBlock64); }

struct Shape64 {
  const double* p;
  int64_t la, ba;
};

int check64(int variant, const Shape64 (&s)[3], int64_t L, int64_t B, int64_t M, const char* what) {
  if (variant < 0 || variant > 3)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown selective D-LinOSS variant code");
  if (L < 0 || B < 0 || M < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (L > INT_MAX / 2 || B * M > INT_MAX / 2 || L * B * M > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  const char* names[3] = {"A", "G", "step"};
  for (int p = 0; p < 3; ++p) {
    if (s[p].p == nullptr)
      return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": null " + names[p]);
    if (!(s[p].la == 1 || s[p].la == L) || !(s[p].ba == 1 || s[p].ba == B))
      return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(names[p]) +
                                                      " must have shape (L,B,M) with optional singleton L/B axes");
  }
  return OSSM_OK;
}

Params64 params64(const Shape64 (&s)[3], int64_t L, int64_t B, int64_t M) {
  Params64 prm{};
  for (int p = 0; p < 3; ++p) {
    prm.v[p].p = s[p].p;
    prm.v[p].t_stride = (s[p].la == 1 && L > 1) ? 0 : s[p].ba * M;
    prm.v[p].by_channel = s[p].ba == B ? 1 : 0;
  }
  prm.M = static_cast<int>(M);
  return prm;
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_sdlinoss_forward_f64(int variant, const double* A, int64_t a_len, int64_t a_batch,
                              const double* G, int64_t g_len, int64_t g_batch, const double* step,
                              int64_t s_len, int64_t s_batch, const void* bu, void* states,
                              int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  const Shape64 shapes[3] = {{A, a_len, a_batch}, {G, g_len, g_batch}, {step, s_len, s_batch}};
  if (length == 0 || batch == 0 || ssm == 0) {
    if (variant < 0 || variant > 3)
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown selective D-LinOSS variant code");
    return OSSM_OK;
  }
  if (int rc = check64(variant, shapes, length, batch, ssm, "sdlinoss_forward_f64")) return rc;
  if (!bu || !states) return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_forward_f64: null pointer");
  const Params64 prm = params64(shapes, length, batch, ssm);
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const int nc = static_cast<int>(batch * ssm), L = static_cast<int>(length);
  const auto* b = static_cast<const double2*>(bu);
  auto* st = static_cast<double2*>(states);
  switch (variant) {
#define OSSM_SDL64_FWD(V)                                                                         \
  case V:                                                                                         \
    hipLaunchKernelGGL(sdl64_forward_kernel<V>, dim3(blocks_for(nc)), dim3(kBlock64), 0, stream, \
                       prm, b, st, L, nc);                                                        \
    break;
    OSSM_SDL64_FWD(OSSM_DLINOSS_IMEX1)
    OSSM_SDL64_FWD(OSSM_DLINOSS_IMEX2)
    OSSM_SDL64_FWD(OSSM_DLINOSS_IM)
    OSSM_SDL64_FWD(OSSM_DLINOSS_EX)
#undef OSSM_SDL64_FWD
  }
  return launch_check("sdl64_forward_kernel");
}

int ossm_sdlinoss_backward_f64(int variant, const double* A, int64_t a_len, int64_t a_batch,
                               const double* G, int64_t g_len, int64_t g_batch,
                               const double* step, int64_t s_len, int64_t s_batch, const void* bu,
                               const void* states, const void* grad_output, double* grad_A,
                               double* grad_G, double* grad_step, void* grad_bu, int64_t length,
                               int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  StreamCall call(stream);
  if (call.status()) return call.status();
  const Shape64 shapes[3] = {{A, a_len, a_batch}, {G, g_len, g_batch}, {step, s_len, s_batch}};
  double* const grads[3] = {grad_A, grad_G, grad_step};
  if (length == 0 || batch == 0 || ssm == 0) {
    if (variant < 0 || variant > 3)
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown selective D-LinOSS variant code");
    // nothing to scan: zero parameter gradients (the reference's zeros_like)
    for (int p = 0; p < 3; ++p) {
      if (grads[p] == nullptr)
        return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_backward_f64: null pointer");
      const long long n = shapes[p].la * shapes[p].ba * ssm;
      if (n <= 0) continue;
      hipLaunchKernelGGL(sdl64_zero_kernel, dim3(blocks_for(n)), dim3(kBlock64), 0, stream,
                         grads[p], n);
      if (int rc = launch_check("sdl64_zero_kernel")) return rc;
    }
    return OSSM_OK;
  }
  if (int rc = check64(variant, shapes, length, batch, ssm, "sdlinoss_backward_f64")) return rc;
  if (!bu || !states || !grad_output || !grad_A || !grad_G || !grad_step || !grad_bu)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "sdlinoss_backward_f64: null pointer");
  const Params64 prm = params64(shapes, length, batch, ssm);
  const int64_t nc = batch * ssm;

  // gradients summed over batch rows go through a workspace first:
  // [L, B, M] per element (broadcast over batch only) or [B, M] time sums
  // (broadcast over both)
  Grads64 dst{};
  bool rb[3];
  size_t offs[3] = {0, 0, 0}, ws_doubles = 0;
  for (int p = 0; p < 3; ++p) {
    const bool rt = shapes[p].la == 1 && length > 1;
    rb[p] = shapes[p].ba == 1 && batch > 1;
    dst.mode[p] = rt ? 1 : (rb[p] ? 2 : 0);
    if (rb[p]) {
      offs[p] = ws_doubles;
      ws_doubles += static_cast<size_t>(rt ? 1 : length) * nc;
    }
  }
  double* ws = nullptr;
  if (ws_doubles > 0) {
    void* raw = nullptr;
    if (int rc = acquire_workspace(call, ws_doubles * sizeof(double), &raw)) return rc;
    ws = static_cast<double*>(raw);
  }
  for (int p = 0; p < 3; ++p) dst.out[p] = rb[p] ? ws + offs[p] : grads[p];

  const int n = static_cast<int>(nc), L = static_cast<int>(length);
  const auto* b = static_cast<const double2*>(bu);
  const auto* st = static_cast<const double2*>(states);
  const auto* go = static_cast<const double2*>(grad_output);
  auto* gi = static_cast<double2*>(grad_bu);
  switch (variant) {
#define OSSM_SDL64_BWD(V)                                                                          \
  case V:                                                                                          \
    hipLaunchKernelGGL(sdl64_backward_kernel<V>, dim3(blocks_for(n)), dim3(kBlock64), 0, stream, \
                       prm, b, st, go, gi, dst, L, n);                                             \
    break;
    OSSM_SDL64_BWD(OSSM_DLINOSS_IMEX1)
    OSSM_SDL64_BWD(OSSM_DLINOSS_IMEX2)
    OSSM_SDL64_BWD(OSSM_DLINOSS_IM)
    OSSM_SDL64_BWD(OSSM_DLINOSS_EX)
#undef OSSM_SDL64_BWD
  }
  if (int rc = launch_check("sdl64_backward_kernel")) return rc;
  for (int p = 0; p < 3; ++p) {
    if (!rb[p]) continue;
    // [R=B rows] summed: (L or 1) outputs of M columns each
    const long long rows_out = dst.mode[p] == 1 ? 1 : length;
    const long long n_out = rows_out * ssm;
    hipLaunchKernelGGL(sdl64_rows_sum_kernel, dim3(blocks_for(n_out)), dim3(kBlock64), 0, stream,
                       dst.out[p], grads[p], n_out, static_cast<int>(batch), static_cast<int>(ssm));
    if (int rc = launch_check("sdl64_rows_sum_kernel")) return rc;
  }
  return OSSM_OK;
}

int ossm_linoss_forward_f64(const void* m11, const void* m12, const void* m21, const void* m22,
                            const void* b_seq, void* states, int64_t length, int64_t batch,
                            int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (length < 0 || batch < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_forward_f64: negative size");
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (length > INT_MAX / 2 || batch * ssm > INT_MAX / 2 || length * batch * ssm > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, "linoss_forward_f64: size exceeds 32-bit indexing");
  if (!m11 || !m12 || !m21 || !m22 || !b_seq || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_forward_f64: null pointer");
  const Lin64 mp{{static_cast<const double2*>(m11), static_cast<const double2*>(m12),
                  static_cast<const double2*>(m21), static_cast<const double2*>(m22)},
                 static_cast<int>(ssm)};
  const int nc = static_cast<int>(batch * ssm);
  hipLaunchKernelGGL(lin64_forward_kernel, dim3(blocks_for(nc)), dim3(kBlock64), 0,
                     static_cast<hipStream_t>(stream_v), mp, static_cast<const double2*>(b_seq),
                     static_cast<double2*>(states), static_cast<int>(length), nc);
  return launch_check("lin64_forward_kernel");
}

int ossm_linoss_backward_f64(const void* m11, const void* m12, const void* m21, const void* m22,
                             const void* states, const void* grad_output, void* grad_m,
                             void* grad_b, int64_t length, int64_t batch, int64_t ssm,
                             ossm_stream_t stream_v) {
  clear_error();
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  StreamCall call(stream);
  if (call.status()) return call.status();
  if (length < 0 || batch < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_backward_f64: negative size");
  if (length > INT_MAX / 2 || batch * ssm > INT_MAX / 2 || length * batch * ssm > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, "linoss_backward_f64: size exceeds 32-bit indexing");
  if (!grad_m) return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_backward_f64: null pointer");
  const long long n_m = 8 * ssm;  // [P, 2, 2] complex128 as doubles
  if (length == 0 || batch == 0 || ssm == 0) {
    if (n_m > 0) {
      hipLaunchKernelGGL(sdl64_zero_kernel, dim3(blocks_for(n_m)), dim3(kBlock64), 0, stream,
                         static_cast<double*>(grad_m), n_m);
      return launch_check("sdl64_zero_kernel");
    }
    return OSSM_OK;
  }
  if (!m11 || !m12 || !m21 || !m22 || !states || !grad_output || !grad_b)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "linoss_backward_f64: null pointer");
  const Lin64 mp{{static_cast<const double2*>(m11), static_cast<const double2*>(m12),
                  static_cast<const double2*>(m21), static_cast<const double2*>(m22)},
                 static_cast<int>(ssm)};
  const int nc = static_cast<int>(batch * ssm);
  void* raw = nullptr;
  if (int rc = acquire_workspace(call, static_cast<size_t>(nc) * 4 * sizeof(double2), &raw)) return rc;
  hipLaunchKernelGGL(lin64_backward_kernel, dim3(blocks_for(nc)), dim3(kBlock64), 0, stream, mp,
                     static_cast<const double2*>(states), static_cast<const double2*>(grad_output),
                     static_cast<double2*>(grad_b), static_cast<double2*>(raw),
                     static_cast<int>(length), nc);
  if (int rc = launch_check("lin64_backward_kernel")) return rc;
  // [B rows][P * 8 doubles] summed over the rows, in order
  hipLaunchKernelGGL(sdl64_rows_sum_kernel, dim3(blocks_for(n_m)), dim3(kBlock64), 0, stream,
                     static_cast<const double*>(raw), static_cast<double*>(grad_m), n_m,
                     static_cast<int>(batch), static_cast<int>(n_m));
  return launch_check("sdl64_rows_sum_kernel");
}

int ossm_dlinoss_forward_f64(int variant, const double* a_diag, const double* g_diag,
                             const double* step, const void* bu, void* states, int64_t length,
                             int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (variant < OSSM_DLINOSS_IMEX1 || variant > OSSM_DLINOSS_EX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  if (length < 0 || batch < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_forward_f64: negative size");
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (length > INT_MAX / 2 || batch * ssm > INT_MAX / 2 || length * batch * ssm > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, "dlinoss_forward_f64: size exceeds 32-bit indexing");
  if (!a_diag || !g_diag || !step || !bu || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_forward_f64: null pointer");
  const DlParams64 prm{a_diag, g_diag, step, static_cast<int>(ssm)};
  const int nc = static_cast<int>(batch * ssm), L = static_cast<int>(length);
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const auto* b = static_cast<const double2*>(bu);
  auto* st = static_cast<double2*>(states);
  switch (variant) {
#define OSSM_DL64_FWD(V)                                                                         \
  case V:                                                                                        \
    hipLaunchKernelGGL(dl64_forward_kernel<V>, dim3(blocks_for(nc)), dim3(kBlock64), 0, stream, \
                       prm, b, st, L, nc);                                                       \
    break;
    OSSM_DL64_FWD(OSSM_DLINOSS_IMEX1)
    OSSM_DL64_FWD(OSSM_DLINOSS_IMEX2)
    OSSM_DL64_FWD(OSSM_DLINOSS_IM)
    OSSM_DL64_FWD(OSSM_DLINOSS_EX)
#undef OSSM_DL64_FWD
  }
  return launch_check("dl64_forward_kernel");
}

int ossm_dlinoss_backward_f64(int variant, const double* a_diag, const double* g_diag,
                              const double* step, const void* bu, const void* states,
                              const void* grad_output, double* grad_a, double* grad_g,
                              double* grad_step, void* grad_bu, int64_t length, int64_t batch,
                              int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  StreamCall call(stream);
  if (call.status()) return call.status();
  if (variant < OSSM_DLINOSS_IMEX1 || variant > OSSM_DLINOSS_EX)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  if (length < 0 || batch < 0 || ssm < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_backward_f64: negative size");
  if (ssm == 0) return OSSM_OK;
  if (!grad_a || !grad_g || !grad_step)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_backward_f64: null pointer");
  if (length == 0 || batch == 0) {
    // nothing to scan: zero parameter gradients (the reference's zeros_like)
    double* const outs[3] = {grad_a, grad_g, grad_step};
    for (double* o : outs) {
      hipLaunchKernelGGL(sdl64_zero_kernel, dim3(blocks_for(ssm)), dim3(kBlock64), 0, stream, o,
                         static_cast<long long>(ssm));
      if (int rc = launch_check("sdl64_zero_kernel")) return rc;
    }
    return OSSM_OK;
  }
  if (length > INT_MAX / 2 || batch * ssm > INT_MAX / 2 || length * batch * ssm > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, "dlinoss_backward_f64: size exceeds 32-bit indexing");
  if (!a_diag || !g_diag || !step || !bu || !states || !grad_output || !grad_bu)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_backward_f64: null pointer");
  const DlParams64 prm{a_diag, g_diag, step, static_cast<int>(ssm)};
  const int nc = static_cast<int>(batch * ssm), L = static_cast<int>(length);
  void* raw = nullptr;
  if (int rc = acquire_workspace(call, static_cast<size_t>(nc) * 6 * sizeof(double), &raw)) return rc;
  auto* part = static_cast<double*>(raw);
  const auto* b = static_cast<const double2*>(bu);
  const auto* st = static_cast<const double2*>(states);
  const auto* go = static_cast<const double2*>(grad_output);
  auto* gi = static_cast<double2*>(grad_bu);
  const int B = static_cast<int>(batch);
  switch (variant) {
#define OSSM_DL64_BWD(V)                                                                          \
  case V:                                                                                         \
    hipLaunchKernelGGL(dl64_backward_kernel<V>, dim3(blocks_for(nc)), dim3(kBlock64), 0, stream, \
                       prm, b, st, go, gi, part, L, nc);                                          \
    if (int rc = launch_check("dl64_backward_kernel")) return rc;                                 \
    hipLaunchKernelGGL(dl64_param_kernel<V>, dim3(blocks_for(ssm)), dim3(kBlock64), 0, stream,   \
                       prm, part, grad_a, grad_g, grad_step, B);                                  \
    break;
    OSSM_DL64_BWD(OSSM_DLINOSS_IMEX1)
    OSSM_DL64_BWD(OSSM_DLINOSS_IMEX2)
    OSSM_DL64_BWD(OSSM_DLINOSS_IM)
    OSSM_DL64_BWD(OSSM_DLINOSS_EX)
#undef OSSM_DL64_BWD
  }
  return launch_check("dl64_param_kernel");
}

}  // extern "C"
