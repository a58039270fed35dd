// D-LinOSS model: per-oscillator coefficients, one step of the recurrence, its
// adjoint and the chain rule to (a, g, dt), shared by the scan kernels and the
// fused layer.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/ossm_scan.h"
#include "scan_device.hpp"
#include "scan_reduce.hpp"

namespace ossm {
namespace {

// D-LinOSS per-oscillator coefficients, named as in the reference forward
// kernels:  new0 = c0*s0 + c1*s1 + c2*bu ;  new1 = c3*s0 + c4*s1 + c5*bu,
// except imex1 (new1 = new0 + s1, dlinoss_imex1.cpp:75-78) and ex
// (new1 = c3*s0 + s1, dlinoss_ex.cpp:70-71).
struct DlCoef {
  float c0, c1, c2, c3, c4, c5;
};

template <int V>
struct Dlinoss {
  using In = float2;    // bu_t
  using GIn = float2;   // grad of x_t
  using GOut = float2;  // grad of bu_t
  using Mat = RMat;
  using Coef = DlCoef;
  // Number of per-oscillator sums the variant's chain rule reads (see accumulate).
  static constexpr int kSums =
      (V == OSSM_DLINOSS_IMEX1 || V == OSSM_DLINOSS_EX) ? 3 : (V == OSSM_DLINOSS_IM ? 5 : 6);
  static constexpr bool kRecompute = true;  // s_{t-1} rebuilt from bu and a checkpoint

  struct Params {
    const float* a;
    const float* g;
    const float* dt;
    int P;
  };

  // The raw per-oscillator parameters (a, g, dt), loaded once per chunk.
  struct Raw {
    float a, g, dt;
  };
  static __device__ __forceinline__ Raw load_raw(const Params& prm, int ch) {
    const int p = ch % prm.P;
    return {prm.a[p], prm.g[p], prm.dt[p]};
  }
  static __device__ __forceinline__ Coef coef(const Params& prm, int ch) {
    return coef_of(load_raw(prm, ch));
  }
  // dlinoss_imex1.cpp:32-48, dlinoss_imex2.cpp:35-47, dlinoss_im.cpp:34-50, dlinoss_ex.cpp:33-42
  static __device__ __forceinline__ Coef coef_of(const Raw& r) {
    const float alpha = r.a, gamma = r.g, sigma = r.dt;
    Coef k;
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      const float inv = 1.f / (1.f + sigma * gamma);
      const float s2i = sigma * sigma * inv;
      k = {inv, -alpha * s2i, s2i, 0.f, 0.f, 0.f};
    } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
      const float s2 = sigma * sigma;
      k = {1.f - sigma * gamma, -sigma * alpha, sigma, sigma - s2 * gamma, 1.f - s2 * alpha, s2};
    } else if constexpr (V == OSSM_DLINOSS_IM) {
      const float s2 = sigma * sigma;
      const float inv = 1.f / (1.f + sigma * gamma + s2 * alpha);
      const float si = sigma * inv;
      k = {inv, -alpha * si, si, si, (1.f + sigma * gamma) * inv, s2 * inv};
    } else {
      k = {1.f - sigma * gamma, -sigma * alpha, sigma, sigma, 0.f, 0.f};
    }
    return k;
  }

  static __device__ __forceinline__ float4 step(const Coef& k, float4 s, float2 bu) {
    const float n0r = s.x * k.c0 + s.z * k.c1 + bu.x * k.c2;
    const float n0i = s.y * k.c0 + s.w * k.c1 + bu.y * k.c2;
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      return make_float4(n0r, n0i, n0r + s.z, n0i + s.w);
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      return make_float4(n0r, n0i, s.x * k.c3 + s.z, s.y * k.c3 + s.w);
    } else {
      return make_float4(n0r, n0i, s.x * k.c3 + s.z * k.c4 + bu.x * k.c5,
                         s.y * k.c3 + s.w * k.c4 + bu.y * k.c5);
    }
  }

  // The homogeneous step as a matrix (columns = step of the unit vectors).
  static __device__ __forceinline__ Mat matrix(const Coef& k) {
    const float4 e0 = step(k, make_float4(1.f, 0.f, 0.f, 0.f), make_float2(0.f, 0.f));
    const float4 e1 = step(k, make_float4(0.f, 0.f, 1.f, 0.f), make_float2(0.f, 0.f));
    return {e0.x, e1.x, e0.z, e1.z};
  }

  // mu_t = carry + (0, g_t): the gradient w.r.t. the new state at t
  // (grad_new0 = grad_state0, grad_new1 = grad_state1 + grad_out).
  static __device__ __forceinline__ float4 mu(float4 carry, float2 go) {
    return make_float4(carry.x, carry.y, carry.z + go.x, carry.w + go.y);
  }

  // carry to t-1 = M^T mu_t, in each variant's reference arithmetic
  // (dlinoss_imex1.cpp:200-208, dlinoss_imex2.cpp:222-230, dlinoss_im.cpp:229-237,
  //  dlinoss_ex.cpp:189-197).
  static __device__ __forceinline__ float4 rev_carry(const Coef& k, float4 m) {
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      const float tr = m.x + m.z, ti = m.y + m.w;
      return make_float4(tr * k.c0, ti * k.c0, m.z + tr * k.c1, m.w + ti * k.c1);
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      return make_float4(m.x * k.c0 + m.z * k.c3, m.y * k.c0 + m.w * k.c3, m.x * k.c1 + m.z,
                         m.y * k.c1 + m.w);
    } else {
      return make_float4(m.x * k.c0 + m.z * k.c3, m.y * k.c0 + m.w * k.c3,
                         m.x * k.c1 + m.z * k.c4, m.y * k.c1 + m.w * k.c4);
    }
  }

  // grad_bu_t = f^T mu_t
  static __device__ __forceinline__ float2 grad_input(const Coef& k, float4 m) {
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      return make_float2((m.x + m.z) * k.c2, (m.y + m.w) * k.c2);
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      return make_float2(m.x * k.c2, m.y * k.c2);
    } else {
      return make_float2(m.x * k.c2 + m.z * k.c5, m.y * k.c2 + m.w * k.c5);
    }
  }

  // The chain rule to (a, g, dt) reads the sums G_ij = sum <mu_i, s_j,t-1>
  // and F_i = sum <mu_i, bu_t> (real inner products) only in the
  // combinations below, so each lane accumulates just those:
  //   imex1: G00 + G10, G01 + G11, F0 + F1  (both rows enter through mu0 + mu1)
  //   ex:    G00, G01, F0 + G10
  //   im:    G00, G01, G11, F0 + G10, F1
  //   imex2: G00, G01, G10, G11, F0, F1
  static __device__ __forceinline__ void accumulate(float* acc, float4 m, float4 sp, float2 bu) {
    // acc += p.x * q.x + p.y * q.y as two fused steps
    auto dot = [](float a, float px, float py, float qx, float qy) {
      return fmaf(py, qy, fmaf(px, qx, a));
    };
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      const float tr = m.x + m.z, ti = m.y + m.w;
      acc[0] = dot(acc[0], tr, ti, sp.x, sp.y);
      acc[1] = dot(acc[1], tr, ti, sp.z, sp.w);
      acc[2] = dot(acc[2], tr, ti, bu.x, bu.y);
    } else if constexpr (V == OSSM_DLINOSS_EX) {
      acc[0] = dot(acc[0], m.x, m.y, sp.x, sp.y);
      acc[1] = dot(acc[1], m.x, m.y, sp.z, sp.w);
      acc[2] = dot(dot(acc[2], m.x, m.y, bu.x, bu.y), m.z, m.w, sp.x, sp.y);
    } else if constexpr (V == OSSM_DLINOSS_IM) {
      acc[0] = dot(acc[0], m.x, m.y, sp.x, sp.y);
      acc[1] = dot(acc[1], m.x, m.y, sp.z, sp.w);
      acc[2] = dot(acc[2], m.z, m.w, sp.z, sp.w);
      acc[3] = dot(dot(acc[3], m.x, m.y, bu.x, bu.y), m.z, m.w, sp.x, sp.y);
      acc[4] = dot(acc[4], m.z, m.w, bu.x, bu.y);
    } else {
      acc[0] = dot(acc[0], m.x, m.y, sp.x, sp.y);  // G00
      acc[1] = dot(acc[1], m.x, m.y, sp.z, sp.w);  // G01
      acc[2] = dot(acc[2], m.z, m.w, sp.x, sp.y);  // G10
      acc[3] = dot(acc[3], m.z, m.w, sp.z, sp.w);  // G11
      acc[4] = dot(acc[4], m.x, m.y, bu.x, bu.y);  // F0
      acc[5] = dot(acc[5], m.z, m.w, bu.x, bu.y);  // F1
    }
  }

  // Chain rule from the oscillator's sums (see accumulate) to (a, g, dt):
  // imex1 dlinoss_imex1.cpp:219-232, im dlinoss_im.cpp:236-263, imex2 / ex by
  // differentiating the coefficient tables of dlinoss_imex2.cpp:35-47 /
  // dlinoss_ex.cpp:33-42 (the terms the reference accumulates per step).
  // out0/1/2 = grad_a, grad_g, grad_step.  Linear in S: applied to a share of
  // the sums (channel ch's, of one chunk), it adds that share's contribution
  // to the outputs.
  static constexpr int kOutsPerColumn = 1;
  static constexpr bool kWaveEpilogue = false;  // one lane per channel (see Linoss)
  // the forward may run persistent (105-109 VGPRs, no spills)
  static constexpr bool kPersistForward = true;
  static __device__ void epilogue(const Params& prm, int ch, int /*chunk*/, const double* S,
                                  float* grad_a, float* grad_g, float* grad_step) {
    const int p = ch % prm.P;
    const double a = prm.a[p], g = prm.g[p], dt = prm.dt[p];
    double ga, gg, gs;
    if constexpr (V == OSSM_DLINOSS_IMEX1) {
      const double G0 = S[0], G1 = S[1], F = S[2];  // G00+G10, G01+G11, F0+F1
      const double inv = 1.0 / (1.0 + dt * g);
      const double s2i = dt * dt * inv;
      const double ginv = G0;
      const double gs2i = F - a * G1;
      ga = -s2i * G1;
      const double inv_total = ginv + gs2i * dt * dt;
      gs = gs2i * (2.0 * dt * inv) - inv_total * g * inv * inv;
      gg = -inv_total * dt * inv * inv;
    } else if constexpr (V == OSSM_DLINOSS_IMEX2) {
      const double G00 = S[0], G01 = S[1], G10 = S[2], G11 = S[3], F0 = S[4], F1 = S[5];
      ga = -dt * G01 - dt * dt * G11;
      gg = -dt * G00 - dt * dt * G10;
      gs = -g * G00 - a * G01 + (1.0 - 2.0 * dt * g) * G10 - 2.0 * dt * a * G11 + F0 +
           2.0 * dt * F1;
    } else if constexpr (V == OSSM_DLINOSS_IM) {
      const double G00 = S[0], G01 = S[1], G11 = S[2], F0G10 = S[3], F1 = S[4];
      const double inv = 1.0 / (1.0 + dt * g + dt * dt * a);
      const double si = dt * inv;
      double gsi = F0G10, ginv = G00;
      const double gs2i = F1;
      gsi += G01 * (-a);
      ga = G01 * (-si);
      ginv += G11 * (1.0 + dt * g);
      const double gt = G11 * inv;
      gg = gt * dt;
      gs = gt * g;
      gs += gsi * inv;
      ginv += gsi * dt;
      gs += gs2i * (2.0 * dt * inv);
      ginv += gs2i * dt * dt;
      const double gden = -ginv * inv * inv;
      ga += gden * dt * dt;
      gg += gden * dt;
      gs += gden * (g + 2.0 * dt * a);
    } else {
      const double G00 = S[0], G01 = S[1], F0G10 = S[2];
      ga = -dt * G01;
      gg = -dt * G00;
      gs = -g * G00 - a * G01 + F0G10;
    }
    atomic_put(grad_a + p, ga);
    atomic_put(grad_g + p, gg);
    atomic_put(grad_step + p, gs);
  }
};

}  // namespace
}  // namespace ossm
