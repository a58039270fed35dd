// Selective D-LinOSS: the parameter views and the per-step coefficients of
// the four discretisations (sdlinoss_imex1.cpp:13-31 and siblings), shared by
// the selective D-LinOSS kernels and, for parameters constant over time, by
// the oscillatory-scan kernels (which then run it as a recurrence with
// per-channel constant coefficients).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ossm_scan.h"

namespace ossm {

// One parameter tensor [La, Ba, M]: element (t, ch) lives at
// p[t * t_stride + (by_channel ? ch : ch % M)].
struct ParamView {
  const float* p;
  long long t_stride;  // Ba * M, or 0 when broadcast over time
  int by_channel;      // 1: Ba == B (index by channel); 0: broadcast over batch (index by m)
};

struct SdlParams {
  ParamView a, g, s;
  int M;
};

// Forward / backward of the selective D-LinOSS scan when A, G and step are all
// constant over time (every parameter view has t_stride 0): the recurrence
// then has one set of coefficients per channel and runs on the
// oscillatory-scan kernels (chunk transitions as matrix powers).  The
// backward adds each chunk's share of the gradients of A, G and step into
// grads[p] (B*M floats for a parameter per batch row, M for one broadcast
// over the batch, as the parameter's view says) with float atomics, after
// the launch itself has zeroed them: one launch.
int sdl_tb_forward(int variant, const SdlParams& prm, const void* bu, void* states, int64_t L,
                   int64_t nc, hipStream_t stream);
int sdl_tb_backward(int variant, const SdlParams& prm, const void* bu, const void* states,
                    const void* gout, void* gbu, float* const (&grads)[3], int64_t L, int64_t nc,
                    hipStream_t stream);

namespace {

constexpr float kDtMin = 1e-6f;
constexpr float kDtMax = 1.0f;
constexpr float kClampMin = 1e-6f;

// ---- per-step coefficients -------------------------------------------------
template <int V>
struct SdlCoef {
  float c0, c1, c2;
};

template <int V>
__device__ __forceinline__ float sdl_alpha(float dt, float g) {
  if constexpr (V == OSSM_DLINOSS_IMEX2 || V == OSSM_DLINOSS_EX) return 1.f - dt * g;
  else return 1.f;
}

template <int V>
__device__ __forceinline__ float sdl_s_raw(float dt, float g, float a) {
  if constexpr (V == OSSM_DLINOSS_IMEX1) return 1.f + dt * g;
  else if constexpr (V == OSSM_DLINOSS_IMEX2) return 1.f + dt * dt * a;
  else if constexpr (V == OSSM_DLINOSS_IM) return 1.f + dt * g + dt * dt * a;
  else return 1.f;
}

__device__ __forceinline__ float sdl_dt(float step_raw) {
  return fminf(fmaxf(step_raw, kDtMin), kDtMax);
}

// 1 / S (exactly 1 for ex, which has no implicit part)
template <int V>
__device__ __forceinline__ float sdl_inv(float dt, float g, float a) {
  if constexpr (V == OSSM_DLINOSS_EX) return 1.f;
  else return 1.f / fmaxf(sdl_s_raw<V>(dt, g, a), kClampMin);
}

// The coefficients given 1/S (computed once per step and reused).
template <int V>
__device__ __forceinline__ SdlCoef<V> sdl_coef_inv(float a, float g, float step_raw, float inv) {
  const float dt = sdl_dt(step_raw);
  const float dt2 = dt * dt;
  return {sdl_alpha<V>(dt, g) * inv, -dt2 * a * inv, dt2 * inv};
}

template <int V>
__device__ __forceinline__ float sdl_inv_of(float a, float g, float step_raw) {
  return sdl_inv<V>(sdl_dt(step_raw), g, a);
}

template <int V>
__device__ __forceinline__ SdlCoef<V> sdl_coef(float a, float g, float step_raw) {
  return sdl_coef_inv<V>(a, g, step_raw, sdl_inv_of<V>(a, g, step_raw));
}

// (w, x) -> (c0 w + c1 x + c2 bu, x + w')
template <int V>
__device__ __forceinline__ float4 sdl_step(const SdlCoef<V>& k, float4 s, float2 bu) {
  const float wr = fmaf(k.c0, s.x, fmaf(k.c1, s.z, k.c2 * bu.x));
  const float wi = fmaf(k.c0, s.y, fmaf(k.c1, s.w, k.c2 * bu.y));
  return make_float4(wr, wi, s.z + wr, s.w + wi);
}

// Parameters broadcast over time.  A step's three parameter gradients (as
// sdl_grad_step forms them) are linear in three contractions of the gradient of
// the new w, gw = (lam.x + lam.z, lam.y + lam.w), with the state before the
// step and the input:
//   px = gw . w_prev,  pz = gw . x_prev,  pb = gw . bu
// (gw . (-a x_prev + bu) = pb - a pz; gw . tmpw = alpha px + dt^2 (pb - a pz)),
// with coefficients that depend only on the parameters.  With the parameters
// constant over time the sums of px, pz, pb over the steps give the summed
// gradients; this is that map (sdl_grad_step's formulas with the per-step
// contractions replaced by their sums).
template <int V>
__device__ __forceinline__ void sdl_param_grads_of_sums(float a, float g, float step_raw, float inv,
                                                        float px, float pz, float pb, float& ga,
                                                        float& gg, float& gs) {
  const float dt = sdl_dt(step_raw);
  const float dt2 = dt * dt;
  const float alpha = sdl_alpha<V>(dt, g);
  const float pc = fmaf(-a, pz, pb);
  float gdt = 0.f, gA = 0.f, gG = 0.f;
  float kin = 1.f;  // gtr = gw * kin
  if constexpr (V != OSSM_DLINOSS_EX) {
    const float s_raw = sdl_s_raw<V>(dt, g, a);
    kin = inv;
    const float gS = -fmaf(alpha, px, dt2 * pc) * (inv * inv) * (s_raw > kClampMin ? 1.f : 0.f);
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
  if constexpr (V == OSSM_DLINOSS_IMEX2 || V == OSSM_DLINOSS_EX) {
    gdt += kin * fmaf(-g, px, 2.f * dt * pc);
    gG += kin * (-dt * px);
  } else {
    gdt += kin * (2.f * dt * pc);
  }
  gA += kin * (-dt2 * pz);
  ga = gA;
  gg = gG;
  gs = (step_raw > kDtMin && step_raw < kDtMax) ? gdt : 0.f;
}

}  // namespace
}  // namespace ossm
