/*
 * Body of the CPU oracle, included twice by scan_oracle.c: once with
 * REAL=float / SFX(x)=x##_f32 and once with REAL=double / SFX(x)=x##_f64.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU kernels, used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker.  The product path never links it.
 *
 * Complex tensors are interleaved (re, im) pairs, exactly the memory layout
 * of c10::complex / torch.complex64 that the reference kernels walk.
 *
 * Variant codes: 0 = imex1, 1 = imex2, 2 = im, 3 = ex.
 */

/* ------------------------------------------------------------------------ */
/* D-LinOSS forward                                                          */
/* ------------------------------------------------------------------------ */

/*
 * Coefficients of  new0 = c00*s0 + c01*s1 + f0*bu,  new1 = c10*s0 + c11*s1 + f1*bu
 * exactly as the reference forward kernels derive them:
 *   imex1: dlinoss_imex1.cpp:32-48  (new1 = new0 + s1, :75-78)
 *   imex2: dlinoss_imex2.cpp:35-47
 *   im:    dlinoss_im.cpp:34-50
 *   ex:    dlinoss_ex.cpp:33-42      (new1 = dt*s0 + s1, :70-71)
 */
static void SFX(dlinoss_coeffs)(int variant, REAL alpha, REAL gamma, REAL sigma, REAL c[6]) {
  switch (variant) {
    case 0: { /* imex1 */
      const REAL denom = (REAL)1 + sigma * gamma;
      const REAL inv = (REAL)1 / denom;
      const REAL s2i = sigma * sigma * inv;
      c[0] = inv;           /* s0 -> new0 */
      c[1] = -alpha * s2i;  /* s1 -> new0 (coeff12) */
      c[2] = s2i;           /* bu -> new0 */
      c[3] = 0; c[4] = 0; c[5] = 0; /* new1 = new0 + s1, handled in the loop */
      break;
    }
    case 1: { /* imex2 */
      const REAL s2 = sigma * sigma;
      c[0] = (REAL)1 - sigma * gamma;
      c[1] = -sigma * alpha;
      c[2] = sigma;
      c[3] = sigma - s2 * gamma;
      c[4] = (REAL)1 - s2 * alpha;
      c[5] = s2;
      break;
    }
    case 2: { /* im */
      const REAL s2 = sigma * sigma;
      const REAL denom = (REAL)1 + sigma * gamma + s2 * alpha;
      const REAL inv = (REAL)1 / denom;
      const REAL si = sigma * inv;
      const REAL s2i = s2 * inv;
      c[0] = inv;
      c[1] = -alpha * si;
      c[2] = si;
      c[3] = si;
      c[4] = ((REAL)1 + sigma * gamma) * inv;
      c[5] = s2i;
      break;
    }
    default: { /* ex */
      c[0] = (REAL)1 - sigma * gamma;
      c[1] = -sigma * alpha;
      c[2] = sigma;
      c[3] = sigma;
      c[4] = 0; c[5] = 0; /* new1 = sigma*s0 + s1, handled in the loop */
      break;
    }
  }
}

/*
 * States s_t = M s_{t-1} + f bu_t per (b, p) channel, s_{-1} = 0.
 * Loop order follows dlinoss_<v>.cpp forward kernels: parallel over the
 * oscillator index p, then batch, then time (e.g. dlinoss_imex1.cpp:51-93).
 * bu: [L, B, P] complex, out: [L, B, P, 2] complex.
 */
void SFX(oracle_dlinoss_forward)(int variant, const REAL* a_diag, const REAL* g_diag,
                                 const REAL* step, const REAL* bu, REAL* out,
                                 int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < ssm; ++p) {
    REAL c[6];
    SFX(dlinoss_coeffs)(variant, a_diag[p], g_diag[p], step[p], c);
    for (int64_t b = 0; b < batch; ++b) {
      const int64_t ch = b * ssm + p;
      REAL s0r = 0, s0i = 0, s1r = 0, s1i = 0;
      for (int64_t t = 0; t < length; ++t) {
        const REAL bur = bu[2 * (t * series + ch)];
        const REAL bui = bu[2 * (t * series + ch) + 1];
        REAL n0r, n0i, n1r, n1i;
        if (variant == 0) {
          n0r = s0r * c[0] + s1r * c[1] + bur * c[2];
          n0i = s0i * c[0] + s1i * c[1] + bui * c[2];
          n1r = n0r + s1r;
          n1i = n0i + s1i;
        } else if (variant == 3) {
          n0r = s0r * c[0] + s1r * c[1] + bur * c[2];
          n0i = s0i * c[0] + s1i * c[1] + bui * c[2];
          n1r = s0r * c[3] + s1r;
          n1i = s0i * c[3] + s1i;
        } else {
          n0r = s0r * c[0] + s1r * c[1] + bur * c[2];
          n0i = s0i * c[0] + s1i * c[1] + bui * c[2];
          n1r = s0r * c[3] + s1r * c[4] + bur * c[5];
          n1i = s0i * c[3] + s1i * c[4] + bui * c[5];
        }
        REAL* o = out + 4 * (t * series + ch);
        o[0] = n0r; o[1] = n0i; o[2] = n1r; o[3] = n1i;
        s0r = n0r; s0i = n0i; s1r = n1r; s1i = n1i;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* D-LinOSS backward                                                         */
/* ------------------------------------------------------------------------ */

/*
 * Reverse adjoint recurrence with per-oscillator parameter-gradient sums kept
 * in one accumulator each, in the reference's order (batch outer, time
 * reversed inner):
 *   imex1: dlinoss_imex1.cpp:96-235   imex2: dlinoss_imex2.cpp:95-250
 *   im:    dlinoss_im.cpp:101-268     ex:    dlinoss_ex.cpp:88-216
 *
 * grad_out is the gradient w.r.t. component 1 (x) of the states.  grad_aux
 * (may be NULL) is an oracle-only extension: a gradient w.r.t. component 0
 * added to grad_new0 the same way grad_out is added to grad_new1.  With
 * grad_aux == NULL the arithmetic is the reference's.  It exists so the
 * layer-level golden fixture, whose loss also touches the auxiliary state,
 * can pin this function.
 */
void SFX(oracle_dlinoss_backward)(int variant, const REAL* a_diag, const REAL* g_diag,
                                  const REAL* step, const REAL* bu, const REAL* states,
                                  const REAL* grad_out, const REAL* grad_aux, REAL* grad_bu,
                                  REAL* grad_a, REAL* grad_g, REAL* grad_step,
                                  int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < ssm; ++p) {
    const REAL alpha = a_diag[p];
    const REAL gamma = g_diag[p];
    const REAL sigma = step[p];
    const REAL s2 = sigma * sigma;
    REAL c[6];
    SFX(dlinoss_coeffs)(variant, alpha, gamma, sigma, c);

    /* accumulators, named after the reference's */
    REAL acc_alpha = 0, acc_gamma = 0, acc_sigma = 0;          /* imex2, ex */
    REAL acc_s2i = 0, acc_inv = 0;                              /* imex1 (+ acc_alpha) */
    REAL acc_c12 = 0, acc_c22 = 0, acc_si = 0, acc_s2i_im = 0, acc_inv_im = 0; /* im */

    /* imex2 per-oscillator derivative factors, dlinoss_imex2.cpp:135-137 */
    const REAL dsp0 = (REAL)1 - (REAL)2 * sigma * gamma;
    const REAL dsp1 = -(REAL)2 * sigma * alpha;
    const REAL dsbu = (REAL)2 * sigma;

    for (int64_t b = 0; b < batch; ++b) {
      const int64_t ch = b * ssm + p;
      REAL g0r = 0, g0i = 0, g1r = 0, g1i = 0;
      for (int64_t t = length - 1; t >= 0; --t) {
        const int64_t idx = t * series + ch;
        const REAL gor = grad_out[2 * idx], goi = grad_out[2 * idx + 1];
        const REAL bur = bu[2 * idx], bui = bu[2 * idx + 1];
        REAL p0r = 0, p0i = 0, p1r = 0, p1i = 0;
        if (t > 0) {
          const REAL* pv = states + 4 * ((t - 1) * series + ch);
          p0r = pv[0]; p0i = pv[1]; p1r = pv[2]; p1i = pv[3];
        }
        const REAL n1r = g1r + gor, n1i = g1i + goi;
        REAL n0r = g0r, n0i = g0i;
        if (grad_aux) { n0r += grad_aux[2 * idx]; n0i += grad_aux[2 * idx + 1]; }
        REAL gbr, gbi, q0r, q0i, q1r, q1i;

        if (variant == 0) { /* imex1, dlinoss_imex1.cpp:170-208 */
          const REAL inv = c[0], c12 = c[1], s2i = c[2];
          const REAL tr = n0r + n1r, ti = n0i + n1i;
          const REAL combr = bur - alpha * p1r, combi = bui - alpha * p1i;
          acc_s2i += tr * combr + ti * combi;
          acc_alpha += tr * (-s2i * p1r) + ti * (-s2i * p1i);
          acc_inv += tr * p0r + ti * p0i;
          gbr = tr * s2i; gbi = ti * s2i;
          q0r = tr * inv; q0i = ti * inv;
          q1r = n1r + tr * c12; q1i = n1i + ti * c12;
        } else if (variant == 1) { /* imex2, dlinoss_imex2.cpp:193-224 */
          acc_alpha += (-sigma) * (n0r * p1r + n0i * p1i);
          acc_alpha += (-s2) * (n1r * p1r + n1i * p1i);
          acc_gamma += (-sigma) * (n0r * p0r + n0i * p0i);
          acc_gamma += (-s2) * (n1r * p0r + n1i * p0i);
          const REAL str = p0r * (-gamma) + p1r * (-alpha) + bur;
          const REAL sti = p0i * (-gamma) + p1i * (-alpha) + bui;
          acc_sigma += n0r * str + n0i * sti;
          const REAL sgr = p0r * dsp0 + p1r * dsp1 + bur * dsbu;
          const REAL sgi = p0i * dsp0 + p1i * dsp1 + bui * dsbu;
          acc_sigma += n1r * sgr + n1i * sgi;
          gbr = n0r * sigma + n1r * s2; gbi = n0i * sigma + n1i * s2;
          q0r = n0r * c[0] + n1r * c[3]; q0i = n0i * c[0] + n1i * c[3];
          q1r = n0r * c[1] + n1r * c[4]; q1i = n0i * c[1] + n1i * c[4];
        } else if (variant == 2) { /* im, dlinoss_im.cpp:205-227 */
          acc_c12 += n0r * p1r + n0i * p1i;
          acc_c22 += n1r * p1r + n1i * p1i;
          acc_si += n0r * bur + n0i * bui;
          acc_si += n1r * p0r + n1i * p0i;
          acc_s2i_im += n1r * bur + n1i * bui;
          acc_inv_im += n0r * p0r + n0i * p0i;
          gbr = n0r * c[2] + n1r * c[5]; gbi = n0i * c[2] + n1i * c[5];
          q0r = n0r * c[0] + n1r * c[3]; q0i = n0i * c[0] + n1i * c[3];
          q1r = n0r * c[1] + n1r * c[4]; q1i = n0i * c[1] + n1i * c[4];
        } else { /* ex, dlinoss_ex.cpp:171-193 */
          acc_alpha += (-sigma) * (n0r * p1r + n0i * p1i);
          acc_gamma += (-sigma) * (n0r * p0r + n0i * p0i);
          const REAL str = p0r * (-gamma) + p1r * (-alpha) + bur;
          const REAL sti = p0i * (-gamma) + p1i * (-alpha) + bui;
          acc_sigma += n0r * str + n0i * sti;
          acc_sigma += n1r * p0r + n1i * p0i;
          gbr = n0r * sigma; gbi = n0i * sigma;
          q0r = n0r * c[0] + n1r * c[3]; q0i = n0i * c[0] + n1i * c[3];
          q1r = n0r * c[1] + n1r; q1i = n0i * c[1] + n1i;
        }
        grad_bu[2 * idx] = gbr;
        grad_bu[2 * idx + 1] = gbi;
        g0r = q0r; g0i = q0i; g1r = q1r; g1i = q1i;
      }
    }

    /* per-variant chain rule to (alpha, gamma, sigma) */
    if (variant == 0) { /* dlinoss_imex1.cpp:219-232 */
      const REAL inv = c[0];
      const REAL inv_total = acc_inv + acc_s2i * s2;
      const REAL inv_sq = inv * inv;
      grad_a[p] = acc_alpha;
      grad_step[p] = acc_s2i * ((REAL)2 * sigma * inv) + inv_total * (-gamma * inv_sq);
      grad_g[p] = inv_total * (-sigma * inv_sq);
    } else if (variant == 2) { /* dlinoss_im.cpp:236-263 */
      const REAL inv = c[0], si = c[2];
      REAL ga = 0, gg = 0, gs = 0;
      REAL gsi = acc_si, ginv = acc_inv_im;
      gsi += acc_c12 * (-alpha);
      ga += acc_c12 * (-si);
      ginv += acc_c22 * ((REAL)1 + sigma * gamma);
      const REAL gt = acc_c22 * inv;
      gg += gt * sigma;
      gs += gt * gamma;
      gs += gsi * inv;
      ginv += gsi * sigma;
      gs += acc_s2i_im * ((REAL)2 * sigma * inv);
      ginv += acc_s2i_im * s2;
      const REAL gden = ginv * (-(inv * inv));
      ga += gden * s2;
      gg += gden * sigma;
      gs += gden * (gamma + (REAL)2 * sigma * alpha);
      grad_a[p] = ga; grad_g[p] = gg; grad_step[p] = gs;
    } else {
      grad_a[p] = acc_alpha; grad_g[p] = acc_gamma; grad_step[p] = acc_sigma;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* LinOSS generic complex 2x2 scan                                           */
/* ------------------------------------------------------------------------ */

/*
 * s_t = M s_{t-1} + b_t with complex M per oscillator.  Follows
 * linoss_scan.cpp:11-73: time outer, batch rows inner (parallel), state inner.
 * m: four complex [P] arrays; b_seq, out: [L, B, P, 2] complex.
 */
void SFX(oracle_linoss_forward)(const REAL* m11, const REAL* m12, const REAL* m21,
                                const REAL* m22, const REAL* b_seq, REAL* out,
                                int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
  REAL* st = (REAL*)calloc((size_t)(series * 4 > 0 ? series * 4 : 1), sizeof(REAL));
  for (int64_t t = 0; t < length; ++t) {
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
      for (int64_t p = 0; p < ssm; ++p) {
        const int64_t ch = b * ssm + p;
        REAL* s = st + 4 * ch;
        const REAL* bv = b_seq + 4 * (t * series + ch);
        REAL* o = out + 4 * (t * series + ch);
        const REAL a11r = m11[2 * p], a11i = m11[2 * p + 1];
        const REAL a12r = m12[2 * p], a12i = m12[2 * p + 1];
        const REAL a21r = m21[2 * p], a21i = m21[2 * p + 1];
        const REAL a22r = m22[2 * p], a22i = m22[2 * p + 1];
        const REAL n0r = (a11r * s[0] - a11i * s[1]) + (a12r * s[2] - a12i * s[3]) + bv[0];
        const REAL n0i = (a11r * s[1] + a11i * s[0]) + (a12r * s[3] + a12i * s[2]) + bv[1];
        const REAL n1r = (a21r * s[0] - a21i * s[1]) + (a22r * s[2] - a22i * s[3]) + bv[2];
        const REAL n1i = (a21r * s[1] + a21i * s[0]) + (a22r * s[3] + a22i * s[2]) + bv[3];
        o[0] = n0r; o[1] = n0i; o[2] = n1r; o[3] = n1i;
        s[0] = n0r; s[1] = n0i; s[2] = n1r; s[3] = n1i;
      }
    }
  }
  free(st);
}

/*
 * Backward of the LinOSS scan, restating _LinossScanFn.backward
 * (linoss.py:83-151): for t = L-1..0,  g_t = grad_out_t + grad_next,
 * grad_b_t = g_t,  grad_M_ij += sum_b g_i * conj(s_j,t-1),
 * grad_next = M^H g_t.  grad_m: [P, 2, 2] complex (m11, m12, m21, m22).
 * The per-step batch sum is formed first and then added, as in the loop.
 */
void SFX(oracle_linoss_backward)(const REAL* m11, const REAL* m12, const REAL* m21,
                                 const REAL* m22, const REAL* states, const REAL* grad_out,
                                 REAL* grad_m, REAL* grad_b,
                                 int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < ssm; ++p) {
    const REAL a11r = m11[2 * p], a11i = m11[2 * p + 1];
    const REAL a12r = m12[2 * p], a12i = m12[2 * p + 1];
    const REAL a21r = m21[2 * p], a21i = m21[2 * p + 1];
    const REAL a22r = m22[2 * p], a22i = m22[2 * p + 1];
    REAL acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    REAL* nxt = (REAL*)calloc((size_t)(batch > 0 ? batch * 4 : 1), sizeof(REAL));
    for (int64_t t = length - 1; t >= 0; --t) {
      REAL step_sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int64_t b = 0; b < batch; ++b) {
        const int64_t ch = b * ssm + p;
        const REAL* go = grad_out + 4 * (t * series + ch);
        REAL* gn = nxt + 4 * b;
        const REAL g0r = go[0] + gn[0], g0i = go[1] + gn[1];
        const REAL g1r = go[2] + gn[2], g1i = go[3] + gn[3];
        REAL* gb = grad_b + 4 * (t * series + ch);
        gb[0] = g0r; gb[1] = g0i; gb[2] = g1r; gb[3] = g1i;
        REAL p0r = 0, p0i = 0, p1r = 0, p1i = 0;
        if (t > 0) {
          const REAL* pv = states + 4 * ((t - 1) * series + ch);
          p0r = pv[0]; p0i = pv[1]; p1r = pv[2]; p1i = pv[3];
        }
        /* g * conj(prev) */
        step_sum[0] += g0r * p0r + g0i * p0i; step_sum[1] += g0i * p0r - g0r * p0i;
        step_sum[2] += g0r * p1r + g0i * p1i; step_sum[3] += g0i * p1r - g0r * p1i;
        step_sum[4] += g1r * p0r + g1i * p0i; step_sum[5] += g1i * p0r - g1r * p0i;
        step_sum[6] += g1r * p1r + g1i * p1i; step_sum[7] += g1i * p1r - g1r * p1i;
        /* M^H g:  prev0 = g0*conj(m11) + g1*conj(m21); prev1 = g0*conj(m12) + g1*conj(m22) */
        gn[0] = (g0r * a11r + g0i * a11i) + (g1r * a21r + g1i * a21i);
        gn[1] = (g0i * a11r - g0r * a11i) + (g1i * a21r - g1r * a21i);
        gn[2] = (g0r * a12r + g0i * a12i) + (g1r * a22r + g1i * a22i);
        gn[3] = (g0i * a12r - g0r * a12i) + (g1i * a22r - g1r * a22i);
      }
      for (int k = 0; k < 8; ++k) acc[k] += step_sum[k];
    }
    free(nxt);
    for (int k = 0; k < 8; ++k) grad_m[8 * p + k] = acc[k];
  }
}

/* ------------------------------------------------------------------------ */
/* Diagonal complex scans (LRU, S5)                                          */
/* ------------------------------------------------------------------------ */

/*
 * x_t = lambda_p * x_{t-1} + b_t per (b, p), x_{-1} = 0.  Follows
 * lru_scan.cpp:10-58 (s5_scan.cpp:10-66 is the same loop): batch rows in
 * parallel, time outer, state inner; the c10::complex product
 * (re = lr*xr - li*xi, im = lr*xi + li*xr) and then the add.
 * lam_re, lam_im: [P]; b_seq, out: [L, B, P] complex.
 */
void SFX(oracle_diag_forward)(const REAL* lam_re, const REAL* lam_im, const REAL* b_seq,
                              REAL* out, int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < batch; ++b) {
    REAL* st = (REAL*)calloc((size_t)(ssm > 0 ? 2 * ssm : 1), sizeof(REAL));
    for (int64_t t = 0; t < length; ++t) {
      for (int64_t p = 0; p < ssm; ++p) {
        const int64_t off = 2 * (t * series + b * ssm + p);
        const REAL lr = lam_re[p], li = lam_im[p];
        const REAL xr = st[2 * p], xi = st[2 * p + 1];
        const REAL nr = (lr * xr - li * xi) + b_seq[off];
        const REAL ni = (lr * xi + li * xr) + b_seq[off + 1];
        st[2 * p] = nr;
        st[2 * p + 1] = ni;
        out[off] = nr;
        out[off + 1] = ni;
      }
    }
    free(st);
  }
}

/*
 * Backward, restating _LRUScanFn.backward (lru.py:52-80; _S5ScanFn.backward,
 * s5.py:137-165, is the same loop): for t = L-1..0,  g_t = grad_out_t +
 * grad_next,  grad_b_t = g_t,  grad_lambda += sum_b g_t * conj(x_{t-1})
 * (x_{-1} = 0),  grad_next = g_t * conj(lambda).  The per-step batch sum is
 * formed first and then added, as in the loop.  grad_lambda: [P] complex.
 */
void SFX(oracle_diag_backward)(const REAL* lam_re, const REAL* lam_im, const REAL* states,
                               const REAL* grad_out, REAL* grad_lambda, REAL* grad_b,
                               int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < ssm; ++p) {
    const REAL lr = lam_re[p], li = lam_im[p];
    REAL accr = 0, acci = 0;
    REAL* nxt = (REAL*)calloc((size_t)(batch > 0 ? 2 * batch : 1), sizeof(REAL));
    for (int64_t t = length - 1; t >= 0; --t) {
      REAL sr = 0, si = 0;
      for (int64_t b = 0; b < batch; ++b) {
        const int64_t off = 2 * (t * series + b * ssm + p);
        const REAL gr = grad_out[off] + nxt[2 * b], gi = grad_out[off + 1] + nxt[2 * b + 1];
        grad_b[off] = gr;
        grad_b[off + 1] = gi;
        REAL xr = 0, xi = 0;
        if (t > 0) {
          xr = states[off - 2 * series];
          xi = states[off - 2 * series + 1];
        }
        sr += gr * xr + gi * xi;
        si += gi * xr - gr * xi;
        /* g * conj(lambda) */
        nxt[2 * b] = gr * lr + gi * li;
        nxt[2 * b + 1] = gi * lr - gr * li;
      }
      accr += sr;
      acci += si;
    }
    free(nxt);
    grad_lambda[2 * p] = accr;
    grad_lambda[2 * p + 1] = acci;
  }
}

/* ------------------------------------------------------------------------ */
/* Selective scan                                                            */
/* ------------------------------------------------------------------------ */

static REAL SFX(sigm)(REAL x) { return (REAL)1 / ((REAL)1 + EXP(-x)); }

/*
 * Forward, restating selective_scan_cpu.cpp:78-166: per (b, d) lane,
 *   h_n = exp(dt*A_dn) * h_n + dt*B_tn*u_t,   y_t = sum_n C_tn*h_n,
 *   out_t = y_t * silu(z_t) when a gate is given.
 * u, dt, gate, out: [B, D, L];  A: [D, N];  Bm, Cm: [B, L, N].
 */
void SFX(oracle_selective_forward)(const REAL* u, const REAL* dt, const REAL* A,
                                   const REAL* Bm, const REAL* Cm, const REAL* gate,
                                   REAL* out, int64_t batch, int64_t dim, int64_t length,
                                   int64_t nstate) {
#pragma omp parallel
  {
    REAL* h = (REAL*)malloc((size_t)(nstate > 0 ? nstate : 1) * sizeof(REAL));
#pragma omp for schedule(static)
    for (int64_t bd = 0; bd < batch * dim; ++bd) {
      const int64_t b = bd / dim, d = bd % dim;
      const REAL* Arow = A + d * nstate;
      const REAL* ul = u + bd * length;
      const REAL* dl = dt + bd * length;
      const REAL* zl = gate ? gate + bd * length : NULL;
      REAL* ol = out + bd * length;
      for (int64_t n = 0; n < nstate; ++n) h[n] = 0;
      for (int64_t t = 0; t < length; ++t) {
        const REAL dts = dl[t], us = ul[t];
        const REAL* Bt = Bm + (b * length + t) * nstate;
        const REAL* Ct = Cm + (b * length + t) * nstate;
        REAL accv = 0;
        for (int64_t n = 0; n < nstate; ++n) {
          const REAL abar = EXP(dts * Arow[n]);
          const REAL upd = FMA(dts * Bt[n], us, abar * h[n]);
          h[n] = upd;
          accv += upd * Ct[n];
        }
        REAL v = accv;
        if (zl) { const REAL z = zl[t]; v *= z * SFX(sigm)(z); }
        ol[t] = v;
      }
    }
    free(h);
  }
}

/*
 * Backward, restating selective_scan_cpu.cpp:168-360: recompute the lane's
 * L x N state history, then walk time in reverse.  The reference adds the
 * dB / dC / dA contributions with `omp atomic` from all lanes; here lanes of
 * one batch row run in order on one thread (dB, dC rows are per batch) and dA
 * is reduced from per-batch partials in batch order, so results are
 * deterministic.  Without a gate, ggate is zero-filled (:355-357).
 */
void SFX(oracle_selective_backward)(const REAL* gout, const REAL* u, const REAL* dt,
                                    const REAL* A, const REAL* Bm, const REAL* Cm,
                                    const REAL* gate, REAL* gu, REAL* gdt, REAL* gA,
                                    REAL* gB, REAL* gC, REAL* ggate, int64_t batch,
                                    int64_t dim, int64_t length, int64_t nstate) {
  const int64_t an = dim * nstate;
  REAL* gA_part = (REAL*)calloc((size_t)(batch * an > 0 ? batch * an : 1), sizeof(REAL));
  for (int64_t i = 0; i < batch * length * nstate; ++i) { gB[i] = 0; gC[i] = 0; }
#pragma omp parallel
  {
    REAL* hist = (REAL*)malloc((size_t)(length * nstate > 0 ? length * nstate : 1) * sizeof(REAL));
    REAL* gs = (REAL*)malloc((size_t)(nstate > 0 ? nstate : 1) * sizeof(REAL));
#pragma omp for schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
      REAL* gAb = gA_part + b * an;
      for (int64_t d = 0; d < dim; ++d) {
        const int64_t bd = b * dim + d;
        const REAL* Arow = A + d * nstate;
        const REAL* ul = u + bd * length;
        const REAL* dl = dt + bd * length;
        const REAL* zl = gate ? gate + bd * length : NULL;
        const REAL* gol = gout + bd * length;
        for (int64_t t = 0; t < length; ++t) {
          const REAL dts = dl[t], us = ul[t];
          const REAL* Bt = Bm + (b * length + t) * nstate;
          for (int64_t n = 0; n < nstate; ++n) {
            const REAL prev = t == 0 ? (REAL)0 : hist[(t - 1) * nstate + n];
            const REAL abar = EXP(dts * Arow[n]);
            hist[t * nstate + n] = FMA(dts * Bt[n], us, abar * prev);
          }
        }
        for (int64_t n = 0; n < nstate; ++n) gs[n] = 0;
        for (int64_t t = length - 1; t >= 0; --t) {
          const REAL* Ct = Cm + (b * length + t) * nstate;
          const REAL* Bt = Bm + (b * length + t) * nstate;
          REAL y = 0;
          for (int64_t n = 0; n < nstate; ++n) y += hist[t * nstate + n] * Ct[n];
          const REAL go = gol[t];
          REAL gyg = go;
          if (zl) {
            const REAL z = zl[t];
            const REAL sg = SFX(sigm)(z);
            gyg = go * (z * sg);
            ggate[bd * length + t] = go * y * (sg * ((REAL)1 + z * ((REAL)1 - sg)));
          }
          REAL gin = 0, gdts = 0;
          const REAL dts = dl[t], us = ul[t];
          for (int64_t n = 0; n < nstate; ++n) {
            const REAL a = Arow[n];
            const REAL st = hist[t * nstate + n];
            const REAL sp = t == 0 ? (REAL)0 : hist[(t - 1) * nstate + n];
            const REAL abar = EXP(dts * a);
            const REAL gacc = gs[n] + gyg * Ct[n];
            gs[n] = gacc * abar;
            gC[(b * length + t) * nstate + n] += gyg * st;
            gB[(b * length + t) * nstate + n] += gacc * dts * us;
            gin += gacc * dts * Bt[n];
            gAb[d * nstate + n] += gacc * (dts * abar * sp);
            gdts += gacc * (a * abar * sp + Bt[n] * us);
          }
          gu[bd * length + t] = gin;
          gdt[bd * length + t] = gdts;
        }
        if (!zl) for (int64_t t = 0; t < length; ++t) ggate[bd * length + t] = 0;
      }
    }
    free(hist);
    free(gs);
  }
  for (int64_t i = 0; i < an; ++i) {
    REAL s = 0;
    for (int64_t b = 0; b < batch; ++b) s += gA_part[b * an + i];
    gA[i] = s;
  }
  free(gA_part);
}

/* ------------------------------------------------------------------------ */
/* Selective D-LinOSS (time- and batch-varying parameters)                   */
/* ------------------------------------------------------------------------ */

/*
 * Restates the reference's CPU kernels: forward sdlinoss_imex1.cpp:33-97,
 * sdlinoss_imex2.cpp:33-97, sdlinoss_im.cpp:33-97, sdlinoss_ex.cpp:25-84;
 * backward sdlinoss_imex1.cpp:99-231, sdlinoss_imex2.cpp:100-230,
 * sdlinoss_im.cpp:100-230, sdlinoss_ex.cpp:86-200.  Parallel over the
 * B*M series, time inner, as there.  A, G, step are materialised [L,B,M]
 * (materialize_param_cpu, sdlinoss_cpu_utils.h:74-82); the per-element
 * parameter gradients are returned [L,B,M] and summed over broadcast axes
 * by the Python wrapper (reduce_broadcast_grad, sdlinoss_cpu_utils.h:84-97).
 */
static REAL SFX(sdl_clamp_step)(REAL raw) {
  const REAL lo = (REAL)1e-6, hi = (REAL)1.0;
  return raw < lo ? lo : (raw > hi ? hi : raw);
}

static REAL SFX(sdl_s_raw)(int variant, REAL dt, REAL g, REAL a) {
  switch (variant) {
    case 0: return (REAL)1 + dt * g;              /* imex1 */
    case 1: return (REAL)1 + dt * dt * a;         /* imex2 */
    case 2: return (REAL)1 + dt * g + dt * dt * a; /* im */
    default: return (REAL)1;                      /* ex: no implicit part */
  }
}

void SFX(oracle_sdlinoss_forward)(int variant, const REAL* A, const REAL* G, const REAL* step,
                                  const REAL* bu, REAL* out, int64_t length, int64_t batch,
                                  int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < series; ++idx) {
    REAL wr = 0, wi = 0, xr = 0, xi = 0;
    for (int64_t t = 0; t < length; ++t) {
      const int64_t off = t * series + idx;
      const REAL a = A[off], g = G[off];
      const REAL dt = SFX(sdl_clamp_step)(step[off]);
      const REAL dt2 = dt * dt;
      const REAL bur = bu[2 * off], bui = bu[2 * off + 1];
      const REAL combr = -a * xr + bur, combi = -a * xi + bui;
      REAL nwr, nwi;
      if (variant == 3) { /* ex */
        const REAL alpha = (REAL)1 - dt * g;
        nwr = FMA(dt2, combr, alpha * wr);
        nwi = FMA(dt2, combi, alpha * wi);
      } else {
        REAL S = SFX(sdl_s_raw)(variant, dt, g, a);
        if (S < (REAL)1e-6) S = (REAL)1e-6;
        const REAL inv = (REAL)1 / S;
        REAL tr, ti;
        if (variant == 1) { /* imex2 */
          const REAL alpha = (REAL)1 - dt * g;
          tr = alpha * wr + dt2 * combr;
          ti = alpha * wi + dt2 * combi;
        } else {
          tr = FMA(dt2, combr, wr);
          ti = FMA(dt2, combi, wi);
        }
        nwr = tr * inv;
        nwi = ti * inv;
      }
      const REAL nxr = xr + nwr, nxi = xi + nwi;
      REAL* o = out + 4 * off;
      o[0] = nwr; o[1] = nwi; o[2] = nxr; o[3] = nxi;
      wr = nwr; wi = nwi; xr = nxr; xi = nxi;
    }
  }
}

void SFX(oracle_sdlinoss_backward)(int variant, const REAL* A, const REAL* G, const REAL* step,
                                   const REAL* bu, const REAL* states, const REAL* grad_out,
                                   REAL* grad_bu, REAL* grad_A, REAL* grad_G, REAL* grad_step,
                                   int64_t length, int64_t batch, int64_t ssm) {
  const int64_t series = batch * ssm;
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < series; ++idx) {
    REAL gwnr = 0, gwni = 0, gxnr = 0, gxni = 0; /* gradients carried from t + 1 */
    for (int64_t t = length - 1; t >= 0; --t) {
      const int64_t off = t * series + idx;
      REAL wpr = 0, wpi = 0, xpr = 0, xpi = 0;
      if (t > 0) {
        const REAL* p = states + 4 * (off - series);
        wpr = p[0]; wpi = p[1]; xpr = p[2]; xpi = p[3];
      }
      const REAL gor = grad_out[2 * off], goi = grad_out[2 * off + 1];
      const REAL gxr = gor + gxnr, gxi = goi + gxni; /* d/dx_t */
      /* d/dw_t through both outputs (x_t = x_{t-1} + w_t) */
      const REAL gwr = gwnr + gxr, gwi = gwni + gxi;
      const REAL a = A[off], g = G[off], raw = step[off];
      const REAL dt = SFX(sdl_clamp_step)(raw);
      const REAL mask = (raw > (REAL)1e-6 && raw < (REAL)1.0) ? (REAL)1 : (REAL)0;
      const REAL dt2 = dt * dt;
      const REAL bur = bu[2 * off], bui = bu[2 * off + 1];
      const REAL combr = -a * xpr + bur, combi = -a * xpi + bui;
      const REAL alpha = (variant == 1 || variant == 3) ? (REAL)1 - dt * g : (REAL)1;
      REAL gs = 0, ga = 0, gg = 0;
      REAL gtr = gwr, gti = gwi; /* d/dtmpw */
      if (variant != 3) {
        const REAL s_raw = SFX(sdl_s_raw)(variant, dt, g, a);
        const REAL S = s_raw < (REAL)1e-6 ? (REAL)1e-6 : s_raw;
        const REAL cm = s_raw > (REAL)1e-6 ? (REAL)1 : (REAL)0;
        const REAL inv = (REAL)1 / S;
        const REAL tmr = alpha * wpr + dt2 * combr, tmi = alpha * wpi + dt2 * combi;
        gtr = gwr * inv;
        gti = gwi * inv;
        const REAL gS = -(gwr * tmr + gwi * tmi) * (inv * inv) * cm;
        if (variant == 0) { gs += gS * g; gg += gS * dt; }
        else if (variant == 1) { gs += gS * ((REAL)2 * dt * a); ga += gS * dt2; }
        else { gs += gS * (g + (REAL)2 * dt * a); ga += gS * dt2; gg += gS * dt; }
      }
      if (variant == 1 || variant == 3) {
        gs += gtr * (-g * wpr + (REAL)2 * dt * combr) + gti * (-g * wpi + (REAL)2 * dt * combi);
        gg += gtr * (-dt * wpr) + gti * (-dt * wpi);
      } else {
        gs += gtr * ((REAL)2 * dt * combr) + gti * ((REAL)2 * dt * combi);
      }
      ga += gtr * (-dt2 * xpr) + gti * (-dt2 * xpi);
      grad_A[off] = ga;
      grad_G[off] = gg;
      grad_step[off] = gs * mask;
      grad_bu[2 * off] = gtr * dt2;
      grad_bu[2 * off + 1] = gti * dt2;
      /* carry to t - 1 */
      gwnr = gtr * alpha; gwni = gti * alpha;
      gxnr = gxr + gtr * (-dt2 * a); gxni = gxi + gti * (-dt2 * a);
    }
  }
}
