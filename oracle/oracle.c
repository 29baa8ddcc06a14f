/*
 * CPU oracle for the conv / GEMM / AdamW path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's arithmetic (mistrjirka/Pytorch-vulkan)
 * used as the parity checker by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg.  Nothing in the product links or calls it.
 *
 * Reductions accumulate in double so the oracle's own rounding stays far below
 * the FP32 tolerances; AdamW is restated in float with the exact operation order
 * of torch.optim.AdamW's single-tensor update (the CPU implementation the
 * reference tests against), compiled without FP contraction.
 *
 * Pinning (tests/test_oracle_*.py): golden fixtures written by CPU PyTorch
 * (tests/golden/make_golden.py), the reference tests' known answers
 * (tests/test_mm.py:29-35, tests/test_conv_dispatch.py:315-333), closed forms
 * (AdamW first step, 1x1 convolution), invariants (Winograd == direct,
 * dB == sum(dY), per-batch bmm == mm) and planted-mistake checks.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Convolution geometry: convolution_params (csrc/ops/convolution.cpp:101-156) */
/* Returns 0 and fills oh/ow, or a negative code naming the failed check.     */
/* ------------------------------------------------------------------------ */
int oracle_conv2d_shape(int64_t n, int64_t cin, int64_t h, int64_t w, int64_t cout, int64_t wcin, int64_t kh,
                        int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                        int64_t groups, int64_t* oh, int64_t* ow) {
  if (!(n > 0 && cin > 0 && cout > 0 && h > 0 && w > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && dh > 0 &&
        dw > 0 && ph >= 0 && pw >= 0 && groups > 0 && cin % groups == 0 && cout % groups == 0 &&
        wcin == cin / groups))
    return -1; /* invalid shapes or parameters */
  const int64_t lim = 2147483647LL;
  const int64_t vals[] = {h, w, kh, kw, sh, sw, ph, pw, dh, dw};
  for (int i = 0; i < 10; ++i)
    if (vals[i] > lim) return -2; /* spatial parameters exceed int32 */
  if (dh * (kh - 1) > lim || dw * (kw - 1) > lim) return -3;
  if (!(h + 2 * ph >= dh * (kh - 1) + 1 && w + 2 * pw >= dw * (kw - 1) + 1)) return -4; /* kernel > padded input */
  *oh = (h + 2 * ph - dh * (kh - 1) - 1) / sh + 1;
  *ow = (w + 2 * pw - dw * (kw - 1) - 1) / sw + 1;
  if (*oh <= 0 || *ow <= 0) return -5;
  return 0;
}

typedef struct {
  int64_t n, cin, h, w, cout, kh, kw, oh, ow, sh, sw, ph, pw, dh, dw, groups;
} conv_p;

static conv_p mkp(const int64_t* d) {
  conv_p p;
  p.n = d[0]; p.cin = d[1]; p.h = d[2]; p.w = d[3]; p.cout = d[4]; p.kh = d[5]; p.kw = d[6]; p.oh = d[7];
  p.ow = d[8]; p.sh = d[9]; p.sw = d[10]; p.ph = d[11]; p.pw = d[12]; p.dh = d[13]; p.dw = d[14]; p.groups = d[15];
  return p;
}

/* Direct forward: conv2d_forward.comp:11-43 (one output, serial ci/kh/kw loop,
 * bias first).  `d` is the 16-value ConvParams vector
 * {n,cin,h,w,cout,kh,kw,oh,ow,sh,sw,ph,pw,dh,dw,groups} (convolution.cpp:45-52
 * order with h,w before cout).  y and mag (optional) are double. */
void oracle_conv2d_forward(const int64_t* d, const float* x, const float* wt, const float* bias, double* y,
                           double* mag) {
  const conv_p p = mkp(d);
  const int64_t cig = p.cin / p.groups, cog = p.cout / p.groups;
  for (int64_t b = 0; b < p.n; ++b)
    for (int64_t oc = 0; oc < p.cout; ++oc) {
      const int64_t g = oc / cog;
      for (int64_t oy = 0; oy < p.oh; ++oy)
        for (int64_t ox = 0; ox < p.ow; ++ox) {
          double s = bias ? (double)bias[oc] : 0.0, m = bias ? fabs((double)bias[oc]) : 0.0;
          for (int64_t c = 0; c < cig; ++c) {
            const int64_t ic = g * cig + c;
            for (int64_t ky = 0; ky < p.kh; ++ky) {
              const int64_t iy = oy * p.sh - p.ph + ky * p.dh;
              if (iy < 0 || iy >= p.h) continue;
              for (int64_t kx = 0; kx < p.kw; ++kx) {
                const int64_t ix = ox * p.sw - p.pw + kx * p.dw;
                if (ix < 0 || ix >= p.w) continue;
                const double t = (double)x[((b * p.cin + ic) * p.h + iy) * p.w + ix] *
                                 (double)wt[((oc * cig + c) * p.kh + ky) * p.kw + kx];
                s += t;
                m += fabs(t);
              }
            }
          }
          const int64_t o = ((b * p.cout + oc) * p.oh + oy) * p.ow + ox;
          y[o] = s;
          if (mag) mag[o] = m;
        }
    }
}

/* Direct dInput: conv2d_backward_input.comp:10-47 (stride-divisibility test,
 * no zero insertion). */
void oracle_conv2d_backward_input(const int64_t* d, const float* dy, const float* wt, double* dx, double* mag) {
  const conv_p p = mkp(d);
  const int64_t cig = p.cin / p.groups, cog = p.cout / p.groups;
  for (int64_t b = 0; b < p.n; ++b)
    for (int64_t ic = 0; ic < p.cin; ++ic) {
      const int64_t g = ic / cig, c = ic % cig;
      for (int64_t iy = 0; iy < p.h; ++iy)
        for (int64_t ix = 0; ix < p.w; ++ix) {
          double s = 0.0, m = 0.0;
          for (int64_t co = 0; co < cog; ++co) {
            const int64_t oc = g * cog + co;
            for (int64_t ky = 0; ky < p.kh; ++ky) {
              const int64_t ty = iy + p.ph - ky * p.dh;
              if (ty < 0 || ty % p.sh != 0) continue;
              const int64_t oy = ty / p.sh;
              if (oy >= p.oh) continue;
              for (int64_t kx = 0; kx < p.kw; ++kx) {
                const int64_t tx = ix + p.pw - kx * p.dw;
                if (tx < 0 || tx % p.sw != 0) continue;
                const int64_t ox = tx / p.sw;
                if (ox >= p.ow) continue;
                const double t = (double)dy[((b * p.cout + oc) * p.oh + oy) * p.ow + ox] *
                                 (double)wt[((oc * cig + c) * p.kh + ky) * p.kw + kx];
                s += t;
                m += fabs(t);
              }
            }
          }
          const int64_t o = ((b * p.cin + ic) * p.h + iy) * p.w + ix;
          dx[o] = s;
          if (mag) mag[o] = m;
        }
    }
}

/* Direct dWeight: conv2d_backward_weight.comp:10-41 (one weight, serial over
 * batch and output positions). */
void oracle_conv2d_backward_weight(const int64_t* d, const float* x, const float* dy, double* dwt, double* mag) {
  const conv_p p = mkp(d);
  const int64_t cig = p.cin / p.groups, cog = p.cout / p.groups;
  for (int64_t oc = 0; oc < p.cout; ++oc) {
    const int64_t g = oc / cog;
    for (int64_t c = 0; c < cig; ++c) {
      const int64_t ic = g * cig + c;
      for (int64_t ky = 0; ky < p.kh; ++ky)
        for (int64_t kx = 0; kx < p.kw; ++kx) {
          double s = 0.0, m = 0.0;
          for (int64_t b = 0; b < p.n; ++b)
            for (int64_t oy = 0; oy < p.oh; ++oy) {
              const int64_t iy = oy * p.sh - p.ph + ky * p.dh;
              if (iy < 0 || iy >= p.h) continue;
              for (int64_t ox = 0; ox < p.ow; ++ox) {
                const int64_t ix = ox * p.sw - p.pw + kx * p.dw;
                if (ix < 0 || ix >= p.w) continue;
                const double t = (double)x[((b * p.cin + ic) * p.h + iy) * p.w + ix] *
                                 (double)dy[((b * p.cout + oc) * p.oh + oy) * p.ow + ox];
                s += t;
                m += fabs(t);
              }
            }
          const int64_t o = ((oc * cig + c) * p.kh + ky) * p.kw + kx;
          dwt[o] = s;
          if (mag) mag[o] = m;
        }
    }
  }
}

/* dBias: conv2d_backward_bias.comp:9-27 (serial per channel). */
void oracle_conv2d_backward_bias(const int64_t* d, const float* dy, double* db, double* mag) {
  const conv_p p = mkp(d);
  for (int64_t oc = 0; oc < p.cout; ++oc) {
    double s = 0.0, m = 0.0;
    for (int64_t b = 0; b < p.n; ++b)
      for (int64_t q = 0; q < p.oh * p.ow; ++q) {
        const double t = (double)dy[(b * p.cout + oc) * p.oh * p.ow + q];
        s += t;
        m += fabs(t);
      }
    db[oc] = s;
    if (mag) mag[oc] = m;
  }
}

/* Winograd F(2x2,3x3) forward for 3x3 / stride 1 / dilation 1, restating
 * conv2d_winograd_weights.comp:17-28 (U = G g G^T), conv2d_winograd_input.comp:
 * 24-37 (V = B^T d B on 4x4 tiles at stride 2) and
 * conv2d_winograd_gemm_output.comp:46-63 (Y = A^T M A + bias), in double.
 * Returns -1 if the geometry is not Winograd-eligible. */
int oracle_conv2d_winograd_forward(const int64_t* d, const float* x, const float* wt, const float* bias, double* y) {
  const conv_p p = mkp(d);
  if (p.kh != 3 || p.kw != 3 || p.sh != 1 || p.sw != 1 || p.dh != 1 || p.dw != 1) return -1;
  const int64_t cig = p.cin / p.groups, cog = p.cout / p.groups;
  const int64_t th = (p.oh + 1) / 2, tw = (p.ow + 1) / 2;
  for (int64_t b = 0; b < p.n; ++b)
    for (int64_t oc = 0; oc < p.cout; ++oc) {
      const int64_t g = oc / cog;
      for (int64_t ty = 0; ty < th; ++ty)
        for (int64_t tx = 0; tx < tw; ++tx) {
          double M[16];
          memset(M, 0, sizeof(M));
          for (int64_t c = 0; c < cig; ++c) {
            const int64_t ic = g * cig + c;
            const float* k = wt + (oc * cig + c) * 9;
            double z[4][3], U[4][4], dd[4][4], v[4][4], zz[4][4];
            for (int cc = 0; cc < 3; ++cc) {
              z[0][cc] = k[cc];
              z[1][cc] = 0.5 * ((double)k[cc] + k[3 + cc] + k[6 + cc]);
              z[2][cc] = 0.5 * ((double)k[cc] - k[3 + cc] + k[6 + cc]);
              z[3][cc] = k[6 + cc];
            }
            for (int r = 0; r < 4; ++r) {
              U[r][0] = z[r][0];
              U[r][1] = 0.5 * (z[r][0] + z[r][1] + z[r][2]);
              U[r][2] = 0.5 * (z[r][0] - z[r][1] + z[r][2]);
              U[r][3] = z[r][2];
            }
            const int64_t y0 = ty * 2 - p.ph, x0 = tx * 2 - p.pw;
            for (int r = 0; r < 4; ++r)
              for (int cc = 0; cc < 4; ++cc) {
                const int64_t iy = y0 + r, ix = x0 + cc;
                dd[r][cc] = (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w)
                                ? (double)x[((b * p.cin + ic) * p.h + iy) * p.w + ix]
                                : 0.0;
              }
            for (int cc = 0; cc < 4; ++cc) {
              zz[0][cc] = dd[0][cc] - dd[2][cc];
              zz[1][cc] = dd[1][cc] + dd[2][cc];
              zz[2][cc] = dd[2][cc] - dd[1][cc];
              zz[3][cc] = dd[1][cc] - dd[3][cc];
            }
            for (int r = 0; r < 4; ++r) {
              v[r][0] = zz[r][0] - zz[r][2];
              v[r][1] = zz[r][1] + zz[r][2];
              v[r][2] = zz[r][2] - zz[r][1];
              v[r][3] = zz[r][1] - zz[r][3];
            }
            for (int r = 0; r < 4; ++r)
              for (int cc = 0; cc < 4; ++cc) M[r * 4 + cc] += U[r][cc] * v[r][cc];
          }
          double r0[4], r1[4];
          for (int cc = 0; cc < 4; ++cc) {
            r0[cc] = M[cc] + M[4 + cc] + M[8 + cc];
            r1[cc] = M[4 + cc] - M[8 + cc] - M[12 + cc];
          }
          const double bv = bias ? (double)bias[oc] : 0.0;
          const double out[2][2] = {{r0[0] + r0[1] + r0[2] + bv, r0[1] - r0[2] - r0[3] + bv},
                                    {r1[0] + r1[1] + r1[2] + bv, r1[1] - r1[2] - r1[3] + bv}};
          for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 2; ++j) {
              const int64_t oy = ty * 2 + i, ox = tx * 2 + j;
              if (oy < p.oh && ox < p.ow) y[((b * p.cout + oc) * p.oh + oy) * p.ow + ox] = out[i][j];
            }
        }
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMM: matmul_strided_bias.comp:27-68 / bmm_strided.comp:13-31 semantics.   */
/* c[b][m][n] = alpha * sum_k a[...]*b[...] + (beta != 0 ? beta*bias : 0)     */
/* with element strides/offsets; bias_kind 0 none, 1 bias[n], 2 bias[m][n].   */
/* ------------------------------------------------------------------------ */
void oracle_gemm(int64_t batch, int64_t M, int64_t N, int64_t K, const float* a, int64_t a_off, int64_t a_sb,
                 int64_t a_sm, int64_t a_sk, const float* bm, int64_t b_off, int64_t b_sb, int64_t b_sk,
                 int64_t b_sn, const float* bias, int bias_kind, int64_t bias_off, int64_t bias_sm, int64_t bias_sn,
                 double alpha, double beta, double* c, double* mag) {
  for (int64_t z = 0; z < batch; ++z)
    for (int64_t i = 0; i < M; ++i)
      for (int64_t j = 0; j < N; ++j) {
        double s = 0.0, m = 0.0;
        for (int64_t k = 0; k < K; ++k) {
          const double t = (double)a[a_off + z * a_sb + i * a_sm + k * a_sk] *
                           (double)bm[b_off + z * b_sb + k * b_sk + j * b_sn];
          s += t;
          m += fabs(t);
        }
        s *= alpha;
        m *= fabs(alpha);
        if (bias_kind != 0 && beta != 0.0) {
          /* beta == 0 ignores the bias entirely (NaN/Inf included). */
          const double bv = bias_kind == 1 ? (double)bias[bias_off + j * bias_sn]
                                           : (double)bias[bias_off + i * bias_sm + j * bias_sn];
          s += beta * bv;
          m += fabs(beta * bv);
        }
        const int64_t o = (z * M + i) * N + j;
        c[o] = s;
        if (mag) mag[o] = m;
      }
}

/* ------------------------------------------------------------------------ */
/* AdamW                                                                      */
/* ------------------------------------------------------------------------ */
static float nan_max(float a, float b) { return (a != a || b != b) ? NAN : (a > b ? a : b); }

/* One AdamW step on one tensor, in place, torch.optim.AdamW single-tensor
 * order (torch/optim/adam.py _single_tensor_adam with decoupled weight decay):
 *   p *= 1 - lr*wd;  m.lerp_(g, 1-b1) (fused multiply-add, as torch's
 *   vectorised lerp);  v = v*b2; v += ((1-b2)*g)*g;
 *   [amsgrad: vmax = max(vmax, v)]
 *   p += (-lr/bc1 * m) / (sqrt(v_or_vmax) / sqrt(bc2) + eps)
 * with bc1 = 1 - b1^step, bc2 = 1 - b2^step in double and every tensor
 * operation in float.  The reference's shader forms the same update with a
 * different association (adamw_fused.comp:24-31); both agree within a few
 * FP32 ulps.  maximize negates g first. */
void oracle_adamw_step(float* p, const float* g, float* m, float* v, float* vmax, int64_t n, double lr, double beta1,
                       double beta2, double eps, double wd, double step, int maximize) {
  const float wdf = (float)(1.0 - lr * wd);
  const float w1 = (float)(1.0 - beta1);
  const float b2 = (float)beta2, w2 = (float)(1.0 - beta2);
  const double bc1 = 1.0 - pow(beta1, step), bc2 = 1.0 - pow(beta2, step);
  const float nss = (float)(-(lr / bc1));
  const float bc2s = (float)sqrt(bc2);
  const float epsf = (float)eps;
  for (int64_t i = 0; i < n; ++i) {
    float gi = maximize ? -g[i] : g[i];
    float pi = p[i] * wdf;
    float mi = m[i];
    /* torch's vectorised lerp (ATen cpu LerpKernel lerp_vec): one fused
     * multiply-add, fma(w, end-self, self) for |w| < 0.5, else
     * fma(w-1, end-self, end). */
    mi = (w1 < 0.5f) ? fmaf(w1, gi - mi, mi) : fmaf(w1 - 1.0f, gi - mi, gi);
    float vi = v[i] * b2;
    vi = vi + (w2 * gi) * gi;
    float vd = vi;
    if (vmax) {
      vd = nan_max(vmax[i], vi);
      vmax[i] = vd;
    }
    const float denom = sqrtf(vd) / bc2s + epsf;
    pi = pi + (nss * mi) / denom;
    p[i] = pi;
    m[i] = mi;
    v[i] = vi;
  }
}

/* Launch grouping of a tensor list (multitensor::partition,
 * csrc/ops/multitensor_plan.h:22-48, with the alias predicate of
 * csrc/ops/adamw.cpp:207-215): consecutive entries share a launch until one
 * conflicts with an entry already in it.  conflict(i, j) is given as a dense
 * row-major count x count 0/1 matrix.  `slots` caps the entries per launch
 * (the reference's 4/8-wide shaders; 0 = unlimited, this build's design).
 * Writes the first index of each group to `starts`, returns the group count. */
int64_t oracle_partition(const uint8_t* conflict, int64_t count, int64_t slots, int64_t* starts) {
  int64_t groups = 0;
  for (int64_t first = 0; first < count;) {
    int64_t last = first + 1;
    while (last < count && (slots == 0 || last - first < slots)) {
      int independent = 1;
      for (int64_t prev = first; prev < last; ++prev)
        if (conflict[prev * count + last] || conflict[last * count + prev]) {
          independent = 0;
          break;
        }
      if (!independent) break;
      ++last;
    }
    starts[groups++] = first;
    first = last;
  }
  return groups;
}
