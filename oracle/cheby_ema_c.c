/*
 * Float64 C restatement of oracle/cheby_ema.py's forward() and ttt_grad()
 * for one batch row, parallel over lanes (OpenMP).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through tests/helpers.py) to
 * check full-size batch rows, where the numpy oracle takes 18-36 s per row.
 * It restates the same float64 steps as the numpy oracle, which cites the
 * reference lines they follow:
 *   softsign       sdpc_kernel.py:1722-1725  (u = x/(1+|x|), +-Inf -> +-1)
 *   Clenshaw       sdpc_kernel.py:1139-1156  (b_k = c_k + 2u b_{k+1} - b_{k+2})
 *   damping, tanh  sdpc_kernel.py:1734-1739  (z = tanh(delta_h p))
 *   NaN policy     sdpc_kernel.py:2086 (z = 0) or 1725 (u = 0)
 *   dynamic lambda sdpc_kernel.py:2188-2194  (clamp(lam_h + shift g, lo, hi))
 *   EMA            chimera_v2_ssm.py:86-101  (s = lam s + (1 - lam) z)
 *   TTT adjoint    sdpc_kernel.py:681-777, 784-915 (a = gL + lam' a')
 * and is pinned against it on the CPU (tests/test_oracle_c.py).
 *
 * Layouts (elements): x row [S][x_ss] (lane stride 1), coeffs of the row
 * [H][c_sh] with c_k of head h, lane j at h*c_sh + k*c_sk + j, g row
 * [S][g_ss] with head stride g_sh (NULL: static lambda), init/fin [D],
 * out [S][D] (float64), grad [H][K][hd] (float64).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define LANE_BLOCK 16

static double softsign64(double x) {
  if (isinf(x)) return x > 0 ? 1.0 : -1.0;
  return x / (1.0 + fabs(x));
}

static double clenshaw64(const double* c, int K, double u) {
  double b1 = 0.0, b2 = 0.0;
  for (int k = K - 1; k >= 1; --k) {
    const double b0 = c[k] + 2.0 * u * b1 - b2;
    b2 = b1;
    b1 = b0;
  }
  return c[0] + u * b1 - b2;
}

typedef struct {
  const float* x;
  long S, D, H, hd, K, x_ss;
  const float* coeffs;
  long c_sh, c_sk;
  const float* damping;
  const float* lam;
  const float* g;
  long g_ss, g_sh;
  double lam_shift, lam_min, lam_max;
  const double* init;
  int clamp_out, nan_zero_u;
} Row;

static double lam_at(const Row* r, long t, long h) {
  const double l = (double)r->lam[h];
  if (!r->g) return l;
  double v = l + r->lam_shift * (double)r->g[t * r->g_ss + h * r->g_sh];
  if (v < r->lam_min) v = r->lam_min;
  if (v > r->lam_max) v = r->lam_max;
  return v;
}

static void lane_coeffs(const Row* r, long d, double* c) {
  const long h = d / r->hd, j = d - h * r->hd;
  for (long k = 0; k < r->K; ++k) c[k] = (double)r->coeffs[h * r->c_sh + k * r->c_sk + j];
}

/* z[t][i] (and u, lambda when asked) for lanes d0 .. d0+n-1. */
static void forward_block(const Row* r, long d0, int n, double* z, double* uc, double* lt, double* s, double* out,
                          double* fin) {
  double c[LANE_BLOCK][16], state[LANE_BLOCK], delta[LANE_BLOCK];
  for (int i = 0; i < n; ++i) {
    lane_coeffs(r, d0 + i, c[i]);
    delta[i] = (double)r->damping[(d0 + i) / r->hd];
    state[i] = r->init ? r->init[d0 + i] : 0.0;
  }
  for (long t = 0; t < r->S; ++t) {
    for (int i = 0; i < n; ++i) {
      const long d = d0 + i, h = d / r->hd;
      const double xv = (double)r->x[t * r->x_ss + d];
      const int nan = isnan(xv);
      const double u = nan ? 0.0 : softsign64(xv);
      double zz = tanh(delta[i] * clenshaw64(c[i], (int)r->K, u));
      if (nan && !r->nan_zero_u) zz = 0.0;
      const double l = lam_at(r, t, h);
      state[i] = l * state[i] + (1.0 - l) * zz;
      double o = state[i];
      if (r->clamp_out) o = o < -1.0 ? -1.0 : (o > 1.0 ? 1.0 : o);
      if (isnan(state[i])) o = state[i];
      out[t * r->D + d] = o;
      const long q = t * LANE_BLOCK + i;
      if (z) z[q] = zz;
      if (uc) uc[q] = u;
      if (lt) lt[q] = l;
      if (s) s[q] = state[i];
    }
  }
  if (fin)
    for (int i = 0; i < n; ++i) fin[d0 + i] = state[i];
}

int osm_oracle_forward_row(const float* x, long S, long D, long H, long K, long x_ss, const float* coeffs, long c_sh,
                           long c_sk, const float* damping, const float* lam, const float* g, long g_ss, long g_sh,
                           double lam_shift, double lam_min, double lam_max, const double* init, int clamp_out,
                           int nan_zero_u, double* out, double* fin) {
  if (K < 1 || K > 16 || H < 1 || D % H) return -1;
  const Row r = {x, S, D, H, D / H, K, x_ss, coeffs, c_sh, c_sk, damping, lam, g, g_ss, g_sh,
                 lam_shift, lam_min, lam_max, init, clamp_out, nan_zero_u};
  const long nb = (D + LANE_BLOCK - 1) / LANE_BLOCK;
#pragma omp parallel for schedule(dynamic)
  for (long b = 0; b < nb; ++b) {
    const long d0 = b * LANE_BLOCK;
    const int n = (int)(D - d0 < LANE_BLOCK ? D - d0 : LANE_BLOCK);
    forward_block(&r, d0, n, NULL, NULL, NULL, NULL, out, fin);
  }
  return 0;
}

/* TTT gradient of one row: grad[h][k][j] = dL/dc_k / (k+1)^2 with
 * L = scale/2 * sum_{t<S-1, d} (out[t] - y[t+1])^2, i.e. gL = scale (out - y)
 * [|s| <= 1]; scale = 2/N for the mean over N = B (S-1) D elements of the
 * whole batch.  target_softsign: y = softsign(x) (NaN where x is NaN), else
 * y = x.  Also writes out and fin like the forward. */
int osm_oracle_ttt_row(const float* x, long S, long D, long H, long K, long x_ss, const float* coeffs, long c_sh,
                       long c_sk, const float* damping, const float* lam, const float* g, long g_ss, long g_sh,
                       double lam_shift, double lam_min, double lam_max, const double* init, int clamp_out,
                       int nan_zero_u, int target_softsign, double scale, double* grad, double* out, double* fin) {
  if (K < 1 || K > 16 || H < 1 || D % H) return -1;
  const Row r = {x, S, D, H, D / H, K, x_ss, coeffs, c_sh, c_sk, damping, lam, g, g_ss, g_sh,
                 lam_shift, lam_min, lam_max, init, clamp_out, nan_zero_u};
  const long hd = D / H, nb = (D + LANE_BLOCK - 1) / LANE_BLOCK;
  int failed = 0;
#pragma omp parallel for schedule(dynamic)
  for (long b = 0; b < nb; ++b) {
    const long d0 = b * LANE_BLOCK;
    const int n = (int)(D - d0 < LANE_BLOCK ? D - d0 : LANE_BLOCK);
    const size_t cells = (size_t)S * LANE_BLOCK;
    double* z = malloc(cells * sizeof(double));
    double* uc = malloc(cells * sizeof(double));
    double* lt = malloc(cells * sizeof(double));
    double* s = malloc(cells * sizeof(double));
    if (!z || !uc || !lt || !s) {
#pragma omp atomic write
      failed = 1;
      free(z), free(uc), free(lt), free(s);
      continue;
    }
    forward_block(&r, d0, n, z, uc, lt, s, out, fin);
    for (int i = 0; i < n; ++i) {
      const long d = d0 + i, h = d / hd, j = d - h * hd;
      const double delta = (double)damping[h];
      double dc[16] = {0};
      double a = 0.0;
      for (long t = S - 1; t >= 0; --t) {
        const long q = t * LANE_BLOCK + i;
        double gl = 0.0;
        if (t < S - 1) {
          const double xn = (double)x[(t + 1) * x_ss + d];
          const double y = target_softsign ? (isnan(xn) ? xn : softsign64(xn)) : xn;
          gl = scale * (out[t * D + d] - y) * (fabs(s[q]) <= 1.0 ? 1.0 : 0.0);
        }
        const double nxt = t + 1 < S ? lt[(t + 1) * LANE_BLOCK + i] : 0.0;
        a = gl + nxt * a;
        double dp = (1.0 - lt[q]) * a * (1.0 - z[q] * z[q]) * delta;
        if (!nan_zero_u && isnan((double)x[t * x_ss + d])) dp = 0.0;
        double tm2 = 1.0, tm1 = uc[q];
        dc[0] += dp;
        if (K > 1) dc[1] += dp * tm1;
        for (long k = 2; k < K; ++k) {
          const double tk = 2.0 * uc[q] * tm1 - tm2;
          dc[k] += dp * tk;
          tm2 = tm1;
          tm1 = tk;
        }
      }
      for (long k = 0; k < K; ++k) grad[(h * K + k) * hd + j] = dc[k] / (double)((k + 1) * (k + 1));
    }
    free(z), free(uc), free(lt), free(s);
  }
  return failed ? -2 : 0;
}
