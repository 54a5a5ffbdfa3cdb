// Uses the library through its C ABI only (include/osm.h and the HIP runtime
// API; no Python, no torch): the fused forward on a small problem in device
// memory, checked against a double-precision restatement in plain loops of
// the reference's fixed-coefficient path (sdpc_kernel.py:1722-1739: softsign,
// Chebyshev series, damping, tanh; the per-head EMA of chimera_v2_ssm.py:
// 86-101, clamped as the reference's scan does), the workspace's fault word
// and launch counter, then one argument error.
// Built by orthossm_amd/build.py; run by tests/test_gpu_c_abi.py.  Prints
// "ok ..." and exits 0 on success.
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "osm.h"

#define HIP_OK(call)                                                       \
  do {                                                                     \
    if ((call) != hipSuccess) {                                            \
      fprintf(stderr, "HIP call failed at line %d: %s\n", __LINE__, #call); \
      return 2;                                                            \
    }                                                                      \
  } while (0)

static unsigned g_seed = 12345u;
static float uniform(float lo, float hi) {  // deterministic LCG
  g_seed = g_seed * 1664525u + 1013904223u;
  return lo + (hi - lo) * (float)(g_seed >> 8) / (float)(1u << 24);
}

// sum_{k<K} c_k T_k(u) by the three-term recurrence, in double.
static double series(double u, const float* c, int K, int stride) {
  double t0 = 1.0, t1 = u, s = c[0];
  if (K > 1) s += c[stride] * u;
  for (int k = 2; k < K; ++k) {
    const double t2 = 2.0 * u * t1 - t0;
    s += c[k * stride] * t2;
    t0 = t1;
    t1 = t2;
  }
  return s;
}

int main(void) {
  const int B = 2, S = 777, H = 4, hd = 16, K = 8, D = H * hd;
  const size_t nx = (size_t)B * S * D, nc = (size_t)B * H * K * hd;
  float* x = (float*)malloc(nx * sizeof(float));
  float* out = (float*)malloc(nx * sizeof(float));
  float* c = (float*)malloc(nc * sizeof(float));
  float damping[H], lam[H] = {0.9995f, 0.997f, 0.95f, 0.99f};
  for (size_t i = 0; i < nx; ++i) x[i] = uniform(-3.0f, 3.0f);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int k = 0; k < K; ++k)
        for (int j = 0; j < hd; ++j) c[(((size_t)b * H + h) * K + k) * hd + j] = uniform(-1.0f, 1.0f) / (k + 1);
  for (int h = 0; h < H; ++h) damping[h] = powf(0.9f, (float)h);

  // Reference, double precision.
  double max_ref = 0.0, max_err = 0.0;
  double* ref = (double*)malloc(nx * sizeof(double));
  for (int b = 0; b < B; ++b)
    for (int d = 0; d < D; ++d) {
      const int h = d / hd, j = d % hd;
      const float* cl = c + ((size_t)b * H + h) * K * hd + j;
      double s = 0.0;
      for (int t = 0; t < S; ++t) {
        const double xv = x[((size_t)b * S + t) * D + d];
        const double u = xv / (1.0 + fabs(xv));
        const double z = tanh(damping[h] * series(u, cl, K, hd));
        s = lam[h] * s + (1.0 - lam[h]) * z;
        const double o = s > 1.0 ? 1.0 : (s < -1.0 ? -1.0 : s);
        ref[((size_t)b * S + t) * D + d] = o;
        if (fabs(o) > max_ref) max_ref = fabs(o);
      }
    }

  // The library, through the C ABI.
  float *dx, *dout, *dc, *ddamp, *dlam;
  HIP_OK(hipMalloc((void**)&dx, nx * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dout, nx * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dc, nc * sizeof(float)));
  HIP_OK(hipMalloc((void**)&ddamp, H * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dlam, H * sizeof(float)));
  HIP_OK(hipMemcpy(dx, x, nx * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dc, c, nc * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ddamp, damping, sizeof(damping), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dlam, lam, sizeof(lam), hipMemcpyHostToDevice));

  osm_cheby_args a;
  memset(&a, 0, sizeof(a));
  a.abi_version = OSM_ABI_VERSION;
  a.flags = 0;
  a.B = B; a.S = S; a.H = H; a.hd = hd; a.K = K;
  a.x = dx; a.x_dtype = OSM_F32; a.x_stride_b = (int64_t)S * D; a.x_stride_s = D;
  a.out = dout; a.out_dtype = OSM_F32; a.out_stride_b = (int64_t)S * D; a.out_stride_s = D;
  a.coeffs = dc; a.c_stride_b = (int64_t)H * K * hd; a.c_stride_h = (int64_t)K * hd; a.c_stride_k = hd;
  a.damping = ddamp; a.lam = dlam;

  const size_t ws_bytes = osm_workspace_bytes(&a, OSM_OP_FWD);
  if (ws_bytes == 0) {
    fprintf(stderr, "osm_workspace_bytes: %s\n", osm_last_error());
    return 1;
  }
  void* ws;
  HIP_OK(hipMalloc(&ws, ws_bytes));
  if (osm_workspace_init(ws, ws_bytes, NULL) != OSM_OK) {
    fprintf(stderr, "osm_workspace_init: %s\n", osm_last_error());
    return 1;
  }
  for (int rep = 0; rep < 2; ++rep) {  // the second call reuses the workspace
    const int rc = osm_cheby_ema_fwd(&a, ws, ws_bytes, NULL);
    if (rc != OSM_OK) {
      fprintf(stderr, "osm_cheby_ema_fwd: %d %s\n", rc, osm_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(out, dout, nx * sizeof(float), hipMemcpyDeviceToHost));
    for (size_t i = 0; i < nx; ++i) {
      const double e = fabs((double)out[i] - ref[i]);
      if (!(e <= max_err)) max_err = e;  // also catches NaN
    }
  }
  const double rel = max_err / max_ref;

  // The workspace header after the two launches: no look-back wait gave up
  // (fault word 0) and the launch counter went 0 -> 2.
  uint32_t* dstatus;
  uint32_t status[2] = {0xffffffffu, 0u};
  HIP_OK(hipMalloc((void**)&dstatus, sizeof(status)));
  if (osm_workspace_status(ws, dstatus, 1, NULL) != OSM_OK) {
    fprintf(stderr, "osm_workspace_status: %s\n", osm_last_error());
    return 1;
  }
  HIP_OK(hipMemcpy(status, dstatus, sizeof(status), hipMemcpyDeviceToHost));
  hipFree(dstatus);
  const int status_ok = status[0] == 0u && status[1] == 2u;

  // Argument errors come back as status codes, before any HIP call.
  osm_cheby_args bad = a;
  bad.K = OSM_MAX_K + 1;
  const int rc_bad = osm_cheby_ema_fwd(&bad, ws, ws_bytes, NULL);
  const int err_ok = rc_bad == OSM_E_SHAPE && strlen(osm_last_error()) > 0;

  hipFree(ws); hipFree(dx); hipFree(dout); hipFree(dc); hipFree(ddamp); hipFree(dlam);
  free(x); free(out); free(c); free(ref);
  if (!(rel <= 1e-5) || !err_ok || !status_ok) {
    fprintf(stderr, "FAILED: max rel err %.3e (limit 1e-5), bad-K status %d, fault word 0x%08x, launches %u\n",
            rel, rc_bad, status[0], status[1]);
    return 1;
  }
  printf("ok: C ABI forward max rel err %.3e over %zu elements; bad K -> status %d; fault word 0, %u launches\n",
         rel, nx, rc_bad, status[1]);
  return 0;
}
