/*
 * osm.h — C ABI of the MI355X (gfx950) Cheby-RKV hot path.
 *
 * One fused operator, per batch b, token t, head h, lane j (d = h*hd + j):
 *
 *   u = x / (1 + |x|)                               softsign
 *   p = sum_{k<K} c[b,h,k,j] T_k(u)                 Clenshaw, K <= 32 (<= 8 for the TTT)
 *   z = tanh(damping[h] * p)                        (z = 0 where x is NaN, or u = 0
 *                                                    with OSM_FLAG_NAN_ZERO_U)
 *   s[t] = lam[b,t,h] s[t-1] + (1 - lam[b,t,h]) z   s[-1] = ema_init (0 if NULL)
 *   out  = clamp(s, -1, 1)                          (OSM_FLAG_NO_CLAMP disables)
 *   lam[b,t,h] = lam_h, or clamp(lam_h + lam_shift * g[b,t,h], lam_min, lam_max)
 *
 * plus the test-time-training (TTT) coefficient gradient
 *
 *   L = mean_{b, t<S-1, d} (out[b,t,d] - y[b,t+1,d])^2,  y = x or softsign(x)
 *   grad[b,h,k,j] = dL/dc[b,h,k,j] / (k+1)^2
 *
 * Reference interfaces replaced (paths relative to the OrthoSSM root):
 *   osm_cheby_ema_fwd  the forward kernel launches
 *                      _launch_ortho_megakernel (sdpc_kernel.py:2290-2344) and
 *                      the _EMAFastPathFn launch (sdpc_kernel.py:1661-1670),
 *                      with the EMA carry InitState/FinalState [B,D]
 *                      (sdpc_kernel.py:1999-2003, 2172-2177) exposed as
 *                      ema_init / ema_final.
 *   osm_cheby_ema_lut_fwd  the direct _fused_clenshaw_ema_kernel launch
 *                      (sdpc_kernel.py:988-1209; precision_tests.py:47-73):
 *                      LUT or Clenshaw series, x_norm, tanh_y, clamped EMA
 *                      from InitState, FinalState.
 *   osm_cheby_ema_ttt  the coefficient-gradient chain of FusedChebyRKVv10.backward:
 *                      _parallel_reverse_ema_kernel (sdpc_kernel.py:2463-2471),
 *                      _parallel_backward_clenshaw_kernel_v10 (2487-2500) and
 *                      grad_c_part.sum (2502), fused with the forward.
 *   osm_cheby_ema_bwd  the backward of the forward: _EMAFastPathFn.backward
 *                      (sdpc_kernel.py:1677-1701, its masked reverse scan
 *                      682-777) and autograd through the fast path's softsign,
 *                      Chebyshev basis, damping and tanh (1722-1739), giving
 *                      dL/dx, dL/dc and dL/d ema_init from dL/dout and
 *                      dL/d ema_final.  With OSM_FLAG_FULL_JACOBIAN and
 *                      z_saved it is the per-chunk FusedChebyRKVv10.backward
 *                      (sdpc_kernel.py:2436-2515) of the full path.
 *   osm_v10_chunked_ttt  the full path of apply_cheby_rkv_v10: its chunk loop
 *                      (sdpc_kernel.py:2574-2606) of FusedChebyRKVv10.forward
 *                      launches (2353-2433) running _ortho_megakernel
 *                      (1890-2287) with the inline Lion update, all chunks in
 *                      one launch.
 *
 * Conventions
 *   - All device pointers are caller-owned; the library allocates nothing.
 *   - Launches are stream-ordered on `stream` (a hipStream_t passed as void*,
 *     NULL = the null stream) and never synchronise the host.
 *   - Returns OSM_OK (0) or a negative osm_status; osm_last_error() gives a
 *     thread-local message.  Argument errors are detected before any HIP call.
 *   - The workspace (osm_workspace_bytes, 256-byte aligned) keeps state between
 *     calls: a launch counter and tagged look-back words.  The library clears
 *     it on the stream the first time it sees a workspace pointer (unless
 *     osm_workspace_init zeroed it) and whenever the layout changes (shape,
 *     K class, static/dynamic lambda, entry point); such a clear keeps the
 *     header's first 64 bytes (launch counter, fault word) and zeroes its
 *     completion counters and the look-back words.  A workspace freed and a new
 *     one allocated at the same address must be passed through
 *     osm_workspace_init.  Two calls that overlap in time must not share one
 *     workspace; if they do, every wave still exits (bounded waits) and the
 *     header's fault word (offset 12) is set to the fault tag of the launch
 *     whose wait gave up; osm_workspace_status reads (and resets) it.  The
 *     launch counter in the header only grows (clears on a layout change
 *     leave it alone); one workspace serves 2^30 launches, after which it
 *     must be passed through osm_workspace_init.
 */
#ifndef ORTHOSSM_AMD_OSM_H
#define ORTHOSSM_AMD_OSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OSM_ABI_VERSION 2
#define OSM_MAX_K 32      /* coefficients per lane: forward and backward */
#define OSM_MAX_K_TTT 8   /* coefficients per lane: the TTT gradient */

typedef enum osm_dtype { OSM_F32 = 0, OSM_BF16 = 1 } osm_dtype;

typedef enum osm_status {
  OSM_OK = 0,
  OSM_E_ARG = -1,         /* NULL pointer, bad ABI version, bad flag */
  OSM_E_SHAPE = -2,       /* dimension out of range or inconsistent */
  OSM_E_DTYPE = -3,       /* unsupported dtype or dtype combination */
  OSM_E_LAYOUT = -4,      /* misaligned pointer or stride */
  OSM_E_WORKSPACE = -5,   /* workspace NULL, too small or misaligned */
  OSM_E_HIP = -6          /* a HIP runtime call or kernel launch failed */
} osm_status;

/* flags */
#define OSM_FLAG_NO_CLAMP 0x1   /* out = s instead of clamp(s, -1, 1) */
#define OSM_FLAG_NAN_ZERO_U 0x2 /* a NaN x counts as u = 0 (the reference's PyTorch
                                   fast path, sdpc_kernel.py:1725) instead of
                                   giving z = 0 (its Triton kernels, 2086) */
#define OSM_FLAG_FULL_JACOBIAN 0x4 /* osm_cheby_ema_bwd only: dL/dx uses 1/(1+|x|)^2
                                      everywhere (NaN where x is NaN), as the
                                      full path's backward (sdpc_kernel.py:2505),
                                      instead of 0 where |x| < 1e-7 or NaN */
#define OSM_FLAG_TIMING_JITTER 0x8 /* test aid, no counterpart in the reference:
                                      every workgroup sleeps a pseudo-random
                                      0-13 us (hash of its index and the launch)
                                      before it publishes to the look-back and
                                      before it combines the words it read, to
                                      perturb the order in which tiles finish;
                                      results are unchanged, bit for bit */
#define OSM_FLAG_POLL_LIMIT_ZERO 0x10 /* test aid, no counterpart in the reference:
                                      a look-back wait whose word is not yet
                                      published when first read gives up at
                                      once instead of polling, as a wait that
                                      passes its poll limit does: the fault
                                      word is set and the outputs that depend
                                      on the missing value are NaN (out,
                                      ema_final, the TTT gradient, the
                                      backward's gradients); every kernel
                                      still exits normally */

/* TTT target y */
typedef enum osm_ttt_target { OSM_TARGET_X = 0, OSM_TARGET_SOFTSIGN = 1 } osm_ttt_target;

/*
 * Operator arguments.  Strides are in elements.  The lane (last) dimension of
 * x, out and coeffs is contiguous; pointers are aligned to their element
 * size and strides are non-negative.  The forward is fastest when hd % 4 == 0,
 * K <= 8 and the x and out rows start on 4-element boundaries (pointers
 * aligned to 4 elements, x_stride_b/x_stride_s and the out strides multiples
 * of 4); other layouts take a one-lane-per-thread geometry, and K > 8 the
 * Clenshaw form of the series.
 */
typedef struct osm_cheby_args {
  int32_t abi_version;      /* = OSM_ABI_VERSION */
  int32_t flags;            /* OSM_FLAG_* */
  int64_t B, S, H, hd, K;   /* hd >= 1, 1 <= K <= OSM_MAX_K (OSM_MAX_K_TTT for the TTT) */

  const void* x;            /* [B,S,H*hd] of x_dtype */
  int32_t x_dtype;
  int64_t x_stride_b, x_stride_s;

  void* out;                /* [B,S,H*hd] of out_dtype */
  int32_t out_dtype;
  int64_t out_stride_b, out_stride_s;

  const float* coeffs;      /* [B,H,K,hd] fp32 */
  int64_t c_stride_b, c_stride_h, c_stride_k;

  const float* damping;     /* [H] fp32 */
  const float* lam;         /* [H] fp32, the static per-head EMA decay */

  const float* g;           /* optional [B,S,H] fp32; stride 0 broadcasts */
  int64_t g_stride_b, g_stride_s, g_stride_h;
  float lam_shift, lam_min, lam_max;

  const float* ema_init;    /* optional [B, H*hd] fp32 contiguous */
  float* ema_final;         /* optional [B, H*hd] fp32 contiguous */
} osm_cheby_args;

/*
 * Backward arguments (with the forward's osm_cheby_args, whose `out` is the
 * saved forward output, read for the clamp mask m = [|out| < 1 - 1e-6]; it
 * may be NULL with OSM_FLAG_NO_CLAMP).  Given dL/dout and dL/d ema_final:
 *
 *   a[t] = m[t] (dL/dout[t] + lam[t+1] a[t+1]),  a past the end = dL/d ema_final
 *   dL/dx[t]  = (1-lam[t]) a[t] damping (1-z^2) p'(u) / (1+|x|)^2   (0 where
 *               |x| < 1e-7 or x is NaN)
 *   dL/dc_k   = sum_t (1-lam[t]) a[t] damping (1-z^2) T_k(u[t])
 *   dL/d ema_init = lam[0] a[0]
 *
 * lambda (static or dynamic) and damping are constants.  grad_out has the
 * dtype of out and grad_x that of x, with the same layout rules as x/out.
 */
typedef struct osm_cheby_bwd_args {
  const void* grad_out;     /* [B,S,H*hd] dL/dout, out_dtype */
  int64_t go_stride_b, go_stride_s;
  const float* grad_state;  /* optional [B, H*hd] fp32 contiguous: dL/d ema_final */
  void* grad_x;             /* [B,S,H*hd] dL/dx, x_dtype (overwritten) */
  int64_t gx_stride_b, gx_stride_s;
  float* grad_coeffs;       /* optional [B,H,K,hd] fp32 contiguous (overwritten) */
  float* grad_init;         /* optional [B, H*hd] fp32 contiguous: dL/d ema_init */
  const void* z_saved;      /* optional [B,S,H*hd] bf16: z of the forward (osm_v10_args.z_save);
                               1 - z^2 is then taken from it instead of recomputed, as the
                               full path's backward does (sdpc_kernel.py:2479-2481).
                               Static lambda and an fp32 out only. */
  int64_t z_stride_b, z_stride_s;
} osm_cheby_bwd_args;

/*
 * The reference's full apply_cheby_rkv_v10 path (S >= seq_threshold): the
 * sequence is cut into chunks of `chunk` tokens; each chunk runs with the
 * current coefficients c and Lion momentum m, per lane:
 *
 *   u = sign(x)(1 - 1/(1 + max(|x|, 1e-7)))   on bf16(x); NaN reads as 0, sign(0) = +1
 *   y = LUT(u) (OSM_V10_USE_LUT: 256-point half table `lut`, linear
 *       interpolation, odd terms times sign(u)) or the 4-term Clenshaw c0..c3
 *   z = tanh(clamp((0.98 - 0.06 h/H) y, -4, 4))   (0 for NaN x)
 *   s = mu s + (1 - mu) z from s = 0 at the chunk start;  out = bf16(s) as fp32
 *   gc_k = sum_{t, t+1 in chunk} gv T_k(u_t),  gv = err/(1 + exp(-3|err|)),
 *          err = u_{t+1} - s_t
 *   Lion: g = gc/(L-1); interp = b1 m + (1-b1) g; m <- b2 m + (1-b2) g;
 *         c <- (lam_h - lr wd) c + lr ss_k sign(interp),
 *         lr = base_lr lr_scale[h] (x gate[b]),
 *         lam_h = lion_lambda[h] (or clamp(lam_h + 0.008 (dyn[b] - 0.5), 0.9, 0.9999))
 *
 * and the next chunk uses the updated (c, m).  Replaces the chunk loop of
 * apply_cheby_rkv_v10 (sdpc_kernel.py:2574-2606) with its per-chunk
 * FusedChebyRKVv10.forward / _launch_ortho_megakernel (2353-2433,
 * 2290-2344).  One launch, no workspace.
 */
#define OSM_V10_USE_LUT 0x1

typedef struct osm_v10_args {
  int32_t abi_version;          /* = OSM_ABI_VERSION */
  int32_t flags;                /* OSM_V10_USE_LUT */
  int64_t B, S, H, hd, K;       /* 1 <= K <= 8 */
  int64_t chunk;                /* tokens per Lion step, >= 1 */
  const void* x;                /* [B,S,H*hd], x_dtype; lane stride 1 */
  int32_t x_dtype;
  int64_t x_stride_b, x_stride_s;
  float* out;                   /* [B,S,H*hd] fp32 (values rounded to bf16) */
  int64_t out_stride_b, out_stride_s;
  const float* coeffs;          /* [B,H,K,hd] fp32, lane stride 1 */
  int64_t c_stride_b, c_stride_h, c_stride_k;
  const float* momentum;        /* [B,H,K,hd] fp32, lane stride 1 */
  int64_t m_stride_b, m_stride_h, m_stride_k;
  float* coeffs_out;            /* [B,H,K,hd] fp32 contiguous: after the last chunk */
  float* momentum_out;          /* [B,H,K,hd] fp32 contiguous */
  const float* lut;             /* [8,256] fp32: T_k on the table grid (with OSM_V10_USE_LUT) */
  const float* lion_lambda;     /* [H] */
  const float* lr_scale;        /* [H] */
  const float* spectral_scale;  /* [K] */
  const float* gate;            /* optional [B]: scales lr */
  const float* dyn_lambda;      /* optional [B]: moves lam_h */
  float ema_momentum, base_lr, beta1, beta2, weight_decay;
  void* z_save;                 /* optional [B,S,H*hd] bf16: z of every token (for the backward) */
  int64_t z_stride_b, z_stride_s;
  float* coeff_hist;            /* optional [ceil(S/chunk),B,H,K,hd] fp32: the coefficients each chunk used */
  const float* ema_momentum_dev; /* optional device fp32 scalar: mu is read from it and
                                   ema_momentum is ignored, so a mu computed on the device
                                   (the engine's schedule, sdpc_engine.py:199-209) never
                                   has to reach the host */
} osm_v10_args;

/*
 * Fixed-coefficient fused forward of the same kernel family: the reference's
 * _fused_clenshaw_ema_kernel (sdpc_kernel.py:988-1209), which
 * precision_tests.py:33-73 launches.  Per lane, over all S tokens:
 *
 *   x_norm = sign(x)(1 - 1/(1 + max(|x|, 1e-7)))   on x as given; NaN reads as 0
 *   y = LUT(x_norm) (OSM_V10_USE_LUT, as osm_v10_args) or Clenshaw over c0..c3
 *       (K <= 4) or c0..c7 (K > 4)
 *   tanh_y = tanh(clamp((0.98 - 0.06 h/H) y, -4, 4))   (0 for NaN x)
 *   s = mu s + (1 - mu) tanh_y from s = ema_init;  out = clamp(s, -1, 1) (fp32)
 *
 * with the carried state clamped to [-1, 1] at every clamp_tile-th token
 * (the kernel's BLOCK_S tile carry), and ema_final = clamp of the state after
 * token S-1.  One launch, no workspace.
 */
typedef struct osm_lut_fwd_args {
  int32_t abi_version;          /* = OSM_ABI_VERSION */
  int32_t flags;                /* OSM_V10_USE_LUT */
  int64_t B, S, H, hd, K;       /* 1 <= K <= 8 */
  int64_t clamp_tile;           /* >= 16, a multiple of 16 */
  const void* x;                /* [B,S,H*hd], x_dtype; lane stride 1 */
  int32_t x_dtype;
  int64_t x_stride_b, x_stride_s;
  const float* coeffs;          /* [B,H,K,hd] fp32, lane stride 1 */
  int64_t c_stride_b, c_stride_h, c_stride_k;
  const float* lut;             /* [8,256] fp32 contiguous (with OSM_V10_USE_LUT) */
  float ema_momentum;
  const float* ema_init;        /* optional [B, H*hd] fp32, lane stride 1 (NULL: 0) */
  int64_t init_stride_b;
  float* out;                   /* [B,S,H*hd] fp32, lane stride 1 */
  int64_t out_stride_b, out_stride_s;
  float* x_norm;                /* optional [B,S,H*hd] fp32, lane stride 1 */
  int64_t xn_stride_b, xn_stride_s;
  float* tanh_y;                /* optional [B,S,H*hd] fp32, lane stride 1 */
  int64_t ty_stride_b, ty_stride_s;
  float* ema_final;             /* optional [B, H*hd] fp32, lane stride 1 */
  int64_t final_stride_b;
} osm_lut_fwd_args;

/* Which entry point a workspace is sized for. */
typedef enum osm_op { OSM_OP_FWD = 0, OSM_OP_TTT = 1, OSM_OP_BWD = 2 } osm_op;

/* ABI version the library was built with (OSM_ABI_VERSION). */
int osm_abi_version(void);

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* osm_last_error(void);

/* Workspace bytes needed by osm_cheby_ema_fwd (op = OSM_OP_FWD),
 * osm_cheby_ema_ttt (OSM_OP_TTT) or osm_cheby_ema_bwd (OSM_OP_BWD).  Reads
 * only the shape fields, dtypes, K, whether g is NULL and (forward) the x/out
 * strides and pointer alignment that choose its geometry; with x or out NULL
 * the forward is sized for its one-lane geometry, which needs the most (so
 * the size serves any later x/out of that shape).  Returns 0 if those are
 * invalid. */
size_t osm_workspace_bytes(const osm_cheby_args* args, int op);

/* Zero-fill `bytes` of workspace on `stream` with a fill kernel. */
int osm_workspace_init(void* workspace, size_t bytes, void* stream);

/* Stream-ordered health check of a workspace, with no host synchronisation:
 * a one-thread kernel on `stream` writes status[0] = the header's fault word
 * (0 if no look-back wait of a launch on this workspace has given up since
 * the last reset, else (epoch << 2 | 3) of the last launch that did, whose
 * results are invalid) and status[1] = the launch counter, into `status`
 * (2 x uint32 of device memory); with reset != 0 it then clears the fault
 * word.  workspace = NULL reads the static scratch of
 * osm_cheby_ema_fwd_static on the current device (after that entry point
 * has run there).  No counterpart in the reference, whose tile loop
 * (sdpc_kernel.py:2006) never waits on another workgroup. */
int osm_workspace_status(void* workspace, uint32_t* status, int reset, void* stream);

/* Fused forward.  Replaces the kernel launches listed in the header comment. */
int osm_cheby_ema_fwd(const osm_cheby_args* args, void* workspace, size_t workspace_bytes,
                      void* stream);

/* The fused forward of osm_cheby_ema_fwd with no workspace argument and no
 * allocation: its look-back words and header live in a static device array
 * of the library (32 MiB on every GPU it runs on, held until the process
 * ends), set up on the first call on a device.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Results
 * are those of osm_cheby_ema_fwd bit for bit.  Shapes whose workspace
 * (osm_workspace_bytes) exceeds 32 MiB return OSM_E_WORKSPACE.  `stream`
 * must belong to the current device.  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (other streams, other
 * threads) race, and must be ordered by the caller.  The array keeps the
 * last call's state (launch counter, look-back words), as a workspace does;
 * osm_workspace_status(NULL, ...) reads its fault word. */
int osm_cheby_ema_fwd_static(const osm_cheby_args* args, void* stream);

/* Fused forward + TTT coefficient gradient.  `grad` is [B,H,K,hd] fp32
 * contiguous and is overwritten.  `target` is an osm_ttt_target. */
int osm_cheby_ema_ttt(const osm_cheby_args* args, float* grad, int target, void* workspace,
                      size_t workspace_bytes, void* stream);

/* The full-path chunk loop described above osm_v10_args, in one launch on
 * `stream`.  Needs no workspace. */
int osm_v10_chunked_ttt(const osm_v10_args* args, void* stream);

/* The fixed-coefficient forward described above osm_lut_fwd_args, in one
 * launch on `stream` (replaces a launch of _fused_clenshaw_ema_kernel,
 * sdpc_kernel.py:988-1209).  Needs no workspace. */
int osm_cheby_ema_lut_fwd(const osm_lut_fwd_args* args, void* stream);

/* Backward of osm_cheby_ema_fwd: writes grad_x and, when non-NULL,
 * grad_coeffs and grad_init.  Replaces the backward listed in the header
 * comment. */
int osm_cheby_ema_bwd(const osm_cheby_args* args, const osm_cheby_bwd_args* bwd, void* workspace,
                      size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ORTHOSSM_AMD_OSM_H */
