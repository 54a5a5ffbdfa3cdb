// C ABI of the Cheby-RKV hot path: argument validation, workspace sizing and
// kernel dispatch.  Declared in include/osm.h.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>

#include "osm.h"
#include "osm_kernels.h"

// The forward's workspace for osm_cheby_ema_fwd_static: a file-scope device
// array, so that entry point allocates nothing.  Every GPU the library runs
// on holds its own copy (at its own address) until the process ends.  In
// host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, once per device, and only
// that address is ever passed to a kernel or a fill.
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return OSM_OK;
}

struct Geometry {
  int n_lbd = 0, n_lb = 0, n_lb_pad = 0, n_tiles = 0;
  int tile = 0;        // tokens per tile
  int lanes = 64;      // lanes per lane-block
  int lpt = 2;         // lanes per thread (forward)
  bool dyn = false;
  int kpad = 8;
  bool empty = false;  // B == 0 or S == 0
};

bool aligned4(const void* p, int esize) { return ((uintptr_t)p % (uintptr_t)(4 * esize)) == 0; }
bool aligned1(const void* p, int esize) { return ((uintptr_t)p % (uintptr_t)esize) == 0; }

// Validates `a` without touching the GPU and fills `geo` for the entry point
// `op` (an osm_op; the forward's tile shape comes from osm::fwd_geometry).
// The forward's two-lane geometries need hd % 4 == 0, x/out rows on
// 4-element boundaries and K <= 8; any other layout, and K up to
// OSM_MAX_K, takes its one-lane geometry.  The backward and the TTT hold
// one lane per thread and need rows aligned to one element; the TTT takes
// K <= OSM_MAX_K_TTT.
int check_args(const osm_cheby_args* a, Geometry* geo, int op, bool shapes_only = false) {
  if (!a) return fail(OSM_E_ARG, "args is NULL");
  if (a->abi_version != OSM_ABI_VERSION)
    return fail(OSM_E_ARG, "abi_version %d does not match library ABI %d", a->abi_version, OSM_ABI_VERSION);
  const int known = OSM_FLAG_NO_CLAMP | OSM_FLAG_NAN_ZERO_U | OSM_FLAG_TIMING_JITTER | OSM_FLAG_POLL_LIMIT_ZERO |
                    (op == OSM_OP_BWD ? OSM_FLAG_FULL_JACOBIAN : 0);
  if (a->flags & ~known) return fail(OSM_E_ARG, "unknown flag bits 0x%x", a->flags);
  if (a->B < 0 || a->S < 0) return fail(OSM_E_SHAPE, "B=%lld and S=%lld must be >= 0", (long long)a->B, (long long)a->S);
  if (a->H < 1 || a->hd < 1)
    return fail(OSM_E_SHAPE, "need H >= 1 and hd >= 1 (H=%lld hd=%lld)", (long long)a->H, (long long)a->hd);
  const int max_k = op == OSM_OP_TTT ? OSM_MAX_K_TTT : OSM_MAX_K;
  if (a->K < 1 || a->K > max_k)
    return fail(OSM_E_SHAPE, "K=%lld outside [1, %d]%s", (long long)a->K, max_k,
                op == OSM_OP_TTT ? " (the TTT gradient)" : "");
  const int64_t D = a->H * a->hd;
  if (D > (int64_t(1) << 28)) return fail(OSM_E_SHAPE, "D=H*hd=%lld too large", (long long)D);
  if (a->x_dtype != OSM_F32 && a->x_dtype != OSM_BF16) return fail(OSM_E_DTYPE, "x_dtype %d unsupported", a->x_dtype);
  if (a->out_dtype != OSM_F32 && a->out_dtype != OSM_BF16)
    return fail(OSM_E_DTYPE, "out_dtype %d unsupported", a->out_dtype);
  geo->dyn = a->g != nullptr;
  geo->kpad = a->K <= 4 ? 4 : (a->K <= 8 ? 8 : (a->K <= 16 ? 16 : 32));
  geo->empty = a->B == 0 || a->S == 0;
  const int xs = a->x_dtype == OSM_F32 ? 4 : 2;
  const int os = a->out_dtype == OSM_F32 ? 4 : 2;
  // A shapes-only query with x or out NULL does not know their alignment:
  // it is sized for the one-lane geometry, the largest workspace.
  const bool rows4 = a->hd % 4 == 0 && a->x && aligned4(a->x, xs) && a->x_stride_b % 4 == 0 &&
                     a->x_stride_s % 4 == 0 && a->out && aligned4(a->out, os) && a->out_stride_b % 4 == 0 &&
                     a->out_stride_s % 4 == 0;
  const bool generic = op == OSM_OP_FWD && (!rows4 || a->K > osm::kMonoMaxK);
  if (geo->empty) return OSM_OK;
  // The backward reads out only for the clamp mask.
  const bool need_out = op != OSM_OP_BWD || !(a->flags & OSM_FLAG_NO_CLAMP);
  if (!shapes_only) {
    if (!a->x || (need_out && !a->out) || !a->coeffs || !a->damping || !a->lam)
      return fail(OSM_E_ARG, "x, out, coeffs, damping and lam must be non-NULL");
    if (!aligned1(a->x, xs) || a->x_stride_b < 0 || a->x_stride_s < 0)
      return fail(OSM_E_LAYOUT, "x must be element-aligned with non-negative strides");
    if (a->out && (!aligned1(a->out, os) || a->out_stride_b < 0 || a->out_stride_s < 0))
      return fail(OSM_E_LAYOUT, "out must be element-aligned with non-negative strides");
    if (geo->dyn && !(a->lam_min <= a->lam_max))
      return fail(OSM_E_ARG, "lam_min %g > lam_max %g", (double)a->lam_min, (double)a->lam_max);
    // Rows of out must not overlap (padding rows of the last tile are masked
    // by extent, which needs out_stride_s >= D and batches after all rows).
    if (a->out && (a->out_stride_s < D || a->out_stride_b < a->S * a->out_stride_s))
      return fail(OSM_E_LAYOUT, "out rows/batches overlap (out_stride_s=%lld < D or out_stride_b too small)",
                  (long long)a->out_stride_s);
    // One tile's byte span must fit a buffer descriptor's 31-bit offsets.
    const int64_t tile_rows = osm::kMaxTileRows + 1;
    if ((tile_rows * a->x_stride_s + D) * xs >= (int64_t(1) << 31) ||
        (tile_rows * a->out_stride_s + D) * os >= (int64_t(1) << 31))
      return fail(OSM_E_LAYOUT, "token stride too large for 31-bit tile offsets");
    if (geo->dyn) {
      if (a->g_stride_b < 0 || a->g_stride_s < 0 || a->g_stride_h < 0)
        return fail(OSM_E_LAYOUT, "g strides must be non-negative");
      if ((tile_rows * a->g_stride_s + a->H * a->g_stride_h + 1) * 4 >= (int64_t(1) << 31))
        return fail(OSM_E_LAYOUT, "g strides too large for 31-bit tile offsets");
    }
    if ((a->H * a->c_stride_h + a->K * a->c_stride_k + a->hd) * 4 >= (int64_t(1) << 31) || a->c_stride_h < 0 ||
        a->c_stride_k < 0 || a->c_stride_b < 0)
      return fail(OSM_E_LAYOUT, "coeffs strides must be non-negative and fit 31-bit offsets");
  }
  osm::FwdShape shape{osm::ttt_tile_tokens(geo->dyn, a->x_dtype), osm::TttTile::LANES, 1};
  if (op == OSM_OP_FWD) shape = osm::fwd_geometry(geo->dyn, a->B, D, a->S, generic);
  if (op == OSM_OP_BWD) shape = osm::FwdShape{osm::bwd_tile_tokens(geo->dyn, geo->kpad), osm::BwdTile::LANES, 1};
  const int64_t tile = shape.tile;
  const int64_t n_lbd = (D + shape.lanes - 1) / shape.lanes;
  const int64_t n_lb = a->B * n_lbd;
  const int64_t n_tiles = (a->S + tile - 1) / tile;
  const int64_t n_lb_pad = (n_lb + 7) / 8 * 8;
  if (n_lb_pad * n_tiles >= (int64_t(1) << 31) || a->S >= (int64_t(1) << 31) - tile)
    return fail(OSM_E_SHAPE, "problem too large: %lld tiles", (long long)(n_lb * n_tiles));
  geo->n_lbd = (int)n_lbd;
  geo->n_lb = (int)n_lb;
  geo->n_lb_pad = (int)n_lb_pad;
  geo->n_tiles = (int)n_tiles;
  geo->tile = (int)tile;
  geo->lanes = shape.lanes;
  geo->lpt = shape.lpt;
  return OSM_OK;
}

osm::FwdParams make_params(const osm_cheby_args* a, const Geometry& geo, void* ws) {
  osm::FwdParams p{};
  p.x = a->x;
  p.out = a->out;
  p.coeffs = a->coeffs;
  p.damping = a->damping;
  p.lam = a->lam;
  p.g = a->g;
  p.ema_init = a->ema_init;
  p.ema_final = a->ema_final;
  p.hdr = reinterpret_cast<unsigned*>(ws);
  p.slots = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + osm::kHeaderBytes);
  p.x_sb = a->x_stride_b;
  p.x_ss = a->x_stride_s;
  p.o_sb = a->out_stride_b;
  p.o_ss = a->out_stride_s;
  p.c_sb = a->c_stride_b;
  p.c_sh = a->c_stride_h;
  p.c_sk = a->c_stride_k;
  p.g_sb = a->g_stride_b;
  p.g_ss = a->g_stride_s;
  p.g_sh = a->g_stride_h;
  p.B = (int)a->B;
  p.S = (int)a->S;
  p.H = (int)a->H;
  p.hd = (int)a->hd;
  osm::div_magic((uint32_t)a->hd, &p.hd_magic, &p.hd_shift);
  p.K = (int)a->K;
  p.D = (int)(a->H * a->hd);
  p.n_lbd = geo.n_lbd;
  p.n_lb = geo.n_lb;
  p.n_lb_pad = geo.n_lb_pad;
  p.n_tiles = geo.n_tiles;
  p.lam_shift = a->lam_shift;
  p.lam_min = a->lam_min;
  p.lam_max = a->lam_max;
  p.clamp_out = (a->flags & OSM_FLAG_NO_CLAMP) ? 0 : 1;
  p.nan_zero_u = (a->flags & OSM_FLAG_NAN_ZERO_U) ? 1 : 0;
  p.jitter = (a->flags & OSM_FLAG_TIMING_JITTER) ? 1 : 0;
  p.poll_limit = (a->flags & OSM_FLAG_POLL_LIMIT_ZERO) ? 0u : osm::kSpinLimit;
  return p;
}

size_t ws_bytes_for(const Geometry& geo, int op, int K) {
  if (geo.empty) return osm::kHeaderBytes;
  if (op == OSM_OP_TTT) return osm::ttt_workspace_bytes(geo.n_lb, geo.n_tiles, geo.dyn, K);
  if (op == OSM_OP_BWD) return osm::bwd_workspace_bytes(geo.n_lb, geo.n_tiles, K);
  return osm::fwd_workspace_bytes(geo.n_lb, geo.n_tiles, geo.lanes, geo.dyn);
}

int check_ws(const Geometry& geo, int op, int K, void* ws, size_t ws_bytes) {
  if (!ws) return fail(OSM_E_WORKSPACE, "workspace is NULL");
  if ((uintptr_t)ws % 256) return fail(OSM_E_WORKSPACE, "workspace must be 256-byte aligned");
  const size_t need = ws_bytes_for(geo, op, K);
  if (ws_bytes < need)
    return fail(OSM_E_WORKSPACE, "workspace has %zu bytes, needs %zu", ws_bytes, need);
  return OSM_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(OSM_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Layout last used on each workspace.  Look-back words carry the tag of the
// launch that wrote them and the header's launch epoch only ever grows (a
// clear on a layout change leaves the header alone), so a word left by an
// earlier launch, of any layout, never matches a later launch's tag: the
// workspace needs no clear between launches.  The look-back words are still
// cleared when the layout changes (other shape, mode or lambda kind), which
// keeps stale payloads of another layout out of the words a launch reads.  A
// workspace seen for the first time is cleared in full (header included),
// unless osm_workspace_init zeroed it.
struct Layout {
  int n_lb, n_tiles, tile, lanes, lpt, kpad;
  bool dyn;
  int op;
  bool operator==(const Layout& o) const {
    return n_lb == o.n_lb && n_tiles == o.n_tiles && tile == o.tile && lanes == o.lanes && lpt == o.lpt &&
           kpad == o.kpad && dyn == o.dyn && op == o.op;
  }
};
const Layout kZeroed{-1, -1, -1, -1, -1, -1, false, -1};
std::mutex g_ws_mu;
std::unordered_map<uintptr_t, Layout> g_ws_layout;

int prepare_workspace(void* ws, size_t need, const Geometry& geo, int op, hipStream_t stream) {
  const Layout now{geo.n_lb, geo.n_tiles, geo.tile, geo.lanes, geo.lpt, geo.kpad, geo.dyn, op};
  bool fresh, clear;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws_layout.find((uintptr_t)ws);
    fresh = it == g_ws_layout.end();
    clear = fresh || !(it->second == now || it->second == kZeroed);
    g_ws_layout[(uintptr_t)ws] = now;
  }
  if (clear) {
    // A known workspace keeps the start of its header (launch epoch, fault
    // word); the completion counters after it and the look-back words are
    // cleared, which also repairs counters that overlapping calls (misuse)
    // left behind.
    const size_t skip = fresh ? 0 : osm::kHeaderKeepBytes;
    const hipError_t e = osm::launch_fill_zero(static_cast<char*>(ws) + skip, need - skip, stream);
    if (e != hipSuccess) {
      std::lock_guard<std::mutex> lk(g_ws_mu);
      g_ws_layout.erase((uintptr_t)ws);
      return hip_fail(e, "workspace clear launch");
    }
  }
  return OSM_OK;
}

// Per-device state of the static scratch, in fixed storage (no allocation
// on the entry point's path): its device address, and the layout of the
// last launch on it (clears follow the rules of prepare_workspace).
constexpr int kMaxDevices = 64;
struct StaticScratch {
  void* ptr;
  bool used;       // a launch has run on it (else the first one clears it in full)
  Layout layout;   // layout of the last launch
};
StaticScratch g_static[kMaxDevices];
std::mutex g_static_mu;

// Device address of the current device's scratch, set up on its first use
// with that device current.  Returns OSM_OK or an error status.
int static_scratch_ptr(int* dev_out, void** ptr_out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(OSM_E_ARG, "device %d beyond the %d the static scratch serves", dev,
                                                 kMaxDevices);
  std::lock_guard<std::mutex> lk(g_static_mu);
  if (!g_static[dev].ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    g_static[dev].ptr = p;
  }
  *dev_out = dev;
  *ptr_out = g_static[dev].ptr;
  return OSM_OK;
}

// S == 0 (or B == 0): nothing to compute; the final state equals the initial one.
int run_empty(const osm_cheby_args* a, hipStream_t stream) {
  if (a->B > 0 && a->ema_final) {
    const size_t n = (size_t)a->B * (size_t)(a->H * a->hd);
    const hipError_t e = a->ema_init ? osm::launch_copy_state(a->ema_init, a->ema_final, n, stream)
                                     : osm::launch_fill_zero(a->ema_final, n * sizeof(float), stream);
    if (e != hipSuccess) return hip_fail(e, "state copy launch");
  }
  return ok();
}

}  // namespace

extern "C" {

int osm_abi_version(void) { return OSM_ABI_VERSION; }

const char* osm_last_error(void) { return g_err.c_str(); }

size_t osm_workspace_bytes(const osm_cheby_args* args, int op) {
  if (op != OSM_OP_FWD && op != OSM_OP_TTT && op != OSM_OP_BWD) {
    fail(OSM_E_ARG, "op %d is not an osm_op", op);
    return 0;
  }
  Geometry geo;
  if (check_args(args, &geo, op, /*shapes_only=*/true) != OSM_OK) return 0;
  return ws_bytes_for(geo, op, (int)args->K);
}

int osm_workspace_init(void* workspace, size_t bytes, void* stream) {
  if (!workspace) return fail(OSM_E_WORKSPACE, "workspace is NULL");
  if ((uintptr_t)workspace % 256 || bytes % 4) return fail(OSM_E_WORKSPACE, "workspace must be 256-byte aligned and a multiple of 4 bytes");
  const hipError_t e = osm::launch_fill_zero(workspace, bytes, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "workspace fill launch");
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    g_ws_layout[(uintptr_t)workspace] = kZeroed;
  }
  return ok();
}

int osm_workspace_status(void* workspace, uint32_t* status, int reset, void* stream) {
  if (!workspace) {
    // The static scratch of osm_cheby_ema_fwd_static on the current device.
    int dev;
    const int rc = static_scratch_ptr(&dev, &workspace);
    if (rc != OSM_OK) return rc;
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static[dev].used)
      return fail(OSM_E_WORKSPACE, "workspace is NULL and osm_cheby_ema_fwd_static has not run on device %d", dev);
  }
  if ((uintptr_t)workspace % 256) return fail(OSM_E_WORKSPACE, "workspace must be 256-byte aligned");
  if (!status || (uintptr_t)status % 4) return fail(OSM_E_ARG, "status must be a 4-byte aligned device pointer");
  const hipError_t e = osm::launch_ws_status(workspace, status, reset ? 1 : 0, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "workspace status launch");
  return ok();
}

int osm_cheby_ema_fwd(const osm_cheby_args* args, void* workspace, size_t workspace_bytes, void* stream) {
  Geometry geo;
  int rc = check_args(args, &geo, OSM_OP_FWD);
  if (rc != OSM_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (geo.empty) return run_empty(args, st);
  rc = check_ws(geo, OSM_OP_FWD, (int)args->K, workspace, workspace_bytes);
  if (rc != OSM_OK) return rc;
  rc = prepare_workspace(workspace, osm::fwd_workspace_bytes(geo.n_lb, geo.n_tiles, geo.lanes, geo.dyn), geo,
                         OSM_OP_FWD, st);
  if (rc != OSM_OK) return rc;
  const osm::FwdParams p = make_params(args, geo, workspace);
  const hipError_t e = osm::launch_fwd(p, args->x_dtype, args->out_dtype, geo.dyn, osm::FwdShape{geo.tile, geo.lanes, geo.lpt}, geo.kpad, st);
  if (e != hipSuccess) return hip_fail(e, "forward kernel launch");
  return ok();
}

int osm_cheby_ema_fwd_static(const osm_cheby_args* args, void* stream) {
  Geometry geo;
  int rc = check_args(args, &geo, OSM_OP_FWD);
  if (rc != OSM_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (geo.empty) return run_empty(args, st);
  const size_t need = osm::fwd_workspace_bytes(geo.n_lb, geo.n_tiles, geo.lanes, geo.dyn);
  if (need > kStaticScratchBytes)
    return fail(OSM_E_WORKSPACE,
                "this shape needs %zu bytes of look-back workspace; the static scratch holds %zu "
                "(use osm_cheby_ema_fwd with a caller workspace)",
                need, kStaticScratchBytes);
  int dev;
  void* ws;
  rc = static_scratch_ptr(&dev, &ws);
  if (rc != OSM_OK) return rc;
  const Layout now{geo.n_lb, geo.n_tiles, geo.tile, geo.lanes, geo.lpt, geo.kpad, geo.dyn, OSM_OP_FWD};
  size_t skip = 0;
  bool clear;
  {
    std::lock_guard<std::mutex> lk(g_static_mu);
    StaticScratch& sc = g_static[dev];
    clear = !sc.used || !(sc.layout == now);
    skip = sc.used ? osm::kHeaderKeepBytes : 0;   // a used scratch keeps its launch counter and fault word
    sc.used = true;
    sc.layout = now;
  }
  if (clear) {
    const hipError_t e = osm::launch_fill_zero(static_cast<char*>(ws) + skip, need - skip, st);
    if (e != hipSuccess) {
      std::lock_guard<std::mutex> lk(g_static_mu);
      g_static[dev].used = false;
      return hip_fail(e, "static scratch clear launch");
    }
  }
  const osm::FwdParams p = make_params(args, geo, ws);
  const hipError_t e = osm::launch_fwd(p, args->x_dtype, args->out_dtype, geo.dyn, osm::FwdShape{geo.tile, geo.lanes, geo.lpt},
                                       geo.kpad, st);
  if (e != hipSuccess) return hip_fail(e, "forward kernel launch");
  return ok();
}

int osm_cheby_ema_ttt(const osm_cheby_args* args, float* grad, int target, void* workspace,
                      size_t workspace_bytes, void* stream) {
  Geometry geo;
  int rc = check_args(args, &geo, OSM_OP_TTT);
  if (rc != OSM_OK) return rc;
  if (!grad && !geo.empty) return fail(OSM_E_ARG, "grad must be non-NULL");
  if (target != OSM_TARGET_X && target != OSM_TARGET_SOFTSIGN)
    return fail(OSM_E_ARG, "target %d is not an osm_ttt_target", target);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (geo.empty) {
    if (args->B > 0 && grad) {
      const size_t n = (size_t)args->B * args->H * args->K * args->hd;
      const hipError_t e = osm::launch_fill_zero(grad, n * sizeof(float), st);
      if (e != hipSuccess) return hip_fail(e, "grad fill launch");
    }
    return run_empty(args, st);
  }
  rc = check_ws(geo, OSM_OP_TTT, (int)args->K, workspace, workspace_bytes);
  if (rc != OSM_OK) return rc;
  // Only the header and look-back words need clearing: the TTT partials are
  // fully written by every launch before they are read.
  const size_t slot_bytes = osm::fwd_workspace_bytes(geo.n_lb, geo.n_tiles, geo.lanes, geo.dyn);
  rc = prepare_workspace(workspace, slot_bytes, geo, OSM_OP_TTT, st);
  if (rc != OSM_OK) return rc;
  osm::FwdParams p = make_params(args, geo, workspace);
  p.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((slot_bytes + 255) / 256) * 256);
  p.ttt_scale = args->S > 1 ? (float)(2.0 / ((double)args->B * (double)(args->S - 1) * (double)p.D)) : 0.0f;
  p.ttt_target = target;
  const hipError_t e = osm::launch_ttt(p, grad, args->x_dtype, args->out_dtype, geo.dyn, geo.tile, geo.kpad, st);
  if (e != hipSuccess) return hip_fail(e, "TTT kernel launch");
  return ok();
}

int osm_v10_chunked_ttt(const osm_v10_args* a, void* stream) {
  if (!a) return fail(OSM_E_ARG, "args is NULL");
  if (a->abi_version != OSM_ABI_VERSION)
    return fail(OSM_E_ARG, "abi_version %d does not match library ABI %d", a->abi_version, OSM_ABI_VERSION);
  if (a->flags & ~OSM_V10_USE_LUT) return fail(OSM_E_ARG, "unknown flag bits 0x%x", a->flags);
  if (a->B < 0 || a->S < 0 || a->H < 1 || a->hd < 1)
    return fail(OSM_E_SHAPE, "need B, S >= 0, H, hd >= 1 (B=%lld S=%lld H=%lld hd=%lld)", (long long)a->B,
                (long long)a->S, (long long)a->H, (long long)a->hd);
  // The reference's kernels clamp the degree to 8 (sdpc_kernel.py:2379);
  // callers pass coefficients past the eighth around the full path.
  constexpr int kMaxKV10 = 8;
  if (a->K < 1 || a->K > kMaxKV10) return fail(OSM_E_SHAPE, "K=%lld outside [1, %d]", (long long)a->K, kMaxKV10);
  if (a->chunk < 1) return fail(OSM_E_SHAPE, "chunk=%lld must be >= 1", (long long)a->chunk);
  if (a->x_dtype != OSM_F32 && a->x_dtype != OSM_BF16) return fail(OSM_E_DTYPE, "x_dtype %d unsupported", a->x_dtype);
  const int64_t D = a->H * a->hd;
  if (D > (int64_t(1) << 28) || a->S >= (int64_t(1) << 31) || a->chunk >= (int64_t(1) << 31))
    return fail(OSM_E_SHAPE, "problem too large");
  if (a->S == 0) return fail(OSM_E_SHAPE, "the full path needs S >= 1");
  if (a->B == 0) return ok();
  if (!a->x || !a->out || !a->coeffs || !a->momentum || !a->coeffs_out || !a->momentum_out || !a->lion_lambda ||
      !a->lr_scale || !a->spectral_scale || ((a->flags & OSM_V10_USE_LUT) && !a->lut))
    return fail(OSM_E_ARG, "x, out, coeffs, momentum, coeffs_out, momentum_out, lion_lambda, lr_scale, "
                           "spectral_scale (and lut with OSM_V10_USE_LUT) must be non-NULL");
  const int xs = a->x_dtype == OSM_F32 ? 4 : 2;
  if ((uintptr_t)a->x % xs || (uintptr_t)a->out % 4 || a->x_stride_b < 0 || a->x_stride_s < 0)
    return fail(OSM_E_LAYOUT, "x and out must be element-aligned with non-negative strides");
  if (a->out_stride_s < D || a->out_stride_b < a->S * a->out_stride_s)
    return fail(OSM_E_LAYOUT, "out rows/batches overlap");
  if (a->z_save && (a->z_stride_s < D || a->z_stride_b < a->S * a->z_stride_s || (uintptr_t)a->z_save % 2))
    return fail(OSM_E_LAYOUT, "z_save rows/batches overlap or z_save misaligned");
  // Rows are addressed through buffer descriptors rebased at every block of
  // kV10Groups * kV10Run tokens: a block and the row after it must fit their
  // 31-bit byte offsets.
  const int64_t lim = int64_t(1) << 31;
  const int64_t blk_rows = osm::kV10Groups * osm::kV10Run + 1;
  if ((blk_rows * a->x_stride_s + D) * xs >= lim || (blk_rows * a->out_stride_s + D) * 4 >= lim ||
      (a->z_save && (blk_rows * a->z_stride_s + D) * 2 >= lim))
    return fail(OSM_E_LAYOUT, "token stride too large: 257 rows span more than 2 GiB");
  if (a->c_stride_b < 0 || a->c_stride_h < 0 || a->c_stride_k < 0 || a->m_stride_b < 0 || a->m_stride_h < 0 ||
      a->m_stride_k < 0)
    return fail(OSM_E_LAYOUT, "coeffs/momentum strides must be non-negative");
  if ((uintptr_t)a->ema_momentum_dev % 4) return fail(OSM_E_LAYOUT, "ema_momentum_dev misaligned");
  osm::V10Params p{};
  p.x = a->x;
  p.out = a->out;
  p.coeffs = a->coeffs;
  p.momentum = a->momentum;
  p.coeffs_out = a->coeffs_out;
  p.momentum_out = a->momentum_out;
  p.lut = a->lut;
  p.lion_lambda = a->lion_lambda;
  p.lr_scale = a->lr_scale;
  p.spectral_scale = a->spectral_scale;
  p.gate = a->gate;
  p.dyn_lambda = a->dyn_lambda;
  p.z_save = a->z_save;
  p.coeff_hist = a->coeff_hist;
  p.x_sb = a->x_stride_b;
  p.x_ss = a->x_stride_s;
  p.o_sb = a->out_stride_b;
  p.o_ss = a->out_stride_s;
  p.z_sb = a->z_stride_b;
  p.z_ss = a->z_stride_s;
  p.c_sb = a->c_stride_b;
  p.c_sh = a->c_stride_h;
  p.c_sk = a->c_stride_k;
  p.m_sb = a->m_stride_b;
  p.m_sh = a->m_stride_h;
  p.m_sk = a->m_stride_k;
  p.B = (int)a->B;
  p.S = (int)a->S;
  p.H = (int)a->H;
  p.hd = (int)a->hd;
  p.K = (int)a->K;
  p.D = (int)D;
  p.chunk = (int)std::min<int64_t>(a->chunk, a->S);
  p.lanes = osm::v10_lanes(a->B, a->H, a->hd);
  p.n_lg = (int)((a->hd + p.lanes - 1) / p.lanes);
  p.mu = a->ema_momentum;
  p.mu_dev = a->ema_momentum_dev;
  p.base_lr = a->base_lr;
  p.beta1 = a->beta1;
  p.beta2 = a->beta2;
  p.wd = a->weight_decay;
  if ((int64_t)p.B * p.H * p.n_lg >= (int64_t(1) << 31)) return fail(OSM_E_SHAPE, "problem too large");
  const hipError_t e = osm::launch_v10(p, a->x_dtype, (a->flags & OSM_V10_USE_LUT) != 0, a->K <= 4 ? 4 : 8,
                                       static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "full-path kernel launch");
  return ok();
}

int osm_cheby_ema_lut_fwd(const osm_lut_fwd_args* a, void* stream) {
  if (!a) return fail(OSM_E_ARG, "args is NULL");
  if (a->abi_version != OSM_ABI_VERSION)
    return fail(OSM_E_ARG, "abi_version %d does not match library ABI %d", a->abi_version, OSM_ABI_VERSION);
  if (a->flags & ~OSM_V10_USE_LUT) return fail(OSM_E_ARG, "unknown flag bits 0x%x", a->flags);
  if (a->B < 0 || a->S < 0 || a->H < 1 || a->hd < 1)
    return fail(OSM_E_SHAPE, "need B, S >= 0, H, hd >= 1 (B=%lld S=%lld H=%lld hd=%lld)", (long long)a->B,
                (long long)a->S, (long long)a->H, (long long)a->hd);
  // The reference kernel loads eight coefficients at most (sdpc_kernel.py:1047-1054).
  if (a->K < 1 || a->K > 8) return fail(OSM_E_SHAPE, "K=%lld outside [1, 8]", (long long)a->K);
  // The carried state is clamped between waves of 16 or 32 tokens.
  if (a->clamp_tile < 16 || a->clamp_tile % 16 || a->clamp_tile >= (int64_t(1) << 30))
    return fail(OSM_E_SHAPE, "clamp_tile=%lld must be a multiple of 16", (long long)a->clamp_tile);
  if (a->x_dtype != OSM_F32 && a->x_dtype != OSM_BF16) return fail(OSM_E_DTYPE, "x_dtype %d unsupported", a->x_dtype);
  const int64_t D = a->H * a->hd;
  if (D > (int64_t(1) << 28) || a->S >= (int64_t(1) << 31)) return fail(OSM_E_SHAPE, "problem too large");
  if (a->B == 0) return ok();
  // (S = 0 reads and writes no rows: only ema_final, from ema_init)
  if (a->S > 0 && (!a->x || !a->coeffs || !a->out || ((a->flags & OSM_V10_USE_LUT) && !a->lut)))
    return fail(OSM_E_ARG, "x, coeffs, out (and lut with OSM_V10_USE_LUT) must be non-NULL");
  const int xs = a->x_dtype == OSM_F32 ? 4 : 2;
  if ((uintptr_t)a->x % xs || a->x_stride_b < 0 || a->x_stride_s < 0)
    return fail(OSM_E_LAYOUT, "x must be element-aligned with non-negative strides");
  // Row outputs: aligned, rows and batches not overlapping.
  struct RowOut {
    const float* p;
    int64_t sb, ss;
    const char* what;
  };
  const RowOut outs[3] = {{a->out, a->out_stride_b, a->out_stride_s, "out"},
                          {a->x_norm, a->xn_stride_b, a->xn_stride_s, "x_norm"},
                          {a->tanh_y, a->ty_stride_b, a->ty_stride_s, "tanh_y"}};
  const int64_t lim = int64_t(1) << 31;
  const int64_t blk_rows = osm::kV10Groups * osm::kV10Run + 1;
  for (const RowOut& o : outs) {
    if (!o.p) continue;
    if ((uintptr_t)o.p % 4 || o.ss < D || o.sb < a->S * o.ss)
      return fail(OSM_E_LAYOUT, "%s misaligned or its rows/batches overlap", o.what);
    if ((blk_rows * o.ss + D) * 4 >= lim) return fail(OSM_E_LAYOUT, "%s token stride too large", o.what);
  }
  if ((blk_rows * a->x_stride_s + D) * xs >= lim)
    return fail(OSM_E_LAYOUT, "token stride too large: 257 rows span more than 2 GiB");
  if (a->c_stride_b < 0 || a->c_stride_h < 0 || a->c_stride_k < 0)
    return fail(OSM_E_LAYOUT, "coeffs strides must be non-negative");
  if (a->ema_init && ((uintptr_t)a->ema_init % 4 || a->init_stride_b < 0))
    return fail(OSM_E_LAYOUT, "ema_init misaligned or with a negative stride");
  if (a->ema_final && ((uintptr_t)a->ema_final % 4 || a->final_stride_b < D))
    return fail(OSM_E_LAYOUT, "ema_final misaligned or its rows overlap");
  osm::V10FixedParams p{};
  p.x = a->x;
  p.out = a->out;
  p.coeffs = a->coeffs;
  p.lut = a->lut;
  p.x_sb = a->x_stride_b;
  p.x_ss = a->x_stride_s;
  p.o_sb = a->out_stride_b;
  p.o_ss = a->out_stride_s;
  p.c_sb = a->c_stride_b;
  p.c_sh = a->c_stride_h;
  p.c_sk = a->c_stride_k;
  p.B = (int)a->B;
  p.S = (int)a->S;
  p.H = (int)a->H;
  p.hd = (int)a->hd;
  p.K = (int)a->K;
  p.D = (int)D;
  p.chunk = (int)std::max<int64_t>(a->S, 1);   // one chunk; none when S = 0
  // Waves of 32 tokens with 8 lanes per workgroup, 16 with 16 lanes: the
  // clamp boundaries fall between waves.
  p.lanes = a->clamp_tile % 32 ? 16 : osm::v10_lanes(a->B, a->H, a->hd);
  p.n_lg = (int)((a->hd + p.lanes - 1) / p.lanes);
  p.mu = a->ema_momentum;
  p.ema_init = a->ema_init;
  p.init_sb = a->init_stride_b;
  p.ema_final = a->ema_final;
  p.final_sb = a->final_stride_b;
  p.xnorm = a->x_norm;
  p.xn_sb = a->xn_stride_b;
  p.xn_ss = a->xn_stride_s;
  p.tanhy = a->tanh_y;
  p.ty_sb = a->ty_stride_b;
  p.ty_ss = a->ty_stride_s;
  p.clamp_tile = (int)a->clamp_tile;
  if ((int64_t)p.B * p.H * p.n_lg >= (int64_t(1) << 31)) return fail(OSM_E_SHAPE, "problem too large");
  const hipError_t e = osm::launch_v10_fixed(p, a->x_dtype, (a->flags & OSM_V10_USE_LUT) != 0, a->K <= 4 ? 4 : 8,
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "fixed-coefficient forward launch");
  return ok();
}

int osm_cheby_ema_bwd(const osm_cheby_args* args, const osm_cheby_bwd_args* bwd, void* workspace,
                      size_t workspace_bytes, void* stream) {
  Geometry geo;
  int rc = check_args(args, &geo, OSM_OP_BWD);
  if (rc != OSM_OK) return rc;
  if (!bwd) return fail(OSM_E_ARG, "bwd is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t D = args->H * args->hd;
  if (geo.empty) {
    // No tokens: dL/dc = 0 and ema_final = ema_init, so dL/d ema_init = dL/d ema_final.
    if (args->B > 0) {
      hipError_t e = hipSuccess;
      if (bwd->grad_coeffs)
        e = osm::launch_fill_zero(bwd->grad_coeffs, (size_t)args->B * args->H * args->K * args->hd * sizeof(float), st);
      if (e == hipSuccess && bwd->grad_init) {
        const size_t n = (size_t)args->B * (size_t)D;
        e = bwd->grad_state ? osm::launch_copy_state(bwd->grad_state, bwd->grad_init, n, st)
                            : osm::launch_fill_zero(bwd->grad_init, n * sizeof(float), st);
      }
      if (e != hipSuccess) return hip_fail(e, "gradient fill launch");
    }
    return ok();
  }
  if (!bwd->grad_out || !bwd->grad_x) return fail(OSM_E_ARG, "grad_out and grad_x must be non-NULL");
  const int xs = args->x_dtype == OSM_F32 ? 4 : 2;
  const int os = args->out_dtype == OSM_F32 ? 4 : 2;
  if (!aligned1(bwd->grad_out, os) || bwd->go_stride_b < 0 || bwd->go_stride_s < 0)
    return fail(OSM_E_LAYOUT, "grad_out must be element-aligned with non-negative strides");
  if (!aligned1(bwd->grad_x, xs))
    return fail(OSM_E_LAYOUT, "grad_x must be element-aligned");
  if (bwd->gx_stride_s < D || bwd->gx_stride_b < args->S * bwd->gx_stride_s)
    return fail(OSM_E_LAYOUT, "grad_x rows/batches overlap (gx_stride_s=%lld < D or gx_stride_b too small)",
                (long long)bwd->gx_stride_s);
  const int64_t tile_rows = osm::kMaxTileRows + 1;
  if ((tile_rows * bwd->go_stride_s + D) * os >= (int64_t(1) << 31) ||
      (tile_rows * bwd->gx_stride_s + D) * xs >= (int64_t(1) << 31))
    return fail(OSM_E_LAYOUT, "token stride too large for 31-bit tile offsets");
  if (bwd->z_saved) {
    if (geo.dyn || args->out_dtype != OSM_F32)
      return fail(OSM_E_ARG, "z_saved needs a static lambda and an fp32 out");
    if (args->K > osm::kMonoMaxK)
      return fail(OSM_E_ARG, "z_saved needs K <= %d (K=%lld)", osm::kMonoMaxK, (long long)args->K);
    if ((uintptr_t)bwd->z_saved % 2 || bwd->z_stride_b < 0 || bwd->z_stride_s < 0 ||
        (tile_rows * bwd->z_stride_s + D) * 2 >= (int64_t(1) << 31))
      return fail(OSM_E_LAYOUT, "z_saved must be bf16-aligned with non-negative strides fitting 31-bit offsets");
  }
  rc = check_ws(geo, OSM_OP_BWD, (int)args->K, workspace, workspace_bytes);
  if (rc != OSM_OK) return rc;
  // Only the header and look-back words need clearing: the partials are
  // fully written by every launch before they are read.
  const size_t slot_bytes = osm::bwd_slot_bytes(geo.n_lb, geo.n_tiles);
  rc = prepare_workspace(workspace, slot_bytes, geo, OSM_OP_BWD, st);
  if (rc != OSM_OK) return rc;
  osm::BwdParams bp{};
  bp.f = make_params(args, geo, workspace);
  bp.f.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((slot_bytes + 255) / 256) * 256);
  bp.gout = bwd->grad_out;
  bp.go_sb = bwd->go_stride_b;
  bp.go_ss = bwd->go_stride_s;
  bp.gx = bwd->grad_x;
  bp.gx_sb = bwd->gx_stride_b;
  bp.gx_ss = bwd->gx_stride_s;
  bp.grad_state = bwd->grad_state;
  bp.grad_init = bwd->grad_init;
  bp.grad_coeffs = bwd->grad_coeffs;
  bp.zs = bwd->z_saved;
  bp.zs_sb = bwd->z_stride_b;
  bp.zs_ss = bwd->z_stride_s;
  bp.full_jac = (args->flags & OSM_FLAG_FULL_JACOBIAN) ? 1 : 0;
  const hipError_t e = osm::launch_bwd(bp, args->x_dtype, args->out_dtype, geo.dyn, geo.tile, geo.kpad, st);
  if (e != hipSuccess) return hip_fail(e, "backward kernel launch");
  return ok();
}

}  // extern "C"
