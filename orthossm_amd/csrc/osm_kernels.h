// Launch parameters, tile geometry and launcher declarations shared by the
// kernel files and the C-ABI layer.  No torch types.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

namespace osm {

// Largest padded coefficient count evaluated in monomial form.  Beyond it
// the monomial coefficients of T_k grow like 2^(k-1) and cancel in fp32, so
// longer series keep their Chebyshev coefficients and use Clenshaw.
constexpr int kMonoMaxK = 8;

// Tile geometry.  A lane-block is LANES (64 or 128) consecutive lanes of one
// batch row; a tile is TILE consecutive tokens of a lane-block and is one
// workgroup.  A thread owns LPT adjacent lanes and a run of R consecutive
// tokens; TPR threads cover the LANES lanes of a row, so one wave instruction
// reads or writes TGW rows x LANES*4 contiguous bytes (fp32).  Token groups
// (runs) are ordered wave-major: tg = wave * TGW + lane_in_wave / TPR.  The
// look-back serves each 64-lane sub-block with WPS waves of WPT words per
// thread, so tiles are grouped in checkpoint runs of CKPT = WPS * WPT.
template <int LPT_, int WAVES_, int R_, int LANES_ = 64, int WPT_ = 8>
struct TileGeo {
  static constexpr int LPT = LPT_;            // lanes per thread
  static constexpr int WAVES = WAVES_;        // waves per workgroup
  static constexpr int R = R_;                // tokens per thread run
  static constexpr int LANES = LANES_;        // lanes per lane-block
  static constexpr int THREADS = WAVES * 64;
  static constexpr int NSUB = LANES / 64;     // 64-lane look-back sub-blocks
  static constexpr int TPR = LANES / LPT;     // threads per row
  static constexpr int TGW = 64 / TPR;        // token groups per wave
  static constexpr int NTG = WAVES * TGW;     // token groups per tile
  static constexpr int TILE = NTG * R;        // tokens per tile
  static constexpr int WPS = WAVES / NSUB;    // look-back waves per sub-block
  static constexpr int WPT = WPT_;            // look-back words per thread
  static constexpr int CKPT = WPS * WPT;      // checkpoint interval, tiles
  static_assert(LANES % 64 == 0 && LANES % LPT == 0 && TPR <= 64 && 64 % TPR == 0, "geometry");
  static_assert(WAVES % NSUB == 0, "look-back waves");
};

// Forward: the run length sets the tile.  Longer runs amortise the per-tile
// scan and look-back over more tokens but give fewer workgroups, so the host
// takes the largest tile that still fills the chip (fwd_geometry).  Dynamic
// lambda keeps a per-token lambda in registers and is limited to the medium
// tile.  Measured on MI355X at BASELINE configs[1] against 128-lane tiles
// with 2 or 4 lanes per thread (256 and 128 tokens) and 64-lane tiles with 4
// lanes per thread: the 64-lane, 2-lane, 512-token tile is fastest.
// The medium and small tiles (dynamic lambda, and short sequences) read one
// look-back word per thread (checkpoints every 8 tiles): every thread runs
// the polling code of each of its words, and at configs[3] one word gives
// 420 us against 429 with two and 449 with eight.  The large tile keeps
// eight (no difference at configs[1]).
using FwdTileLarge = TileGeo<2, 8, 32>;           // 512 tokens x 64 lanes
// Dynamic lambda at 512 tokens: the per-token lambda lives in LDS (formed
// once per token and head), which leaves the registers for the run; one
// look-back word per thread (two per word pair: A and B).
using FwdTileLargeDyn = TileGeo<2, 8, 32, 64, 1>;
using FwdTileMedium = TileGeo<2, 8, 16, 64, 1>;   // 256 tokens x 64 lanes
using FwdTileSmall = TileGeo<2, 8, 8, 64, 1>;     // 128 tokens x 64 lanes
// One lane per thread: any head size, rows aligned to one element, and the
// Chebyshev form of longer series (more than kMonoMaxK coefficients), whose
// coefficients take twice the registers.  Used only where the geometries
// above do not apply.
using FwdTileGeneric = TileGeo<1, 8, 16, 64, 1>;  // 128 tokens x 64 lanes
constexpr int kMaxTileRows = 512;              // bound on TILE (+1 row read past a tile)

// Geometry of a forward launch.
struct FwdShape {
  int tile;    // tokens per tile
  int lanes;   // lanes per lane-block
  int lpt;     // lanes per thread
};
// `generic`: the one-lane geometry (head size not a multiple of 4, rows not
// on 4-element boundaries, or more than 8 coefficients).
FwdShape fwd_geometry(bool dyn, int64_t B, int64_t D, int64_t S, bool generic);

// TTT: keeps the raw x and w = (1-lam)(1-2r) (r = 1/(1+exp(2 damping p)))
// of every token of the run in registers, u = softsign(x) in LDS, plus 2K
// gradient accumulators per lane: one lane per thread (half the
// accumulators of two).  Measured on MI355X at BASELINE configs[4] (bf16),
// with u in LDS: 24-token runs 1001-1008 us against 1047-1056 with 20, 1025
// with 28 and 1092-1095 with 16 (longer runs amortise the per-thread setup,
// chain, composition and reduction over more tokens; at the 128-VGPR bound
// of two workgroups per CU the compiler spills 19 registers at 24 tokens,
// mostly on the rare slow path, and 40 at 28); 2 lanes x 8 or 16 tokens
// +10-20% (an earlier version).
// One look-back word per thread (checkpoints every 8 tiles): the kernel is
// VALU-bound, and every thread runs the polling code of each of its words
// (at 16-token runs 1147 us with two words against 1254 with eight and 1177
// with four; at 20-token runs one word 1069 against 1086 with two).
using TttTile = TileGeo<1, 8, 24, 64, 1>;   // 192 tokens
int ttt_tile_tokens(bool dyn, int x_dtype);

// Backward: one lane per thread (the clamp mask makes the adjoint map's A
// differ per lane); x and dL/dout of the run stay in registers between the
// passes (plus lambda per token with a dynamic lambda), and the look-back
// reads two words (A, B) per predecessor.  Four look-back words per thread
// (checkpoints every 32 tiles) instead of eight brought the static kernel from
// 101 to 77 VGPRs, three workgroups per CU instead of two: 129 against 141 us
// at BASELINE configs[1] on MI355X; two words (checkpoints every 16 tiles)
// 116.9 against 118.2 us with four.  24-token runs (94 VGPRs, two
// workgroups per CU) 113.8-114.4 against 116.5-116.8 us for 16 tokens; 20
// tokens 114.3, 28 tokens 118.2, 32 tokens 114.2; 8-token runs are slower
// (185 us).
using BwdTile = TileGeo<1, 8, 24, 64, 2>;   // 192 tokens
// More than 8 coefficients (Chebyshev form, kpad 16): 12-token runs; more
// than 16 (kpad 32): 4-token runs, room for 3 x 32 coefficient and gradient
// registers.
using BwdTileCheb = TileGeo<1, 8, 12, 64, 2>;   // 96 tokens
using BwdTileCheb32 = TileGeo<1, 8, 4, 64, 2>;  // 32 tokens
int bwd_tile_tokens(bool dyn, int kpad);

// Upper bound on polls of one look-back word (each poll is a device-scope
// load plus a short sleep: about a second in total).  It only guarantees
// that every wave exits if the dispatch-order assumption of the look-back
// ever failed or two calls overlapped on one workspace.  A launch with
// OSM_FLAG_POLL_LIMIT_ZERO (a test aid) polls no word a second time.
constexpr unsigned kSpinLimit = 1u << 20;

// Workspace: a kHeaderBytes header (launch epoch, fault word, completion
// counters), then the look-back words, then (TTT and backward) per-tile
// partials.
constexpr size_t kHeaderBytes = 2048;
// Header bytes kept when a known workspace changes layout (the launch epoch
// and the fault word; the completion counters from this offset on are
// cleared with the look-back words).
constexpr size_t kHeaderKeepBytes = 64;

struct FwdParams {
  const void* x;
  void* out;
  const float* coeffs;
  const float* damping;
  const float* lam;
  const float* g;
  const float* ema_init;
  float* ema_final;
  unsigned long long* slots;   // look-back words [n_lb][n_tiles][LANES][words]
  unsigned* hdr;               // WsHeader
  float* partials;             // TTT per-tile partials (TTT kernels only)
  float* mono_tab;             // TTT: scaled monomial coefficients [n_lb][KP][64], formed once per launch
  const unsigned* mono_form;   // TTT: [n_lb] 1 where mono_tab holds Chebyshev coefficients instead
  int64_t x_sb, x_ss, o_sb, o_ss;
  int64_t c_sb, c_sh, c_sk;
  int64_t g_sb, g_ss, g_sh;
  int B, S, H, hd, K, D;
  uint32_t hd_magic;           // n / hd = (umulhi(n, hd_magic) + n) >> hd_shift for 0 <= n < 2^31
  int hd_shift;
  int n_lbd;                   // lane-blocks per batch row = ceil(D / LANES)
  int n_lb;                    // B * n_lbd
  int n_lb_pad;                // n_lb rounded up to a multiple of 8; grid = n_lb_pad * n_tiles
  int n_tiles;                 // ceil(S / TILE)
  float lam_shift, lam_min, lam_max;
  int clamp_out;
  int nan_zero_u;              // NaN x counts as u = 0 (else z = 0)
  int jitter;                  // OSM_FLAG_TIMING_JITTER: pseudo-random delays (test aid)
  unsigned poll_limit;         // look-back polls before a wait gives up: kSpinLimit, or 0 under
                               // OSM_FLAG_POLL_LIMIT_ZERO (test aid)
  float ttt_scale;             // 2 / (B*(S-1)*D)
  int ttt_target;
};

// Backward launch: the forward's parameters (x, out = the saved forward
// output, coefficients, lambda, shapes, workspace) plus the gradient streams.
struct BwdParams {
  FwdParams f;
  const void* gout;            // dL/dout, dtype of out
  void* gx;                    // dL/dx, dtype of x
  int64_t go_sb, go_ss, gx_sb, gx_ss;
  const float* grad_state;     // dL/d ema_final [B,D] or NULL
  float* grad_init;            // dL/d ema_init [B,D] or NULL
  float* grad_coeffs;          // [B,H,K,hd]
  const void* zs;              // saved z, bf16 [B,S,D], or NULL (recompute)
  int64_t zs_sb, zs_ss;
  int full_jac;                // dL/dx with 1/(1+|x|)^2 everywhere (no 1e-7 cutoff)
};

// Full-path launch (online TTT over chunks with an inline Lion update): one
// workgroup per (batch row, head, group of `lanes` lanes) walks the chunks in
// order.  Needs no workspace.  The chunks of a lane are sequential, so the
// lanes are the only parallelism: 16 lanes per workgroup when that still
// gives >= 512 workgroups, else 8 (v10_lanes).
constexpr int kV10Groups = 64;    // token groups (runs) per 256-token block
constexpr int kV10Run = 4;        // tokens per run
int v10_lanes(int64_t B, int64_t H, int64_t hd);
struct V10Params {
  const void* x;
  float* out;
  const float* coeffs;
  const float* momentum;
  float* coeffs_out;
  float* momentum_out;
  const float* lut;            // [8][256] fp32 (LUT mode)
  const float* lion_lambda;    // [H]
  const float* lr_scale;       // [H]
  const float* spectral_scale; // [K]
  const float* gate;           // [B] or NULL
  const float* dyn_lambda;     // [B] or NULL
  void* z_save;                // bf16 [B,S,D] or NULL
  float* coeff_hist;           // [n_chunks][B,H,K,hd] or NULL
  const float* mu_dev;         // device scalar overriding mu, or NULL
  int64_t x_sb, x_ss, o_sb, o_ss, z_sb, z_ss;
  int64_t c_sb, c_sh, c_sk, m_sb, m_sh, m_sk;
  int B, S, H, hd, K, D, chunk, n_lg;
  int lanes;                   // lanes per workgroup (8 or 16)
  float mu, base_lr, beta1, beta2, wd;
};

// The fixed-coefficient forward (osm_cheby_ema_lut_fwd) on the same kernel:
// one chunk of S tokens, no Lion, x as given, EMA from ema_init, out =
// clamp(s) in fp32, the carried state clamped every clamp_tile tokens, and
// optional x_norm, tanh_y and ema_final outputs.  (A separate struct, so the
// full path's kernel arguments stay as they are.)
struct V10FixedParams : V10Params {
  const float* ema_init;       // [B, D] (row stride init_sb) or NULL (0)
  float* ema_final;            // [B, D] (row stride final_sb) or NULL
  float* xnorm;                // [B,S,D] fp32 or NULL
  float* tanhy;                // [B,S,D] fp32 or NULL
  int64_t init_sb, final_sb, xn_sb, xn_ss, ty_sb, ty_ss;
  int clamp_tile;              // tokens between clamps of the carried state
};

// Multiplier and shift that divide by v (1 <= v < 2^31) for dividends
// 0 <= n < 2^31: s = ceil(log2 v), m = floor(2^32 (2^s - v) / v) + 1
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994, the round-up variant).
inline void div_magic(uint32_t v, uint32_t* magic, int* shift) {
  int s = 0;
  while ((uint64_t(1) << s) < v) ++s;
  *shift = s;
  *magic = (uint32_t)((((uint64_t(1) << s) - v) << 32) / v + 1);
}

// Workspace layout helpers (bytes).
size_t slot_words(bool dyn);
size_t fwd_workspace_bytes(int n_lb, int n_tiles, int lanes, bool dyn);
size_t ttt_workspace_bytes(int n_lb, int n_tiles, bool dyn, int K);
size_t bwd_workspace_bytes(int n_lb, int n_tiles, int K);
size_t bwd_slot_bytes(int n_lb, int n_tiles);

// Launchers: return hipSuccess or the launch error.
hipError_t launch_fwd(const FwdParams& p, int x_dtype, int out_dtype, bool dyn, FwdShape shape, int kpad,
                      hipStream_t stream);
hipError_t launch_ttt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, bool dyn, int tile,
                      int kpad, hipStream_t stream);
hipError_t launch_bwd(const BwdParams& p, int x_dtype, int out_dtype, bool dyn, int tile, int kpad,
                      hipStream_t stream);
hipError_t launch_v10(const V10Params& p, int x_dtype, bool use_lut, int kpad, hipStream_t stream);
hipError_t launch_v10_fixed(const V10FixedParams& p, int x_dtype, bool use_lut, int kpad, hipStream_t stream);
hipError_t launch_fill_zero(void* ptr, size_t bytes, hipStream_t stream);
hipError_t launch_copy_state(const float* src, float* dst, size_t n, hipStream_t stream);
hipError_t launch_ws_status(void* ws, unsigned* dst, int reset, hipStream_t stream);

}  // namespace osm
