// Launch parameters and launcher declarations shared by the kernel files and
// the C-ABI layer.  Host-visible only; no torch types.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace osm {

// Tile geometry of the fused kernels: 4 waves of 64 threads, 16 token groups
// of R tokens each, 64 lanes per lane-block.  The forward uses R = kRun
// (kTile = 256 tokens); the TTT kernel keeps more per-token state in
// registers and uses R = kRunTTT (kTileTTT = 128 tokens).
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRun = 16;
constexpr int kTile = kWaves * 4 * kRun;        // 256 tokens
constexpr int kRunTTT = 8;
constexpr int kTileTTT = kWaves * 4 * kRunTTT;  // 128 tokens

struct FwdParams {
  const void* x;
  void* out;
  const float* coeffs;
  const float* damping;
  const float* lam;
  const float* g;
  const float* ema_init;
  float* ema_final;
  unsigned long long* slots;   // look-back words [n_lb][n_tiles][64][words]
  unsigned* hdr;               // WsHeader
  float* partials;             // TTT per-tile partials (TTT kernels only)
  int64_t x_sb, x_ss, o_sb, o_ss;
  int64_t c_sb, c_sh, c_sk;
  int64_t g_sb, g_ss, g_sh;
  int B, S, H, hd, K, D;
  int n_lbd;                   // lane-blocks per batch row = ceil(D / 64)
  int n_lb;                    // B * n_lbd
  int n_tiles;                 // ceil(S / kTile)
  float lam_shift, lam_min, lam_max;
  int clamp_out;
  float ttt_scale;             // 2 / (B*(S-1)*D)
  int ttt_target;
};

// Workspace layout helpers (bytes).
size_t slot_words(bool dyn);
size_t fwd_workspace_bytes(int n_lb, int n_tiles, bool dyn);
size_t ttt_workspace_bytes(int n_lb, int n_tiles, bool dyn, int K);

// Launchers: return hipSuccess or the launch error.
hipError_t launch_fwd(const FwdParams& p, int x_dtype, int out_dtype, bool dyn, int kpad,
                      hipStream_t stream);
hipError_t launch_ttt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, bool dyn,
                      int kpad, hipStream_t stream);
hipError_t launch_fill_zero(void* ptr, size_t bytes, hipStream_t stream);
hipError_t launch_copy_state(const float* src, float* dst, size_t n, hipStream_t stream);

}  // namespace osm
