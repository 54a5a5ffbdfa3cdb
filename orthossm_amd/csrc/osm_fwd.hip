// Fused Cheby-RKV forward for gfx950: softsign -> Clenshaw -> damping ->
// tanh -> EMA scan, one pass over HBM (x read once, out written once).
//
// Reference counterpart: the forward part of _ortho_megakernel
// (sdpc_kernel.py:2006-2124) and _fused_clenshaw_ema_kernel
// (sdpc_kernel.py:988-1209).  The reference walks S serially inside each of
// B*H*ceil(hd/32) programs; here every (lane-block, 256-token tile) is its own
// workgroup and tiles are chained by the single-pass look-back of osm_chain.h.
//
// Per workgroup (256 threads, tile of 256 tokens x 64 lanes):
//   1. take a tile ticket;
//   2. load x for 16 tokens x 4 lanes per thread and compute
//      w = (1-lam) * tanh(damping * p(u)) in registers;
//   3. serial EMA from 0 over those 16 tokens -> run aggregate (A, B);
//      token-group scan in LDS -> tile aggregate, published;
//   4. look-back -> carry-in;
//   5. replay s = lam*s + w from the carry, store out (and ema_final).
#include "osm_chain.h"

namespace osm {
namespace {

// w = (1 - lam) * tanh(damping * p) for one element, with c pre-scaled by
// 2*log2(e)*damping.  A NaN x gives w = 0 (z = 0), as sdpc_kernel.py:2086.
template <int KP>
__device__ __forceinline__ float ema_input(float x, const float* c, float one_m, float neg2_one_m) {
  const float u = softsign(x);
  const float r = tanh_r(clenshaw<KP>(u, c));
  const float w = __builtin_fmaf(neg2_one_m, r, one_m);
  return (x == x) ? w : 0.0f;
}

template <bool DYN, typename XT, typename OT, int KP>
__global__ void __launch_bounds__(kThreads) cheby_ema_fwd_kernel(const FwdParams p) {
  constexpr int R = kRun;
  constexpr int WORDS = DYN ? 2 : 1;
  __shared__ ChainLds L;

  const ThreadPos q = thread_pos();
  const TileInfo ti = claim_tile(L, p.hdr, p.n_lb, p.n_lbd, p.n_tiles);
  if (!ti.valid) {  // corrupted header: touch nothing, let the launch drain
    finish_block(p.hdr, ti.epoch);
    return;
  }
  const int b = ti.b;
  const int d0 = ti.lbd * kLanes + q.l4 * kLPT;
  const bool lane_ok = d0 < p.D;
  const int h = lane_ok ? d0 / p.hd : 0;
  const int j0 = d0 - h * p.hd;
  const int t0 = ti.tile * kTile + q.tg * R;

  // Coefficients of this thread's 4 lanes, pre-scaled by 2*log2(e)*damping[h]
  // so the damping multiply and the exp -> exp2 conversion cost nothing.
  float c[kLPT][KP];
  {
    const float kap = kTwoLog2e * p.damping[h];
    const float* cb = p.coeffs + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + j0;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
#pragma unroll
      for (int i = 0; i < kLPT; ++i)
        c[i][k] = (lane_ok && k < p.K) ? kap * cb[(int64_t)k * p.c_sk + i] : 0.0f;
    }
  }
  const float lam_h = p.lam[h];

  // Issue every token load of this thread's run up front.
  float w[R][kLPT];
  {
    const XT* xrow = reinterpret_cast<const XT*>(p.x) + (int64_t)b * p.x_sb + d0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = t0 + r;
      if (lane_ok && t < p.S) {
        Lanes4<XT>::load(xrow + (int64_t)t * p.x_ss, w[r]);
      } else {
#pragma unroll
        for (int i = 0; i < kLPT; ++i) w[r][i] = 0.0f;
      }
    }
  }
  float lamv[DYN ? R : 1];
  if constexpr (DYN) {
    const float* gp = p.g + (int64_t)b * p.g_sb + (int64_t)h * p.g_sh;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = t0 + r;
      lamv[r] = (t < p.S) ? __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, gp[(int64_t)t * p.g_ss], lam_h),
                                                    p.lam_min, p.lam_max)
                          : 1.0f;
    }
  }

  // Pass 1: w in registers and the run aggregate (A, B) from a zero state.
  float A = 1.0f;
  float Bv[kLPT] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (t0 + r < p.S) {
      const float lam = DYN ? lamv[r] : lam_h;
      const float one_m = 1.0f - lam;
      const float n2 = -2.0f * one_m;
#pragma unroll
      for (int i = 0; i < kLPT; ++i) {
        w[r][i] = ema_input<KP>(w[r][i], c[i], one_m, n2);
        Bv[i] = __builtin_fmaf(lam, Bv[i], w[r][i]);
      }
      A *= lam;
    } else {
#pragma unroll
      for (int i = 0; i < kLPT; ++i) w[r][i] = 0.0f;
    }
  }

  unsigned long long* lane_slots = p.slots + ((size_t)ti.lb * p.n_tiles * kLanes + q.wl) * WORDS;
  const size_t tile_stride = (size_t)kLanes * WORDS;
  float pA, pB[kLPT], aggA, aggB;
  tile_scan<DYN>(L, q, ti, A, Bv, pA, pB, aggA, aggB, lane_slots, tile_stride);

  const int dl = ti.lbd * kLanes + q.wl;
  const bool dl_ok = dl < p.D;
  const float init_wl = (p.ema_init && dl_ok) ? p.ema_init[(int64_t)b * p.D + dl] : 0.0f;
  const float lam_wl = DYN ? 0.0f : p.lam[dl_ok ? dl / p.hd : 0];
  look_back<DYN, R>(L, q, ti, aggA, aggB, lane_slots, tile_stride, init_wl, lam_wl, p.hdr);

  // Pass 2: replay the recurrence from the true carry and store out.
  float s[kLPT];
#pragma unroll
  for (int i = 0; i < kLPT; ++i) s[i] = __builtin_fmaf(pA, L.carry[q.l4 * kLPT + i], pB[i]);
  OT* orow = reinterpret_cast<OT*>(p.out) + (int64_t)b * p.o_sb + d0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = t0 + r;
    if (t < p.S) {
      const float lam = DYN ? lamv[r] : lam_h;
      float o[kLPT];
#pragma unroll
      for (int i = 0; i < kLPT; ++i) {
        s[i] = __builtin_fmaf(lam, s[i], w[r][i]);
        o[i] = p.clamp_out ? __builtin_amdgcn_fmed3f(s[i], -1.0f, 1.0f) : s[i];
      }
      if (lane_ok) Lanes4<OT>::store(orow + (int64_t)t * p.o_ss, o);
    }
  }
  // Padding tokens leave s unchanged, so the last token group of the last
  // tile holds s[S-1] (the unclamped state).
  if (ti.is_last && q.tg == kNTG - 1 && lane_ok && p.ema_final) {
#pragma unroll
    for (int i = 0; i < kLPT; ++i) p.ema_final[(int64_t)b * p.D + d0 + i] = s[i];
  }
  finish_block(p.hdr, ti.epoch);
}

template <bool DYN, typename XT, typename OT>
hipError_t launch_k(const FwdParams& p, int kpad, hipStream_t stream) {
  const unsigned grid = (unsigned)p.n_lb * (unsigned)p.n_tiles;
  if (kpad == 4)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<DYN, XT, OT, 4>), dim3(grid), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<DYN, XT, OT, 8>), dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <bool DYN>
hipError_t launch_dt(const FwdParams& p, int x_dtype, int out_dtype, int kpad, hipStream_t stream) {
  if (x_dtype == 0 && out_dtype == 0) return launch_k<DYN, float, float>(p, kpad, stream);
  if (x_dtype == 0 && out_dtype == 1) return launch_k<DYN, float, __bf16>(p, kpad, stream);
  if (x_dtype == 1 && out_dtype == 0) return launch_k<DYN, __bf16, float>(p, kpad, stream);
  return launch_k<DYN, __bf16, __bf16>(p, kpad, stream);
}

// Grid-stride zero fill (graph-capturable, unlike hipMemsetAsync nodes).
__global__ void fill_zero_kernel(unsigned* p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

__global__ void copy_state_kernel(const float* src, float* dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace

size_t slot_words(bool dyn) { return dyn ? 2 : 1; }

size_t fwd_workspace_bytes(int n_lb, int n_tiles, bool dyn) {
  return sizeof(WsHeader) + (size_t)n_lb * (size_t)n_tiles * kLanes * slot_words(dyn) * 8;
}

hipError_t launch_fwd(const FwdParams& p, int x_dtype, int out_dtype, bool dyn, int kpad, hipStream_t stream) {
  return dyn ? launch_dt<true>(p, x_dtype, out_dtype, kpad, stream)
             : launch_dt<false>(p, x_dtype, out_dtype, kpad, stream);
}

hipError_t launch_fill_zero(void* ptr, size_t bytes, hipStream_t stream) {
  const size_t words = bytes / 4;
  if (words == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((words + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<unsigned*>(ptr), words);
  return hipGetLastError();
}

hipError_t launch_copy_state(const float* src, float* dst, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(copy_state_kernel, dim3(blocks), dim3(256), 0, stream, src, dst, n);
  return hipGetLastError();
}

}  // namespace osm
