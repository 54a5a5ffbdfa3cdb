// Fused Cheby-RKV forward + TTT coefficient gradient for gfx950.
//
// Loss L = mean_{b, t<S-1, d} (out[t] - y[t+1])^2 (y = x or softsign(x)).
// Its adjoint is a reverse recurrence
//     gL[t] = 2/N (out[t] - y[t+1]) * [-1 <= s[t] <= 1],   t < S-1 (0 at S-1)
//     a[t]  = gL[t] + lam[t+1] a[t+1]
//     dL/dc_k = sum_t a[t] D[t] T_k(u[t]),  D = (1-lam) * damping * (1 - z^2)
// (reference chain: _parallel_reverse_ema_kernel, sdpc_kernel.py:681-777;
// _parallel_backward_clenshaw_kernel_v10, sdpc_kernel.py:784-915; the
// per-tile partial sum, sdpc_kernel.py:2502).
//
// One pass over HBM: each tile runs the forward of osm_fwd.hip (x read once,
// out written once), then sweeps its tokens backwards.  a[t] inside a tile is
// a[t] = at[t] + Lam[t] * rho, where at is the tile-local reverse scan from
// zero, Lam[t] the decay product to the tile end and rho the (unknown)
// reverse carry from later tiles.  The tile therefore emits
//     P_k = sum_t at[t] D[t] T_k(u[t]),   Q_k = sum_t Lam[t] D[t] T_k(u[t])
// and its reverse map rho_prev = Ar * rho + Br.  Two small kernels merge the
// tiles of each lane from the end of the sequence (rho = 0 there) in a fixed
// order: G_k = sum_tiles (P_k + rho_tile Q_k), scaled by 1/(k+1)^2.
#include "osm_chain.h"

namespace osm {
namespace {

using G = TttGeo;
constexpr int kChunk = 16;  // tiles merged per thread by the first merge kernel

template <int KP>
__host__ __device__ constexpr int n_fields() {
  return 2 * KP + 2;  // P_0..P_{KP-1}, Q_0..Q_{KP-1}, Ar, Br
}

// Sum over the token groups of a wave (lanes wl, wl^TPR, ...).
__device__ __forceinline__ float wave_sum_tg(float v) {
#pragma unroll
  for (int m = G::TPR; m < 64; m *= 2) v += __shfl_xor(v, m);
  return v;
}

template <bool DYN, typename XT, typename OT, int KP>
__global__ void __launch_bounds__(G::THREADS) cheby_ema_ttt_kernel(const FwdParams p) {
  constexpr int R = G::R;
  constexpr int LPT = G::LPT;
  constexpr int NTG = G::NTG;
  constexpr int WORDS = DYN ? 2 : 1;
  constexpr int F = n_fields<KP>();
  __shared__ ChainLds<G> L;
  __shared__ float sh_y0[NTG][kLanes];      // target y at each token group's first token
  __shared__ float sh_rA[NTG][G::TPR];      // reverse map of each run
  __shared__ float sh_rB[NTG][kLanes];
  __shared__ float sh_red[G::WAVES][2 * KP][kLanes];

  const ThreadPos q = thread_pos<G>();
  const Tags tags = launch_tags(p.hdr);
  const TileInfo ti = tile_info(blockIdx.x, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles);
  if (ti.pad) {
    finish_block(p.hdr, tags.epoch);
    return;
  }
  const int b = ti.b;
  const int d0 = ti.lbd * kLanes + q.lt * LPT;
  const bool lane_ok = d0 < p.D;
  const int h = lane_ok ? d0 / p.hd : 0;
  const int j0 = d0 - h * p.hd;
  const int t0 = ti.tile * G::TILE + q.tg * R;
  const bool soft_target = p.ttt_target == 1;

  const float delta = p.damping[h];
  float c[LPT][KP];
  {
    const float kap = kTwoLog2e * delta;
    const float* cb = p.coeffs + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + j0;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
#pragma unroll
      for (int i = 0; i < LPT; ++i)
        c[i][k] = (lane_ok && k < p.K) ? kap * cb[(int64_t)k * p.c_sk + i] : 0.0f;
    }
  }
  const float lam_h = p.lam[h];

  const XT* xrow = reinterpret_cast<const XT*>(p.x) + (int64_t)b * p.x_sb + d0;
  float xv[R][LPT];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = t0 + r;
    if (lane_ok && t < p.S) {
      LaneVec<XT, LPT>::load(xrow + (int64_t)t * p.x_ss, xv[r]);
    } else {
#pragma unroll
      for (int i = 0; i < LPT; ++i) xv[r][i] = 0.0f;
    }
  }
  // Target of the token after the run: the next token group's first token
  // (through LDS) or, for the last group, the next tile's first row.
  float y_after[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) y_after[i] = 0.0f;
  if (q.tg == NTG - 1 && lane_ok && t0 + R < p.S) LaneVec<XT, LPT>::load(xrow + (int64_t)(t0 + R) * p.x_ss, y_after);

  float lamv[R];
  {
    const float* gp = DYN ? p.g + (int64_t)b * p.g_sb + (int64_t)h * p.g_sh : nullptr;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = t0 + r;
      if (t < p.S) {
        lamv[r] = DYN ? __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, gp[(int64_t)t * p.g_ss], lam_h),
                                                p.lam_min, p.lam_max)
                      : lam_h;
      } else {
        lamv[r] = 1.0f;
      }
    }
  }

  // Pass 1: r = 1/(1+exp(2 damping p)) per element and the run aggregate.
  float rr[R][LPT];
  float A = 1.0f;
  float Bv[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) Bv[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float lam = lamv[r];
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float x = xv[r][i];
      rr[r][i] = tanh_r(clenshaw<KP>(softsign(x), c[i]));
      const float w = (x == x) ? __builtin_fmaf(n2, rr[r][i], one_m) : 0.0f;
      Bv[i] = __builtin_fmaf(lam, Bv[i], (t0 + r < p.S) ? w : 0.0f);
    }
    A *= lam;
  }

  // Targets at the first token of each run, for the neighbouring run.
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const float x = xv[0][i];
    sh_y0[q.tg][q.lt * LPT + i] = (soft_target && x == x) ? softsign(x) : x;
  }

  unsigned long long* lane_slots = p.slots + ((size_t)ti.lb * p.n_tiles * kLanes + q.wl) * WORDS;
  const size_t tile_stride = (size_t)kLanes * WORDS;
  float pA, pB[LPT], aggA, aggB;
  tile_scan<G, DYN>(L, q, ti, tags, A, Bv, pA, pB, aggA, aggB, lane_slots, tile_stride);  // syncs sh_y0 too

  const int dl = ti.lbd * kLanes + q.wl;
  const bool dl_ok = dl < p.D;
  const float init_wl = (p.ema_init && dl_ok) ? p.ema_init[(int64_t)b * p.D + dl] : 0.0f;
  const float lam_wl = DYN ? 0.0f : p.lam[dl_ok ? dl / p.hd : 0];
  {
    LookBack<G, DYN> lbk;
    look_back_issue<G, DYN>(lbk, q, ti, lane_slots, tile_stride);
    look_back_finish<G, DYN>(lbk, L, q, ti, tags, aggA, aggB, lane_slots, tile_stride, init_wl, lam_wl, p.hdr);
  }

  if (q.tg < NTG - 1) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) y_after[i] = sh_y0[q.tg + 1][q.lt * LPT + i];
  } else if (soft_target) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) y_after[i] = (y_after[i] == y_after[i]) ? softsign(y_after[i]) : y_after[i];
  }

  // Pass 2 (forward): s from the carry, out, and the loss gradient gL.
  float gl[R][LPT];
  {
    float s[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) s[i] = __builtin_fmaf(pA, L.carry[q.lt * LPT + i], pB[i]);
    OT* orow = reinterpret_cast<OT*>(p.out) + (int64_t)b * p.o_sb + d0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = t0 + r;
      const float lam = lamv[r];
      const float one_m = 1.0f - lam;
      const float n2 = -2.0f * one_m;
      float o[LPT];
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const float x = xv[r][i];
        const float w = (x == x && t < p.S) ? __builtin_fmaf(n2, rr[r][i], one_m) : 0.0f;
        s[i] = __builtin_fmaf(lam, s[i], w);
        o[i] = p.clamp_out ? __builtin_amdgcn_fmed3f(s[i], -1.0f, 1.0f) : s[i];
        float y;
        if (r + 1 < R) {
          const float xn = xv[r + 1][i];
          y = (soft_target && xn == xn) ? softsign(xn) : xn;
        } else {
          y = y_after[i];
        }
        const bool pass = !p.clamp_out || (s[i] >= -1.0f && s[i] <= 1.0f);
        gl[r][i] = (t < p.S - 1 && pass) ? p.ttt_scale * (o[i] - y) : 0.0f;
      }
      if (lane_ok && t < p.S) LaneVec<OT, LPT>::store(orow + (int64_t)t * p.o_ss, o);
    }
    if (ti.is_last && q.tg == NTG - 1 && lane_ok && p.ema_final) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) p.ema_final[(int64_t)b * p.D + d0 + i] = s[i];
    }
  }

  // Reverse sweep over the run: at (local adjoint), Lam (decay to run end).
  float P[KP][LPT], Q[KP][LPT];
#pragma unroll
  for (int k = 0; k < KP; ++k)
#pragma unroll
    for (int i = 0; i < LPT; ++i) P[k][i] = Q[k][i] = 0.0f;
  float at[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) at[i] = 0.0f;
  float Lam = 1.0f, lam_next = 1.0f;
  const float dsc = 4.0f * delta;  // 1 - z^2 = 4 r (1 - r)
#pragma unroll
  for (int r = R - 1; r >= 0; --r) {
    const int t = t0 + r;
    const float lam = lamv[r];
    Lam *= lam_next;
    const float dl_scale = (t < p.S) ? (1.0f - lam) * dsc : 0.0f;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float x = xv[r][i];
      const bool ok = x == x;
      at[i] = __builtin_fmaf(lam_next, at[i], gl[r][i]);
      const float rv = rr[r][i];
      const float D = ok ? dl_scale * rv * (1.0f - rv) : 0.0f;
      const float u = ok ? softsign(x) : 0.0f;
      const float vp = at[i] * D;
      const float vq = Lam * D;
      const float u2 = u + u;
      float Tm2 = 1.0f, Tm1 = u;
      P[0][i] += vp;
      Q[0][i] += vq;
      if (KP > 1) {
        P[1][i] = __builtin_fmaf(vp, u, P[1][i]);
        Q[1][i] = __builtin_fmaf(vq, u, Q[1][i]);
      }
#pragma unroll
      for (int k = 2; k < KP; ++k) {
        const float Tk = __builtin_fmaf(u2, Tm1, -Tm2);
        P[k][i] = __builtin_fmaf(vp, Tk, P[k][i]);
        Q[k][i] = __builtin_fmaf(vq, Tk, Q[k][i]);
        Tm2 = Tm1;
        Tm1 = Tk;
      }
    }
    lam_next = lam;
  }
  // Run reverse map: rho_prev = lam[t0] * (at[t0] + Lam[t0] * rho_run).
  const float rA = lam_next * Lam;
  float rB[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) rB[i] = lam_next * at[i];
  sh_rA[q.tg][q.lt] = rA;
#pragma unroll
  for (int i = 0; i < LPT; ++i) sh_rB[q.tg][q.lt * LPT + i] = rB[i];
  __syncthreads();

  // rho_run(tg) = alpha + beta * rho_tile, from the later runs in fixed order.
  float alpha[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) alpha[i] = 0.0f;
  float beta = 1.0f;
  for (int g = NTG - 1; g > q.tg; --g) {
    const float a = sh_rA[g][q.lt];
#pragma unroll
    for (int i = 0; i < LPT; ++i) alpha[i] = __builtin_fmaf(a, alpha[i], sh_rB[g][q.lt * LPT + i]);
    beta *= a;
  }
  float* part = p.partials + ((size_t)ti.lb * p.n_tiles + ti.tile) * F * kLanes;
  if (q.tg == 0) {
    // Tile reverse map: rho_prev_tile = rA*(alpha + beta*rho_tile) + rB.
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      part[(size_t)(2 * KP) * kLanes + q.lt * LPT + i] = rA * beta;
      part[(size_t)(2 * KP + 1) * kLanes + q.lt * LPT + i] = __builtin_fmaf(rA, alpha[i], rB[i]);
    }
  }
  // Tile partials: P' = sum_runs (P + alpha Q), Q' = sum_runs beta Q.
#pragma unroll
  for (int k = 0; k < KP; ++k) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float pv = wave_sum_tg(__builtin_fmaf(alpha[i], Q[k][i], P[k][i]));
      const float qv = wave_sum_tg(beta * Q[k][i]);
      if (q.wl < G::TPR) {
        sh_red[q.wave][k][q.lt * LPT + i] = pv;
        sh_red[q.wave][KP + k][q.lt * LPT + i] = qv;
      }
    }
  }
  __syncthreads();
  for (int v = q.wave; v < 2 * KP; v += G::WAVES) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < G::WAVES; ++w) acc += sh_red[w][v][q.wl];
    part[(size_t)v * kLanes + q.wl] = acc;
  }
  finish_block(p.hdr, tags.epoch);
}

// Merge formula, earlier tile/chunk e followed by combined later part c:
//   P = P_c + P_e + Br_c Q_e,  Q = Q_c + Ar_c Q_e,  Ar = Ar_e Ar_c,  Br = Ar_e Br_c + Br_e.
template <int KP>
__device__ __forceinline__ void merge_into(float (&acc)[2 * KP + 2], const float* rec, int stride) {
  const float Ar_c = acc[2 * KP], Br_c = acc[2 * KP + 1];
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const float Pe = rec[(size_t)k * stride];
    const float Qe = rec[(size_t)(KP + k) * stride];
    acc[k] = acc[k] + __builtin_fmaf(Br_c, Qe, Pe);
    acc[KP + k] = __builtin_fmaf(Ar_c, Qe, acc[KP + k]);
  }
  const float Ar_e = rec[(size_t)(2 * KP) * stride];
  const float Br_e = rec[(size_t)(2 * KP + 1) * stride];
  acc[2 * KP] = Ar_e * Ar_c;
  acc[2 * KP + 1] = __builtin_fmaf(Ar_e, Br_c, Br_e);
}

// Level 1: each thread merges up to kChunk consecutive tiles of one lane.
template <int KP>
__global__ void __launch_bounds__(64) ttt_merge_chunks(const float* partials, float* chunks, int n_tiles,
                                                       int n_chunks) {
  constexpr int F = n_fields<KP>();
  const int chunk = blockIdx.x, lb = blockIdx.y, l = threadIdx.x;
  float acc[F];
#pragma unroll
  for (int v = 0; v < F; ++v) acc[v] = 0.0f;
  acc[2 * KP] = 1.0f;  // identity map
  const int first = chunk * kChunk;
  const int last = min(first + kChunk, n_tiles) - 1;
  for (int t = last; t >= first; --t)
    merge_into<KP>(acc, partials + ((size_t)lb * n_tiles + t) * F * kLanes + l, kLanes);
  float* dst = chunks + ((size_t)lb * n_chunks + chunk) * F * kLanes + l;
#pragma unroll
  for (int v = 0; v < F; ++v) dst[(size_t)v * kLanes] = acc[v];
}

// Level 2: merge the chunks of each lane from the sequence end (rho = 0) and
// write grad[b,h,k,j] = G_k / (k+1)^2.
template <int KP>
__global__ void __launch_bounds__(64) ttt_finalize(const float* chunks, float* grad, int n_chunks, int n_lbd, int D,
                                                   int hd, int H, int K) {
  constexpr int F = n_fields<KP>();
  const int lb = blockIdx.x, l = threadIdx.x;
  float acc[F];
#pragma unroll
  for (int v = 0; v < F; ++v) acc[v] = 0.0f;
  acc[2 * KP] = 1.0f;
  for (int c = n_chunks - 1; c >= 0; --c)
    merge_into<KP>(acc, chunks + ((size_t)lb * n_chunks + c) * F * kLanes + l, kLanes);
  const int b = lb / n_lbd;
  const int d = (lb - b * n_lbd) * kLanes + l;
  if (d >= D) return;
  const int h = d / hd, j = d - h * hd;
  float* gdst = grad + (((size_t)b * H + h) * K) * hd + j;
#pragma unroll
  for (int k = 0; k < KP; ++k)
    if (k < K) gdst[(size_t)k * hd] = acc[k] / (float)((k + 1) * (k + 1));
}

template <bool DYN, typename XT, typename OT, int KP>
hipError_t launch_all(const FwdParams& p, float* grad, hipStream_t stream) {
  const unsigned grid = (unsigned)p.n_lb_pad * (unsigned)p.n_tiles;
  hipLaunchKernelGGL((cheby_ema_ttt_kernel<DYN, XT, OT, KP>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int n_chunks = (p.n_tiles + kChunk - 1) / kChunk;
  float* chunks = p.partials + (size_t)p.n_lb * p.n_tiles * n_fields<KP>() * kLanes;
  hipLaunchKernelGGL((ttt_merge_chunks<KP>), dim3(n_chunks, p.n_lb), dim3(64), 0, stream, p.partials, chunks,
                     p.n_tiles, n_chunks);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ttt_finalize<KP>), dim3(p.n_lb), dim3(64), 0, stream, chunks, grad, n_chunks, p.n_lbd, p.D,
                     p.hd, p.H, p.K);
  return hipGetLastError();
}

template <bool DYN, typename XT, typename OT>
hipError_t launch_k(const FwdParams& p, float* grad, int kpad, hipStream_t stream) {
  return kpad == 4 ? launch_all<DYN, XT, OT, 4>(p, grad, stream) : launch_all<DYN, XT, OT, 8>(p, grad, stream);
}

template <bool DYN>
hipError_t launch_dt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, int kpad, hipStream_t stream) {
  if (x_dtype == 0 && out_dtype == 0) return launch_k<DYN, float, float>(p, grad, kpad, stream);
  if (x_dtype == 0 && out_dtype == 1) return launch_k<DYN, float, __bf16>(p, grad, kpad, stream);
  if (x_dtype == 1 && out_dtype == 0) return launch_k<DYN, __bf16, float>(p, grad, kpad, stream);
  return launch_k<DYN, __bf16, __bf16>(p, grad, kpad, stream);
}

}  // namespace

size_t ttt_workspace_bytes(int n_lb, int n_tiles, bool dyn, int K) {
  const int kpad = K <= 4 ? 4 : 8;
  const size_t F = 2 * kpad + 2;
  const size_t n_chunks = (n_tiles + kChunk - 1) / kChunk;
  const size_t slots = (fwd_workspace_bytes(n_lb, n_tiles, dyn) + 255) / 256 * 256;
  return slots + ((size_t)n_lb * n_tiles + (size_t)n_lb * n_chunks) * F * kLanes * sizeof(float);
}

hipError_t launch_ttt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, bool dyn, int kpad,
                      hipStream_t stream) {
  return dyn ? launch_dt<true>(p, grad, x_dtype, out_dtype, kpad, stream)
             : launch_dt<false>(p, grad, x_dtype, out_dtype, kpad, stream);
}

}  // namespace osm
