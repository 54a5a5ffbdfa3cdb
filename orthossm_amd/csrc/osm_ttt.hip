// Fused Cheby-RKV forward + TTT coefficient gradient for gfx950.
//
// Loss L = mean_{b, t<S-1, d} (out[t] - y[t+1])^2 (y = x or softsign(x)).
// With e[t] = out[t] - y[t+1] (0 at t = S-1, and where the output clamp
// binds) the adjoint of the state is the reverse recurrence
//     a[t] = (2/N) e[t] + lam[t+1] a[t+1]
// and dL/dc_k = sum_t a[t] D[t] T_k(u[t]),  D = (1-lam) damping (1 - z^2)
// (reference chain: _parallel_reverse_ema_kernel, sdpc_kernel.py:681-777;
// _parallel_backward_clenshaw_kernel_v10, sdpc_kernel.py:784-915; the
// per-tile partial sum, sdpc_kernel.py:2502).
//
// One pass over HBM: each tile runs the forward of osm_fwd.hip (x read once,
// out written once) and accumulates the gradient in the same forward sweep.
// Swapping the order of summation turns the reverse adjoint into forward
// accumulators: for a run of tokens t0..T, followed by the adjoint rho =
// a[T+1] from later tokens,
//     sum_t a[t] v[t] = sum_t e[t] F[t] + lam[T+1] F[T] rho,
//     F[t] = lam[t] F[t-1] + v[t]            (F[t0-1] = 0),
// with v = D T_k(u) for each k.  So a run yields P_k = sum_t e[t] F_k[t], the
// end values F_k[T], and its adjoint map a[t0] = alpha + beta rho.  Runs are
// composed in LDS into the tile's (P, Q) and map; two small kernels merge the
// tiles of each lane from the end of the sequence (rho = 0) in a fixed order:
// G_k = sum_tiles (P_k + Q_k rho_tile), scaled by 1/(k+1)^2.
#include "osm_tile.h"

namespace osm {
namespace {

constexpr int kChunk = 16;  // tiles merged per thread by the first merge kernel

template <int KP>
__host__ __device__ constexpr int n_fields() {
  return 2 * KP + 2;  // P_0..P_{KP-1}, Q_0..Q_{KP-1}, Ar (beta), Br (alpha)
}

// Raw x of a thread's run (R tokens x LPT lanes), kept between the passes
// (pass 2 needs x as the target y and for the NaN checks of its slow path).
// Pass 1 reads row r with first(r, i), then calls seal(r): from then on the
// row is read with get(r, i).  seal() hides the value from the compiler, so
// it keeps the raw x instead of pass 1's unpacked values alive across the
// look-back; for bf16 with one lane per thread it also packs two tokens per
// register.
template <typename XT, int R, int LPT>
struct XRun;

template <int R, int LPT>
struct XRun<float, R, LPT> {
  float v[R][LPT];
  __device__ __forceinline__ void load_all(const TileAddr& a) {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      BufVec<float, LPT>::load(a.x, a.vx, so, v[r]);
      so = next_off(so, a.sx);
    }
  }
  __device__ __forceinline__ float first(int r, int i) const { return v[r][i]; }
  __device__ __forceinline__ void seal(int r) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) asm volatile("" : "+v"(v[r][i]));
  }
  __device__ __forceinline__ float get(int r, int i) const { return v[r][i]; }
};

template <int R>
struct XRun<__bf16, R, 2> {
  unsigned v[R];   // both lanes of a row
  __device__ __forceinline__ void load_all(const TileAddr& a) {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v[r] = __builtin_amdgcn_raw_buffer_load_b32(a.x, a.vx, so, kNT);
      so = next_off(so, a.sx);
    }
  }
  __device__ __forceinline__ float get(int r, int i) const {
    return __uint_as_float(i == 0 ? v[r] << 16 : v[r] & 0xffff0000u);
  }
  __device__ __forceinline__ float first(int r, int i) const { return get(r, i); }
  __device__ __forceinline__ void seal(int r) { asm volatile("" : "+v"(v[r])); }
};

template <int R>
struct XRun<__bf16, R, 1> {
  static_assert(R % 2 == 0, "token pairs");
  unsigned raw[R];     // as loaded (low 16 bits)
  unsigned v[R / 2];   // rows 2m, 2m+1 packed, once sealed
  __device__ __forceinline__ void load_all(const TileAddr& a) {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      raw[r] = __builtin_amdgcn_raw_buffer_load_b16(a.x, a.vx, so, kNT);
      so = next_off(so, a.sx);
    }
  }
  __device__ __forceinline__ float first(int r, int) const { return __uint_as_float(raw[r] << 16); }
  __device__ __forceinline__ void seal(int r) {
    if (r & 1) {
      v[r / 2] = raw[r - 1] | (raw[r] << 16);
      asm volatile("" : "+v"(v[r / 2]));
    }
  }
  __device__ __forceinline__ float get(int r, int) const {
    return __uint_as_float((r & 1) ? v[r / 2] & 0xffff0000u : v[r / 2] << 16);
  }
};

// Target y of one x value.
template <bool SOFT>
__device__ __forceinline__ float target_of(float x) {
  if constexpr (SOFT) return (x == x) ? softsign(x) : x;
  return x;
}

// Gradient state of one thread's run.
template <int KP, int LPT>
struct RunGrad {
  float F[KP][LPT];   // forward-discounted basis sums
  float P[KP][LPT];   // sum_t e[t] F[t]
  float al[LPT];      // adjoint at the run start from this run's e (unscaled)
  float Lp;           // prod of lam over (t0, t]
};

// Pass 2 over a thread's run, in token order: the EMA from the carried state
// s, out = clamp(s), e[t] = out[t] - y[t+1], and the gradient accumulators.
// SLOW handles, per element, NaN inputs (u = 0; D = 0 unless nan_zero_u), a binding clamp
// (e = 0 where |s| > 1), the sequence end (e = 0 for t >= S-1) and the
// ema_final capture; the fast variant assumes none of them occurs in the run.
template <class G, bool DYN, bool SOFT, bool SLOW, typename XT, typename OT, int KP>
__device__ __forceinline__ void ttt_pass2(RunGrad<KP, G::LPT>& rg, float (&s)[G::LPT], const XRun<XT, G::R, G::LPT>& xr,
                                          const float* ul, const float (&rr)[G::R][G::LPT],
                                          const float (&lamv)[G::R], float om2, const float (&y_after)[G::LPT],
                                          const TileAddr& a, float lo, float hi, int t_first, int S, bool clamp,
                                          bool nan_zero_u, float* fin) {
  constexpr int R = G::R, LPT = G::LPT;
#pragma unroll
  for (int k = 0; k < KP; ++k)
#pragma unroll
    for (int i = 0; i < LPT; ++i) rg.F[k][i] = rg.P[k][i] = 0.0f;
#pragma unroll
  for (int i = 0; i < LPT; ++i) rg.al[i] = 0.0f;
  rg.Lp = 1.0f;
  f32x4 ug[LPT];   // u of tokens 4m .. 4m+3 of each lane
  // Under a static lambda the products Lp are lambda^r, which the compiler
  // would otherwise share with pass 1's run aggregate and keep in registers
  // across the look-back; a hidden copy of lambda keeps them here.
  float lam_lp = lamv[0];
  if constexpr (!DYN) asm volatile("" : "+v"(lam_lp));
  uint32_t so = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float lam = lamv[r];
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
    if (r > 0) rg.Lp *= DYN ? lam : lam_lp;
    if (r % 4 == 0) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) ug[i] = *reinterpret_cast<const f32x4*>(ul + i * R + r);
    }
    float yn[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      if (r + 1 < R) {
        // softsign target: u of the next token (NaN where x is NaN, as x)
        if constexpr (SOFT) yn[i] = r % 4 != 3 ? ug[i][(r + 1) % 4] : ul[i * R + r + 1];
        else yn[i] = xr.get(r + 1, i);
      } else {
        yn[i] = y_after[i];
      }
    }
    float o[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float rv = rr[r][i];
      float D;
      if constexpr (DYN) {
        s[i] = __builtin_fmaf(lam, s[i], __builtin_fmaf(n2, rv, one_m));
        D = __builtin_fmaf(-rv, rv, rv) * one_m;   // (1 - lam) r (1 - r) = (1 - lam)(1 - z^2) / 4
      } else {
        // rv is w = (1 - lam) z: s = lam s + w, D = (1 - lam)^2 - w^2 = (1 - lam)^2 (1 - z^2)
        s[i] = __builtin_fmaf(lam, s[i], rv);
        D = __builtin_fmaf(-rv, rv, om2);
      }
      // On the fast path |s| <= 1 over the run (or the clamp is off), so the
      // clamp is the identity there.
      o[i] = SLOW ? __builtin_amdgcn_fmed3f(s[i], lo, hi) : s[i];
      float e = o[i] - yn[i];
      float uu = ug[i][r % 4];
      if constexpr (SLOW) {
        const int t = t_first + r;
        const bool pass = !clamp || __builtin_fabsf(s[i]) <= 1.0f;
        e = (t < S - 1 && pass) ? e : 0.0f;
        const bool ok = xr.get(r, i) == xr.get(r, i);
        D = (ok || nan_zero_u) ? D : 0.0f;
        uu = ok ? uu : 0.0f;
        if (fin && t == S - 1) fin[i] = s[i];
      }
      rg.al[i] = __builtin_fmaf(rg.Lp, e, rg.al[i]);
      // v_k = D T_k(u) by the Chebyshev recurrence on the scaled values.
      float vm2 = D, vm1 = D * uu;
      const float u2 = uu + uu;
      rg.F[0][i] = __builtin_fmaf(lam, rg.F[0][i], vm2);
      rg.P[0][i] = __builtin_fmaf(e, rg.F[0][i], rg.P[0][i]);
      if (KP > 1) {
        rg.F[1][i] = __builtin_fmaf(lam, rg.F[1][i], vm1);
        rg.P[1][i] = __builtin_fmaf(e, rg.F[1][i], rg.P[1][i]);
      }
#pragma unroll
      for (int k = 2; k < KP; ++k) {
        const float vk = __builtin_fmaf(u2, vm1, -vm2);
        rg.F[k][i] = __builtin_fmaf(lam, rg.F[k][i], vk);
        rg.P[k][i] = __builtin_fmaf(e, rg.F[k][i], rg.P[k][i]);
        vm2 = vm1;
        vm1 = vk;
      }
    }
    BufVec<OT, LPT>::store(a.out, a.vo, so, o);
    so = next_off(so, a.so);

  }
}

// Per-lane scale of the gradient sums: 2/N and the constant part of the
// derivative (1-lam) damping (1-z^2): 4 damping times D = (1-lam) r (1-r)
// (dynamic lambda), damping / (1-lam) times D = (1-lam)^2 (1-z^2) (static; 0
// at lam = 1, where D is 0).
template <bool DYN>
__device__ __forceinline__ float ttt_lane_scale(const FwdParams& p, int h) {
  if constexpr (DYN) return p.ttt_scale * 4.0f * p.damping[h];
  const float lam = p.lam[h];
  // (a reciprocal, not a division: within an ulp, and the division's
  // expansion measured 0.8% of the kernel)
  return lam != 1.0f ? p.ttt_scale * p.damping[h] * __builtin_amdgcn_rcpf(1.0f - lam) : 0.0f;
}

// Sum over the token groups of a wave (lanes wl, wl ^ TPR, ...).
template <class G>
__device__ __forceinline__ float wave_sum_tg(float v) {
#pragma unroll
  for (int m = G::TPR; m < 64; m *= 2) v += __shfl_xor(v, m);
  return v;
}

// Two workgroups (4 waves per SIMD) per CU: at most 128 VGPRs.
template <class G, bool DYN, bool SOFT, typename XT, typename OT, int KP>
__global__ void __launch_bounds__(G::THREADS) __attribute__((amdgpu_waves_per_eu(4)))
cheby_ema_ttt_kernel(const FwdParams p) {
  constexpr int R = G::R;
  constexpr int LPT = G::LPT;
  constexpr int NTG = G::NTG;
  constexpr int F = n_fields<KP>();
  static_assert(G::LANES == kLanes, "partials and merges assume 64-lane lane-blocks");
  static_assert(R % 4 == 0, "u moves through LDS four tokens at a time");
  __shared__ ChainLds<G> L;
  __shared__ float mono[KP][kLanes];
  __shared__ float sh_y0[NTG][kLanes];      // target y at each run's first token
  __shared__ float sh_lam0[NTG][G::TPR];    // lambda at each run's first token
  __shared__ float sh_al[NTG][kLanes];      // run adjoint maps a[t0] = alpha + beta rho
  __shared__ float sh_be[NTG][G::TPR];
  __shared__ float sh_pw[2][kLanes];        // static lambda: run and tile decay of each lane
  // u of every element of the tile (pass 1 -> pass 2 of the same wave), then
  // the per-wave gradient sums (after the barrier that follows pass 2).
  // (16-byte aligned: pass 1 and pass 2 move u as f32x4)
  __shared__ union __attribute__((aligned(16))) {
    float u[NTG][G::LANES][R];   // [token group][lane][token of the run]
    float red[G::WAVES][2 * KP][kLanes];
  } sh_ur;

  const ThreadPos q = thread_pos<G>();
  const Tags tags = launch_tags(p.hdr);
  const TileInfo ti = tile_info<G>(blockIdx.x, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles);
  if (ti.pad) {
    finish_block(p.hdr, tags.epoch);
    return;
  }
  const TileAddr a = tile_addr<G, DYN, XT, OT>(p, q, ti);
  // This wave's monomial coefficient (wave w holds coefficient w of the 64
  // lanes), formed once per launch by ttt_mono_prep; loaded before x.
  static_assert(G::NSUB == 1 && KP <= G::WAVES, "one coefficient per wave");
  const float mono_w = q.wave < KP ? p.mono_tab[((size_t)ti.lb * KP + q.wave) * kLanes + q.wl] : 0.0f;
  // the form of the table (1: Chebyshev coefficients, see ttt_mono_prep)
  const bool cheb = __builtin_amdgcn_readfirstlane(p.mono_form[ti.lb]) != 0;

  // x rows of the run (raw), g (dynamic lambda), and for the tile's last run
  // the row after the tile (its target y and lambda).
  XRun<XT, R, LPT> xr;
  xr.load_all(a);
  const float lam_h = p.lam[a.h];
  float lamv[R];
  if constexpr (DYN) {
    uint32_t sg = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      lamv[r] = load_f32_shared(a.g, a.vg, sg);   // a line of g serves every lane-block of the row
      sg = next_off(sg, a.sg);
    }
  }
  const bool last_run = q.tg == NTG - 1;
  float x_after[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) x_after[i] = 0.0f;
  float g_after = 0.0f;
  if (last_run) {
    BufVec<XT, LPT>::load(a.x, a.vx, (uint32_t)R * a.sx, x_after);
    if constexpr (DYN) {
      g_after = load_f32_shared(a.g, a.vg, (uint32_t)R * a.sg);
    }
  }

  if (q.wave < KP) mono[q.wave][q.wl] = mono_w;
  if constexpr (!DYN) {
    // lambda^R and lambda^TILE of each lane, by the last two waves
    if (q.wave >= G::WAVES - 2) {
      const int d = ti.lbd * kLanes + q.wl;
      const float lam = p.lam[d < p.D ? div_hd(d, p) : 0];
      sh_pw[q.wave - (G::WAVES - 2)][q.wl] = q.wave == G::WAVES - 2 ? pow_n<R>(lam) : static_tile_A<G>(lam);
    }
  }
  __syncthreads();
  float c[LPT][KP];
  mono_read<G, KP>(mono, q, c);

  // Pass 1: r = 1/(1+exp(2 damping p)) per element (kept as w = (1-lam)(1-2r)
  // = (1-lam) z under a static lambda) and the run aggregate; u to LDS.
  float* const ul = &sh_ur.u[q.tg][q.lt * LPT][0];
  f32x4 uw[LPT];
  float rr[R][LPT];
  float A = 1.0f;
  float Bv[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) Bv[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float lam = lam_h;
    if constexpr (DYN) lam = __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, lamv[r], lam_h), p.lam_min, p.lam_max);
    lamv[r] = lam;
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float u = softsign_fast(xr.first(r, i));
      uw[i][r % 4] = u;
      if (r % 4 == 3) *reinterpret_cast<f32x4*>(ul + i * R + r - 3) = uw[i];
      const float rv = tanh_r(horner<KP>(u, c[i]));
      const float w = __builtin_fmaf(n2, rv, one_m);
      rr[r][i] = DYN ? rv : w;
      Bv[i] = __builtin_fmaf(lam, Bv[i], w);
    }
    if constexpr (DYN) A *= lam;
    xr.seal(r);
  }
  if constexpr (!DYN) A = sh_pw[0][q.lt * LPT];
  bool bad = false;
#pragma unroll
  for (int i = 0; i < LPT; ++i) bad |= Bv[i] != Bv[i];
  if (bad || cheb) {
    // Rare: a NaN input (z = 0 there: r = 1/2 gives w = 0; or u = 0 with
    // nan_zero_u), or a lane-block whose series is in the Chebyshev form (a
    // coefficient exceeds kMonoBound: the loop above ran Horner on Chebyshev
    // coefficients, so r is redone with Clenshaw); recompute the aggregate.
#pragma unroll
    for (int i = 0; i < LPT; ++i) Bv[i] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float one_m = 1.0f - lamv[r];
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const float x = xr.get(r, i);
        if (cheb || x != x) {
          float rv;
          if (x == x)
            rv = tanh_r(clenshaw<KP>(softsign_fast(x), c[i]));
          else
            rv = p.nan_zero_u ? tanh_r(cheb ? clenshaw<KP>(0.0f, c[i]) : c[i][0]) : 0.5f;
          rr[r][i] = DYN ? rv : __builtin_fmaf(-2.0f * one_m, rv, one_m);
        }
        const float w = DYN ? __builtin_fmaf(-2.0f * one_m, rr[r][i], one_m) : rr[r][i];
        Bv[i] = __builtin_fmaf(lamv[r], Bv[i], w);
      }
    }
  }

  // Target and lambda at each run's first token, for the preceding run.
#pragma unroll
  for (int i = 0; i < LPT; ++i) sh_y0[q.tg][q.lt * LPT + i] = target_of<SOFT>(xr.get(0, i));
  sh_lam0[q.tg][q.lt] = lamv[0];

  const LaneSlots ls = lane_slots<G, DYN>(p.slots, ti, p.n_tiles);
  float pA, pB[LPT], aggA, aggB;
  jitter(p.jitter, tags.epoch, 0);
  tile_scan<G, DYN>(L, q, ti, tags, A, Bv, pA, pB, aggA, aggB, ls);  // syncs sh_y0 too
  {
    const int dc = ti.lbd * G::LANES + carry_lane<G>(q);
    const float init_c = (p.ema_init && q.wave < G::NSUB && dc < p.D) ? p.ema_init[(int64_t)ti.b * p.D + dc] : 0.0f;
    // static lambda: the tile's decay as the look-back recomputes it
    if constexpr (!DYN) aggA = sh_pw[1][carry_lane<G>(q)];
    const int dlk = ti.lbd * G::LANES + look_lane<G>(q);
    const float a_look = DYN ? 0.0f : sh_pw[1][look_lane<G>(q)];
    LookBack<G, DYN> lbk;
    look_back_issue<G, DYN>(lbk, q, ti, ls);
    jitter(p.jitter, tags.epoch, 1);
    look_back_finish<G, DYN>(lbk, L, q, ti, tags, aggA, aggB, ls, init_c, a_look, p.hdr, p.poll_limit);
  }

  float y_after[LPT];
  float lam_after;
  if (!last_run) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) y_after[i] = sh_y0[q.tg + 1][q.lt * LPT + i];
    lam_after = sh_lam0[q.tg + 1][q.lt];
  } else {
#pragma unroll
    for (int i = 0; i < LPT; ++i) y_after[i] = target_of<SOFT>(x_after[i]);
    lam_after = DYN ? __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, g_after, lam_h), p.lam_min, p.lam_max)
                    : lam_h;
  }

  // Pass 2 from the carried state.
  // |s| <= 1 at the run start keeps |s| <= 1 over the run when 0 <= lambda
  // <= 1 (s is then a convex combination of it and values of tanh, and the
  // fp32 update cannot round past 1), so the clamp can only bind if the
  // carried state is already out of range; with the clamp off it is the
  // identity except on NaN.  The fast path assumes neither happens.
  const bool clamp = p.clamp_out != 0;
  float s[LPT];
  bool big = DYN ? !(p.lam_min >= 0.0f && p.lam_max <= 1.0f) : !(lam_h >= 0.0f && lam_h <= 1.0f);
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    s[i] = __builtin_fmaf(pA, L.carry[q.lt * LPT + i], pB[i]);
    big |= clamp ? !(__builtin_fabsf(s[i]) <= 1.0f) : s[i] != s[i];
  }
  const float lo = clamp ? -1.0f : -__builtin_inff();
  const float hi = clamp ? 1.0f : __builtin_inff();
  const int t_first = ti.tile * G::TILE + q.tg * R;
  float* fin = (ti.is_last && p.ema_final && a.vo != kOffOOB)
                   ? p.ema_final + (int64_t)ti.b * p.D + ti.lbd * kLanes + q.lt * LPT
                   : nullptr;
  const float om2 = (1.0f - lam_h) * (1.0f - lam_h);
  // A NaN state at the run start (a look-back wait that gave up, or a NaN
  // ema_init) makes every later state of the run NaN; the slow pass 2 takes
  // it, and its output and gradient terms are replaced by NaN below.
  bool nan_s = false;
#pragma unroll
  for (int i = 0; i < LPT; ++i) nan_s |= s[i] != s[i];
  RunGrad<KP, LPT> rg;
  if (bad || big || ti.is_last)
    ttt_pass2<G, DYN, SOFT, true, XT, OT, KP>(rg, s, xr, ul, rr, lamv, om2, y_after, a, lo, hi, t_first, p.S,
                                               clamp, p.nan_zero_u != 0, fin);
  else
    ttt_pass2<G, DYN, SOFT, false, XT, OT, KP>(rg, s, xr, ul, rr, lamv, om2, y_after, a, lo, hi, t_first,
                                                p.S, clamp, false, fin);

  if (nan_s) {
    // The clamp (v_med3_f32) turned the NaN states into bounds: store NaN,
    // and make this run's gradient terms NaN, so the records and the
    // gradient are NaN (the float64 definition gives NaN there too).
    static_assert(LPT == 1, "one lane per thread: the NaN state is the thread's");
    const float qnan = __builtin_nanf("");
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float o[LPT] = {qnan};
      BufVec<OT, LPT>::store(a.out, a.vo, so, o);
      so = next_off(so, a.so);
    }
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      rg.al[i] = qnan;
#pragma unroll
      for (int k = 0; k < KP; ++k) rg.P[k][i] = qnan;
    }
  }

  // Compose the runs of the tile: rho of run g = Ar_g + Br_g rho_tile.
  const float beta = rg.Lp * lam_after;
#pragma unroll
  for (int i = 0; i < LPT; ++i) sh_al[q.tg][q.lt * LPT + i] = rg.al[i];
  sh_be[q.tg][q.lt] = beta;
  __syncthreads();
  float Ar[LPT], Br = 1.0f;
#pragma unroll
  for (int i = 0; i < LPT; ++i) Ar[i] = 0.0f;
  for (int g = NTG - 1; g > q.tg; --g) {
    const float bg = sh_be[g][q.lt];
#pragma unroll
    for (int i = 0; i < LPT; ++i) Ar[i] = __builtin_fmaf(bg, Ar[i], sh_al[g][q.lt * LPT + i]);
    Br *= bg;
  }
  float* part = p.partials + ((size_t)ti.lb * p.n_tiles + ti.tile) * F * kLanes;
  if (q.tg == 0) {
    // Tile map: a[tile start] = al_0 + beta_0 (Ar_0 + Br_0 rho_tile).
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      part[(size_t)(2 * KP) * kLanes + q.lt * LPT + i] = beta * Br;
      part[(size_t)(2 * KP + 1) * kLanes + q.lt * LPT + i] = __builtin_fmaf(beta, Ar[i], rg.al[i]);
    }
  }
  const float ks = ttt_lane_scale<DYN>(p, a.h);
  // Run contributions P + lam_after F (Ar + Br rho_tile), summed over runs;
  // the per-lane scale is applied to the sums.
  const float cB = lam_after * Br;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const float pv = wave_sum_tg<G>(__builtin_fmaf(lam_after * Ar[i], rg.F[k][i], rg.P[k][i]));
      const float qv = wave_sum_tg<G>(cB * rg.F[k][i]);
      if (q.wl < G::TPR) {
        sh_ur.red[q.wave][k][q.lt * LPT + i] = pv;
        sh_ur.red[q.wave][KP + k][q.lt * LPT + i] = qv;
      }
    }
  }
  __syncthreads();
  // scale of lane wl (the thread's own lane when LPT = 1)
  const int dw = ti.lbd * kLanes + q.wl;
  const float ks_w = LPT == 1 ? ks : ttt_lane_scale<DYN>(p, dw < p.D ? div_hd(dw, p) : 0);
  for (int v = q.wave; v < 2 * KP; v += G::WAVES) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < G::WAVES; ++w) acc += sh_ur.red[w][v][q.wl];
    part[(size_t)v * kLanes + q.wl] = ks_w * acc;
  }
  finish_block(p.hdr, tags.epoch);
}

// The scaled monomial coefficients of every lane-block, as the forward forms
// them per tile (mono_issue / mono_store): coefficient j of lane l from
// c_{j+2i} in float64 with the factors cheb_mono(j, i), times 2 log2(e)
// damping_h, rounded once.  Thread (j, lane) of block lb; lanes >= D get 0.
// When one of them exceeds kMonoBound (as the forward decides per tile), the
// lane-block keeps its Chebyshev coefficients instead (c_j times the same
// scale, for Clenshaw) and form[lb] = 1, else 0.
template <int KP>
__global__ void __launch_bounds__(64 * KP) ttt_mono_prep(const FwdParams p, float* tab, unsigned* form) {
  const int lb = blockIdx.x, j = threadIdx.x / kLanes, l = threadIdx.x % kLanes;
  const int b = lb / p.n_lbd;
  const int d = (lb - b * p.n_lbd) * kLanes + l;
  float cm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float kap = 0.0f;
  if (d < p.D) {
    const int h = div_hd(d, p);
    const float* c = p.coeffs + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (d - h * p.hd);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = j + 2 * i;
      cm[i] = k < p.K ? c[(int64_t)k * p.c_sk] : 0.0f;
    }
    kap = kTwoLog2e * p.damping[h];
  }
  double acc = 0.0;
  switch (j) {
    case 0: acc = mono_coef<0>(cm); break;
    case 1: acc = mono_coef<1>(cm); break;
    case 2: acc = mono_coef<2>(cm); break;
    case 3: acc = mono_coef<3>(cm); break;
    case 4: acc = mono_coef<4>(cm); break;
    case 5: acc = mono_coef<5>(cm); break;
    case 6: acc = mono_coef<6>(cm); break;
    default: acc = mono_coef<7>(cm); break;
  }
  const float v = (float)(acc * (double)kap);
  const bool cheb = __syncthreads_or(!(__builtin_fabsf(v) <= kMonoBound)) != 0;
  tab[((size_t)lb * KP + j) * kLanes + l] = cheb ? (float)((double)cm[0] * (double)kap) : v;
  if (threadIdx.x == 0) form[lb] = cheb ? 1u : 0u;
}

// Merge of the records n-1 .. 0 of one lane (record i at base + i * rstride,
// fields kLanes apart) for coefficient k, from the sequence end: record e
// before the merged later part c gives
//   P = P_c + P_e + Br_c Q_e,  Q = Q_c + Ar_c Q_e,  Ar = Ar_e Ar_c,  Br = Ar_e Br_c + Br_e.
// The loads of NB records are issued together.
template <int KP, int NB>
__device__ __forceinline__ void merge_lane(const float* base, size_t rstride, int n, int k, float& P, float& Q,
                                           float& Ar, float& Br) {
  P = 0.0f, Q = 0.0f, Ar = 1.0f, Br = 0.0f;
  for (int top = n - 1; top >= 0; top -= NB) {
    float Pe[NB], Qe[NB], Ae[NB], Be[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float* r = base + (size_t)max(top - j, 0) * rstride;
      Pe[j] = r[(size_t)k * kLanes];
      Qe[j] = r[(size_t)(KP + k) * kLanes];
      Ae[j] = r[(size_t)(2 * KP) * kLanes];
      Be[j] = r[(size_t)(2 * KP + 1) * kLanes];
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (top - j >= 0) {
        P = P + __builtin_fmaf(Br, Qe[j], Pe[j]);
        Q = __builtin_fmaf(Ar, Qe[j], Q);
        const float br = __builtin_fmaf(Ae[j], Br, Be[j]);
        Ar = Ae[j] * Ar;
        Br = br;
      }
    }
  }
}

// Level 1: thread (k, lane) merges coefficient k of up to kChunk consecutive
// tiles of one lane.
template <int KP>
__global__ void __launch_bounds__(64 * KP) ttt_merge_chunks(const float* partials, float* chunks, int n_tiles,
                                                            int n_chunks) {
  constexpr int F = n_fields<KP>();
  const int chunk = blockIdx.x, lb = blockIdx.y, l = threadIdx.x % kLanes, k = threadIdx.x / kLanes;
  const int first = chunk * kChunk;
  const int n = min(first + kChunk, n_tiles) - first;
  float P, Q, Ar, Br;
  merge_lane<KP, kChunk>(partials + ((size_t)lb * n_tiles + first) * F * kLanes + l, (size_t)F * kLanes, n, k, P, Q,
                         Ar, Br);
  float* dst = chunks + ((size_t)lb * n_chunks + chunk) * F * kLanes + l;
  dst[(size_t)k * kLanes] = P;
  dst[(size_t)(KP + k) * kLanes] = Q;
  if (k == 0) {
    dst[(size_t)(2 * KP) * kLanes] = Ar;
    dst[(size_t)(2 * KP + 1) * kLanes] = Br;
  }
}

// Level 2: merge the chunks of each lane from the sequence end (rho = 0) and
// write grad[b,h,k,j] = G_k / (k+1)^2; thread (k, lane).
template <int KP>
__global__ void __launch_bounds__(64 * KP) ttt_finalize(const float* chunks, float* grad, int n_chunks, int n_lbd,
                                                        int D, int hd, int H, int K) {
  constexpr int F = n_fields<KP>();
  const int lb = blockIdx.x, l = threadIdx.x % kLanes, k = threadIdx.x / kLanes;
  float P, Q, Ar, Br;
  merge_lane<KP, 8>(chunks + (size_t)lb * n_chunks * F * kLanes + l, (size_t)F * kLanes, n_chunks, k, P, Q, Ar, Br);
  const int b = lb / n_lbd;
  const int d = (lb - b * n_lbd) * kLanes + l;
  if (d >= D || k >= K) return;
  const int h = d / hd, j = d - h * hd;
  grad[(((size_t)b * H + h) * K + k) * hd + j] = P / (float)((k + 1) * (k + 1));
}

template <class G, bool DYN, bool SOFT, typename XT, typename OT, int KP>
hipError_t launch_all(const FwdParams& p0, float* grad, hipStream_t stream) {
  const int n_chunks = (p0.n_tiles + kChunk - 1) / kChunk;
  float* chunks = p0.partials + (size_t)p0.n_lb * p0.n_tiles * n_fields<KP>() * kLanes;
  FwdParams p = p0;
  p.mono_tab = chunks + (size_t)p.n_lb * n_chunks * n_fields<KP>() * kLanes;
  unsigned* form = reinterpret_cast<unsigned*>(p.mono_tab + (size_t)p.n_lb * KP * kLanes);
  p.mono_form = form;
  hipLaunchKernelGGL((ttt_mono_prep<KP>), dim3(p.n_lb), dim3(64 * KP), 0, stream, p, p.mono_tab, form);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const unsigned grid = (unsigned)p.n_lb_pad * (unsigned)p.n_tiles;
  hipLaunchKernelGGL((cheby_ema_ttt_kernel<G, DYN, SOFT, XT, OT, KP>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ttt_merge_chunks<KP>), dim3(n_chunks, p.n_lb), dim3(64 * KP), 0, stream, p.partials, chunks,
                     p.n_tiles, n_chunks);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ttt_finalize<KP>), dim3(p.n_lb), dim3(64 * KP), 0, stream, chunks, grad, n_chunks, p.n_lbd,
                     p.D, p.hd, p.H, p.K);
  return hipGetLastError();
}

template <class G, bool DYN, typename XT, typename OT>
hipError_t launch_k(const FwdParams& p, float* grad, int kpad, hipStream_t stream) {
  const bool soft = p.ttt_target == 1;
  if (kpad == 4)
    return soft ? launch_all<G, DYN, true, XT, OT, 4>(p, grad, stream) : launch_all<G, DYN, false, XT, OT, 4>(p, grad, stream);
  return soft ? launch_all<G, DYN, true, XT, OT, 8>(p, grad, stream) : launch_all<G, DYN, false, XT, OT, 8>(p, grad, stream);
}

// Geometry; must agree with ttt_tile_tokens.
template <bool DYN, typename XT, typename OT>
hipError_t launch_geo(const FwdParams& p, float* grad, int tile, int kpad, hipStream_t stream) {
  if (tile != TttTile::TILE) return hipErrorInvalidValue;
  return launch_k<TttTile, DYN, XT, OT>(p, grad, kpad, stream);
}

template <bool DYN>
hipError_t launch_dt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, int tile, int kpad,
                     hipStream_t stream) {
  if (x_dtype == 0 && out_dtype == 0) return launch_geo<DYN, float, float>(p, grad, tile, kpad, stream);
  if (x_dtype == 0 && out_dtype == 1) return launch_geo<DYN, float, __bf16>(p, grad, tile, kpad, stream);
  if (x_dtype == 1 && out_dtype == 0) return launch_geo<DYN, __bf16, float>(p, grad, tile, kpad, stream);
  return launch_geo<DYN, __bf16, __bf16>(p, grad, tile, kpad, stream);
}

}  // namespace

int ttt_tile_tokens(bool, int) { return TttTile::TILE; }

size_t ttt_workspace_bytes(int n_lb, int n_tiles, bool dyn, int K) {
  const int kpad = K <= 4 ? 4 : 8;
  const size_t F = 2 * kpad + 2;
  const size_t n_chunks = (n_tiles + kChunk - 1) / kChunk;
  const size_t slots = (fwd_workspace_bytes(n_lb, n_tiles, TttTile::LANES, dyn) + 255) / 256 * 256;
  // per-tile partials, per-chunk merges, the coefficient table and its form words
  return slots + (((size_t)n_lb * n_tiles + (size_t)n_lb * n_chunks) * F + (size_t)n_lb * kpad) * kLanes * sizeof(float) +
         (size_t)n_lb * sizeof(unsigned);
}

hipError_t launch_ttt(const FwdParams& p, float* grad, int x_dtype, int out_dtype, bool dyn, int tile, int kpad,
                      hipStream_t stream) {
  return dyn ? launch_dt<true>(p, grad, x_dtype, out_dtype, tile, kpad, stream)
             : launch_dt<false>(p, grad, x_dtype, out_dtype, tile, kpad, stream);
}

}  // namespace osm
