// Backward of the fused Cheby-RKV forward for gfx950: dL/dx, dL/dc and
// dL/d ema_init from dL/dout (and dL/d ema_final), one pass over HBM (x,
// dL/dout and the saved output read once, dL/dx written once).
//
// Reference counterpart: the gradient of the PyTorch fast path
// (sdpc_kernel.py:1708-1744), i.e. autograd through softsign, Chebyshev
// basis, damping and tanh, with the EMA's own backward
// _EMAFastPathFn.backward (sdpc_kernel.py:1677-1701) and its masked reverse
// scan _parallel_reverse_ema_kernel (sdpc_kernel.py:682-777).
//
// Math, per lane, tokens t < S:
//   a[t] = m[t] (dL/dout[t] + v[t+1]),  v[t] = lam[t] a[t],  v[S] = dL/d ema_final
//   m[t] = [|out[t]| < 1 - 1e-6] on the saved output (1 without the clamp)
//   e[t] = a[t] (1 - lam[t]) r (1 - r),  r = 1 / (1 + exp(2 damping p)),
//          so that dL/dp = 4 damping e   (1 - tanh^2 = 4 r (1 - r))
//   dL/dc_k  = 4 damping sum_t e[t] T_k(u[t])
//   dL/dx[t] = 2 ln2 e[t] y'(u[t]) / (1 + |x[t]|)^2,  y = 2 log2(e) damping p
//              (0 where |x| < 1e-7 or x is NaN, as the reference's softsign
//              clamps |x| at 1e-7 and masks NaN with torch.where)
//   dL/d ema_init = v[0]
// v[t] = lam[t] m[t] (dL/dout[t] + v[t+1]) is an affine map of v[t+1]
// (A = lam m, B = lam m dL/dout), so runs and tiles compose like the
// forward's EMA and tiles are chained from the end of the sequence with the
// look-back of osm_chain.h: chain index c covers tile n_tiles-1-c, and
// inside a tile the runs are scanned last one first.
//
// Per workgroup (512 threads, a tile of G::TILE tokens x 64 lanes, one lane
// per thread and a run of R tokens per thread):
//   1. load x, dL/dout, the saved output (for the mask) and g;
//   2. pass 1, last token first: the run's map (A, B);
//   3. token-group scan and look-back -> v after the tile;
//   4. pass 2, last token first: a, e, dL/dx stored, sum_t e T_k(u) kept in
//      registers;
//   5. the tile's sums over its runs -> partials[lane-block][tile][k][lane].
// A small kernel adds the partials over tiles in a fixed order (results do
// not depend on timing) and scales them into dL/dc.
#include "osm_tile.h"

namespace osm {
namespace {

constexpr float kMaskBound = 0.999999f;         // 1 - 1e-6 rounded to fp32, as the reference compares in fp32
constexpr float kSoftsignGradMin = 1e-7f;       // the reference's clamp of |x| in the softsign
constexpr float kTwoLn2 = 1.3862943611198906f;  // dL/dx from y' = 2 log2(e) damping p'

// One [B,S,*] tensor's rows of a tile: descriptor from the tile's first row
// to the end of row S-1, per-thread lane offset, uniform step per token.
struct RowStream {
  Rsrc r;
  uint32_t v, s;
};

template <class G, typename T>
__device__ __forceinline__ RowStream row_stream(const void* base, int64_t sb, int64_t ss, const FwdParams& p,
                                                const ThreadPos& q, const TileInfo& tm) {
  RowStream st;
  const int t_tile = tm.tile * G::TILE;
  const int d0 = tm.lbd * G::LANES + q.lt * G::LPT;
  const uint64_t rows_after = (uint64_t)(p.S - 1 - t_tile);
  const char* b = static_cast<const char*>(base) + ((int64_t)tm.b * sb + (int64_t)t_tile * ss) * sizeof(T);
  st.r = make_rsrc(b, (rows_after * ss + p.D) * sizeof(T));
  st.s = (uint32_t)(ss * sizeof(T));
  st.v = d0 < p.D ? (uint32_t)(((int64_t)q.tg * G::R * ss + d0) * sizeof(T)) : kOffOOB;
  return st;
}

// Steps a uniform byte offset back by `step` (see next_off).
__device__ __forceinline__ uint32_t prev_off(uint32_t off, uint32_t step) {
  off -= step;
  asm volatile("" : "+s"(off));
  return off;
}

// sum_t e T_k(u) for k < KP, T_k by the Chebyshev recurrence.
template <int KP>
__device__ __forceinline__ void accumulate_basis(float (&Gk)[KP], float e, float u) {
  Gk[0] += e;
  if constexpr (KP > 1) Gk[1] = __builtin_fmaf(e, u, Gk[1]);
  const float u2 = u + u;
  float tm2 = 1.0f, tm1 = u;
#pragma unroll
  for (int k = 2; k < KP; ++k) {
    const float tk = __builtin_fmaf(u2, tm1, -tm2);
    Gk[k] = __builtin_fmaf(e, tk, Gk[k]);
    tm2 = tm1;
    tm1 = tk;
  }
}

// Pass 2 over a thread's run, last token first, from v = v[t_end + 1].
// c: the lane's scaled series coefficients (monomial, y = sum c_j u^j, or
// Chebyshev, y = sum c_k T_k(u), for more than kMonoMaxK of them; see
// series()); dm[m] = (m+1) c[m+1] times 2 ln2 (and 1 - lam for a static
// lambda): y' = sum dm[m] u^m, or sum dm[m] U_m(u) in the Chebyshev form.  SLOW handles, per
// element, tokens >= S (r >= n_valid: identity map, no contribution), the clamp mask
// (mbits bit r set: m = 0), NaN inputs (u = 0; e = 0 unless nan_zero_u);
// the fast variant assumes none of them occurs in the run.  ZS: 1 - z^2 comes
// from the saved z (zv) instead of the recomputed series.  full_jac: dL/dx
// uses 1/(1+|x|)^2 everywhere (NaN for a NaN x) instead of 0 below 1e-7.
// cheb (slow variant only): c and dm are in the Chebyshev form of a tile
// whose monomial coefficients exceed kMonoBound.
template <class G, bool DYN, bool SLOW, bool ZS, typename XT, int KP>
__device__ __forceinline__ void bwd_pass2(float& v, float (&Gk)[KP], const float (&xv)[G::R], const float (&gv)[G::R],
                                          const float (&zv)[ZS ? G::R : 1], const float (&lamv)[G::R], float lam_h,
                                          const float (&c)[KP], const float (&dm)[KP > 1 ? KP - 1 : 1],
                                          const RowStream& gx, int n_valid, unsigned mbits, bool nan_zero_u,
                                          bool full_jac, bool cheb) {
  constexpr int R = G::R;
  uint32_t so = (uint32_t)(R - 1) * gx.s;
  asm volatile("" : "+s"(so));
#pragma unroll
  for (int r = R - 1; r >= 0; --r) {
    float lam = DYN ? lamv[r] : lam_h;
    const float x = xv[r];
    float av = gv[r] + v;
    bool live = true;
    if constexpr (SLOW) {
      const bool valid = r < n_valid;
      if constexpr (!DYN) lam = valid ? lam : 1.0f;   // (DYN: pass 1 already set lamv[r] = 1)
      av = ((mbits >> r) & 1u) ? 0.0f : av;
      live = valid && (x == x || nan_zero_u);
    }
    v = lam * av;
    const float ir = __builtin_amdgcn_rcpf(1.0f + __builtin_fabsf(x));
    float u = __builtin_copysignf(1.0f - ir, x);
    if constexpr (SLOW) u = (x == x) ? u : 0.0f;
    float hq;   // r (1 - r) = (1 - z^2) / 4
    if constexpr (ZS) {
      hq = 0.25f * __builtin_fmaf(-zv[r], zv[r], 1.0f);
    } else {
      float y;
      if (SLOW && cheb)
        y = series_as<KP, true>(u, c);
      else
        y = series_as<KP, false>(u, c);
      const float rr = tanh_r(y);
      hq = __builtin_fmaf(-rr, rr, rr);
    }
    float e = av * hq;
    if constexpr (DYN) e *= 1.0f - lam;
    if constexpr (SLOW) e = live ? e : 0.0f;
    float dy = 0.0f;
    if constexpr (KP > 1) {
      if (SLOW && cheb)
        dy = dseries_as<KP - 1, true>(u, dm);
      else
        dy = dseries_as<KP - 1, false>(u, dm);
    }
    float gxv[1] = {e * dy * ir * ir};
    if (!full_jac) gxv[0] = __builtin_fabsf(x) >= kSoftsignGradMin ? gxv[0] : 0.0f;
    BufVec<XT, 1>::store(gx.r, gx.v, so, gxv);
    if (r > 0) so = prev_off(so, gx.s);
    accumulate_basis<KP>(Gk, e, u);
  }
}

// Two workgroups (4 waves per SIMD) per CU: at most 128 VGPRs.
template <class G, bool DYN, bool ZS, typename XT, typename OT, int KP>
__global__ void __launch_bounds__(G::THREADS) __attribute__((amdgpu_waves_per_eu(4)))
cheby_ema_bwd_kernel(const BwdParams bp) {
  constexpr int R = G::R;
  static_assert(G::LPT == 1 && G::LANES == kLanes && G::TGW == 1, "one lane per thread, one run per wave");
  const FwdParams& p = bp.f;
  __shared__ ChainLds<G> L;
  __shared__ float mono[KP][kLanes];
  __shared__ float sh_red[G::WAVES][KP][kLanes];

  // Highest wave priority while the tile's loads are issued (here and
  // before the x loads below), so that they enter the memory pipeline ahead
  // of other workgroups' arithmetic (measured at BASELINE configs[1] on
  // MI355X: 121.8 against 124.0 us).
  __builtin_amdgcn_s_setprio(3);
  const ThreadPos q = thread_pos<G>();
  ThreadPos qc = q;
  qc.tg = G::NTG - 1 - q.tg;   // chain order: the tile's last run first
  const Tags tags = launch_tags(p.hdr);
  const TileInfo ti = tile_info<G>(blockIdx.x, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles);   // tile = chain index
  if (ti.pad) {
    finish_block(p.hdr, tags.epoch);
    return;
  }
  TileInfo tm = ti;
  tm.tile = p.n_tiles - 1 - ti.tile;   // tile in sequence order
  const TileAddr a = tile_addr<G, DYN, XT, OT>(p, q, tm);
  const RowStream go = row_stream<G, OT>(bp.gout, bp.go_sb, bp.go_ss, p, q, tm);
  const RowStream gx = row_stream<G, XT>(bp.gx, bp.gx_sb, bp.gx_ss, p, q, tm);
  const auto ml = mono_issue<KP, G>(p, q, ti, a);

  // dL/dout, the saved output and g first: pass 1 needs only them, and the
  // x loads are issued after it (below) so that they are in flight during
  // the chain while the saved output's registers are free again.
  const bool clamp = p.clamp_out != 0;
  float xv[R], gv[R], ov[R], lamv[R];
  {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t[1];
      BufVec<OT, 1>::load(go.r, go.v, so, t);
      gv[r] = t[0];
      so = next_off(so, go.s);
    }
  }
  if (clamp) {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t[1];
      BufVec<OT, 1>::load(a.out, a.vo, so, t);
      ov[r] = t[0];
      so = next_off(so, a.so);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) ov[r] = 0.0f;
  }
  const float lam_h = p.lam[a.h];
  if constexpr (DYN) {
    uint32_t sg = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      lamv[r] = load_f32_shared(a.g, a.vg, sg);   // a line of g serves every lane-block of the row
      sg = next_off(sg, a.sg);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  __shared__ unsigned mono_big[KP * G::NSUB];
  mono_store<KP, G>(ml, q, mono, mono_big);   // read after the chain's barriers

  // Pass 1: the run's map v[t0] = A v[t_end + 1] + B, last token first.
  // Tokens of this run that are < S (wave-uniform: one run per wave).
  const int n_valid = p.S - (tm.tile * G::TILE + __builtin_amdgcn_readfirstlane(q.tg) * R);
  const bool tail = tm.tile == p.n_tiles - 1;
  bool masked = false;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (clamp) masked |= !(__builtin_fabsf(ov[r]) < kMaskBound);
    if constexpr (DYN)
      lamv[r] = __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, lamv[r], lam_h), p.lam_min, p.lam_max);
  }
  const bool slow1 = tail || masked;
  float A = 1.0f, Bv[1] = {0.0f};
  unsigned mbits = 0;
  if (!slow1) {
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      const float lam = DYN ? lamv[r] : lam_h;
      Bv[0] = lam * (gv[r] + Bv[0]);
      if constexpr (DYN) A *= lam;
    }
    if constexpr (!DYN) A = pow_n<R>(lam_h);
  } else {
    // Tokens >= S (last tile) are the identity; a zero mask cuts the chain.
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      const bool valid = r < n_valid;
      const bool m = !clamp || !valid || __builtin_fabsf(ov[r]) < kMaskBound;
      mbits |= m ? 0u : (1u << r);
      float lam = valid ? (DYN ? lamv[r] : lam_h) : 1.0f;
      if constexpr (DYN) lamv[r] = lam;
      lam = m ? lam : 0.0f;
      Bv[0] = lam * (gv[r] + Bv[0]);
      A *= lam;
    }
  }

  // x loads (kept in order after pass 1 by the barrier).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_setprio(3);
  {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t[1];
      BufVec<XT, 1>::load(a.x, a.vx, so, t);
      xv[r] = t[0];
      so = next_off(so, a.sx);
    }
  }
  float zv[ZS ? R : 1];
  if constexpr (ZS) {
    const RowStream zs = row_stream<G, __bf16>(bp.zs, bp.zs_sb, bp.zs_ss, p, q, tm);
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t[1];
      BufVec<__bf16, 1>::load(zs.r, zs.v, so, t);
      zv[r] = t[0];
      so = next_off(so, zs.s);
    }
  }

  __builtin_amdgcn_s_setprio(0);
  const LaneSlots ls = lane_slots<G, true>(p.slots, ti, p.n_tiles);
  float pA, pB[1], aggA, aggB;
  jitter(p.jitter, tags.epoch, 0);
  tile_scan<G, true>(L, qc, ti, tags, A, Bv, pA, pB, aggA, aggB, ls);
  {
    const int dc = ti.lbd * G::LANES + carry_lane<G>(q);
    const float init_c =
        (bp.grad_state && q.wave < G::NSUB && dc < p.D) ? bp.grad_state[(int64_t)ti.b * p.D + dc] : 0.0f;
    LookBack<G, true> lbk;
    look_back_issue<G, true>(lbk, q, ti, ls);
    jitter(p.jitter, tags.epoch, 1);
    look_back_finish<G, true>(lbk, L, q, ti, tags, aggA, aggB, ls, init_c, 0.0f, p.hdr, p.poll_limit);
  }
  float v = __builtin_fmaf(pA, L.carry[q.lt], pB[0]);

  // Pass 2.
  float c[1][KP];
  // Monomial form unless a coefficient of the tile exceeds kMonoBound; a
  // tile in the Chebyshev form (rare with up to kMonoMaxK coefficients)
  // rewrites the table and takes the slow pass 2, which evaluates either.
  const bool cheb = tile_cheb<KP, G>(mono_big);
  if (KP <= kMonoMaxK && cheb) {
    mono_store_cheb<KP, G>(p, q, ti, a, mono);
    __syncthreads();
  }
  mono_read<G, KP>(mono, q, c);
  float dm[KP > 1 ? KP - 1 : 1];
  {
    const float ks = kTwoLn2 * (DYN ? 1.0f : 1.0f - lam_h);
#pragma unroll
    for (int j = 1; j < KP; ++j) dm[j - 1] = (float)j * ks * c[0][j];
    if constexpr (KP == 1) dm[0] = 0.0f;
  }
  float Gk[KP];
#pragma unroll
  for (int k = 0; k < KP; ++k) Gk[k] = 0.0f;
  bool bad = false;
#pragma unroll
  for (int r = 0; r < R; ++r) bad |= xv[r] != xv[r];
  const bool full_jac = bp.full_jac != 0;
  const bool cheb2 = KP <= kMonoMaxK && cheb;   // (above kMonoMaxK both variants use Clenshaw)
  if (slow1 || bad || cheb2)
    bwd_pass2<G, DYN, true, ZS, XT, KP>(v, Gk, xv, gv, zv, lamv, lam_h, c[0], dm, gx, n_valid, mbits,
                                        p.nan_zero_u != 0, full_jac, cheb2);
  else
    bwd_pass2<G, DYN, false, ZS, XT, KP>(v, Gk, xv, gv, zv, lamv, lam_h, c[0], dm, gx, n_valid, 0u, false,
                                         full_jac, false);

  // dL/d ema_init = v[0], held by the first run of tile 0.
  if (tm.tile == 0 && q.tg == 0 && bp.grad_init) {
    const int d = tm.lbd * G::LANES + q.lt;
    if (d < p.D) bp.grad_init[(int64_t)tm.b * p.D + d] = v;
  }

  // The tile's partial sums: runs (one per wave) added in wave order.
#pragma unroll
  for (int k = 0; k < KP; ++k) sh_red[q.wave][k][q.wl] = Gk[k];
  __syncthreads();
  float* part = p.partials + ((size_t)ti.lb * p.n_tiles + tm.tile) * KP * kLanes;
  for (int k = q.wave; k < KP; k += G::WAVES) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < G::WAVES; ++w) acc += sh_red[w][k][q.wl];
    part[(size_t)k * kLanes + q.wl] = acc;
  }
  finish_block(p.hdr, tags.epoch);
}

// dL/dc[b,h,k,j] = 4 damping_h (1 - lam_h if static) * sum over the tiles of
// lane-block lb.  Block (k, lb): slice sl of kRedSlices adds tiles sl,
// sl + kRedSlices, ... of each lane, then the slices are added in order, so
// the result does not depend on timing.
constexpr int kRedSlices = 16;

template <int KP>
__global__ void __launch_bounds__(kRedSlices * kLanes) bwd_reduce(const float* partials, float* grad,
                                                                 const float* damping, const float* lam, int dyn,
                                                                 int n_tiles, int n_lbd, int D, int hd, int H, int K) {
  __shared__ float red[kRedSlices][kLanes];
  const int k = blockIdx.x, lb = blockIdx.y;
  const int sl = threadIdx.x / kLanes, l = threadIdx.x - sl * kLanes;
  const float* src = partials + (size_t)lb * n_tiles * KP * kLanes + (size_t)k * kLanes + l;
  float acc = 0.0f;
#pragma unroll 8
  for (int t = sl; t < n_tiles; t += kRedSlices) acc += src[(size_t)t * KP * kLanes];
  red[sl][l] = acc;
  __syncthreads();
  if (sl != 0) return;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kRedSlices; ++i) sum += red[i][l];
  const int b = lb / n_lbd;
  const int d = (lb - b * n_lbd) * kLanes + l;
  if (d >= D || k >= K) return;
  const int h = d / hd, j = d - h * hd;
  const float scale = 4.0f * damping[h] * (dyn ? 1.0f : 1.0f - lam[h]);
  grad[(((size_t)b * H + h) * K + k) * hd + j] = sum * scale;
}

template <class G, bool DYN, bool ZS, typename XT, typename OT, int KP>
hipError_t launch_all(const BwdParams& bp, hipStream_t stream) {
  const FwdParams& p = bp.f;
  const unsigned grid = (unsigned)p.n_lb_pad * (unsigned)p.n_tiles;
  hipLaunchKernelGGL((cheby_ema_bwd_kernel<G, DYN, ZS, XT, OT, KP>), dim3(grid), dim3(G::THREADS), 0, stream, bp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bp.grad_coeffs) return e;
  hipLaunchKernelGGL((bwd_reduce<KP>), dim3(KP, p.n_lb), dim3(kRedSlices * kLanes), 0, stream, p.partials,
                     bp.grad_coeffs, p.damping, p.lam, DYN ? 1 : 0, p.n_tiles, p.n_lbd, p.D, p.hd, p.H, p.K);
  return hipGetLastError();
}

template <bool DYN, typename XT, typename OT>
hipError_t launch_k(const BwdParams& bp, int tile, int kpad, hipStream_t stream) {
  if (kpad == 16) {
    // Chebyshev form: shorter runs leave room for 3 x 16 coefficient and
    // gradient registers.
    if (tile != BwdTileCheb::TILE) return hipErrorInvalidValue;
    if (bp.zs) return hipErrorInvalidValue;
    return launch_all<BwdTileCheb, DYN, false, XT, OT, 16>(bp, stream);
  }
  if (kpad == 32) {
    if (tile != BwdTileCheb32::TILE) return hipErrorInvalidValue;
    if (bp.zs) return hipErrorInvalidValue;
    return launch_all<BwdTileCheb32, DYN, false, XT, OT, 32>(bp, stream);
  }
  using G = BwdTile;
  if (tile != G::TILE) return hipErrorInvalidValue;
  if (bp.zs) {
    // Saved z (the full path's backward): static lambda and an fp32 output only.
    if constexpr (!DYN && std::is_same<OT, float>::value) {
      if (kpad == 4) return launch_all<G, false, true, XT, OT, 4>(bp, stream);
      return launch_all<G, false, true, XT, OT, 8>(bp, stream);
    }
    return hipErrorInvalidValue;
  }
  if (kpad == 4) return launch_all<G, DYN, false, XT, OT, 4>(bp, stream);
  return launch_all<G, DYN, false, XT, OT, 8>(bp, stream);
}

template <bool DYN>
hipError_t launch_dt(const BwdParams& bp, int x_dtype, int out_dtype, int tile, int kpad, hipStream_t stream) {
  if (x_dtype == 0 && out_dtype == 0) return launch_k<DYN, float, float>(bp, tile, kpad, stream);
  if (x_dtype == 0 && out_dtype == 1) return launch_k<DYN, float, __bf16>(bp, tile, kpad, stream);
  if (x_dtype == 1 && out_dtype == 0) return launch_k<DYN, __bf16, float>(bp, tile, kpad, stream);
  return launch_k<DYN, __bf16, __bf16>(bp, tile, kpad, stream);
}

}  // namespace

int bwd_tile_tokens(bool, int kpad) {
  return kpad > 16 ? BwdTileCheb32::TILE : (kpad > kMonoMaxK ? BwdTileCheb::TILE : BwdTile::TILE);
}

size_t bwd_slot_bytes(int n_lb, int n_tiles) { return fwd_workspace_bytes(n_lb, n_tiles, kLanes, true); }

size_t bwd_workspace_bytes(int n_lb, int n_tiles, int K) {
  const size_t kpad = K <= 4 ? 4 : (K <= 8 ? 8 : (K <= 16 ? 16 : 32));
  const size_t slots = (bwd_slot_bytes(n_lb, n_tiles) + 255) / 256 * 256;
  return slots + (size_t)n_lb * n_tiles * kpad * kLanes * sizeof(float);
}

hipError_t launch_bwd(const BwdParams& p, int x_dtype, int out_dtype, bool dyn, int tile, int kpad,
                      hipStream_t stream) {
  return dyn ? launch_dt<true>(p, x_dtype, out_dtype, tile, kpad, stream)
             : launch_dt<false>(p, x_dtype, out_dtype, tile, kpad, stream);
}

}  // namespace osm
