// Fused Cheby-RKV forward for gfx950: softsign -> Clenshaw -> damping ->
// tanh -> EMA scan, one pass over HBM (x read once, out written once).
//
// Reference counterpart: the forward part of _ortho_megakernel
// (sdpc_kernel.py:2006-2124) and _fused_clenshaw_ema_kernel
// (sdpc_kernel.py:988-1209).  The reference walks S serially inside each of
// B*H*ceil(hd/32) programs; here every (lane-block, tile) is one workgroup
// and tiles are chained by the single-pass look-back of osm_chain.h.
//
// Per workgroup (512 threads; tile of G::TILE tokens x 64 lanes):
//   1. load x (and g, coefficients) through buffer descriptors;
//   2. pass 1: w = (1-lam) * tanh(damping * p(u)) in registers, serial EMA
//      from 0 over each thread's run -> run aggregate (A, B);
//   3. token-group scan in LDS -> tile aggregate, published;
//   4. look-back -> carry-in;
//   5. pass 2: replay s = lam*s + w from the carry, store out.
// All tensor traffic uses buffer descriptors (osm_device.h): no per-element
// address arithmetic and no bounds branches.
#include <type_traits>

#include "osm_tile.h"

namespace osm {
namespace {

// lambda of the tokens of a thread's run: lam[r] for r < R.  Static: the
// head's lambda.  Dynamic: a row of the tile's per-token lambda in LDS
// (formed once per token and head by the workgroup, see the kernel).
template <bool DYN>
struct RunLam;
template <>
struct RunLam<false> {
  float lam;
  __device__ __forceinline__ float operator[](int) const { return lam; }
};
template <>
struct RunLam<true> {
  const float* row;   // 16-byte aligned
  // four tokens per LDS read (the reads of one quad are shared after unrolling)
  __device__ __forceinline__ float operator[](int r) const {
    return reinterpret_cast<const f32x4*>(row)[r >> 2][r & 3];
  }
};

// Exact input for the rare path (see pass1_exact): +-Inf -> u = +-1; NaN x
// -> w = 0 as sdpc_kernel.py:2086, or (nan_zero_u) u = 0 as
// sdpc_kernel.py:1725.
template <int KP>
__device__ __forceinline__ float ema_input_exact(float x, const float (&a)[KP], float one_m, float neg2_one_m,
                                                 bool nan_zero_u, bool cheb) {
  const bool ok = x == x;
  const float u = ok ? softsign(x) : 0.0f;
  // both forms, then a select: a branch per element on the tile's form
  // splits the unrolled rare path into many blocks and costs registers
  float pc = series_as<KP, true>(u, a), pm = series_as<KP, false>(u, a);
  asm volatile("" : "+v"(pc), "+v"(pm));
  const float r = tanh_r(cheb ? pc : pm);
  const float w = __builtin_fmaf(neg2_one_m, r, one_m);
  return (ok || nan_zero_u) ? w : 0.0f;
}

// Rare path: a run whose aggregate is NaN saw a NaN or infinite input (or
// non-finite coefficients).  Reload its x and recompute with the exact
// special-value handling, in the series form of the tile (cheb: Clenshaw).
template <class G, bool DYN, typename XT, int KP>
__device__ __forceinline__ void pass1_exact(float (&w)[G::R][G::LPT], const TileAddr& a, const float (&c)[G::LPT][KP],
                                            const RunLam<DYN>& lamv, float (&Bv)[G::LPT], bool nan_zero_u,
                                            bool cheb) {
#pragma unroll
  for (int i = 0; i < G::LPT; ++i) Bv[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < G::R; ++r) {
    float xv[G::LPT];
    BufVec<XT, G::LPT>::load(a.x, a.vx, (uint32_t)r * a.sx, xv);
    const float lam = lamv[r];
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
#pragma unroll
    for (int i = 0; i < G::LPT; ++i) {
      w[r][i] = ema_input_exact<KP>(xv[i], c[i], one_m, n2, nan_zero_u, cheb);
      Bv[i] = __builtin_fmaf(lam, Bv[i], w[r][i]);
    }
    // one row at a time: the scheduler would otherwise issue every row's
    // reload first and hold them beside w (spills with a dynamic lambda)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Pass 2 over a thread's run: s = lam*s + w from the carried state, out =
// clamp(s, lo, hi).  FINAL: also stores the state at run index r_fin to fin
// (when fin is non-NULL).  NANP: a NaN state is stored as NaN (the clamp,
// v_med3_f32, would return a bound); taken when the carried state is NaN,
// which a look-back wait that gave up leaves (or a NaN ema_init).
template <class G, bool DYN, typename OT, bool FINAL, bool NANP>
__device__ __forceinline__ void pass2(float (&s)[G::LPT], const float (&w)[G::R][G::LPT], const RunLam<DYN>& lamv,
                                      const TileAddr& a, float lo, float hi, int r_fin, float* fin) {
  uint32_t so = 0;
#pragma unroll
  for (int r = 0; r < G::R; ++r) {
    float o[G::LPT];
#pragma unroll
    for (int i = 0; i < G::LPT; ++i) {
      s[i] = __builtin_fmaf(lamv[r], s[i], w[r][i]);
      o[i] = __builtin_amdgcn_fmed3f(s[i], lo, hi);
      if constexpr (NANP) o[i] = s[i] == s[i] ? o[i] : s[i];
    }
    if constexpr (FINAL) {
      if (r == r_fin && fin) {
#pragma unroll
        for (int i = 0; i < G::LPT; ++i) fin[i] = s[i];
      }
    }
    BufVec<OT, G::LPT>::store(a.out, a.vo, so, o);
    so = next_off(so, a.so);
  }
}

// Two workgroups (4 waves per SIMD) per CU: at most 128 VGPRs.
template <class G, bool DYN, typename XT, typename OT, int KP>
__global__ void __launch_bounds__(G::THREADS) __attribute__((amdgpu_waves_per_eu(4)))
cheby_ema_fwd_kernel(const FwdParams p) {
  constexpr int R = G::R;
  constexpr int LPT = G::LPT;
  __shared__ ChainLds<G> L;

  // Highest wave priority until the tile's loads are issued: a workgroup
  // that has just started gets its loads into the memory pipeline ahead of
  // the arithmetic of older workgroups on the CU (measured at BASELINE
  // configs[1] on MI355X: 52.0 against 53.5 us).
  __builtin_amdgcn_s_setprio(3);
  const ThreadPos q = thread_pos<G>();
  const Tags tags = launch_tags(p.hdr);
  const TileInfo ti = tile_info<G>(blockIdx.x, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles);
  if (ti.pad) {
    finish_block(p.hdr, tags.epoch);
    return;
  }
  const TileAddr a = tile_addr<G, DYN, XT, OT>(p, q, ti);

  // Monomial coefficients (loads first, converted after the x loads).
  __shared__ float mono[KP][G::LANES];
  const auto ml = mono_issue<KP, G>(p, q, ti, a);

  const float lam_h = p.lam[a.h];
  // Dynamic lambda: the workgroup loads g for the tile's tokens and the
  // heads its lanes span (one value per token and head, not one per thread)
  // and forms lambda = clamp(lam_h + lam_shift g) once into LDS,
  // lam_s[head - h0][token]; threads read their run's row from there in
  // both passes instead of holding R values in registers.  g and lam_h are
  // loaded before x: forming lambda waits for them, and loads complete in
  // order, so with x issued first that wait was a wait for all of x.
  constexpr int NHB = DYN ? (LPT == 1 ? G::LANES : G::LANES / 4) : 1;   // heads a lane-block can span
  constexpr int kGL = 2;   // g loads per thread held in registers (the rest: a rare loop)
  static_assert(!DYN || (R % 4 == 0 && G::TILE % 4 == 0), "runs read lambda four tokens at a time");
  __shared__ __attribute__((aligned(16))) float lam_s[NHB][DYN ? G::TILE : 1];
  int h0 = 0, n_gl = 0;
  float glv[kGL], lhv[kGL];
  if constexpr (DYN) {
    const int d0 = ti.lbd * G::LANES;
    h0 = div_hd(d0, p);
    n_gl = (div_hd(min(d0 + G::LANES, p.D) - 1, p) - h0 + 1) * G::TILE;
#pragma unroll
    for (int i = 0; i < kGL; ++i) {
      const int idx = q.tid + i * G::THREADS;
      const int t = idx % G::TILE, hh = idx / G::TILE;
      // (each 128-byte line of g, four tokens of every head, is read by all
      // the lane-blocks of the row)
      glv[i] = load_f32_shared(a.g, idx < n_gl ? (uint32_t)((t * p.g_ss + (h0 + hh) * p.g_sh) * 4) : kOffOOB, 0);
      lhv[i] = p.lam[min(h0 + hh, p.H - 1)];   // (idx >= n_gl: not used)
    }
  }

  // x rows of this thread's run.
  float w[R][LPT];
  {
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      BufVec<XT, LPT>::load(a.x, a.vx, so, w[r]);
      so = next_off(so, a.sx);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  __shared__ unsigned mono_big[KP * G::NSUB];
  mono_store<KP, G>(ml, q, mono, mono_big);
  if constexpr (DYN) {
    auto lam_of = [&](int idx, float gv, float lh) {
      const int t = idx % G::TILE, hh = idx / G::TILE;
      lam_s[hh][t] = __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, gv, lh), p.lam_min, p.lam_max);
    };
#pragma unroll
    for (int i = 0; i < kGL; ++i)
      if (q.tid + i * G::THREADS < n_gl) lam_of(q.tid + i * G::THREADS, glv[i], lhv[i]);
    for (int idx = q.tid + kGL * G::THREADS; idx < n_gl; idx += G::THREADS) {   // small heads only
      const int t = idx % G::TILE, hh = idx / G::TILE;
      const float gv = load_f32_shared(a.g, (uint32_t)((t * p.g_ss + (h0 + hh) * p.g_sh) * 4), 0);
      lam_of(idx, gv, p.lam[h0 + hh]);
    }
  }
  __syncthreads();
  // Monomial form unless a coefficient of the tile exceeds kMonoBound (rare:
  // the Chebyshev coefficients replace the table, one more barrier).
  const bool cheb = tile_cheb<KP, G>(mono_big);
  if (KP <= kMonoMaxK && cheb) {
    mono_store_cheb<KP, G>(p, q, ti, a, mono);
    __syncthreads();
  }
  float c[LPT][KP];
  mono_read<G, KP>(mono, q, c);
  RunLam<DYN> lamv;
  if constexpr (DYN)
    lamv.row = &lam_s[min(max(a.h - h0, 0), NHB - 1)][q.tg * R];   // (lanes >= D: any row)
  else
    lamv.lam = lam_h;

  // Pass 1: w = (1 - lam) * tanh(damping * p(u)) in place of x, and the run
  // aggregate (A, B) from a zero state.  softsign as copysign(1 - 1/(1+|x|), x):
  // +-Inf and huge |x| give +-1 (the reciprocal underflows to 0; absolute
  // error of u ~ 6e-8); a NaN x yields a NaN w, so a run containing one is
  // recomputed by pass1_exact.  tanh as 1 - 2/(1 + exp2(y)) with y from the
  // pre-scaled coefficients.  Tokens >= S of the last tile read x = 0 and are
  // processed like the others: they only feed the last tile's own aggregate
  // (never published) and the carries of later, equally padded, token groups.
  float A = 1.0f;
  float Bv[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) Bv[i] = 0.0f;
  // kRB rows at a time, the polynomial steps interleaved across the rows'
  // elements: each Horner step depends on the previous one, so independent
  // chains keep the VALU pipeline busy.
  constexpr int kRB = 2;
  static_assert(R % kRB == 0, "row block");
#pragma unroll
  for (int r0 = 0; r0 < R; r0 += kRB) {
    float u[kRB][LPT], py[kRB][LPT];
#pragma unroll
    for (int rr = 0; rr < kRB; ++rr) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        u[rr][i] = softsign_fast(w[r0 + rr][i]);
        py[rr][i] = c[i][KP - 1];
      }
    }
    if constexpr (KP > kMonoMaxK) {
      // Chebyshev form (more than kMonoMaxK terms): Clenshaw per element.
#pragma unroll
      for (int rr = 0; rr < kRB; ++rr)
#pragma unroll
        for (int i = 0; i < LPT; ++i) py[rr][i] = series<KP>(u[rr][i], c[i]);
    } else {
#pragma unroll
      for (int j = KP - 2; j >= 0; --j)
#pragma unroll
        for (int rr = 0; rr < kRB; ++rr)
#pragma unroll
          for (int i = 0; i < LPT; ++i) py[rr][i] = __builtin_fmaf(py[rr][i], u[rr][i], c[i][j]);
    }
#pragma unroll
    for (int rr = 0; rr < kRB; ++rr) {
      const float lam = lamv[r0 + rr];
      const float one_m = 1.0f - lam;
      const float n2 = -2.0f * one_m;
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        w[r0 + rr][i] = __builtin_fmaf(n2, tanh_r(py[rr][i]), one_m);
        Bv[i] = __builtin_fmaf(lam, Bv[i], w[r0 + rr][i]);
      }
      if constexpr (DYN) A *= lam;
    }
  }
  if constexpr (!DYN) A = pow_n<R>(lam_h);
  bool bad = false;
#pragma unroll
  for (int i = 0; i < LPT; ++i) bad |= Bv[i] != Bv[i];
  // A tile in the Chebyshev form (always above kMonoMaxK coefficients, else
  // rare) redoes the run in the rare path with Clenshaw: with up to
  // kMonoMaxK coefficients the loop above, which then ran Horner on the
  // Chebyshev coefficients, stays the one straight-line pass of the common
  // case.
  if (bad || (KP <= kMonoMaxK && cheb)) pass1_exact<G, DYN, XT, KP>(w, a, c, lamv, Bv, p.nan_zero_u != 0, cheb);
  const unsigned fin_prev = finish_issue(p.hdr, tags.epoch);

  const LaneSlots ls = lane_slots<G, DYN>(p.slots, ti, p.n_tiles);
  float pA, pB[LPT], aggA, aggB;
  jitter(p.jitter, tags.epoch, 0);
  tile_scan<G, DYN>(L, q, ti, tags, A, Bv, pA, pB, aggA, aggB, ls);
  {
    const int dc = ti.lbd * G::LANES + carry_lane<G>(q);
    const float init_c = (p.ema_init && q.wave < G::NSUB && dc < p.D) ? p.ema_init[(int64_t)ti.b * p.D + dc] : 0.0f;
    // static lambda: the tile's decay as the look-back recomputes it
    if constexpr (!DYN)
      if (q.wave < G::NSUB) aggA = static_tile_A<G>(p.lam[dc < p.D ? div_hd(dc, p) : 0]);
    const int dlk = ti.lbd * G::LANES + look_lane<G>(q);
    const float a_look = DYN ? 0.0f : static_tile_A<G>(p.lam[dlk < p.D ? div_hd(dlk, p) : 0]);
    LookBack<G, DYN> lbk;
    look_back_issue<G, DYN>(lbk, q, ti, ls);
    jitter(p.jitter, tags.epoch, 1);
    look_back_finish<G, DYN>(lbk, L, q, ti, tags, aggA, aggB, ls, init_c, a_look, p.hdr, p.poll_limit);
  }
  finish_complete(p.hdr, tags.epoch, fin_prev);

  // Pass 2: replay the recurrence from the true carry and store out.
  float s[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) s[i] = __builtin_fmaf(pA, L.carry[q.lt * LPT + i], pB[i]);
  const float lo = p.clamp_out ? -1.0f : -__builtin_inff();
  const float hi = p.clamp_out ? 1.0f : __builtin_inff();
  bool nan_s = false;
#pragma unroll
  for (int i = 0; i < LPT; ++i) nan_s |= s[i] != s[i];
  if (!ti.is_last) {
    if (!nan_s)
      pass2<G, DYN, OT, false, false>(s, w, lamv, a, lo, hi, 0, nullptr);
    else
      pass2<G, DYN, OT, false, true>(s, w, lamv, a, lo, hi, 0, nullptr);
  } else {
    // The last tile also yields ema_final: the unclamped state at token S-1,
    // from the one run that holds it.
    const int r_last = p.S - 1 - (ti.tile * G::TILE + q.tg * R);
    float* fin = (p.ema_final && a.vo != kOffOOB && r_last >= 0 && r_last < R)
                     ? p.ema_final + (int64_t)ti.b * p.D + ti.lbd * G::LANES + q.lt * LPT
                     : nullptr;
    pass2<G, DYN, OT, true, true>(s, w, lamv, a, lo, hi, r_last, fin);
  }
}

template <class G, bool DYN, typename XT, typename OT>
hipError_t launch_g(const FwdParams& p, int kpad, hipStream_t stream) {
  const unsigned grid = (unsigned)p.n_lb_pad * (unsigned)p.n_tiles;
  if (kpad == 4)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<G, DYN, XT, OT, 4>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  else if (kpad == 8)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<G, DYN, XT, OT, 8>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// The one-lane geometry also serves the Chebyshev form (kpad 16 and 32);
// K <= 4 runs with kpad 8 there (zero coefficients), one instantiation fewer.
template <bool DYN, typename XT, typename OT>
hipError_t launch_generic(const FwdParams& p, int kpad, hipStream_t stream) {
  using G = FwdTileGeneric;
  const unsigned grid = (unsigned)p.n_lb_pad * (unsigned)p.n_tiles;
  if (kpad <= 8)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<G, DYN, XT, OT, 8>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  else if (kpad == 16)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<G, DYN, XT, OT, 16>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  else if (kpad == 32)
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<G, DYN, XT, OT, 32>), dim3(grid), dim3(G::THREADS), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <class G>
bool is_shape(FwdShape s) {
  return s.tile == G::TILE && s.lanes == G::LANES && s.lpt == G::LPT;
}

template <bool DYN, typename XT, typename OT>
hipError_t launch_k(const FwdParams& p, FwdShape s, int kpad, hipStream_t stream) {
  if (is_shape<FwdTileGeneric>(s)) return launch_generic<DYN, XT, OT>(p, kpad, stream);
  if constexpr (!DYN) {
    if (is_shape<FwdTileLarge>(s)) return launch_g<FwdTileLarge, DYN, XT, OT>(p, kpad, stream);
  } else {
    if (is_shape<FwdTileLargeDyn>(s)) return launch_g<FwdTileLargeDyn, DYN, XT, OT>(p, kpad, stream);
  }
  if (is_shape<FwdTileMedium>(s)) return launch_g<FwdTileMedium, DYN, XT, OT>(p, kpad, stream);
  if (is_shape<FwdTileSmall>(s)) return launch_g<FwdTileSmall, DYN, XT, OT>(p, kpad, stream);
  return hipErrorInvalidValue;
}

template <bool DYN>
hipError_t launch_dt(const FwdParams& p, int x_dtype, int out_dtype, FwdShape s, int kpad, hipStream_t stream) {
  if (x_dtype == 0 && out_dtype == 0) return launch_k<DYN, float, float>(p, s, kpad, stream);
  if (x_dtype == 0 && out_dtype == 1) return launch_k<DYN, float, __bf16>(p, s, kpad, stream);
  if (x_dtype == 1 && out_dtype == 0) return launch_k<DYN, __bf16, float>(p, s, kpad, stream);
  return launch_k<DYN, __bf16, __bf16>(p, s, kpad, stream);
}

// Grid-stride zero fill (graph-capturable, unlike hipMemsetAsync nodes).
__global__ void fill_zero_kernel(unsigned* p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Header status: dst[0] = fault word, dst[1] = launch epoch; the fault word
// is cleared afterwards when `reset` (one thread: the read and the clear are
// ordered by program order on one address).
__global__ void ws_status_kernel(unsigned* hdr, unsigned* dst, int reset) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const unsigned fault = __hip_atomic_load(hdr + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned epoch = __hip_atomic_load(hdr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    dst[0] = fault;
    dst[1] = epoch;
    if (reset) __hip_atomic_store(hdr + 3, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ void copy_state_kernel(const float* src, float* dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace

FwdShape fwd_geometry(bool dyn, int64_t B, int64_t D, int64_t S, bool generic) {
  if (generic) return {FwdTileGeneric::TILE, FwdTileGeneric::LANES, FwdTileGeneric::LPT};
  // The largest tile that still leaves >= kMinTiles workgroups with work (2
  // per CU on a 256-CU MI355X, the residency of the large tile); dynamic
  // lambda holds more per-token state and is limited to the medium tile.
  constexpr int64_t kMinTiles = 512;
  auto n_work = [&](int tile, int lanes) { return B * ((D + lanes - 1) / lanes) * ((S + tile - 1) / tile); };
  static_assert(FwdTileLarge::TILE == FwdTileLargeDyn::TILE && FwdTileLarge::LANES == FwdTileLargeDyn::LANES &&
                    FwdTileLarge::LPT == FwdTileLargeDyn::LPT,
                "the static and dynamic large tiles share a shape");
  if (n_work(FwdTileLarge::TILE, FwdTileLarge::LANES) >= kMinTiles)
    return {FwdTileLarge::TILE, FwdTileLarge::LANES, FwdTileLarge::LPT};
  if (n_work(FwdTileMedium::TILE, FwdTileMedium::LANES) >= kMinTiles)
    return {FwdTileMedium::TILE, FwdTileMedium::LANES, FwdTileMedium::LPT};
  return {FwdTileSmall::TILE, FwdTileSmall::LANES, FwdTileSmall::LPT};
}

size_t slot_words(bool dyn) { return dyn ? 2 : 1; }

size_t fwd_workspace_bytes(int n_lb, int n_tiles, int lanes, bool dyn) {
  return kHeaderBytes + (size_t)n_lb * (size_t)n_tiles * (size_t)lanes * slot_words(dyn) * 8;
}

hipError_t launch_fwd(const FwdParams& p, int x_dtype, int out_dtype, bool dyn, FwdShape shape, int kpad,
                      hipStream_t stream) {
  return dyn ? launch_dt<true>(p, x_dtype, out_dtype, shape, kpad, stream)
             : launch_dt<false>(p, x_dtype, out_dtype, shape, kpad, stream);
}

hipError_t launch_fill_zero(void* ptr, size_t bytes, hipStream_t stream) {
  const size_t words = bytes / 4;
  if (words == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((words + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<unsigned*>(ptr), words);
  return hipGetLastError();
}

hipError_t launch_ws_status(void* ws, unsigned* dst, int reset, hipStream_t stream) {
  hipLaunchKernelGGL(ws_status_kernel, dim3(1), dim3(64), 0, stream, static_cast<unsigned*>(ws), dst, reset);
  return hipGetLastError();
}

hipError_t launch_copy_state(const float* src, float* dst, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(copy_state_kernel, dim3(blocks), dim3(256), 0, stream, src, dst, n);
  return hipGetLastError();
}

}  // namespace osm
