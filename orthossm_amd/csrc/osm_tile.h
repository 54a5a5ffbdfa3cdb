// Per-tile addressing and coefficient set-up shared by the forward and TTT
// kernels: buffer descriptors rebased on the tile, the thread's lane offsets,
// and the monomial form of each lane's Chebyshev series.
#pragma once

#include "osm_chain.h"

namespace osm {

// Descriptors of one tile and this thread's offsets into them.
struct TileAddr {
  Rsrc x, out, g, c;
  uint32_t vx, vo, vg;       // per-thread byte offsets (kOffOOB: lanes >= D)
  uint32_t sx, so, sg, sc;   // uniform byte steps: one token (x, out, g), one k (coeffs)
  int h;                     // head of the thread's lanes
};

// x, out (and g) descriptors start at the tile's first row and end after row
// S-1: rows past the sequence read 0 and their stores are dropped, and rows
// after the tile (still < S) can be read through the same descriptor.
// n / hd for 0 <= n < 2^31 (the multiplier and shift come from the host).
__device__ __forceinline__ int div_hd(int n, const FwdParams& p) {
  return (int)((__umulhi((uint32_t)n, p.hd_magic) + (uint32_t)n) >> p.hd_shift);
}

template <class G, bool DYN, typename XT, typename OT>
__device__ __forceinline__ TileAddr tile_addr(const FwdParams& p, const ThreadPos& q, const TileInfo& ti) {
  TileAddr a;
  const int t_tile = ti.tile * G::TILE;
  const int d0 = ti.lbd * G::LANES + q.lt * G::LPT;
  const bool lane_ok = d0 < p.D;
  const uint64_t rows_after = (uint64_t)(p.S - 1 - t_tile);
  a.h = lane_ok ? div_hd(d0, p) : 0;
  const int64_t row0 = (int64_t)q.tg * G::R;
  const char* xb = static_cast<const char*>(p.x) + ((int64_t)ti.b * p.x_sb + (int64_t)t_tile * p.x_ss) * sizeof(XT);
  a.x = make_rsrc(xb, (rows_after * p.x_ss + p.D) * sizeof(XT));
  a.sx = (uint32_t)(p.x_ss * sizeof(XT));
  a.vx = lane_ok ? (uint32_t)((row0 * p.x_ss + d0) * sizeof(XT)) : kOffOOB;
  char* ob = static_cast<char*>(p.out) + ((int64_t)ti.b * p.o_sb + (int64_t)t_tile * p.o_ss) * sizeof(OT);
  a.out = make_rsrc(ob, (rows_after * p.o_ss + p.D) * sizeof(OT));
  a.so = (uint32_t)(p.o_ss * sizeof(OT));
  a.vo = lane_ok ? (uint32_t)((row0 * p.o_ss + d0) * sizeof(OT)) : kOffOOB;
  if constexpr (DYN) {
    const char* gb = reinterpret_cast<const char*>(p.g) + ((int64_t)ti.b * p.g_sb + (int64_t)t_tile * p.g_ss) * 4;
    a.g = make_rsrc(gb, (rows_after * p.g_ss + (uint64_t)(p.H - 1) * p.g_sh + 1) * 4);
    a.sg = (uint32_t)(p.g_ss * 4);
    a.vg = (uint32_t)((row0 * p.g_ss + (int64_t)a.h * p.g_sh) * 4);
  }
  const char* cb = reinterpret_cast<const char*>(p.coeffs) + (int64_t)ti.b * p.c_sb * 4;
  a.c = make_rsrc(cb, kMaxExtent);
  a.sc = (uint32_t)(p.c_sk * 4);
  return a;
}

// Advances a uniform byte offset by `step` in a way the compiler cannot fold:
// otherwise every r * step product is materialised in its own SGPR.
__device__ __forceinline__ uint32_t next_off(uint32_t off, uint32_t step) {
  off += step;
  asm volatile("" : "+s"(off));
  return off;
}

// Coefficients of the series for the tile's lanes, scaled by
// 2*log2(e)*damping (the tanh argument in exp2 units): the monomial form for
// KP <= kMonoMaxK, the Chebyshev coefficients themselves above (evaluated by
// Clenshaw, see series()).  The work is split in units (coefficient j,
// 64-lane sub-block sb); wave w takes units w, w + WAVES, ... and forms
// coefficient j of its 64 lanes from <= 4 Chebyshev coefficients
// (cheb_mono) in float64 (monomial form) or scales c_j (Chebyshev form);
// results are shared through LDS.
// Split in three steps so the caller can issue these loads before its bulk
// loads (the conversion then waits only for them) and convert after issuing
// those:
//   auto m = mono_issue(...);  <bulk loads>;  mono_store(m, ...);
//   __syncthreads();  mono_read(...)
template <int KP, class G>
struct MonoLoad {
  static constexpr int NU = KP * G::NSUB;                   // units
  static constexpr int NJ = (NU + G::WAVES - 1) / G::WAVES;  // units per wave
  static constexpr int NT = KP > kMonoMaxK ? 1 : 4;          // coefficients read per unit
  float cm[NJ][NT];
  float kap[NJ];
  int w;   // wave index (wave-uniform)
};

template <int KP, class G>
__device__ __forceinline__ MonoLoad<KP, G> mono_issue(const FwdParams& p, const ThreadPos& q, const TileInfo& ti,
                                                      const TileAddr& a) {
  MonoLoad<KP, G> m;
  m.w = __builtin_amdgcn_readfirstlane(q.wave);
#pragma unroll
  for (int n = 0; n < m.NJ; ++n) {
    const int u = m.w + n * G::WAVES;
    const int j = u / G::NSUB;
    const int d = ti.lbd * G::LANES + (u % G::NSUB) * kLanes + q.wl;
    const bool ok = u < m.NU && d < p.D;
    const int h = ok ? div_hd(d, p) : 0;
    const uint32_t vc = ok ? (uint32_t)(((int64_t)h * p.c_sh + (d - h * p.hd)) * 4) : kOffOOB;
#pragma unroll
    for (int i = 0; i < m.NT; ++i) {
      // Unconditional loads (an unused unit or k >= K reads 0 through the
      // out-of-range offset): a branch here would make the compiler convert
      // each value inside it and so wait for every load on the spot, before
      // the caller's bulk loads are issued.
      // (every tile of the lane-block, all on one XCD, reads them)
      const int k = j + 2 * i;
      m.cm[n][i] = load_f32_shared(a.c, k < p.K ? vc : kOffOOB, (uint32_t)k * a.sc);
    }
    m.kap[n] = kTwoLog2e * p.damping[h];
  }
  return m;
}

// Which form a tile evaluates its series in.  The monomial form (Horner, K-1
// FMAs) is exact in exact arithmetic, but its coefficients cancel: its fp32
// error grows with sum_j |a_j| (a_j scaled as stored, in exp2 units), about
// ten times faster than Clenshaw's with the size of the Chebyshev
// coefficients.  A tile uses the monomial form while every scaled monomial
// coefficient of its lanes satisfies |a_j| <= kMonoBound (NaN counts as
// above), else the Chebyshev form (Clenshaw, 2(K-1) operations) on c_k
// scaled the same way.  The bound keeps every draw of the benchmark's
// c_k ~ N(0, 1/(k+1)^2) (largest |a_j|, a_5 = 2 log2(e) (16 c_5 - 112 c_7),
// has a standard deviation of 41) and every coefficient set inside the
// full path's Lion bound 8.31/(k+1)^1.5 (|a_5| <= 145) on Horner, and
// sends coefficients of order one and larger (c_k ~ N(0, 1): |a_5| ~ 330)
// to Clenshaw.
constexpr float kMonoBound = 256.0f;

// mono_store writes coefficient j of every unit; with KP <= kMonoMaxK it
// also writes, per unit, whether one of its 64 values exceeds kMonoBound
// (`big`, one word per unit, read after the next barrier by tile_cheb).
template <int KP, class G>
__device__ __forceinline__ void mono_store(const MonoLoad<KP, G>& m, const ThreadPos& q,
                                           float (&mono)[KP][G::LANES], unsigned (&big)[KP * G::NSUB]) {
#pragma unroll
  for (int n = 0; n < m.NJ; ++n) {
    const int u = m.w + n * G::WAVES;
    if (u < m.NU) {
      const int j = u / G::NSUB;
      double acc = 0.0;
      if constexpr (KP > kMonoMaxK) {
        acc = (double)m.cm[n][0];
      } else {
        // j is wave-uniform: a scalar branch to the constants of coefficient j
        switch (j) {
          case 0: acc = mono_coef<0>(m.cm[n]); break;
          case 1: acc = mono_coef<1>(m.cm[n]); break;
          case 2: acc = mono_coef<2>(m.cm[n]); break;
          case 3: acc = mono_coef<3>(m.cm[n]); break;
          case 4: acc = mono_coef<4>(m.cm[n]); break;
          case 5: acc = mono_coef<5>(m.cm[n]); break;
          case 6: acc = mono_coef<6>(m.cm[n]); break;
          default: acc = mono_coef<7>(m.cm[n]); break;
        }
      }
      const float v = (float)(acc * (double)m.kap[n]);
      mono[j][(u % G::NSUB) * kLanes + q.wl] = v;
      if constexpr (KP <= kMonoMaxK) {
        const bool over = __ballot(!(__builtin_fabsf(v) <= kMonoBound)) != 0;
        if (q.wl == 0) big[u] = over ? 1u : 0u;
      }
    }
  }
}

// True when the tile evaluates the Chebyshev form (uniform over the tile):
// always above kMonoMaxK coefficients, else when a unit's flag is set.
template <int KP, class G>
__device__ __forceinline__ bool tile_cheb(const unsigned (&big)[KP * G::NSUB]) {
  if constexpr (KP > kMonoMaxK) return true;
  unsigned f = 0;
#pragma unroll
  for (int u = 0; u < KP * G::NSUB; ++u) f |= big[u];
  return __builtin_amdgcn_readfirstlane(f) != 0;
}

// The Chebyshev form of a tile's coefficients in place of the monomial one
// (tiles that tile_cheb sends to Clenshaw): unit (j, sub-block) holds
// c_j times 2 log2(e) damping_h, rounded once, as mono_store forms it above
// kMonoMaxK coefficients.  Loads c_j again (a rare path); the caller orders
// the writes before mono_read with a barrier.
template <int KP, class G>
__device__ __forceinline__ void mono_store_cheb(const FwdParams& p, const ThreadPos& q, const TileInfo& ti,
                                                const TileAddr& a, float (&mono)[KP][G::LANES]) {
  constexpr int NU = KP * G::NSUB;
  const int w = __builtin_amdgcn_readfirstlane(q.wave);
  for (int u = w; u < NU; u += G::WAVES) {
    const int j = u / G::NSUB;
    const int d = ti.lbd * G::LANES + (u % G::NSUB) * kLanes + q.wl;
    const bool ok = d < p.D;
    const int h = ok ? div_hd(d, p) : 0;
    const uint32_t vc = ok && j < p.K ? (uint32_t)(((int64_t)h * p.c_sh + (d - h * p.hd)) * 4) : kOffOOB;
    float v[1];
    BufVec<float, 1>::load(a.c, vc, (uint32_t)j * a.sc, v);
    mono[j][(u % G::NSUB) * kLanes + q.wl] = (float)((double)v[0] * (double)(kTwoLog2e * p.damping[h]));
  }
}

template <class G, int KP>
__device__ __forceinline__ void mono_read(const float (&mono)[KP][G::LANES], const ThreadPos& q,
                                          float (&c)[G::LPT][KP]) {
#pragma unroll
  for (int j = 0; j < KP; ++j)
#pragma unroll
    for (int i = 0; i < G::LPT; ++i) c[i][j] = mono[j][q.lt * G::LPT + i];
}

// Fast softsign copysign(1 - 1/(1 + |x|), x): +-Inf and huge |x| give +-1
// (the reciprocal underflows to 0); absolute error ~6e-8; NaN stays NaN.
__device__ __forceinline__ float softsign_fast(float x) {
  return __builtin_copysignf(1.0f - __builtin_amdgcn_rcpf(1.0f + __builtin_fabsf(x)), x);
}

}  // namespace osm
