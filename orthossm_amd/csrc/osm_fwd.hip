// Fused Cheby-RKV forward for gfx950: softsign -> Clenshaw -> damping ->
// tanh -> EMA scan, one pass over HBM (x read once, out written once).
//
// Reference counterpart: the forward part of _ortho_megakernel
// (sdpc_kernel.py:2006-2124) and _fused_clenshaw_ema_kernel
// (sdpc_kernel.py:988-1209).  The reference walks S serially inside each of
// B*H*ceil(hd/32) programs; here tiles of 256 tokens x 64 lanes are spread
// over persistent workgroups and chained by the single-pass look-back of
// osm_chain.h.
//
// Each workgroup (FwdGeoT: 512 threads) loops over tiles of its class, with
// the next tile's x, g and coefficients loaded while the current tile is
// processed:
//   1. pass 1 on the prefetched tile: w = (1-lam) * tanh(damping * p(u)) in
//      registers; serial EMA from 0 over each thread's run -> (A, B);
//   2. token-group scan in LDS -> tile aggregate, published;
//   3. look-back loads issued, then the next tile's loads issued (vector
//      memory counters retire in order, so the look-back wait does not wait
//      for the prefetch);
//   4. carry-in resolved; replay s = lam*s + w from it, store out.
// All tensor traffic uses buffer descriptors (osm_device.h): no per-element
// address arithmetic, no bounds branches.
#include <stdlib.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "osm_chain.h"

namespace osm {
namespace {

template <bool DYN>
using Geo = FwdGeoT<DYN>;

// Fast path: w = (1 - lam) * tanh(damping * p) with c pre-scaled by
// 2*log2(e)*damping.  softsign as copysign(1 - 1/(1 + |x|), x): +-Inf and
// huge |x| give +-1 (the reciprocal underflows to 0), and a NaN x yields a
// NaN w, so runs containing one are recomputed by ema_input_exact
// (NaN x -> w = 0 as sdpc_kernel.py:2086).  Absolute error of u ~ 6e-8.
template <int KP>
__device__ __forceinline__ float ema_input_fast(float x, const float* c, float one_m, float neg2_one_m) {
  const float u = __builtin_copysignf(1.0f - __builtin_amdgcn_rcpf(1.0f + __builtin_fabsf(x)), x);
  const float r = tanh_r(clenshaw<KP>(u, c));
  return __builtin_fmaf(neg2_one_m, r, one_m);
}

template <int KP>
__device__ __forceinline__ float ema_input_exact(float x, const float* c, float one_m, float neg2_one_m) {
  const float r = tanh_r(clenshaw<KP>(softsign(x), c));
  const float w = __builtin_fmaf(neg2_one_m, r, one_m);
  return (x == x) ? w : 0.0f;
}

// Descriptors of one tile and this thread's offsets into them.
template <bool DYN, typename XT, typename OT>
struct TileAddr {
  Rsrc x, out, g, c;
  uint32_t vx, vo, vg, vc;   // per-thread byte offsets (kOffOOB: lanes >= D)
  uint32_t sx, so, sg, sc;   // uniform byte steps: one token (x, out, g), one k (coeffs)
  int h;
};

template <bool DYN, typename XT, typename OT>
__device__ __forceinline__ TileAddr<DYN, XT, OT> tile_addr(const FwdParams& p, const ThreadPos& q,
                                                           const TileInfo& ti) {
  TileAddr<DYN, XT, OT> a;
  const int t_tile = ti.tile * Geo<DYN>::TILE;
  const int d0 = ti.lbd * kLanes + q.lt * Geo<DYN>::LPT;
  const bool lane_ok = d0 < p.D;
  const uint64_t rows_after = (uint64_t)(p.S - 1 - t_tile);
  a.h = lane_ok ? d0 / p.hd : 0;
  const int j0 = d0 - a.h * p.hd;
  const int64_t row0 = (int64_t)q.tg * Geo<DYN>::R;
  // x and out: the extent ends after row S-1, so padding rows read 0 and
  // their stores are dropped.
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
  a.vc = lane_ok ? (uint32_t)(((int64_t)a.h * p.c_sh + j0) * 4) : kOffOOB;
  return a;
}

// Registers holding one tile's inputs for this thread.
template <bool DYN, int KP>
struct TileInputs {
  float x[Geo<DYN>::R][Geo<DYN>::LPT];
  float g[DYN ? Geo<DYN>::R : 1];
  float c[Geo<DYN>::LPT][KP];   // raw coefficients (0 beyond K and for lanes >= D)
  float lam, damp;
};

// Advances a uniform byte offset by `step` in a way the compiler cannot fold:
// otherwise every r * step product is hoisted out of the tile loop and held
// in its own SGPR for the whole kernel.
__device__ __forceinline__ uint32_t next_off(uint32_t off, uint32_t step) {
  off += step;
  asm volatile("" : "+s"(off));
  return off;
}

template <bool DYN, typename XT, typename OT, int KP>
__device__ __forceinline__ void load_tile(TileInputs<DYN, KP>& in, const FwdParams& p,
                                          const TileAddr<DYN, XT, OT>& a) {
  uint32_t so = 0;
#pragma unroll
  for (int r = 0; r < Geo<DYN>::R; ++r) {
    BufVec<XT, Geo<DYN>::LPT>::load(a.x, a.vx, so, in.x[r]);
    so = next_off(so, a.sx);
  }
  if constexpr (DYN) {
    uint32_t sg = 0;
#pragma unroll
    for (int r = 0; r < Geo<DYN>::R; ++r) {
      float gv[1];
      BufVec<float, 1>::load(a.g, a.vg, sg, gv);
      in.g[r] = gv[0];
      sg = next_off(sg, a.sg);
    }
  }
  uint32_t sc = 0;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    float cv[Geo<DYN>::LPT];
    if (k < p.K) {
      BufVec<float, Geo<DYN>::LPT>::load(a.c, a.vc, sc, cv);
      sc = next_off(sc, a.sc);
    } else {
#pragma unroll
      for (int i = 0; i < Geo<DYN>::LPT; ++i) cv[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < Geo<DYN>::LPT; ++i) in.c[i][k] = cv[i];
  }
  in.lam = p.lam[a.h];
  in.damp = p.damping[a.h];
}

// Pass 1 over this thread's run: w (in place of x) and the run aggregate.
// Tokens >= S in the last tile read x = 0 and are processed like the others:
// they only feed the last tile's own aggregate (never published) and the
// carries of later, equally padded, token groups, whose stores are dropped.
template <bool DYN, int KP>
__device__ __forceinline__ void pass1(TileInputs<DYN, KP>& in, const FwdParams& p, const float (&c)[Geo<DYN>::LPT][KP],
                                      float (&lamv)[DYN ? Geo<DYN>::R : 1], float& A, float (&Bv)[Geo<DYN>::LPT]) {
  A = 1.0f;
#pragma unroll
  for (int i = 0; i < Geo<DYN>::LPT; ++i) Bv[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < Geo<DYN>::R; ++r) {
    float lam = in.lam;
    if constexpr (DYN) {
      lam = __builtin_amdgcn_fmed3f(__builtin_fmaf(p.lam_shift, in.g[r], in.lam), p.lam_min, p.lam_max);
      lamv[r] = lam;
    }
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
#pragma unroll
    for (int i = 0; i < Geo<DYN>::LPT; ++i) {
      const float w = ema_input_fast<KP>(in.x[r][i], c[i], one_m, n2);
      in.x[r][i] = w;
      Bv[i] = __builtin_fmaf(lam, Bv[i], w);
    }
    A *= lam;
  }
}

// Rare path: a run whose aggregate is NaN saw a NaN or infinite input (or
// non-finite coefficients).  Reload its x and recompute with the exact
// special-value handling.
template <bool DYN, typename XT, typename OT, int KP>
__device__ __forceinline__ void pass1_exact(TileInputs<DYN, KP>& in, const FwdParams& p, const TileAddr<DYN, XT, OT>& a,
                                         const float (&c)[Geo<DYN>::LPT][KP], const float (&lamv)[DYN ? Geo<DYN>::R : 1],
                                         float (&Bv)[Geo<DYN>::LPT]) {
#pragma unroll
  for (int i = 0; i < Geo<DYN>::LPT; ++i) Bv[i] = 0.0f;
  for (int r = 0; r < Geo<DYN>::R; ++r) {
    float xv[Geo<DYN>::LPT];
    BufVec<XT, Geo<DYN>::LPT>::load(a.x, a.vx, (uint32_t)r * a.sx, xv);
    const float lam = DYN ? lamv[r] : in.lam;
    const float one_m = 1.0f - lam;
    const float n2 = -2.0f * one_m;
#pragma unroll
    for (int i = 0; i < Geo<DYN>::LPT; ++i) {
      const float w = ema_input_exact<KP>(xv[i], c[i], one_m, n2);
      in.x[r][i] = w;
      Bv[i] = __builtin_fmaf(lam, Bv[i], w);
    }
  }
}

// PERSIST: persistent blocks taking tiles by class tickets, with the next
// tile prefetched; otherwise one tile per block (v = blockIdx.x).
template <bool DYN, typename XT, typename OT, int KP, bool PERSIST>
__global__ void __launch_bounds__(Geo<DYN>::THREADS) cheby_ema_fwd_kernel(const FwdParams p) {
  using G = Geo<DYN>;
  constexpr int R = Geo<DYN>::R;
  constexpr int LPT = Geo<DYN>::LPT;
  constexpr int WORDS = DYN ? 2 : 1;
  __shared__ ChainLds<G> L;

  const ThreadPos q = thread_pos<G>();
  const Tags tags = launch_tags(p.hdr);
  const int cls = blockIdx.x & 7;
  const int n_virt = p.n_lb_pad * p.n_tiles;

  int v;
  if constexpr (PERSIST) {
    if (q.tid == 0) L.next_v = ticket_to_tile(take_ticket(p.hdr, cls), cls, p.n_lb, p.n_lb_pad, p.n_tiles);
    __syncthreads();
    v = L.next_v;
    __syncthreads();  // everyone has read next_v before thread 0 rewrites it
  } else {
    v = blockIdx.x;
    if (v % p.n_lb_pad >= p.n_lb) v = n_virt;  // padding block: nothing to do
  }

  TileInputs<DYN, KP> in;
  TileAddr<DYN, XT, OT> a;
  if (v < n_virt) {
    a = tile_addr<DYN, XT, OT>(p, q, tile_info(v, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles));
    load_tile<DYN, XT, OT, KP>(in, p, a);
  }

  while (v < n_virt) {
    const TileInfo ti = tile_info(v, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles);
    const TileAddr<DYN, XT, OT> cur = a;
    unsigned pending = 0;
    if (PERSIST && q.tid == 0) pending = take_ticket(p.hdr, cls);   // waited for only after pass 1

    // Pass 1.
    const float lam_h = in.lam;
    float lamv[DYN ? R : 1];
    float A, Bv[LPT];
    float c[LPT][KP];
    {
      const float kap = kTwoLog2e * in.damp;
#pragma unroll
      for (int i = 0; i < LPT; ++i)
#pragma unroll
        for (int k = 0; k < KP; ++k) c[i][k] = kap * in.c[i][k];
    }
    pass1<DYN, KP>(in, p, c, lamv, A, Bv);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < LPT; ++i) bad |= Bv[i] != Bv[i];
    if (bad) pass1_exact<DYN, XT, OT, KP>(in, p, cur, c, lamv, Bv);
    if (PERSIST && q.tid == 0) L.next_v = ticket_to_tile(pending, cls, p.n_lb, p.n_lb_pad, p.n_tiles);

    unsigned long long* lane_slots = p.slots + ((size_t)ti.lb * p.n_tiles * kLanes + q.wl) * WORDS;
    const size_t tile_stride = (size_t)kLanes * WORDS;
    float pA, pB[LPT], aggA, aggB;
    tile_scan<G, DYN>(L, q, ti, tags, A, Bv, pA, pB, aggA, aggB, lane_slots, tile_stride);
    const int vn = PERSIST ? L.next_v : n_virt;

    const int dl = ti.lbd * kLanes + q.wl;
    const bool dl_ok = dl < p.D;
    const float init_wl = (p.ema_init && dl_ok) ? p.ema_init[(int64_t)ti.b * p.D + dl] : 0.0f;
    const float lam_wl = DYN ? 0.0f : p.lam[dl_ok ? dl / p.hd : 0];
    LookBack<G, DYN> lbk;
    look_back_issue<G, DYN>(lbk, q, ti, lane_slots, tile_stride);
    // Move the current tile's w out of the prefetch registers, then prefetch.
    float w[R][LPT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < LPT; ++i) w[r][i] = in.x[r][i];
    if (PERSIST && vn < n_virt) {
      a = tile_addr<DYN, XT, OT>(p, q, tile_info(vn, p.n_lb, p.n_lb_pad, p.n_lbd, p.n_tiles));
      load_tile<DYN, XT, OT, KP>(in, p, a);
    }
    look_back_finish<G, DYN>(lbk, L, q, ti, tags, aggA, aggB, lane_slots, tile_stride, init_wl, lam_wl, p.hdr);

    // Pass 2: replay the recurrence from the true carry and store out.
    float s[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) s[i] = __builtin_fmaf(pA, L.carry[q.lt * LPT + i], pB[i]);
    const int t0 = ti.tile * Geo<DYN>::TILE + q.tg * R;
    const int r_last = p.S - 1 - t0;   // run index of token S-1 (in range only for one run)
    float s_last[LPT];
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float lam = DYN ? lamv[r] : lam_h;
      float o[LPT];
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        s[i] = __builtin_fmaf(lam, s[i], w[r][i]);
        o[i] = p.clamp_out ? __builtin_amdgcn_fmed3f(s[i], -1.0f, 1.0f) : s[i];
      }
      if (ti.is_last && r == r_last) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) s_last[i] = s[i];
      }
      BufVec<OT, LPT>::store(cur.out, cur.vo, so, o);
      so = next_off(so, cur.so);
    }
    // ema_final = unclamped state at token S-1, from the run that holds it.
    if (ti.is_last && r_last >= 0 && r_last < R && cur.vo != kOffOOB && p.ema_final) {
      const int d0 = ti.lbd * kLanes + q.lt * LPT;
#pragma unroll
      for (int i = 0; i < LPT; ++i) p.ema_final[(int64_t)ti.b * p.D + d0 + i] = s_last[i];
    }
    v = vn;
  }
  finish_block(p.hdr, tags.epoch);
}

// Blocks that can be resident at once for `fn` on the current device.
int resident_blocks(const void* fn, int threads) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t key = ((uint64_t)(uintptr_t)fn << 8) ^ (uint64_t)dev;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess || per_cu < 1) per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
  const int n = per_cu * cus;
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = n;
  return n;
}

// Schedule of the forward kernel: OSM_FWD_SCHEDULE=persistent|oneshot
// (default oneshot).  Both produce identical results.
bool persistent_schedule() {
  static const bool v = [] {
    const char* e = getenv("OSM_FWD_SCHEDULE");
    return e && std::string(e) == "persistent";
  }();
  return v;
}

template <bool DYN, typename XT, typename OT, int KP>
hipError_t launch_one(const FwdParams& p, hipStream_t stream) {
  const int n_virt = p.n_lb_pad * p.n_tiles;
  if (persistent_schedule()) {
    const void* fn = reinterpret_cast<const void*>(&cheby_ema_fwd_kernel<DYN, XT, OT, KP, true>);
    int grid = resident_blocks(fn, Geo<DYN>::THREADS);
    grid = grid < n_virt ? grid : n_virt;
    grid = grid / 8 * 8;
    if (grid < 8) grid = 8;
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<DYN, XT, OT, KP, true>), dim3(grid), dim3(Geo<DYN>::THREADS), 0, stream, p);
  } else {
    hipLaunchKernelGGL((cheby_ema_fwd_kernel<DYN, XT, OT, KP, false>), dim3(n_virt), dim3(Geo<DYN>::THREADS), 0, stream,
                       p);
  }
  return hipGetLastError();
}

template <bool DYN, typename XT, typename OT>
hipError_t launch_k(const FwdParams& p, int kpad, hipStream_t stream) {
  return kpad == 4 ? launch_one<DYN, XT, OT, 4>(p, stream) : launch_one<DYN, XT, OT, 8>(p, stream);
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
  return kHeaderBytes + (size_t)n_lb * (size_t)n_tiles * kLanes * slot_words(dyn) * 8;
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
