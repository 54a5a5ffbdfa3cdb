// Tile chaining protocol shared by the fused kernels: tile assignment, the
// token-group scan inside a tile, and the single-pass checkpointed look-back
// that hands each tile its EMA carry-in.
//
// The EMA s[t] = lam[t] s[t-1] + w[t] composes as affine maps f(s) = A s + B.
// A tile's aggregate is (A, B) = composition over its tokens from a zero
// state.  Tiles are grouped in runs of G::CKPT; the carry into tile t of
// group m is
//     carry = f_{t-1}( ... f_{CKPT m}( C_m ) ... )
// where C_m is the state after tile CKPT m - 1 (the checkpoint, ema_init for
// m = 0).  Every tile publishes its aggregate except the last tile of a
// group, which publishes its inclusive state as the next checkpoint.  The
// composition order is fixed, so results do not depend on timing.
//
// A lane-block is G::LANES consecutive lanes of one batch row (64 or 128);
// the look-back works on 64-lane sub-blocks: sub-block sb is served by waves
// sb*WPS .. sb*WPS+WPS-1, each reading WPT predecessor tiles, so that
// CKPT = WPS * WPT.  Look-back words are laid out [lane-block][tile][lane].
//
// Tile order.  Virtual tile v covers tile v / n_lb_pad of the lane-block in
// slot v % n_lb_pad, with n_lb_pad = n_lb rounded up to a multiple of 8
// (tile_info maps slots to lane-blocks so that consecutive lane-blocks share
// a class; virtual tiles with lane-block >= n_lb are padding and are
// skipped).  A tile waits only on earlier tiles of its lane-block:
// v - k*n_lb_pad, the same slot and class v % 8.  Block b handles v = b.  Awaited blocks have a lower index at a
// stride that is a multiple of 8; workgroups go to the 8 XCDs round-robin by
// index and in index order within an XCD, so each awaited block sits on the
// same XCD and was dispatched before the waiter.  The waits are bounded
// (kSpinLimit), so a broken assumption surfaces as a fault flag, not a hang.
#pragma once

#include "osm_device.h"
#include "osm_kernels.h"

namespace osm {

template <class G>
struct ChainLds {
  float A[G::NTG][G::TPR];      // token-group aggregate A (one per thread)
  float B[G::NTG][G::LANES];    // token-group aggregate B per lane
  float mA[G::WAVES][kLanes];   // look-back partial maps per wave (lane of its sub-block)
  float mB[G::WAVES][kLanes];
  float carry[G::LANES];        // resolved carry-in of the tile
};

struct TileInfo {
  int v, tile, lb, b, lbd;
  bool is_last, is_ckpt;
  bool pad;  // padding tile: no lane-block
};

struct Tags {
  unsigned epoch, agg, pre;
};

// Thread coordinates inside the workgroup: wave, lane in wave (wl), thread in
// its row (lt: lanes lt*LPT .. lt*LPT+LPT-1 of the lane-block) and token
// group (tg).
struct ThreadPos {
  int tid, wave, wl, lt, tg;
};

template <class G>
__device__ __forceinline__ ThreadPos thread_pos() {
  ThreadPos q;
  q.tid = threadIdx.x;
  q.wave = q.tid >> 6;
  q.wl = q.tid & 63;
  q.lt = q.wl % G::TPR;
  q.tg = q.wave * G::TGW + q.wl / G::TPR;
  return q;
}

// Lane (within the lane-block) whose look-back words this thread reads, and
// the lane whose carry it resolves (waves < NSUB only).
template <class G>
__device__ __forceinline__ int look_lane(const ThreadPos& q) {
  return (q.wave / G::WPS) * kLanes + q.wl;
}
template <class G>
__device__ __forceinline__ int carry_lane(const ThreadPos& q) {
  return q.wave * kLanes + q.wl;
}

// Launch epoch: constant for the whole launch (the last block bumps it only
// after every block of this launch has read it).
__device__ __forceinline__ Tags launch_tags(unsigned* hdr_words) {
  Tags t;
  t.epoch = __hip_atomic_load(hdr_words, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  t.agg = make_tag(t.epoch, kKindAgg);
  t.pre = make_tag(t.epoch, kKindPre);
  return t;
}

template <class G>
__device__ __forceinline__ TileInfo tile_info(int v, int n_lb, int n_lb_pad, int n_lbd, int n_tiles) {
  TileInfo ti;
  ti.v = v;
  ti.tile = v / n_lb_pad;
  // Slot s = v mod n_lb_pad (XCD class s mod 8) serves lane-block
  // (s mod 8) * m + s / 8, m = n_lb_pad / 8: the m consecutive lane-blocks
  // c m .. c m + m - 1 all belong to class c, so the lane-blocks of a batch
  // row share one XCD and its L2 (they read the same lines of g, one value
  // per head per token), and every class still holds m lane-blocks.
  const int s = v - ti.tile * n_lb_pad;
  ti.lb = (s & 7) * (n_lb_pad >> 3) + (s >> 3);
  ti.pad = ti.lb >= n_lb;
  ti.b = ti.lb / n_lbd;
  ti.lbd = ti.lb - ti.b * n_lbd;
  ti.is_last = ti.tile == n_tiles - 1;
  ti.is_ckpt = (ti.tile % G::CKPT) == G::CKPT - 1;
  return ti;
}

// Look-back words of one lane-block: [tile][LANES][words].
struct LaneSlots {
  unsigned long long* base;   // tile 0, lane 0 of the lane-block
  size_t tile_stride;         // words per tile
  int words;                  // 1 (B) or 2 (B, A)
  __device__ __forceinline__ unsigned long long* at(int tile, int lane) const {
    return base + (size_t)tile * tile_stride + (size_t)lane * words;
  }
};

template <class G, bool DYN>
__device__ __forceinline__ LaneSlots lane_slots(unsigned long long* slots, const TileInfo& ti, int n_tiles) {
  LaneSlots s;
  s.words = DYN ? 2 : 1;
  s.tile_stride = (size_t)G::LANES * s.words;
  s.base = slots + (size_t)ti.lb * n_tiles * s.tile_stride;
  return s;
}

// Aggregate A of a full tile under a static lambda, lambda^TILE rounded once
// (the producing workgroup publishes only B and uses the same value for its
// checkpoint; an error in A would repeat at every tile of the carry chain).
template <class G>
__device__ __forceinline__ float static_tile_A(float lam) {
  return pow_n<G::TILE>(lam);
}

// Test aid (OSM_FLAG_TIMING_JITTER): the workgroup sleeps 0..15 x ~0.85 us,
// a hash of its index, the launch epoch and `site`, so tiles publish and
// combine in orders the normal schedule rarely produces.  Every wait of the
// look-back is on a word a predecessor publishes without waiting on later
// tiles, so a delay only postpones, and results must not change.
__device__ __forceinline__ void jitter(int on, unsigned epoch, unsigned site) {
  if (!on) return;
  unsigned h = (blockIdx.x * 0x9E3779B1u) ^ (epoch * 0x85EBCA77u) ^ (site * 0xC2B2AE3Du);
  h ^= h >> 15;
  h *= 0x2C1B3C6Du;
  h ^= h >> 12;
  const unsigned n = __builtin_amdgcn_readfirstlane(h & 15u);
  for (unsigned i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(32);
}

// Token-group scan.  In: this thread's run aggregate (A, Bv).  Out: (pA, pB)
// mapping the tile carry to the state before this thread's first token; in
// waves < NSUB, (aggA, aggB) = the tile aggregate of carry_lane(q), which is
// published unless the tile is a checkpoint or the last tile.
template <class G, bool DYN>
__device__ __forceinline__ void tile_scan(ChainLds<G>& L, const ThreadPos& q, const TileInfo& ti, const Tags& tg,
                                          float A, const float (&Bv)[G::LPT], float& pA, float (&pB)[G::LPT],
                                          float& aggA, float& aggB, const LaneSlots& ls) {
  constexpr int LPT = G::LPT;
  L.A[q.tg][q.lt] = A;
#pragma unroll
  for (int i = 0; i < LPT; ++i) L.B[q.tg][q.lt * LPT + i] = Bv[i];
  __syncthreads();
  pA = 1.0f;
#pragma unroll
  for (int i = 0; i < LPT; ++i) pB[i] = 0.0f;
  for (int g = 0; g < q.tg; ++g) {
    const float a = L.A[g][q.lt];
#pragma unroll
    for (int i = 0; i < LPT; ++i) pB[i] = __builtin_fmaf(a, pB[i], L.B[g][q.lt * LPT + i]);
    pA *= a;
  }
  aggA = 1.0f;
  aggB = 0.0f;
  if (q.wave < G::NSUB) {
    const int cl = carry_lane<G>(q);
    for (int g = 0; g < G::NTG; ++g) {
      const float a = L.A[g][cl / LPT];
      aggB = __builtin_fmaf(a, aggB, L.B[g][cl]);
      aggA *= a;
    }
    if (!ti.is_ckpt && !ti.is_last) {
      unsigned long long* mine = ls.at(ti.tile, cl);
      if (DYN) publish(mine + 1, tg.agg, aggA);
      publish(mine, tg.agg, aggB);
    }
  }
}

// Look-back in two halves so that a caller can issue other loads in between:
// look_back_issue reads (without waiting) the words this thread needs;
// look_back_finish waits for the ones not yet published, combines, and
// leaves the carry-in of every lane in L.carry.  Thread (wave, wl) reads
// lane look_lane of WPT predecessor tiles; waves < NSUB also read the
// checkpoint of their carry lane.
template <class G, bool DYN>
struct LookBack {
  unsigned long long vB[G::WPT];
  unsigned long long vA[DYN ? G::WPT : 1];
  unsigned long long vck;
  int beg, end, g0;
};

template <class G, bool DYN>
__device__ __forceinline__ void look_back_issue(LookBack<G, DYN>& st, const ThreadPos& q, const TileInfo& ti,
                                                const LaneSlots& ls) {
  const int ll = look_lane<G>(q);
  st.g0 = (ti.tile / G::CKPT) * G::CKPT;
  st.beg = st.g0 + (q.wave % G::WPS) * G::WPT;
  st.end = min(st.beg + G::WPT, ti.tile);
#pragma unroll
  for (int i = 0; i < G::WPT; ++i) {
    if (st.beg + i < st.end) {
      const unsigned long long* s = ls.at(st.beg + i, ll);
      st.vB[i] = peek(s);
      if constexpr (DYN) st.vA[i] = peek(s + 1);
    }
  }
  st.vck = 0;
  if (q.wave < G::NSUB && st.g0 > 0) st.vck = peek(ls.at(st.g0 - 1, carry_lane<G>(q)));
}

// `a_look` is the full-tile decay static_tile_A of look_lane's static lambda
// (unused when DYN); `init_carry` the initial state of carry_lane (waves <
// NSUB); `limit` the poll limit of await_word.  A wait that gives up yields
// NaN, so the carry (and a checkpoint published from it) is NaN.
template <class G, bool DYN>
__device__ __forceinline__ void look_back_finish(LookBack<G, DYN>& st, ChainLds<G>& L, const ThreadPos& q,
                                                 const TileInfo& ti, const Tags& tg, float aggA, float aggB,
                                                 const LaneSlots& ls, float init_carry, float a_look,
                                                 unsigned* hdr_words, unsigned limit) {
  if (ti.tile > 0) {
    const int ll = look_lane<G>(q);
    float mA = 1.0f, mB = 0.0f;
    if (st.beg < st.end) {
      const float Afull = DYN ? 1.0f : a_look;
#pragma unroll
      for (int i = 0; i < G::WPT; ++i) {
        if (st.beg + i < st.end) {
          const unsigned long long* s = ls.at(st.beg + i, ll);
          const float Bp = await_word(s, st.vB[i], tg.agg, hdr_words, limit);
          float Ap = Afull;
          if constexpr (DYN) Ap = await_word(s + 1, st.vA[i], tg.agg, hdr_words, limit);
          mB = __builtin_fmaf(Ap, mB, Bp);
          mA *= Ap;
        }
      }
    }
    L.mA[q.wave][q.wl] = mA;
    L.mB[q.wave][q.wl] = mB;
    float ck = init_carry;
    if (q.wave < G::NSUB && st.g0 > 0)
      ck = await_word(ls.at(st.g0 - 1, carry_lane<G>(q)), st.vck, tg.pre, hdr_words, limit);
    __syncthreads();
    if (q.wave < G::NSUB) {
      const int w0 = q.wave * G::WPS;   // the waves that read this sub-block
      float carry = ck;
#pragma unroll
      for (int w = 0; w < G::WPS; ++w) carry = __builtin_fmaf(L.mA[w0 + w][q.wl], carry, L.mB[w0 + w][q.wl]);
      L.carry[carry_lane<G>(q)] = carry;
      if (ti.is_ckpt && !ti.is_last)
        publish(ls.at(ti.tile, carry_lane<G>(q)), tg.pre, __builtin_fmaf(aggA, carry, aggB));
    }
  } else if (q.wave < G::NSUB) {
    L.carry[carry_lane<G>(q)] = init_carry;
  }
  __syncthreads();
}

// Counting the blocks of a launch, in two halves: finish_issue counts this
// block (thread 0), finish_complete acts on the count.  The last block of its
// class resets the class counter; the last class bumps the epoch for the next
// launch.  Safe once this block's epoch read (launch_tags) has returned,
// which the increment's data dependency on the epoch enforces: blocks of
// this launch use the epoch they read at their start, so a bump while some
// of them still publish or wait changes nothing for them.  Split so that the
// counter's round trip overlaps the block's work and its result is read
// before the block's bulk stores (loads and stores share one wait counter, so
// reading it after them would wait for every store).
__device__ __forceinline__ unsigned finish_issue(unsigned* hdr_words, unsigned epoch) {
  unsigned prev = 0;
  if (threadIdx.x == 0) {
    WsHeader* hdr = reinterpret_cast<WsHeader*>(hdr_words);
    unsigned one = 1u;
    asm volatile("" : "+v"(one) : "v"(epoch));   // the count depends on the epoch value
    prev = __hip_atomic_fetch_add(&hdr->cls[blockIdx.x & 7u].done, one, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  }
  return prev;
}

__device__ __forceinline__ void finish_complete(unsigned* hdr_words, unsigned epoch, unsigned prev) {
  if (threadIdx.x == 0) {
    WsHeader* hdr = reinterpret_cast<WsHeader*>(hdr_words);
    const unsigned cls = blockIdx.x & 7u;
    const unsigned cls_size = (gridDim.x - cls + 7u) >> 3;
    if (prev == cls_size - 1u) {
      __hip_atomic_store(&hdr->cls[cls].done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned n_cls = gridDim.x < 8u ? gridDim.x : 8u;
      const unsigned prev_all = __hip_atomic_fetch_add(&hdr->done_all, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
      if (prev_all == n_cls - 1u) {
        __hip_atomic_store(&hdr->done_all, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&hdr->epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Both halves at once (blocks without a tile, and the end of a kernel).
__device__ __forceinline__ void finish_block(unsigned* hdr_words, unsigned epoch) {
  finish_complete(hdr_words, epoch, finish_issue(hdr_words, epoch));
}

}  // namespace osm
