// Tile chaining protocol shared by the fused kernels: ticketed tiles, the
// token-group scan inside a tile, and the single-pass checkpointed look-back
// that hands each tile its EMA carry-in.
//
// The EMA s[t] = lam[t] s[t-1] + w[t] composes as affine maps f(s) = A s + B.
// A tile's aggregate is (A, B) = composition over its tokens from a zero
// state.  Tiles are grouped in runs of kCkpt = 64; the carry into tile t of
// group m is
//     carry = f_{t-1}( ... f_{64m}( C_m ) ... )
// where C_m is the state after tile 64m-1 (the checkpoint, ema_init for m=0).
// Every tile publishes its aggregate except the last tile of a group, which
// publishes its inclusive state as the next checkpoint.  The composition
// order is fixed, so results do not depend on timing.
#pragma once

#include "osm_device.h"
#include "osm_kernels.h"

namespace osm {

constexpr int kNTG = kWaves * kTGW;   // 16 token groups per tile
constexpr int kWPT = kCkpt / kWaves;  // look-back words read per thread

struct ChainLds {
  unsigned ticket, epoch;
  float A[kNTG][kTPR];        // token-group aggregate A (one per thread = per 4 lanes)
  float B[kNTG][kLanes];      // token-group aggregate B per lane
  float mA[kWaves][kLanes];   // look-back partial maps per wave
  float mB[kWaves][kLanes];
  float carry[kLanes];        // resolved carry-in of the tile
};

struct TileInfo {
  int tile, lb, b, lbd;
  unsigned epoch, tag_agg, tag_pre;
  bool is_last, is_ckpt;
  bool valid;  // false only if the header was corrupted (ticket out of range)
};

// Thread coordinates inside the workgroup.
struct ThreadPos {
  int tid, wave, wl, l4, tg;
};

__device__ __forceinline__ ThreadPos thread_pos() {
  ThreadPos q;
  q.tid = threadIdx.x;
  q.wave = q.tid >> 6;
  q.wl = q.tid & 63;
  q.l4 = q.wl & (kTPR - 1);
  q.tg = q.wave * kTGW + (q.wl >> 4);
  return q;
}

// Thread 0 takes the next ticket; tickets are handed out in start order, so
// all tiles with a lower ticket are resident or finished.
__device__ __forceinline__ TileInfo claim_tile(ChainLds& L, unsigned* hdr_words, int n_lb, int n_lbd,
                                               int n_tiles) {
  WsHeader* hdr = reinterpret_cast<WsHeader*>(hdr_words);
  if (threadIdx.x == 0) {
    L.ticket = __hip_atomic_fetch_add(&hdr->ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.epoch = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  TileInfo ti;
  const unsigned raw = L.ticket;
  ti.valid = raw < (unsigned)n_lb * (unsigned)n_tiles;
  if (!ti.valid && threadIdx.x == 0) raise_fault(hdr_words);
  const int ticket = ti.valid ? (int)raw : 0;
  ti.tile = ticket / n_lb;
  ti.lb = ticket - ti.tile * n_lb;
  ti.b = ti.lb / n_lbd;
  ti.lbd = ti.lb - ti.b * n_lbd;
  ti.epoch = L.epoch;
  ti.tag_agg = make_tag(ti.epoch, kKindAgg);
  ti.tag_pre = make_tag(ti.epoch, kKindPre);
  ti.is_last = ti.tile == n_tiles - 1;
  ti.is_ckpt = (ti.tile % kCkpt) == kCkpt - 1;
  return ti;
}

// Aggregate A of a full tile of R-token runs under a static lambda, in the
// same multiplication order as the producing workgroup's scan.
template <int R>
__device__ __forceinline__ float static_tile_A(float lam) {
  float a = 1.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) a *= lam;
  float A = 1.0f;
#pragma unroll
  for (int q = 0; q < kNTG; ++q) A *= a;
  return A;
}

// Token-group scan.  In: this thread's run aggregate (A, Bv).  Out: (pA, pB)
// mapping the tile carry to the state before this thread's first token; in
// wave 0, (aggA, aggB) = the tile aggregate of lane wl, which is published
// unless the tile is a checkpoint or the last tile.
template <bool DYN>
__device__ __forceinline__ void tile_scan(ChainLds& L, const ThreadPos& q, const TileInfo& ti, float A,
                                          const float (&Bv)[kLPT], float& pA, float (&pB)[kLPT], float& aggA,
                                          float& aggB, unsigned long long* lane_slots, size_t tile_stride) {
  L.A[q.tg][q.l4] = A;
#pragma unroll
  for (int i = 0; i < kLPT; ++i) L.B[q.tg][q.l4 * kLPT + i] = Bv[i];
  __syncthreads();
  pA = 1.0f;
#pragma unroll
  for (int i = 0; i < kLPT; ++i) pB[i] = 0.0f;
  for (int g = 0; g < q.tg; ++g) {
    const float a = L.A[g][q.l4];
#pragma unroll
    for (int i = 0; i < kLPT; ++i) pB[i] = __builtin_fmaf(a, pB[i], L.B[g][q.l4 * kLPT + i]);
    pA *= a;
  }
  aggA = 1.0f;
  aggB = 0.0f;
  if (q.wave == 0) {
    for (int g = 0; g < kNTG; ++g) {
      const float a = L.A[g][q.wl >> 2];
      aggB = __builtin_fmaf(a, aggB, L.B[g][q.wl]);
      aggA *= a;
    }
    if (!ti.is_ckpt && !ti.is_last) {
      unsigned long long* mine = lane_slots + (size_t)ti.tile * tile_stride;
      if (DYN) publish(mine + 1, ti.tag_agg, aggA);
      publish(mine, ti.tag_agg, aggB);
    }
  }
}

// Look-back: leaves the carry-in of every lane of the tile in L.carry.
// `lam_static` is the static lambda of lane wl (unused when DYN).
template <bool DYN, int R>
__device__ __forceinline__ void look_back(ChainLds& L, const ThreadPos& q, const TileInfo& ti, float aggA,
                                          float aggB, const unsigned long long* lane_slots, size_t tile_stride,
                                          float init_wl, float lam_static_wl, unsigned* hdr_words) {
  if (ti.tile > 0) {
    const int g0 = (ti.tile / kCkpt) * kCkpt;
    const int beg = g0 + q.wave * kWPT;
    const int end = min(beg + kWPT, ti.tile);
    float mA = 1.0f, mB = 0.0f;
    if (beg < end) {
      const float Afull = DYN ? 1.0f : static_tile_A<R>(lam_static_wl);
      unsigned long long vB[kWPT];
      unsigned long long vA[DYN ? kWPT : 1];
#pragma unroll
      for (int i = 0; i < kWPT; ++i) {
        if (beg + i < end) {
          const unsigned long long* s = lane_slots + (size_t)(beg + i) * tile_stride;
          vB[i] = peek(s);
          if constexpr (DYN) vA[i] = peek(s + 1);
        }
      }
#pragma unroll
      for (int i = 0; i < kWPT; ++i) {
        if (beg + i < end) {
          const unsigned long long* s = lane_slots + (size_t)(beg + i) * tile_stride;
          const float Bp = await_word(s, vB[i], ti.tag_agg, hdr_words);
          float Ap = Afull;
          if constexpr (DYN) Ap = await_word(s + 1, vA[i], ti.tag_agg, hdr_words);
          mB = __builtin_fmaf(Ap, mB, Bp);
          mA *= Ap;
        }
      }
    }
    L.mA[q.wave][q.wl] = mA;
    L.mB[q.wave][q.wl] = mB;
    float ck = 0.0f;
    if (q.wave == 0) {
      if (g0 == 0) {
        ck = init_wl;
      } else {
        const unsigned long long* s = lane_slots + (size_t)(g0 - 1) * tile_stride;
        ck = await_word(s, peek(s), ti.tag_pre, hdr_words);
      }
    }
    __syncthreads();
    if (q.wave == 0) {
      float carry = ck;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) carry = __builtin_fmaf(L.mA[w][q.wl], carry, L.mB[w][q.wl]);
      L.carry[q.wl] = carry;
      if (ti.is_ckpt && !ti.is_last)
        publish(const_cast<unsigned long long*>(lane_slots) + (size_t)ti.tile * tile_stride, ti.tag_pre,
                __builtin_fmaf(aggA, carry, aggB));
    }
  } else if (q.wave == 0) {
    L.carry[q.wl] = init_wl;
  }
  __syncthreads();
}

// The last block of the launch re-arms the header for the next launch.
__device__ __forceinline__ void finish_block(unsigned* hdr_words, unsigned epoch) {
  if (threadIdx.x == 0) {
    WsHeader* hdr = reinterpret_cast<WsHeader*>(hdr_words);
    const unsigned prev = __hip_atomic_fetch_add(&hdr->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) {
      __hip_atomic_store(&hdr->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&hdr->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&hdr->epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace osm
