// Device-side building blocks shared by the Cheby-RKV kernels (gfx950).
//
// Data layout in HBM (all row-major):
//   x, out     [B, S, D]      D = H*hd lanes, lane stride 1
//   coeffs     [B, H, K, hd]  fp32
//   g          [B, S, H]      fp32 (optional, any strides)
//   ema state  [B, D]         fp32
// Work decomposition: see TileGeo in osm_kernels.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "osm_kernels.h"

namespace osm {

constexpr int kLanes = 64;                // lanes per look-back sub-block (one wave)
constexpr float kTwoLog2e = 2.8853900817779268f;  // 2*log2(e): tanh via exp2

// Workspace header (first kHeaderBytes of every workspace).
//   epoch      launch counter; tags every published look-back word.  Read by
//              every block at start, bumped by the last block of the launch.
//   fault      0, or the fault tag (make_tag(epoch, kKindFault)) of the last
//              launch in which a look-back wait exceeded kSpinLimit (results
//              of that launch are invalid).  Sticky until osm_workspace_status
//              resets it or a full clear; a waiter gives up early only on the
//              tag of its own launch, so an old fault does not disturb later
//              launches.
//   done_all   classes finished in the running launch (reset by the last one)
//   cls[c]     per class c = blockIdx % 8 (one XCD under round-robin
//              dispatch): `done` counts its finished blocks; the last block
//              of the class resets it.  One 128-byte line per class: no
//              cross-class contention.
struct WsHeader {
  unsigned epoch;
  unsigned reserved0[2];
  unsigned fault;          // byte offset 12
  unsigned reserved1[12];
  unsigned done_all;       // byte offset 64
  unsigned reserved2[15];
  struct {
    unsigned done;
    unsigned reserved[31];
  } cls[8];                // byte offsets 128 + 128 c
};
static_assert(sizeof(WsHeader) <= kHeaderBytes, "header fits");
static_assert(offsetof(WsHeader, fault) < kHeaderKeepBytes && offsetof(WsHeader, done_all) == kHeaderKeepBytes,
              "a layout change keeps the epoch and the fault word and clears the counters");

// A look-back word is one 64-bit value: high 32 bits = (epoch << 2) | kind,
// low 32 bits = an fp32 payload.  Because tag and payload travel in one
// atomic access, relaxed agent-scope loads/stores suffice (no fences, hence
// no L2 write-back or invalidate on gfx950).
enum : unsigned { kKindAgg = 1u, kKindPre = 2u, kKindFault = 3u };

__device__ __forceinline__ unsigned make_tag(unsigned epoch, unsigned kind) {
  return ((epoch & 0x3fffffffu) << 2) | kind;
}

__device__ __forceinline__ void publish(unsigned long long* slot, unsigned tag, float v) {
  const unsigned long long w = ((unsigned long long)tag << 32) | (unsigned long long)__float_as_uint(v);
  __hip_atomic_store(slot, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long peek(const unsigned long long* slot) {
  return __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Fault tag of the launch whose look-back words carry `tag` (any kind).
__device__ __forceinline__ unsigned fault_tag_of(unsigned tag) { return (tag & ~3u) | kKindFault; }

__device__ __forceinline__ void raise_fault(unsigned* hdr_words, unsigned fault_tag) {
  __hip_atomic_store(hdr_words + 3, fault_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin until `slot` carries `tag`, starting from an already-loaded value.
// The producer of every awaited word was dispatched earlier and publishes
// without waiting on anything later (osm_chain.h), so the loop ends;
// `limit` polls (kSpinLimit, or 0 under OSM_FLAG_POLL_LIMIT_ZERO) bound it
// anyway.  A wait that gives up sets the fault word to this launch's fault
// tag and returns a quiet NaN: every carry composed from it is NaN, so the
// outputs that depend on the missing value are NaN (the kernels store a NaN
// state unclamped), not plausible numbers.
__device__ __forceinline__ float await_word(const unsigned long long* slot, unsigned long long w, unsigned tag,
                                            unsigned* hdr_words, unsigned limit) {
  unsigned polls = 0;
  while ((unsigned)(w >> 32) != tag) {
    ++polls;
    // Give up when over the limit or when another wave of this launch
    // already gave up (a fault left by an earlier launch is ignored).
    const unsigned ftag = fault_tag_of(tag);
    if (polls > limit ||
        ((polls & 1023u) == 0 &&
         __hip_atomic_load(hdr_words + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ftag)) {
      raise_fault(hdr_words, ftag);
      return __builtin_nanf("");
    }
    __builtin_amdgcn_s_sleep(1);
    w = peek(slot);
  }
  return __uint_as_float((unsigned)w);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// N-lane streaming load / store (non-temporal: every element is touched once)
// for fp32 and bf16.  bf16 is widened exactly; stores round to nearest even
// (v_cvt_pk_bf16_f32 on gfx950).
template <typename T, int N>
struct LaneVec;

template <>
struct LaneVec<float, 1> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[1]) { v[0] = __builtin_nontemporal_load(p); }
  static __device__ __forceinline__ void store(float* p, const float (&v)[1]) { __builtin_nontemporal_store(v[0], p); }
};

template <>
struct LaneVec<float, 2> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[2]) {
    const f32x2 q = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(p));
    v[0] = q.x;
    v[1] = q.y;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[2]) {
    const f32x2 q = {v[0], v[1]};
    __builtin_nontemporal_store(q, reinterpret_cast<f32x2*>(p));
  }
};

template <>
struct LaneVec<float, 4> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    const f32x4 q = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(q, reinterpret_cast<f32x4*>(p));
  }
};

template <>
struct LaneVec<__bf16, 1> {
  static __device__ __forceinline__ void load(const __bf16* p, float (&v)[1]) {
    const unsigned short q = __builtin_nontemporal_load(reinterpret_cast<const unsigned short*>(p));
    v[0] = __uint_as_float((unsigned)q << 16);
  }
  static __device__ __forceinline__ void store(__bf16* p, const float (&v)[1]) {
    const __bf16 q = (__bf16)v[0];
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned short, q), reinterpret_cast<unsigned short*>(p));
  }
};

template <>
struct LaneVec<__bf16, 2> {
  static __device__ __forceinline__ void load(const __bf16* p, float (&v)[2]) {
    const unsigned q = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p));
    v[0] = __uint_as_float(q << 16);
    v[1] = __uint_as_float(q & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(__bf16* p, const float (&v)[2]) {
    const f32x2 f = {v[0], v[1]};
    const bf16x2 q = __builtin_convertvector(f, bf16x2);
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned, q), reinterpret_cast<unsigned*>(p));
  }
};

template <>
struct LaneVec<__bf16, 4> {
  static __device__ __forceinline__ void load(const __bf16* p, float (&v)[4]) {
    const u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(__bf16* p, const float (&v)[4]) {
    const f32x4 f = {v[0], v[1], v[2], v[3]};
    const bf16x4 q = __builtin_convertvector(f, bf16x4);
    __builtin_nontemporal_store(__builtin_bit_cast(u32x2, q), reinterpret_cast<u32x2*>(p));
  }
};

// ---------------------------------------------------------------------------
// Buffer-descriptor access (raw buffer loads/stores).  A descriptor holds a
// 48-bit base and a byte extent; an access at voffset + soffset beyond the
// extent reads 0 and drops stores.  Kernels rebase descriptors per tile
// (uniform, in SGPRs), give each thread a fixed VGPR lane offset (kOffOOB for
// lanes outside the tensor) and step tokens with a uniform SGPR offset, so
// no per-element 64-bit address arithmetic or bounds branch is needed.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRsrcWord3 = 0x00020000;       // gfx9-family raw buffer format
constexpr uint32_t kOffOOB = 0x80000000u;    // out of range of every descriptor we build
constexpr uint32_t kMaxExtent = 0x7fffffffu;
constexpr int kNT = 2;                       // cache policy: non-temporal streaming

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint64_t extent_bytes) {
  const uint32_t n = extent_bytes > kMaxExtent ? kMaxExtent : (uint32_t)extent_bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, kRsrcWord3);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T, int N>
struct BufVec;

template <>
struct BufVec<float, 1> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[1]) {
    v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, kNT));
  }
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[1]) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, vo, so, kNT);
  }
};

template <>
struct BufVec<float, 2> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[2]) {
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kNT);
    v[0] = __uint_as_float(q.x);
    v[1] = __uint_as_float(q.y);
  }
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[2]) {
    const u32x2 q = {__float_as_uint(v[0]), __float_as_uint(v[1])};
    __builtin_amdgcn_raw_buffer_store_b64(q, r, vo, so, kNT);
  }
};

template <>
struct BufVec<float, 4> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[4]) {
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, kNT);
    v[0] = __uint_as_float(q.x); v[1] = __uint_as_float(q.y); v[2] = __uint_as_float(q.z); v[3] = __uint_as_float(q.w);
  }
  // A VALU instruction that overwrites the data registers of a store wider
  // than 64 bits right after it was seen on MI355X to corrupt the store's
  // first dword now and then (the compiler placed no wait state there), so
  // the store is followed by two wait states that no instruction can be
  // scheduled into.
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[4]) {
    const u32x4 q = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
    __builtin_amdgcn_raw_buffer_store_b128(q, r, vo, so, kNT);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 1");
    __builtin_amdgcn_sched_barrier(0);
  }
};

template <>
struct BufVec<__bf16, 1> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[1]) {
    v[0] = __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, kNT) << 16);
  }
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[1]) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (__bf16)v[0]), r, vo, so, kNT);
  }
};

// One fp32 value with the default cache policy, for data that several
// workgroups of one XCD read at different times (the coefficients, g, x lines
// split between workgroups): with the non-temporal hint the L2 may drop the
// line before the others have read it.
__device__ __forceinline__ float load_f32_shared(Rsrc r, uint32_t vo, uint32_t so) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
}

template <>
struct BufVec<__bf16, 2> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[2]) {
    const unsigned q = __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, kNT);
    v[0] = __uint_as_float(q << 16);
    v[1] = __uint_as_float(q & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[2]) {
    const f32x2 f = {v[0], v[1]};
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, __builtin_convertvector(f, bf16x2)), r, vo,
                                          so, kNT);
  }
};

template <>
struct BufVec<__bf16, 4> {
  static __device__ __forceinline__ void load(Rsrc r, uint32_t vo, uint32_t so, float (&v)[4]) {
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kNT);
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
  static __device__ __forceinline__ void store(Rsrc r, uint32_t vo, uint32_t so, const float (&v)[4]) {
    const f32x4 f = {v[0], v[1], v[2], v[3]};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, __builtin_convertvector(f, bf16x4)), r, vo, so,
                                          kNT);
  }
};

// softsign u = x / (1 + |x|).  x is first clamped to +-1e30 so that +-Inf
// gives +-1 (1e30 / (1 + 1e30) rounds to 1).  A NaN x is handled by the caller.
__device__ __forceinline__ float softsign(float x) {
  const float xc = __builtin_amdgcn_fmed3f(x, -1e30f, 1e30f);
  return xc * __builtin_amdgcn_rcpf(1.0f + __builtin_fabsf(xc));
}

// Clenshaw evaluation of sum_{k<KP} c[k] T_k(u):
//   b_k = c_k + 2u b_{k+1} - b_{k+2},  p = c_0 + u b_1 - b_2.
// Coefficients beyond the caller's K are zero, which leaves p unchanged.
template <int KP>
__device__ __forceinline__ float clenshaw(float u, const float* c) {
  const float u2 = u + u;
  float b1 = c[KP - 1];
  float b2 = 0.0f;
#pragma unroll
  for (int k = KP - 2; k >= 1; --k) {
    const float b0 = __builtin_fmaf(u2, b1, c[k] - b2);
    b2 = b1;
    b1 = b0;
  }
  return __builtin_fmaf(u, b1, c[0] - b2);
}

// Monomial form of a Chebyshev series.  T_k has only powers u^j with
// j = k - 2i, so coefficient j of sum_{k<8} c_k T_k(u) is
//     sum_{i<4} cheb_mono(j, i) * c_{j+2i}
// with the textbook expansions T_0 = 1, T_1 = u, T_2 = 2u^2 - 1,
// T_3 = 4u^3 - 3u, T_4 = 8u^4 - 8u^2 + 1, T_5 = 16u^5 - 20u^3 + 5u,
// T_6 = 32u^6 - 48u^4 + 18u^2 - 1, T_7 = 64u^7 - 112u^5 + 56u^3 - 7u.
// Evaluating the series as Horner on these coefficients takes K-1 FMAs per
// point against 2(K-1) operations for Clenshaw; in fp32 both errors stay
// ~1e-6 for |c_k| = O(1), |u| <= 1 at K = 8.  A constexpr function rather
// than a table in device memory: with j a template argument the factors are
// instruction constants (a table indexed at run time is a memory load on the
// path to every tile's first arithmetic).
__host__ __device__ constexpr float cheb_mono(int j, int i) {
  switch (j * 4 + i) {
    case 0: return 1.0f;   case 1: return -1.0f;   case 2: return 1.0f;   case 3: return -1.0f;  // u^0: T_0,T_2,T_4,T_6
    case 4: return 1.0f;   case 5: return -3.0f;   case 6: return 5.0f;   case 7: return -7.0f;  // u^1: T_1,T_3,T_5,T_7
    case 8: return 2.0f;   case 9: return -8.0f;   case 10: return 18.0f;                        // u^2: T_2,T_4,T_6
    case 12: return 4.0f;  case 13: return -20.0f; case 14: return 56.0f;                        // u^3: T_3,T_5,T_7
    case 16: return 8.0f;  case 17: return -48.0f;                                               // u^4: T_4,T_6
    case 20: return 16.0f; case 21: return -112.0f;                                              // u^5: T_5,T_7
    case 24: return 32.0f;                                                                       // u^6: T_6
    case 28: return 64.0f;                                                                       // u^7: T_7
    default: return 0.0f;
  }
}

// Monomial coefficient J (unscaled) from the Chebyshev coefficients
// c_{J+2i}, i < 4, in float64.  Terms whose factor is 0 are left out: they
// pair only with c_k for k >= 8, which the callers load as 0.
template <int J>
__device__ __forceinline__ double mono_coef(const float (&cm)[4]) {
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (cheb_mono(J, i) != 0.0f) acc = __builtin_fma((double)cheb_mono(J, i), (double)cm[i], acc);
  return acc;
}

// Horner evaluation of sum_j a[j] u^j.
template <int KP>
__device__ __forceinline__ float horner(float u, const float (&a)[KP]) {
  float p = a[KP - 1];
#pragma unroll
  for (int j = KP - 2; j >= 0; --j) p = __builtin_fmaf(p, u, a[j]);
  return p;
}

// The series of a lane from the coefficients the kernels hold in registers:
// monomial coefficients (Horner) for KP <= kMonoMaxK, Chebyshev coefficients
// (Clenshaw) above.
template <int KP>
__device__ __forceinline__ float series(float u, const float (&c)[KP]) {
  if constexpr (KP > kMonoMaxK)
    return clenshaw<KP>(u, c);
  else
    return horner<KP>(u, c);
}

// The series in the form a tile chose: CHEB (or more than kMonoMaxK
// coefficients) = Chebyshev coefficients by Clenshaw, else monomial
// coefficients by Horner.
template <int KP, bool CHEB>
__device__ __forceinline__ float series_as(float u, const float (&c)[KP]) {
  if constexpr (CHEB || KP > kMonoMaxK)
    return clenshaw<KP>(u, c);
  else
    return horner<KP>(u, c);
}

// Clenshaw evaluation of sum_{m<N} d[m] U_m(u) in the second-kind basis
// (U_0 = 1, U_1 = 2u, U_m = 2u U_{m-1} - U_{m-2}):
//   b_m = d_m + 2u b_{m+1} - b_{m+2},  sum = b_0.
// With d[m] = (m+1) c[m+1] it is the derivative of sum_k c_k T_k(u), since
// T_k' = k U_{k-1}.
template <int N>
__device__ __forceinline__ float clenshaw_u(float u, const float (&d)[N]) {
  const float u2 = u + u;
  float b1 = 0.0f, b2 = 0.0f;
#pragma unroll
  for (int m = N - 1; m >= 0; --m) {
    const float b0 = __builtin_fmaf(u2, b1, d[m] - b2);
    b2 = b1;
    b1 = b0;
  }
  return b1;
}

// The derivative of series_as from dm[m] = (m+1) c[m+1] (times a scale):
// sum dm[m] U_m(u) by Clenshaw in the Chebyshev form (T_k' = k U_{k-1}),
// sum dm[m] u^m by Horner in the monomial form.
template <int N, bool CHEB>
__device__ __forceinline__ float dseries_as(float u, const float (&dm)[N]) {
  if constexpr (CHEB || N + 1 > kMonoMaxK)
    return clenshaw_u<N>(u, dm);
  else
    return horner<N>(u, dm);
}

// x^N by repeated squaring in float64, rounded once to fp32 (within about
// half an ulp of the exact power; a float chain of N products, or squaring in
// fp32, errs by several ulps, and over a long sequence the carried state
// accumulates that error tile after tile when lambda is close to 1).  Under a
// static lambda the kernels form the decay of an R-token run as
// pow_n<R>(lambda) and that of a full tile, for checkpoints and the
// look-back alike, as pow_n<TILE>(lambda) (static_tile_A).
template <int N>
__device__ __forceinline__ double pow_n_f64(double x) {
  if constexpr (N == 0) return 1.0;
  else if constexpr (N == 1) return x;
  else {
    const double h = pow_n_f64<N / 2>(x);
    return N % 2 ? h * h * x : h * h;
  }
}
template <int N>
__device__ __forceinline__ float pow_n(float x) {
  return (float)pow_n_f64<N>((double)x);
}

// Given y2 = 2*log2(e) * damping * p, returns r = 1 / (1 + exp(2*damping*p));
// then tanh(damping*p) = 1 - 2r.  exp2 overflow to +Inf gives r = 0 (z = 1);
// underflow to 0 gives r = 1 (z = -1).
__device__ __forceinline__ float tanh_r(float y2) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y2));
}

}  // namespace osm
