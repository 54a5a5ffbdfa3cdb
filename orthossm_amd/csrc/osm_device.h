// Device-side building blocks shared by the Cheby-RKV kernels (gfx950).
//
// Data layout in HBM (all row-major):
//   x, out     [B, S, D]      D = H*hd lanes, lane stride 1
//   coeffs     [B, H, K, hd]  fp32
//   g          [B, S, H]      fp32 (optional, any strides)
//   ema state  [B, D]         fp32
//
// Work decomposition shared by the kernels: a lane-block is 64 consecutive
// lanes of one batch row; a tile is T consecutive tokens of a lane-block.  A
// thread owns 4 adjacent lanes (one 16-byte fp32 vector or 8-byte bf16
// vector) and a run of R consecutive tokens; 16 threads cover the 64 lanes of
// a row, so each wave instruction touches 4 rows x 256 contiguous bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace osm {

constexpr int kWave = 64;
constexpr int kLPT = 4;                   // lanes per thread
constexpr int kTPR = 16;                  // threads per 64-lane row segment
constexpr int kLanes = kLPT * kTPR;       // lanes per lane-block
constexpr int kTGW = kWave / kTPR;        // token groups per wave
constexpr int kCkpt = 64;                 // checkpoint interval of the look-back, in tiles
constexpr float kTwoLog2e = 2.8853900817779268f;  // 2*log2(e): tanh via exp2

// Workspace header (first 256 bytes of every workspace).
//   ticket  next tile ticket of the running launch (reset to 0 by the last block)
//   done    blocks finished in the running launch  (reset to 0 by the last block)
//   epoch   launch counter; tags every published look-back word
//   fault   set to 1 if a launch saw an out-of-range ticket or a look-back
//           wait exceeded kSpinLimit (results of that launch are invalid);
//           only a zero fill clears it
struct WsHeader {
  unsigned ticket;
  unsigned done;
  unsigned epoch;
  unsigned fault;
  unsigned pad[60];
};
static_assert(sizeof(WsHeader) == 256, "header is 256 bytes");

// Upper bound on polls of one look-back word (each poll is a device-scope
// load plus a short sleep, so this is many seconds).  It only guarantees that
// every wave exits even if the header was corrupted by overlapping calls.
constexpr unsigned kSpinLimit = 1u << 24;

// A look-back word is one 64-bit value: high 32 bits = (epoch << 2) | kind,
// low 32 bits = an fp32 payload.  Because tag and payload travel in one
// atomic access, relaxed agent-scope loads/stores suffice (no fences, hence
// no L2 write-back or invalidate on gfx950).
enum : unsigned { kKindAgg = 1u, kKindPre = 2u };

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

__device__ __forceinline__ void raise_fault(unsigned* hdr_words) {
  __hip_atomic_store(hdr_words + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin until `slot` carries `tag`, starting from an already-loaded value.
// The producer of every awaited word has a lower tile ticket, so it is
// resident or finished and publishes without waiting on anyone: the loop
// ends.  kSpinLimit bounds it anyway (fault flag, payload 0).
__device__ __forceinline__ float await_word(const unsigned long long* slot, unsigned long long w, unsigned tag,
                                            unsigned* hdr_words) {
  unsigned polls = 0;
  while ((unsigned)(w >> 32) != tag) {
    if (++polls > kSpinLimit) {
      raise_fault(hdr_words);
      return 0.0f;
    }
    __builtin_amdgcn_s_sleep(1);
    w = peek(slot);
  }
  return __uint_as_float((unsigned)w);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// 4-lane vector load / store for fp32 and bf16 element types.
template <typename T>
struct Lanes4;

template <>
struct Lanes4<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    f32x4 q = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(q, reinterpret_cast<f32x4*>(p));
  }
};

template <>
struct Lanes4<__bf16> {
  static __device__ __forceinline__ void load(const __bf16* p, float (&v)[4]) {
    const u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
  // Round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
  static __device__ __forceinline__ void store(__bf16* p, const float (&v)[4]) {
    const f32x4 f = {v[0], v[1], v[2], v[3]};
    const bf16x4 q = __builtin_convertvector(f, bf16x4);
    __builtin_nontemporal_store(__builtin_bit_cast(u32x2, q), reinterpret_cast<u32x2*>(p));
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

// Given y2 = 2*log2(e) * damping * p, returns r = 1 / (1 + exp(2*damping*p));
// then tanh(damping*p) = 1 - 2r.  exp2 overflow to +Inf gives r = 0 (z = 1);
// underflow to 0 gives r = 1 (z = -1).
__device__ __forceinline__ float tanh_r(float y2) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y2));
}

}  // namespace osm
