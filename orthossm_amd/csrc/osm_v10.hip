// The reference's full apply_cheby_rkv_v10 path for gfx950: online TTT over
// chunks with an inline Lion update, in one launch.
//
// Reference counterpart: the chunk loop of apply_cheby_rkv_v10
// (sdpc_kernel.py:2574-2606), each chunk a FusedChebyRKVv10.forward
// (2353-2433) running _ortho_megakernel (1890-2287): one kernel launch and a
// few host-side casts per chunk, with the updated coefficients and momentum
// fed to the next chunk.  Per chunk (length L <= chunk):
//   x -> bf16; u = sign(x)(1 - 1/(1 + max(|x|, 1e-7))), NaN read as 0 and
//   sign(0) = +1; y = LUT interpolation of sum_k c_k T_k(u) (256-point half
//   table, odd terms times sign(u)) or the 4-term Clenshaw fallback;
//   z = tanh(clamp(gamma_h y, -4, 4)) (0 for NaN x); s = mu s + (1-mu) z from 0;
//   out = bf16(s); gc_k = sum over (t, t+1) of gv T_k(u_t) with
//   gv = err / (1 + exp(-3|err|)), err = u_{t+1} - s_t; then Lion on (c, m).
//
// Chunks depend on each other only through (c, m) of each lane, so one
// workgroup owns LW lanes of one (batch row, head) and walks the
// chunks in order; the dependency never leaves the workgroup.  A chunk is
// processed in 256-token blocks: thread (run g, lane l) owns kV10Run tokens;
// runs are composed by a shuffle scan inside each wave and across waves in
// LDS; the proxy-gradient sums are reduced over the runs in a fixed order,
// and (lanes x K) threads apply Lion and publish the next chunk's
// coefficients through LDS.
#include <type_traits>

#include "osm_tile.h"

namespace osm {
namespace {

constexpr int kBlockTok = kV10Groups * kV10Run;      // 256 tokens per block
constexpr float kLog2e = 1.4426950408889634f;
// Floats per LUT row in LDS: the 8 values of T_k padded to 12, so that the
// 16-byte reads of random rows by the lanes of a wave spread over more LDS
// banks than with 8 (rows i and i' collide when 12 (i - i') = 0 mod the
// bank count).  Measured at the configs[1] shape on MI355X: 221 against
// 227 us with the XCD order below.
constexpr int kLutStride = 12;
// Workgroup order: the workgroups whose lanes share 128-byte lines of x go
// to one XCD, so each line is fetched into one L2 (with consecutive indices
// the 4 workgroups of a line sat on 4 XCDs and every line was fetched 4
// times): 227 against 270 us at the configs[1] shape.
constexpr bool kXcdLines = true;

// x rounded to bf16 (round to nearest even), as the reference casts on entry.
template <typename XT>
__device__ __forceinline__ float to_bf16_value(float v);
template <>
__device__ __forceinline__ float to_bf16_value<float>(float v) {
  return (float)(__bf16)v;
}
template <>
__device__ __forceinline__ float to_bf16_value<__bf16>(float v) {
  return v;   // loaded from bf16 already
}

// One x value with the default cache policy (not non-temporal): each
// 128-byte line of x is read by the 128 / (4 LW) workgroups of one XCD,
// which reach it at different times (with the non-temporal hint, x was read
// 1.05-1.15 times over from HBM).
template <typename XT>
__device__ __forceinline__ float load_x(Rsrc r, uint32_t vo, uint32_t so);
template <>
__device__ __forceinline__ float load_x<float>(Rsrc r, uint32_t vo, uint32_t so) {
  return load_f32_shared(r, vo, so);
}
template <>
__device__ __forceinline__ float load_x<__bf16>(Rsrc r, uint32_t vo, uint32_t so) {
  return __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0) << 16);
}

// The megakernel's softsign on a bf16 value: |u| and sign(u); NaN reads as 0.
__device__ __forceinline__ void v10_softsign(float xb, float& absu, float& sgn) {
  const float xs = xb == xb ? xb : 0.0f;
  const float ax = __builtin_fmaxf(__builtin_fabsf(xs), 1e-7f);
  absu = 1.0f - __builtin_amdgcn_rcpf(1.0f + ax);
  sgn = xs >= 0.0f ? 1.0f : -1.0f;
}

// The KP proxy-gradient sums of a wave's runs, reduce-scattered: the sum of
// v over the runs of lane l (lanes l, l + LW, l + 2 LW, .. of the wave) is
// the butterfly v += v[lane ^ o] for o = LW, 2 LW, .. 32, and here each step
// serves two of the sums at once, so that after the last step lane (run gw,
// l) holds the full sum of coefficient gw (and, with LW = 16 and KP = 8,
// of gw + 4), which it stores to ws[k][l].  The steps, with the same sums
// (each adds a lane's partial sum and its partner's) as the butterfly:
//   o = 8 (LW = 8): a DPP row rotate by 8 (lane ^ 8 inside each 16-lane row)
//     of the value the partner keeps (lanes with bit 3 set keep the odd one
//     of a pair of sums, the others the even one);
//   o = 16: v_permlane16_swap of a pair (a, b) gives (rows a0, b0, a2, b2)
//     and (rows a1, b1, a3, b3): their sum holds a's pair sums in the even
//     rows and b's in the odd rows;
//   o = 32: v_permlane32_swap of (a, b) gives (lower a, lower b) and (upper
//     a, upper b): their sum holds a's sums in the lower half and b's in the
//     upper half.
// (Lane layout of the two swaps, for equal operands, checked by a probe
// kernel: rows 0, 0, 2, 2 and 1, 1, 3, 3; lower half twice and upper half
// twice.)  With KP = 4 the last step has one value and adds the halves as
// the butterfly does.
__device__ __forceinline__ void swap16(float& a, float& b) {
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  const u32x2v r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r.x);
  b = __uint_as_float(r.y);
}
__device__ __forceinline__ void swap32(float& a, float& b) {
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  const u32x2v r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r.x);
  b = __uint_as_float(r.y);
}
// pair sum for o = 16 / 32: a + b after the swap
__device__ __forceinline__ float pair16(float a, float b) {
  swap16(a, b);
  return a + b;
}
__device__ __forceinline__ float pair32(float a, float b) {
  swap32(a, b);
  return a + b;
}

template <int LW, int KP>
__device__ __forceinline__ void store_run_sums(const float (&gc)[KP], float (&ws)[8][LW], int l, int gw) {
  static_assert(LW == 8 || LW == 16, "8 or 16 lanes per workgroup");
  static_assert(KP == 4 || KP == 8, "4 or 8 coefficients");
  constexpr int N1 = LW == 8 ? KP / 2 : KP;   // values left after the o = 8 step
  float a[N1];
  if constexpr (LW == 8) {
    const bool odd = (threadIdx.x & 8) != 0;
#pragma unroll
    for (int i = 0; i < N1; ++i) {
      const float keep = odd ? gc[2 * i + 1] : gc[2 * i];
      const float give = odd ? gc[2 * i] : gc[2 * i + 1];
      a[i] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(give), 0x128, 0xF, 0xF, false));
    }
  } else {
#pragma unroll
    for (int i = 0; i < N1; ++i) a[i] = gc[i];
  }
  constexpr int N2 = N1 / 2;   // after o = 16
  float b[N2];
#pragma unroll
  for (int i = 0; i < N2; ++i) b[i] = pair16(a[2 * i], a[2 * i + 1]);
  if constexpr (N2 == 1) {
    // one value (LW = 8, KP = 4): lane (gw, l) holds coefficient gw & 3
    const float v = pair32(b[0], b[0]);
    if (gw < 4) ws[gw][l] = v;
  } else {
    // N2 = 2 (LW = 8, KP = 8: coefficient gw) or N2 = 4 (LW = 16, KP = 8:
    // coefficients gw and gw + 4) or N2 = 2 (LW = 16, KP = 4: gw)
#pragma unroll
    for (int i = 0; i < N2 / 2; ++i) ws[gw + 4 * i][l] = pair32(b[2 * i], b[2 * i + 1]);
  }
}

// 16-byte aligned: LUT rows are read as f32x4.
template <int LW>
struct __attribute__((aligned(16))) V10Lds {
  static constexpr int NW = kV10Groups * LW / 64;   // waves per workgroup
  float lut[256][kLutStride];        // T_k at the table's grid, k contiguous (rows 48 bytes apart)
  float cs[8][LW];                   // coefficients of the current chunk
  float ms[8][LW];                   // Lion momentum
  float wA[NW][LW], wB[NW][LW];      // each wave's composed EMA map over its runs
  float carry[LW];                   // EMA state entering the block
  float ws[NW][8][LW];               // each wave's proxy-gradient sums
};

// LW lanes per workgroup (8 or 16); kV10Groups runs of kV10Run tokens per
// 256-token block.  A wave holds 64 / LW runs of the same LW lanes: runs are
// composed inside a wave with shuffles and across waves through LDS, both
// in a fixed order.
//
// FIXED: the fixed-coefficient forward of _fused_clenshaw_ema_kernel
// (sdpc_kernel.py:988-1209) on the same machinery: one chunk of S tokens, x
// as given (no bf16 rounding), the 8-term Clenshaw fallback above four
// coefficients (1148-1156; the megakernel's fallback stops at four,
// 2070-2077), the EMA from ema_init with the carried state clamped to
// [-1, 1] at every clamp_tile-th token boundary (the kernel's tile carry,
// 1193-1200), out = clamp(s) in fp32, x_norm and tanh_y stored, the state
// after token S-1 to ema_final; no proxy gradient and no Lion.
template <typename XT, int KP, bool LUT, int LW, bool FIXED, typename P>
__global__ void __launch_bounds__(kV10Groups * LW) v10_chunked_kernel(const P p) {
  static_assert(FIXED == std::is_same<P, V10FixedParams>::value, "fixed forward, fixed parameters");
  constexpr int kThreads = kV10Groups * LW;
  constexpr int GPW = 64 / LW;        // runs per wave
  constexpr int R = kV10Run;
  __shared__ V10Lds<LW> L;
  const int tid = threadIdx.x;
  const int l = tid % LW, g = tid / LW;
  const int wave = tid >> 6, gw = (tid & 63) / LW;   // run inside the wave
  int lg = blockIdx.x % p.n_lg;
  int bh = blockIdx.x / p.n_lg;
  if constexpr (kXcdLines) {
    // Workgroups go to the 8 XCDs round-robin by index.  The 128 / (4 LW)
    // consecutive lane groups of a head that share 128-byte lines of x (fp32)
    // are given indices with the same residue mod 8, so their lines are
    // fetched into one XCD's L2 once.
    constexpr int kShare = 128 / (4 * LW);
    const int grid = gridDim.x;
    if (p.n_lg % kShare == 0 && grid % (8 * kShare) == 0) {
      const int v = blockIdx.x, xcd = v & 7, slot = v >> 3;
      const int line = (slot / kShare) * 8 + xcd;          // line group, global
      const int q = slot % kShare;
      const int lines_per_head = p.n_lg / kShare;
      lg = (line % lines_per_head) * kShare + q;
      bh = line / lines_per_head;
    }
  }
  const int h = bh % p.H, b = bh / p.H;
  const int j = lg * LW + l;                 // lane inside the head
  const bool lane_ok = j < p.hd;
  const int d = h * p.hd + j;

  // Tables and the lanes' starting coefficients and momentum (the fixed
  // forward with S = 0 has neither: it only passes ema_init through).
  const bool rows = !FIXED || p.S > 0;
  if constexpr (LUT) {
    if (rows)
      for (int i = tid; i < 256 * 8; i += kThreads) L.lut[i % 256][i / 256] = p.lut[i];
  }
  if (tid < KP * LW) {
    const int k = tid / LW, ll = tid % LW, jj = lg * LW + ll;
    const bool ok = rows && jj < p.hd && k < p.K;
    L.cs[k][ll] = ok ? p.coeffs[(int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)k * p.c_sk + jj] : 0.0f;
    L.ms[k][ll] = ok && !FIXED ? p.momentum[(int64_t)b * p.m_sb + (int64_t)h * p.m_sh + (int64_t)k * p.m_sk + jj] : 0.0f;
  }
  const float gamma = 0.98f - 0.06f * (float)h / (float)p.H;
  const float mu = p.mu_dev ? *p.mu_dev : p.mu, one_m = 1.0f - mu;
  // Decays of full blocks (every token valid): a run's mu^R as the runs
  // form it, its powers for the scan steps, and this thread's weights of the
  // earlier waves' maps.
  struct {
    float run_pow[4];                 // ar^(2^j), ar = mu^R
    float run_lead;                   // ar^gw: runs of this wave before this thread's
    float wave_pow;                   // aw^wave, aw = ar^GPW
    float wave_w[V10Lds<LW>::NW];     // aw^(wave-1-q) for q < wave, else 0
  } kc;
  {
    float ar = 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) ar *= mu;
    kc.run_pow[0] = ar;
#pragma unroll
    for (int j = 1; j < 4; ++j) kc.run_pow[j] = kc.run_pow[j - 1] * kc.run_pow[j - 1];
    float aw = 1.0f;
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg) aw *= ar;
    kc.run_lead = 1.0f;
    for (int gg = 0; gg < gw; ++gg) kc.run_lead *= ar;
    kc.wave_pow = 1.0f;
    for (int q = 0; q < wave; ++q) kc.wave_pow *= aw;
    float pw = 1.0f;
#pragma unroll
    for (int q = V10Lds<LW>::NW - 1; q >= 0; --q) {
      kc.wave_w[q] = q < wave ? pw : 0.0f;
      if (q < wave) pw *= aw;
    }
  }
  // Lion constants of this thread's (k, lane) slot, loaded once (the threads
  // tid < KP * LW apply Lion after every chunk).
  float lion_lr = 0.0f, lion_decay = 0.0f, lion_ss = 0.0f;
  if (!FIXED && tid < KP * LW) {
    const int k = tid / LW;
    lion_lr = p.base_lr * p.lr_scale[h];
    float lam = p.lion_lambda[h];
    if (p.dyn_lambda) lam = __builtin_fminf(__builtin_fmaxf(lam + 0.008f * (p.dyn_lambda[b] - 0.5f), 0.90f), 0.9999f);
    if (p.gate) lion_lr *= p.gate[b];
    lion_decay = lam - lion_lr * p.wd;
    lion_ss = k < p.K ? p.spectral_scale[k] : 0.0f;
  }

  // This batch row of x, out and z.  Descriptors are rebased at each block
  // (uniform row t_blk) and end after row S-1, so a batch row may exceed the
  // 31-bit reach of one descriptor; a thread's offsets stay inside its block
  // (the host checks that 257 rows fit).  Rows past S read 0, stores past S
  // are dropped.
  const char* const xb0 = static_cast<const char*>(p.x) + (int64_t)b * p.x_sb * (int64_t)sizeof(XT);
  const char* const ob0 = reinterpret_cast<const char*>(p.out) + (int64_t)b * p.o_sb * 4;
  const char* const zb0 = p.z_save ? static_cast<const char*>(p.z_save) + (int64_t)b * p.z_sb * 2 : ob0;
  auto rows_from = [&](const char* base, int64_t stride, int64_t elem, int t_blk) {
    return make_rsrc(base + (int64_t)t_blk * stride * elem, ((uint64_t)(p.S - 1 - t_blk) * stride + p.D) * elem);
  };
  const uint32_t x_row = (uint32_t)(p.x_ss * sizeof(XT));   // bytes per token
  const uint32_t o_row = (uint32_t)(p.o_ss * 4);
  const uint32_t z_row = (uint32_t)(p.z_ss * 2);
  const char* xnb0 = ob0;
  const char* tyb0 = ob0;
  uint32_t xn_row = 0, ty_row = 0;
  if constexpr (FIXED) {
    if (p.xnorm) xnb0 = reinterpret_cast<const char*>(p.xnorm) + (int64_t)b * p.xn_sb * 4;
    if (p.tanhy) tyb0 = reinterpret_cast<const char*>(p.tanhy) + (int64_t)b * p.ty_sb * 4;
    xn_row = (uint32_t)(p.xn_ss * 4);
    ty_row = (uint32_t)(p.ty_ss * 4);
  }
  __syncthreads();

  // x rows of a run, double-buffered: the rows of the next block (or of the
  // next chunk's first block) are in flight while this block computes.  A
  // run also loads the row after it (the next run's first token, or the
  // first token after the block), for the pair (t, t+1) of its last token.
  // Rows past S read 0; rows past the chunk are loaded but not used.
  const int n_chunks = (p.S + p.chunk - 1) / p.chunk;
  float xcur[R + 1], xnxt[R + 1];
  // Rows of this thread's run in the block starting at row t_blk.
  auto load_run = [&](float (&dst)[R + 1], int t_blk) {
    const Rsrc xr = rows_from(xb0, p.x_ss, (int64_t)sizeof(XT), t_blk);
    const uint32_t vo_ = lane_ok ? (uint32_t)(g * R) * x_row + (uint32_t)(d * sizeof(XT)) : kOffOOB;
    uint32_t so = 0;
#pragma unroll
    for (int r = 0; r <= R; ++r) {
      dst[r] = load_x<XT>(xr, vo_, so);
      so = next_off(so, x_row);
    }
  };
  // The part of pass 1 that does not depend on the coefficients, per token:
  // x as bf16, the softsign, and with the LUT (rows) the table index, the
  // fraction and the table rows at both points.
  struct TokPre {
    float xb, absu, sgn, fr;
    float ta[KP], tb[KP];
  };
  auto prep = [&](float xr, TokPre& f, bool with_rows) {
    f.xb = FIXED ? xr : to_bf16_value<XT>(xr);
    v10_softsign(f.xb, f.absu, f.sgn);
    if constexpr (LUT) {
      if (!with_rows) return;
      const float fidx = f.absu * 255.0f;
      const int i0 = min((int)fidx, 254);
      f.fr = __builtin_fminf(__builtin_fmaxf(fidx - (float)i0, 0.0f), 1.0f);
      const f32x4* ra = reinterpret_cast<const f32x4*>(&L.lut[i0][0]);
      const f32x4* rb = reinterpret_cast<const f32x4*>(&L.lut[i0 + 1][0]);
#pragma unroll
      for (int q4 = 0; q4 < KP / 4; ++q4) {
        const f32x4 va = ra[q4], vb = rb[q4];
        f.ta[4 * q4] = va.x; f.ta[4 * q4 + 1] = va.y; f.ta[4 * q4 + 2] = va.z; f.ta[4 * q4 + 3] = va.w;
        f.tb[4 * q4] = vb.x; f.tb[4 * q4 + 1] = vb.y; f.tb[4 * q4 + 2] = vb.z; f.tb[4 * q4 + 3] = vb.w;
      }
    }
  };
  // Token 0 of every run is prepared ahead of its block, so that its table
  // reads are off the chunk's chain: for a chunk's first block by the first
  // wave of each SIMD while it waits for the second at the reduction
  // barrier, and by the others while wave 0 applies Lion.  Measured at the
  // configs[1] shape, bit-identical: one token ahead, all waves during
  // Lion, 152.6-153.7 against 153.9-155.0 us; two and three tokens ahead
  // 162.6 and 170.2 us (their reads outgrow the window); the first waves
  // before the barrier 150.4-150.6 against 151.1-151.6 us.
  TokPre f0;
  if (!FIXED || n_chunks > 0) load_run(xcur, 0);   // (the fixed forward takes S = 0: no rows)
  // Wait for these rows here, once.  Without it the compiler, merging this
  // path with the loop's back edge, waits for the next block's prefetched
  // rows at the start of every block (vmcnt 4..1 before each row's use),
  // which exposes a full memory latency per chunk (283 against 299 us at
  // the configs[1] shape).  s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15).
  __builtin_amdgcn_s_waitcnt(0xF70);
  if (!FIXED || n_chunks > 0) prep(xcur[0], f0, true);

  for (int ch = 0; ch < n_chunks; ++ch) {
    const int t_chunk = ch * p.chunk;
    const int len = min(p.chunk, p.S - t_chunk);
    float c[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k) c[k] = L.cs[k][l];
    if (p.coeff_hist && g == 0 && lane_ok) {
      float* hst = p.coeff_hist + (size_t)ch * p.B * p.H * p.K * p.hd + (((size_t)b * p.H + h) * p.K) * p.hd + j;
      for (int k = 0; k < p.K && k < KP; ++k) hst[(size_t)k * p.hd] = c[k];
    }
    float gc[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k) gc[k] = 0.0f;
    if (tid < LW) {
      float c0 = 0.0f;
      if constexpr (FIXED) {
        const int jj = lg * LW + tid;
        if (p.ema_init && jj < p.hd) c0 = p.ema_init[(int64_t)b * p.init_sb + h * p.hd + jj];
      }
      L.carry[tid] = c0;
    }

    for (int blk = 0; blk * kBlockTok < len; ++blk) {
      const int r0 = blk * kBlockTok + g * R;            // run start inside the chunk
      const int n_valid = max(0, min(R, len - r0));
      const int t_blk = t_chunk + blk * kBlockTok;         // block start in the sequence
      // Prefetch the next block's rows.
      int t_next = -1;
      if ((blk + 1) * kBlockTok < len)
        t_next = t_chunk + (blk + 1) * kBlockTok;
      else if (ch + 1 < n_chunks)
        t_next = t_chunk + p.chunk;
      if (t_next >= 0) load_run(xnxt, t_next);
      const Rsrc orr = rows_from(ob0, p.o_ss, 4, t_blk);
      const Rsrc zr = rows_from(zb0, p.z_save ? p.z_ss : p.o_ss, p.z_save ? 2 : 4, t_blk);

      float u[R + 1], w[R], zs[R];
      float A = 1.0f, Bv = 0.0f;
      // A block whose runs are all inside the chunk skips the per-token
      // checks (each loop below comes in both versions; the choice is the
      // same for the whole workgroup): only the last token of a run may
      // lack its pair (the chunk's last token), checked once per run.
      // (the fixed-coefficient forward takes the general path, whose wave
      // composition clamps the carried state at tile boundaries)
      const bool full = !FIXED && (blk + 1) * kBlockTok <= len;
      auto pass1 = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
        for (int r = 0; r <= R; ++r) {
          TokPre tp;
          if (r > 0) prep(xcur[r], tp, r < R);   // the row after the run: u only
          const TokPre& f = r == 0 ? f0 : tp;
          const float xb = f.xb, sgn = f.sgn;
          u[r] = sgn * f.absu;
          if (r == R) break;
          float y;
          if constexpr (LUT) {
            const float fr = f.fr;
            const float* ta = f.ta;
            const float* tb = f.tb;
            // the series at both table points, then one interpolation (linear
            // in the table: the value of interpolating each T_k, up to rounding)
            float ae = 0.0f, ao = 0.0f, be = 0.0f, bo = 0.0f;
#pragma unroll
            for (int k = 0; k < KP; ++k) {
              if (k & 1) {
                ao = __builtin_fmaf(c[k], ta[k], ao);
                bo = __builtin_fmaf(c[k], tb[k], bo);
              } else {
                ae = __builtin_fmaf(c[k], ta[k], ae);
                be = __builtin_fmaf(c[k], tb[k], be);
              }
            }
            const float ya = __builtin_fmaf(sgn, ao, ae), yb = __builtin_fmaf(sgn, bo, be);
            y = __builtin_fmaf(fr, yb - ya, ya);
          } else if (FIXED && KP > 4) {
            // Clenshaw over all eight terms, as _fused_clenshaw_ema_kernel
            // above four coefficients: b_k = 2u b_{k+1} - b_{k+2} + c_k,
            // y = u b_1 - b_2 + c_0 (zeros past K).
            const float uu = u[r], u2 = uu + uu;
            float bk1 = c[KP - 1], bk2 = 0.0f;
#pragma unroll
            for (int k = KP - 2; k >= 1; --k) {
              const float bk = __builtin_fmaf(u2, bk1, c[k]) - bk2;
              bk2 = bk1;
              bk1 = bk;
            }
            y = __builtin_fmaf(uu, bk1, c[0]) - bk2;
          } else {
            const float uu = u[r], u2 = uu + uu;
            const float c3 = c[3], c2 = c[2];
            const float b2 = __builtin_fmaf(u2, c3, c2);
            const float b1 = __builtin_fmaf(u2, b2, c[1]) - c3;
            y = __builtin_fmaf(uu, b1, c[0]) - b2;
          }
          const float yc = __builtin_amdgcn_fmed3f(gamma * y, -4.0f, 4.0f);
          const float e2 = __builtin_amdgcn_exp2f(2.0f * kLog2e * yc);
          float z = (e2 - 1.0f) * __builtin_amdgcn_rcpf(e2 + 1.0f);
          z = xb == xb ? z : 0.0f;
          w[r] = one_m * z;
          if (FULL || r < n_valid) {
            Bv = __builtin_fmaf(mu, Bv, w[r]);
            A *= mu;
          }
          zs[r] = z;
        }
        // z for the backward after the loop (a branch per token would cut the
        // run into one basic block per token)
        if (p.z_save) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (FULL || r < n_valid) {
              // default cache policy, as for out
              __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (__bf16)zs[r]), zr,
                                                    lane_ok ? (uint32_t)(g * R) * z_row + (uint32_t)(d * 2) : kOffOOB,
                                                    (uint32_t)r * z_row, 0);
            }
          }
        }
        if constexpr (FIXED) {
          // x_norm = u and tanh_y = z of the valid tokens, fp32
          const uint32_t xo = lane_ok ? (uint32_t)(g * R) * xn_row + (uint32_t)(d * 4) : kOffOOB;
          const uint32_t yo = lane_ok ? (uint32_t)(g * R) * ty_row + (uint32_t)(d * 4) : kOffOOB;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (r < n_valid) {
              if (p.xnorm)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(u[r]), rows_from(xnb0, p.xn_ss, 4, t_blk), xo,
                                                      (uint32_t)r * xn_row, 0);
              if (p.tanhy)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(zs[r]), rows_from(tyb0, p.ty_ss, 4, t_blk), yo,
                                                      (uint32_t)r * ty_row, 0);
            }
          }
        }
      };
      if (full)
        pass1(std::true_type{});
      else
        pass1(std::false_type{});
      // Compose the runs: inclusive scan inside the wave (later map applied
      // after earlier: A = A_l A_e, B = A_l B_e + B_l), then the waves.
      float s;
      if (full) {
        // Every run of a full block decays by ar = mu^R and every wave by aw =
        // mu^(R GPW): the scan carries B alone with constant factors, and the
        // state before wave q is carry aw^q + sum_{p<q} aw^(q-1-p) B_p, the
        // waves' B read together (every wave waits one LDS round trip, not q).
        float iB = Bv;
#pragma unroll
        for (int o = 1, j = 0; o < GPW; o <<= 1, ++j) {
          const float pB = __shfl_up(iB, o * LW, 64);
          if (gw >= o) iB = __builtin_fmaf(kc.run_pow[j], pB, iB);
        }
        float eB = __shfl_up(iB, LW, 64);
        if (gw == 0) eB = 0.0f;
        if (gw == GPW - 1) L.wB[wave][l] = iB;
        __syncthreads();
        float sw = L.carry[l] * kc.wave_pow;
#pragma unroll
        for (int q = 0; q < V10Lds<LW>::NW; ++q) sw = __builtin_fmaf(kc.wave_w[q], L.wB[q][l], sw);
        s = __builtin_fmaf(kc.run_lead, sw, eB);
      } else {
        float iA = A, iB = Bv;
#pragma unroll
        for (int o = 1; o < GPW; o <<= 1) {
          const float pA = __shfl_up(iA, o * LW, 64), pB = __shfl_up(iB, o * LW, 64);
          if (gw >= o) {
            iB = __builtin_fmaf(iA, pB, iB);
            iA *= pA;
          }
        }
        float eA = __shfl_up(iA, LW, 64), eB = __shfl_up(iB, LW, 64);
        if (gw == 0) {
          eA = 1.0f;
          eB = 0.0f;
        }
        if (gw == GPW - 1) {
          L.wA[wave][l] = iA;
          L.wB[wave][l] = iB;
        }
        __syncthreads();
        s = L.carry[l];
        for (int q = 0; q < wave; ++q) {
          s = __builtin_fmaf(L.wA[q][l], s, L.wB[q][l]);
          if constexpr (FIXED) {
            // the carried state at a tile boundary (token t_blk + (q+1) GPW R)
            if ((t_blk - t_chunk + (q + 1) * GPW * R) % p.clamp_tile == 0) s = __builtin_amdgcn_fmed3f(s, -1.0f, 1.0f);
          }
        }
        s = __builtin_fmaf(eA, s, eB);
      }
      // Replay, store bf16(s), proxy gradient.
      const uint32_t ovo = lane_ok ? (uint32_t)(g * R) * o_row + (uint32_t)(d * 4) : kOffOOB;
      auto replay = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (FULL || r < n_valid) {
            s = __builtin_fmaf(mu, s, w[r]);
            const float so = __builtin_amdgcn_fmed3f(s, -1.0f, 1.0f);
            const float ov[1] = {FIXED ? so : (float)(__bf16)so};
            // default cache policy: the 32-byte pieces that the workgroups of
            // one XCD store into a 128-byte line merge in its L2 before they
            // are written (non-temporal stores reached HBM as partial lines:
            // 1.84x the output bytes)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ov[0]), orr, ovo, (uint32_t)r * o_row, 0);
            if (!FIXED && ((FULL && r + 1 < R) || r0 + r + 1 < len)) {
              const float err = u[r + 1] - so;
              const float gv = err * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-3.0f * kLog2e * __builtin_fabsf(err)));
              const float uu = u[r], u2 = uu + uu;
              gc[0] += gv;
              if constexpr (KP > 1) gc[1] = __builtin_fmaf(gv, uu, gc[1]);
              float tm2 = 1.0f, tm1 = uu;
#pragma unroll
              for (int k = 2; k < KP; ++k) {
                const float tk = __builtin_fmaf(u2, tm1, -tm2);
                gc[k] = __builtin_fmaf(gv, tk, gc[k]);
                tm2 = tm1;
                tm1 = tk;
              }
            }
          }
        }
      };
      if (full)
        replay(std::true_type{});
      else
        replay(std::false_type{});
      if constexpr (FIXED) {
        // the clamped state after token S-1, from the run that holds it
        if (p.ema_final && lane_ok && n_valid > 0 && r0 + n_valid == len)
          p.ema_final[(int64_t)b * p.final_sb + d] = __builtin_amdgcn_fmed3f(s, -1.0f, 1.0f);
      }
      if (len > kBlockTok) {
        // The next block of this chunk starts from this block's end state
        // (a one-block chunk has no next block: the carry restarts at 0).
        __syncthreads();   // all reads of the carry and the wave maps done
        if (g == kV10Groups - 1) {
          // state after the block's last valid token (invalid tokens are skipped)
          float cs = s;
          if constexpr (FIXED)
            if ((t_blk - t_chunk + kBlockTok) % p.clamp_tile == 0) cs = __builtin_amdgcn_fmed3f(cs, -1.0f, 1.0f);
          L.carry[l] = cs;
        }
        __syncthreads();
      }
#pragma unroll
      for (int r = 0; r <= R; ++r) xcur[r] = xnxt[r];
      if ((blk + 1) * kBlockTok < len) prep(xcur[0], f0, true);   // the next block of this chunk
    }

    if constexpr (FIXED) continue;   // no proxy gradient, no Lion
    // Reduce the proxy gradient over the runs (a fixed butterfly inside each
    // wave, reduce-scattered over the coefficients, then the waves in
    // order), then Lion.
    store_run_sums<LW, KP>(gc, L.ws[wave], l, gw);
    // The first wave of each SIMD reaches the barrier early: it prepares its
    // token 0 of the next chunk here, the others while Lion runs.
    const bool early = wave < V10Lds<LW>::NW / 2;
    if (early && ch + 1 < n_chunks) prep(xcur[0], f0, true);
    __syncthreads();
    if (tid < KP * LW) {
      const int k = tid / LW, ll = tid % LW;
      float G = 0.0f;
#pragma unroll
      for (int q = 0; q < V10Lds<LW>::NW; ++q) G += L.ws[q][k][ll];
      if (k < p.K) {
        const float inv_s = 1.0f / (float)(len - 1);   // len = 1: inf, as the reference (NaN momentum)
        const float gk = G * inv_s;
        const float m = L.ms[k][ll];
        const float interp = p.beta1 * m + (1.0f - p.beta1) * gk;
        const float sg = interp > 0.0f ? 1.0f : (interp < 0.0f ? -1.0f : 0.0f);
        L.ms[k][ll] = p.beta2 * m + (1.0f - p.beta2) * gk;
        L.cs[k][ll] = lion_decay * L.cs[k][ll] + lion_lr * lion_ss * sg;
      }
    }
    // token 0 of the next chunk's first block, while Lion runs
    if (!early && ch + 1 < n_chunks) prep(xcur[0], f0, true);
    __syncthreads();
  }

  if constexpr (FIXED) {
    // No tokens: the state passes through unclamped, as the reference's
    // carry does when its tile loop runs zero times.
    if (p.S == 0 && p.ema_final && tid < LW && lg * LW + tid < p.hd) {
      const int jj = lg * LW + tid;
      p.ema_final[(int64_t)b * p.final_sb + h * p.hd + jj] =
          p.ema_init ? p.ema_init[(int64_t)b * p.init_sb + h * p.hd + jj] : 0.0f;
    }
  }
  if (!FIXED && tid < KP * LW) {
    const int k = tid / LW, ll = tid % LW, jj = lg * LW + ll;
    if (jj < p.hd && k < p.K) {
      const size_t o = (((size_t)b * p.H + h) * p.K + k) * p.hd + jj;
      p.coeffs_out[o] = L.cs[k][ll];
      p.momentum_out[o] = L.ms[k][ll];
    }
  }
}

template <typename XT, bool LUT, int LW, bool FIXED, typename P>
hipError_t launch_w(const P& p, int kpad, hipStream_t stream) {
  const unsigned grid = (unsigned)(p.B * p.H * p.n_lg);
  if (kpad == 4)
    hipLaunchKernelGGL((v10_chunked_kernel<XT, 4, LUT, LW, FIXED, P>), dim3(grid), dim3(kV10Groups * LW), 0, stream, p);
  else
    hipLaunchKernelGGL((v10_chunked_kernel<XT, 8, LUT, LW, FIXED, P>), dim3(grid), dim3(kV10Groups * LW), 0, stream, p);
  return hipGetLastError();
}

template <typename XT, bool LUT, bool FIXED, typename P>
hipError_t launch_x(const P& p, int kpad, hipStream_t stream) {
  if (p.lanes == 8) return launch_w<XT, LUT, 8, FIXED>(p, kpad, stream);
  if (p.lanes == 16) return launch_w<XT, LUT, 16, FIXED>(p, kpad, stream);
  return hipErrorInvalidValue;
}

}  // namespace

int v10_lanes(int64_t B, int64_t H, int64_t hd) {
  return B * H * ((hd + 15) / 16) >= 512 ? 16 : 8;
}

hipError_t launch_v10(const V10Params& p, int x_dtype, bool use_lut, int kpad, hipStream_t stream) {
  if (x_dtype == 0)
    return use_lut ? launch_x<float, true, false>(p, kpad, stream) : launch_x<float, false, false>(p, kpad, stream);
  return use_lut ? launch_x<__bf16, true, false>(p, kpad, stream) : launch_x<__bf16, false, false>(p, kpad, stream);
}

hipError_t launch_v10_fixed(const V10FixedParams& p, int x_dtype, bool use_lut, int kpad, hipStream_t stream) {
  if (x_dtype == 0)
    return use_lut ? launch_x<float, true, true>(p, kpad, stream) : launch_x<float, false, true>(p, kpad, stream);
  return use_lut ? launch_x<__bf16, true, true>(p, kpad, stream) : launch_x<__bf16, false, true>(p, kpad, stream);
}

}  // namespace osm
