// fbs_run.h - the SpiralCore/FBS integer decode step for gfx950 (MI355X): the device code of
// the three kernels (fbs_prefill.hip, fbs_decode.hip, fbs_rows.hip), which differ only in the
// phase compiled in.
//
// One 64-lane wavefront runs one sequence through every step of its run (teacher-forced
// sequences, greedy decode, or scoring). Per step (RS crates/uor-r4-integer/src/stack/
// session.rs:4129-4403 `stack_step_fbs`; twin fbs_core.h:635-675):
//   the token's writer row in; per layer the fine RMSNorm and gain, the FBS projections
//   (gathers through LDS by a precomputed per-lane program), the quaternion recurrence with its
//   output gate and the causal window read from the sequence's ring in HBM, the shared-exponent
//   requantize and residual add, and the same for the Hamilton feed-forward gate; the final
//   norm, the Q12 query, and the drawer writer (drawer scores, P rounds of lowest
//   (score, drawer), then the lowest (L1, token) over the kept drawers' CSR members, scanned by
//   lane groups of d/32 lanes with packed v_sad_u16 on biased rows).
// The recurrence state of every layer stays in LDS for the whole run; only the window ring,
// the table rows and the outputs touch HBM. Reductions are exact integer max, sum and
// lexicographic min over DPP lane exchanges, so the outputs do not depend on lane order.
// A block is one wavefront: lanes hand data to each other through LDS under wavefront-scope
// fences (LDS operations of a wavefront complete in order), never through a workgroup barrier.
#ifndef UOR_FBS_RUN_H
#define UOR_FBS_RUN_H

#include <hip/hip_runtime.h>

#include "fbs_device.h"
#include "fbs_int.h"

namespace fbs {

static_assert(kRsqrtSeedWords + kRecipSeedWords == kSeedWords, "seed table size");

// ---------------------------------------------------------------------------------------------
// Wave-level primitives.

// Paired blocks of two or more quaternions a lane, or with Hamming reads, keep the recurrence
// state in a per-block global buffer (beside the window sums) instead of LDS, so that four of
// their blocks share a CU's LDS.
template <int Q, bool HM = false>
constexpr bool kPairStateGlobal = Q >= 2 || HM;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kDppXor1 = 0xb1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  uint32_t lo = dpp32<CTRL>((uint32_t)v), hi = dpp32<CTRL>((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t uniform32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint32_t lane32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t lane64(uint64_t v, int l) {
  return ((uint64_t)lane32((uint32_t)(v >> 32), l) << 32) | lane32((uint32_t)v, l);
}

struct OpMax {
  template <class T>
  __device__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct OpMin {
  template <class T>
  __device__ T operator()(T a, T b) const { return a < b ? a : b; }
};
struct OpAdd {
  template <class T>
  __device__ T operator()(T a, T b) const { return a + b; }
};

// The op over all 64 lanes, returned uniform: butterflies inside each row of 16, then the four
// row results read as scalars.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce32(uint32_t v, Op op) {
  v = op(v, dpp32<kDppXor1>(v));
  v = op(v, dpp32<kDppXor2>(v));
  v = op(v, dpp32<kDppHalfMirror>(v));
  v = op(v, dpp32<kDppMirror>(v));
  return op(op(lane32(v, 0), lane32(v, 16)), op(lane32(v, 32), lane32(v, 48)));
}
template <class Op>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, Op op) {
  v = op(v, dpp64<kDppXor1>(v));
  v = op(v, dpp64<kDppXor2>(v));
  v = op(v, dpp64<kDppHalfMirror>(v));
  v = op(v, dpp64<kDppMirror>(v));
  return op(op(lane64(v, 0), lane64(v, 16)), op(lane64(v, 32), lane64(v, 48)));
}
// The wave's maximum of m and sum of s together, both returned uniform: each exchange step is
// applied to both before the next, so one reduction's DPP waits are filled with the other's work.
__device__ __forceinline__ void wave_max32_add64(uint32_t &m, uint64_t &s) {
  m = OpMax()(m, dpp32<kDppXor1>(m));
  s += dpp64<kDppXor1>(s);
  m = OpMax()(m, dpp32<kDppXor2>(m));
  s += dpp64<kDppXor2>(s);
  m = OpMax()(m, dpp32<kDppHalfMirror>(m));
  s += dpp64<kDppHalfMirror>(s);
  m = OpMax()(m, dpp32<kDppMirror>(m));
  s += dpp64<kDppMirror>(s);
  m = OpMax()(OpMax()(lane32(m, 0), lane32(m, 16)), OpMax()(lane32(m, 32), lane32(m, 48)));
  s = (lane64(s, 0) + lane64(s, 16)) + (lane64(s, 32) + lane64(s, 48));
}
// The bit length of the wave's largest magnitude from each lane's largest: the bit length of a
// maximum is the maximum of the bit lengths, so a 32-bit reduction takes the place of a 64-bit one.
__device__ __forceinline__ int32_t wave_bitlen_max(uint64_t v) {
  return (int32_t)wave_reduce32((uint32_t)bitlen64(v), OpMax());
}

// Sums over aligned groups of S lanes (S a power of two), every lane of a group getting its
// group's sum, for U independent values at once (each exchange step is applied to all U before
// the next, so the DPP read-after-write waits are filled with independent work).
template <int S, int U>
__device__ __forceinline__ void group_sums(uint32_t (&v)[U]) {
  if constexpr (S >= 2) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += dpp32<kDppXor1>(v[u]);
  }
  if constexpr (S >= 4) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += dpp32<kDppXor2>(v[u]);
  }
  if constexpr (S >= 8) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += dpp32<kDppHalfMirror>(v[u]);
  }
  if constexpr (S >= 16) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += dpp32<kDppMirror>(v[u]);
  }
  if constexpr (S >= 32) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += (uint32_t)__shfl_xor((int)v[u], 16);
  }
  if constexpr (S >= 64) {
#pragma unroll
    for (int u = 0; u < U; u++) v[u] += (uint32_t)__shfl_xor((int)v[u], 32);
  }
}

// v_sad_u16 on gfx950 sums the absolute differences of both 16-bit halves:
// d = |a[15:0] - b[15:0]| + |a[31:16] - b[31:16]| + c (unsigned halves; measured on MI355X and
// held by the parity tests). Inline asm keeps the optimiser from reasoning about the halves.
__device__ __forceinline__ uint32_t sad2_u16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_sad_u16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// x mod W for the model's window W through its reciprocal M.w_recip = floor(2^32 / W), which the
// host forms: q = floor(x w_recip / 2^32) is floor(x / W) or one less (x < 2^32), so the remainder
// x - q W lies in [0, 2 W) and one step fixes it. The kernels divide by no variable with the
// compiler's `%`, whose expansion goes through a float reciprocal estimate.
__device__ __forceinline__ uint32_t mod_window(const DevModel &M, uint32_t x) {
  const uint32_t q = (uint32_t)(((uint64_t)x * M.w_recip) >> 32);
  const uint32_t r = x - q * M.W;
  return r >= M.W ? r - M.W : r;
}

// One state word's share of a slot state's fingerprint: the word and its index mixed by
// multiplication (splitmix64's constants), summed over the state's words modulo 2^32.
__device__ __forceinline__ uint32_t state_fp_word(int64_t v, uint32_t index) {
  const uint64_t u = (uint64_t)v ^ ((uint64_t)index * 0x9E3779B97F4A7C15ull);
  const uint64_t m = (u ^ (u >> 31)) * 0xBF58476D1CE4E5B9ull;
  return (uint32_t)(m >> 32) ^ (uint32_t)m;
}

// ---------------------------------------------------------------------------------------------
// Step pieces.

// Out of line: the step's rare forms (wide sums, slow grid codes, widths that are not powers of
// two), so that the served loop's hot code stays compact in the instruction cache.
__device__ __noinline__ NormFactor norm_factor_slow(uint64_t sum, uint32_t n, int64_t eps) {
  return norm_factor(sum, n, eps);
}
// The power-of-two widths' RMSNorm factor as one shared copy for the kernel's norms: the
// lane-parallel form (norm_factor_wave, every lane of the wave active), or norm_factor_pow2 for
// an input outside its estimates' ranges. `seed_lds`: the block's seed tables in LDS.
typedef __attribute__((address_space(3))) const uint32_t lds_u32;
__device__ __noinline__ NormFactor norm_factor_lds(uint64_t sum, uint32_t log2n, int64_t eps,
                                                   lds_u32 *seed_lds) {
  const uint32_t *seeds = (const uint32_t *)seed_lds;
  const Seeds sd(seeds, seeds + kRsqrtSeedWords);
  bool ok;
  NormFactor f = norm_factor_wave(sum, log2n, eps, sd, ok);
  if (!ok) f = norm_factor_pow2(sum, log2n, eps, sd);
  return f;
}
__device__ __noinline__ int64_t norm_gain_slow(uint64_t r, uint32_t huge, int64_t y, uint32_t desc,
                                               int32_t code) {
  NormFactor f;
  f.r = r;
  f.huge = huge != 0;
  return grid_apply64_desc(norm_apply24(f, y), (uint16_t)desc, (int16_t)code);
}
// shift_wide(mh 2^32 + ml + (keep wide) << 16, 31) (raw: the split form of hamilton32_hl) or of
// (mh 2^64 + ml) + (keep wide) << 16 (a snapped transition's i128).
__device__ __noinline__ int64_t transport_wide(int64_t mh, int64_t ml, uint64_t keep, int64_t wide,
                                               uint32_t raw) {
  const i128 moved = raw ? ((i128)mh << 32) + (i128)ml
                         : (i128)(((u128)(uint64_t)mh << 64) | (u128)(uint64_t)ml);
  const u128 drive_term = (u128)((i128)keep * (i128)wide) << 16;
  return shift_wide((i128)((u128)moved + drive_term), 31);
}
__device__ __noinline__ int64_t gate_wide14(int64_t gh, int64_t gl) {
  return shift_wide(((i128)gh << 32) + (i128)gl, 14);
}

// Fine RMSNorm then the per-channel grid gain, for the lane's channels
// (RS stack/kernels.rs:569-620, session.rs:4057-4061). gain: the lane's 4 codes per quaternion.
template <int Q>
__device__ __forceinline__ void norm_gain(const DevModel &M, const Seeds &sd,
                                          const int32_t (&x)[Q][4], const bool (&qv)[Q],
                                          const short4 (&gain)[Q], const ushort4 (&gdesc)[Q],
                                          int64_t (&out)[Q][4]) {
  // The largest magnitude and, beside it, the sum of squares as if the pre-shift were 0 (it is
  // wherever the largest magnitude is below 2^24, and then every square is below 2^48): both
  // reductions run interleaved, and only a non-zero pre-shift sums the shifted values again.
  uint32_t mx = 0;
  uint64_t sum = 0;
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k])
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const uint32_t a = uabs32(x[k][c]);
        mx = a > mx ? a : mx;
        sum += (uint64_t)a * a;  // used only when every a < 2^24
      }
  wave_max32_add64(mx, sum);
  int32_t sh = bitlen64(mx) - 24;
  if (sh < 0) sh = 0;
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) out[k][c] = qv[k] ? (int64_t)x[k][c] : 0;
  if (sh > 0) {
    sum = 0;
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int64_t y = qv[k] ? shift((int64_t)x[k][c], sh) : 0;
        out[k][c] = y;
        const uint32_t a = (uint32_t)uabs64(y);  // |y| <= 2^24: the shift leaves 24 bits
        sum += (uint64_t)a * a;
      }
    sum = wave_reduce64(sum, OpAdd());
  }
  const int64_t eps = sh == 0 ? M.eps0 : M.eps_int[sh];
  const NormFactor f = M.log2d != 0xffu ? norm_factor_lds(sum, M.log2d, eps, (lds_u32 *)sd.rsq_seed)
                                         : norm_factor_slow(sum, M.d, eps);
  if (!f.huge && M.gains_fast) {
    // The common case, one uniform branch: r < 2^62 and |y| <= 2^24 keep every normed value
    // below 2^48 in magnitude, where each gain's descriptor form is exact.
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const uint16_t gd[4] = {gdesc[k].x, gdesc[k].y, gdesc[k].z, gdesc[k].w};
#pragma unroll
      for (int c = 0; c < 4; c++) out[k][c] = grid_desc_apply(norm_apply24_fast(f, out[k][c]), gd[c]);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < Q; k++) {
    const int16_t gc[4] = {gain[k].x, gain[k].y, gain[k].z, gain[k].w};
    const uint16_t gd[4] = {gdesc[k].x, gdesc[k].y, gdesc[k].z, gdesc[k].w};
#pragma unroll
    for (int c = 0; c < 4; c++) out[k][c] = norm_gain_slow(f.r, f.huge, out[k][c], gd[c], gc[c]);
  }
}

// Publish v (exponent -24) for the FBS gathers: word 2 i + s holds to_exp_i32 of v_i (s = 0)
// or of its saturating negation (s = 1), at exponent -16 (session.rs:4037-4053: the negation
// comes before the rounding shift).
template <int Q>
__device__ __forceinline__ void publish64(int32_t *xbar, const int64_t (&v)[Q][4],
                                          const bool (&qv)[Q], const uint32_t (&qi)[Q]) {
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      int32_t p[4], n[4];
#pragma unroll
      for (int c = 0; c < 4; c++) publish64_pair(v[k][c], &p[c], &n[c]);
      int4 *dst = (int4 *)(xbar + 8 * qi[k]);
      dst[0] = make_int4(p[0], n[0], p[1], n[1]);
      dst[1] = make_int4(p[2], n[2], p[3], n[3]);
    }
}

// Publish 16-bit activations at exponent `exp` for gather16 (to_exp_i32 of +-a to -16).
__device__ __forceinline__ void publish16(int32_t *xbar, uint32_t channel0, const int32_t (&a)[4],
                                          int32_t exp) {
  int32_t p[4], n[4];
#pragma unroll
  for (int c = 0; c < 4; c++) publish16_pair(a[c], exp, &p[c], &n[c]);
  int4 *dst = (int4 *)(xbar + 2 * channel0);
  dst[0] = make_int4(p[0], n[0], p[1], n[1]);
  dst[1] = make_int4(p[2], n[2], p[3], n[3]);
}

__device__ __forceinline__ uint32_t prog_word(const uint16_t *prog, uint32_t slot, uint32_t lane) {
  return prog[slot * kWave + lane];
}

// The snapped transition or gate (RS stack/kernels.rs:1474-1557), out of line: the 120-root
// scan is long and served only by snapped artifacts. The quaternion comes back by value (in
// registers), so no caller array lives in private memory.
struct Quat64 {
  int64_t v[4];
  uint32_t root;  // the chosen root's index
};
__device__ __noinline__ Quat64 snap_rotation_dev(const int8_t *ico, int4 raw, uint64_t lambda) {
  const int32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
  Quat64 q;
  q.root = snap_rotation(ico, r, lambda, q.v);
  return q;
}
// The snapped gates' and transitions' 128-bit Hamilton products, out of line (snapped artifacts
// only): shift_wide(q (x) r, sh) by value, or the product's high and low 64 bits.
__device__ __noinline__ Quat64 hamilton64_shift(int64_t q0, int64_t q1, int64_t q2, int64_t q3,
                                                int64_t r0, int64_t r1, int64_t r2, int64_t r3,
                                                uint32_t sh) {
  const int64_t q[4] = {q0, q1, q2, q3}, r[4] = {r0, r1, r2, r3};
  i128 prod[4];
  hamilton64(q, r, prod);
  Quat64 o;
#pragma unroll
  for (int c = 0; c < 4; c++) o.v[c] = shift_wide(prod[c], sh);
  o.root = 0;
  return o;
}
struct Wide4 {
  int64_t hi[4], lo[4];
};
__device__ __noinline__ Wide4 hamilton64_wide(int64_t q0, int64_t q1, int64_t q2, int64_t q3,
                                              int64_t r0, int64_t r1, int64_t r2, int64_t r3) {
  const int64_t q[4] = {q0, q1, q2, q3}, r[4] = {r0, r1, r2, r3};
  i128 prod[4];
  hamilton64(q, r, prod);
  Wide4 o;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    o.hi[c] = (int64_t)(prod[c] >> 64);
    o.lo[c] = (int64_t)(uint64_t)prod[c];
  }
  return o;
}

// The snap trace's byte of a site (fbs_core.h:488-501, claude-134): the chosen root, or 255 where
// none was chosen (served unsnapped) or the raw quaternion is zero.
constexpr uint32_t kTraceNone = 255;
__device__ __forceinline__ uint32_t trace_root(const int32_t (&raw)[4], uint32_t root) {
  return (raw[0] | raw[1] | raw[2] | raw[3]) == 0 ? kTraceNone : root;
}
__device__ __forceinline__ uint32_t snap_rotation_to(const int8_t *ico, int4 raw, uint64_t lambda,
                                                     int64_t (&out)[4]) {
  const Quat64 q = snap_rotation_dev(ico, raw, lambda);
#pragma unroll
  for (int c = 0; c < 4; c++) out[c] = q.v[c];
  return q.root;
}

// The Hamilton gate on rhs (session.rs:4951-4968, :4005-4025): shift_wide(q (x) rhs, 15) with
// q the gate's unit quaternion (lambda 2^31, epsilon 0) or its icosian. Raw gates use q = 2 u
// exactly, so the product is formed from u and shifted by 14.
// Returns the gate's snap trace byte.
__device__ __forceinline__ uint32_t gate_apply(const DevModel &M, const Seeds &sd,
                                               const int32_t (&raw)[4], const int64_t (&rhs)[4],
                                               int64_t (&out)[4]) {
  i128 prod[4];
  if (M.raw_gates) {
    int32_t u[4];
    unit_q30(raw, kGateEps, u, sd);
    hamilton32(u, rhs, prod);
#pragma unroll
    for (int c = 0; c < 4; c++) out[c] = shift_wide(prod[c], 14);
    return kTraceNone;
  }
  int64_t q[4];
  const uint32_t root =
      snap_rotation_to(M.icosian, make_int4(raw[0], raw[1], raw[2], raw[3]), 1ull << 31, q);
  const Quat64 p = hamilton64_shift(q[0], q[1], q[2], q[3], rhs[0], rhs[1], rhs[2], rhs[3], 15);
#pragma unroll
  for (int c = 0; c < 4; c++) out[c] = p.v[c];
  return trace_root(raw, root);
}

// One MLP quaternion of the Hamilton feed-forward gate (session.rs:4005-4025): the gate of gq
// applied to up. Raw gates use q = 2 u, and u (x) up fits in 64 bits.
__device__ __forceinline__ uint32_t mlp_gate(const DevModel &M, const Seeds &sd,
                                             const int32_t (&gq)[4], const int32_t (&up)[4],
                                             int64_t (&mo)[4]) {
  if (M.raw_gates) {
    int32_t u[4];
    int64_t prod[4];
    unit_q30(gq, kGateEps, u, sd);
    hamilton32x32(u, up, prod);
#pragma unroll
    for (int c = 0; c < 4; c++) mo[c] = shift_i64(prod[c], 14);
    return kTraceNone;
  }
  const int64_t up64[4] = {up[0], up[1], up[2], up[3]};
  return gate_apply(M, sd, gq, up64, mo);
}

// gate_apply split in two for paired blocks: gate_quat forms the gate's quaternion (the unit
// quaternion u of a raw gate, or the snapped gate at lambda 2^31), gate_mul applies it.
__device__ __forceinline__ void gate_quat(const DevModel &M, const Seeds &sd, const int32_t (&raw)[4],
                                          int64_t (&g)[4]) {
  if (M.raw_gates) {
    int32_t u[4];
    unit_q30(raw, kGateEps, u, sd);
#pragma unroll
    for (int c = 0; c < 4; c++) g[c] = u[c];
  } else {
    snap_rotation_to(M.icosian, make_int4(raw[0], raw[1], raw[2], raw[3]), 1ull << 31, g);
  }
}
__device__ __forceinline__ void gate_mul(const DevModel &M, const int64_t (&g)[4],
                                         const int64_t (&rhs)[4], int64_t (&out)[4]) {
  i128 prod[4];
  if (M.raw_gates) {
    const int32_t u[4] = {(int32_t)g[0], (int32_t)g[1], (int32_t)g[2], (int32_t)g[3]};
    hamilton32(u, rhs, prod);
#pragma unroll
    for (int c = 0; c < 4; c++) out[c] = shift_wide(prod[c], 14);
  } else {
    const Quat64 p = hamilton64_shift(g[0], g[1], g[2], g[3], rhs[0], rhs[1], rhs[2], rhs[3], 15);
#pragma unroll
    for (int c = 0; c < 4; c++) out[c] = p.v[c];
  }
}

// ---------------------------------------------------------------------------------------------
// The writer.

constexpr uint32_t kWindowChunk = 8; // window rows in flight per lane
constexpr uint32_t kPrologueLayers = 8;  // layers whose state words a lane loads all at once
constexpr int kScanUnroll = 4;       // row groups per pipeline stage

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// Copies n <= 64 words from global src to LDS dst (one per lane) without passing through
// registers (global_load_lds_dword); complete after wait_lds_dma().
__device__ __forceinline__ void lds_dma_words(const uint32_t *src, uint32_t *dst, uint32_t n,
                                              uint32_t lane) {
  if (lane < n) __builtin_amdgcn_global_load_lds((global_void *)(src + lane), (lds_void *)dst, 4, 0, 0);
}
// Copies n quads (16 bytes each, 16-byte aligned) from global src to LDS dst, lane i of the
// wavefront taking quad i < min(n, 64) (global_load_lds_dwordx4: each lane's 16 bytes land at
// dst + 16 i; dst uniform); complete after an s_waitcnt.
__device__ __forceinline__ void lds_dma_quads(const uint32_t *src, uint32_t *dst, uint32_t n,
                                              uint32_t lane) {
  if (lane < n) __builtin_amdgcn_global_load_lds((global_void *)(src + 4 * lane), (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void wait_lds_dma() {
  __builtin_amdgcn_s_waitcnt(0);
  wave_sync();
}

// A row of d channels is 4 (d / 32) pieces of 16 bytes (8 channels). The S lanes of a row
// group take pieces sub + S w (w < 4), so each of the four loads reads S consecutive pieces of
// every row (whole 128-byte spans for S = 8) rather than one piece of each 64-byte segment.
struct ScanGeom {
  uint32_t grp, sub;  // this lane's row within a round and its first piece
  uint32_t stride;    // row stride in table words (d)
  uint32_t last;      // the row's last piece
  uint32_t valid;     // bit w: piece sub + S w lies inside the row
  bool full;          // every lane's four pieces lie inside the row (d = 32 S)
};

// Loads the rows of U row groups starting at candidate k0 (ids from the LDS list, or base_id + k
// for the nearest head). Addresses are clamped into range so that every lane loads. Row offsets
// fit 24-bit products (vocab < 2^24, d <= 1024). T8: the int8 table's rows (8 bytes a piece,
// into .x and .y, widened by scan_rows).
template <int S, int U, bool Full, bool T8>
__device__ __forceinline__ void scan_load(const DevModel &M, const uint32_t *list, uint32_t fill,
                                          uint32_t k0, const ScanGeom &g, uint32_t base_id,
                                          uint4 (&r)[U][4], uint32_t (&t)[U]) {
  constexpr uint32_t rows = kWave / S;
#pragma unroll
  for (int u = 0; u < U; u++) {
    uint32_t k = k0 + u * rows + g.grp;
    k = k < fill ? k : fill - 1;
    t[u] = list ? list[k] : base_id + k;
    if (T8) {
      const uint2 *row = (const uint2 *)(M.table8 + __umul24(t[u], g.stride));
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t piece = g.sub + S * w;
        const uint2 b = row[Full || piece <= g.last ? piece : g.last];
        r[u][w].x = b.x;
        r[u][w].y = b.y;
      }
    } else {
      const uint4 *row = (const uint4 *)(M.table_b + __umul24(t[u], g.stride));
      if (Full) {
#pragma unroll
        for (int w = 0; w < 4; w++) r[u][w] = row[g.sub + S * w];
      } else {
#pragma unroll
        for (int w = 0; w < 4; w++) {
          const uint32_t piece = g.sub + S * w;
          r[u][w] = row[piece <= g.last ? piece : g.last];
        }
      }
    }
  }
}

// Four biased bytes (code + 128) of `x` as two words of 16-bit halves, each (code + 128) << 8:
// a byte permute places bytes 0, 1 (lo) and 2, 3 (hi) in the halves' high bytes (the query is
// scaled to match, scan_setup).
__device__ __forceinline__ void widen8(uint32_t x, uint32_t &lo, uint32_t &hi) {
  lo = __builtin_amdgcn_perm(0u, x, 0x010C000Cu);  // bytes 0, 1 as the high bytes of two u16
  hi = __builtin_amdgcn_perm(0u, x, 0x030C020Cu);  // bytes 2, 3
}

// One row piece's L1 against the query: eight 16-bit channels (i16 table), or T8 the piece's
// eight int8 codes (x, y) widened at the SAD, so that a stage in flight holds the raw bytes.
template <bool T8>
__device__ __forceinline__ uint32_t piece_sad(const uint4 &p, const uint32_t (&qpk)[16], int w,
                                              uint32_t acc) {
  if (T8) {
    uint32_t lo, hi;
    widen8(p.x, lo, hi);
    acc = sad2_u16(lo, qpk[4 * w + 0], acc);
    acc = sad2_u16(hi, qpk[4 * w + 1], acc);
    widen8(p.y, lo, hi);
    acc = sad2_u16(lo, qpk[4 * w + 2], acc);
    return sad2_u16(hi, qpk[4 * w + 3], acc);
  }
  acc = sad2_u16(p.x, qpk[4 * w + 0], acc);
  acc = sad2_u16(p.y, qpk[4 * w + 1], acc);
  acc = sad2_u16(p.z, qpk[4 * w + 2], acc);
  return sad2_u16(p.w, qpk[4 * w + 3], acc);
}

template <int S, int U, bool Full, bool T8>
__device__ __forceinline__ uint64_t scan_score(const uint32_t (&qpk)[16], uint32_t fill,
                                               uint32_t k0, const ScanGeom &g,
                                               const uint4 (&r)[U][4], const uint32_t (&t)[U],
                                               uint64_t best) {
  constexpr uint32_t rows = kWave / S;
  uint32_t acc[U];
  if (Full) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      acc[u] = 0;
#pragma unroll
      for (int w = 0; w < 4; w++) acc[u] = piece_sad<T8>(r[u][w], qpk, w, acc[u]);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) {
      acc[u] = 0;
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t a = piece_sad<T8>(r[u][w], qpk, w, 0u);
        acc[u] += (g.valid >> w) & 1 ? a : 0;  // a piece past the row's end adds nothing
      }
    }
  }
  group_sums<S, U>(acc);
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint64_t cand = ((uint64_t)acc[u] << 32) | t[u];
    const bool ok = k0 + u * rows + g.grp < fill;
    best = ok && cand < best ? cand : best;
  }
  return best;
}

// Lowest (L1, token) over `fill` >= 1 candidates, two stages in flight: the rows of the next U
// row groups load while the current ones are scored. Full: every piece of every lane lies
// inside the row (compiled apart, so that the common widths carry no clamps or masks). T8: an
// int8 table, whose rows load as bytes and widen in registers before the same scoring (kernels
// of their own, so that neither form carries the other's registers).
template <int S, bool Full, bool T8>
__device__ __forceinline__ uint64_t scan_rows(const DevModel &M, const uint32_t (&qpk)[16],
                                              const uint32_t *list, uint32_t fill,
                                              uint32_t base_id, const ScanGeom &g, uint64_t best) {
  constexpr int U = kScanUnroll;
  constexpr uint32_t chunk = (kWave / S) * U;
  uint4 ra[U][4], rb[U][4];
  uint32_t ta[U], tb[U];
  scan_load<S, U, Full, T8>(M, list, fill, 0, g, base_id, ra, ta);
  for (uint32_t k0 = 0; k0 < fill; k0 += 2 * chunk) {
    scan_load<S, U, Full, T8>(M, list, fill, k0 + chunk, g, base_id, rb, tb);
    best = scan_score<S, U, Full, T8>(qpk, fill, k0, g, ra, ta, best);
    scan_load<S, U, Full, T8>(M, list, fill, k0 + 2 * chunk, g, base_id, ra, ta);
    best = scan_score<S, U, Full, T8>(qpk, fill, k0 + chunk, g, rb, tb, best);
  }
  return best;
}

template <int S, bool T8>
__device__ __forceinline__ uint64_t scan_list(const DevModel &M, const uint32_t (&qpk)[16],
                                              const uint32_t *list, uint32_t fill,
                                              uint32_t base_id, const ScanGeom &g, uint64_t best) {
  return g.full ? scan_rows<S, true, T8>(M, qpk, list, fill, base_id, g, best)
                : scan_rows<S, false, T8>(M, qpk, list, fill, base_id, g, best);
}

// Drawers per lane held in registers by the writer (models of at most 64 kDrawerRegs drawers);
// up to 64 kScoreRegs drawers keep only their scores in registers; larger drawer counts score
// through LDS.
constexpr uint32_t kDrawerRegs = 4;
constexpr uint32_t kScoreRegs = 16;

// A lane's drawers c = lane + 64 i (i < kDrawerRegs): their two 8-value keys and CSR ranges.
struct DrawerRegs {
  int4 key[kDrawerRegs][2];
  uint32_t beg[kDrawerRegs], end[kDrawerRegs];
};

__device__ __forceinline__ bool drawers_in_regs(const DevModel &M) {
  return M.head != 1 && M.D <= kWave * kDrawerRegs;
}

__device__ __forceinline__ void load_drawers(const DevModel &M, uint32_t lane, DrawerRegs &dr) {
#pragma unroll
  for (uint32_t i = 0; i < kDrawerRegs; i++) {
    const uint32_t c = lane + kWave * i;
    if (c < M.D) {
      const int4 *key = (const int4 *)(M.keys + 16u * c);
      dr.key[i][0] = key[0];
      dr.key[i][1] = key[1];
      dr.beg[i] = M.offsets[c];
      dr.end[i] = M.offsets[c + 1];
    }
  }
}

// The scan geometry of this lane (S lanes per row, lane groups of S) and its four pieces of
// the query as biased pairs: qpk[4 w + j] = (q[c] + 2^15) | (q[c + 1] + 2^15) << 16 with
// c = 8 (sub + S w) + 2 j; T8: packed for the int8 table's widened rows instead.
template <int S, bool T8>
__device__ __forceinline__ void scan_setup(const DevModel &M, const int32_t *q, uint32_t lane,
                                           ScanGeom &g, uint32_t (&qpk)[16]) {
  const uint32_t d = M.d, pieces = d >> 3;  // S is the power of two >= d / 32
  g.grp = lane / S;
  g.stride = d;
  g.sub = lane % S;
  g.last = pieces - 1;
  g.full = uniform32(pieces == 4 * S);
  g.valid = 0;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const uint32_t piece = g.sub + S * w;
    const bool in = piece < pieces;
    g.valid |= (uint32_t)in << w;
    const uint32_t c = 8 * (in ? piece : 0);
    if (T8) {
      // Against (code + 128) << s: the query offset by 128 << s and clamped to the table's range
      // [0, 255 << s], which adds the same amount to every candidate's L1 on the channel (the
      // clamped-off distance), so the lowest (L1, token) is unchanged. Both sides are then
      // scaled by 2^(8 - s) (s <= 8), so a row's byte is the high byte of its u16 as loaded:
      // every candidate's L1 is multiplied by the same power of two, which keeps the order and
      // the ties, and stays below 2^26 for d <= 1024.
      const int32_t lo = -(128 << M.t8_shift), hi = 127 << M.t8_shift;
      const uint32_t up = 8 - M.t8_shift;
      auto b = [&](int32_t v) -> uint32_t {
        const int32_t x = v < lo ? lo : v > hi ? hi : v;
        return (uint32_t)(x - lo) << up;
      };
#pragma unroll
      for (int j = 0; j < 4; j++) qpk[4 * w + j] = b(q[c + 2 * j]) | (b(q[c + 2 * j + 1]) << 16);
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++)
        qpk[4 * w + j] = (uint32_t)(q[c + 2 * j] + 32768) | ((uint32_t)(q[c + 2 * j + 1] + 32768) << 16);
    }
  }
}

// The whole-table nearest head over tokens [lo, hi) (session.rs:4418-4445).
template <int S, bool T8>
__device__ __forceinline__ uint64_t scan_nearest(const DevModel &M, const uint32_t (&qpk)[16],
                                                 uint32_t lo, uint32_t hi, const ScanGeom &g,
                                                 uint64_t best) {
  for (uint32_t b = lo; b < hi; b += kListCap) {
    const uint32_t fill = hi - b < kListCap ? hi - b : kListCap;
    best = scan_list<S, T8>(M, qpk, nullptr, fill, b, g, best);
  }
  return best;
}

// Drawer selection of the keyed writer (session.rs:4069-4100): scores are the L1 of the query's
// first and last 8-blocks to each drawer's two keys, packed with the drawer index so that the
// minimum is the reference's first maximum; P rounds take the lowest. Writes the kept drawers in
// selection order to kept[]; lane p < P ends with kept drawer p's CSR range.
__device__ __forceinline__ void writer_select(const DevModel &M, const int32_t *q, uint32_t *dscore,
                                              uint32_t *kept, uint32_t lane, uint32_t &my_beg,
                                              uint32_t &my_end) {
  const uint32_t d = M.d;
  int32_t qa[8], qb[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    qa[i] = q[i];
    qb[i] = q[d - 8 + i];
  }
  my_beg = 0;
  my_end = 0;
  if (drawers_in_regs(M)) {
    // Scores and ranges in registers: each round takes the wave's minimum, its owner lane
    // retires it and hands over its range.
    DrawerRegs dr;
    load_drawers(M, lane, dr);
    uint32_t sc[kDrawerRegs];
#pragma unroll
    for (uint32_t i = 0; i < kDrawerRegs; i++) {
      // The keys' i16 values, two per word, low half first.
      const int32_t ka[4] = {dr.key[i][0].x, dr.key[i][0].y, dr.key[i][0].z, dr.key[i][0].w};
      const int32_t kb[4] = {dr.key[i][1].x, dr.key[i][1].y, dr.key[i][1].z, dr.key[i][1].w};
      uint32_t s = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int32_t a = (j & 1) ? ka[j >> 1] >> 16 : (int32_t)(int16_t)ka[j >> 1];
        const int32_t b = (j & 1) ? kb[j >> 1] >> 16 : (int32_t)(int16_t)kb[j >> 1];
        s += uabs32(qa[j] - a);
        s += uabs32(qb[j] - b);
      }
      const uint32_t c = lane + kWave * i;
      sc[i] = c < M.D ? (s << 12) | c : UINT32_MAX;
    }
    for (uint32_t p = 0; p < M.P; p++) {
      uint32_t local = sc[0];
#pragma unroll
      for (uint32_t i = 1; i < kDrawerRegs; i++) local = sc[i] < local ? sc[i] : local;
      const uint32_t pick = wave_reduce32(local, OpMin()) & 0xfffu;
      const uint32_t slot = pick / kWave;
      uint32_t b = dr.beg[0], e = dr.end[0];
#pragma unroll
      for (uint32_t i = 1; i < kDrawerRegs; i++)
        if (slot == i) {
          b = dr.beg[i];
          e = dr.end[i];
        }
      b = lane32(b, (int)(pick & (kWave - 1)));
      e = lane32(e, (int)(pick & (kWave - 1)));
#pragma unroll
      for (uint32_t i = 0; i < kDrawerRegs; i++) sc[i] = (sc[i] & 0xfffu) == pick ? UINT32_MAX : sc[i];
      if (lane == p) {
        my_beg = b;
        my_end = e;
      }
      if (lane == 0) kept[p] = pick;
    }
    wave_sync();
  } else if (M.head != 1 && M.D <= kWave * kScoreRegs) {
    // Scores in registers (drawer c = lane + 64 i), keys read once; each round takes the
    // wave's minimum and its owner lane retires it. Ranges load after the rounds.
    uint32_t sc[kScoreRegs];
#pragma unroll
    for (uint32_t i = 0; i < kScoreRegs; i++) {
      const uint32_t c = lane + kWave * i;
      uint32_t s = UINT32_MAX;
      if (c < M.D) {
        const int4 *key = (const int4 *)(M.keys + 16u * c);
        const int4 k4[2] = {key[0], key[1]};
        const int16_t *kk = (const int16_t *)k4;
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          v += uabs32(qa[j] - (int32_t)kk[j]);
          v += uabs32(qb[j] - (int32_t)kk[8 + j]);
        }
        s = (v << 12) | c;
      }
      sc[i] = s;
    }
    for (uint32_t p = 0; p < M.P; p++) {
      uint32_t local = sc[0];
#pragma unroll
      for (uint32_t i = 1; i < kScoreRegs; i++) local = sc[i] < local ? sc[i] : local;
      const uint32_t pick = wave_reduce32(local, OpMin()) & 0xfffu;
#pragma unroll
      for (uint32_t i = 0; i < kScoreRegs; i++) sc[i] = (sc[i] & 0xfffu) == pick ? UINT32_MAX : sc[i];
      if (lane == 0) kept[p] = pick;
    }
    wave_sync();
    if (lane < M.P) {
      const uint32_t c = kept[lane];
      my_beg = M.offsets[c];
      my_end = M.offsets[c + 1];
    }
  } else {
    for (uint32_t c = lane; c < M.D; c += kWave) {
      const int4 *key = (const int4 *)(M.keys + 16u * c);
      const int4 k4[2] = {key[0], key[1]};
      const int16_t *kk = (const int16_t *)k4;
      uint32_t sc = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        sc += uabs32(qa[i] - (int32_t)kk[i]);
        sc += uabs32(qb[i] - (int32_t)kk[8 + i]);
      }
      dscore[c] = (sc << 12) | c;
    }
    wave_sync();
    for (uint32_t p = 0; p < M.P; p++) {
      uint32_t local = UINT32_MAX;
      for (uint32_t c = lane; c < M.D; c += kWave) local = dscore[c] < local ? dscore[c] : local;
      const uint32_t pick = wave_reduce32(local, OpMin()) & 0xfffu;
      wave_sync();
      if ((pick & (kWave - 1)) == lane) dscore[pick] = UINT32_MAX;
      if (lane == 0) kept[p] = pick;
      wave_sync();
    }
    // Each drawer's CSR range, loaded by lane p for kept drawer p (all at once).
    if (lane < M.P) {
      const uint32_t c = kept[lane];
      my_beg = M.offsets[c];
      my_end = M.offsets[c + 1];
    }
  }
}

// The lowest (L1, token) over the members of the ranges lanes 0..P-1 hold (session.rs:4100-4121):
// member ids are staged in `list` (at most `cap` per segment) and scanned.
template <int S, bool T8>
__device__ __forceinline__ uint64_t scan_members(const DevModel &M, const uint32_t (&qpk)[16],
                                                 uint32_t *list, uint32_t cap, const ScanGeom &g,
                                                 uint32_t lane, uint32_t my_beg, uint32_t my_end,
                                                 uint64_t best) {
  uint32_t p = 0, done = 0;  // next drawer, members of it already staged
  while (p < M.P) {
    uint32_t fill = 0;
    while (p < M.P && fill < cap) {
      const uint32_t beg = lane32(my_beg, (int)p) + done, end = lane32(my_end, (int)p);
      const uint32_t take = end - beg < cap - fill ? end - beg : cap - fill;
      for (uint32_t o = 0; o < take; o += kWave)
        lds_dma_words(M.members + beg + o, list + fill + o, take - o, lane);
      fill += take;
      done += take;
      if (beg + take == end) {
        p++;
        done = 0;
      }
    }
    wait_lds_dma();
    if (fill) best = scan_list<S, T8>(M, qpk, list, fill, 0, g, best);
    wave_sync();
  }
  return best;
}

// The native vector writer (RS stack/session.rs:4069-4121, TW 580-623) over keyed drawers,
// or the whole-table nearest head (session.rs:4418-4445). `q` holds the query (d words) in
// LDS. Returns the token (UINT32_MAX when no row was scored); writes the kept drawers in
// selection order to kept[] and kept_out (nullable).
template <int S, bool T8>
__device__ __forceinline__ uint32_t writer(const DevModel &M, const int32_t *q, uint32_t *dscore,
                                           uint32_t *kept, uint32_t *list, uint32_t lane,
                                           uint32_t *kept_out) {
  ScanGeom g;
  uint32_t qpk[16];
  scan_setup<S, T8>(M, q, lane, g, qpk);
  uint64_t best = UINT64_MAX;
  if (M.head == 1) {
    best = scan_nearest<S, T8>(M, qpk, 0, M.vocab, g, best);
    if (kept_out && lane < M.P) kept_out[lane] = 0;
  } else {
    uint32_t my_beg, my_end;
    writer_select(M, q, dscore, kept, lane, my_beg, my_end);
    if (kept_out && lane < M.P) kept_out[lane] = kept[lane];
    best = scan_members<S, T8>(M, qpk, list, M.list_cap, g, lane, my_beg, my_end, best);
  }
  best = wave_reduce64(best, OpMin());
  return (uint32_t)best;
}

// ---------------------------------------------------------------------------------------------
// One step of the session (RS stack/session.rs:4129-4403, TW 635-675) at ring slot `base`.
// Returns 0 or the reference's status code; the chosen token goes to *chosen when the writer
// runs.

struct Lds {
  int32_t *xbar;     // gather crossbar, 2 max(d, m) words; also the query
  int64_t *mlp_out;  // m values
  uint32_t *dscore;  // D
  uint32_t *kept;    // kMaxProbes
  uint32_t *list;    // kListCap
  int64_t *st;       // L * d recurrence state
  int32_t *wq;       // d: the query of the writer's last run
  uint32_t *wmeta;   // 4: [0] that run's token, [1] nonzero once wq holds a query,
                     //    [2] paired blocks: the step reuses that run's result, [3] a serving
                     //    slot's state fingerprint as loaded
  Seeds seeds;       // the reciprocal and reciprocal square root seed tables
  // Paired blocks only (null otherwise):
  int64_t *wide;     // d: the window sums, wave 1 -> wave 0
  int64_t *gq;       // d: the output gates' quaternions, wave 1 -> wave 0
  uint32_t *rng;     // 2 kMaxProbes: the kept drawers' CSR ranges (begins, then ends)
  uint64_t *pair;    // 4: each wave's MLP maximum magnitude, then each wave's best candidate
  // Hamming models only (null otherwise):
  uint32_t *tok;     // context: the session's tokens x_0..x_t
  uint8_t *hdist;    // context: one head's distances at the row
  uint32_t *hpick;   // kMaxHamKept: one head's chosen positions
  uint32_t *hwgt;    // kMaxHamKept: their Q31 weights
  uint32_t *hhist;   // kHamBins: one head's distance histogram
  uint32_t *hwd;     // kHamBins: the Q31 weight of each distance under the head's margin
  uint32_t *hnib;    // d / 4: the sign nibbles of the row's point
  uint32_t *hreq;    // kHamReqWords: paired blocks, a read's request to wave 1 and its counts
  // A model with a place read only (null otherwise): its register (fbs_hamming.h).
  uint32_t *pst;     // kPlaceWords: the register's scalars
  uint16_t *uend;    // context: the end of the finished user turn holding the position, or 0
  uint16_t *farm;    // context: at a row whose token arms, the place its question found + 1
  // The part clocks' kernels only: [wave][kParts] cycle counters.
  uint64_t *clk;
};

// A traced position (the traced kernels, DT): its record and the forced replay's inputs.
struct DtCtx {
  uint8_t *rec;          // this position's record (decision_layout), or null
  uint32_t reads_at;     // the reads' part of the record
  uint32_t decisions;    // the record holds the rate buckets
  const uint8_t *fb;     // this position's forced buckets [L][d/4] (255: none), or null
  const uint64_t *codes; // the sequence's forced codes [len][reads][heads][2], or null
  const uint8_t *mask;   // [len][reads][heads]: bit 0 the query is forced, bit 1 the key
};

}  // namespace fbs

#include "fbs_hamming.h"

namespace fbs {

// HM: the model's Hamming reads run at their hooks (row t of the session, `pay` its payload
// caches). `trace` (nullable): the position's snap trace, per layer the transition's root per
// lane, the output gate's per lane, then the feed-forward gate's per MLP quaternion
// (fbs_core.h:488-501).
template <int Q, int SW, bool HM, bool T8, bool DT = false>
__device__ __forceinline__ int step(const DevModel &M, const Lds &S, int32_t *ring, uint32_t base, uint32_t lane,
                    const bool (&qv)[Q], const uint32_t (&qi)[Q], uint32_t tok, bool want_writer,
                    uint32_t *chosen, uint32_t *kept_out, int32_t *query_out, uint32_t t,
                    int64_t *pay, uint8_t *trace, const DtCtx *dc = nullptr) {
  if (tok >= M.vocab) return 1;
  const uint32_t d = M.d, W = M.W, nq = M.nq;
  if (HM) {  // the read at this row needs x_0..=x_t (session.rs:4149-4152)
    if (lane == 0) S.tok[t] = tok;
    wave_sync();
    // The place read's register moves on this token, before the row's readout (:4154-4162).
    if (M.ham.place) place_advance<Q>(M, S, t, lane, qv, qi);
  }
  int32_t x[Q][4];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    uint2 w = qv[k] ? *(const uint2 *)(M.table_b + (uint64_t)tok * d + 4 * qi[k])
                    : make_uint2(0x80008000u, 0x80008000u);
    const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int16_t v = (int16_t)(uint16_t)(((ww[c >> 1] >> (16 * (c & 1))) & 0xffffu) ^ 0x8000u);
      x[k][c] = (int32_t)v << 4;  // to_exp_i32(v, -12, -16)
    }
  }
  for (uint32_t l = 0; l < M.L; l++) {
    const DevLayer ly = M.layers[l];
    int32_t *ring_l = ring + (uint64_t)l * W * d;
    // The layer's loads first: gains, biases and the gather program.
    short4 g_rec[Q], g_mlp[Q], tap0[Q];
    ushort4 gd_rec[Q], gd_mlp[Q];
    uint2 td0[Q];
    int4 cbias[Q], rbias[Q];
    int32_t dbias[Q], doff[Q];
    uint32_t pw_drive[Q][4], pw_gate[Q][4], pw_rot[Q][4], pw_dec[Q], pw_out[Q][4], pw_down[Q][4];
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const uint32_t qq = qv[k] ? qi[k] : 0, ch = 4 * qq;
      g_rec[k] = *(const short4 *)(ly.rec_gain + ch);
      g_mlp[k] = *(const short4 *)(ly.mlp_gain + ch);
      tap0[k] = *(const short4 *)(ly.taps + ch);
      gd_rec[k] = *(const ushort4 *)(ly.rec_gain_desc + ch);
      gd_mlp[k] = *(const ushort4 *)(ly.mlp_gain_desc + ch);
      td0[k] = *(const uint2 *)(ly.taps_desc + ch);
      cbias[k] = *(const int4 *)(ly.conv_bias + ch);
      rbias[k] = *(const int4 *)(ly.gate_bias + nq + ch);
      dbias[k] = ly.gate_bias[qq];
      doff[k] = ly.decay_offset[qq];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        pw_drive[k][c] = prog_word(ly.prog, M.s_rec_in + 4 * k + c, lane);
        pw_gate[k][c] = prog_word(ly.prog, M.s_rec_in + 4 * Q + 4 * k + c, lane);
        pw_rot[k][c] = prog_word(ly.prog, M.s_rec_gate + Q + 4 * k + c, lane);
        pw_out[k][c] = prog_word(ly.prog, M.s_rec_out + 4 * k + c, lane);
        pw_down[k][c] = prog_word(ly.prog, M.s_mlp_down + 4 * k + c, lane);
      }
      pw_dec[k] = prog_word(ly.prog, M.s_rec_gate + k, lane);
    }
    // ---- recurrence block
    int64_t v[Q][4];
    norm_gain<Q>(M, S.seeds, x, qv, g_rec, gd_rec, v);
    publish64<Q>(S.xbar, v, qv, qi);
    wave_sync();
    int32_t drive[Q][4], gv[Q][4], rot[Q][4], dec[Q];
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const int32_t rb[4] = {rbias[k].x, rbias[k].y, rbias[k].z, rbias[k].w};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        drive[k][c] = S.xbar[pw_drive[k][c]];
        gv[k][c] = S.xbar[pw_gate[k][c]];
        rot[k][c] = sat_add32(S.xbar[pw_rot[k][c]], rb[c]);
      }
      dec[k] = sat_add32(S.xbar[pw_dec[k]], dbias[k]);
    }
    wave_sync();
    int64_t sc[Q][4];
    uint64_t mx = 0;
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) {
#pragma unroll
        for (int c = 0; c < 4; c++) sc[k][c] = 0;
        continue;
      }
      const uint32_t ch = 4 * qi[k];
      // Lane weights (session.rs:4989-5026): geometric decay and keep from the 16-step table.
      int32_t sq = sat_add32(dec[k], doff[k]);
      sq = sq < 0 ? 0 : sq > 65536 ? 65536 : sq;
      uint32_t idx = (uint32_t)sq >> 12;
      idx = idx > 15 ? 15 : idx;
      if (DT && dc->decisions) {
        // Q5's decision trace (BucketTrace::decide, session.rs:2192-2215): a forced entry
        // replaces the score's; the score and the entry used are recorded.
        const uint32_t at = l * nq + qi[k];
        if (dc->fb && dc->fb[at] != 255) idx = dc->fb[at];
        *(int32_t *)(dc->rec + 4u * at) = sq;
        dc->rec[4u * M.L * nq + at] = (uint8_t)idx;
      }
      const uint64_t lambda = 1ull << (30 - idx), keep = M.keep_q31[idx];
      // The causal window (session.rs:4842-4868): tap 0 on the drive, tap s on the drive s
      // positions back (ring slot base - s), then the drive enters slot base. Rows and taps
      // load kWindowChunk at a time; the first chunk is in flight during the rotation.
      int4 hb[kWindowChunk];
      uint2 tb[kWindowChunk];  // tap_desc pairs: channels 0, 1 in .x, 2, 3 in .y
      auto load_chunk = [&](uint32_t s0) {
#pragma unroll
        for (uint32_t i = 0; i < kWindowChunk; i++) {
          const uint32_t s = s0 + i;
          if (s <= W) {
            const uint32_t sl = base >= s ? base - s : base + W - s;
            hb[i] = *(const int4 *)(ring_l + (uint64_t)sl * d + ch);
            tb[i] = *(const uint2 *)(ly.taps_desc + (uint64_t)s * d + ch);
          }
        }
      };
      load_chunk(1);
      // The transition's rotation (session.rs:5097-5145).
      int32_t T[4];
      int64_t T64[4];
      uint32_t root = kTraceNone;
      if (M.raw_transition) {
        int32_t u[4];
        unit_q30(rot[k], kRotationEps, u, S.seeds);
#pragma unroll
        for (int c = 0; c < 4; c++) T[c] = u[c] >> idx;  // (lambda u) >> 30, lambda = 2^(30-idx)
      } else {
        root = trace_root(rot[k], snap_rotation_to(M.icosian, make_int4(rot[k][0], rot[k][1],
                                                                         rot[k][2], rot[k][3]),
                                                    lambda, T64));
      }
      uint8_t *lt = trace ? trace + (uint64_t)l * (2 * nq + M.nm) : nullptr;
      if (lt) lt[qi[k]] = (uint8_t)root;
      int64_t wide[4];
      if (M.taps_fast) {
        const uint2 t0 = td0[k];
        wide[0] = wadd64(cbias[k].x, tap_desc_apply(drive[k][0], t0.x, 0));
        wide[1] = wadd64(cbias[k].y, tap_desc_apply(drive[k][1], t0.x, 1));
        wide[2] = wadd64(cbias[k].z, tap_desc_apply(drive[k][2], t0.y, 0));
        wide[3] = wadd64(cbias[k].w, tap_desc_apply(drive[k][3], t0.y, 1));
        for (uint32_t s0 = 1; s0 <= W; s0 += kWindowChunk) {
          if (s0 > 1) load_chunk(s0);
#pragma unroll
          for (uint32_t i = 0; i < kWindowChunk; i++)
            if (s0 + i <= W) {
              wide[0] = wadd64(wide[0], tap_desc_apply(hb[i].x, tb[i].x, 0));
              wide[1] = wadd64(wide[1], tap_desc_apply(hb[i].y, tb[i].x, 1));
              wide[2] = wadd64(wide[2], tap_desc_apply(hb[i].z, tb[i].y, 0));
              wide[3] = wadd64(wide[3], tap_desc_apply(hb[i].w, tb[i].y, 1));
            }
        }
      } else {
        // A tap outside the descriptor form somewhere in the model: the reference routine.
        const short4 t0 = tap0[k];
        wide[0] = wadd64(cbias[k].x, grid_apply(drive[k][0], t0.x));
        wide[1] = wadd64(cbias[k].y, grid_apply(drive[k][1], t0.y));
        wide[2] = wadd64(cbias[k].z, grid_apply(drive[k][2], t0.z));
        wide[3] = wadd64(cbias[k].w, grid_apply(drive[k][3], t0.w));
        for (uint32_t s = 1; s <= W; s++) {
          const uint32_t sl = base >= s ? base - s : base + W - s;
          const int4 hh = *(const int4 *)(ring_l + (uint64_t)sl * d + ch);
          const short4 t = *(const short4 *)(ly.taps + (uint64_t)s * d + ch);
          wide[0] = wadd64(wide[0], grid_apply(hh.x, t.x));
          wide[1] = wadd64(wide[1], grid_apply(hh.y, t.y));
          wide[2] = wadd64(wide[2], grid_apply(hh.z, t.z));
          wide[3] = wadd64(wide[3], grid_apply(hh.w, t.w));
        }
      }
      *(int4 *)(ring_l + (uint64_t)base * d + ch) =
          make_int4(drive[k][0], drive[k][1], drive[k][2], drive[k][3]);
      // Transport: h <- shift_wide(T (x) h + (keep wide) << 16, 31).
      int64_t *hp = S.st + (uint64_t)l * d + ch;
      int64_t h[4] = {hp[0], hp[1], hp[2], hp[3]};
      i128 moved[4];
      if (M.raw_transition)
        hamilton32(T, h, moved);
      else
        hamilton64(T64, h, moved);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        u128 drive_term = (u128)((i128)keep * (i128)wide[c]) << 16;
        h[c] = shift_wide((i128)((u128)moved[c] + drive_term), 31);
        hp[c] = h[c];
      }
      // Output gate on the moved state (session.rs:4951-4968).
      int64_t rhs[4], o[4];
#pragma unroll
      for (int c = 0; c < 4; c++) rhs[c] = shift(h[c], kResidualExp - kStateExp);
      const uint32_t groot = gate_apply(M, S.seeds, gv[k], rhs, o);
      if (lt) lt[nq + qi[k]] = (uint8_t)groot;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        sc[k][c] = o[c];
        uint64_t a = uabs64(o[c]);
        mx = a > mx ? a : mx;
      }
    }
    // quantize16 over the d outputs (kernels.rs:545-553), then gather16 of rec_out.
    int32_t qs = wave_bitlen_max(mx) - 15;
    if (qs < 0) qs = 0;
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k]) {
        int32_t a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) a[c] = quantize_elem(sc[k][c], qs);
        publish16(S.xbar, 4 * qi[k], a, kProductExp + qs);
      }
    wave_sync();
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], S.xbar[pw_out[k][c]]);
    wave_sync();
    // ---- feed-forward block: the Hamilton gate of mlp_gate on mlp_up (session.rs:4005-4025).
    // The gather words of MLP quaternion group j load one group ahead (the first during the
    // norm), so that their latency hides behind the previous work.
    uint32_t pg[4], pu[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      pg[c] = prog_word(ly.prog, M.s_mlp_gate + c, lane);
      pu[c] = prog_word(ly.prog, M.s_mlp_up + c, lane);
    }
    norm_gain<Q>(M, S.seeds, x, qv, g_mlp, gd_mlp, v);
    publish64<Q>(S.xbar, v, qv, qi);
    wave_sync();
    uint64_t mmx = 0;
#pragma unroll 1
    for (uint32_t j = 0; j < M.mpl; j++) {
      const uint32_t mq = lane + kWave * j;
      int32_t gq[4], up[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        gq[c] = S.xbar[pg[c]];
        up[c] = S.xbar[pu[c]];
      }
      if (j + 1 < M.mpl) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
          pg[c] = prog_word(ly.prog, M.s_mlp_gate + 4 * (j + 1) + c, lane);
          pu[c] = prog_word(ly.prog, M.s_mlp_up + 4 * (j + 1) + c, lane);
        }
      }
      if (mq < M.nm) {
        int64_t mo[4];
        const uint32_t mroot = mlp_gate(M, S.seeds, gq, up, mo);
        if (trace) trace[(uint64_t)l * (2 * nq + M.nm) + 2 * nq + mq] = (uint8_t)mroot;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          S.mlp_out[4 * mq + c] = mo[c];
          uint64_t a = uabs64(mo[c]);
          mmx = a > mmx ? a : mmx;
        }
      }
    }
    qs = wave_bitlen_max(mmx) - 15;
    if (qs < 0) qs = 0;
    wave_sync();
#pragma unroll 1
    for (uint32_t j = 0; j < M.mpl; j++) {
      const uint32_t mq = lane + kWave * j;
      if (mq < M.nm) {
        int32_t a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) a[c] = quantize_elem(S.mlp_out[4 * mq + c], qs);
        publish16(S.xbar, 4 * mq, a, kProductExp + qs);
      }
    }
    wave_sync();
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], S.xbar[pw_down[k][c]]);
    wave_sync();
    if (HM) {  // the stream read after l + 1 layers (session.rs:4252-4276)
      const int32_t r = M.ham.at[l + 1];
      if (r >= 0 && l + 1 < M.L) ham_stream<Q, DT>(M, M.ham.reads[r], (uint32_t)r, S, t, pay, lane, qv, qi, x, dc);
    }
  }
  // Final norm, gain and the Q12 query (session.rs:4294-4295, 4364-4366).
  short4 g_fin[Q];
  ushort4 gd_fin[Q];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    g_fin[k] = *(const short4 *)(M.final_gain + 4 * (qv[k] ? qi[k] : 0));
    gd_fin[k] = *(const ushort4 *)(M.final_gain_desc + 4 * (qv[k] ? qi[k] : 0));
  }
  int64_t v[Q][4];
  norm_gain<Q>(M, S.seeds, x, qv, g_fin, gd_fin, v);
  if (HM) {  // the readout read on the final norm's output (session.rs:4296-4320)
    const int32_t r = M.ham.at[M.L];
    if (r >= 0) ham_readout<Q, DT>(M, M.ham.reads[r], (uint32_t)r, S, t, pay, lane, qv, qi, v, dc);
  }
  int4 qq[Q];
  bool same = true;  // this lane's channels equal the query of the writer's last run
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      int32_t qa[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int32_t y = to_exp_i32(v[k][c], kNormFineExp, kQ12Exp);
        qa[c] = y > 32767 ? 32767 : y < -32768 ? -32768 : y;
      }
      qq[k] = make_int4(qa[0], qa[1], qa[2], qa[3]);
      *(int4 *)(S.xbar + 4 * qi[k]) = qq[k];
      if (query_out) *(int4 *)(query_out + 4 * qi[k]) = qq[k];
      const int4 old = *(const int4 *)(S.wq + 4 * qi[k]);
      same = same && old.x == qa[0] && old.y == qa[1] && old.z == qa[2] && old.w == qa[3];
    }
  wave_sync();
  if (want_writer) {
    // The writer's token and kept drawers are a function of the query alone: a query equal to
    // the last one the writer ran on (a sequence settled on a fixed point) takes its result.
    if (S.wmeta[1] != 0 && __all(same)) {
      *chosen = S.wmeta[0];
      if (kept_out && lane < M.P) kept_out[lane] = M.head == 1 ? 0u : S.kept[lane];
    } else {
      *chosen = writer<SW, T8>(M, S.xbar, S.dscore, S.kept, S.list, lane, kept_out);
#pragma unroll
      for (int k = 0; k < Q; k++)
        if (qv[k]) *(int4 *)(S.wq + 4 * qi[k]) = qq[k];
      if (lane == 0) {
        S.wmeta[0] = *chosen;
        S.wmeta[1] = M.writer_memory;
      }
    }
  }
  wave_sync();
  return 0;
}

// ---------------------------------------------------------------------------------------------
// Paired blocks: one sequence on the two wavefronts of a 128-lane block, for batches that would
// leave SIMDs without a second wave. Wave 0 holds the residual stream and the recurrence state:
// the norms, the transition and transport, the output gate's product and its requantize, the
// final query and the writer's drawer selection. Wave 1 owns the window ring: it adds tap 0 to
// the window sums it formed during the previous step, writes the drive into the ring and forms
// the output gate's quaternion while wave 0 forms the transition, then sums the next step's
// window while wave 0 runs the transport. The MLP's quaternion groups (and their requantize)
// alternate between the waves, and each wave scans half of the writer's candidates. The two
// waves meet at block barriers, numbered alike in step_main and step_window: every path through
// a step reaches the same barriers in the same order on both waves (the branches between them
// depend only on values both waves hold: the model, the step's token and want_writer, and the
// reuse flag read after barrier 6).

// Both waves of the block meet; LDS writes before it are visible to the other wave after it.
// Global loads in flight stay in flight (LDS-only fences).
__device__ __forceinline__ void pair_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The part clocks (Part): with ON, lap(p) adds the shader-clock cycles since the last lap to the
// wave's counter p in LDS (lane 0 writes it); without, every call compiles to nothing, so the
// served kernels carry no clock code. The clock read waits for the wave's LDS operations, not for
// its global loads.
template <bool ON>
struct PartClock {
  uint64_t t = 0;
  uint64_t *acc = nullptr;  // LDS: this wave's kParts counters
  __device__ __forceinline__ void start() {
    if constexpr (ON) t = __builtin_amdgcn_s_memtime();
  }
  __device__ __forceinline__ void lap(uint32_t part) {
    if constexpr (ON) {
      const uint64_t now = __builtin_amdgcn_s_memtime();
      if (threadIdx.x % kWave == 0) acc[part] += now - t;
      t = now;
    }
  }
  // A barrier timed as its own part (the wait), the work before it as `before`.
  __device__ __forceinline__ void sync(uint32_t before, uint32_t barrier) {
    lap(before);
    pair_sync();
    lap(barrier);
  }
};

// Clips the ranges that lanes 0..P-1 hold to the positions [lo, hi) of their concatenation.
__device__ __forceinline__ void clip_ranges(uint32_t P, uint32_t lane, uint32_t lo, uint32_t hi,
                                            uint32_t &my_beg, uint32_t &my_end) {
  uint32_t nb = my_beg, ne = my_end, cum = 0;
  for (uint32_t p = 0; p < P; p++) {
    const uint32_t b = lane32(my_beg, (int)p), len = lane32(my_end, (int)p) - b;
    const uint32_t from = lo > cum ? (lo - cum < len ? lo - cum : len) : 0;
    const uint32_t to = hi > cum ? (hi - cum < len ? hi - cum : len) : 0;
    if (lane == p) {
      nb = b + from;
      ne = b + (to > from ? to : from);
    }
    cum += len;
  }
  my_beg = nb;
  my_end = ne;
}

// The MLP's requantize (quantize16, kernels.rs:545-553) for groups j0, j0 + 2, ...: S.mlp_out
// at the shared shift of both waves' maxima, published for the mlp_down gathers.
__device__ __forceinline__ void pair_requant(const DevModel &M, const Lds &S, uint32_t lane,
                                             uint32_t j0) {
  const uint64_t bl = S.pair[0] > S.pair[1] ? S.pair[0] : S.pair[1];  // bit lengths
  int32_t qs = (int32_t)bl - 15;
  if (qs < 0) qs = 0;
#pragma unroll 1
  for (uint32_t j = j0; j < M.mpl; j += 2) {
    const uint32_t mq = lane + kWave * j;
    if (mq < M.nm) {
      int32_t a[4];
#pragma unroll
      for (int c = 0; c < 4; c++) a[c] = quantize_elem(S.mlp_out[4 * mq + c], qs);
      publish16(S.xbar, 4 * mq, a, kProductExp + qs);
    }
  }
}

// MLP group j's gather words (gate and up) for this lane, nothing past the last group; read by
// global loads, which the LDS waits before their use do not wait for (a flat load's would).
__device__ __forceinline__ void pair_mlp_words(const DevModel &M, const DevLayer &ly, uint32_t lane,
                                               uint32_t j, uint32_t (&pg)[4], uint32_t (&pu)[4]) {
  if (j < M.mpl) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      pg[c] = gload(ly.prog + (M.s_mlp_gate + 4 * j + c) * kWave + lane);
      pu[c] = gload(ly.prog + (M.s_mlp_up + 4 * j + c) * kWave + lane);
    }
  }
}

// MLP quaternion groups j0, j0 + 2, ... of the feed-forward gate (session.rs:4005-4025) into
// S.mlp_out; pg/pu hold group j0's gather words. Returns the bit length of the groups' largest
// magnitude.
__device__ __forceinline__ uint64_t pair_mlp(const DevModel &M, const Lds &S, const DevLayer &ly,
                                             uint32_t lane, uint32_t j0, uint32_t (&pg)[4],
                                             uint32_t (&pu)[4]) {
  uint64_t mmx = 0;
#pragma unroll 1
  for (uint32_t j = j0; j < M.mpl; j += 2) {
    const uint32_t mq = lane + kWave * j;
    int32_t gq[4], up[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      gq[c] = S.xbar[pg[c]];
      up[c] = S.xbar[pu[c]];
    }
    pair_mlp_words(M, ly, lane, j + 2, pg, pu);  // the next group's (none past the last)
    if (mq < M.nm) {
      int64_t mo[4];
      mlp_gate(M, S.seeds, gq, up, mo);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        S.mlp_out[4 * mq + c] = mo[c];
        uint64_t a = uabs64(mo[c]);
        mmx = a > mmx ? a : mmx;
      }
    }
  }
  return (uint64_t)wave_bitlen_max(mmx);
}


// The writer on both waves, after barrier 6 (the query is in the crossbar, wmeta[2] says whether
// the step reuses the last result): wave 0 selects the drawers, each wave scans half of the
// candidates (by position in the kept drawers' concatenated members, or half of the table for
// the nearest head), and both return the lower (L1, token).
template <int SW, bool T8, bool CLK>
__device__ __forceinline__ uint32_t pair_writer(const DevModel &M, const Lds &S, uint32_t wave,
                                                uint32_t lane, uint32_t *kept_out,
                                                PartClock<CLK> &clk) {
  if (S.wmeta[2]) {
    if (wave == 0 && kept_out && lane < M.P) kept_out[lane] = M.head == 1 ? 0u : S.kept[lane];
    clk.lap(kPartSelect);
    return S.wmeta[0];
  }
  if (wave == 0 && M.head != 1) {
    uint32_t b, e;
    writer_select(M, S.xbar, S.dscore, S.kept, lane, b, e);
    if (lane < M.P) {
      S.rng[lane] = b;
      S.rng[kMaxProbes + lane] = e;
    }
  }
  clk.sync(kPartSelect, kPartSync7);  // 7: the kept drawers and their ranges
  ScanGeom g;
  uint32_t qpk[16];
  scan_setup<SW, T8>(M, S.xbar, lane, g, qpk);
  uint64_t best = UINT64_MAX;
  if (M.head == 1) {
    const uint32_t half = M.vocab / 2;
    best = scan_nearest<SW, T8>(M, qpk, wave ? half : 0, wave ? M.vocab : half, g, best);
    if (wave == 0 && kept_out && lane < M.P) kept_out[lane] = 0;
  } else {
    if (wave == 0 && kept_out && lane < M.P) kept_out[lane] = S.kept[lane];
    uint32_t my_beg = lane < M.P ? S.rng[lane] : 0, my_end = lane < M.P ? S.rng[kMaxProbes + lane] : 0;
    // Wave 0 takes 17/32 of a scan of 1,024 candidates or more (the ring wave, at normal
    // priority, scans more slowly: 43.7 K against 38.2 K cycles a token for equal halves at C3),
    // and half of a shorter one.
    const uint32_t total = wave_reduce32(my_end - my_beg, OpAdd());
    const uint32_t half = total >= 1024 ? (uint32_t)(((uint64_t)total * 17 + 31) / 32) : (total + 1) / 2;
    clip_ranges(M.P, lane, wave ? half : 0, wave ? total : half, my_beg, my_end);
    const uint32_t cap = M.list_cap / 2;  // each wave its half of the staging list
    best = scan_members<SW, T8>(M, qpk, S.list + wave * cap, cap, g, lane, my_beg, my_end, best);
  }
  best = wave_reduce64(best, OpMin());
  if (lane == 0) S.pair[2 + wave] = best;
  clk.sync(kPartScan, kPartSync8);  // 8: both waves' best candidates
  const uint64_t b0 = S.pair[2], b1 = S.pair[3];
  return (uint32_t)(b0 < b1 ? b0 : b1);
}

// Wave 0 of a paired block: the step (RS stack/session.rs:4129-4403) but the window and its
// ring, the output gates' quaternions and the odd MLP groups.
template <int Q, int SW, bool T8, bool CLK, bool HM = false>
__device__ __forceinline__ int step_main(const DevModel &M, const Lds &S, uint32_t lane,
                                         const bool (&qv)[Q], const uint32_t (&qi)[Q], uint32_t tok,
                                         bool want_writer, uint32_t *chosen, uint32_t *kept_out,
                                         int32_t *query_out, PartClock<CLK> &clk,
                                         int64_t *gst, uint32_t t = 0, int64_t *pay = nullptr,
                                         bool defer = false) {
  if (tok >= M.vocab) return 1;
  if constexpr (HM) {  // the read at this row needs x_0..=x_t (session.rs:4149-4152)
    if (lane == 0) S.tok[t] = tok;
    wave_sync();
    // The place read's register moves on this token, before the row's readout (:4154-4162).
    if (M.ham.place) place_advance<Q>(M, S, t, lane, qv, qi);
  }
  const uint32_t d = M.d, nq = M.nq;
  int32_t x[Q][4];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    uint2 w = qv[k] ? *(const uint2 *)(M.table_b + (uint64_t)tok * d + 4 * qi[k])
                    : make_uint2(0x80008000u, 0x80008000u);
    const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int16_t v = (int16_t)(uint16_t)(((ww[c >> 1] >> (16 * (c & 1))) & 0xffffu) ^ 0x8000u);
      x[k][c] = (int32_t)v << 4;  // to_exp_i32(v, -12, -16)
    }
  }
  clk.lap(kPartEmbed);
  for (uint32_t l = 0; l < M.L; l++) {
    const DevLayer ly = M.layers[l];
    short4 g_rec[Q], g_mlp[Q];
    ushort4 gd_rec[Q], gd_mlp[Q];
    int4 rbias[Q];
    int32_t dbias[Q], doff[Q];
    uint32_t pw_rot[Q][4], pw_dec[Q], pw_out[Q][4], pw_down[Q][4];
    // The feed-forward block's gains and gather words: loaded here for one quaternion a lane,
    // where registers allow their latency to hide behind the recurrence block, and at the
    // feed-forward block for more (their registers would spill to scratch across the block).
    auto load_ffn = [&]() {
#pragma unroll
      for (int k = 0; k < Q; k++) {
        const uint32_t ch = 4 * (qv[k] ? qi[k] : 0);
        g_mlp[k] = *(const short4 *)(ly.mlp_gain + ch);
        gd_mlp[k] = *(const ushort4 *)(ly.mlp_gain_desc + ch);
#pragma unroll
        for (int c = 0; c < 4; c++) pw_down[k][c] = prog_word(ly.prog, M.s_mlp_down + 4 * k + c, lane);
      }
    };
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const uint32_t qq = qv[k] ? qi[k] : 0, ch = 4 * qq;
      g_rec[k] = *(const short4 *)(ly.rec_gain + ch);
      gd_rec[k] = *(const ushort4 *)(ly.rec_gain_desc + ch);
      rbias[k] = *(const int4 *)(ly.gate_bias + nq + ch);
      dbias[k] = ly.gate_bias[qq];
      doff[k] = ly.decay_offset[qq];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        pw_rot[k][c] = prog_word(ly.prog, M.s_rec_gate + Q + 4 * k + c, lane);
        pw_out[k][c] = prog_word(ly.prog, M.s_rec_out + 4 * k + c, lane);
      }
      pw_dec[k] = prog_word(ly.prog, M.s_rec_gate + k, lane);
    }
    if constexpr (Q == 1) load_ffn();
    clk.lap(kPartLoads);
    int64_t v[Q][4];
    norm_gain<Q>(M, S.seeds, x, qv, g_rec, gd_rec, v);
    publish64<Q>(S.xbar, v, qv, qi);
    // Two or more quaternions a lane keep the state in the block's global buffer (each lane its
    // own channels): its loads are issued here, to land during the barrier's wait.
    int64_t hg[Q][4];
    if constexpr (kPairStateGlobal<Q, HM>) {
#pragma unroll
      for (int k = 0; k < Q; k++) {
        const longlong2 *src = (const longlong2 *)(gst + (uint64_t)l * d + 4 * (qv[k] ? qi[k] : 0));
        const longlong2 a = src[0], b = src[1];
        hg[k][0] = a.x;
        hg[k][1] = a.y;
        hg[k][2] = b.x;
        hg[k][3] = b.y;
      }
    }
    clk.sync(kPartNormRec, kPartSync1);  // 1: the normed activations
    int32_t rot[Q][4], dec[Q];
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const int32_t rb[4] = {rbias[k].x, rbias[k].y, rbias[k].z, rbias[k].w};
#pragma unroll
      for (int c = 0; c < 4; c++) rot[k][c] = sat_add32(S.xbar[pw_rot[k][c]], rb[c]);
      dec[k] = sat_add32(S.xbar[pw_dec[k]], dbias[k]);
    }
    // Lane weights (session.rs:4989-5026), the transition's rotation (session.rs:5097-5145)
    // and its product with the state, which do not wait for the window.
    // T (x) h: a raw transition's as mh 2^32 + ml (hamilton32_hl), a snapped one's i128 as its
    // high and low 64 bits.
    uint64_t keep[Q];
    int64_t mh[Q][4], ml[Q][4];
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) {
        keep[k] = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) mh[k][c] = ml[k][c] = 0;
        continue;
      }
      int32_t sq = sat_add32(dec[k], doff[k]);
      sq = sq < 0 ? 0 : sq > 65536 ? 65536 : sq;
      uint32_t idx = (uint32_t)sq >> 12;
      idx = idx > 15 ? 15 : idx;
      keep[k] = M.keep_q31[idx];
      int64_t h[4];
      if constexpr (kPairStateGlobal<Q, HM>) {
#pragma unroll
        for (int c = 0; c < 4; c++) h[c] = hg[k][c];
      } else {
        const int64_t *hp = S.st + (uint64_t)l * d + 4 * qi[k];
#pragma unroll
        for (int c = 0; c < 4; c++) h[c] = hp[c];
      }
      if (M.raw_transition) {
        int32_t u[4], T[4];
        unit_q30(rot[k], kRotationEps, u, S.seeds);
#pragma unroll
        for (int c = 0; c < 4; c++) T[c] = u[c] >> idx;  // (lambda u) >> 30, lambda = 2^(30-idx)
        hamilton32_hl(T, h, mh[k], ml[k]);
      } else {
        int64_t T64[4];
        snap_rotation_to(M.icosian, make_int4(rot[k][0], rot[k][1], rot[k][2], rot[k][3]),
                          1ull << (30 - idx), T64);
        const Wide4 mv = hamilton64_wide(T64[0], T64[1], T64[2], T64[3], h[0], h[1], h[2], h[3]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          mh[k][c] = mv.hi[c];
          ml[k][c] = mv.lo[c];
        }
      }
    }
    clk.sync(kPartTransition, kPartSync2);  // 2: the window sums and the output gates' quaternions
    // Transport: h <- shift_wide(T (x) h + (keep wide) << 16, 31). A raw transition whose sums
    // lie in transport_fast's ranges on every lane takes its 64-bit form (one uniform branch).
    int64_t h[Q][4];
    {
      bool fast = M.raw_transition != 0;
      int64_t wide[Q][4];
#pragma unroll
      for (int k = 0; k < Q; k++) {
        const uint32_t ch = 4 * (qv[k] ? qi[k] : 0);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          wide[k][c] = S.wide[ch + c];
          fast = fast && (!qv[k] || transport_fast_ok(mh[k][c], wide[k][c], keep[k]));
        }
      }
      if (__all(fast)) {
#pragma unroll
        for (int k = 0; k < Q; k++)
#pragma unroll
          for (int c = 0; c < 4; c++) h[k][c] = transport_fast(mh[k][c], ml[k][c], keep[k], wide[k][c]);
      } else {
#pragma unroll
        for (int k = 0; k < Q; k++)
#pragma unroll
          for (int c = 0; c < 4; c++)
            h[k][c] = transport_wide(mh[k][c], ml[k][c], keep[k], wide[k][c], M.raw_transition);
      }
    }
    // Output gate on the moved state (session.rs:4951-4968): a raw gate's product in its 64-bit
    // form where every lane's sums allow it (gate_shift14_fast).
    int64_t sc[Q][4];
    uint64_t mx = 0;
    {
      int64_t gh[Q][4], gl[Q][4];
      bool fast = M.raw_gates != 0;
#pragma unroll
      for (int k = 0; k < Q; k++) {
        const uint32_t ch = 4 * (qv[k] ? qi[k] : 0);
        if (qv[k]) {
          if constexpr (kPairStateGlobal<Q, HM>) {
            longlong2 *dst = (longlong2 *)(gst + (uint64_t)l * d + ch);
            dst[0] = make_longlong2(h[k][0], h[k][1]);
            dst[1] = make_longlong2(h[k][2], h[k][3]);
          } else {
            int64_t *hp = S.st + (uint64_t)l * d + ch;
#pragma unroll
            for (int c = 0; c < 4; c++) hp[c] = h[k][c];
          }
        }
        int64_t rhs[4];
#pragma unroll
        for (int c = 0; c < 4; c++) rhs[c] = shift(h[k][c], kResidualExp - kStateExp);
        if (M.raw_gates) {
          const int32_t u[4] = {(int32_t)S.gq[ch], (int32_t)S.gq[ch + 1], (int32_t)S.gq[ch + 2],
                                (int32_t)S.gq[ch + 3]};
          hamilton32_hl(u, rhs, gh[k], gl[k]);
#pragma unroll
          for (int c = 0; c < 4; c++) fast = fast && (!qv[k] || gate_fast_ok(gh[k][c]));
        } else {
          const int64_t g[4] = {S.gq[ch], S.gq[ch + 1], S.gq[ch + 2], S.gq[ch + 3]};
          gate_mul(M, g, rhs, sc[k]);
        }
      }
      if (M.raw_gates) {
        if (__all(fast)) {
#pragma unroll
          for (int k = 0; k < Q; k++)
#pragma unroll
            for (int c = 0; c < 4; c++) sc[k][c] = gate_shift14_fast(gh[k][c], gl[k][c]);
        } else {
#pragma unroll
          for (int k = 0; k < Q; k++)
#pragma unroll
            for (int c = 0; c < 4; c++) sc[k][c] = gate_wide14(gh[k][c], gl[k][c]);
        }
      }
#pragma unroll
      for (int k = 0; k < Q; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
          if (!qv[k]) sc[k][c] = 0;
          const uint64_t a = uabs64(sc[k][c]);
          mx = a > mx ? a : mx;
        }
    }
    clk.lap(kPartTransport);
    // The feed-forward block's gather words, loaded a phase ahead: the norm's factor is a call,
    // whose entry waits for every load in flight, so loads issued just before it are waited for
    // whole (global loads, so that the LDS waits in between do not wait for them).
    uint32_t pg[4], pu[4];
    pair_mlp_words(M, ly, lane, 0, pg, pu);
    // quantize16 over the d outputs (kernels.rs:545-553), then gather16 of rec_out.
    int32_t qs = wave_bitlen_max(mx) - 15;
    if (qs < 0) qs = 0;
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k]) {
        int32_t a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) a[c] = quantize_elem(sc[k][c], qs);
        publish16(S.xbar, 4 * qi[k], a, kProductExp + qs);
      }
    wave_sync();
    clk.lap(kPartRequantRec);
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], S.xbar[pw_out[k][c]]);
    wave_sync();
    clk.lap(kPartResidualRec);
    // ---- feed-forward block: wave 0 takes the even quaternion groups.
    if constexpr (Q != 1) load_ffn();
    norm_gain<Q>(M, S.seeds, x, qv, g_mlp, gd_mlp, v);
    publish64<Q>(S.xbar, v, qv, qi);
    clk.sync(kPartNormMlp, kPartSync3);  // 3: the normed activations
    const uint64_t mbl = pair_mlp(M, S, ly, lane, 0, pg, pu);
    if (lane == 0) S.pair[0] = mbl;
    clk.sync(kPartMlp, kPartSync4);  // 4: both waves' MLP outputs and maxima
    pair_requant(M, S, lane, 0);
    clk.sync(kPartRequantMlp, kPartSync5);  // 5: the requantized MLP outputs
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], S.xbar[pw_down[k][c]]);
    wave_sync();
    clk.lap(kPartResidualMlp);
    if constexpr (HM) {  // the stream read after l + 1 layers (session.rs:4252-4276)
      const int32_t r = M.ham.at[l + 1];
      if (r >= 0 && l + 1 < M.L)
        ham_stream<Q, false, true>(M, M.ham.reads[r], (uint32_t)r, S, t, pay, lane, qv, qi, x);
    }
  }
  // A model with a readout read runs it at every row: a typed one keeps the row's payload.
  const bool readout = HM && M.ham.at[M.L] >= 0;
  if (!want_writer && !readout) return 0;
  // Final norm, gain and the Q12 query (session.rs:4294-4295, 4364-4366).
  short4 g_fin[Q];
  ushort4 gd_fin[Q];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    g_fin[k] = *(const short4 *)(M.final_gain + 4 * (qv[k] ? qi[k] : 0));
    gd_fin[k] = *(const ushort4 *)(M.final_gain_desc + 4 * (qv[k] ? qi[k] : 0));
  }
  int64_t v[Q][4];
  norm_gain<Q>(M, S.seeds, x, qv, g_fin, gd_fin, v);
  if constexpr (HM) {  // the readout read on the final norm's output (session.rs:4296-4320)
    if (readout) {
      const uint32_t r = (uint32_t)M.ham.at[M.L];
      ham_readout<Q, false, true>(M, M.ham.reads[r], r, S, t, pay, lane, qv, qi, v);
    }
    if (!want_writer) return 0;
  }
  int4 qq[Q];
  bool same = true;  // this lane's channels equal the query of the writer's last run
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      int32_t qa[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int32_t y = to_exp_i32(v[k][c], kNormFineExp, kQ12Exp);
        qa[c] = y > 32767 ? 32767 : y < -32768 ? -32768 : y;
      }
      qq[k] = make_int4(qa[0], qa[1], qa[2], qa[3]);
      *(int4 *)(S.xbar + 4 * qi[k]) = qq[k];
      if (query_out) *(int4 *)(query_out + 4 * qi[k]) = qq[k];
      const int4 old = *(const int4 *)(S.wq + 4 * qi[k]);
      same = same && old.x == qa[0] && old.y == qa[1] && old.z == qa[2] && old.w == qa[3];
    }
  // The writer's token and kept drawers are a function of the query alone: a query equal to
  // the last one the writer ran on (a sequence settled on a fixed point) takes its result.
  const bool reuse = S.wmeta[1] != 0 && __all(same);
  if (lane == 0) S.wmeta[2] = reuse;
  if (defer) {
    // The deferred writer: the remembered result, or the drawer selection alone (wmeta[2] = 2:
    // a job for the drawer-major scan, whose token the memory takes once it is known).
    if (reuse) {
      if (kept_out && lane < M.P) kept_out[lane] = S.kept[lane];
      *chosen = S.wmeta[0];
      return 0;
    }
    wave_sync();
    uint32_t b, e;
    writer_select(M, S.xbar, S.dscore, S.kept, lane, b, e);
    if (kept_out && lane < M.P) kept_out[lane] = S.kept[lane];
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k]) *(int4 *)(S.wq + 4 * qi[k]) = qq[k];
    if (lane == 0) {
      S.wmeta[1] = 0;
      S.wmeta[2] = 2;
    }
    *chosen = UINT32_MAX;
    return 0;
  }
  clk.sync(kPartFinal, kPartSync6);  // 6: the query and the reuse flag
  *chosen = pair_writer<SW, T8, CLK>(M, S, 0, lane, kept_out, clk);
  if (!reuse) {
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k]) *(int4 *)(S.wq + 4 * qi[k]) = qq[k];
    if (lane == 0) {
      S.wmeta[0] = *chosen;
      S.wmeta[1] = M.writer_memory;
    }
  }
  return 0;
}

// Tap k on the lane's four channels of x: tap_desc words (fast taps) or grid codes.
__device__ __forceinline__ void tap4(const DevModel &M, const DevLayer &ly, uint32_t k, uint32_t ch,
                                     const int4 &x, int64_t (&acc)[4]) {
  if (M.taps_fast) {
    const uint2 t = *(const uint2 *)(ly.taps_desc + (uint64_t)k * M.d + ch);
    acc[0] = wadd64(acc[0], tap_desc_apply(x.x, t.x, 0));
    acc[1] = wadd64(acc[1], tap_desc_apply(x.y, t.x, 1));
    acc[2] = wadd64(acc[2], tap_desc_apply(x.z, t.y, 0));
    acc[3] = wadd64(acc[3], tap_desc_apply(x.w, t.y, 1));
  } else {
    const short4 t = *(const short4 *)(ly.taps + (uint64_t)k * M.d + ch);
    acc[0] = wadd64(acc[0], grid_apply(x.x, t.x));
    acc[1] = wadd64(acc[1], grid_apply(x.y, t.y));
    acc[2] = wadd64(acc[2], grid_apply(x.z, t.z));
    acc[3] = wadd64(acc[3], grid_apply(x.w, t.w));
  }
}

// The window over earlier positions for a step whose ring slot is `base`: tap s on the drive
// s positions back (ring slot base - s), for s = s1..W, added to acc (session.rs:4842-4868;
// wrapping sums, so the order of the terms does not matter). Rows and taps load kWindowChunk at
// a time.
__device__ __forceinline__ void window_sum(const DevModel &M, const DevLayer &ly,
                                           const int32_t *ring_l, uint32_t base, uint32_t s1,
                                           uint32_t ch, int64_t (&acc)[4], uint32_t s2 = 0) {
  const uint32_t d = M.d, W = s2 ? s2 : M.W;  // taps s1..W (the last tap s2 when given)
  if (M.taps_fast) {
    for (uint32_t s0 = s1; s0 <= W; s0 += kWindowChunk) {
      int4 hb[kWindowChunk];
      uint2 tb[kWindowChunk];  // tap_desc pairs: channels 0, 1 in .x, 2, 3 in .y
#pragma unroll
      for (uint32_t i = 0; i < kWindowChunk; i++) {
        const uint32_t s = s0 + i;
        if (s <= W) {
          const uint32_t sl = base >= s ? base - s : base + M.W - s;
          hb[i] = *(const int4 *)(ring_l + (uint64_t)sl * d + ch);
          tb[i] = *(const uint2 *)(ly.taps_desc + (uint64_t)s * d + ch);
        }
      }
#pragma unroll
      for (uint32_t i = 0; i < kWindowChunk; i++)
        if (s0 + i <= W) {
          acc[0] = wadd64(acc[0], tap_desc_apply(hb[i].x, tb[i].x, 0));
          acc[1] = wadd64(acc[1], tap_desc_apply(hb[i].y, tb[i].x, 1));
          acc[2] = wadd64(acc[2], tap_desc_apply(hb[i].z, tb[i].y, 0));
          acc[3] = wadd64(acc[3], tap_desc_apply(hb[i].w, tb[i].y, 1));
        }
    }
  } else {
    // A tap outside the descriptor form somewhere in the model: the reference routine.
    for (uint32_t s = s1; s <= W; s++) {
      const uint32_t sl = base >= s ? base - s : base + M.W - s;
      tap4(M, ly, s, ch, *(const int4 *)(ring_l + (uint64_t)sl * d + ch), acc);
    }
  }
}

// Wave 1 of a paired block: the causal window (session.rs:4842-4868) read from and written to
// the sequence's ring, the output gates' quaternions, the odd MLP groups and half of the writer.
// The window's terms over earlier positions (taps 1..W) do not depend on the step's input, so
// wave 1 sums them for the next step while wave 0 runs the transport, and keeps them in `hist`
// (L x d i64 per block); the first step of a launch sums its own (`fresh`).
template <int Q, int SW, bool T8, bool CLK, bool HM = false>
__device__ __forceinline__ int step_window(const DevModel &M, const Lds &S, int32_t *ring,
                                           int64_t *hist, uint32_t base, uint32_t lane,
                                           const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                           uint32_t tok, bool want_writer, bool fresh,
                                           uint32_t *chosen, PartClock<CLK> &clk,
                                           int64_t *pay = nullptr, bool defer = false) {
  if (tok >= M.vocab) return 1;
  const uint32_t d = M.d, W = M.W;
  const uint32_t next = base + 1 == W ? 0 : base + 1;  // the next step's ring slot
  // Windows of 16 rows or more: the next step's taps 2..split are summed before barrier 1, where
  // this wave waits for the norm, and taps split+1..W after barrier 2 (none of their ring rows is
  // the one this step writes); shorter windows sum every tap after barrier 2. Measured: W = 32,
  // taps 2..16 first 2.9 % faster than 2..8 (2..12, 2..20 and 2..24 no better); W = 16, taps
  // 2..4 first 1.7 % faster than none (2..6 slower in one-token serving launches).
  const uint32_t split = W > 16 ? 1 + (W - 1) / 2 : W == 16 ? 1 + (W - 1) / 4 : 1;
  for (uint32_t l = 0; l < M.L; l++) {
    const DevLayer ly = M.layers[l];
    int32_t *ring_l = ring + (uint64_t)l * W * d;
    int64_t *hist_l = hist + (uint64_t)l * d;
    int4 cbias[Q];
    uint32_t pw_drive[Q][4], pw_gate[Q][4];
    int64_t sum[Q][4];   // taps 1..W over the earlier positions
    int64_t part[Q][4];  // the next step's taps 2..split
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const uint32_t ch = 4 * (qv[k] ? qi[k] : 0);
      cbias[k] = *(const int4 *)(ly.conv_bias + ch);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        pw_drive[k][c] = prog_word(ly.prog, M.s_rec_in + 4 * k + c, lane);
        pw_gate[k][c] = prog_word(ly.prog, M.s_rec_in + 4 * Q + 4 * k + c, lane);
      }
      if (fresh) {
#pragma unroll
        for (int c = 0; c < 4; c++) sum[k][c] = 0;
        if (qv[k]) window_sum(M, ly, ring_l, base, 1, ch, sum[k]);
      } else {
        const longlong2 *hp = (const longlong2 *)(hist_l + ch);
        const longlong2 a = hp[0], b = hp[1];
        sum[k][0] = a.x;
        sum[k][1] = a.y;
        sum[k][2] = b.x;
        sum[k][3] = b.y;
      }
    }
#pragma unroll
    for (int k = 0; k < Q; k++) {
#pragma unroll
      for (int c = 0; c < 4; c++) part[k][c] = 0;
      if (qv[k]) window_sum(M, ly, ring_l, next, 2, 4 * qi[k], part[k], split);
    }
    // The first MLP group's gather words, for after barrier 3.
    uint32_t pg[4], pu[4];
    pair_mlp_words(M, ly, lane, 1, pg, pu);
    clk.sync(kPartLoads, kPartSync1);  // 1: the normed activations
    int4 drive[Q];
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) continue;
      const uint32_t ch = 4 * qi[k];
      int32_t gv[4];
#pragma unroll
      for (int c = 0; c < 4; c++) gv[c] = S.xbar[pw_gate[k][c]];
      drive[k] = make_int4(S.xbar[pw_drive[k][0]], S.xbar[pw_drive[k][1]], S.xbar[pw_drive[k][2]],
                           S.xbar[pw_drive[k][3]]);
      // Tap 0 on the drive and the conv bias, then the drive enters ring slot base.
      int64_t wide[4] = {cbias[k].x, cbias[k].y, cbias[k].z, cbias[k].w};
      tap4(M, ly, 0, ch, drive[k], wide);
#pragma unroll
      for (int c = 0; c < 4; c++) S.wide[ch + c] = wadd64(wide[c], sum[k][c]);
      *(int4 *)(ring_l + (uint64_t)base * d + ch) = drive[k];
      int64_t gate[4];
      gate_quat(M, S.seeds, gv, gate);
#pragma unroll
      for (int c = 0; c < 4; c++) S.gq[ch + c] = gate[c];
    }
    clk.sync(kPartTransition, kPartSync2);  // 2: the window sums and the output gates' quaternions
    // One-token serving launches (defer): the next step's window sums wait for nothing on the
    // recurrence wave's path, so this wave yields the issue slots it shares with another
    // block's recurrence wave until barrier 3 and takes them back for the MLP groups (in decode
    // launches it keeps the low priority throughout: measured faster there, slower here).
    if (defer) __builtin_amdgcn_s_setprio(0);
    // The next step's terms over earlier positions: tap 1 on this step's drive, taps
    // split+1..W from the ring (slots next - s, none of them the slot just written), added to
    // taps 2..split.
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) continue;
      const uint32_t ch = 4 * qi[k];
      int64_t acc[4] = {part[k][0], part[k][1], part[k][2], part[k][3]};
      tap4(M, ly, 1, ch, drive[k], acc);
      if (split < W) window_sum(M, ly, ring_l, next, split + 1, ch, acc);
      longlong2 *hp = (longlong2 *)(hist_l + ch);
      hp[0] = make_longlong2(acc[0], acc[1]);
      hp[1] = make_longlong2(acc[2], acc[3]);
    }
    clk.sync(kPartTransport, kPartSync3);  // 3: the normed activations
    if (defer) __builtin_amdgcn_s_setprio(3);  // the MLP groups, on both waves' path
    const uint64_t mbl = pair_mlp(M, S, ly, lane, 1, pg, pu);
    if (lane == 0) S.pair[1] = mbl;
    clk.sync(kPartMlp, kPartSync4);  // 4: both waves' MLP outputs and maxima
    pair_requant(M, S, lane, 1);
    clk.sync(kPartRequantMlp, kPartSync5);  // 5: the requantized MLP outputs
    if constexpr (HM) {  // the stream read's odd heads (ham_help), as step_main requests it
      const int32_t r = M.ham.at[l + 1];
      if (r >= 0 && l + 1 < M.L) ham_help<Q>(M, S, pay, lane, qv, qi);
    }
  }
  if constexpr (HM) {  // the readout read's odd heads, at every row (step_main)
    if (M.ham.at[M.L] >= 0) ham_help<Q>(M, S, pay, lane, qv, qi);
  }
  if (!want_writer || defer) return 0;  // the deferred writer runs on wave 0 alone
  clk.sync(kPartFinal, kPartSync6);  // 6: the query and the reuse flag
  *chosen = pair_writer<SW, T8, CLK>(M, S, 1, lane, nullptr, clk);
  return 0;
}

// The phase a kernel is compiled for. Prefill: decode launches with no generated step (the
// prompt, its last choice, the state out). Decode: decode launches that generate. Rows: the
// teacher-forced modes, sequences and score.
enum Phase : int { kPhasePrefill = 0, kPhaseDecode = 1, kPhaseRows = 2 };

// NW = 1: one wavefront per sequence (step); NW = 2: paired blocks (step_main, step_window).
// HM: a model with Hamming reads (one wavefront per sequence); T8: a model with an int8 table,
// whose writer scans its bytes.
// CLK: the part clocks (paired decode only), each sequence's counters to A.out_parts.
template <int Q, int SW, int PH, int NW, bool HM = false, bool T8 = false, bool CLK = false,
          bool DT = false>
__device__ __forceinline__ void run(const DevModel &M, const RunArgs &A) {
  static_assert(!HM || !T8, "the Hamming kernels' writer scans the 16-bit table");
  static_assert(!CLK || NW == 2, "the part clocks time paired blocks");
  extern __shared__ __align__(16) int32_t lds[];
  Lds S;
  {
    uint32_t at = 0;  // words; every region starts 16-byte aligned
    // The seed tables (rsqrt, then reciprocal) at the start.
    uint32_t *seed_lds = (uint32_t *)(lds + at);
    at += kRsqrtSeedWords + kRecipSeedWords;
    S.xbar = lds + at;
    at += M.xbar_words;
    S.mlp_out = (int64_t *)(lds + at);
    at += 2 * M.m;
    S.dscore = (uint32_t *)(lds + at);
    at += (M.D + 3u) & ~3u;
    S.kept = (uint32_t *)(lds + at);
    at += kMaxProbes;
    S.list = (uint32_t *)(lds + at);
    at += M.list_cap;
    S.wq = lds + at;
    at += (M.d + 3u) & ~3u;
    S.wmeta = (uint32_t *)(lds + at);
    at += 4;
    if (threadIdx.x == 0) S.wmeta[1] = 0;  // no query remembered yet
    S.st = nullptr;
    if (!(NW == 2 && kPairStateGlobal<Q, HM>)) {  // lds_bytes' state
      S.st = (int64_t *)(lds + at);
      at += 2 * M.L * M.d;
    }
    S.wide = S.gq = nullptr;
    S.rng = nullptr;
    S.pair = nullptr;
    if (NW == 2) {  // pair_lds_bytes
      S.wide = (int64_t *)(lds + at);
      at += 2 * M.d;
      S.gq = (int64_t *)(lds + at);
      at += 2 * M.d;
      S.rng = (uint32_t *)(lds + at);
      at += 2 * kMaxProbes;
      S.pair = (uint64_t *)(lds + at);
      at += 8;
    }
    S.tok = nullptr;
    S.hdist = nullptr;
    S.hpick = S.hwgt = S.hhist = S.hwd = S.hnib = S.hreq = nullptr;
    S.pst = nullptr;
    S.uend = S.farm = nullptr;
    if (HM) {  // ham_lds_bytes
      S.tok = (uint32_t *)(lds + at);
      at += M.context;
      S.hdist = (uint8_t *)(lds + at);
      at += ((M.context + 15u) & ~15u) / 4u;
      S.hpick = (uint32_t *)(lds + at);
      at += kMaxHamKept;
      S.hwgt = (uint32_t *)(lds + at);
      at += kMaxHamKept;
      S.hhist = (uint32_t *)(lds + at);
      at += kHamBins;
      S.hwd = (uint32_t *)(lds + at);
      at += kHamBins;
      S.hnib = (uint32_t *)(lds + at);
      at += M.d / 4;
      S.hreq = (uint32_t *)(lds + at);
      at += kHamReqWords;
      if (M.ham.place) {  // place_lds_bytes
        const uint32_t words = ((2u * M.context + 15u) & ~15u) / 4u;
        S.pst = (uint32_t *)(lds + at);
        at += kPlaceWords;
        S.uend = (uint16_t *)(lds + at);
        at += words;
        S.farm = (uint16_t *)(lds + at);
        at += words;
      }
    }
    S.clk = nullptr;
    if (CLK) {  // clock_lds_bytes
      S.clk = (uint64_t *)(lds + at);
      at += 4 * kParts;
    }
    // The seed tables by direct loads into LDS (16 bytes a lane, no registers), waited for with
    // the first sequence's loads below.
    // Wave w copies quads 64 w, 64 (w + NW), ... of each table (a copy's LDS base is the wave's).
    const uint32_t *rs = rsqrt_seed_table(), *rc = recip_seed_table();
    const uint32_t wl = threadIdx.x % kWave, wv = uniform32(threadIdx.x / kWave);
    for (uint32_t q = wv * kWave; q < kRsqrtSeedWords / 4; q += NW * kWave)
      lds_dma_quads(rs + 4 * q, seed_lds + 4 * q, kRsqrtSeedWords / 4 - q, wl);
    for (uint32_t q = wv * kWave; q < kRecipSeedWords / 4; q += NW * kWave)
      lds_dma_quads(rc + 4 * q, seed_lds + kRsqrtSeedWords + 4 * q, kRecipSeedWords / 4 - q, wl);
    S.seeds = Seeds(seed_lds, seed_lds + kRsqrtSeedWords);
  }
  // The wave index read as a scalar, so that the compiler treats the role branches as uniform.
  const uint32_t lane = threadIdx.x % kWave, wave = uniform32(threadIdx.x / kWave);
  // Paired blocks: wave 0 keeps the recurrence state, wave 1 the window ring.
  const bool keeps_state = NW == 1 || wave == 0, keeps_ring = NW == 1 || wave == 1;
  // The deferred writer (RunArgs::job_flag): compiled into the paired prefill kernels, the
  // one-token serving launches' family.
  constexpr bool kDefer = PH == kPhasePrefill && NW == 2 && !HM && !CLK && !DT;
  const bool defer = kDefer && A.job_flag != nullptr;
  const bool writes_out = wave == 0 && lane == 0;
  PartClock<CLK> clk;
  if constexpr (CLK) clk.acc = S.clk + wave * kParts;
  // The recurrence wave is the step's critical path (its instructions issue one after another,
  // each waiting for the last), while the ring wave's window sums have slack: the recurrence
  // wave takes the issue slots first wherever waves on its SIMD compete for them. In one-token
  // serving launches the ring wave raises its priority too, but for its next-step window sums
  // (step_window).
  if (NW == 2 && (wave == 0 || defer)) __builtin_amdgcn_s_setprio(3);
  const uint32_t d = M.d, L = M.L, W = M.W;
  int32_t *const block_ring = A.ring + (uint64_t)blockIdx.x * L * W * d;
  int64_t *hist = NW == 2 ? A.hist + (uint64_t)blockIdx.x * L * d : nullptr;
  // The recurrence state: LDS, or for paired blocks of two or more quaternions a lane the
  // block's global buffer after every block's window sums.
  int64_t *const stb = NW == 2 && kPairStateGlobal<Q, HM>
                           ? A.hist + ((uint64_t)gridDim.x + blockIdx.x) * L * d
                           : S.st;
  bool qv[Q];
  uint32_t qi[Q];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    qi[k] = lane + kWave * k;
    qv[k] = qi[k] < M.nq;
  }
  for (uint32_t s = blockIdx.x; s < A.n; s += gridDim.x) {
    const uint32_t sl = A.slots ? A.slots[s] : s;  // the session's index in the state arrays
    if (sl >= A.capacity) {
      if (writes_out) A.status[s] = kStatusSlot;
      continue;
    }
    // Fresh or resumed session: state, window rows (row r = the drive r + 1 positions back)
    // and position (LayerState::Recurrence, session.rs:1850).
    uint32_t pos = A.in_position ? A.in_position[sl] : 0u;
    uint32_t base = mod_window(M, pos);
    // A slot's history is its ring; otherwise the block's ring takes the rows.
    int32_t *ring = A.slots ? A.out_history + (uint64_t)sl * L * W * d : block_ring;
    // A serving slot's cache: the window sums its last launch formed for this position (paired
    // blocks take them in place of summing the window at the first step) and the writer's memory
    // of its last query, which depends on the model alone, so it is taken whenever it holds one.
    uint8_t *const ce = A.cache ? A.cache + (uint64_t)sl * A.cache_stride : nullptr;
    bool fresh = true;
    uint32_t fp_tag = 0;  // the fingerprint of the state the cached sums were formed beside
    uint32_t fp_acc = 0;
    if (ce) {
      const SlotCacheLayout cl = slot_cache_layout(M);
      const uint32_t *head = (const uint32_t *)ce;
      const uint4 h4 = *(const uint4 *)head;
      if (NW == 2) {
        hist = (int64_t *)(ce + cl.sums);
        fresh = h4.x != pos + 1;
        fp_tag = h4.w;
      }
      if (wave == 0 && M.writer_memory) {
        // The remembered query and kept drawers by direct loads into LDS, issued beside the
        // head's load rather than after it: a slot without a memory then leaves the block with
        // none (its last session's is overwritten).
        for (uint32_t q = 0; q < (d + 3) / 4; q += kWave)
          lds_dma_quads((const uint32_t *)(ce + cl.query) + 4 * q, (uint32_t *)S.wq + 4 * q,
                        (d + 3) / 4 - q, lane);
        lds_dma_quads((const uint32_t *)(ce + cl.kept), S.kept, kMaxProbes / 4, lane);
        if (lane == 0) {
          S.wmeta[0] = h4.z;
          S.wmeta[1] = h4.y != 0;
        }
      }
    }
    // The session's state: into LDS by direct loads where the state lives in LDS (its
    // fingerprint is then read back after the prologue's wait), else word by word.
    constexpr bool kStateLds = !(NW == 2 && kPairStateGlobal<Q, HM>);
    const bool state_done = kStateLds && keeps_state && A.in_state;
    if (state_done) {
      const uint32_t *src = (const uint32_t *)(A.in_state + (uint64_t)sl * L * d);
      const uint32_t quads = L * d / 2;  // L d i64
      for (uint32_t q = 0; q < quads; q += kWave)
        lds_dma_quads(src + 4 * q, (uint32_t *)stb + 4 * q, quads - q, lane);
    }
    for (uint32_t l = 0; l < L; l++)
#pragma unroll
      for (int k = 0; k < Q; k++)
        if (qv[k]) {
          uint32_t ch = 4 * qi[k];
          if (keeps_state && !state_done)
#pragma unroll
            for (int c = 0; c < 4; c++) {
              const uint64_t at = (uint64_t)l * d + ch + c;
              const int64_t v = A.in_state ? A.in_state[((uint64_t)sl * L + l) * d + ch + c] : 0;
              stb[at] = v;
              if (NW == 2 && ce) fp_acc += state_fp_word(v, (uint32_t)at);
            }
          if (keeps_ring && !A.slots)
            for (uint32_t r = 0; r < W; r++) {
              uint32_t slot = base + W - 1 - r;  // (base - 1 - r) mod W, from [0, 2 W - 1)
              slot = slot >= W ? slot - W : slot;
              int4 h = make_int4(0, 0, 0, 0);
              if (A.in_history) h = *(const int4 *)(A.in_history + (((uint64_t)sl * L + l) * W + r) * d + ch);
              *(int4 *)(ring + ((uint64_t)l * W + slot) * d + ch) = h;
            }
        }
    // Hamming models: the session's tokens into LDS, and its payload caches: the caller's
    // out_payloads (the resumed rows copied in first, each lane its own channels) or the block's.
    // A resumed token outside the vocabulary refuses the sequence (status 1) before any read
    // indexes a table by it.
    int64_t *pay = nullptr;
    bool bad_stream = false;
    if (HM) {
      uint32_t bad = 0;
      for (uint32_t i = lane; i < M.context; i += kWave) {
        const uint32_t v = A.in_stream && i < pos ? A.in_stream[(uint64_t)sl * M.context + i] : 0u;
        bad |= v >= M.vocab ? 1u : 0u;
        S.tok[i] = v;
      }
      bad_stream = wave_reduce32(bad, OpMax()) != 0;
      // The place read's register over the resumed tokens: the state their steps left (it
      // depends on the tokens and the model alone).
      if (M.ham.place && keeps_state) {  // paired blocks: wave 0 keeps the register
        place_init(M, S, lane);
        if (!bad_stream)
          for (uint32_t r = 0; r < pos; r++) place_advance<Q>(M, S, r, lane, qv, qi);
      }
      const uint64_t stride = (uint64_t)M.ham.slots * M.context * d;
      pay = A.out_payloads ? A.out_payloads + (uint64_t)sl * stride : A.pay + (uint64_t)blockIdx.x * stride;
      if (A.in_payloads && A.in_payloads != A.out_payloads && keeps_state)
        for (uint32_t c = 0; c < M.ham.slots; c++)
          for (uint32_t r = 0; r < pos; r++)
#pragma unroll
            for (int k = 0; k < Q; k++)
              if (qv[k]) {
                const uint64_t o = ((uint64_t)c * M.context + r) * d + 4 * qi[k];
                const longlong2 *src = (const longlong2 *)(A.in_payloads + (uint64_t)sl * stride + o);
                longlong2 *dst = (longlong2 *)(pay + o);
                dst[0] = src[0];
                dst[1] = src[1];
              }
    }
    // A serving slot's cached sums hold only beside the state they were formed with: a slot
    // whose state the host rewrote at the same position (a restore) sums its window afresh.
    if (NW == 2 && ce && wave == 0 && !state_done) {
      const uint32_t fp = wave_reduce32(fp_acc, OpAdd());
      if (lane == 0) S.wmeta[3] = fp;
    }
    uint64_t t_real = 0;
    if constexpr (CLK) {
      for (uint32_t i = lane; i < kParts; i += kWave) clk.acc[i] = 0;
      t_real = __builtin_amdgcn_s_memrealtime();
    }
    __builtin_amdgcn_s_waitcnt(0);  // the direct loads into LDS (seed tables, memory, state)
    if (NW == 2 && ce && state_done) {  // wave 0: the loaded state's fingerprint
      wave_sync();
      for (uint32_t l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < Q; k++)
          if (qv[k])
#pragma unroll
            for (int c = 0; c < 4; c++) {
              const uint64_t at = (uint64_t)l * d + 4 * qi[k] + c;
              fp_acc += state_fp_word(stb[at], (uint32_t)at);
            }
      const uint32_t fp = wave_reduce32(fp_acc, OpAdd());
      if (lane == 0) S.wmeta[3] = fp;
    }
    if (NW == 2)
      pair_sync();
    else
      wave_sync();
    clk.start();
    if (NW == 2 && ce) fresh = fresh || S.wmeta[3] != fp_tag;
    int status = bad_stream ? 1 : 0;
    uint32_t chosen = 0;
    constexpr bool decode = PH != kPhaseRows;
    const uint32_t *toks = A.tokens + (uint64_t)s * A.len;
    const uint32_t steps = bad_stream ? 0u : PH == kPhaseDecode ? A.len + A.gen : A.len;
    unsigned long long hits = 0;
    uint32_t done = 0;  // steps run
    for (uint32_t t = 0; t < steps; t++) {
      if (pos >= M.context && !(A.slide && A.slide[sl])) {  // set_context_slide: continue
        status = 2;
        break;
      }
      // Decode: the prompt's tokens, then each choice fed back (fbs-toks.rs:1513-1533); the
      // writer runs at the prompt's last step and every generated one. Sequences and score:
      // every token of the row, the writer wherever its choice is used.
      const uint32_t tok = PH == kPhaseDecode && t >= A.len ? chosen : toks[t];
      const uint64_t at = (uint64_t)s * A.len + t;
      const bool seq = !decode && A.mode == kModeSequences;
      const bool want = decode ? t + 1 >= A.len : (seq || A.out_tokens || t + 1 < A.len);
      // Sequences: every position's kept drawers and query; decode: the last step's.
      const bool last = decode && t + 1 == steps;
      uint32_t *kept_out = !A.out_kept ? nullptr
                           : seq       ? A.out_kept + at * M.P
                           : last      ? A.out_kept + (uint64_t)s * M.P
                                       : nullptr;
      int32_t *query_out = !A.out_query ? nullptr
                           : seq        ? A.out_query + at * d
                           : last       ? A.out_query + (uint64_t)s * d
                                        : nullptr;
      if (NW == 1) {
        // Sequences: every position's trace; decode: every step's, len + gen a sequence (not
        // with Hamming reads, whose serving slots are refused).
        uint8_t *trace = !A.out_trace || (HM && decode) ? nullptr
                         : A.out_trace + (decode ? (uint64_t)s * (A.len + A.gen) + t : at) *
                                             ((uint64_t)M.L * (2 * M.nq + M.nm));
        if (DT) {
          // The traced kernels: every position's record (sequences), and the forced replay.
          const uint32_t R = HM ? M.ham.nreads : 0u, H = HM ? M.ham.heads : 0u;
          DtCtx dc;
          dc.rec = A.out_dtrace + at * A.dstride;
          dc.decisions = A.decisions;
          dc.reads_at = A.decisions ? decision_bucket_bytes(M.L, M.nq) : 0u;
          dc.fb = A.force_buckets ? A.force_buckets + at * ((uint64_t)M.L * M.nq) : nullptr;
          dc.codes = A.force_codes ? A.force_codes + (uint64_t)s * A.len * R * H * 2 : nullptr;
          dc.mask = A.force_mask ? A.force_mask + (uint64_t)s * A.len * R * H : nullptr;
          status = step<Q, SW, HM, T8, true>(M, S, ring, base, lane, qv, qi, tok, want, &chosen,
                                             kept_out, query_out, pos, pay, trace, &dc);
        } else {
          status = step<Q, SW, HM, T8>(M, S, ring, base, lane, qv, qi, tok, want, &chosen, kept_out,
                                       query_out, pos, pay, trace);
        }
      } else {
        // The lane's indices pass through an empty asm at every step, so that the compiler forms
        // the lane's addresses inside the loop instead of holding them across the kernel.
        uint32_t ln = lane, qs[Q];
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int k = 0; k < Q; k++) {
          qs[k] = qi[k];
          asm volatile("" : "+v"(qs[k]));
        }
        if (wave == 0)
          status = step_main<Q, SW, T8, CLK, HM>(M, S, ln, qv, qs, tok, want, &chosen, kept_out,
                                                 query_out, clk, stb, pos, pay, defer);
        else
          status = step_window<Q, SW, T8, CLK, HM>(M, S, ring, hist, base, ln, qv, qs, tok, want,
                                                   t == 0 && fresh, &chosen, clk, pay, defer);
        if constexpr (kDefer) {
          // A deferred writer's job: the query as biased pairs, the session in each kept
          // drawer's list, its best reset (the scan kernel's atomic minimum starts there).
          if (defer && wave == 0 && status == 0) {
            wave_sync();
            if (S.wmeta[2] == 2) {
              uint32_t *jq = A.job_query + (uint64_t)s * (d / 2);
#pragma unroll
              for (int k = 0; k < Q; k++)
                if (qv[k]) {
                  const int4 q = *(const int4 *)(S.xbar + 4 * qi[k]);
                  // As scan_setup packs it: biased 16-bit pairs, or for an int8 table the query
                  // clamped to the table's range and scaled to meet its widened codes.
                  uint32_t b[4];
                  const int32_t qa[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                  for (int c = 0; c < 4; c++) {
                    if (T8) {
                      const int32_t lo = -(128 << M.t8_shift), hi = 127 << M.t8_shift;
                      const int32_t x = qa[c] < lo ? lo : qa[c] > hi ? hi : qa[c];
                      b[c] = (uint32_t)(x - lo) << (8 - M.t8_shift);
                    } else {
                      b[c] = (uint32_t)(qa[c] + 32768);
                    }
                  }
                  *(uint2 *)(jq + 2 * qi[k]) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
                }
              if (lane < M.P) {
                const uint32_t c = S.kept[lane];
                const uint32_t at = atomicAdd(A.drawer_count + c, 1u);
                if (at < A.list_stride) {
                  A.drawer_list[(uint64_t)c * A.list_stride + at] = s;
                  if (at % kServeSessions == 0) {  // this session opens a slice: its items
                    const uint32_t b = M.offsets[c], e = M.offsets[c + 1];
                    const uint32_t nch = (e - b + kServeRows - 1) / kServeRows;
                    const uint32_t i0 = nch ? atomicAdd(A.item_count, nch) : 0u;
                    for (uint32_t k = 0; k < nch && i0 + k < A.item_cap; k++) {
                      const uint32_t m0 = b + kServeRows * k;
                      A.items[i0 + k] = make_uint4(m0, e - m0 < kServeRows ? e - m0 : kServeRows,
                                                   c * A.list_stride + at, c);
                    }
                  }
                }
              }
              if (lane == 0) {
                A.job_best[s] = ~0ull;
                A.job_flag[s] = 1u;
              }
            }
          }
        }
      }
      if (status) break;
      done++;
      pos++;
      base = base + 1 == W ? 0 : base + 1;
      if (writes_out) {
        if (decode) {
          if (want) A.out_tokens[(uint64_t)s * (A.gen + 1) + t + 1 - A.len] = chosen;
        } else {
          if (A.out_tokens) A.out_tokens[at] = chosen;
          if (!seq && t + 1 < A.len && chosen == toks[t + 1]) hits++;
        }
      }
      clk.lap(kPartStep);
    }
    if constexpr (CLK) {
      const uint64_t real = __builtin_amdgcn_s_memrealtime() - t_real;
      pair_sync();  // both waves' counters
      uint64_t *o = A.out_parts + (uint64_t)s * kPartWords;
      for (uint32_t i = threadIdx.x; i < 2 * kParts; i += 2 * kWave) o[i] = S.clk[i];
      if (writes_out) {
        o[2 * kParts] = done;
        o[2 * kParts + 1] = real;
      }
    }
    if (!decode && A.mode == kModeScore && writes_out && hits) atomicAdd(A.matches, hits);
    if (decode && (status == 0 || A.slots)) {
      for (uint32_t l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < Q; k++)
          if (qv[k]) {
            uint32_t ch = 4 * qi[k];
            if (A.out_state && keeps_state)
#pragma unroll
              for (int c = 0; c < 4; c++)
                A.out_state[((uint64_t)sl * L + l) * d + ch + c] = stb[(uint64_t)l * d + ch + c];
            if (A.out_history && keeps_ring && !A.slots)
              for (uint32_t r = 0; r < W; r++) {
                uint32_t slot = base + W - 1 - r;  // (base - 1 - r) mod W, from [0, 2 W - 1)
                slot = slot >= W ? slot - W : slot;
                *(int4 *)(A.out_history + (((uint64_t)sl * L + l) * W + r) * d + ch) =
                    *(const int4 *)(ring + ((uint64_t)l * W + slot) * d + ch);
              }
          }
      if (A.out_position && writes_out) A.out_position[sl] = pos;
      if (HM && A.out_stream)
        for (uint32_t i = lane; i < M.context; i += kWave)
          A.out_stream[(uint64_t)sl * M.context + i] = S.tok[i];
    }
    if (writes_out) A.status[s] = status;
    if (NW == 2)
      pair_sync();
    else
      wave_sync();
    if (ce && wave == 0) {
      // The slot's cache for its next launch: the sums the last step formed (paired blocks) hold
      // for the slot's position, and the writer's memory as the block holds it.
      const SlotCacheLayout cl = slot_cache_layout(M);
      uint32_t *head = (uint32_t *)ce;
      for (uint32_t i = lane; i < d; i += kWave) ((int32_t *)(ce + cl.query))[i] = S.wq[i];
      if (lane < kMaxProbes) ((uint32_t *)(ce + cl.kept))[lane] = S.kept[lane];
      uint32_t fp = 0;
      if (NW == 2) {
        uint32_t acc = 0;
        for (uint32_t l = 0; l < L; l++)
#pragma unroll
          for (int k = 0; k < Q; k++)
            if (qv[k])
#pragma unroll
              for (int c = 0; c < 4; c++) {
                const uint64_t at = (uint64_t)l * d + 4 * qi[k] + c;
                acc += state_fp_word(stb[at], (uint32_t)at);
              }
        fp = wave_reduce32(acc, OpAdd());
      }
      if (lane == 0) {
        head[0] = NW == 2 && (done > 0 || !fresh) ? pos + 1 : 0u;
        head[1] = S.wmeta[1] != 0;
        head[2] = S.wmeta[0];
        head[3] = fp;
      }
      wave_sync();
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no direct load into LDS outlives the block
}

// The (quaternions per lane, lanes per writer row) pairs widths 32..1024 produce:
// d <= 256 -> Q 1 with S 1, 2, 4, 8; d <= 512 -> Q 2, S 16; d <= 1024 -> Q 4, S 32.
using KernelFn = void (*)(DevModel, RunArgs);
struct KernelSet {
  KernelFn q1s1, q1s2, q1s4, q1s8, q2s16, q4s32;
};

// Launches the member of `k` for the model's shape: one block of `waves` wavefronts per
// resident sequence.
inline hipError_t launch_shape(const KernelSet &k, const DevModel &M, const RunArgs &A,
                               uint32_t grid, uint32_t waves, size_t lds, hipStream_t stream) {
  uint32_t S = 1;
  while (S < M.d / 32) S <<= 1;
  KernelFn f = M.qpl == 1 && S == 1    ? k.q1s1
               : M.qpl == 1 && S == 2  ? k.q1s2
               : M.qpl == 1 && S == 4  ? k.q1s4
               : M.qpl == 1 && S == 8  ? k.q1s8
               : M.qpl == 2 && S == 16 ? k.q2s16
               : M.qpl == 4 && S == 32 ? k.q4s32
                                       : nullptr;
  if (!f) return hipErrorInvalidValue;
  DevModel m = M;
  RunArgs a = A;
  void *args[] = {&m, &a};
  hipError_t e = hipLaunchKernel((const void *)f, dim3(grid), dim3(waves * kWave), args, lds, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

// The phase's kernels, one family per translation unit (so that the units compile in parallel):
// FBS_ONE_KERNELS: `NAME<Q, SW>` (one wavefront per sequence); FBS_PAIR_KERNELS: `NAME_pair<Q, SW>`
// (paired blocks, at most 256 registers per lane so that two waves share each SIMD);
// FBS_HAM_KERNELS: `NAME_ham<Q, SW>` (one wavefront per sequence with the Hamming reads; their
// writer scans the 16-bit table); FBS_ONE8_KERNELS / FBS_PAIR8_KERNELS: `NAME_8`, `NAME_pair8`,
// the first two for an int8 table. Each defines `hipError_t launch_NAME[_pair|_ham|_8|_pair8](M,
// A, grid, lds, stream)`.
#define FBS_ONE_KERNELS(NAME, PH)                                                            \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME(DevModel M, RunArgs A) {                         \
    run<Q, SW, PH, 1>(M, A);                                                                  \
  }                                                                                           \
  hipError_t launch_##NAME(const DevModel &M, const RunArgs &A, uint32_t grid, size_t lds,    \
                           hipStream_t stream) {                                              \
    static const KernelSet k = {NAME<1, 1>, NAME<1, 2>, NAME<1, 4>,                           \
                                NAME<1, 8>, NAME<2, 16>, NAME<4, 32>};                         \
    return launch_shape(k, M, A, grid, 1, lds, stream);                                       \
  }
#define FBS_ONE8_KERNELS(NAME, PH)                                                           \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME##_8(DevModel M, RunArgs A) {                     \
    run<Q, SW, PH, 1, false, true>(M, A);                                                     \
  }                                                                                           \
  hipError_t launch_##NAME##_8(const DevModel &M, const RunArgs &A, uint32_t grid, size_t lds, \
                               hipStream_t stream) {                                          \
    static const KernelSet k = {NAME##_8<1, 1>, NAME##_8<1, 2>, NAME##_8<1, 4>,               \
                                NAME##_8<1, 8>, NAME##_8<2, 16>, NAME##_8<4, 32>};             \
    return launch_shape(k, M, A, grid, 1, lds, stream);                                       \
  }
#define FBS_PAIR8_KERNELS(NAME, PH)                                                          \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(128, 2) void NAME##_pair8(DevModel M, RunArgs A) {             \
    run<Q, SW, PH, 2, false, true>(M, A);                                                     \
  }                                                                                           \
  hipError_t launch_##NAME##_pair8(const DevModel &M, const RunArgs &A, uint32_t grid,        \
                                   size_t lds, hipStream_t stream) {                          \
    static const KernelSet k = {NAME##_pair8<1, 1>, NAME##_pair8<1, 2>, NAME##_pair8<1, 4>,   \
                                NAME##_pair8<1, 8>, NAME##_pair8<2, 16>, NAME##_pair8<4, 32>}; \
    return launch_shape(k, M, A, grid, 2, lds, stream);                                       \
  }
#define FBS_PAIR_KERNELS(NAME, PH)                                                           \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(128, 2) void NAME##_pair(DevModel M, RunArgs A) {              \
    run<Q, SW, PH, 2>(M, A);                                                                  \
  }                                                                                           \
  hipError_t launch_##NAME##_pair(const DevModel &M, const RunArgs &A, uint32_t grid,         \
                                  size_t lds, hipStream_t stream) {                           \
    static const KernelSet k = {NAME##_pair<1, 1>, NAME##_pair<1, 2>, NAME##_pair<1, 4>,      \
                                NAME##_pair<1, 8>, NAME##_pair<2, 16>, NAME##_pair<4, 32>};    \
    return launch_shape(k, M, A, grid, 2, lds, stream);                                       \
  }
// FBS_PAIR_HAM_KERNELS: `NAME_pair_ham<Q, SW>`, the paired kernels with the Hamming reads (each
// read's heads shared between the waves, ham_help); `launch_NAME_pair_ham(M, A, grid, lds,
// stream)`.
#define FBS_PAIR_HAM_KERNELS(NAME, PH)                                                       \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(128, 2) void NAME##_pair_ham(DevModel M, RunArgs A) {          \
    run<Q, SW, PH, 2, true>(M, A);                                                            \
  }                                                                                           \
  hipError_t launch_##NAME##_pair_ham(const DevModel &M, const RunArgs &A, uint32_t grid,     \
                                      size_t lds, hipStream_t stream) {                       \
    static const KernelSet k = {NAME##_pair_ham<1, 1>, NAME##_pair_ham<1, 2>,                 \
                                NAME##_pair_ham<1, 4>, NAME##_pair_ham<1, 8>,                 \
                                NAME##_pair_ham<2, 16>, NAME##_pair_ham<4, 32>};              \
    return launch_shape(k, M, A, grid, 2, lds, stream);                                       \
  }
// FBS_DT_KERNELS: `NAME_dt<Q, SW>`, `NAME_dt8<Q, SW>` and `NAME_dt_ham<Q, SW>`, the traced
// one-wavefront kernels (the decision and Hamming traces with the forced replay) of a 16-bit
// table, an int8 table and a model with Hamming reads; `launch_NAME_dt(M, A, grid, lds, stream)`
// picks by the model.
#define FBS_DT_KERNELS(NAME, PH)                                                             \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME##_dt(DevModel M, RunArgs A) {                    \
    run<Q, SW, PH, 1, false, false, false, true>(M, A);                                       \
  }                                                                                           \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME##_dt8(DevModel M, RunArgs A) {                   \
    run<Q, SW, PH, 1, false, true, false, true>(M, A);                                        \
  }                                                                                           \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME##_dt_ham(DevModel M, RunArgs A) {                \
    run<Q, SW, PH, 1, true, false, false, true>(M, A);                                        \
  }                                                                                           \
  hipError_t launch_##NAME##_dt(const DevModel &M, const RunArgs &A, uint32_t grid,           \
                                size_t lds, hipStream_t stream) {                             \
    static const KernelSet a = {NAME##_dt<1, 1>, NAME##_dt<1, 2>, NAME##_dt<1, 4>,            \
                                NAME##_dt<1, 8>, NAME##_dt<2, 16>, NAME##_dt<4, 32>};          \
    static const KernelSet b = {NAME##_dt8<1, 1>, NAME##_dt8<1, 2>, NAME##_dt8<1, 4>,         \
                                NAME##_dt8<1, 8>, NAME##_dt8<2, 16>, NAME##_dt8<4, 32>};       \
    static const KernelSet c = {NAME##_dt_ham<1, 1>, NAME##_dt_ham<1, 2>, NAME##_dt_ham<1, 4>, \
                                NAME##_dt_ham<1, 8>, NAME##_dt_ham<2, 16>, NAME##_dt_ham<4, 32>}; \
    return launch_shape(M.ham.heads ? c : M.table8 ? b : a, M, A, grid, 1, lds, stream);        \
  }
// FBS_PAIR_CLK_KERNELS: `NAME_pair_clk<Q, SW>` and `NAME_pair8_clk<Q, SW>`, the paired kernels
// with the part clocks; `launch_NAME_pair_clk(M, A, grid, lds, stream)` picks by the table.
#define FBS_PAIR_CLK_KERNELS(NAME, PH)                                                       \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(128, 2) void NAME##_pair_clk(DevModel M, RunArgs A) {          \
    run<Q, SW, PH, 2, false, false, true>(M, A);                                              \
  }                                                                                           \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(128, 2) void NAME##_pair8_clk(DevModel M, RunArgs A) {         \
    run<Q, SW, PH, 2, false, true, true>(M, A);                                               \
  }                                                                                           \
  hipError_t launch_##NAME##_pair_clk(const DevModel &M, const RunArgs &A, uint32_t grid,     \
                                      size_t lds, hipStream_t stream) {                       \
    static const KernelSet k16 = {NAME##_pair_clk<1, 1>, NAME##_pair_clk<1, 2>,               \
                                  NAME##_pair_clk<1, 4>, NAME##_pair_clk<1, 8>,               \
                                  NAME##_pair_clk<2, 16>, NAME##_pair_clk<4, 32>};            \
    static const KernelSet k8 = {NAME##_pair8_clk<1, 1>, NAME##_pair8_clk<1, 2>,              \
                                 NAME##_pair8_clk<1, 4>, NAME##_pair8_clk<1, 8>,              \
                                 NAME##_pair8_clk<2, 16>, NAME##_pair8_clk<4, 32>};           \
    return launch_shape(M.table8 ? k8 : k16, M, A, grid, 2, lds, stream);                     \
  }
#define FBS_HAM_KERNELS(NAME, PH)                                                            \
  template <int Q, int SW>                                                                    \
  __global__ __launch_bounds__(64) void NAME##_ham(DevModel M, RunArgs A) {                   \
    run<Q, SW, PH, 1, true>(M, A);                                                            \
  }                                                                                           \
  hipError_t launch_##NAME##_ham(const DevModel &M, const RunArgs &A, uint32_t grid,          \
                                 size_t lds, hipStream_t stream) {                            \
    static const KernelSet k = {NAME##_ham<1, 1>, NAME##_ham<1, 2>, NAME##_ham<1, 4>,         \
                                NAME##_ham<1, 8>, NAME##_ham<2, 16>, NAME##_ham<4, 32>};       \
    return launch_shape(k, M, A, grid, 1, lds, stream);                                       \
  }

}  // namespace fbs

#endif
