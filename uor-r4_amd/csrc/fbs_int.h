// fbs_int.h - exact integer arithmetic of the SpiralCore/FBS step, for gfx950 and the host.
//
// Every routine here is bit-exact with the reference's integer kernels
// (crates/uor-r4-integer/src/stack/kernels.rs, session.rs; its C++ twin
// docs/labs/d11-exporter-float-trunk/instrument/src/fbs_core.h): round-half-up shifts that
// saturate, products modulo 2^64 / 2^128, floor square roots and floor quotients. The reference
// forms its roots digit by digit and its quotients by hardware or restoring division; a GPU has
// neither, so this file computes them from fixed-point reciprocal estimates (a seed table and
// Newton steps) and then corrects the estimate with exact integer checks. The correction loops
// make the result exact for every input whatever the estimate's error; the estimates only
// decide how many correction steps run (at most one or two for every input class the tests
// sweep). No floating point is used anywhere.
//
// The functions are __host__ __device__ so that the same code is compiled into the kernels and
// into a host library that the CPU tests check against the oracle.
#ifndef UOR_FBS_INT_H
#define UOR_FBS_INT_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FBS_HD __host__ __device__ __forceinline__

namespace fbs {

typedef __int128 i128;
typedef unsigned __int128 u128;

constexpr int32_t kResidualExp = -16;  // RS stack/kernels.rs:34
constexpr int32_t kProductExp = -32;   // RS stack/kernels.rs:37
constexpr int32_t kStateExp = -32;     // RS stack/session.rs:72
constexpr int32_t kNormFineExp = -24;  // RS stack/kernels.rs:566
constexpr int32_t kQ12Exp = -12;       // RS stack/session.rs:475
constexpr int32_t kGridExpBias = 64;   // RS stack/kernels.rs:39
constexpr uint64_t kPhiLo = 2654435769ull;   // PHI_Q32 - 2^32, RS stack/mod.rs:167
constexpr uint64_t kRotationEps = 4295;      // RS stack/session.rs:141
constexpr uint64_t kGateEps = 0;             // RS stack/session.rs:144

// ---------------------------------------------------------------------------------------------
// Scalar conventions (RS stack/kernels.rs:41-135).

FBS_HD int64_t sat_add64(int64_t a, int64_t b) {
  int64_t r;
  if (__builtin_add_overflow(a, b, &r)) return b > 0 ? INT64_MAX : INT64_MIN;
  return r;
}
FBS_HD int64_t sat_neg64(int64_t v) { return v == INT64_MIN ? INT64_MAX : -v; }
FBS_HD int32_t sat_add32(int32_t a, int32_t b) {
  int64_t s = (int64_t)a + b;
  return s > INT32_MAX ? INT32_MAX : s < INT32_MIN ? INT32_MIN : (int32_t)s;
}
FBS_HD int32_t clamp_i32(int64_t v) {
  return v > INT32_MAX ? INT32_MAX : v < INT32_MIN ? INT32_MIN : (int32_t)v;
}
FBS_HD int64_t wadd64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
FBS_HD uint64_t uabs64(int64_t v) { return v < 0 ? 0ull - (uint64_t)v : (uint64_t)v; }
FBS_HD uint32_t uabs32(int32_t v) { return v < 0 ? 0u - (uint32_t)v : (uint32_t)v; }
FBS_HD int clz64(uint64_t v) { return v ? __builtin_clzll(v) : 64; }
FBS_HD int bitlen64(uint64_t v) { return 64 - clz64(v); }
FBS_HD int clz128(u128 v) {
  uint64_t hi = (uint64_t)(v >> 64);
  return hi ? clz64(hi) : 64 + clz64((uint64_t)v);
}

// `shift`: round-half-up arithmetic shift right by s, or a saturating shift left for s < 0
// (RS stack/kernels.rs:41-62).
FBS_HD int64_t shift(int64_t v, int32_t s) {
  if (s > 0) {
    if (s >= 63) return v < 0 ? -1 : 0;
    return sat_add64(v, (int64_t)1 << (s - 1)) >> s;
  }
  if (s < 0) {
    uint32_t k = (uint32_t)(-(int64_t)s);
    if (k > 63) k = 63;
    int64_t limit = INT64_MAX >> k;
    if (v > limit) return INT64_MAX;
    if (v < -limit) return INT64_MIN;
    return (int64_t)((uint64_t)v << k);
  }
  return v;
}

// `shift_wide`: round-half-up shift of an i128 (wrapping add of the half), clamped to i64
// (RS stack/kernels.rs:64-74). s <= 127.
FBS_HD int64_t shift_wide(i128 v, uint32_t s) {
  i128 r = s == 0 ? v : (i128)((u128)v + ((u128)1 << (s - 1))) >> s;
  if (r > (i128)INT64_MAX) return INT64_MAX;
  if (r < (i128)INT64_MIN) return INT64_MIN;
  return (int64_t)r;
}

// `to_exp_i32` (RS stack/kernels.rs:76-80).
FBS_HD int32_t to_exp_i32(int64_t v, int32_t from, int32_t to) {
  return clamp_i32(shift(v, to - from));
}

// `grid_apply`: v (16 + (|c| & 15)) 2^((|c| >> 4) - 68) rounded half up, then the sign of c;
// the product wraps modulo 2^64 like `scale_16_plus` (RS stack/kernels.rs:95-135).
FBS_HD int64_t grid_apply(int64_t v, int16_t code) {
  if (code == 0) return 0;
  uint32_t c = code < 0 ? (uint32_t)(-(int32_t)code) : (uint32_t)code;
  int32_t e = (int32_t)(c >> 4) - kGridExpBias;
  int64_t scaled = (int64_t)((uint64_t)v * (uint64_t)(16 + (c & 15)));
  scaled = shift(scaled, 4 - e);
  return code < 0 ? sat_neg64(scaled) : scaled;
}

// The same for a 32-bit input, whose product (16 + m) v never wraps.
FBS_HD int64_t grid_apply32(int32_t v, int16_t code) { return grid_apply((int64_t)v, code); }

// A grid code prepared for the kernels (16 bits): bits 0-5 the multiplier 16 + m (0 for the zero
// code), bit 6 the sign, bits 7-12 the right shift sh = 4 - e. With the sign folded in,
// grid_apply(v, code) = (v (+-(16 + m)) + 2^(sh-1) - [code < 0]) >> sh, because
// -floor((p + 2^(sh-1)) / 2^sh) = floor((-p + 2^(sh-1) - 1) / 2^sh). The form holds whenever
// 1 <= sh <= 62 and |v| (16 + m) + 2^(sh-1) < 2^63: always for a 32-bit v, and for a 64-bit v
// below 2^57 in magnitude. `grid_desc` returns kGridDescSlow for a code outside 1 <= sh <= 62.
constexpr uint16_t kGridDescSlow = 0xffff;

FBS_HD uint16_t grid_desc(int16_t code) {
  if (code == 0) return (uint16_t)(1u << 7);  // multiplier 0, shift 1: (0 + 1) >> 1 = 0
  uint32_t c = code < 0 ? (uint32_t)(-(int32_t)code) : (uint32_t)code;
  int32_t sh = 4 - ((int32_t)(c >> 4) - kGridExpBias);
  if (sh < 1 || sh > 62) return kGridDescSlow;
  return (uint16_t)((16 + (c & 15)) | (code < 0 ? 64u : 0u) | ((uint32_t)sh << 7));
}

FBS_HD int64_t grid_desc_apply(int64_t v, uint16_t desc) {
  const int32_t mag = desc & 63, neg = (desc >> 6) & 1;
  const uint32_t sh = (desc >> 7) & 63;
  const int32_t mul = (mag ^ -neg) + neg;
  return (v * mul + (((int64_t)1 << (sh - 1)) - neg)) >> sh;
}

// The window taps' descriptor (16 bits, two per word): bits 0-5 the signed multiplier
// +-(16 + m) (0 for the zero code), bits 6-11 the shift sh - 1. For a 32-bit v, with
// p = v mul and neg = [code < 0] (the multiplier's sign bit),
// grid_apply(v, code) = floor((p - neg + 2^(sh-1)) / 2^sh) = ((p - neg) >> (sh - 1)) + 1) >> 1.
// Valid for the codes grid_desc serves (1 <= sh <= 62); |p| < 2^36.
FBS_HD uint16_t tap_desc(int16_t code) {
  if (code == 0) return 0;  // multiplier 0, shift 1: ((0 >> 0) + 1) >> 1 = 0
  const uint32_t c = code < 0 ? (uint32_t)(-(int32_t)code) : (uint32_t)code;
  const int32_t sh = 4 - ((int32_t)(c >> 4) - kGridExpBias);
  if (sh < 1 || sh > 62) return kGridDescSlow;
  const int32_t mul = code < 0 ? -(int32_t)(16 + (c & 15)) : (int32_t)(16 + (c & 15));
  return (uint16_t)(((uint32_t)mul & 63u) | ((uint32_t)(sh - 1) << 6));
}

// grid_apply(v, code) for the tap descriptor in bits 16 h .. 16 h + 11 of `word`.
FBS_HD int64_t tap_desc_apply(int32_t v, uint32_t word, int h) {
  const int32_t mul = (int32_t)(word << (26 - 16 * h)) >> 26;  // sign-extended 6 bits
  const uint32_t shm1 = (word >> (16 * h + 6)) & 63u;
  const int64_t p = (int64_t)v * mul + (mul >> 31);            // v mul - neg
  return ((p >> shm1) + 1) >> 1;
}

// grid_apply for a 32-bit input through its descriptor (every valid code has one or is slow).
FBS_HD int64_t grid_apply32_desc(int32_t v, uint16_t desc, int16_t code) {
  if (desc == kGridDescSlow) return grid_apply((int64_t)v, code);
  const int32_t mag = desc & 63, neg = (desc >> 6) & 1;
  const uint32_t sh = (desc >> 7) & 63;
  const int32_t mul = (mag ^ -neg) + neg;
  return ((int64_t)v * (int64_t)mul + (((int64_t)1 << (sh - 1)) - neg)) >> sh;
}

// grid_apply for a 64-bit input: the descriptor form below 2^57, the reference routine above.
FBS_HD int64_t grid_apply64_desc(int64_t v, uint16_t desc, int16_t code) {
  if (desc == kGridDescSlow || v >= ((int64_t)1 << 57) || v <= -((int64_t)1 << 57))
    return grid_apply(v, code);
  return grid_desc_apply(v, desc);
}

// ---------------------------------------------------------------------------------------------
// Reciprocal and reciprocal-square-root seeds (compile-time tables, no floating point).

constexpr uint64_t ce_isqrt64(uint64_t n) {
  uint64_t r = 0, b = 1ull << 62;
  while (b > n) b >>= 2;
  while (b) {
    if (n >= r + b) {
      n -= r + b;
      r = (r >> 1) + b;
    } else {
      r >>= 1;
    }
    b >>= 2;
  }
  return r;
}

struct alignas(16) Seed384 {
  uint32_t v[384];
};
struct alignas(16) Seed256 {
  uint32_t v[256];
};

// rsqrt seed: bucket i = t >> 23 in [128, 512) of t in [2^30, 2^32); entry ~ 2^46 / sqrt(mid).
constexpr Seed384 make_rsqrt_seed() {
  Seed384 s{};
  for (int i = 0; i < 384; i++) {
    uint64_t mid = ((uint64_t)(2 * (i + 128) + 1)) << 22;   // bucket middle, < 2^32
    uint64_t root = ce_isqrt64(mid << 30);                   // sqrt(mid) 2^15
    s.v[i] = (uint32_t)((1ull << 61) / root);                // 2^46 / sqrt(mid)
  }
  return s;
}
// reciprocal seed: bucket i = d >> 23 in [256, 512) of d in [2^31, 2^32); entry ~ 2^63 / mid.
constexpr Seed256 make_recip_seed() {
  Seed256 s{};
  for (int i = 0; i < 256; i++) {
    uint64_t mid = ((uint64_t)(2 * (i + 256) + 1)) << 22;
    uint64_t v = (1ull << 63) / mid;
    s.v[i] = v > 0xffffffffull ? 0xffffffffu : (uint32_t)v;
  }
  return s;
}

// The seed tables, in global (constant) memory; the kernels copy them to LDS and pass that copy.
FBS_HD const uint32_t *rsqrt_seed_table() {
  static constexpr Seed384 seed = make_rsqrt_seed();
  return seed.v;
}
FBS_HD const uint32_t *recip_seed_table() {
  static constexpr Seed256 seed = make_recip_seed();
  return seed.v;
}
constexpr uint32_t kRsqrtSeedWords = 384, kRecipSeedWords = 256;

// The two tables as a pair of pointers (global by default).
struct Seeds {
  const uint32_t *rsq_seed;
  const uint32_t *rcp_seed;
  FBS_HD Seeds() : rsq_seed(rsqrt_seed_table()), rcp_seed(recip_seed_table()) {}
  FBS_HD Seeds(const uint32_t *r, const uint32_t *q) : rsq_seed(r), rcp_seed(q) {}
};

// The high 32 bits of a 32 x 32 product.
FBS_HD uint32_t mulhi32(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }

// y ~ 2^46 / sqrt(t) for t in [2^30, 2^32); y in [2^30, 2^31], relative error below 2^-27.
// Every product is 32 x 32 bits: y stays below 2^31 before the clamp and f = (3 2^32 - p) / 2
// below 2^33 (both checked over every input), so y f / 2^32 = y [f >= 2^32] + mulhi(y, f mod 2^32).
FBS_HD uint32_t rsqrt_q46(uint32_t t, const uint32_t *tab) {
  uint32_t y = tab[(t >> 23) - 128];
#pragma unroll
  for (int it = 0; it < 2; it++) {
    // Newton: y <- y (3 - t y^2 / 2^92) / 2, with p = t y^2 / 2^60 ~ 2^32.
    const uint32_t y2 = mulhi32(y, y);                        // y^2 / 2^32 <= 2^30
    const uint64_t p = ((uint64_t)t * y2) >> 28;              // ~ 2^32
    const uint64_t f = ((3ull << 32) - p) >> 1;               // ~ 2^32, < 2^33
    y = mulhi32(y, (uint32_t)f) + ((f >> 32) ? y : 0u);
    y = y > (1u << 31) ? 1u << 31 : y < (1u << 30) ? 1u << 30 : y;
  }
  return y;
}
FBS_HD uint32_t rsqrt_q46(uint32_t t) { return rsqrt_q46(t, rsqrt_seed_table()); }

// w ~ 2^63 / d for d in [2^31, 2^32); w in (2^31, 2^32), relative error below 2^-30. w stays
// below 2^32 and (2^63 - d w) / 2^31 inside +-2^23.1 at every step (checked over every input),
// so each product is 32 x 32 bits.
FBS_HD uint32_t recip_q63(uint32_t d, const uint32_t *tab) {
  uint32_t w = tab[(d >> 23) - 256];
#pragma unroll
  for (int it = 0; it < 2; it++) {
    // Newton: w <- w + w (2^63 - d w) / 2^63.
    const int32_t es = (int32_t)((int64_t)((1ull << 63) - (uint64_t)d * w) >> 31);
    w = (uint32_t)((int64_t)w + (((int64_t)es * (int64_t)(uint64_t)w) >> 32));
  }
  return w;
}
FBS_HD uint32_t recip_q63(uint32_t d) { return recip_q63(d, recip_seed_table()); }

// ---------------------------------------------------------------------------------------------
// Floor square root of a u128 (RS stack/kernels.rs:408-430 `stack_isqrt`): the result is
// isqrt(n << z) >> (z / 2) for the even z that puts n's top bit at 126 or 127; the normalised
// root is estimated from a 32-bit reciprocal square root, refined by two Newton steps on the
// exact remainder, and corrected to the floor.
FBS_HD uint64_t isqrt128(u128 n) {
  if (n == 0) return 0;
  int z = clz128(n) & ~1;
  u128 nn = n << z;                                  // [2^126, 2^128)
  uint32_t t = (uint32_t)(nn >> 96);                 // [2^30, 2^32)
  uint64_t y = rsqrt_q46(t);                         // 2^46 / sqrt(t)
  // sqrt(nn) ~ sqrt(t) 2^48 = t y 2^2.
  u128 s = ((u128)((uint64_t)t * y)) << 2;
  if (s >= ((u128)1 << 64)) s = ((u128)1 << 64) - 1;
#pragma unroll
  for (int it = 0; it < 2; it++) {
    // s += (nn - s^2) / (2 s), with 1 / (2 s) ~ y / 2^95.
    i128 diff = (i128)(nn - s * s);                  // small and signed
    i128 corr = ((diff >> 32) * (i128)y) >> 63;
    s = (u128)((i128)s + corr);
    if ((i128)s < 0) s = 0;
    if (s >= ((u128)1 << 64)) s = ((u128)1 << 64) - 1;
  }
  // sqrt(nn) < 2^64, so s + 1 <= 2^64 - 1 whenever the second loop runs.
  while (s * s > nn) s -= 1;
  while (s < ((u128)1 << 64) - 1 && (s + 1) * (s + 1) <= nn) s += 1;
  return (uint64_t)s >> (z >> 1);
}

// A normalised divisor and its reciprocal, for several quotients by one divisor.
struct Divisor {
  uint64_t d;   // the divisor
  uint64_t dn;  // d << z, in [2^63, 2^64)
  uint64_t v;   // ~ 2^127 / dn, relative error near 2^-60
  int z;
};

FBS_HD Divisor make_divisor(uint64_t d) {
  Divisor r;
  r.d = d;
  if (d == 0) {
    r.dn = 0;
    r.v = 0;
    r.z = 0;
    return r;
  }
  r.z = clz64(d);
  r.dn = d << r.z;
  uint64_t w = recip_q63((uint32_t)(r.dn >> 32));    // ~ 2^63 / (dn >> 32) ~ 2^95 / dn
  // One Newton step at 128 bits: v = w 2^32 + v (2^127 - dn v) / 2^127.
  u128 v0 = (u128)w << 32;
  i128 e = (i128)(((u128)1 << 127) - (u128)r.dn * v0);
  i128 corr = ((e >> 64) * (i128)v0) >> 63;
  u128 v = (u128)((i128)v0 + corr);
  if (v >= ((u128)1 << 64)) v = ((u128)1 << 64) - 1;
  r.v = (uint64_t)v;
  return r;
}

// floor(n / d) (RS stack/kernels.rs:345-360), zero for a zero divisor. Requires a quotient
// below 2^64.
FBS_HD uint64_t divq(u128 n, const Divisor &dv) {
  if (dv.d == 0) return 0;
  u128 nn = n << dv.z;                               // < 2^64 dn, so no bits are lost
  uint64_t nh = (uint64_t)(nn >> 64);
  u128 q = ((u128)nh * dv.v) >> 63;                  // under-estimate of nn / dn
  if (q >= ((u128)1 << 64)) q = ((u128)1 << 64) - 1;
  // Remainder-based refinement, then the exact floor.
  i128 rem = (i128)(nn - q * dv.dn);
  i128 step = ((rem >> 32) * (i128)(dv.v >> 32)) >> 63;
  q = (u128)((i128)q + step);
  rem = (i128)(nn - q * dv.dn);
  while (rem < 0) {
    q -= 1;
    rem += (i128)dv.dn;
  }
  while (rem >= (i128)dv.dn) {
    q += 1;
    rem -= (i128)dv.dn;
  }
  return (uint64_t)q;
}

FBS_HD uint64_t div128_64(u128 n, uint64_t d) { return divq(n, make_divisor(d)); }

// A Hamming candidate's weight at `distance` bits under a head's margin (bits at Q16), at Q31:
// max(0, m - d) / max(m, 1), floored (RS stack/hamming.rs:243-252 `copy_weight_q31`). At most
// 2^31, so it fits 32 bits.
FBS_HD uint32_t copy_weight_q31(int32_t margin_q16, uint32_t distance) {
  const int64_t over = (int64_t)margin_q16 - ((int64_t)distance << 16);
  if (over <= 0) return 0;
  const uint64_t m = (uint64_t)(margin_q16 > (1 << 16) ? margin_q16 : (1 << 16));
  return (uint32_t)div128_64((u128)((uint64_t)over << 31), m);
}

// ---------------------------------------------------------------------------------------------
// Vector kernels, one element at a time.

// RMSNorm's per-vector factor (RS stack/kernels.rs:569-620 `stack_rms_norm_fine`, TW 294-330):
// from the sum of the squared pre-shifted values, the multiplier r = floor(2^96 / s) with
// s = isqrt(ms << 68) truncated to 128 bits; `huge` marks s = 1, where r = 2^96.
struct NormFactor {
  uint64_t r;
  bool huge;
};

FBS_HD NormFactor norm_factor(uint64_t sum, uint32_t n, int64_t eps_int) {
  uint64_t mean = n == 0 ? 0 : div128_64((u128)sum, n);
  int64_t ms = wadd64((int64_t)mean, eps_int);
  if (ms < 1) ms = 1;
  u128 wide = (u128)(uint64_t)ms << 68;              // truncated to 128 bits as the reference
  uint64_t s = isqrt128(wide);
  NormFactor f;
  if (s <= 1) {
    f.r = 0;
    f.huge = true;
  } else {
    f.r = div128_64((u128)1 << 96, s);
    f.huge = false;
  }
  return f;
}

// A signed remainder below 2^66 in magnitude as hi 2^64 + lo (hi small and signed).
struct Rem96 {
  int64_t hi;
  uint64_t lo;
};

// n - q d for a remainder n, q < 2^32 and d < 2^64.
FBS_HD Rem96 rem_sub_qd(Rem96 n, uint32_t q, uint64_t d) {
  const uint64_t p1 = (uint64_t)q * (uint32_t)d, p2 = (uint64_t)q * (uint32_t)(d >> 32);  // q d = p2 2^32 + p1
  const uint64_t pl = p1 + (p2 << 32);
  const uint64_t ph = (p2 >> 32) + (pl < p1);
  Rem96 r;
  r.lo = n.lo - pl;
  r.hi = n.hi - (int64_t)ph - (int64_t)(n.lo < pl);
  return r;
}

// One step each way toward 0 <= r < d: the quotient q and remainder r of a digit whose estimate
// is within [q - UP, q + 1].
template <int UP>
FBS_HD void digit_fix(uint64_t &q, Rem96 &r, uint64_t d) {
  if (r.hi < 0) {  // q one too large
    q -= 1;
    const uint64_t lo = r.lo + d;
    r.hi += (int64_t)(lo < d);
    r.lo = lo;
  }
#pragma unroll
  for (int i = 0; i < UP; i++)
    if (r.hi > 0 || r.lo >= d) {
      q += 1;
      r.hi -= (int64_t)(r.lo < d);
      r.lo -= d;
    }
}

// floor(2^96 / s) for s in [2^34, 2^64), as two 31-bit quotient digits of 2^E / D with
// D = s 2^zs normalised and E = 96 + zs. w = recip_q63(D / 2^32) is 2^95 / D within a relative
// [-2^-30.4, 2^-31] (the seed error, checked over every input, and the truncation of D), so each
// digit estimate is within [q - 3, q + 1] and the exact remainder (below 2^66, kept in 96 bits)
// fixes it in fixed steps.
// div_2p96_w takes w = recip_q63(D / 2^32) from the caller, which may hold it already.
FBS_HD uint64_t div_2p96_w(uint64_t s, uint32_t w) {
  const int zs = clz64(s);                            // [0, 29]
  const uint64_t D = s << zs;                         // [2^63, 2^64)
  const int E = 96 + zs;
  // Digit 1: Q1 = floor(2^(E-31) / D) <= 2^31.
  uint64_t q1 = w >> (126 - E);
  Rem96 n1;
  n1.hi = (int64_t)1 << (E - 95);
  n1.lo = 0;
  Rem96 r1 = rem_sub_qd(n1, (uint32_t)q1, D);
  digit_fix<2>(q1, r1, D);
  // Digit 2: Q0 = floor(R1 2^31 / D) < 2^31, R1 in [0, D).
  const uint64_t R = r1.lo;
  uint64_t q0 = ((uint64_t)(uint32_t)(R >> 32) * w + mulhi32((uint32_t)R, w)) >> 32;
  Rem96 n2;
  n2.hi = (int64_t)(R >> 33);
  n2.lo = R << 31;
  Rem96 r0 = rem_sub_qd(n2, (uint32_t)q0, D);
  digit_fix<3>(q0, r0, D);
  return (q1 << 31) + q0;
}

FBS_HD uint64_t div_2p96(uint64_t s, const Seeds &sd = Seeds()) {
  const uint64_t top = (s << clz64(s)) >> 32;         // D / 2^32
  return div_2p96_w(s, recip_q63((uint32_t)top, sd.rcp_seed));
}

// norm_factor for n = 2^log2n in 64-bit steps (the kernels' form; equal to norm_factor).
// With m = ms mod 2^60 and M = 16 m < 2^64, s = isqrt(m 2^68) = isqrt(M 2^64) =
// floor(2^32 sqrt(M)). M is normalised to Mn = M 4^k in [2^62, 2^64); its root t = isqrt(Mn) in
// [2^31, 2^32) comes from the 32-bit reciprocal square root within 1 (as in unit_q30) and one
// step each way; then s = t 2^J + f with J = 32 - k and f = floor(2^J (sqrt(Mn) - t)) =
// floor(2^J rem / (t + sqrt(Mn))), rem = Mn - t^2 <= 2 t. The divisor t + sqrt(Mn) lies in
// [2 t, 2 t + 1) and 2^J rem / (2 t (2 t + 1)) < 1, so f is fh = floor(2^(J-1) rem / t) or
// fh - 1 (and below 2^J). fh comes from the 32-bit reciprocal of t, refined once on the exact
// remainder (within [fh - 1, fh]) and fixed by one step. Writing 2^(J-1) rem = fh t + rho
// (0 <= rho < t), the exact test f (2^(J+1) t + f) <= rem 4^J for f = fh reads
// fh^2 <= 2^(J+1) rho.
FBS_HD NormFactor norm_factor_pow2(uint64_t sum, uint32_t log2n, int64_t eps_int,
                                    const Seeds &sd = Seeds()) {
  NormFactor out;
  int64_t ms = wadd64((int64_t)(sum >> log2n), eps_int);
  if (ms < 1) ms = 1;
  const uint64_t m = (uint64_t)ms & ((1ull << 60) - 1);
  if (m == 0) {  // isqrt(0) = 0, raised to 1: r = 2^96
    out.r = 0;
    out.huge = true;
    return out;
  }
  const uint64_t M = m << 4;
  const int z = clz64(M) & ~1;
  const uint64_t mn = M << z;
  const int J = 32 - (z >> 1);                        // [3, 32]
  // Every product below has 32-bit factors: mt, y and t are below 2^32, |diff| / 2^16 below
  // 2^31 (t is within 2^6 of the root before its Newton step).
  const uint32_t mt = (uint32_t)(mn >> 32);
  const uint32_t y = rsqrt_q46(mt, sd.rsq_seed);
  uint64_t t = ((uint64_t)mt * y) >> 30;
  t = t > 0xffffffffull ? 0xffffffffull : t;
  const int64_t diff = (int64_t)(mn - (uint64_t)(uint32_t)t * (uint32_t)t);
  t = (uint64_t)((int64_t)t + (((int64_t)(int32_t)(diff >> 16) * (int64_t)(uint64_t)y) >> 47));
  t = t > 0xffffffffull ? 0xffffffffull : t < (1ull << 31) ? (1ull << 31) : t;
  uint64_t sq = (uint64_t)(uint32_t)t * (uint32_t)t;
  if (sq > mn) {
    t -= 1;
    sq -= 2 * t + 1;
  }
  if (t < 0xffffffffull && sq + 2 * t + 1 <= mn) {
    sq += 2 * t + 1;
    t += 1;
  }
  const uint64_t rem = mn - sq;                       // [0, 2 t] <= 2^33 - 2
  const uint64_t num = rem << (J - 1);                // < 2^64
  const uint32_t w = recip_q63((uint32_t)t, sd.rcp_seed); // ~ 2^63 / t
  uint64_t fh = ((uint64_t)(uint32_t)(num >> 32) * w) >> 31;  // [q - 9, q]
  const uint64_t r0 = num - fh * t;                   // [0, 10 t)
  fh += ((uint64_t)(uint32_t)(r0 >> 4) * w) >> 59;    // [q - 1, q]
  uint64_t rho = num - fh * t;                        // [0, 2 t)
  if (rho >= t) {
    fh += 1;
    rho -= t;
  }
  uint64_t f = fh;
  if (fh >> J) {
    f = fh - 1;                                       // f < 2^J
  } else if (fh) {
    const bool big = (rho >> (63 - J)) != 0;          // 2^(J+1) rho >= 2^64 > fh^2
    if (!big && (uint64_t)(uint32_t)fh * (uint32_t)fh > (rho << (J + 1))) f = fh - 1;  // fh < 2^J
  }
  const uint64_t s = (t << J) + f;                    // >= 2^34
  // s = t 2^J + f with t in [2^31, 2^32) and f < 2^J, so s normalised to [2^63, 2^64) is
  // t 2^32 + f 2^(32-J): its top 32 bits are t, whose reciprocal w is at hand.
  out.r = div_2p96_w(s, w);
  out.huge = false;
  return out;
}

// The largest k in [0, 64) with ok(k), for an ok that holds up to some k and fails after it, or
// -1 when ok(0) fails. In device code every lane of the wave (all 64 active) tests its own k and
// one ballot gives the answer; on the host the same 64 tests run in turn.
template <class F>
FBS_HD int last_ok64(F ok) {
#ifdef __HIP_DEVICE_COMPILE__
  const uint64_t m = (uint64_t)__ballot(ok((int)(threadIdx.x & 63u)));
  return m ? 63 - __builtin_clzll(m) : -1;
#else
  int k = -1;
  for (int i = 0; i < 64; i++)
    if (ok(i)) k = i;
  return k;
#endif
}

// norm_factor_pow2 with its corrections made in parallel: each exact quantity (the root t, its
// extension f, the quotient r) is estimated to within 32 and then found as the last of 64
// consecutive candidates that passes its exact test, one candidate per lane of the wave.
// The estimates come from one reciprocal square root y ~ 2^46 / sqrt(mt) (mt the top 32 bits of
// the normalised mean square, relative error below 2^-28.9):
//   t  = isqrt(mn):                       t0 = mt y / 2^30, within 12 of t;
//   f  = floor(2^J (sqrt(mn) - t)):        f0 = rem 2^(J-1) y / 2^62, within 12 of f;
//   r  = floor(2^96 / s), s = t 2^J + f:  r0 = y 2^(34-J) refined by one Newton step on the exact
//                                          2^96 - r0 s, within 32 of r wherever r < 2^61.
// `ok` is false where a candidate window does not hold its answer strictly inside (an input
// beyond the estimates' ranges); the caller then takes norm_factor_pow2.
FBS_HD NormFactor norm_factor_wave(uint64_t sum, uint32_t log2n, int64_t eps_int, const Seeds &sd,
                                   bool &ok) {
  NormFactor out;
  ok = true;
  int64_t ms = wadd64((int64_t)(sum >> log2n), eps_int);
  if (ms < 1) ms = 1;
  const uint64_t m = (uint64_t)ms & ((1ull << 60) - 1);
  if (m == 0) {  // isqrt(0) = 0, raised to 1: r = 2^96
    out.r = 0;
    out.huge = true;
    return out;
  }
  out.huge = false;
  const uint64_t M = m << 4;
  const int z = clz64(M) & ~1;
  const uint64_t mn = M << z;                         // [2^62, 2^64)
  const int J = 32 - (z >> 1);                        // [3, 32]
  const uint32_t mt = (uint32_t)(mn >> 32);
  const uint32_t y = rsqrt_q46(mt, sd.rsq_seed);
  // t: candidates tb + k, tested t^2 <= mn (t < 2^32, so t^2 < 2^64).
  const uint64_t tb = (((uint64_t)mt * y) >> 30) - 32;
  // (The tests combine their conditions without branching: every lane evaluates all of them.)
  const int kt = last_ok64([&](int k) {
    const uint64_t c = tb + (uint64_t)k;
    return (c <= 0xffffffffull) & (c * c <= mn);
  });
  const uint64_t t = tb + (uint64_t)(kt < 0 ? 0 : kt);
  const uint64_t rem = mn - t * t;                    // [0, 2 t]
  const uint64_t num = rem << (J - 1);                // rem 2^(J-1) < 2^64
  // f: candidates fb + k below 2^J, tested f (2^(J+1) t + f) <= rem 4^J, that is
  // f^2 <= 2^(J+1) (num - f t).
  const uint64_t f0 = (((num >> 32) * y) + ((((uint64_t)(uint32_t)num) * y) >> 32)) >> 30;
  const uint64_t fb = f0 > 32 ? f0 - 32 : 0;
  const uint64_t flim = 1ull << J;
  const int kf = last_ok64([&](int k) {
    const uint64_t c = fb + (uint64_t)k;
    const uint64_t ct = c * t;                        // c < 2^32 where it counts, t < 2^32
    const uint64_t rho = num - ct;
    // 2^(J+1) rho >= 2^64 > c^2 where rho >> (63 - J) is not zero.
    return (c < flim) & (ct <= num) & (((rho >> (63 - J)) != 0) | (c * c <= (rho << (J + 1))));
  });
  const uint64_t f = fb + (uint64_t)(kf < 0 ? 0 : kf);
  const uint64_t sv = (t << J) + f;                   // [2^34, 2^64)
  // r: candidates rb + k, tested r s <= 2^96.
  const uint64_t r0 = (uint64_t)y << (34 - J);
  const u128 p0 = (u128)r0 * sv;
  const i128 e = (i128)(((u128)1 << 96) - p0);        // |e| < 2^69
  const i128 corr = ((e >> 32) * (i128)r0) >> 64;
  const int64_t r1 = (int64_t)((i128)r0 + corr);
  const uint64_t rb = (uint64_t)(r1 - 32);
  const int kr = last_ok64([&](int k) {
    const uint64_t c = rb + (uint64_t)k;
    return (u128)c * sv <= ((u128)1 << 96);
  });
  out.r = rb + (uint64_t)(kr < 0 ? 0 : kr);
  // Each answer must lie strictly inside its window (or at the end of f's range).
  ok = kt > 0 && kt < 63 && (kf > 0 || fb == 0) && (kf < 63 || fb + 63 >= flim - 1) && kr > 0 &&
       kr < 63 && r1 > 32;
  return out;
}

// One normalised value: round(r y / 2^38) with the sign of y, clamped to i64.
FBS_HD int64_t norm_apply(NormFactor f, int64_t y) {
  uint64_t u = uabs64(y);
  u128 mag = f.huge ? ((u128)u << 96) : (u128)f.r * u;
  i128 p = y < 0 ? (i128)(0 - mag) : (i128)mag;
  i128 r = (i128)((u128)p + ((u128)1 << 37)) >> 38;
  if (r > (i128)INT64_MAX) return INT64_MAX;
  if (r < (i128)INT64_MIN) return INT64_MIN;
  return (int64_t)r;
}

// norm_apply for |y| < 2^24 (every pre-shifted norm input) and r < 2^62 (every factor but the
// huge one): with P = r |y| = A + B 2^32 (A = r_lo |y|, B = r_hi |y|), floor((P + h) / 2^38) =
// floor((B + floor((A + h) / 2^32)) / 2^6); h = 2^37 for y >= 0, 2^37 - 1 for the negated form
// (floor((-P + 2^37) / 2^38) = -floor((P + 2^37 - 1) / 2^38)).
FBS_HD int64_t norm_apply24_fast(NormFactor f, int64_t y) {
  const uint32_t u = (uint32_t)(y < 0 ? -y : y);
  const uint64_t A = (uint64_t)(uint32_t)f.r * u, B = (f.r >> 32) * (uint64_t)u;
  const uint64_t h = y < 0 ? (1ull << 37) - 1 : (1ull << 37);
  const int64_t mag = (int64_t)((B + ((A + h) >> 32)) >> 6);
  return y < 0 ? -mag : mag;
}
FBS_HD int64_t norm_apply24(NormFactor f, int64_t y) {
  if (f.huge) return norm_apply(f, y);
  const uint32_t u = (uint32_t)(y < 0 ? -y : y);
  const uint64_t A = (uint64_t)(uint32_t)f.r * u, B = (f.r >> 32) * (uint64_t)u;
  const uint64_t h = y < 0 ? (1ull << 37) - 1 : (1ull << 37);
  const int64_t mag = (int64_t)((B + ((A + h) >> 32)) >> 6);
  return y < 0 ? -mag : mag;
}

// eps at the square exponent of pre-shift sh (kernels.rs:596-602): shift(mantissa,
// (2 (-16 + sh)) - eps_exp), never negative.
FBS_HD int64_t norm_eps(int64_t eps_mantissa, int32_t eps_exp, int32_t sh) {
  int64_t e = shift(eps_mantissa, (kResidualExp + sh) * 2 - eps_exp);
  return e < 0 ? 0 : e;
}

// quantize16's element rule: clamp(shift(v, s), +-32767) (RS stack/kernels.rs:545-553).
FBS_HD int32_t quantize_elem(int64_t v, int32_t s) {
  // shift(v, s) for 0 <= s <= 62: the half is added with saturation, as the reference does.
  int64_t y = s == 0 ? v : sat_add64(v, (int64_t)1 << (s - 1)) >> s;
  return (int32_t)(y > 32767 ? 32767 : y < -32767 ? -32767 : y);
}

// to_exp_i32 of a and of -a (|a| <= 32767) from exponent `exp` to -16: a << -k clamped to the
// i32 range, or rounded half up by k = -16 - exp (zero once k >= 17, as |a| + 2^(k-1) < 2^k).
FBS_HD void publish16_pair(int32_t a, int32_t exp, int32_t *p, int32_t *n) {
  const int32_t k = kResidualExp - exp;
  if (k <= 0) {
    const int32_t l = -k > 40 ? 40 : -k;
    *p = clamp_i32((int64_t)a << l);
    *n = clamp_i32(-(int64_t)a << l);
  } else if (k <= 16) {
    const int32_t h = 1 << (k - 1);
    *p = (a + h) >> k;
    *n = (-a + h) >> k;
  } else {
    *p = 0;
    *n = 0;
  }
}

// to_exp_i32(v, -24, -16) and to_exp_i32(sat_neg64(v), -24, -16): values beyond +-2^40 clamp
// to the i32 range either way, so v is clamped there first and the shift cannot overflow.
FBS_HD void publish64_pair(int64_t v, int32_t *p, int32_t *n) {
  const int64_t lim = (int64_t)1 << 40;
  const int64_t c = v > lim ? lim : v < -lim ? -lim : v;
  *p = clamp_i32((c + 128) >> 8);
  *n = clamp_i32((128 - c) >> 8);
}

// ---------------------------------------------------------------------------------------------
// Quaternions.

// Hamilton product a (x) b modulo 2^128 (RS stack/kernels.rs:998-1030, TW 363-370).
FBS_HD void hamilton64(const int64_t a[4], const int64_t b[4], i128 o[4]) {
#define FBS_P(i, j) ((i128)a[i] * (i128)b[j])
  o[0] = FBS_P(0, 0) - FBS_P(1, 1) - FBS_P(2, 2) - FBS_P(3, 3);
  o[1] = FBS_P(0, 1) + FBS_P(1, 0) + FBS_P(2, 3) - FBS_P(3, 2);
  o[2] = FBS_P(0, 2) - FBS_P(1, 3) + FBS_P(2, 0) + FBS_P(3, 1);
  o[3] = FBS_P(0, 3) + FBS_P(1, 2) - FBS_P(2, 1) + FBS_P(3, 0);
#undef FBS_P
}

// a (x) b for a 32-bit left operand: the same sums, from 32 x 32 partial products. b = H 2^32
// + L with H signed and L read as signed (L - 2^32 [L >= 2^31]); the borrow goes into the high
// sum. With |a| summing to at most 2^31 + 4 (every unit or snapped quaternion times lambda
// <= 2^31) neither 64-bit sum can overflow, so the result equals hamilton64's.
FBS_HD void hamilton32_hl(const int32_t a[4], const int64_t b[4], int64_t Ho[4], int64_t Lo[4]) {
  int32_t hi[4], lo[4], bor[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    hi[j] = (int32_t)(b[j] >> 32);
    lo[j] = (int32_t)(uint32_t)b[j];
    bor[j] = lo[j] < 0 ? 1 : 0;
  }
  const int sgn[4][4] = {{1, -1, -1, -1}, {1, 1, 1, -1}, {1, -1, 1, 1}, {1, 1, -1, 1}};
  const int idx[4][4] = {{0, 1, 2, 3}, {1, 0, 3, 2}, {2, 3, 0, 1}, {3, 2, 1, 0}};
  // Output k sums sgn[k][i] a[i] b[idx[k][i]].
#pragma unroll
  for (int k = 0; k < 4; k++) {
    int64_t H = 0, L = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int j = idx[k][i];
      int64_t ph = (int64_t)a[i] * (int64_t)hi[j] + (bor[j] ? (int64_t)a[i] : 0);
      int64_t pl = (int64_t)a[i] * (int64_t)lo[j];
      if (sgn[k][i] > 0) {
        H += ph;
        L += pl;
      } else {
        H -= ph;
        L -= pl;
      }
    }
    Ho[k] = H;
    Lo[k] = L;
  }
}
FBS_HD void hamilton32(const int32_t a[4], const int64_t b[4], i128 o[4]) {
  int64_t H[4], L[4];
  hamilton32_hl(a, b, H, L);
#pragma unroll
  for (int k = 0; k < 4; k++) o[k] = ((i128)H[k] << 32) + (i128)L[k];
}

// shift_wide(H 2^32 + L, 14) (the raw output gate's product, session.rs:4951-4968) for |H| < 2^44:
// H 2^18 + floor((L + 2^13) / 2^14). |L| <= (2^31 + 4) 2^31 (hamilton32's bound), so nothing
// wraps, and the sum stays below 2^63 in magnitude: shift_wide's clamp never acts.
FBS_HD int64_t gate_shift14_fast(int64_t H, int64_t L) {
  return H * (1ll << 18) + ((L + (1ll << 13)) >> 14);
}

// The transport (session.rs:5097-5145): shift_wide(H 2^32 + L + keep wide 2^16, 31) for
// |H| < 2^59, keep <= 2^31 and -2^45 <= wide < 2^45. With wide = wh 2^32 + wl (wl < 2^32) and
// K = keep wl < 2^63 = (K >> 15) 2^15 + (K mod 2^15), the sum is 2^31 (2 H + keep wh 2^17 + (K >> 15))
// + Z with Z = L + (K mod 2^15) 2^16, so the shift is that bracket plus floor((Z + 2^30) / 2^31).
// The terms are below 2^60, 2^61, 2^48 and 2^32 in magnitude: nothing wraps and the clamp never
// acts.
FBS_HD int64_t transport_fast(int64_t H, int64_t L, uint64_t keep, int64_t wide) {
  const int64_t wh = wide >> 32;
  const uint64_t K = keep * (uint64_t)(uint32_t)wide;
  const int64_t Z = L + (int64_t)((K & 0x7fffu) << 16);
  return 2 * H + (int64_t)keep * wh * (1ll << 17) + (int64_t)(K >> 15) + ((Z + (1ll << 30)) >> 31);
}
// The fast forms' ranges.
FBS_HD bool gate_fast_ok(int64_t H) { return (uint64_t)(H + (1ll << 44)) < (1ull << 45); }
FBS_HD bool transport_fast_ok(int64_t H, int64_t wide, uint64_t keep) {
  return (uint64_t)(H + (1ll << 59)) < (1ull << 60) && (uint64_t)(wide + (1ll << 45)) < (1ull << 46) &&
         keep <= (1ull << 31);
}

// a (x) b for 32-bit operands: each partial product fits in i64 and, with |a| summing to at
// most 2^31 + 4, so does each sum of four.
FBS_HD void hamilton32x32(const int32_t a[4], const int32_t b[4], int64_t o[4]) {
#define FBS_Q(i, j) ((int64_t)a[i] * (int64_t)b[j])
  o[0] = FBS_Q(0, 0) - FBS_Q(1, 1) - FBS_Q(2, 2) - FBS_Q(3, 3);
  o[1] = FBS_Q(0, 1) + FBS_Q(1, 0) + FBS_Q(2, 3) - FBS_Q(3, 2);
  o[2] = FBS_Q(0, 2) - FBS_Q(1, 3) + FBS_Q(2, 0) + FBS_Q(3, 1);
  o[3] = FBS_Q(0, 3) + FBS_Q(1, 2) - FBS_Q(2, 1) + FBS_Q(3, 0);
#undef FBS_Q
}

// shift_wide of an i64 value (round half up, no clamp needed): s in [1, 62].
FBS_HD int64_t shift_i64(int64_t v, uint32_t s) { return (v >> s) + ((v >> (s - 1)) & 1); }

// Sign of da + db phi, exactly (RS stack/kernels.rs:1180-1215, TW 393-408).
FBS_HD bool diff_positive(int64_t da, int64_t db) {
  i128 p = (i128)da * 2 + db;
  if (db == 0) return p > 0;
  u128 b2 = (u128)uabs64(db) * uabs64(db) * 5;
  u128 pa = (u128)(p < 0 ? -p : p);
  u128 p2 = pa * pa;
  if (db > 0) return p >= 0 || b2 > p2;
  return p > 0 && p2 > b2;
}

// The icosian with the largest exact dot product with raw, the lowest index on ties
// (RS stack/kernels.rs:1420-1474 `stack_snap_select`). ico: 120 x 4 x (a, b), coordinate
// (a + b phi) / 2.
FBS_HD uint32_t snap_select(const int8_t *ico, const int32_t raw[4]) {
  uint32_t best = 0;
  int64_t best_a = 0, best_b = 0;
  for (uint32_t r = 0; r < 120; r++) {
    int64_t a = 0, b = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      a += (int64_t)raw[c] * ico[8 * r + 2 * c];
      b += (int64_t)raw[c] * ico[8 * r + 2 * c + 1];
    }
    if (r == 0 || diff_positive(a - best_a, b - best_b)) {
      best = r;
      best_a = a;
      best_b = b;
    }
  }
  return best;
}

// `stack_snap_rotation` (RS stack/kernels.rs:1530-1557, TW 435-445).
FBS_HD uint32_t snap_rotation(const int8_t *ico, const int32_t raw[4], uint64_t lambda, int64_t o[4]) {
  uint32_t r = snap_select(ico, raw);
  uint64_t lambda_phi = lambda + ((lambda * kPhiLo + (1ull << 31)) >> 32);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    int64_t sum = (int64_t)(lambda * (uint64_t)(int64_t)ico[8 * r + 2 * c] +
                            lambda_phi * (uint64_t)(int64_t)ico[8 * r + 2 * c + 1]);
    o[c] = shift(sum, 1);
  }
  return r;
}

// The unit quaternion of `stack_rotation` at Q30 before lambda, in 128-bit arithmetic (RS stack/session.rs:5165-5181):
// u_c = sign(v_c) floor(|v_c| 2^46 / s), s = isqrt((sum v^2 + eps) << 32); all zero for s = 0.
// |u_c| <= 2^30 and sum u_c^2 <= 2^60.
FBS_HD void unit_q30_wide(const int32_t raw[4], uint64_t eps, int32_t u[4]) {
  u128 square = eps;
#pragma unroll
  for (int c = 0; c < 4; c++) square += (u128)((uint64_t)((int64_t)raw[c] * raw[c]));
  uint64_t s = isqrt128(square << 32);
  Divisor dv = make_divisor(s);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint64_t a = uabs32(raw[c]);
    uint64_t m = s == 0 ? 0 : divq((u128)a << 46, dv);
    u[c] = raw[c] < 0 ? -(int32_t)m : (int32_t)m;
  }
}

// unit_q30 in 64-bit arithmetic without data-dependent branches (the kernels' form; equal to
// unit_q30_wide for every input). With X = sum v^2 + eps < 2^65 + 2^13 and Y = X 2^32:
//  1. Xn = X 4^k in [2^62, 2^64) (k = -1: Xn = floor(X / 4)); y = rsqrt_q46(Xn / 2^32) ~
//     2^62 / sqrt(Xn) (relative error within 2^-28.9, checked over every input); r = Xn/2^32
//     y / 2^30 and one Newton step on the exact remainder give r within 1 of isqrt(Xn).
//  2. s0 = r 2^j + floor((Xn - r^2) (y / 4) / 2^(61 - j)) for j = 16 - k > 0, or r >> -j, is
//     within 1 of s = isqrt(Y); the remainder Y - s0^2 is below 2^63 in magnitude, so its
//     value modulo 2^64 is exact, and one step down and one up give s.
//  3. w = recip_q63 of the top 32 bits of s normalised (relative error in [-2^-30.4, 0],
//     checked over every input; truncating s adds at most 2^-31) puts (a 2^46 w) / s within
//     0.76 of a 2^46 / s <= 2^30 + 2^14, so q0 is within 1 of the floor; one step each way on
//     the exact remainder a 2^46 - q0 s (small, exact modulo 2^64) gives q.
FBS_HD void unit_q30(const int32_t raw[4], uint64_t eps, int32_t u[4], const Seeds &sd = Seeds()) {
  uint32_t a[4];
  uint64_t xl = eps;
  uint32_t xh = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    a[c] = uabs32(raw[c]);
    const uint64_t t = xl + (uint64_t)a[c] * a[c];
    xh += t < xl;
    xl = t;
  }
  // X = 0 (all zero, eps 0) gives u = 0 by the same steps on X = 1.
  xl = (xh == 0 && xl == 0) ? 1 : xl;
  // Both normalisations are formed and one is kept by masks (one basic block, so that the
  // scheduler can interleave independent rotations).
  // z is taken mod 64 so that the unused form stays a defined shift when xl = 0 (then xh != 0
  // and the mask keeps the other form).
  const int z = clz64(xl) & 62;
  const uint64_t big = 0ull - (uint64_t)(xh != 0);
  const uint64_t xn = ((((uint64_t)xh << 62) | (xl >> 2)) & big) | ((xl << z) & ~big);
  const int j = xh ? 17 : 16 - (z >> 1);              // [-15, 17]
  // As in norm_factor_pow2, every product but the fraction's has 32-bit factors.
  const uint32_t xt = (uint32_t)(xn >> 32);
  const uint32_t y = rsqrt_q46(xt, sd.rsq_seed);
  uint64_t r = ((uint64_t)xt * y) >> 30;
  r = r > 0xffffffffull ? 0xffffffffull : r;
  const int64_t diff = (int64_t)(xn - (uint64_t)(uint32_t)r * (uint32_t)r);
  r = (uint64_t)((int64_t)r + (((int64_t)(int32_t)(diff >> 16) * (int64_t)(uint64_t)y) >> 47));
  r = r > 0xffffffffull ? 0xffffffffull : r < (1ull << 31) ? (1ull << 31) : r;
  const int64_t rem = (int64_t)(xn - (uint64_t)(uint32_t)r * (uint32_t)r);  // [-2^33, 2^34]
  const int jp = j > 0 ? j : 0, jn = j > 0 ? 0 : -j;
  const int64_t f = (rem * (int64_t)(y >> 2)) >> (61 - jp);
  const uint64_t frac = 0ull - (uint64_t)(j > 0);
  uint64_t s = (((r << jp) + (uint64_t)f) & frac) | ((r >> jn) & ~frac);
  // Y - s^2 modulo 2^64: s < 2^50, so s^2 mod 2^64 = sl^2 + (2 sh sl mod 2^32) 2^32.
  const uint32_t sl = (uint32_t)s, shi = (uint32_t)(s >> 32);
  int64_t dy = (int64_t)((xl << 32) - ((uint64_t)sl * sl + ((uint64_t)(2u * shi * sl) << 32)));
  const bool down = dy < 0;
  dy = down ? dy + (int64_t)(2 * s - 1) : dy;
  s = down ? s - 1 : s;
  const bool up = dy >= (int64_t)(2 * s + 1);
  s = up ? s + 1 : s;
  // u_c = floor(a_c 2^46 / s), s in [2^16, 2^49].
  const int zs = clz64(s);
  const uint32_t w = recip_q63((uint32_t)((s << zs) >> 32), sd.rcp_seed);  // ~ 2^95 / (s << zs)
  const int sh = 49 - zs;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint64_t q = ((uint64_t)a[c] * w) >> sh;        // below 2^31
    int64_t rq = (int64_t)(((uint64_t)a[c] << 46) - (uint64_t)(uint32_t)q * s);
    const bool qd = rq < 0;
    rq = qd ? rq + (int64_t)s : rq;
    q = qd ? q - 1 : q;
    q = rq >= (int64_t)s ? q + 1 : q;
    u[c] = raw[c] < 0 ? -(int32_t)q : (int32_t)q;
  }
}

// (lambda u) >> 30 for lambda = 2^p (p <= 31): u << (p - 30) or floor(u / 2^(30 - p)).
FBS_HD int64_t scale_pow2(int32_t u, uint32_t p) {
  return p >= 30 ? (int64_t)u << (p - 30) : (int64_t)(u >> (30 - p));
}

// `stack_rotation` for any lambda (RS stack/session.rs:5165-5181, TW 459-474).
FBS_HD void rotation(const int32_t raw[4], uint64_t lambda, uint64_t eps, int64_t o[4]) {
  int32_t u[4];
  unit_q30(raw, eps, u);
#pragma unroll
  for (int c = 0; c < 4; c++) o[c] = (int64_t)(((i128)lambda * (i128)u[c]) >> 30);
}

}  // namespace fbs

#endif
