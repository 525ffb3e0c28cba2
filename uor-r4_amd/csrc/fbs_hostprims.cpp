// fbs_hostprims.cpp - the device arithmetic of fbs_int.h compiled for the host, exported so the
// CPU tests can check it against the oracle over millions of inputs (the kernels include the
// very same header). Not part of the C ABI: a separate test library, libuor_fbs_hostprims.so.
#include "fbs_int.h"

using namespace fbs;

extern "C" {

uint64_t fbs_hp_isqrt128(uint64_t hi, uint64_t lo) { return isqrt128(((u128)hi << 64) | lo); }

uint64_t fbs_hp_div128_64(uint64_t nhi, uint64_t nlo, uint64_t d) {
  return div128_64(((u128)nhi << 64) | nlo, d);
}

// Batched forms for speed: out[i] = isqrt128(hi[i]:lo[i]).
void fbs_hp_isqrt128_many(const uint64_t *hi, const uint64_t *lo, uint64_t *out, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = isqrt128(((u128)hi[i] << 64) | lo[i]);
}
void fbs_hp_div_many(const uint64_t *nhi, const uint64_t *nlo, const uint64_t *d, uint64_t *out,
                     uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = div128_64(((u128)nhi[i] << 64) | nlo[i], d[i]);
}

uint32_t fbs_hp_rsqrt_q46(uint32_t t) { return rsqrt_q46(t); }

// out[i] = div_2p96(s[i]) = floor(2^96 / s[i]) for s[i] in [2^34, 2^64).
void fbs_hp_div_2p96_many(const uint64_t *s, uint64_t *out, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = div_2p96(s[i]);
}

// norm_factor_wave against norm_factor on n (sum, eps) pairs at 2^log2n: mismatches among the
// inputs it accepts (ok), and in *refused the inputs it sends to the fallback.
uint64_t fbs_hp_norm_factor_wave_check(const uint64_t *sum, const int64_t *eps, uint64_t n,
                                       uint32_t log2n, uint64_t *refused) {
  uint64_t bad = 0, no = 0;
  for (uint64_t i = 0; i < n; i++) {
    NormFactor a = norm_factor(sum[i], 1u << log2n, eps[i]);
    bool ok;
    NormFactor b = norm_factor_wave(sum[i], log2n, eps[i], Seeds(), ok);
    if (!ok) {
      no++;
      continue;
    }
    if (a.huge != b.huge || (!a.huge && a.r != b.r)) bad++;
  }
  *refused = no;
  return bad;
}

// norm_factor_pow2 against norm_factor on n (sum, eps) pairs at 2^log2n: mismatches.
uint64_t fbs_hp_norm_factor_check(const uint64_t *sum, const int64_t *eps, uint64_t n, uint32_t log2n) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; i++) {
    NormFactor a = norm_factor(sum[i], 1u << log2n, eps[i]);
    NormFactor b = norm_factor_pow2(sum[i], log2n, eps[i]);
    bad += a.r != b.r || a.huge != b.huge;
  }
  return bad;
}

// publish16_pair / publish64_pair / quantize_elem against the reference conversions.
uint64_t fbs_hp_publish_check(const int64_t *v, uint64_t n) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; i++) {
    int32_t p, q;
    publish64_pair(v[i], &p, &q);
    bad += p != to_exp_i32(v[i], kNormFineExp, kResidualExp);
    bad += q != to_exp_i32(sat_neg64(v[i]), kNormFineExp, kResidualExp);
    for (int32_t s = 0; s <= 49; s++) {
      int64_t y = shift(v[i], s);
      int32_t ref = (int32_t)(y > 32767 ? 32767 : y < -32767 ? -32767 : y);
      int32_t a = quantize_elem(v[i], s);
      bad += a != ref;
      int32_t e = kProductExp + s;
      publish16_pair(a, e, &p, &q);
      bad += p != to_exp_i32(a, e, kResidualExp);
      bad += q != to_exp_i32(-(int64_t)a, e, kResidualExp);
    }
  }
  return bad;
}

// hamilton32x32 then shift_i64(.., 14) against hamilton32 and shift_wide(.., 14).
uint64_t fbs_hp_hamilton_mlp_check(const int32_t *a, const int32_t *b, uint64_t n) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; i++) {
    int64_t b64[4] = {b[4 * i], b[4 * i + 1], b[4 * i + 2], b[4 * i + 3]};
    int64_t x[4];
    i128 y[4];
    hamilton32x32(a + 4 * i, b + 4 * i, x);
    hamilton32(a + 4 * i, b64, y);
    for (int k = 0; k < 4; k++) bad += shift_i64(x[k], 14) != shift_wide(y[k], 14);
  }
  return bad;
}
uint64_t fbs_hp_recip_q63(uint32_t d) { return recip_q63(d); }

int64_t fbs_hp_shift(int64_t v, int32_t s) { return shift(v, s); }
int64_t fbs_hp_grid_apply(int64_t v, int16_t code) { return grid_apply(v, code); }
int64_t fbs_hp_grid32_desc(int32_t v, int16_t code) { return grid_apply32_desc(v, grid_desc(code), code); }
int64_t fbs_hp_grid64_desc(int64_t v, int16_t code) { return grid_apply64_desc(v, grid_desc(code), code); }

// Every valid grid code against n inputs v[]: mismatches of the descriptor forms (the gains'
// grid_desc forms, and the taps' tap_desc form in both halves of a word).
uint64_t fbs_hp_grid_check(const int64_t *v, uint64_t n) {
  uint64_t bad = 0;
  for (int32_t code = -2047; code <= 2047; code++) {
    uint32_t field = (uint32_t)(code < 0 ? -code : code) >> 4;
    if (code != 0 && (field < 1 || field > 127)) continue;
    uint16_t d = grid_desc((int16_t)code);
    uint16_t t = tap_desc((int16_t)code);
    const uint32_t word0 = 0xa5a50000u | t, word1 = ((uint32_t)t << 16) | 0x5a5au;
    for (uint64_t i = 0; i < n; i++) {
      bad += grid_apply64_desc(v[i], d, (int16_t)code) != grid_apply(v[i], (int16_t)code);
      int32_t v32 = (int32_t)v[i];
      const int64_t want = grid_apply((int64_t)v32, (int16_t)code);
      bad += grid_apply32_desc(v32, d, (int16_t)code) != want;
      if (t != kGridDescSlow) bad += (tap_desc_apply(v32, word0, 0) != want) + (tap_desc_apply(v32, word1, 1) != want);
    }
  }
  return bad;
}

// rotation(raw, lambda, eps) for n quaternions: raw n*4 i32, out n*4 i64.
void fbs_hp_rotation_many(const int32_t *raw, uint64_t lambda, uint64_t eps, int64_t *out,
                          uint64_t n) {
  for (uint64_t i = 0; i < n; i++) rotation(raw + 4 * i, lambda, eps, out + 4 * i);
}

// unit_q30 (64-bit form) against unit_q30_wide on n quaternions: the number of differing lanes.
uint64_t fbs_hp_unit_check(const int32_t *raw, uint64_t eps, uint64_t n) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; i++) {
    int32_t a[4], b[4];
    unit_q30(raw + 4 * i, eps, a);
    unit_q30_wide(raw + 4 * i, eps, b);
    for (int c = 0; c < 4; c++) bad += a[c] != b[c];
  }
  return bad;
}

void fbs_hp_snap_rotation_many(const int8_t *ico, const int32_t *raw, uint64_t lambda,
                               int64_t *out, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) snap_rotation(ico, raw + 4 * i, lambda, out + 4 * i);
}

// hamilton32 vs hamilton64 on n pairs: returns the number of mismatching outputs.
uint64_t fbs_hp_hamilton_check(const int32_t *a, const int64_t *b, uint64_t n) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; i++) {
    int64_t a64[4] = {a[4 * i], a[4 * i + 1], a[4 * i + 2], a[4 * i + 3]};
    i128 x[4], y[4];
    hamilton32(a + 4 * i, b + 4 * i, x);
    hamilton64(a64, b + 4 * i, y);
    for (int k = 0; k < 4; k++) bad += x[k] != y[k];
  }
  return bad;
}

// RMSNorm on one vector, as the kernel composes it (max, pre-shift, sum, factor, apply).
void fbs_hp_rms_norm_fine(const int32_t *x, uint32_t n, int64_t eps_m, int32_t eps_e,
                          int64_t *out) {
  uint32_t max = 0;
  for (uint32_t i = 0; i < n; i++) {
    uint32_t a = uabs32(x[i]);
    if (a > max) max = a;
  }
  int32_t sh = bitlen64(max) - 24;
  if (sh < 0) sh = 0;
  uint64_t sum = 0;
  for (uint32_t i = 0; i < n; i++) {
    int64_t y = shift(x[i], sh);
    out[i] = y;
    sum += uabs64(y) * uabs64(y);
  }
  NormFactor f = norm_factor(sum, n, norm_eps(eps_m, eps_e, sh));
  if ((n & (n - 1)) == 0) {  // the kernels' form for power-of-two widths must agree
    NormFactor g = norm_factor_pow2(sum, (uint32_t)__builtin_ctz(n), norm_eps(eps_m, eps_e, sh));
    if (g.r != f.r || g.huge != f.huge) {
      for (uint32_t i = 0; i < n; i++) out[i] = INT64_MIN;
      return;
    }
  }
  for (uint32_t i = 0; i < n; i++) out[i] = norm_apply24(f, out[i]);
}

}  // extern "C"
