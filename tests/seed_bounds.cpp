// Exhaustive checks of the kernels' reciprocal and reciprocal-square-root estimates
// (uor-r4_amd/csrc/fbs_int.h), over every input they take:
//   rsqrt_q46(t), t in [2^30, 2^32): within 2^-28.9 of 2^46 / sqrt(t), in [2^30, 2^31], and equal
//     to the same Newton iteration carried in 64-bit products;
//   recip_q63(d), d in [2^31, 2^32): within [-2^-30.4, 0] of 2^63 / d, below 2^32, and equal to the
//     same iteration in 64-bit products.
// The comparisons of error use long double (a test, not served code). Prints one line per routine
// with its mismatch count and worst errors; exits nonzero on any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <thread>
#include <vector>

#include "../uor-r4_amd/csrc/fbs_int.h"

using namespace fbs;

static uint32_t rsqrt_wide(uint32_t t, const uint32_t *tab) {
  uint64_t y = tab[(t >> 23) - 128];
  for (int it = 0; it < 2; it++) {
    uint64_t y2 = (y * y) >> 32, p = ((uint64_t)t * y2) >> 28, f = ((3ull << 32) - p) >> 1;
    y = (y * f) >> 32;
    if (y > (1ull << 31)) y = 1ull << 31;
    if (y < (1ull << 30)) y = 1ull << 30;
  }
  return (uint32_t)y;
}
static uint64_t recip_wide(uint32_t d, const uint32_t *tab) {
  uint64_t w = tab[(d >> 23) - 256];
  for (int it = 0; it < 2; it++) {
    int64_t e = (int64_t)((1ull << 63) - (uint64_t)d * w);
    w = (uint64_t)((int64_t)w + (((e >> 31) * (int64_t)w) >> 32));
  }
  return w;
}

struct Acc {
  uint64_t bad = 0;
  long double lo = 0, hi = 0;
};

int main() {
  const unsigned T = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 4;
  const uint32_t *rt = rsqrt_seed_table(), *ct = recip_seed_table();
  std::vector<Acc> ra(T), ca(T);
  std::vector<std::thread> th;
  for (unsigned k = 0; k < T; k++)
    th.emplace_back([&, k] {
      Acc &a = ra[k];
      const uint64_t lo = 1ull << 30, n = 3ull << 30;
      for (uint64_t t = lo + k * (n / T); t < lo + (k + 1 == T ? n : (k + 1) * (n / T)); t++) {
        const uint32_t y = rsqrt_q46((uint32_t)t, rt);
        const long double exact = std::ldexp(1.0L, 46) / std::sqrt((long double)t);
        const long double rel = ((long double)y - exact) / exact;
        a.lo = rel < a.lo ? rel : a.lo;
        a.hi = rel > a.hi ? rel : a.hi;
        a.bad += y != rsqrt_wide((uint32_t)t, rt) || y < (1u << 30) || y > (1u << 31) ||
                 std::fabs(rel) > std::ldexp(1.0L, -28) / std::pow(2.0L, 0.9L);
      }
      Acc &c = ca[k];
      const uint64_t dlo = 1ull << 31, dn = 1ull << 31;
      for (uint64_t d = dlo + k * (dn / T); d < dlo + (k + 1 == T ? dn : (k + 1) * (dn / T)); d++) {
        const uint64_t w = recip_q63((uint32_t)d, ct);
        const long double exact = std::ldexp(1.0L, 63) / (long double)d;
        const long double rel = ((long double)w - exact) / exact;
        c.lo = rel < c.lo ? rel : c.lo;
        c.hi = rel > c.hi ? rel : c.hi;
        c.bad += w != recip_wide((uint32_t)d, ct) || w >= (1ull << 32) ||
                 rel < -std::ldexp(1.0L, -30) / std::pow(2.0L, 0.4L) || rel > 0;
      }
    });
  for (auto &t : th) t.join();
  Acc r, c;
  for (unsigned k = 0; k < T; k++) {
    r.bad += ra[k].bad, c.bad += ca[k].bad;
    r.lo = ra[k].lo < r.lo ? ra[k].lo : r.lo, r.hi = ra[k].hi > r.hi ? ra[k].hi : r.hi;
    c.lo = ca[k].lo < c.lo ? ca[k].lo : c.lo, c.hi = ca[k].hi > c.hi ? ca[k].hi : c.hi;
  }
  printf("rsqrt_q46 bad %llu rel [%.3Lf, %.3Lf] (log2 |.|)\n", (unsigned long long)r.bad,
         r.lo ? std::log2(-r.lo) : -99.0L, r.hi ? std::log2(r.hi) : -99.0L);
  printf("recip_q63 bad %llu rel [%.3Lf, %.3Lf] (log2 |.|)\n", (unsigned long long)c.bad,
         c.lo ? std::log2(-c.lo) : -99.0L, c.hi ? std::log2(c.hi) : -99.0L);
  return r.bad || c.bad;
}
