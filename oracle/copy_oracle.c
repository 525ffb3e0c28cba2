/*
 * copy_oracle.c - CPU restatement of the copy heads' Hamming read, for tests only.
 *
 * TEST INFRASTRUCTURE: the parity checker of the HIP read (uor_copy_mean_rows); only tests/
 * and bench.py's cpu_baseline leg load it. It follows CopyHeads
 * (crates/uor-r4-integer/src/stack/hamming.rs) function by function with 128-bit sums, as the
 * Rust does. Pinned by the reference's own copy-rule tests (hamming.rs:705-1058), restated in
 * tests/test_copy_oracle.py with their literal expectations.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/uor_copy.h"

typedef __int128 i128;

static uint32_t popcount64(uint64_t x) { return (uint32_t)__builtin_popcountll(x); }

static uint64_t code(const uor_copy_heads *m, uint32_t token, uint32_t h) {
  return m->codes[(size_t)token * m->copy + h];
}

/* joined (:379-385) */
static uint64_t joined(const uor_copy_heads *m, uint32_t near, uint32_t far, uint32_t h) {
  uint64_t c = code(m, near, h), first = m->pair_first[h];
  return first ? (c & first) | (code(m, far, h) & ~first) : c;
}

/* query_at (:389-391), key_at (:395-397) */
static uint64_t query_at(const uor_copy_heads *m, const uint32_t *tok, size_t t, uint32_t h) {
  return joined(m, tok[t], tok[t ? t - 1 : 0], h);
}
static uint64_t key_at(const uor_copy_heads *m, const uint32_t *tok, size_t s, uint32_t h) {
  return joined(m, tok[s - 1], tok[s >= 2 ? s - 2 : 0], h);
}

/* copy_weight_q31 (:243-252) */
static uint64_t weight_q31(int32_t margin_q16, uint32_t distance) {
  int64_t margin = margin_q16, over = margin - ((int64_t)distance << 16);
  if (over <= 0) return 0;
  uint64_t den = (uint64_t)(margin > (1 << 16) ? margin : (1 << 16));
  return ((uint64_t)over << 31) / den;
}

typedef struct {
  size_t s;
  uint32_t d;
} Pick;

static int cmp_pick(const void *a, const void *b) {
  const Pick *x = (const Pick *)a, *y = (const Pick *)b;
  if (x->d != y->d) return x->d < y->d ? -1 : 1;
  return x->s < y->s ? -1 : x->s > y->s;
}

/* choose_ruled (:356-371) with nearest (:690-701), latest_of (:584-598), longest_of (:601-615).
 * Returns the number of picks. */
static size_t choose_ruled(const uor_copy_heads *m, uint32_t h, const uint32_t *tok, size_t len,
                           int opening, Pick *out) {
  if (len == 0) return 0;
  size_t t = len - 1;
  uint32_t rule = m->rule;
  if (rule == UOR_COPY_LONGEST_AFTER_OPENING) {
    int opens = m->has_marker ? (len >= 2 && tok[t - 1] == m->marker[0] && tok[t] == m->marker[1])
                              : opening;
    rule = opens ? UOR_COPY_LATEST_EXACT : UOR_COPY_LONGEST_EXACT;
  }
  uint64_t q = query_at(m, tok, t, h);
  if (rule == UOR_COPY_MEAN) {
    size_t n = 0;
    Pick *all = (Pick *)malloc(sizeof(Pick) * (t ? t : 1));
    for (size_t s = 1; s < t; s++) all[n++] = (Pick){s, popcount64(q ^ key_at(m, tok, s, h))};
    qsort(all, n, sizeof(Pick), cmp_pick);
    if (n > m->kept) n = m->kept;
    memcpy(out, all, n * sizeof(Pick));
    free(all);
    return n;
  }
  if (rule == UOR_COPY_LATEST_EXACT || rule == UOR_COPY_LATEST_NEAREST) {
    int have = 0;
    Pick best = {0, 0};
    for (size_t s = 1; s < t; s++) {
      uint32_t d = popcount64(q ^ key_at(m, tok, s, h));
      if (rule == UOR_COPY_LATEST_EXACT && d != 0) continue;
      if (!have || d <= best.d) {
        best = (Pick){s, d};
        have = 1;
      }
    }
    if (have) out[0] = best;
    return (size_t)have;
  }
  /* longest_of with longer_at (:349-352) */
  size_t kd = m->pair_first[h] ? 2 : 1;
  long exact = -1, longer = -1;
  for (size_t s = 1; s < t; s++) {
    if (key_at(m, tok, s, h) != q) continue;
    exact = (long)s;
    if (s > kd && code(m, tok[s - 1 - kd], h) == code(m, tok[t - kd], h)) longer = (long)s;
  }
  long pick = longer >= 0 ? longer : exact;
  if (pick < 0) return 0;
  out[0] = (Pick){(size_t)pick, 0};
  return 1;
}

/* mean_by (:506-538) for one stream: returns found (0: None). */
static int mean_row(const uor_copy_heads *m, const uint32_t *tok, size_t len, int opening,
                    int64_t *out, int32_t *chosen) {
  i128 *sum = (i128 *)calloc(m->width, sizeof(i128));
  i128 *head = (i128 *)malloc(m->width * sizeof(i128));
  Pick picks[UOR_COPY_MAX_KEPT];
  i128 found = 0;
  for (uint32_t h = 0; h < m->copy; h++) {
    size_t n = choose_ruled(m, h, tok, len, opening, picks);
    if (chosen) {
      for (uint32_t k = 0; k < m->kept; k++)
        chosen[h * m->kept + k] = k < n ? (int32_t)(picks[k].s | (size_t)picks[k].d << 24) : -1;
    }
    memset(head, 0, m->width * sizeof(i128));
    i128 count = 0;
    for (size_t k = 0; k < n; k++) {
      uint64_t w = weight_q31(m->margins_q16[h], picks[k].d);
      if (w == 0) continue;
      count++;
      const int16_t *row = m->table + (size_t)tok[picks[k].s] * m->width;
      for (uint32_t c = 0; c < m->width; c++) head[c] += (i128)row[c] * (i128)w;
    }
    if (count == 0) continue;
    found++;
    for (uint32_t c = 0; c < m->width; c++) sum[c] += head[c] / count;
  }
  for (uint32_t c = 0; c < m->width; c++) out[c] = found ? (int64_t)(sum[c] / found) : 0;
  free(sum);
  free(head);
  return found > 0;
}

int copy_oracle_mean_rows(const uor_copy_heads *m, const uint32_t *tokens, const int32_t *lengths,
                          const uint8_t *opening, uint32_t rows, uint32_t stride, int64_t *out,
                          uint8_t *found, int32_t *chosen) {
  for (uint32_t r = 0; r < rows; r++)
    found[r] = (uint8_t)mean_row(m, tokens + (size_t)r * stride, (size_t)lengths[r],
                                 opening ? opening[r] : 0, out + (size_t)r * m->width,
                                 chosen ? chosen + (size_t)r * m->copy * m->kept : NULL);
  return 0;
}
