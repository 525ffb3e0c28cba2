/*
 * fbs_oracle.c - CPU restatement of UOR-R4's SpiralCore/FBS integer step (TEST INFRASTRUCTURE:
 * the parity checker and timed CPU baseline; never linked into the product).
 *
 * Reference lines are cited per function: RS = crates/uor-r4-integer/src/, TW =
 * docs/labs/d11-exporter-float-trunk/instrument/src/fbs_core.h (the reference's own C++ twin,
 * held equal to the Rust session by its tests/parity.rs). Every product is formed modulo 2^64
 * or 2^128 exactly as the reference's wrapping products; no floating point anywhere.
 */
#include "fbs_oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

enum {
  RESIDUAL_EXP = -16,   /* RS stack/kernels.rs:34 */
  PRODUCT_EXP = -32,    /* RS stack/kernels.rs:37 */
  STATE_EXP = -32,      /* RS stack/session.rs:72 */
  NORM_FINE_EXP = -24,  /* RS stack/kernels.rs:566 */
  Q12_EXP = -12,        /* RS stack/session.rs:475 */
  GRID_EXP_BIAS = 64,   /* RS stack/kernels.rs:39 */
  CELLS = 256,          /* session.rs:4069-4121: 16 x 16 root-pair cells */
  NEAREST_BLOCK = 16    /* RS stack/session.rs:4412 */
};
#define PHI_LO 2654435769ull          /* PHI_Q32 - 2^32, RS stack/mod.rs:167 */
#define ROTATION_EPSILON 4295ull      /* RS stack/session.rs:141 */
#define GATE_EPSILON 0ull             /* RS stack/session.rs:144 */

/* ------------------------------------------------------------------------------------------
 * Scalar conventions (RS stack/kernels.rs:41-135, TW 131-220). */

static int64_t sat_add64(int64_t a, int64_t b) {
  int64_t r;
  if (__builtin_add_overflow(a, b, &r)) return b > 0 ? INT64_MAX : INT64_MIN;
  return r;
}
static int64_t sat_neg64(int64_t v) { return v == INT64_MIN ? INT64_MAX : -v; }
static int32_t sat_add32(int32_t a, int32_t b) {
  int64_t s = (int64_t)a + b;
  return s > INT32_MAX ? INT32_MAX : s < INT32_MIN ? INT32_MIN : (int32_t)s;
}
static int64_t wadd64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static i128 wadd128(i128 a, i128 b) { return (i128)((u128)a + (u128)b); }
static i128 wsub128(i128 a, i128 b) { return (i128)((u128)a - (u128)b); }
static i128 wmul128(i128 a, i128 b) { return (i128)((u128)a * (u128)b); }
static uint64_t uabs64(int64_t v) { return v < 0 ? 0ull - (uint64_t)v : (uint64_t)v; }
static int bitlen64(uint64_t v) { return v ? 64 - __builtin_clzll(v) : 0; }

/* `shift`: round-half-up arithmetic shift right by s (left when negative), saturating to
 * the i64 range (RS stack/kernels.rs:41-62). */
static int64_t shift(int64_t v, int32_t s) {
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

/* `shift_wide`: round-half-up shift of an i128, clamped to i64 (RS stack/kernels.rs:64-74). */
static int64_t shift_wide(i128 v, uint32_t s) {
  i128 r = s == 0 ? v : wadd128(v, (i128)1 << (s - 1)) >> s;
  if (r > (i128)INT64_MAX) return INT64_MAX;
  if (r < (i128)INT64_MIN) return INT64_MIN;
  return (int64_t)r;
}

/* `to_exp_i32` (RS stack/kernels.rs:76-80). */
static int32_t to_exp_i32(int64_t v, int32_t from, int32_t to) {
  int64_t s = shift(v, to - from);
  return s > INT32_MAX ? INT32_MAX : s < INT32_MIN ? INT32_MIN : (int32_t)s;
}

/* `grid_apply`: v * (16 + (|c| & 15)) * 2^((|c| >> 4) - 68), rounded half up, sign of c;
 * the product (16 + m) v wraps modulo 2^64 like `scale_16_plus` (RS stack/kernels.rs:95-135). */
static int64_t grid_apply(int64_t v, int16_t code) {
  if (code == 0) return 0;
  uint32_t c = code < 0 ? (uint32_t)(-(int32_t)code) : (uint32_t)code;
  int32_t e = (int32_t)(c >> 4) - GRID_EXP_BIAS;
  int64_t scaled = (int64_t)((uint64_t)v * (uint64_t)(16 + (c & 15)));
  scaled = shift(scaled, 4 - e);
  return code < 0 ? sat_neg64(scaled) : scaled;
}

/* Floor square root of a u128, digit by digit (RS stack/kernels.rs:408-430). */
static u128 isqrt128(u128 v) {
  if (v == 0) return 0;
  int top = 127 - (int)((uint64_t)(v >> 64) ? __builtin_clzll((uint64_t)(v >> 64))
                                           : 64 + __builtin_clzll((uint64_t)v));
  u128 bit = (u128)1 << (top & ~1), rem = v, root = 0;
  while (bit) {
    if (rem >= root + bit) {
      rem -= root + bit;
      root = (root >> 1) + bit;
    } else {
      root >>= 1;
    }
    bit >>= 2;
  }
  return root;
}

/* Floor division, zero for a zero divisor (RS stack/kernels.rs:345-360). */
static u128 div128(u128 n, u128 d) { return d == 0 ? 0 : n / d; }

/* ------------------------------------------------------------------------------------------
 * Vector kernels. */

/* `stack_quantize16`: shared-exponent requantize to +-32767 (RS stack/kernels.rs:545-553,
 * TW 275-290). Returns the new exponent. */
static int32_t quantize16(const int64_t *v, uint32_t n, int32_t exp, int16_t *out) {
  uint64_t max = 0;
  for (uint32_t i = 0; i < n; i++) {
    uint64_t a = uabs64(v[i]);
    if (a > max) max = a;
  }
  int32_t s = bitlen64(max) - 15;
  if (s < 0) s = 0;
  for (uint32_t i = 0; i < n; i++) {
    int64_t y = shift(v[i], s);
    out[i] = (int16_t)(y > 32767 ? 32767 : y < -32767 ? -32767 : y);
  }
  return exp + s;
}

/* `stack_rms_norm_fine` = `rms_norm_into(.., 38, true)`: x / rms(x) at 2^-24, rounded
 * (RS stack/kernels.rs:569-620, TW 294-330). */
static void rms_norm_fine(const int32_t *x, uint32_t n, int64_t eps_m, int32_t eps_e,
                          int64_t *out) {
  uint32_t max = 0;
  for (uint32_t i = 0; i < n; i++) {
    uint32_t a = x[i] < 0 ? 0u - (uint32_t)x[i] : (uint32_t)x[i];
    if (a > max) max = a;
  }
  int32_t sh = bitlen64(max) - 24;
  if (sh < 0) sh = 0;
  uint64_t sum = 0;
  for (uint32_t i = 0; i < n; i++) {
    int64_t y = shift((int64_t)x[i], sh);
    out[i] = y;
    sum += uabs64(y) * uabs64(y);
  }
  int64_t mean = (int64_t)(sum / (n ? n : 1));
  int32_t square_exp = (RESIDUAL_EXP + sh) * 2;
  int64_t eps_int = shift(eps_m, square_exp - eps_e);
  if (eps_int < 0) eps_int = 0;
  int64_t ms = wadd64(mean, eps_int);
  if (ms < 1) ms = 1;
  u128 s = isqrt128((u128)(uint64_t)ms << 68);
  if (s < 1) s = 1;
  u128 r = div128((u128)1 << 96, s);
  for (uint32_t i = 0; i < n; i++) {
    u128 mag = r * (u128)uabs64(out[i]);
    i128 p = out[i] < 0 ? (i128)(0 - mag) : (i128)mag;
    i128 y = wadd128(p, (i128)1 << 37) >> 38;
    out[i] = y > (i128)INT64_MAX ? INT64_MAX : y < (i128)INT64_MIN ? INT64_MIN : (int64_t)y;
  }
}

/* `stack_fbs_gather`: block o of the output takes atom atoms[o]'s 8 values, lane code & 7,
 * negated (saturating) under code & 8, converted from x_exp to -16
 * (RS stack/session.rs:4033-4053, TW 337-360). */
static void gather64(const uor_fbs_map *map, const int64_t *x, int32_t x_exp, int32_t *out) {
  for (uint32_t o = 0; o < map->blocks; o++) {
    const int64_t *atom = x + 8u * map->atoms[o];
    for (uint32_t j = 0; j < 8; j++) {
      uint8_t code = map->codes[8u * o + j];
      int64_t v = atom[code & 7];
      if (code & 8) v = sat_neg64(v);
      out[8u * o + j] = to_exp_i32(v, x_exp, RESIDUAL_EXP);
    }
  }
}
static void gather16(const uor_fbs_map *map, const int16_t *x, int32_t x_exp, int32_t *out) {
  for (uint32_t o = 0; o < map->blocks; o++) {
    const int16_t *atom = x + 8u * map->atoms[o];
    for (uint32_t j = 0; j < 8; j++) {
      uint8_t code = map->codes[8u * o + j];
      int64_t v = atom[code & 7];
      if (code & 8) v = sat_neg64(v);
      out[8u * o + j] = to_exp_i32(v, x_exp, RESIDUAL_EXP);
    }
  }
}

/* Hamilton product a (x) b modulo 2^128 (RS stack/kernels.rs:998-1030, TW 363-370). */
static void hamilton(const int64_t a[4], const int64_t b[4], i128 o[4]) {
  i128 p[4][4];
  for (int i = 0; i < 4; i++)
    for (int j = 0; j < 4; j++) p[i][j] = wmul128((i128)a[i], (i128)b[j]);
  o[0] = wsub128(wsub128(wsub128(p[0][0], p[1][1]), p[2][2]), p[3][3]);
  o[1] = wsub128(wadd128(wadd128(p[0][1], p[1][0]), p[2][3]), p[3][2]);
  o[2] = wadd128(wadd128(wsub128(p[0][2], p[1][3]), p[2][0]), p[3][1]);
  o[3] = wadd128(wsub128(wadd128(p[0][3], p[1][2]), p[2][1]), p[3][0]);
}

/* Sign of da + db phi, exactly: 2(da + db phi) = P + db sqrt5 with P = 2 da + db, decided by
 * P and by P^2 against 5 db^2 (RS stack/kernels.rs:1180-1215, TW 393-408). */
static int diff_positive(int64_t da, int64_t db) {
  i128 p = (i128)da * 2 + db;
  if (db == 0) return p > 0;
  u128 b2 = (u128)uabs64(db) * uabs64(db) * 5;
  u128 p2 = (u128)(p < 0 ? -p : p) * (u128)(p < 0 ? -p : p);
  if (db > 0) return p >= 0 || b2 > p2;
  return p > 0 && p2 > b2;
}

/* The icosian root with the largest exact dot product with raw, lowest index on ties: the
 * 120-root scan that `stack_snap_select`'s candidate tables reproduce
 * (RS stack/kernels.rs:1420-1474, TW 410-430). Root coordinate c is (a + b phi)/2. */
static uint32_t snap_select(const int8_t *ico, const int32_t raw[4]) {
  uint32_t best = 0;
  int64_t best_a = 0, best_b = 0;
  for (uint32_t r = 0; r < 120; r++) {
    int64_t a = 0, b = 0;
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

/* `stack_snap_rotation`: the chosen root times lambda at Q31, lambda phi rounded at Q31
 * (RS stack/kernels.rs:1530-1557, TW 435-445). Returns the root's index (the snap trace's). */
static uint32_t snap_rotation(const int8_t *ico, const int32_t raw[4], uint64_t lambda, int64_t o[4]) {
  uint32_t r = snap_select(ico, raw);
  uint64_t lambda_phi = lambda + ((lambda * PHI_LO + (1ull << 31)) >> 32);
  for (int c = 0; c < 4; c++) {
    int64_t sum = (int64_t)(lambda * (uint64_t)(int64_t)ico[8 * r + 2 * c] +
                            lambda_phi * (uint64_t)(int64_t)ico[8 * r + 2 * c + 1]);
    o[c] = shift(sum, 1);
  }
  return r;
}

/* `stack_rotation`: lambda raw/|raw| at Q31; the unit at Q30 by floor division of magnitudes,
 * signed, then (lambda unit) >> 30 (RS stack/session.rs:5165-5181, TW 459-474). */
static void rotation(const int32_t raw[4], uint64_t lambda, uint64_t eps, int64_t o[4]) {
  u128 square = 0;
  for (int c = 0; c < 4; c++) square += (u128)((int64_t)raw[c] * raw[c]);
  u128 norm = isqrt128((square + eps) << 32);
  for (int c = 0; c < 4; c++) {
    int64_t v = raw[c];
    i128 mag = (i128)div128((u128)uabs64(v) << 46, norm);
    i128 unit = v < 0 ? -mag : mag;
    o[c] = (int64_t)(wmul128((i128)lambda, unit) >> 30);
  }
}

/* A quaternion as the artifact serves it, returning its snap trace byte (TW 476-502, claude-134):
 * the chosen root's index, or 255 where none was chosen (served unsnapped) or the raw
 * quaternion is zero (its tie selects root 0). */
#define TRACE_NONE 255u
static uint32_t serve_rotation(const int8_t *ico, uint32_t raw_form, const int32_t raw[4],
                               uint64_t lambda, uint64_t eps, int64_t o[4]) {
  uint32_t chosen = TRACE_NONE;
  if (raw_form)
    rotation(raw, lambda, eps, o);
  else
    chosen = snap_rotation(ico, raw, lambda, o);
  return (raw[0] | raw[1] | raw[2] | raw[3]) == 0 ? TRACE_NONE : chosen;
}

/* ------------------------------------------------------------------------------------------
 * The resolved model: the reference image plus the extension's choices. */

typedef struct {
  const uor_fbs_model *m;
  uint32_t d, mlp, lanes, g, L, W, D, P, head;
  int reference_writer; /* 256 root-pair cells, t mod 256, no keys: session.rs:4069-4121 */
  const int16_t *const *wide_taps;
  const int32_t *keys;
  const uint32_t *offsets, *members;
  const int8_t *t8;
  uint32_t t8_shift;
  struct Ham *ham; /* the Hamming reads, or NULL */
} O;

struct Ham;
static struct Ham *ham_build(const O *o, const uor_fbs_hamming *hm);
static void ham_free(struct Ham *h);

static void resolve(O *o, const uor_fbs_model *m, const uor_fbs_ext *e) {
  memset(o, 0, sizeof *o);
  o->m = m;
  o->d = m->width;
  o->mlp = m->mlp;
  o->lanes = m->width / 4;
  o->g = o->lanes + m->width;
  o->L = m->layer_count;
  o->W = (e && e->window) ? e->window : 3;
  o->D = (e && e->drawers) ? e->drawers : CELLS;
  o->P = (e && e->probes) ? e->probes : m->kept;
  o->head = e ? e->head : 0;
  o->wide_taps = e ? e->wide_taps : NULL;
  o->keys = e ? e->drawer_keys : NULL;
  o->offsets = e ? e->drawer_offsets : NULL;
  o->members = e ? e->drawer_members : NULL;
  o->t8 = e ? e->table_i8 : NULL;
  o->t8_shift = e ? e->table_shift : 0;
  o->reference_writer = o->D == CELLS && !o->keys && !o->offsets;
  o->ham = (e && e->hamming) ? ham_build(o, e->hamming) : NULL;
}

static void unresolve(O *o) {
  ham_free(o->ham);
  o->ham = NULL;
}

/* Writer-table value of token t, channel i, at Q12 (the i16 table, or code << shift). */
static int32_t row_value(const O *o, uint32_t t, uint32_t i) {
  uint64_t at = (uint64_t)t * o->d + i;
  if (o->t8) return (int32_t)((uint32_t)(int32_t)o->t8[at] << o->t8_shift);
  return o->m->writer_table[at];
}

static int16_t tap(const O *o, uint32_t l, uint32_t s, uint32_t i) {
  if (o->wide_taps) return o->wide_taps[l][(uint64_t)s * o->d + i];
  return o->m->layers[l].taps[(uint64_t)s * o->d + i];
}

static uint64_t row_l1(const O *o, const int32_t *q, uint32_t t) {
  uint64_t sum = 0;
  for (uint32_t i = 0; i < o->d; i++) {
    int64_t diff = (int64_t)q[i] - row_value(o, t, i);
    sum += (uint64_t)(diff < 0 ? -diff : diff);
  }
  return sum;
}

/* The native vector writer exactly as the reference states it (RS stack/session.rs:4069-4121,
 * TW 580-623): ports, 256 cells, kept rounds of first-max, candidates kept + 256 j. */
static uint32_t writer_reference(const O *o, const int32_t *q, uint32_t *kept, uint64_t *cand) {
  const uor_fbs_model *m = o->m;
  int64_t pa[16], pb[16], cells[CELLS];
  for (int r = 0; r < 16; r++) {
    int64_t sa = 0, sb = 0;
    for (int i = 0; i < 8; i++) {
      int64_t da = (int64_t)q[i] - m->roots_q12[8 * r + i];
      int64_t db = (int64_t)q[o->d - 8 + i] - m->roots_q12[8 * r + i];
      sa += da < 0 ? -da : da;
      sb += db < 0 ? -db : db;
    }
    pa[r] = -sa;
    pb[r] = -sb;
  }
  for (int c = 0; c < CELLS; c++) cells[c] = wadd64(pa[c >> 4], pb[c & 15]);
  for (uint32_t k = 0; k < o->P; k++) {
    int best = 0;
    for (int c = 1; c < CELLS; c++)
      if (cells[c] > cells[best]) best = c;
    kept[k] = (uint32_t)best;
    cells[best] = INT64_MIN;
  }
  uint32_t token = UINT32_MAX;
  int64_t token_score = INT64_MIN;
  for (uint32_t k = 0; k < o->P; k++) {
    for (uint32_t t = kept[k]; t < m->vocab; t += CELLS) {
      int64_t score = -(int64_t)row_l1(o, q, t);
      if (cand) (*cand)++;
      if (score > token_score || (score == token_score && t < token)) {
        token = t;
        token_score = score;
      }
    }
  }
  return token;
}

/* The writer over D keyed drawers (extension; reduces to writer_reference for the 256
 * root-pair keys and t mod 256 membership): drawer score -(L1(q[0..8], keyA) +
 * L1(q[d-8..d], keyB)); P rounds of first-max (ties to the lower drawer); the lexicographic
 * minimum (L1, id) over the kept drawers' members. */
static uint32_t writer_drawers(const O *o, const int32_t *q, uint32_t *kept, uint64_t *cand) {
  const uor_fbs_model *m = o->m;
  int64_t *score = (int64_t *)malloc(sizeof(int64_t) * o->D);
  for (uint32_t c = 0; c < o->D; c++) {
    int32_t ka[8], kb[8];
    for (int i = 0; i < 8; i++) {
      if (o->keys) {
        ka[i] = o->keys[16ull * c + i];
        kb[i] = o->keys[16ull * c + 8 + i];
      } else { /* root pairs: only valid for D = 256 (checked by the caller's image) */
        ka[i] = m->roots_q12[8 * (c >> 4) + i];
        kb[i] = m->roots_q12[8 * (c & 15) + i];
      }
    }
    int64_t s = 0;
    for (int i = 0; i < 8; i++) {
      int64_t da = (int64_t)q[i] - ka[i], db = (int64_t)q[o->d - 8 + i] - kb[i];
      s += (da < 0 ? -da : da) + (db < 0 ? -db : db);
    }
    score[c] = -s;
  }
  for (uint32_t k = 0; k < o->P; k++) {
    uint32_t best = 0;
    for (uint32_t c = 1; c < o->D; c++)
      if (score[c] > score[best]) best = c;
    kept[k] = best;
    score[best] = INT64_MIN;
  }
  free(score);
  uint32_t token = UINT32_MAX;
  uint64_t best_l1 = UINT64_MAX;
  for (uint32_t k = 0; k < o->P; k++) {
    uint32_t c = kept[k];
    if (o->offsets) {
      for (uint32_t j = o->offsets[c]; j < o->offsets[c + 1]; j++) {
        uint32_t t = o->members[j];
        uint64_t l1 = row_l1(o, q, t);
        if (cand) (*cand)++;
        if (l1 < best_l1 || (l1 == best_l1 && t < token)) {
          token = t;
          best_l1 = l1;
        }
      }
    } else {
      for (uint32_t t = c; t < m->vocab; t += o->D) {
        uint64_t l1 = row_l1(o, q, t);
        if (cand) (*cand)++;
        if (l1 < best_l1 || (l1 == best_l1 && t < token)) {
          token = t;
          best_l1 = l1;
        }
      }
    }
  }
  return token;
}

/* `stack_whole_table_nearest`: L1 argmin over every row, a row left as soon as its partial
 * sum passes the best after a 16-value block, ties to the smaller id
 * (RS stack/session.rs:4418-4445). */
static uint32_t writer_nearest(const O *o, const int32_t *q, uint64_t *cand) {
  uint32_t token = UINT32_MAX;
  int64_t best = INT64_MAX;
  for (uint32_t t = 0; t < o->m->vocab; t++) {
    int64_t sum = 0;
    int whole = 1;
    for (uint32_t i0 = 0; i0 < o->d; i0 += NEAREST_BLOCK) {
      for (uint32_t i = i0; i < i0 + NEAREST_BLOCK && i < o->d; i++) {
        int64_t diff = (int64_t)q[i] - row_value(o, t, i);
        sum += diff < 0 ? -diff : diff;
      }
      if (sum > best) {
        whole = 0;
        break;
      }
    }
    if (cand) (*cand)++;
    if (whole && sum < best) {
      token = t;
      best = sum;
    }
  }
  return token;
}

static uint32_t writer(const O *o, const int32_t *q, uint32_t *kept, uint64_t *cand) {
  if (o->head == 1) {
    memset(kept, 0, sizeof(uint32_t) * o->P); /* session.rs:4372: no cells kept */
    return writer_nearest(o, q, cand);
  }
  return o->reference_writer ? writer_reference(o, q, kept, cand) : writer_drawers(o, q, kept, cand);
}


/* ------------------------------------------------------------------------------------------
 * The Hamming reads of a lut-stack/6 stack (RS stack/hamming.rs): at the stream read after
 * `depth` layers the residual becomes x + w_c (.) c + w_y (.) y, on the readout the final norm's
 * output n + w_c (.) (c - n) + w_y (.) y (or (y - n) for a read that asks), c the copy heads'
 * mean and y the type heads' (ServedHamming::stream/readout :1831-1913, stream_sum :1918-1925,
 * readout_sum :1933-1940, readout_ask_sum :1946-1953). */

#define COPY_MEAN_EXP (-43)     /* RS stack/hamming.rs:175 */
#define HAMMING_WEIGHT_EXP (-24) /* RS stack/format.rs:59 */
#define TYPE_MEAN_SHIFT 31u     /* RS stack/hamming.rs:1364 */
#define STREAM_SHIFT ((uint32_t)(RESIDUAL_EXP - HAMMING_WEIGHT_EXP - COPY_MEAN_EXP))
#define NORM_RAISE ((uint32_t)(NORM_FINE_EXP - COPY_MEAN_EXP))
#define READOUT_SHIFT ((uint32_t)(NORM_FINE_EXP - HAMMING_WEIGHT_EXP - COPY_MEAN_EXP))
#define STREAM_COPY_RAISE ((uint32_t)(COPY_MEAN_EXP - RESIDUAL_EXP + (int)TYPE_MEAN_SHIFT))
#define READOUT_TYPE_DROP ((uint32_t)(COPY_MEAN_EXP - NORM_FINE_EXP + (int)TYPE_MEAN_SHIFT))

typedef struct {
  const uor_fbs_hamming_read *r;
  int64_t *qu, *ku, *vu; /* width/4 unit quaternions at Q31 (`units`, :541-548) */
  int typed;             /* type heads served: some w_y is not zero (:1574-1599) */
  int asks;              /* its type heads ask from the question table (:1147) */
  int slot;              /* its payload cache, for a typed read that does not ask; else -1 */
  uint64_t *codes;       /* vocab * heads: every entry's code through the key rotation
                            (`vocab_codes` :566-582), copy heads first, then type heads */
  uint32_t heads;
} HR;

typedef struct Ham {
  uint32_t heads, copy, hw, kept, rule, has_marker, marker[2], n, slots;
  uint64_t *pair;  /* per copy head: the first half's bits under copy key 2, else 0 */
  HR *reads;
  int *at;         /* layers + 1: the read at each depth, -1 none */
  const uor_fbs_place *place; /* the readout read's place read, or NULL */
} Ham;

typedef struct {
  size_t s;
  uint32_t d;
} Pick;

/* The Hamming trace and Q5's forced replay at one step (session.rs:2361-2370, 2438-2520;
 * hamming.rs:1378-1421, 1686-1740, 1787-1814): the sequence's forced codes and this position's
 * trace record. NULL members: nothing forced, nothing recorded. */
typedef struct {
  const uint64_t *codes;  /* [len][reads][heads][2]: the forced query and key of each head */
  const uint8_t *mask;    /* [len][reads][heads]: bit 0 the query is forced, bit 1 the key */
  uint32_t reads, heads;
  uint8_t *rec;           /* this position's record (fbs_oracle_decision_stride bytes) */
  size_t reads_at;        /* the reads' part of the record */
  const uint8_t *buckets; /* this position's forced rate buckets [L][lanes], 255: none */
  int decisions;          /* record the rate buckets */
} Tr;

static size_t tr_head_bytes(uint32_t kept) { return (20 + 4 * (size_t)kept + 7) & ~(size_t)7; }

static int tr_forced(const Tr *tr, uint32_t ri, uint32_t head, size_t step, int role, uint64_t *code) {
  if (!tr || !tr->mask) return 0;
  size_t at = ((size_t)step * tr->reads + ri) * tr->heads + head;
  if (!(tr->mask[at] & (1u << role))) return 0;
  *code = tr->codes[2 * at + (size_t)role];
  return 1;
}

/* Head record: query u64, key u64, the kept count u32 and the kept positions u32 (the order
 * `nearest` and the rules keep them). */
static void tr_record(const Tr *tr, size_t off, uint64_t query, uint64_t key, const Pick *picks,
                      size_t n) {
  uint8_t *p = tr->rec + off;
  memcpy(p, &query, 8);
  memcpy(p + 8, &key, 8);
  uint32_t c = (uint32_t)n;
  memcpy(p + 16, &c, 4);
  for (size_t k = 0; k < n; k++) {
    uint32_t v = (uint32_t)picks[k].s;
    memcpy(p + 20 + 4 * k, &v, 4);
  }
}

static i128 shl128(i128 v, uint32_t s) { return (i128)((u128)v << s); }

/* `round_shift` (:1353-1360): v / 2^s rounded half away from zero. */
static i128 round_shift(i128 v, uint32_t s) {
  i128 half = (i128)1 << (s - 1);
  return v >= 0 ? (v + half) >> s : -((half - v) >> s);
}

static int64_t clamp64(i128 v) {
  return v > (i128)INT64_MAX ? INT64_MAX : v < (i128)INT64_MIN ? INT64_MIN : (int64_t)v;
}

/* `stream_sum` (:1918-1925). */
static int32_t stream_sum(int32_t x, int32_t w_c, i128 c, int32_t w_y, i128 y) {
  uint32_t sh = STREAM_SHIFT + STREAM_COPY_RAISE;
  i128 sum = shl128(x, sh) + shl128(wmul128(w_c, c), STREAM_COPY_RAISE) + wmul128(w_y, y);
  i128 r = round_shift(sum, sh);
  return r > INT32_MAX ? INT32_MAX : r < INT32_MIN ? INT32_MIN : (int32_t)r;
}

/* `readout_sum` (:1933-1940): c present where a copy head matched. */
static int64_t readout_sum(int64_t n, int32_t w_c, const i128 *c, int32_t w_y, i128 y) {
  i128 moved = c ? wmul128(w_c, *c - shl128(n, NORM_RAISE)) : 0;
  i128 typed = round_shift(wmul128(w_y, y), READOUT_TYPE_DROP);
  return clamp64(round_shift(shl128(n, READOUT_SHIFT) + moved + typed, READOUT_SHIFT));
}

/* `readout_ask_sum` (:1946-1953): each move present where a head of its kind matched. */
static int64_t readout_ask_sum(int64_t n, int32_t w_c, const i128 *c, int32_t w_y, const i128 *y) {
  i128 raised = shl128(n, NORM_RAISE);
  i128 copied = c ? wmul128(w_c, *c - raised) : 0;
  i128 asked = y ? wmul128(w_y, *y - raised) : 0;
  return clamp64(round_shift(shl128(n, READOUT_SHIFT) + copied + asked, READOUT_SHIFT));
}

/* `copy_weight_q31` (:243-252). */
static uint64_t ham_weight(int32_t margin_q16, uint32_t distance) {
  int64_t margin = margin_q16, over = margin - ((int64_t)distance << 16);
  if (over <= 0) return 0;
  return ((uint64_t)over << 31) / (uint64_t)(margin > (1 << 16) ? margin : (1 << 16));
}

/* `head_code` (:550-564): head h's sign word of `point` through `units`, the unit on the left. */
static uint64_t head_code(const int64_t *units, const int64_t *point, uint32_t h, uint32_t hw) {
  uint64_t word = 0;
  for (uint32_t c = 0; c < hw; c += 4) {
    uint32_t at = h * hw + c;
    i128 o[4];
    hamilton(units + at, point + at, o);
    for (int i = 0; i < 4; i++)
      if (o[i] >= 0) word |= 1ull << (c + i);
  }
  return word;
}

static int cmp_pick(const void *a, const void *b) {
  const Pick *x = (const Pick *)a, *y = (const Pick *)b;
  if (x->d != y->d) return x->d < y->d ? -1 : 1;
  return x->s < y->s ? -1 : x->s > y->s;
}

static uint64_t ham_code(const HR *r, uint32_t token, uint32_t head) {
  return r->codes[(size_t)token * r->heads + head];
}
/* `joined` (:379-385), `query_at` (:389-391), `key_at` (:395-397). */
static uint64_t ham_joined(const Ham *h, const HR *r, uint32_t near, uint32_t far, uint32_t head) {
  uint64_t c = ham_code(r, near, head), first = h->pair[head];
  return first ? (c & first) | (ham_code(r, far, head) & ~first) : c;
}

/* `nearest` (:690-701): the min(kept, t - 1) positions 1 <= s < t nearest by popcount, ties to
 * the earlier position; `key[s]` is position s's code. */
static size_t ham_nearest(uint64_t query, size_t t, uint32_t kept, const uint64_t *key, Pick *out) {
  if (t < 2) return 0;
  Pick *all = malloc(sizeof(Pick) * t);
  size_t n = 0;
  for (size_t s = 1; s < t; s++) all[n++] = (Pick){s, (uint32_t)__builtin_popcountll(query ^ key[s])};
  qsort(all, n, sizeof(Pick), cmp_pick);
  if (n > kept) n = kept;
  memcpy(out, all, n * sizeof(Pick));
  free(all);
  return n;
}

/* Copy head `head`'s positions at the last row of tok[0..=t] under the rule in force
 * (`choose_ruled` :356-371, `latest_of` :584-598, `longest_of` :601-615, `longer_at` :349-352);
 * `opening` is the caller's reply mark (this build passes none). */
static size_t ham_copy_choose(const Ham *h, const HR *r, uint32_t head, const uint32_t *tok,
                              size_t t, int opening, uint64_t *key, Pick *out, const Tr *tr,
                              uint32_t ri, uint64_t *query_used) {
  uint32_t rule = h->rule;
  if (rule == UOR_FBS_COPY_LONGEST_AFTER_OPENING) {
    int opens = h->has_marker ? (t >= 1 && tok[t - 1] == h->marker[0] && tok[t] == h->marker[1])
                              : opening;
    rule = opens ? UOR_FBS_COPY_LATEST_EXACT : UOR_FBS_COPY_LONGEST_EXACT;
  }
  /* `choose_forced` (:450-466): a forced query replaces the row's, a forced key candidate s's. */
  uint64_t q = ham_joined(h, r, tok[t], tok[t ? t - 1 : 0], head);
  tr_forced(tr, ri, head, t, 0, &q);
  *query_used = q;
  for (size_t s = 1; s < t; s++) {
    key[s] = ham_joined(h, r, tok[s - 1], tok[s >= 2 ? s - 2 : 0], head);
    tr_forced(tr, ri, head, s, 1, &key[s]);
  }
  if (rule == UOR_FBS_COPY_MEAN) return ham_nearest(q, t, h->kept, key, out);
  if (rule == UOR_FBS_COPY_LATEST_EXACT || rule == UOR_FBS_COPY_LATEST_NEAREST) {
    size_t best = 0;
    uint32_t least = 0;
    for (size_t s = 1; s < t; s++) {
      uint32_t d = (uint32_t)__builtin_popcountll(q ^ key[s]);
      if (rule == UOR_FBS_COPY_LATEST_EXACT && d != 0) continue;
      if (!best || d <= least) {
        best = s;
        least = d;
      }
    }
    if (!best) return 0;
    out[0] = (Pick){best, least};
    return 1;
  }
  /* longest exact: the latest exact match whose token before the key also agrees by the head's
   * code, else the latest exact match. */
  size_t kd = h->pair[head] ? 2 : 1, ex = 0, lg = 0;
  for (size_t s = 1; s < t; s++) {
    if (key[s] != q) continue;
    ex = s;
    if (s > kd && ham_code(r, tok[s - 1 - kd], head) == ham_code(r, tok[t - kd], head)) lg = s;
  }
  size_t pick = lg ? lg : ex;
  if (!pick) return 0;
  out[0] = (Pick){pick, 0};
  return 1;
}

/* One head's weighted sum over its picks into acc (width), `point(s, i)` the value brought back
 * from position s; returns the count of positions inside the margin (`mean_by` :506-538,
 * TypeHeads::mean_by :1282-1334). */
typedef struct {
  const O *o;
  const uint32_t *tok;
  const int64_t *payloads; /* NULL: table points of each position's own token */
} Brought;

static i128 brought(const Brought *b, size_t s, uint32_t i) {
  if (b->payloads) return b->payloads[s * b->o->d + i];
  return row_value(b->o, b->tok[s], i);
}

static uint32_t ham_head_sum(const Brought *b, const Pick *picks, size_t n, int32_t margin,
                             i128 *acc) {
  uint32_t d = b->o->d, count = 0;
  for (uint32_t i = 0; i < d; i++) acc[i] = 0;
  for (size_t k = 0; k < n; k++) {
    uint64_t w = ham_weight(margin, picks[k].d);
    if (!w) continue;
    count++;
    for (uint32_t i = 0; i < d; i++) acc[i] += brought(b, picks[k].s, i) * (i128)w;
  }
  return count;
}

/* The copy heads' mean at row t (`CopyHeads::mean_at` :482-504): returns 0 when no head found a
 * position inside its margin. */
static int ham_copy_mean(const O *o, const HR *r, const uint32_t *tok, size_t t, i128 *c,
                         const Tr *tr, uint32_t ri, size_t rec_at) {
  const Ham *h = o->ham;
  uint32_t d = o->d, found = 0;
  i128 *head = malloc(sizeof(i128) * d);
  uint64_t *key = malloc(sizeof(uint64_t) * (t + 2));
  Pick *picks = malloc(sizeof(Pick) * (h->kept + 1));
  for (uint32_t i = 0; i < d; i++) c[i] = 0;
  Brought b = {o, tok, NULL};
  for (uint32_t k = 0; k < h->copy; k++) {
    uint64_t q;
    size_t n = ham_copy_choose(h, r, k, tok, t, 0, key, picks, tr, ri, &q);
    if (tr && tr->rec) {
      /* The record (`record` :1787-1814): the key at t is x_{t-1}'s code (0 at row 0). */
      uint64_t kt = 0;
      if (t > 0) {
        kt = ham_joined(h, r, tok[t - 1], tok[t >= 2 ? t - 2 : 0], k);
        tr_forced(tr, ri, k, t, 1, &kt);
      }
      tr_record(tr, rec_at + k * tr_head_bytes(h->kept), q, kt, picks, n);
    }
    uint32_t count = ham_head_sum(&b, picks, n, r->r->margin[k], head);
    if (!count) continue;
    found++;
    for (uint32_t i = 0; i < d; i++) c[i] += head[i] / (i128)count;
  }
  if (found)
    for (uint32_t i = 0; i < d; i++) c[i] /= (i128)found;
  free(head);
  free(key);
  free(picks);
  return found > 0;
}

/* `TypeHeads::asked_point` (:1161-1181): (table + a)[x_t] at Q28 plus the carried rows. */
static void ham_asked_point(const O *o, const HR *r, const uint32_t *tok, size_t t, int64_t *p) {
  uint32_t d = o->d;
  const int16_t *a = r->r->ask;
  for (uint32_t i = 0; i < d; i++)
    p[i] = (int64_t)(row_value(o, tok[t], i) + a[(size_t)tok[t] * d + i]) * 65536;
  if (r->r->carry && r->r->carry_rows) {
    size_t reach = r->r->carry_rows < t ? r->r->carry_rows : t;
    for (size_t s = 1; s <= reach; s++) {
      uint32_t v = tok[t - s];
      int64_t gain = r->r->carry[v];
      for (uint32_t i = 0; i < d; i++)
        p[i] += gain * (int64_t)(row_value(o, v, i) + a[(size_t)v * d + i]);
    }
  }
}

/* The type heads' mean at row t (`ServedHamming::type_mean` :1750-1783, TypeHeads::mean and
 * ask_mean :1254-1280): for a read that asks, the question codes of the asked point through the
 * key rotation and the kept tokens' table points (at COPY_MEAN_EXP); otherwise `point`'s payload
 * is kept at row t first, the query codes are `point`'s through the query rotation and the kept
 * positions' payloads come back (at the point's exponent minus 31). */
static int ham_type_mean(const O *o, const HR *r, const uint32_t *tok, size_t t,
                         const int64_t *point, int64_t *payloads, i128 *y, const Tr *tr,
                         size_t rec_at) {
  const Ham *h = o->ham;
  uint32_t d = o->d, found = 0, types = h->heads - h->copy;
  const uint32_t ri = (uint32_t)(r - h->reads);
  int64_t *asked = NULL;
  if (r->asks) {
    asked = malloc(sizeof(int64_t) * d);
    ham_asked_point(o, r, tok, t, asked);
  } else {
    for (uint32_t q = 0; q < d / 4; q++) {
      i128 rot[4];
      hamilton(r->vu + 4 * q, point + 4 * q, rot);
      for (int k = 0; k < 4; k++) payloads[t * d + 4 * q + k] = clamp64(round_shift(rot[k], 31));
    }
  }
  i128 *head = malloc(sizeof(i128) * d);
  uint64_t *key = malloc(sizeof(uint64_t) * (t + 2));
  Pick *picks = malloc(sizeof(Pick) * (h->kept + 1));
  for (uint32_t i = 0; i < d; i++) y[i] = 0;
  Brought b = {o, tok, r->asks ? NULL : payloads};
  for (uint32_t j = 0; j < types; j++) {
    uint64_t query = r->asks ? head_code(r->ku, asked, h->copy + j, h->hw)
                             : head_code(r->qu, point, h->copy + j, h->hw);
    tr_forced(tr, ri, h->copy + j, t, 0, &query);
    for (size_t s = 1; s < t; s++) {
      key[s] = ham_code(r, tok[s - 1], h->copy + j);
      tr_forced(tr, ri, h->copy + j, s, 1, &key[s]);
    }
    size_t n = ham_nearest(query, t, h->kept, key, picks);
    if (tr && tr->rec) {
      uint64_t kt = 0;
      if (t > 0) {
        kt = ham_code(r, tok[t - 1], h->copy + j);
        tr_forced(tr, ri, h->copy + j, t, 1, &kt);
      }
      tr_record(tr, rec_at + (h->copy + j) * tr_head_bytes(h->kept), query, kt, picks, n);
    }
    uint32_t count = ham_head_sum(&b, picks, n, r->r->margin[h->copy + j], head);
    if (!count) continue;
    found++;
    for (uint32_t i = 0; i < d; i++) y[i] += head[i] / (i128)count;
  }
  if (found)
    for (uint32_t i = 0; i < d; i++) y[i] /= (i128)found;
  free(asked);
  free(head);
  free(key);
  free(picks);
  return found > 0;
}

/* The stream read after `depth` layers on the residual x (ServedHamming::stream :1831-1866). */
/* The record offset of read ri's heads: after the buckets, each earlier read's served heads. */
static size_t tr_read_at(const O *o, const Tr *tr, uint32_t ri) {
  const Ham *h = o->ham;
  size_t at = tr->reads_at;
  for (uint32_t i = 0; i < ri; i++)
    at += (h->copy + (h->reads[i].typed ? h->heads - h->copy : 0)) * tr_head_bytes(h->kept);
  return at;
}

static void ham_stream(const O *o, uint32_t depth, const uint32_t *tok, size_t t, int32_t *x,
                       int64_t *payloads, const Tr *tr) {
  const Ham *h = o->ham;
  if (depth == o->L || h->at[depth] < 0) return;
  const uint32_t ri = (uint32_t)h->at[depth];
  const HR *r = &h->reads[ri];
  const size_t rec_at = tr && tr->rec ? tr_read_at(o, tr, ri) : 0;
  uint32_t d = o->d;
  i128 *c = malloc(sizeof(i128) * d), *y = malloc(sizeof(i128) * d);
  int has_c = h->copy ? ham_copy_mean(o, r, tok, t, c, tr, ri, rec_at) : 0, has_y = 0;
  if (r->typed) {
    int64_t *point = malloc(sizeof(int64_t) * d);
    for (uint32_t i = 0; i < d; i++) point[i] = x[i];
    has_y = ham_type_mean(o, r, tok, t, point,
                          r->slot >= 0 ? payloads + (size_t)r->slot * o->m->context * d : NULL, y,
                          tr, rec_at);
    free(point);
    if (has_y && r->asks)
      for (uint32_t i = 0; i < d; i++) y[i] = shl128(y[i], STREAM_COPY_RAISE);
  }
  if (has_c || has_y)
    for (uint32_t i = 0; i < d; i++)
      x[i] = stream_sum(x[i], r->r->weight[i], has_c ? c[i] : 0, r->r->weight[d + i], has_y ? y[i] : 0);
  free(c);
  free(y);
}

/* The readout read on the final norm's output n (ServedHamming::readout :1883-1913). At a row the
 * place read opens, `offer` (>= 0) is the place: the table's point of the token there, at
 * 2^COPY_MEAN_EXP (a Q12 point at a Q31 weight of one), is the copy term in place of the copy
 * heads' mean (:1895-1899). */
static void ham_readout(const O *o, const uint32_t *tok, size_t t, int64_t *n, int64_t *payloads,
                        long offer, const Tr *tr) {
  const Ham *h = o->ham;
  if (h->at[o->L] < 0) return;
  const uint32_t ri = (uint32_t)h->at[o->L];
  const HR *r = &h->reads[ri];
  const size_t rec_at = tr && tr->rec ? tr_read_at(o, tr, ri) : 0;
  uint32_t d = o->d;
  i128 *c = malloc(sizeof(i128) * d), *y = malloc(sizeof(i128) * d);
  int has_c = 0, has_y = 0;
  if (offer >= 0) {
    /* The trace records the copy heads' choices at an open row too (`record` runs first). */
    if (tr && tr->rec && h->copy) ham_copy_mean(o, r, tok, t, c, tr, ri, rec_at);
    for (uint32_t i = 0; i < d; i++) c[i] = shl128((i128)row_value(o, tok[offer], i), 31);
    has_c = 1;
  } else if (h->copy) {
    has_c = ham_copy_mean(o, r, tok, t, c, tr, ri, rec_at);
  }
  if (r->typed)
    has_y = ham_type_mean(o, r, tok, t, n,
                          r->slot >= 0 ? payloads + (size_t)r->slot * o->m->context * d : NULL, y,
                          tr, rec_at);
  if (has_c || has_y)
    for (uint32_t i = 0; i < d; i++) {
      const i128 *ci = has_c ? &c[i] : NULL;
      n[i] = r->asks ? readout_ask_sum(n[i], r->r->weight[i], ci, r->r->weight[d + i], has_y ? &y[i] : NULL)
                     : readout_sum(n[i], r->r->weight[i], ci, r->r->weight[d + i], has_y ? y[i] : 0);
    }
  free(c);
  free(y);
}

/* Builds the served reads (ServedHamming::new :1571-1609 with CopyHeads::new :287-313 and
 * TypeHeads::new :1130-1145): units of the three rotations, every vocabulary entry's key code
 * per head, the copy heads' pair masks and rule. */
static Ham *ham_build(const O *o, const uor_fbs_hamming *hm) {
  Ham *h = calloc(1, sizeof(Ham));
  uint32_t d = o->d, V = o->m->vocab;
  h->heads = hm->heads;
  h->copy = hm->heads / 2;
  h->hw = d / hm->heads;
  h->kept = hm->kept;
  h->n = hm->read_count;
  h->has_marker = hm->copy_longest != 0;
  h->marker[0] = hm->marker[0];
  h->marker[1] = hm->marker[1];
  h->rule = hm->rule != UOR_FBS_COPY_ARTIFACT ? hm->rule
            : hm->copy_longest          ? UOR_FBS_COPY_LONGEST_AFTER_OPENING
            : hm->copy_latest           ? UOR_FBS_COPY_LATEST_EXACT
                                        : UOR_FBS_COPY_MEAN;
  h->pair = calloc(h->copy ? h->copy : 1, sizeof(uint64_t));
  for (uint32_t k = 0; k < h->copy; k++) {
    uint32_t key = hm->copy_keys ? hm->copy_keys[k] : hm->copy_key;
    h->pair[k] = key == 2 ? (1ull << (h->hw / 2)) - 1 : 0;
  }
  h->at = malloc(sizeof(int) * (o->L + 1));
  for (uint32_t l = 0; l <= o->L; l++) h->at[l] = -1;
  h->place = hm->place;
  h->reads = calloc(h->n, sizeof(HR));
  for (uint32_t i = 0; i < h->n; i++) {
    HR *r = &h->reads[i];
    r->r = &hm->reads[i];
    h->at[r->r->depth] = (int)i;
    int64_t **u[3] = {&r->qu, &r->ku, &r->vu};
    const int32_t *raw[3] = {r->r->query_rotation, r->r->key_rotation, r->r->value_rotation};
    for (int k = 0; k < 3; k++) {
      *u[k] = malloc(sizeof(int64_t) * d);
      for (uint32_t q = 0; q < d / 4; q++) rotation(raw[k] + 4 * q, 1ull << 31, GATE_EPSILON, *u[k] + 4 * q);
    }
    r->typed = 0;
    for (uint32_t c = 0; c < d; c++) r->typed |= r->r->weight[d + c] != 0;
    r->asks = r->r->ask != NULL;
    /* The place read's ask heads find a place and bring nothing back: the readout read then
     * serves no type heads (`typed = places.is_none() && ...`, :1580-1590). */
    if (hm->place && r->r->depth == o->L) r->typed = r->asks = 0;
    r->slot = (r->typed && !r->asks) ? (int)h->slots++ : -1;
    r->heads = h->heads;
    r->codes = malloc(sizeof(uint64_t) * (size_t)V * h->heads);
    int64_t *point = malloc(sizeof(int64_t) * d);
    for (uint32_t v = 0; v < V; v++) {
      for (uint32_t c = 0; c < d; c++) point[c] = row_value(o, v, c);
      for (uint32_t k = 0; k < h->heads; k++)
        r->codes[(size_t)v * h->heads + k] = head_code(r->ku, point, k, h->hw);
    }
    free(point);
  }
  return h;
}

/* ------------------------------------------------------------------------------------------
 * The place read (fbs_snapshot.rs:2716-3135, served by hamming.rs:1510-1533 and 1625-1634): a
 * register over the session's tokens, every step an integer compare or an index. */

typedef struct {
  int role;               /* the turn being read: 0 none, 1 system, 2 user, 3 assistant */
  size_t start;           /* its first content row */
  size_t nu, *ua, *ub;    /* the contents [ua, ub) of the document's finished user turns */
  size_t nf, *fat, *fpos; /* the finds of the user turn being read: (row, place) */
  int has_place;          /* the register: a place and the end of its turn's content */
  size_t place, pend;
  long offer;             /* the place offered at the row read last, or -1 */
  int over, answered;
} Place;

/* What the register did at one row (PlaceRow, :2860-2877): -1 for none. */
typedef struct {
  long held, offer;
  int stepped;
  long asked_a, asked_b;   /* at a reply's start: the user turn it answers */
  size_t nfound;           /* its finds, and the last of them */
  long found_at, found_pos;
} PlaceRowOut;

static void place_alloc(Place *pl, size_t context) {
  memset(pl, 0, sizeof *pl);
  size_t n = context + 1;
  pl->ua = calloc(n, sizeof(size_t));
  pl->ub = calloc(n, sizeof(size_t));
  pl->fat = calloc(n, sizeof(size_t));
  pl->fpos = calloc(n, sizeof(size_t));
  pl->offer = -1;
}

static void place_free(Place *pl) {
  free(pl->ua); free(pl->ub); free(pl->fat); free(pl->fpos);
}

static void place_reset(Place *pl) {
  pl->role = 0;
  pl->start = pl->nu = pl->nf = pl->place = pl->pend = 0;
  pl->has_place = pl->over = pl->answered = 0;
  pl->offer = -1;
}

static int ends_with(const uint32_t *tok, size_t len, const uint32_t *m, uint32_t ml) {
  if (ml > len) return 0;
  for (uint32_t i = 0; i < ml; i++)
    if (tok[len - ml + i] != m[i]) return 0;
  return 1;
}

static int place_has(const uor_fbs_place *pm, uint32_t vocab, uint32_t token, int bit) {
  return token < vocab && (pm->class_table[token] & bit) != 0;
}

/* PlaceTurns::push (:2801-2837): the role whose marker ends at the last token, 0 for none. */
static int place_turns_push(const uor_fbs_place *pm, Place *pl, const uint32_t *tok, size_t len) {
  if (!len) return 0;
  if (tok[len - 1] == pm->bos) {
    pl->role = 0;
    pl->start = 0;
    pl->nu = 0;
    return 0;
  }
  const uint32_t *mk[3] = {pm->system, pm->user, pm->assistant};
  const uint32_t ml[3] = {pm->system_len, pm->user_len, pm->assistant_len};
  for (int r = 0; r < 3; r++) {
    if (!ml[r] || !ends_with(tok, len, mk[r], ml[r])) continue;
    const size_t m = len - ml[r];
    const int after_sep = ends_with(tok, m, pm->sep, pm->sep_len);
    if (pl->role == 0) {
      if (!(m > 0 && (tok[m - 1] == pm->bos || after_sep))) continue;
    } else {
      const size_t a = pl->start;
      if (!(after_sep && m >= a + pm->sep_len)) continue;
      size_t b = m - pm->sep_len;
      if (b > a && tok[b - 1] == pm->eos) b--;
      if (pl->role == 2) {
        pl->ua[pl->nu] = a;
        pl->ub[pl->nu] = b;
        pl->nu++;
      }
    }
    pl->role = r + 1;
    pl->start = len;
    return r + 1;
  }
  return 0;
}

typedef long (*PlaceFind)(const void *ctx, const Place *pl, const uint32_t *tok, size_t t);

/* PlaceState::advance / read (:2937-3090) without the caller's asks: the last token of
 * tok[0..len) read, every earlier one read before it. `find` answers a row of a user turn's
 * content with the place its question finds among the finished user turns, or -1. */
static void place_read(const uor_fbs_place *pm, uint32_t vocab, Place *pl, const uint32_t *tok,
                       size_t len, PlaceFind find, const void *ctx, PlaceRowOut *row) {
  row->held = row->offer = row->asked_a = row->asked_b = row->found_at = row->found_pos = -1;
  row->stepped = 0;
  row->nfound = 0;
  if (!len) return;
  const size_t t = len - 1;
  const uint32_t token = tok[t];
  /* The step: the row before was offered the token at the place, and this token is it. */
  const long at = pl->offer;
  pl->offer = -1;
  if (at >= 0 && pl->has_place && (size_t)at == pl->place && token == tok[pl->place]) {
    const size_t next = pl->place + 1;
    if (next >= pl->pend || place_has(pm, vocab, tok[next], UOR_FBS_PLACE_STOP)) {
      pl->has_place = 0;
    } else {
      pl->place = next;
      row->stepped = 1;
    }
  }
  if (token == pm->bos) {
    pl->nf = 0;
    pl->has_place = 0;
    pl->answered = 0;
  }
  const int role = place_turns_push(pm, pl, tok, len);
  if (role == 2) {
    pl->nf = 0;
    pl->has_place = 0;
    pl->answered = 0;
  } else if (role == 3) {
    pl->over = 0;
    pl->has_place = 0;
    const int asked = pl->nu > 0 && !pl->answered;
    pl->answered = 1;
    if (asked) {
      const size_t ca = pl->ua[pl->nu - 1], cb = pl->ub[pl->nu - 1];
      long armed = -1;
      for (size_t i = 0; i < pl->nf; i++) {
        if (pl->fat[i] < ca || pl->fat[i] >= cb) continue;
        row->found_at = (long)pl->fat[i];
        row->found_pos = (long)pl->fpos[i];
        row->nfound++;
        if (place_has(pm, vocab, tok[pl->fat[i]], UOR_FBS_PLACE_ARM)) armed = (long)pl->fpos[i];
      }
      pl->nf = 0;
      for (size_t u = 0; armed >= 0 && u + 1 < pl->nu; u++)
        if ((size_t)armed >= pl->ua[u] && (size_t)armed < pl->ub[u]) {
          pl->has_place = 1;
          pl->place = (size_t)armed;
          pl->pend = pl->ub[u];
          break;
        }
      row->asked_a = (long)ca;
      row->asked_b = (long)cb;
    }
  }
  if (pl->role == 2 && t >= pl->start && pl->nu > 0) {
    const long pos = find(ctx, pl, tok, t);
    if (pos >= 0) {
      pl->fat[pl->nf] = t;
      pl->fpos[pl->nf] = (size_t)pos;
      pl->nf++;
    }
  } else if (pl->role == 3) {
    const size_t a = pl->start;
    if (token == pm->eos && t >= a) {
      pl->over = 1;
      pl->has_place = 0;
    }
    if (t + 1 >= a && !pl->over) {
      row->held = pl->has_place ? (long)pl->place : -1;
      const int open = place_has(pm, vocab, token, UOR_FBS_PLACE_OPEN);
      if (row->held >= 0 && (row->stepped || open)) row->offer = row->held;
    }
  }
  pl->offer = row->offer;
}

/* place_pick (:3117-3135): per head the nearest key over the candidate positions (>= 2), the
 * later on ties, kept inside the head's margin (m > d 2^16); then the later of the heads'. */
typedef uint64_t (*PlaceKey)(const void *ctx, uint32_t head, size_t s);
static long place_pick(const uint64_t *queries, const int32_t *margins, uint32_t heads,
                       const size_t *ra, const size_t *rb, size_t nr, PlaceKey key, const void *ctx) {
  long found = -1;
  for (uint32_t j = 0; j < heads; j++) {
    long best = -1;
    uint32_t least = 0;
    for (size_t u = 0; u < nr; u++)
      for (size_t s = ra[u] < 2 ? 2 : ra[u]; s < rb[u]; s++) {
        const uint32_t dd = (uint32_t)__builtin_popcountll(queries[j] ^ key(ctx, j, s));
        if (best < 0 || dd <= least) {
          best = (long)s;
          least = dd;
        }
      }
    if (best >= 0 && (int64_t)margins[j] > ((int64_t)least << 16) && best > found) found = best;
  }
  return found;
}

typedef struct {
  const O *o;
  const HR *r;
  const uint32_t *tok;
  uint64_t first;
} PlaceFindCtx;

static uint64_t place_joined(uint64_t near, uint64_t far, uint64_t first) {
  return (near & first) | (far & ~first);
}

static uint64_t place_key(const void *ctx, uint32_t j, size_t s) {
  const PlaceFindCtx *c = ctx;
  const uint32_t head = c->o->ham->copy + j;
  return place_joined(ham_code(c->r, c->tok[s - 1], head), ham_code(c->r, c->tok[s - 2], head), c->first);
}

/* ServedPlace::find (hamming.rs:1525-1533) with place_find (fbs_snapshot.rs:3093-3108): head j
 * asks with its question code for x_t (the ask point's code through the key rotation, window
 * from row 0) in the first half of its bits and x_{t-1}'s key code in the rest; its key at s
 * is x_{s-1}'s key code in the first half and x_{s-2}'s in the rest. */
static long place_find_row(const void *ctx, const Place *pl, const uint32_t *tok, size_t t) {
  const O *o = ctx;
  const Ham *h = o->ham;
  if (t < 1) return -1;
  const HR *r = &h->reads[h->at[o->L]];
  const uint32_t d = o->d, types = h->heads - h->copy;
  const uint64_t first = (1ull << (h->hw / 2)) - 1;
  int64_t *p = malloc(sizeof(int64_t) * d);
  ham_asked_point(o, r, tok, t, p);
  uint64_t *q = malloc(sizeof(uint64_t) * types);
  for (uint32_t j = 0; j < types; j++)
    q[j] = place_joined(head_code(r->ku, p, h->copy + j, h->hw), ham_code(r, tok[t - 1], h->copy + j), first);
  PlaceFindCtx c = {o, r, tok, first};
  const long found = place_pick(q, r->r->margin + h->copy, types, pl->ua, pl->ub, pl->nu, place_key, &c);
  free(p);
  free(q);
  return found;
}

static void ham_free(Ham *h) {
  if (!h) return;
  for (uint32_t i = 0; i < h->n; i++) {
    free(h->reads[i].qu);
    free(h->reads[i].ku);
    free(h->reads[i].vu);
    free(h->reads[i].codes);
  }
  free(h->reads);
  free(h->pair);
  free(h->at);
  free(h);
}

/* ------------------------------------------------------------------------------------------
 * One sequence's session. */

typedef struct {
  int32_t *x, *branches, *gate_out, *proj, *gate, *up, *query;
  int64_t *scratch, *wide;
  int16_t *act;
  int64_t *state;   /* L * d */
  int32_t *history; /* L * W * d, row 0 the newest drive */
  uint32_t *kept;
  uint32_t position;
  uint64_t candidates;
  uint32_t *tokens;  /* the session's tokens x_0..x_{position-1} (IntegerStackSession::tokens) */
  int64_t *payloads; /* [typed read][context][width]: the type heads' payloads (hamming_payloads) */
  int64_t *normed;   /* width: the final norm's output (the readout read's input) */
  int slide;         /* a full context continues (set_context_slide, session.rs:2391-2402) */
  uint8_t *trace;    /* this step's snap trace (layers * (2 lanes + mlp / 4) bytes), or NULL */
  Place place;       /* the place read's register and turns (session.rs:2239-2241) */
  long held, offer;  /* the register after the last step (last_place, session.rs:2626-2631) */
  Tr *tr;            /* the traces and forced replay of this step, or NULL */
} S;

static void session_alloc(const O *o, S *s) {
  uint32_t d = o->d, wide = d > o->mlp ? d : o->mlp;
  memset(s, 0, sizeof *s);
  s->x = calloc(d, 4);
  s->branches = calloc(2 * d, 4);
  s->gate_out = calloc(o->g, 4);
  s->proj = calloc(d, 4);
  s->gate = calloc(o->mlp, 4);
  s->up = calloc(o->mlp, 4);
  s->query = calloc(d, 4);
  s->scratch = calloc(wide, 8);
  s->wide = calloc(d, 8);
  s->act = calloc(wide, 2);
  s->state = calloc((size_t)o->L * d, 8);
  s->history = calloc((size_t)o->L * o->W * d, 4);
  s->kept = calloc(o->P ? o->P : 1, 4);
  s->tokens = calloc(o->m->context ? o->m->context : 1, 4);
  s->payloads = calloc(o->ham && o->ham->slots ? (size_t)o->ham->slots * o->m->context * d : 1, 8);
  s->normed = calloc(d, 8);
  place_alloc(&s->place, o->m->context);
  s->held = s->offer = -1;
}

static void session_free(S *s) {
  free(s->x); free(s->branches); free(s->gate_out); free(s->proj); free(s->gate); free(s->up);
  free(s->query); free(s->scratch); free(s->wide); free(s->act); free(s->state);
  free(s->history); free(s->kept); free(s->tokens); free(s->payloads); free(s->normed);
  place_free(&s->place);
}

static void session_reset(const O *o, S *s) {
  memset(s->state, 0, sizeof(int64_t) * o->L * o->d);
  memset(s->history, 0, sizeof(int32_t) * o->L * o->W * o->d);
  s->position = 0;
  memset(s->tokens, 0, 4ull * o->m->context);
  if (o->ham && o->ham->slots) memset(s->payloads, 0, 8ull * o->ham->slots * o->m->context * o->d);
  place_reset(&s->place);
  s->held = s->offer = -1;
}

/* The place register over a resumed session's tokens x_0..x_{position-1}: the state it holds
 * after stepping them (the register depends on the tokens and the model alone). */
static void place_replay(const O *o, S *s) {
  if (!o->ham || !o->ham->place) return;
  place_reset(&s->place);
  PlaceRowOut row;
  for (size_t t = 0; t < s->position; t++) {
    place_read(o->ham->place, o->m->vocab, &s->place, s->tokens, t + 1, place_find_row, o, &row);
    s->held = row.held;
    s->offer = row.offer;
  }
}

/* `stack_recurrence_core` with geometric gates, learned rotations and the Hamilton output
 * gate (RS stack/session.rs:4822-4982, `stack_lanes` :5097-5145, `stack_lane_weights`
 * :4989-5026; TW 508-561). The causal window reads W prior drive rows (reference W = 3,
 * `CONVOLUTION_WIDTH` = 4 taps, session.rs:85). Returns the exponent of s->act[..d]. */
static int32_t recurrence(const O *o, uint32_t l, int64_t *state, int32_t *hist, S *s,
                          uint8_t *trace) {
  const uor_fbs_model *m = o->m;
  const uor_fbs_layer *ly = m->layers + l;
  uint32_t d = o->d, W = o->W;
  for (uint32_t i = 0; i < o->g; i++) s->gate_out[i] = sat_add32(s->gate_out[i], ly->gate_bias[i]);
  const int32_t *drive = s->branches, *gate = s->branches + d;
  for (uint32_t i = 0; i < d; i++) {
    int64_t c = wadd64(ly->conv_bias[i], grid_apply(drive[i], tap(o, l, 0, i)));
    for (uint32_t k = 1; k <= W; k++)
      c = wadd64(c, grid_apply(hist[(uint64_t)(k - 1) * d + i], tap(o, l, k, i)));
    s->wide[i] = c;
  }
  /* Age the history: the oldest row drops off, the drive becomes row 0. */
  memmove(hist + d, hist, sizeof(int32_t) * (uint64_t)(W - 1) * d);
  memcpy(hist, drive, sizeof(int32_t) * d);
  const int32_t *decays = s->gate_out, *rot = s->gate_out + o->lanes;
  for (uint32_t lane = 0; lane < o->lanes; lane++) {
    int32_t sq = sat_add32(decays[lane], ly->decay_offset[lane]);
    if (sq < 0) sq = 0;
    if (sq > 65536) sq = 65536;
    uint32_t idx = (uint32_t)sq >> 12;
    if (idx > 15) idx = 15;
    /* Q5's decision trace (BucketTrace::decide, session.rs:2192-2215): a forced entry replaces
     * the score's; the score and the entry used are recorded. */
    if (s->tr && s->tr->decisions) {
      const size_t at = (size_t)l * o->lanes + lane;
      if (s->tr->buckets && s->tr->buckets[at] != 255) idx = s->tr->buckets[at];
      int32_t score = sq;
      memcpy(s->tr->rec + 4 * at, &score, 4);
      s->tr->rec[(size_t)4 * o->L * o->lanes + at] = (uint8_t)idx;
    }
    uint64_t lambda = 1ull << (30 - idx), keep = m->keep_q31[idx];
    int64_t t[4];
    uint32_t root = serve_rotation(m->icosian, m->raw_transition, rot + 4 * lane, lambda, ROTATION_EPSILON, t);
    if (trace) trace[lane] = (uint8_t)root;
    int64_t *h = state + 4 * lane;
    int64_t held[4] = {h[0], h[1], h[2], h[3]};
    i128 moved[4];
    hamilton(t, held, moved);
    for (int k = 0; k < 4; k++) {
      i128 drive_term = wmul128((i128)keep, (i128)s->wide[4 * lane + k]);
      h[k] = shift_wide(wadd128(moved[k], (i128)((u128)drive_term << 16)), 31);
    }
  }
  for (uint32_t lane = 0; lane < o->lanes; lane++) {
    int64_t q[4], rhs[4];
    i128 prod[4];
    uint32_t root = serve_rotation(m->icosian, m->raw_gates, gate + 4 * lane, 1ull << 31, GATE_EPSILON, q);
    if (trace) trace[o->lanes + lane] = (uint8_t)root;
    for (int k = 0; k < 4; k++) rhs[k] = shift(state[4 * lane + k], RESIDUAL_EXP - STATE_EXP);
    hamilton(q, rhs, prod);
    for (int k = 0; k < 4; k++) s->scratch[4 * lane + k] = shift_wide(prod[k], 15);
  }
  return quantize16(s->scratch, d, PRODUCT_EXP, s->act);
}

/* The Hamilton branch of `stack_swiglu` (RS stack/session.rs:4005-4025, TW 566-578). */
static void hamilton_gate(const O *o, const int32_t *gate, const int32_t *up, int64_t *out,
                          uint8_t *trace) {
  const uor_fbs_model *m = o->m;
  for (uint32_t j = 0; j < o->mlp / 4; j++) {
    int64_t q[4], rhs[4];
    i128 prod[4];
    uint32_t root = serve_rotation(m->icosian, m->raw_gates, gate + 4 * j, 1ull << 31, GATE_EPSILON, q);
    if (trace) trace[j] = (uint8_t)root;
    for (int k = 0; k < 4; k++) rhs[k] = up[4 * j + k];
    hamilton(q, rhs, prod);
    for (int k = 0; k < 4; k++) out[4 * j + k] = shift_wide(prod[k], 15);
  }
}

/* `stack_step_fbs` with the Hamming reads and without the address/pair/Q31/memory hooks
 * (RS stack/session.rs:4129-4403, TW 635-675): the token joins the session's tokens first, the
 * stream read follows a layer at its depth (:4252-4276), the readout read moves the final norm's
 * output before the query (:4296-4320). */
static int step(const O *o, S *s, uint32_t token, uint32_t *out_token) {
  const uor_fbs_model *m = o->m;
  uint32_t d = o->d;
  if (token >= m->vocab) return UOR_FBS_ERR_TOKEN;
  /* A session with the slide on steps past its context (session.rs:4143-4151); a model with
   * Hamming reads refuses the slide (can_slide_tokens, :1146-1151), so its tokens stay inside. */
  if (s->position >= m->context && !s->slide) return UOR_FBS_ERR_CONTEXT;
  if (o->ham) s->tokens[s->position] = token;
  const size_t t = s->position;
  /* The place read's register moves on this token, before the row's readout (:4154-4162). */
  if (o->ham && o->ham->place) {
    PlaceRowOut row;
    place_read(o->ham->place, m->vocab, &s->place, s->tokens, t + 1, place_find_row, o, &row);
    s->held = row.held;
    s->offer = row.offer;
  }
  for (uint32_t i = 0; i < d; i++) s->x[i] = to_exp_i32(row_value(o, token, i), Q12_EXP, RESIDUAL_EXP);
  for (uint32_t l = 0; l < o->L; l++) {
    const uor_fbs_layer *ly = m->layers + l;
    int64_t *state = s->state + (uint64_t)l * d;
    int32_t *hist = s->history + (uint64_t)l * o->W * d;
    rms_norm_fine(s->x, d, m->eps_mantissa, m->eps_exp, s->scratch);
    for (uint32_t i = 0; i < d; i++) s->scratch[i] = grid_apply(s->scratch[i], ly->rec_gain[i]);
    gather64(&ly->rec_in, s->scratch, NORM_FINE_EXP, s->branches);
    gather64(&ly->rec_gate, s->scratch, NORM_FINE_EXP, s->gate_out);
    /* The position's snap trace, per layer: the transition's root per lane, the output gate's,
     * then the feed-forward gate's per 4 MLP channels (TW 488-496). */
    uint8_t *lt = s->trace ? s->trace + (uint64_t)l * (2 * o->lanes + o->mlp / 4) : NULL;
    int32_t act_exp = recurrence(o, l, state, hist, s, lt);
    gather16(&ly->rec_out, s->act, act_exp, s->proj);
    for (uint32_t i = 0; i < d; i++) s->x[i] = sat_add32(s->x[i], s->proj[i]);
    rms_norm_fine(s->x, d, m->eps_mantissa, m->eps_exp, s->scratch);
    for (uint32_t i = 0; i < d; i++) s->scratch[i] = grid_apply(s->scratch[i], ly->mlp_gain[i]);
    gather64(&ly->mlp_gate, s->scratch, NORM_FINE_EXP, s->gate);
    gather64(&ly->mlp_up, s->scratch, NORM_FINE_EXP, s->up);
    hamilton_gate(o, s->gate, s->up, s->scratch, lt ? lt + 2 * o->lanes : NULL);
    act_exp = quantize16(s->scratch, o->mlp, PRODUCT_EXP, s->act);
    gather16(&ly->mlp_down, s->act, act_exp, s->proj);
    for (uint32_t i = 0; i < d; i++) s->x[i] = sat_add32(s->x[i], s->proj[i]);
    if (o->ham) ham_stream(o, l + 1, s->tokens, t, s->x, s->payloads, s->tr);
  }
  rms_norm_fine(s->x, d, m->eps_mantissa, m->eps_exp, s->scratch);
  for (uint32_t i = 0; i < d; i++) s->normed[i] = grid_apply(s->scratch[i], m->final_gain[i]);
  if (o->ham)
    ham_readout(o, s->tokens, t, s->normed, s->payloads, o->ham->place ? s->offer : -1, s->tr);
  for (uint32_t i = 0; i < d; i++) {
    int32_t q = to_exp_i32(s->normed[i], NORM_FINE_EXP, Q12_EXP);
    s->query[i] = q > 32767 ? 32767 : q < -32768 ? -32768 : q;
  }
  *out_token = writer(o, s->query, s->kept, &s->candidates);
  s->position++;
  return UOR_FBS_OK;
}

/* ------------------------------------------------------------------------------------------
 * Batched drivers: sequence i goes to thread i % T. */


typedef struct {
  const O *o;
  int kind; /* 0 sequences, 1 decode, 2 score */
  const uint32_t *tokens;
  uint64_t n;
  uint32_t len, prompt_len, gen;
  uint32_t *out_tokens, *out_kept, *out_reply;
  int32_t *out_query;
  const int64_t *in_state;
  const int32_t *in_history;
  const uint32_t *in_position;
  int64_t *out_state;
  int32_t *out_history;
  uint32_t *out_position;
  uint64_t *out_candidates;
  const uint32_t *in_tokens;   /* [n][context], the session's tokens (Hamming reads) */
  uint32_t *out_tokens_ctx;
  const int64_t *in_payloads;  /* [n][typed reads][context][width] */
  int64_t *out_payloads;
  uint64_t matches;
  uint8_t *out_trace; /* sequences: every position's snap trace */
  int64_t *out_place; /* sequences: every position's (held, offered) place, -1 for none */
  uint8_t *out_dtrace;          /* sequences: every position's decision / Hamming trace record */
  size_t dstride;               /* its bytes a position */
  int decisions;                /* record the rate buckets */
  const uint8_t *force_buckets; /* [n][len][L][lanes], 255: not forced */
  const uint64_t *force_codes;  /* [n][len][reads][heads][2] */
  const uint8_t *force_mask;    /* [n][len][reads][heads] */
  int slide;
  int tid, threads, status;
} Job;

static void *run_job(void *arg) {
  Job *j = (Job *)arg;
  const O *o = j->o;
  uint32_t d = o->d;
  uint64_t sw = (uint64_t)o->L * d, hw = (uint64_t)o->L * o->W * d;
  S s;
  session_alloc(o, &s);
  s.slide = j->slide;
  s.trace = NULL;
  const uint64_t stride = (uint64_t)o->L * (2 * o->lanes + o->mlp / 4);
  for (uint64_t i = (uint64_t)j->tid; i < j->n && j->status == 0; i += (uint64_t)j->threads) {
    session_reset(o, &s);
    s.candidates = 0;
    if (j->kind != 1) {
      const uint32_t *row = j->tokens + i * j->len;
      for (uint32_t t = 0; t < j->len; t++) {
        uint32_t tok;
        s.trace = j->out_trace ? j->out_trace + (i * j->len + t) * stride : NULL;
        Tr tr;
        s.tr = NULL;
        if (j->out_dtrace) {
          const uint32_t nr = o->ham ? o->ham->n : 0, nh = o->ham ? o->ham->heads : 0;
          const size_t lanes = (size_t)o->L * o->lanes;
          tr.codes = j->force_codes ? j->force_codes + i * j->len * nr * nh * 2 : NULL;
          tr.mask = j->force_mask ? j->force_mask + i * j->len * nr * nh : NULL;
          tr.reads = nr;
          tr.heads = nh;
          tr.rec = j->out_dtrace + (i * j->len + t) * j->dstride;
          tr.reads_at = j->decisions ? (5 * lanes + 7) & ~(size_t)7 : 0;
          tr.buckets = j->force_buckets ? j->force_buckets + (i * j->len + t) * lanes : NULL;
          tr.decisions = j->decisions;
          s.tr = &tr;
        }
        int err = step(o, &s, row[t], &tok);
        if (err) {
          j->status = err;
          break;
        }
        uint64_t at = i * j->len + t;
        if (j->out_tokens) j->out_tokens[at] = tok;
        if (j->out_kept) memcpy(j->out_kept + at * o->P, s.kept, 4ull * o->P);
        if (j->out_query) memcpy(j->out_query + at * d, s.query, 4ull * d);
        if (j->out_place) {
          j->out_place[2 * at] = s.held;
          j->out_place[2 * at + 1] = s.offer;
        }
        if (j->kind == 2 && t + 1 < j->len && tok == row[t + 1]) j->matches++;
      }
      continue;
    }
    /* Decode: the fbs-toks run (fbs-toks.rs:1513-1533) from an optional saved state. */
    if (j->in_state) memcpy(s.state, j->in_state + i * sw, 8 * sw);
    if (j->in_history) memcpy(s.history, j->in_history + i * hw, 4 * hw);
    if (j->in_position) s.position = j->in_position[i];
    const uint64_t ctx = o->m->context, pw = o->ham ? (uint64_t)o->ham->slots * ctx * d : 0;
    if (j->in_tokens) memcpy(s.tokens, j->in_tokens + i * ctx, 4 * ctx);
    if (j->in_payloads && pw) memcpy(s.payloads, j->in_payloads + i * pw, 8 * pw);
    if (j->in_tokens) place_replay(o, &s);
    const uint32_t *prompt = j->tokens + i * j->prompt_len;
    uint32_t *reply = j->out_reply + i * ((uint64_t)j->gen + 1);
    uint32_t next = 0;
    int err = 0;
    for (uint32_t t = 0; t < j->prompt_len && !err; t++) err = step(o, &s, prompt[t], &next);
    if (!err) reply[0] = next;
    for (uint32_t t = 0; t < j->gen && !err; t++) {
      err = step(o, &s, next, &next);
      if (!err) reply[t + 1] = next;
    }
    if (err) {
      j->status = err;
      break;
    }
    if (j->out_state) memcpy(j->out_state + i * sw, s.state, 8 * sw);
    if (j->out_history) memcpy(j->out_history + i * hw, s.history, 4 * hw);
    if (j->out_position) j->out_position[i] = s.position;
    if (j->out_candidates) j->out_candidates[i] = s.candidates;
    if (j->out_tokens_ctx) memcpy(j->out_tokens_ctx + i * ctx, s.tokens, 4 * ctx);
    if (j->out_payloads && pw) memcpy(j->out_payloads + i * pw, s.payloads, 8 * pw);
  }
  session_free(&s);
  return NULL;
}

static int run_jobs(Job *proto, int threads) {
  if (threads < 1) threads = 1;
  if ((uint64_t)threads > proto->n) threads = proto->n ? (int)proto->n : 1;
  Job *jobs = calloc((size_t)threads, sizeof(Job));
  pthread_t *ids = calloc((size_t)threads, sizeof(pthread_t));
  for (int t = 0; t < threads; t++) {
    jobs[t] = *proto;
    jobs[t].tid = t;
    jobs[t].threads = threads;
  }
  for (int t = 1; t < threads; t++) pthread_create(&ids[t], NULL, run_job, &jobs[t]);
  run_job(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(ids[t], NULL);
  int status = 0;
  uint64_t matches = 0;
  for (int t = 0; t < threads; t++) {
    if (jobs[t].status && !status) status = jobs[t].status;
    matches += jobs[t].matches;
  }
  proto->matches = matches;
  free(jobs);
  free(ids);
  return status;
}

int fbs_oracle_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *tokens,
                         uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                         uint32_t *out_kept, int32_t *out_query, int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 0;
  j.tokens = tokens;
  j.n = sequences;
  j.len = len;
  j.out_tokens = out_tokens;
  j.out_kept = out_kept;
  j.out_query = out_query;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

/* fbs_host_trace_sequences (TW host_kernel.cpp:31-49): the sequences with every position's snap
 * trace, fbs_oracle_trace_stride bytes a position. */
uint64_t fbs_oracle_trace_stride(const uor_fbs_model *m) {
  return (uint64_t)m->layer_count * (2 * (m->width / 4) + m->mlp / 4);
}

int fbs_oracle_trace_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *tokens,
                               uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                               uint32_t *out_kept, int32_t *out_query, uint8_t *out_trace,
                               int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 0;
  j.tokens = tokens;
  j.n = sequences;
  j.len = len;
  j.out_tokens = out_tokens;
  j.out_kept = out_kept;
  j.out_query = out_query;
  j.out_trace = out_trace;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

int fbs_oracle_decode(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *prompts,
                      uint32_t sequences, uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                      const int64_t *in_state, const int32_t *in_history,
                      const uint32_t *in_position, int64_t *out_state, int32_t *out_history,
                      uint32_t *out_position, uint64_t *out_candidates, int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 1;
  j.tokens = prompts;
  j.n = sequences;
  j.prompt_len = prompt_len;
  j.gen = gen;
  j.out_reply = out_reply;
  j.in_state = in_state;
  j.in_history = in_history;
  j.in_position = in_position;
  j.out_state = out_state;
  j.out_history = out_history;
  j.out_position = out_position;
  j.out_candidates = out_candidates;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

/* fbs_oracle_decode with every session's context slide on (set_context_slide,
 * session.rs:2391-2402): a full context continues; refused for a model with Hamming reads. */
int fbs_oracle_decode_slide(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *prompts,
                            uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                            uint32_t *out_reply, const int64_t *in_state, const int32_t *in_history,
                            const uint32_t *in_position, int64_t *out_state, int32_t *out_history,
                            uint32_t *out_position, int threads) {
  O o;
  resolve(&o, m, ext);
  if (o.ham) {
    unresolve(&o);
    return UOR_FBS_ERR_SHAPE;
  }
  Job j = {0};
  j.o = &o;
  j.kind = 1;
  j.slide = 1;
  j.tokens = prompts;
  j.n = sequences;
  j.prompt_len = prompt_len;
  j.gen = gen;
  j.out_reply = out_reply;
  j.in_state = in_state;
  j.in_history = in_history;
  j.in_position = in_position;
  j.out_state = out_state;
  j.out_history = out_history;
  j.out_position = out_position;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

int fbs_oracle_decode_stream(const uor_fbs_model *m, const uor_fbs_ext *ext,
                             const uint32_t *prompts, uint32_t sequences, uint32_t prompt_len,
                             uint32_t gen, uint32_t *out_reply, const int64_t *in_state,
                             const int32_t *in_history, const uint32_t *in_position,
                             const uint32_t *in_tokens, const int64_t *in_payloads,
                             int64_t *out_state, int32_t *out_history, uint32_t *out_position,
                             uint32_t *out_tokens, int64_t *out_payloads, int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 1;
  j.tokens = prompts;
  j.n = sequences;
  j.prompt_len = prompt_len;
  j.gen = gen;
  j.out_reply = out_reply;
  j.in_state = in_state;
  j.in_history = in_history;
  j.in_position = in_position;
  j.out_state = out_state;
  j.out_history = out_history;
  j.out_position = out_position;
  j.in_tokens = in_tokens;
  j.out_tokens_ctx = out_tokens;
  j.in_payloads = in_payloads;
  j.out_payloads = out_payloads;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

uint32_t fbs_oracle_hamming_typed(const uor_fbs_model *m, const uor_fbs_ext *ext) {
  O o;
  resolve(&o, m, ext);
  uint32_t n = o.ham ? o.ham->slots : 0;
  unresolve(&o);
  return n;
}

/* The read at one row, as the reference's hook tests drive it (tests.rs:5579-5623, 8380-8470):
 * tok[0..=t] the window, `x` (width, the stream read at `depth` < layers) or `n` (width, the
 * readout read at depth = layers) read in place, `payloads` the typed reads' caches. */
int fbs_oracle_hamming_row(const uor_fbs_model *m, const uor_fbs_ext *ext, uint32_t depth,
                           const uint32_t *tok, uint32_t t, int32_t *x, int64_t *n,
                           int64_t *payloads) {
  O o;
  resolve(&o, m, ext);
  if (!o.ham) return UOR_FBS_ERR_ARGUMENT;
  if (depth < o.L)
    ham_stream(&o, depth, tok, t, x, payloads, NULL);
  else
    ham_readout(&o, tok, t, n, payloads, -1, NULL);
  unresolve(&o);
  return 0;
}

/* Every vocabulary entry's code per head through read r's key rotation (vocab * heads). */
int fbs_oracle_hamming_codes(const uor_fbs_model *m, const uor_fbs_ext *ext, uint32_t r,
                             uint64_t *out) {
  O o;
  resolve(&o, m, ext);
  if (!o.ham || r >= o.ham->n) return UOR_FBS_ERR_ARGUMENT;
  memcpy(out, o.ham->reads[r].codes, sizeof(uint64_t) * (size_t)m->vocab * o.ham->heads);
  unresolve(&o);
  return 0;
}

int32_t fbs_oracle_stream_sum(int32_t x, int32_t w_c, int64_t c_hi, uint64_t c_lo, int32_t w_y,
                              int64_t y_hi, uint64_t y_lo) {
  return stream_sum(x, w_c, (i128)(((u128)(uint64_t)c_hi << 64) | c_lo), w_y,
                    (i128)(((u128)(uint64_t)y_hi << 64) | y_lo));
}
int64_t fbs_oracle_readout_sum(int64_t n, int32_t w_c, int has_c, int64_t c_hi, uint64_t c_lo,
                               int32_t w_y, int64_t y_hi, uint64_t y_lo) {
  i128 c = (i128)(((u128)(uint64_t)c_hi << 64) | c_lo);
  return readout_sum(n, w_c, has_c ? &c : NULL, w_y, (i128)(((u128)(uint64_t)y_hi << 64) | y_lo));
}
int64_t fbs_oracle_readout_ask_sum(int64_t n, int32_t w_c, int has_c, int64_t c_hi, uint64_t c_lo,
                                   int32_t w_y, int has_y, int64_t y_hi, uint64_t y_lo) {
  i128 c = (i128)(((u128)(uint64_t)c_hi << 64) | c_lo), y = (i128)(((u128)(uint64_t)y_hi << 64) | y_lo);
  return readout_ask_sum(n, w_c, has_c ? &c : NULL, w_y, has_y ? &y : NULL);
}

int fbs_oracle_score(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *rows,
                     uint64_t n_rows, uint32_t len, uint32_t *out_argmin,
                     uint64_t *out_matches, int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 2;
  j.tokens = rows;
  j.n = n_rows;
  j.len = len;
  j.out_tokens = out_argmin;
  int status = run_jobs(&j, threads);
  if (out_matches) *out_matches = j.matches;
  unresolve(&o);
  return status;
}

/* ------------------------------------------------------------------------------------------
 * Exported scalar routines (for the closed-form tests). */

int64_t fbs_oracle_shift(int64_t v, int32_t s) { return shift(v, s); }
int64_t fbs_oracle_shift_wide(int64_t hi, uint64_t lo, uint32_t s) {
  return shift_wide((i128)(((u128)(uint64_t)hi << 64) | lo), s);
}
int64_t fbs_oracle_grid_apply(int64_t v, int16_t code) { return grid_apply(v, code); }
void fbs_oracle_isqrt(uint64_t hi, uint64_t lo, uint64_t out[2]) {
  u128 r = isqrt128(((u128)hi << 64) | lo);
  out[0] = (uint64_t)(r >> 64);
  out[1] = (uint64_t)r;
}
void fbs_oracle_div_u128(uint64_t nhi, uint64_t nlo, uint64_t dhi, uint64_t dlo, uint64_t out[2]) {
  u128 r = div128(((u128)nhi << 64) | nlo, ((u128)dhi << 64) | dlo);
  out[0] = (uint64_t)(r >> 64);
  out[1] = (uint64_t)r;
}
uint32_t fbs_oracle_snap_select(const int8_t *icosian, const int32_t raw[4]) {
  return snap_select(icosian, raw);
}
int fbs_oracle_diff_positive(int64_t da, int64_t db) { return diff_positive(da, db); }
void fbs_oracle_serve_rotation(const int8_t *icosian, uint32_t raw_form, const int32_t raw[4],
                               uint64_t lambda, uint64_t epsilon, int64_t out[4]) {
  serve_rotation(icosian, raw_form, raw, lambda, epsilon, out);
}
int32_t fbs_oracle_quantize16(const int64_t *v, uint32_t n, int32_t exp, int16_t *out) {
  return quantize16(v, n, exp, out);
}
void fbs_oracle_rms_norm_fine(const int32_t *x, uint32_t n, int64_t eps_mantissa, int32_t eps_exp,
                              int64_t *out) {
  rms_norm_fine(x, n, eps_mantissa, eps_exp, out);
}
uint32_t fbs_oracle_writer(const uor_fbs_model *m, const uor_fbs_ext *ext, const int32_t *query,
                           uint32_t *kept, uint64_t *candidates) {
  O o;
  resolve(&o, m, ext);
  uint64_t c = 0;
  uint32_t t = writer(&o, query, kept, &c);
  if (candidates) *candidates = c;
  unresolve(&o);
  return t;
}

/* ------------------------------------------------------------------------------------------
 * The place read's pieces, for the tests that pin them (the reference's place_tests,
 * fbs_snapshot.rs:3136-3370, and a_session_serves_the_place_read, stack/tests.rs:8882-8930). */

/* Teacher-forced sequences with every position's place register after the step (last_place:
 * held, offered; -1 for none), besides fbs_oracle_sequences' outputs. */
int fbs_oracle_place_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext,
                               const uint32_t *tokens, uint32_t sequences, uint32_t len,
                               uint32_t *out_tokens, int32_t *out_query, int64_t *out_place,
                               int threads) {
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 0;
  j.tokens = tokens;
  j.n = sequences;
  j.len = len;
  j.out_tokens = out_tokens;
  j.out_query = out_query;
  j.out_place = out_place;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}

typedef struct {
  const int64_t *finds; /* (row, place) pairs */
  uint32_t n;
} InjectedFinds;

static long injected_find(const void *ctx, const Place *pl, const uint32_t *tok, size_t t) {
  (void)pl;
  (void)tok;
  const InjectedFinds *f = ctx;
  for (uint32_t i = 0; i < f->n; i++)
    if (f->finds[2 * i] == (int64_t)t) return (long)f->finds[2 * i + 1];
  return -1;
}

/* The register over tokens[0..n) from a fresh state, the question at each row finds[2i] finding
 * finds[2i+1] and every other row nothing (the tests' `rows`, fbs_snapshot.rs:3161-3165). Per row,
 * 8 values: held, offer, stepped, asked content start and end, the asked finds' count and the
 * last of them (row, place); -1 for none. */
int fbs_oracle_place_rows(const uor_fbs_place *pm, uint32_t vocab, const uint32_t *tokens,
                          uint64_t n, const int64_t *finds, uint32_t nfinds, int64_t *out) {
  Place pl;
  place_alloc(&pl, n);
  InjectedFinds f = {finds, nfinds};
  for (uint64_t t = 0; t < n; t++) {
    PlaceRowOut row;
    place_read(pm, vocab, &pl, tokens, t + 1, injected_find, &f, &row);
    int64_t *o = out + 8 * t;
    o[0] = row.held;
    o[1] = row.offer;
    o[2] = row.stepped;
    o[3] = row.asked_a;
    o[4] = row.asked_b;
    o[5] = (int64_t)row.nfound;
    o[6] = row.found_at;
    o[7] = row.found_pos;
  }
  place_free(&pl);
  return 0;
}

typedef struct {
  const uint64_t *keys;
} PickKeys;

static uint64_t pick_key(const void *ctx, uint32_t j, size_t s) {
  (void)j;
  return ((const PickKeys *)ctx)->keys[s];
}

/* place_pick over candidate ranges [ranges[2u], ranges[2u+1]), every head's key at position s
 * keys[s] (the tests' key closure). Returns the position, or -1. */
int64_t fbs_oracle_place_pick(const uint64_t *queries, const int32_t *margins, uint32_t heads,
                              const uint64_t *ranges, uint32_t nranges, const uint64_t *keys) {
  size_t *ra = calloc(nranges + 1, sizeof(size_t)), *rb = calloc(nranges + 1, sizeof(size_t));
  for (uint32_t u = 0; u < nranges; u++) {
    ra[u] = ranges[2 * u];
    rb[u] = ranges[2 * u + 1];
  }
  PickKeys k = {keys};
  const long found = place_pick(queries, margins, heads, ra, rb, nranges, pick_key, &k);
  free(ra);
  free(rb);
  return found;
}

/* ------------------------------------------------------------------------------------------
 * The Hamming trace and Q5's decision trace with forced replay (session.rs:2361-2370,
 * 2438-2520), teacher-forced from fresh sessions. A position's record: with `decisions`, each
 * layer's rate scores (i32, [L][lanes]) and entries used (u8, [L][lanes]), padded to 8 bytes;
 * then each read in depth order, each served head (the copy heads, then the type heads where the
 * read serves them): the query (u64), the key at the row (u64, 0 at row 0), the kept count (u32)
 * and the kept positions (u32 each, `kept` of them), padded to 8 bytes. */
uint64_t fbs_oracle_decision_stride(const uor_fbs_model *m, const uor_fbs_ext *ext, int decisions) {
  O o;
  resolve(&o, m, ext);
  size_t at = decisions ? (5 * (size_t)o.L * o.lanes + 7) & ~(size_t)7 : 0;
  if (o.ham)
    for (uint32_t i = 0; i < o.ham->n; i++)
      at += (o.ham->copy + (o.ham->reads[i].typed ? o.ham->heads - o.ham->copy : 0)) *
            tr_head_bytes(o.ham->kept);
  unresolve(&o);
  return at;
}

int fbs_oracle_decision_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext,
                                  const uint32_t *tokens, uint32_t sequences, uint32_t len,
                                  int decisions, const uint8_t *force_buckets,
                                  const uint64_t *force_codes, const uint8_t *force_mask,
                                  uint32_t *out_tokens, int32_t *out_query, uint8_t *out_trace,
                                  int threads) {
  const uint64_t stride = fbs_oracle_decision_stride(m, ext, decisions);
  O o;
  resolve(&o, m, ext);
  Job j = {0};
  j.o = &o;
  j.kind = 0;
  j.tokens = tokens;
  j.n = sequences;
  j.len = len;
  j.out_tokens = out_tokens;
  j.out_query = out_query;
  j.out_dtrace = out_trace;
  j.dstride = stride;
  j.decisions = decisions;
  j.force_buckets = force_buckets;
  j.force_codes = force_codes;
  j.force_mask = force_mask;
  int status = run_jobs(&j, threads);
  unresolve(&o);
  return status;
}
