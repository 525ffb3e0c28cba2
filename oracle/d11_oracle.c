/*
 * d11_oracle.c - CPU restatement of the discrete M1 evaluator, for tests only.
 *
 * TEST INFRASTRUCTURE. The parity checker of the HIP row scorer (uor_d11_score_rows) and the
 * CPU baseline bench.py times beside it. Only tests/ and bench.py's cpu_baseline leg load it.
 *
 * It follows IntegerDiscreteModel (crates/uor-r4-integer/src/discrete_d11.rs) statement by
 * statement, serial and without the product's tables of precomputed root actions: every
 * function names the lines it restates. Inputs are the product's model image
 * (include/uor_d11.h); the geometry tables come from uor-r4_amd/csrc/d11_tables.h (data).
 *
 * Pinning: tests/test_d11_oracle.py runs the reference's own witness tests on it
 * (discrete_d11.rs:2088-2250: route writer, context transport, Flock and Relation copy
 * successor with their literal read vectors, losses and relation scores; :2306-2458: the
 * trunk's joint pointer), checks the geometry tables against closed forms, and brute-forces the
 * writer's orderings on random models.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/uor_d11.h"
#include "../uor-r4_amd/csrc/d11_tables.h"

#define MAX_NODES 512
#define EDGE_TYPES 5

typedef struct {
  int child[3]; /* -1 for an atom leaf */
  int atom;     /* -1 for an inner node */
  int level, first, last;
} Node;

typedef struct {
  int count, frontier_len;
  Node nodes[MAX_NODES];
  int frontier[32];
} Plan;

/* build_row_plan (discrete_d11.rs:813-884). */
static int build_row_plan(int length, Plan *p) {
  if (length < 1 || length > (int)UOR_D11_MAX_CONTEXT) return -1;
  p->count = 0;
  p->frontier_len = 0;
  for (int atom = 0; atom < length; atom++) {
    p->frontier[p->frontier_len++] = p->count;
    Node *n = &p->nodes[p->count++];
    n->child[0] = n->child[1] = n->child[2] = -1;
    n->atom = atom;
    n->level = 0;
    n->first = n->last = atom;
    for (;;) {
      int f = p->frontier_len;
      if (f < 3) break;
      int c0 = p->frontier[f - 3], c1 = p->frontier[f - 2], c2 = p->frontier[f - 1];
      int lv = p->nodes[c0].level;
      if (p->nodes[c1].level != lv || p->nodes[c2].level != lv) break;
      Node *q = &p->nodes[p->count];
      q->child[0] = c0;
      q->child[1] = c1;
      q->child[2] = c2;
      q->atom = -1;
      q->level = lv + 1;
      q->first = p->nodes[c0].first;
      q->last = p->nodes[c2].last;
      p->frontier_len = f - 3;
      p->frontier[p->frontier_len++] = p->count;
      p->count++;
    }
  }
  return 0;
}

typedef struct {
  int32_t x[8];
} Vec8;

/* root_id (:725-727). */
static int root_id(const int32_t *x) {
  for (int r = 0; r < 16; r++) {
    int same = 1;
    for (int d = 0; d < 8; d++)
      if (x[d] != kD11Roots[r][d]) same = 0;
    if (same) return r;
  }
  return -1;
}

/* action (:729-738). */
static Vec8 action(int a, const int32_t *x) {
  Vec8 y;
  for (int d = 0; d < 8; d++) {
    int axis = kD11Axes[(a << 3) + d];
    int32_t v = x[axis & 7];
    y.x[d] = (axis & 8) ? -v : v;
  }
  return y;
}

static int compose(int a, int b) { return kD11Compose[(a << 6) + b]; }

/* root_cost (:744-753). */
static void root_cost(const int32_t *x, int root, uint32_t *dist, uint32_t *ham) {
  uint32_t d = 0, h = 0;
  for (int k = 0; k < 8; k++) {
    int32_t y = kD11Roots[root][k];
    int32_t diff = x[k] - y;
    d += (uint32_t)(diff < 0 ? -diff : diff);
    h += x[k] != y;
  }
  *dist = d;
  *ham = h;
}

/* snap (:755-778): the nearest n-fold root by (distance, Hamming), lowest root on ties. */
static int snap(const int32_t *x, int n) {
  int best = 0;
  uint32_t bd = UINT32_MAX, bh = UINT32_MAX;
  for (int r = 0; r < 16; r++) {
    uint32_t dist = 0, ham = 0;
    for (int d = 0; d < 8; d++) {
      int32_t y = 0, v = kD11Roots[r][d];
      for (int k = 0; k < n; k++) y += v;
      int32_t diff = x[d] - y;
      dist += (uint32_t)(diff < 0 ? -diff : diff);
      ham += x[d] != y;
    }
    if (dist < bd || (dist == bd && ham < bh)) {
      best = r;
      bd = dist;
      bh = ham;
    }
  }
  return best;
}

static Vec8 root_vec(int r) {
  Vec8 v;
  for (int d = 0; d < 8; d++) v.x[d] = kD11Roots[r][d];
  return v;
}

/* ---------------------------------------------------------------------------------------- */
/* The trunk's sparse count tables: (key, token) -> count, a sorted copy searched by halves. */

typedef struct {
  uint64_t *pairs; /* key << 32 | token, ascending */
  uint32_t *counts;
  uint64_t n;
} Sparse;

typedef struct {
  const uor_d11_model *m;
  int trunk;
  Sparse sp[12];
  uint8_t (*roots4)[4]; /* [vocab][4] codebook roots */
  /* with_state_transport_knockout (:1283-1304): the model with identity routes and zero gates */
  int knockout;
  uor_d11_model km;
  uint32_t *kroutes;
  int32_t *kgates;
} Oracle;

static int cmp_u64_idx(const void *a, const void *b, void *ctx) {
  const uint64_t *k = (const uint64_t *)ctx;
  uint64_t x = k[*(const uint64_t *)a], y = k[*(const uint64_t *)b];
  return x < y ? -1 : x > y;
}

static void sparse_build(Sparse *s, const uint32_t *tri, uint64_t n) {
  s->n = n;
  s->pairs = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));
  s->counts = (uint32_t *)malloc((n ? n : 1) * sizeof(uint32_t));
  uint64_t *keys = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));
  uint64_t *idx = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));
  for (uint64_t i = 0; i < n; i++) {
    keys[i] = (uint64_t)tri[3 * i] << 32 | tri[3 * i + 1];
    idx[i] = i;
  }
  qsort_r(idx, n, sizeof(uint64_t), cmp_u64_idx, keys);
  for (uint64_t i = 0; i < n; i++) {
    s->pairs[i] = keys[idx[i]];
    s->counts[i] = tri[3 * idx[i] + 2];
  }
  free(keys);
  free(idx);
}

/* DiscreteSparseCountTable::get (:451-456). */
static uint32_t sparse_get(const Sparse *s, uint32_t key, uint32_t tok) {
  uint64_t want = (uint64_t)key << 32 | tok, lo = 0, hi = s->n;
  while (lo < hi) {
    uint64_t mid = (lo + hi) / 2;
    if (s->pairs[mid] < want) lo = mid + 1;
    else hi = mid;
  }
  return lo < s->n && s->pairs[lo] == want ? s->counts[lo] : 0;
}

/* The index range of `key`'s entries (tokens ascending, as the BTreeMap iterates). */
static void sparse_range(const Sparse *s, uint32_t key, uint64_t *b, uint64_t *e) {
  uint64_t lo = 0, hi = s->n, want = (uint64_t)key << 32;
  while (lo < hi) {
    uint64_t mid = (lo + hi) / 2;
    if (s->pairs[mid] < want) lo = mid + 1;
    else hi = mid;
  }
  *b = lo;
  hi = s->n;
  want = ((uint64_t)key + 1) << 32;
  while (lo < hi) {
    uint64_t mid = (lo + hi) / 2;
    if (s->pairs[mid] < want) lo = mid + 1;
    else hi = mid;
  }
  *e = lo;
}

enum { T_READ = 0, T_REC = 1, T_READ_REC = 2, T_QUERY = 7, T_QUERY_READ = 8, T_QUERY_REC = 9 };

static const int32_t *token_block(const uor_d11_model *m, uint32_t tok, int b) {
  return m->table + ((size_t)tok * m->blocks + b) * 8;
}

/* ---------------------------------------------------------------------------------------- */
/* route_read (:1337-1451). Returns a row status. `trace` (NULL: none): the row's trace words,
 * filled with UINT32_MAX by the caller; `knockout`: the knocked-out read (:1346-1361). */
static int route_read(const uor_d11_model *m, const uint32_t *prefix, int length, const Plan *p,
                      Vec8 *out, int knockout, uint32_t *trace) {
  const uint32_t last_token = prefix[length - 1];
  const uint32_t tstride = UOR_D11_ROUTE_TRACE_HEADER_WORDS + m->stages * UOR_D11_ROUTE_TRACE_STAGE_WORDS;
  if (knockout) {
    for (uint32_t b = 0; b < m->blocks; b++) {
      memcpy(out[b].x, token_block(m, last_token, b), sizeof out[b].x);
      if (trace) {
        uint32_t *w = trace + b * tstride;
        int r = root_id(out[b].x);
        w[0] = (uint32_t)p->frontier_len;
        w[1] = r < 0 ? UINT32_MAX : (uint32_t)r;
        w[2] = 0;
      }
    }
    return UOR_D11_ROW_OK;
  }
  for (uint32_t b = 0; b < m->blocks; b++) {
    const int32_t *query = token_block(m, last_token, b);
    uint32_t *w = trace ? trace + b * tstride : NULL;
    int node = 0, root = 0, total = 0, resolved = 0;
    for (uint32_t stage = 0; stage < m->stages; stage++) {
      int frame = (int)m->routes[b * m->stages + stage];
      uint32_t *ws = w ? w + UOR_D11_ROUTE_TRACE_HEADER_WORDS + stage * UOR_D11_ROUTE_TRACE_STAGE_WORDS : NULL;
      if (ws) {
        ws[0] = (uint32_t)frame;
        ws[1] = (uint32_t)root;
      }
      Vec8 q = action(frame, query);
      int count = stage == 0 ? p->frontier_len : 3;
      int best = 0, goal = 0;
      uint32_t bd = UINT32_MAX, bh = UINT32_MAX;
      for (int port = 0; port < count; port++) {
        int r = stage == 0 ? port : kD11Branch[root][port];
        uint32_t dist, ham;
        root_cost(q.x, r, &dist, &ham);
        if (dist < bd || (dist == bd && ham < bh)) {
          best = port;
          bd = dist;
          bh = ham;
          goal = r;
        }
      }
      total = compose(kD11Bfs[(root << 4) + goal], total);
      root = goal;
      int next;
      if (stage == 0) {
        next = p->frontier[best];
      } else {
        if (p->nodes[node].atom >= 0) return UOR_D11_ROW_ROUTE; /* stepped past a leaf */
        next = p->nodes[node].child[best];
      }
      if (ws) {
        ws[2] = (uint32_t)best;
        ws[3] = (uint32_t)goal;
        ws[4] = (uint32_t)total;
        ws[5] = (uint32_t)next;
      }
      if (p->nodes[next].atom >= 0) {
        out[b] = action(total, token_block(m, prefix[p->nodes[next].atom], b));
        resolved = 1;
        if (w) {
          w[0] = (uint32_t)p->frontier_len;
          w[2] = stage + 1;
          w[3] = (uint32_t)p->nodes[next].atom;
        }
        break;
      }
      node = next;
    }
    if (!resolved) return UOR_D11_ROW_ROUTE;
    if (w) {
      int r = root_id(out[b].x);
      if (r < 0) return UOR_D11_ROW_ORBIT;
      w[1] = (uint32_t)r;
    }
  }
  return UOR_D11_ROW_OK;
}

/* flock_or_relation_read (:1453-1741). rel_out (blocks x count) receives the relation scores.
 * `trace` (NULL: none): the row's trace words, filled with UINT32_MAX by the caller; then every
 * level is visited, gated or not, as the traced read does (:1649-1652). `rel_trace` (relation
 * reads; NULL: none): blocks x `rel_stride` words, filled likewise. */
static int flock_or_relation_read(const uor_d11_model *m, const uint32_t *prefix, int length,
                                  const Plan *p, int kept, int sweeps, int relation, Vec8 *out,
                                  int32_t *rel_out, uint32_t *trace, uint32_t *rel_trace,
                                  int rel_stride) {
  const uint32_t tstride = UOR_D11_ACTIVE_TRACE_HEADER_WORDS + m->stages * UOR_D11_ACTIVE_TRACE_LEVEL_WORDS;
  const int blocks = (int)m->blocks, stages = (int)m->stages, nodes = p->count;
  const uint32_t last_token = prefix[length - 1];
  const int32_t *rgates = m->gates + blocks * stages;
  static __thread int frame[MAX_NODES];
  static __thread Vec8 payload[MAX_NODES];
  static __thread int32_t rel[MAX_NODES], prev[MAX_NODES];
  for (int b = 0; b < blocks; b++) {
    int f = b == 0 ? blocks - 1 : 0;
    const int32_t *query_frame = token_block(m, last_token, f);
    Vec8 u;
    memcpy(u.x, token_block(m, last_token, b), sizeof u.x);
    int fq = root_id(query_frame);
    if (fq < 0 || root_id(u.x) < 0) return UOR_D11_ROW_ORBIT;
    uint32_t *w = trace ? trace + b * tstride : NULL;
    if (w) {
      w[0] = (uint32_t)fq;
      w[3] = (uint32_t)root_id(u.x);
    }
    for (int i = 0; i < nodes; i++) {
      const Node *n = &p->nodes[i];
      if (n->atom >= 0) {
        uint32_t tok = prefix[n->atom];
        frame[i] = root_id(token_block(m, tok, f));
        if (frame[i] < 0) return UOR_D11_ROW_ORBIT;
        memcpy(payload[i].x, token_block(m, tok, b), sizeof payload[i].x);
      } else {
        int c0 = n->child[0];
        frame[i] = frame[c0];
        int32_t sum[8] = {0};
        for (int k = 0; k < 3; k++) {
          int ch = n->child[k];
          Vec8 carried = action(kD11Bfs[(frame[ch] << 4) + frame[c0]], payload[ch].x);
          for (int d = 0; d < 8; d++) sum[d] += carried.x[d];
        }
        payload[i] = root_vec(snap(sum, 3));
      }
    }
    for (int i = 0; i < nodes; i++) rel[i] = 0;
    if (relation) {
      for (int i = 0; i < nodes; i++) {
        uint32_t dist, ham;
        root_cost(query_frame, frame[i], &dist, &ham);
        prev[i] = 8 - (int32_t)dist;
      }
      for (int sw = 0; sw < sweeps; sw++) {
        for (int i = 0; i < nodes; i++) {
          const Node *ni = &p->nodes[i];
          if (ni->last >= length) continue;
          int li = ni->level;
          for (int e = 0; e < EDGE_TYPES; e++) {
            int gt = rgates[li * EDGE_TYPES + e];
            if (gt == 0) continue;
            int32_t esum = 0;
            if (e == 0) {
              if (ni->atom < 0)
                for (int k = 0; k < 3; k++)
                  if (p->nodes[ni->child[k]].last < length) esum += prev[ni->child[k]];
              for (int q = i + 1; q < nodes; q++) {
                const Node *np_ = &p->nodes[q];
                if (np_->atom < 0 && np_->last < length &&
                    (np_->child[0] == i || np_->child[1] == i || np_->child[2] == i))
                  esum += prev[q];
              }
            } else if (e == 1) {
              for (int q = i + 1; q < nodes; q++) {
                const Node *np_ = &p->nodes[q];
                if (np_->atom >= 0 || np_->last >= length) continue;
                int c0 = np_->child[0], c1 = np_->child[1], c2 = np_->child[2];
                if (i == c0 && p->nodes[c1].last < length) {
                  esum += prev[c1];
                } else if (i == c1) {
                  if (p->nodes[c0].last < length) esum += prev[c0];
                  if (p->nodes[c2].last < length) esum += prev[c2];
                } else if (i == c2 && p->nodes[c1].last < length) {
                  esum += prev[c1];
                }
              }
            } else if (e == 2) {
              for (int j = 0; j < i; j++)
                if (p->nodes[j].last < length && p->nodes[j].level == li &&
                    p->nodes[j].last + 1 == ni->first)
                  esum += prev[j];
            } else if (e == 3) {
              if (li == 0) {
                uint32_t tid = prefix[ni->last];
                for (int j = 0; j < i; j++)
                  if (p->nodes[j].last < length && p->nodes[j].level == 0 &&
                      prefix[p->nodes[j].last] == tid)
                    esum = prev[j];
              }
            } else {
              for (int j = 0; j < i; j++)
                if (p->nodes[j].last < length && p->nodes[j].level == li && frame[j] == frame[i])
                  esum = prev[j];
            }
            rel[i] += gt > 0 ? esum : -esum;
          }
        }
        memcpy(prev, rel, sizeof(int32_t) * nodes);
      }
      if (rel_out) memcpy(rel_out + (size_t)b * nodes, rel, sizeof(int32_t) * nodes);
      if (rel_trace)
        for (int i = 0; i < nodes; i++) rel_trace[(size_t)b * rel_stride + i] = (uint32_t)rel[i];
    }
    int terms = 1;
    for (int l = 0; l < stages; l++) {
      int gate = m->gates[b * stages + l];
      if (gate == 0 && !w) continue;
      int top[8], found = 0, eligible = 0;
      int32_t kr[8];
      uint32_t kd[8], kh[8];
      for (int node = 0; node < nodes; node++) {
        const Node *n = &p->nodes[node];
        if (n->level != l || n->last + 1 >= length) continue;
        eligible++;
        uint32_t dist, ham;
        root_cost(query_frame, frame[node], &dist, &ham);
        int32_t rs = rel[node];
        int at = found;
        while (at > 0) {
          int o = top[at - 1];
          int better = rs > kr[at - 1] ||
                       (rs == kr[at - 1] &&
                        (dist < kd[at - 1] ||
                         (dist == kd[at - 1] &&
                          (ham < kh[at - 1] ||
                           (ham == kh[at - 1] &&
                            (n->last > p->nodes[o].last ||
                             (n->last == p->nodes[o].last && node < o)))))));
          if (!better) break;
          if (at < kept) {
            top[at] = top[at - 1];
            kr[at] = kr[at - 1];
            kd[at] = kd[at - 1];
            kh[at] = kh[at - 1];
          }
          at--;
        }
        if (at < kept) {
          top[at] = node;
          kr[at] = rs;
          kd[at] = dist;
          kh[at] = ham;
          if (found < kept) found++;
        }
      }
      uint32_t *wl = w ? w + UOR_D11_ACTIVE_TRACE_HEADER_WORDS + l * UOR_D11_ACTIVE_TRACE_LEVEL_WORDS : NULL;
      if (wl) {
        wl[0] = (uint32_t)(gate + 1);
        wl[1] = (uint32_t)found;
        wl[3] = (uint32_t)eligible;
      }
      if (found == 0) continue;
      int32_t sum[8] = {0};
      for (int k = 0; k < found; k++) {
        Vec8 carried = action(kD11Bfs[(frame[top[k]] << 4) + fq], payload[top[k]].x);
        for (int d = 0; d < 8; d++) sum[d] += carried.x[d];
      }
      int mroot = snap(sum, found);
      if (wl) {
        wl[2] = (uint32_t)mroot;
        for (int k = 0; k < found; k++) {
          int act = kD11Bfs[(frame[top[k]] << 4) + fq];
          Vec8 carried = action(act, payload[top[k]].x);
          int cr = root_id(carried.x);
          if (cr < 0) return UOR_D11_ROW_ORBIT;
          wl[4 + k] = (uint32_t)top[k];
          wl[12 + k] = (uint32_t)act;
          wl[20 + k] = (uint32_t)cr;
        }
      }
      if (gate == 0) continue;
      for (int d = 0; d < 8; d++) u.x[d] += gate > 0 ? kD11Roots[mroot][d] : -kD11Roots[mroot][d];
      terms++;
    }
    out[b] = root_vec(snap(u.x, terms));
    if (w) {
      w[1] = (uint32_t)root_id(out[b].x);
      w[2] = (uint32_t)terms;
    }
  }
  return UOR_D11_ROW_OK;
}

/* ---------------------------------------------------------------------------------------- */
/* The trunk's joint-pointer gate (:463-685). */

static uint16_t pack4(const uint8_t r[4]) {
  return (uint16_t)((r[0] & 15) | (r[1] & 15) << 4 | (r[2] & 15) << 8 | (r[3] & 15) << 12);
}

static int cl06_inverse(int a) { return compose(a, compose(a, a)); }

static int trunk_gate(const Oracle *o, const uint32_t *prefix, int length, Vec8 *q) {
  const uor_d11_model *m = o->m;
  const uor_d11_trunk *t = m->trunk;
  uint8_t read_roots[4];
  for (int b = 0; b < 4; b++) {
    int r = root_id(q[b].x);
    if (r < 0) return UOR_D11_ROW_ORBIT;
    read_roots[b] = (uint8_t)r;
  }
  uint16_t read_code = pack4(read_roots);
  /* compute_rec_code (:601-644) */
  int last = length - 1, prevp = last > 0 ? last - 1 : 0, mid = last / 2;
  uint8_t out_roots[4];
  static __thread int acc_at[UOR_D11_MAX_CONTEXT];
  for (int b = 0; b < 4; b++) {
    int acc = 0;
    for (int pos = 0; pos < length; pos++) {
      int r = o->roots4[prefix[pos]][b];
      acc = compose((int)t->step_candidates[(b << 4) + r], acc);
      acc_at[pos] = acc;
    }
    int f_last = acc_at[last];
    int h_prev = compose(f_last, cl06_inverse(acc_at[prevp]));
    int h_mid = compose(f_last, cl06_inverse(acc_at[mid]));
    Vec8 qc = root_vec(o->roots4[prefix[last]][b]);
    Vec8 rp = root_vec(o->roots4[prefix[prevp]][b]), rm = root_vec(o->roots4[prefix[mid]][b]);
    Vec8 rs = root_vec(o->roots4[prefix[0]][b]);
    Vec8 prev_rot = action(h_prev, rp.x), mid_rot = action(h_mid, rm.x);
    Vec8 full_rot = action(f_last, rs.x);
    int32_t sum[8];
    for (int d = 0; d < 8; d++) sum[d] = qc.x[d] + prev_rot.x[d] + mid_rot.x[d] + full_rot.x[d];
    Vec8 snapped = root_vec(snap(sum, 4));
    Vec8 normalized = action((int)t->norm_candidates[b], snapped.x);
    int nr = root_id(normalized.x);
    if (nr < 0) return UOR_D11_ROW_ORBIT;
    out_roots[b] = (uint8_t)nr;
  }
  uint16_t rec_code = pack4(out_roots);
  /* orbit_root_causal_successor (:470-498) */
  int has_ptr = 0;
  uint32_t ptr = 0;
  if (length >= 2) {
    const uint8_t *qr = o->roots4[prefix[last]];
    for (int pos = 0; pos < last; pos++) {
      const uint8_t *pr = o->roots4[prefix[pos]];
      if (pr[0] == qr[0] && pr[1] == qr[1] && pr[2] == qr[2] && pr[3] == qr[3]) {
        has_ptr = 1;
        ptr = prefix[pos + 1];
      }
    }
  }
  /* select_level3_joint_pointer_global (:546-599) */
  uint32_t qtok = prefix[last];
  uint32_t best_tok = t->unigram[0], best_u = 0;
  uint64_t best_s = 0;
  const uint32_t keys[3] = {qtok, read_code, rec_code};
  const int src[3] = {T_QUERY, T_READ, T_REC};
  for (int k = 0; k < 4; k++) {
    uint64_t b = 0, e = 0;
    if (k < 3) {
      sparse_range(&o->sp[src[k]], keys[k], &b, &e);
    } else {
      if (!has_ptr) break;
    }
    for (uint64_t i = b; i < (k < 3 ? e : b + 1); i++) {
      uint32_t tok = k < 3 ? (uint32_t)(o->sp[src[k]].pairs[i] & 0xffffffffu) : ptr;
      if (tok >= m->vocabulary) continue;
      uint64_t c_q = sparse_get(&o->sp[T_QUERY], qtok, tok);
      uint64_t c_qr = sparse_get(&o->sp[T_QUERY_READ], qtok << 16 | read_code, tok);
      uint64_t c_r = sparse_get(&o->sp[T_READ], read_code, tok);
      uint64_t c_qc = sparse_get(&o->sp[T_QUERY_REC], qtok << 16 | rec_code, tok);
      uint64_t c_rr = sparse_get(&o->sp[T_READ_REC], (uint32_t)read_code << 16 | rec_code, tok);
      uint64_t boost = has_ptr && ptr == tok ? 256u : 0u;
      uint64_t s = (c_qr << 6) + (c_qc << 5) + (c_rr << 3) + (c_r << 1) + c_q + boost;
      uint32_t u = t->unigram[1 + tok];
      if (s > best_s || (s == best_s && s > 0 && u > best_u) ||
          (s == best_s && s > 0 && u == best_u && tok < best_tok)) {
        best_s = s;
        best_u = u;
        best_tok = tok;
      }
    }
  }
  /* apply_joint_pointer_gate (:646-684) */
  const uint8_t *target = o->roots4[best_tok];
  for (int b = 0; b < 4; b++) {
    Vec8 rot = action(kD11Bfs[(read_roots[b] << 4) + target[b]], q[b].x);
    q[b] = root_vec(snap(rot.x, 1));
  }
  return UOR_D11_ROW_OK;
}

/* ---------------------------------------------------------------------------------------- */
/* address_distance and token_distance (:1743-1757). */
static uint32_t address_distance(const uor_d11_model *m, const Vec8 *q, uint32_t cell) {
  uint32_t a, b, h;
  root_cost(q[0].x, (int)(cell >> 4), &a, &h);
  root_cost(q[m->blocks - 1].x, (int)(cell & 15), &b, &h);
  return a + b;
}

static uint32_t token_distance(const uor_d11_model *m, const Vec8 *q, uint32_t tok) {
  uint32_t sum = 0;
  for (uint32_t b = 0; b < m->blocks; b++) {
    const int32_t *v = token_block(m, tok, b);
    for (int d = 0; d < 8; d++) {
      int32_t diff = q[b].x[d] - v[d];
      sum += (uint32_t)(diff < 0 ? -diff : diff);
    }
  }
  return sum;
}

/* checked_scaled_add (:780-795) on the u32 range the records carry. */
static uint32_t scaled(uint32_t v, uint32_t times) { return v * times; }

/* The words of one row's trace and of its relation trace (0 unless a relation read): the
 * traced evaluation's layout (:293-297, :1474-1478). */
static uint32_t trace_words(const uor_d11_model *m) {
  return m->blocks * (m->read_mode == UOR_D11_READ_ROUTE
                          ? UOR_D11_ROUTE_TRACE_HEADER_WORDS + m->stages * UOR_D11_ROUTE_TRACE_STAGE_WORDS
                          : UOR_D11_ACTIVE_TRACE_HEADER_WORDS + m->stages * UOR_D11_ACTIVE_TRACE_LEVEL_WORDS);
}

static int max_nodes(const uor_d11_model *m) {
  static __thread Plan p;
  return build_row_plan((int)m->context, &p) == 0 ? p.count : 0;
}

/* evaluate_prefix_internal (:1772-1890) and observe_target (:1892-1993) of one row; with
 * `trace`, evaluate_prefix_traced's words (rel_trace: blocks x rel_stride). */
static void score_row(const Oracle *o, const uint32_t *prefix, int length, uint32_t target,
                      uor_d11_row_out *out, int32_t *rel_out, uint32_t *trace, uint32_t *rel_trace,
                      int rel_stride) {
  const uor_d11_model *m = o->m;
  memset(out, 0, sizeof *out);
  if (trace)
    for (uint32_t i = 0; i < trace_words(m); i++) trace[i] = UINT32_MAX;
  if (rel_trace)
    for (uint32_t i = 0; i < m->blocks * (uint32_t)rel_stride; i++) rel_trace[i] = UINT32_MAX;
  if (length < 1 || length > (int)m->context) {
    out->status = UOR_D11_ROW_PREFIX_LENGTH;
    return;
  }
  for (int i = 0; i < length; i++)
    if (prefix[i] >= m->vocabulary) {
      out->status = UOR_D11_ROW_PREFIX_TOKEN;
      return;
    }
  if (target >= m->vocabulary) {
    out->status = UOR_D11_ROW_TARGET_TOKEN;
    return;
  }
  static __thread Plan plan;
  build_row_plan(length, &plan);
  Vec8 q[UOR_D11_MAX_BLOCKS];
  const int relation = m->read_mode == UOR_D11_READ_RELATION;
  int st = m->read_mode == UOR_D11_READ_ROUTE
               ? route_read(m, prefix, length, &plan, q, o->knockout, trace)
               : flock_or_relation_read(m, prefix, length, &plan, (int)m->read_kept,
                                        relation ? (int)m->read_sweeps : 0, relation, q, rel_out,
                                        trace, relation ? rel_trace : NULL, rel_stride);
  if (st == UOR_D11_ROW_OK && o->trunk && !o->knockout) st = trunk_gate(o, prefix, length, q);
  if (st != UOR_D11_ROW_OK) {
    out->status = st;
    return;
  }
  uint8_t occupied[256] = {0}, used[256] = {0};
  for (uint32_t t = 0; t < m->vocabulary; t++) occupied[m->cells[t]] = 1;
  uint32_t admitted[16];
  int na = 0;
  for (uint32_t k = 0; k < m->kept_cells; k++) {
    int best = -1;
    uint32_t cost = UINT32_MAX;
    for (uint32_t c = 0; c < 256; c++)
      if (occupied[c] && !used[c]) {
        uint32_t d = address_distance(m, q, c);
        if (d < cost || (d == cost && (best < 0 || (int)c < best))) {
          best = (int)c;
          cost = d;
        }
      }
    if (best < 0) break;
    used[best] = 1;
    admitted[na++] = (uint32_t)best;
  }
  uint32_t ranked[8], distance[8];
  for (int k = 0; k < 8; k++) ranked[k] = distance[k] = UINT32_MAX;
  int found = 0;
  for (uint32_t tok = 0; tok < m->vocabulary; tok++) {
    int in = 0;
    for (int k = 0; k < na; k++) in |= admitted[k] == m->cells[tok];
    if (!in) continue;
    uint32_t d = token_distance(m, q, tok);
    int at = found;
    while (at > 0) {
      int pv = at - 1;
      if (!(d < distance[pv] || (d == distance[pv] && tok < ranked[pv]))) break;
      if (at < 8) {
        ranked[at] = ranked[pv];
        distance[at] = distance[pv];
      }
      at--;
    }
    if (at < 8) {
      ranked[at] = tok;
      distance[at] = d;
      if (found < 8) found++;
    }
  }
  for (uint32_t b = 0; b < m->blocks; b++) memcpy(out->read_vector + 8 * b, q[b].x, 32);
  out->admitted_count = na;
  for (int k = 0; k < na; k++) out->admitted[k] = admitted[k];
  if (found == 0) { /* evaluate_prefix fails: the record holds the status alone */
    memset(out, 0, sizeof *out);
    out->status = UOR_D11_ROW_ZERO_TOKENS;
    return;
  }
  out->top8_count = found;
  for (int k = 0; k < found; k++) out->top8[k] = ranked[k];
  out->prediction = ranked[0];
  /* observe_target */
  uint32_t tcell = m->cells[target], trivals = 0, arivals = 0;
  uint32_t rival_d = UINT32_MAX, rival_a = UINT32_MAX;
  for (int k = 0; k < na; k++) {
    uint32_t cell = admitted[k], cost = address_distance(m, q, cell);
    if (cell != tcell) {
      arivals++;
      if (cost < rival_a) rival_a = cost;
    }
    for (uint32_t tok = 0; tok < m->vocabulary; tok++)
      if (m->cells[tok] == cell && tok != target) {
        trivals++;
        uint32_t d = token_distance(m, q, tok);
        if (d < rival_d) rival_d = d;
      }
  }
  uint32_t width = m->blocks << 3;
  uint32_t td = token_distance(m, q, target), ad = address_distance(m, q, tcell);
  uint32_t th = (rival_d == UINT32_MAX || width + td <= rival_d) ? 0 : width + td - rival_d;
  uint32_t ah = (rival_a == UINT32_MAX || 8 + ad <= rival_a) ? 0 : 8 + ad - rival_a;
  uint32_t rank = 1;
  for (uint32_t c = 0; c < 256; c++)
    if (occupied[c]) {
      uint32_t d = address_distance(m, q, c);
      if (d < ad || (d == ad && c < tcell)) rank++;
    }
  uint32_t rh = rank > m->kept_cells ? rank - m->kept_cells : 0;
  out->token_rivals = trivals;
  out->address_rivals = arivals;
  out->token_hinge = th;
  out->address_hinge = ah;
  out->rank_hinge = rh;
  out->loss_ta = scaled(th, 8) + scaled(ah, width);
  out->loss_tr = scaled(th, 8) + scaled(rh, width);
  out->selected_loss =
      m->objective_policy == UOR_D11_POLICY_OCCUPIED_CELL_RANK ? out->loss_tr : out->loss_ta;
}

static void oracle_init(Oracle *o, const uor_d11_model *m) {
  memset(o, 0, sizeof *o);
  o->m = m;
  o->trunk = m->trunk != NULL;
  o->knockout = (m->flags & UOR_D11_FLAG_STATE_TRANSPORT_KNOCKOUT) != 0;
  if (o->knockout) {
    size_t nr = (size_t)m->blocks * m->stages;
    size_t ng = nr + (m->read_mode == UOR_D11_READ_RELATION ? (size_t)m->stages * EDGE_TYPES : 0);
    o->kroutes = (uint32_t *)calloc(nr ? nr : 1, sizeof(uint32_t)); /* IDENTITY = 0 (:278) */
    o->kgates = (int32_t *)calloc(ng ? ng : 1, sizeof(int32_t));
    o->km = *m;
    o->km.routes = o->kroutes;
    o->km.gates = o->kgates;
    o->m = &o->km;
  }
  if (o->trunk) {
    for (int i = 0; i < 12; i++) sparse_build(&o->sp[i], m->trunk->sparse[i], m->trunk->sparse_rows[i]);
    o->roots4 = (uint8_t(*)[4])malloc((size_t)m->vocabulary * 4);
    for (uint32_t t = 0; t < m->vocabulary; t++)
      for (int b = 0; b < 4; b++) o->roots4[t][b] = (uint8_t)root_id(token_block(m, t, b));
  }
}

static void oracle_free(Oracle *o) {
  free(o->kroutes);
  free(o->kgates);
  if (o->trunk) {
    for (int i = 0; i < 12; i++) {
      free(o->sp[i].pairs);
      free(o->sp[i].counts);
    }
    free(o->roots4);
  }
}

typedef struct {
  const Oracle *o;
  const uint32_t *prefixes;
  const int32_t *lengths;
  const uint32_t *targets;
  uint32_t rows, stride, start, step;
  uor_d11_row_out *out;
  uint32_t *trace, *rel_trace; /* NULL: untraced */
  uint32_t trace_words;
  int rel_stride;
} Job;

static void *run_job(void *arg) {
  Job *j = (Job *)arg;
  const uint32_t B = j->o->m->blocks;
  for (uint32_t r = j->start; r < j->rows; r += j->step)
    score_row(j->o, j->prefixes + (size_t)r * j->stride, j->lengths[r], j->targets[r], j->out + r,
              NULL, j->trace ? j->trace + (size_t)r * j->trace_words : NULL,
              j->rel_trace ? j->rel_trace + (size_t)r * B * j->rel_stride : NULL, j->rel_stride);
  return NULL;
}

/* Every row, spread over `threads` POSIX threads (<= 0: one). */
int d11_oracle_score_rows(const uor_d11_model *m, const uint32_t *prefixes, const int32_t *lengths,
                          const uint32_t *targets, uint32_t rows, uint32_t stride,
                          uor_d11_row_out *out, int threads) {
  Oracle o;
  oracle_init(&o, m);
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  Job jobs[64];
  for (int t = 0; t < threads; t++) {
    jobs[t] = (Job){&o, prefixes, lengths, targets, rows, stride, (uint32_t)t, (uint32_t)threads, out,
                    NULL, NULL, 0, 0};
    if (t > 0) pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  run_job(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(th[t], NULL);
  oracle_free(&o);
  return 0;
}

/* A loaded oracle (the model and its sorted trunk tables, as from_bytes builds them once), so
 * that timing covers the rows alone. */
void *d11_oracle_open(const uor_d11_model *m) {
  Oracle *o = (Oracle *)malloc(sizeof(Oracle));
  oracle_init(o, m);
  return o;
}

void d11_oracle_close(void *h) {
  oracle_free((Oracle *)h);
  free(h);
}

int d11_oracle_score_open(void *h, const uint32_t *prefixes, const int32_t *lengths,
                          const uint32_t *targets, uint32_t rows, uint32_t stride,
                          uor_d11_row_out *out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  Job jobs[64];
  for (int t = 0; t < threads; t++) {
    jobs[t] = (Job){(const Oracle *)h, prefixes, lengths, targets, rows, stride, (uint32_t)t,
                    (uint32_t)threads, out, NULL, NULL, 0, 0};
    if (t > 0) pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  run_job(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(th[t], NULL);
  return 0;
}

/* One row with its relation scores (blocks x node count of the row's plan), as
 * DiscretePrefixEvaluation::relation_scores (:386-388). Returns the node count. */
int d11_oracle_row_relation(const uor_d11_model *m, const uint32_t *prefix, int32_t length,
                            uint32_t target, uor_d11_row_out *out, int32_t *relation_scores) {
  Oracle o;
  oracle_init(&o, m);
  score_row(&o, prefix, length, target, out, relation_scores, NULL, NULL, 0);
  oracle_free(&o);
  Plan p;
  return build_row_plan(length, &p) == 0 ? p.count : 0;
}

/* build_row_plan's node count and frontier length (fbs_binder_summary, :905-910). */
int d11_oracle_plan(int32_t length, int32_t *nodes, int32_t *frontier) {
  Plan p;
  if (build_row_plan(length, &p)) return -1;
  *nodes = p.count;
  *frontier = p.frontier_len;
  return 0;
}

/* The words of one row's trace and, in `*relation_words`, of its relation trace (blocks x a
 * full context's node count; 0 unless a relation read). */
uint32_t d11_oracle_trace_words(const uor_d11_model *m, uint32_t *relation_words) {
  *relation_words = m->read_mode == UOR_D11_READ_RELATION ? m->blocks * (uint32_t)max_nodes(m) : 0;
  return trace_words(m);
}

/* evaluate_prefix_traced (:1768-1770) and observe_target for every row: the records, `trace`
 * rows x d11_oracle_trace_words words and, for a relation read, `relation_trace` rows x its
 * relation words (NULL: not wanted). A row whose status is not 0 has no trace (the reference
 * returns an error); its words are unspecified. */
int d11_oracle_score_rows_traced(const uor_d11_model *m, const uint32_t *prefixes,
                                 const int32_t *lengths, const uint32_t *targets, uint32_t rows,
                                 uint32_t stride, uor_d11_row_out *out, uint32_t *trace,
                                 uint32_t *relation_trace, int threads) {
  Oracle o;
  oracle_init(&o, m);
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  Job jobs[64];
  const int rel_stride = m->read_mode == UOR_D11_READ_RELATION ? max_nodes(m) : 0;
  for (int t = 0; t < threads; t++) {
    jobs[t] = (Job){&o, prefixes, lengths, targets, rows, stride, (uint32_t)t, (uint32_t)threads, out,
                    trace, rel_stride ? relation_trace : NULL, trace_words(m), rel_stride};
    if (t > 0) pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  run_job(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(th[t], NULL);
  oracle_free(&o);
  return 0;
}
