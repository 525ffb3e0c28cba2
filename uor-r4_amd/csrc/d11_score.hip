// d11_score.hip - the discrete M1 row scorer on MI355X: IntegerDiscreteModel::evaluate_prefix
// and observe_target (crates/uor-r4-integer/src/discrete_d11.rs:1761-1995) for a panel of
// (prefix, target) rows, the work of the reference's d11_score_rows
// (docs/labs/m1-d11-artifact-scorer/instrument/src/scorer.cu:12-41, one thread per row with a
// 22.5 KB scratch record in global memory).
//
// Here one wavefront scores one row, four rows per block. Every block of the discrete table is
// one of the 16 orbit roots (the loader refuses anything else), so the kernel works on root ids:
// a route state applied to a root, the snap of three carried roots, and the L1 and Hamming
// distances between roots are tables built once per model (from the same definitions the
// oracle restates) and staged into LDS with the 64 x 64 state product. Per block of the read:
//   - the binder tree is folded level by level, the lanes taking a level's nodes in parallel;
//   - the relation read's edges visit at most one parent, one sibling pair, one left neighbour,
//     the previous atom with the same token and the previous node of the level with the same
//     frame; the first three come from the row plan, the last two are found per row with
//     ballots (the reference's O(nodes^2) scans, same result);
//   - each level's kept nodes are the top keys of (relation score, distance, Hamming, last
//     position, node) packed into 64 bits, chosen by wave-wide maxima;
// the trunk's recurrence code is a segmented scan of route-state products (16 lanes per block);
// the trunk's sparse count tables are sorted (key, token) arrays searched by halves; the
// writer admits cells and ranks their tokens with wave-wide minima of packed keys.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/uor_d11.h"
#include "d11_tables.h"

namespace d11 {

constexpr int kWaves = 8;  // rows per block
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxNodes = 512;
constexpr int kMaxLevels = 8;
constexpr int kPerLane = kMaxNodes / 64;  // a level's nodes per lane
constexpr uint32_t kNone = 0x1ff;
constexpr int kRecWords = sizeof(uor_d11_row_out) / 4;
static_assert(sizeof(uor_d11_row_out) == 656, "record layout");

// One prefix length's binder tree (build_row_plan, discrete_d11.rs:813-884) with the
// neighbours the relation read's edges use.
struct Plan {
  uint16_t count, frontier_len;
  uint16_t level_start[kMaxLevels + 1];  // nodes of level l: order[level_start[l] ..)
  uint16_t frontier[16];
  uint32_t node[kMaxNodes];   // c0 | c1 << 9 | c2 << 18 | level << 27 | inner << 30 (atom: c0)
  uint32_t link[kMaxNodes];   // first | last << 8 | parent << 16 | slot in parent << 25
  uint16_t left[kMaxNodes];   // the same-level node ending just before this one, or 0xffff
  uint16_t order[kMaxNodes];  // nodes by (level, index)
};

// Root-id tables of the geometry (derived from d11_tables.h at model creation).
struct Geo {
  uint8_t act[64][16];    // root id of route state a applied to root r
  uint8_t snap3[4096];    // snap(root i + root j + root k, 3)
  uint8_t dist[16][16];   // L1 distance between roots
  uint8_t ham[16][16];    // coordinates that differ
  uint8_t bfs[256];
  uint8_t branch[16][4];
  uint8_t compose[64][64];  // state a after state b
  int8_t roots[16][8];
};
static_assert(sizeof(Geo) % 4 == 0, "staged in words");

// The trunk's sparse tables the evaluation reads, in this order.
enum { S_QUERY = 0, S_QUERY_READ, S_READ, S_QUERY_REC, S_READ_REC, S_REC, kSparse };
constexpr int kSparseSource[kSparse] = {7, 8, 0, 9, 2, 1};  // index in the container's 12

struct DevModel {
  uint32_t vocab, blocks, context, kept_cells, stages, read_mode, read_kept, read_sweeps, policy;
  uint32_t trunk, unigram_best;
  uint32_t knockout;    // with_state_transport_knockout: routes and gates already zeroed
  uint32_t trace_block;  // trace words per block of the read
  uint32_t rel_stride;   // relation trace words per block: a full context's node count
  uint32_t occupied[8];
  const Geo *geo;
  const uint8_t *troot;      // [vocab][blocks] root ids
  const uint8_t *cell;       // [vocab]
  const uint32_t *cell_off;  // [257]
  const uint16_t *cell_tok;  // [vocab], each cell's tokens ascending
  const uint8_t *routes;     // [blocks][stages]
  const int8_t *gates;       // [blocks][stages] then [stages][5]
  const Plan *plans;         // [context], prefix lengths 1..context
  const uint32_t *unigram;   // [vocab]
  const uint16_t *code4;     // [vocab] the four block roots packed 4 bits each
  const uint8_t *step;       // [64]
  const uint8_t *norm;       // [4]
  const uint64_t *pairs[kSparse];  // key << 32 | token, ascending
  const uint32_t *counts[kSparse];
  const uint32_t *bucket[kSparse];  // [65537]: first entry whose key >> shift is >= b
  uint64_t rows[kSparse];
};
// Bucket shift per table: the 16-bit keys (token, read code, recurrence code) index their
// buckets directly; the composite keys bucket by their high half.
constexpr int kBucketShift[kSparse] = {0, 16, 0, 16, 16, 0};
constexpr uint32_t kBuckets = 65536;

struct WaveLds {
  uint16_t tok[256];
  int16_t prevocc[256];  // node of the previous atom with the same token, -1 none
  uint8_t frame[kMaxNodes];
  uint8_t payload[kMaxNodes];
  int32_t prev[kMaxNodes];
  int32_t rel[kMaxNodes];
  int16_t samef[kMaxNodes];  // previous node of the level with the same frame, -1 none
  uint32_t rec[kRecWords];   // the record: admitted cells and top 8 are kept here as found
  uint8_t qroot[UOR_D11_MAX_BLOCKS];  // the read, one root per block
  int16_t lastf[16];                  // a level's last node so far, per frame
  uint64_t tokbits[4][14];            // per 64 positions: the tokens' 13 bit planes, then valid
};

// Lanes whose value equals this lane's, from the bit-plane ballots of a 64-lane group.
template <int BITS>
__device__ __forceinline__ uint64_t same_as(uint32_t v, const uint64_t *planes, uint64_t valid) {
  uint64_t m = valid;
#pragma unroll
  for (int k = 0; k < BITS; k++) m &= (v >> k & 1) ? planes[k] : ~planes[k];
  return m;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-wide reductions: butterflies inside each row of 16 lanes through DPP, then the four rows'
// results read as scalars (uniform). Every lane must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t lane32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
constexpr int kXor1 = 0xb1, kXor2 = 0x4e, kHalfMirror = 0x141, kMirror = 0x140;

#define D11_WAVE_REDUCE32(NAME, OP)                                                   \
  __device__ __forceinline__ uint32_t NAME(uint32_t v) {                              \
    v = OP(v, dpp32<kXor1>(v));                                                       \
    v = OP(v, dpp32<kXor2>(v));                                                       \
    v = OP(v, dpp32<kHalfMirror>(v));                                                 \
    v = OP(v, dpp32<kMirror>(v));                                                     \
    return OP(OP(lane32(v, 0), lane32(v, 16)), OP(lane32(v, 32), lane32(v, 48)));    \
  }
__device__ __forceinline__ uint32_t op_min(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t op_max(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t op_add(uint32_t a, uint32_t b) { return a + b; }
D11_WAVE_REDUCE32(wave_min32, op_min)
D11_WAVE_REDUCE32(wave_max32, op_max)
D11_WAVE_REDUCE32(wave_sum32, op_add)
#undef D11_WAVE_REDUCE32

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  return (uint64_t)dpp32<CTRL>((uint32_t)(v >> 32)) << 32 | dpp32<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t lane64(uint64_t v, int l) {
  return (uint64_t)lane32((uint32_t)(v >> 32), l) << 32 | lane32((uint32_t)v, l);
}
__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
  v = max64(v, dpp64<kXor1>(v));
  v = max64(v, dpp64<kXor2>(v));
  v = max64(v, dpp64<kHalfMirror>(v));
  v = max64(v, dpp64<kMirror>(v));
  return max64(max64(lane64(v, 0), lane64(v, 16)), max64(lane64(v, 32), lane64(v, 48)));
}

// snap(x, n) (discrete_d11.rs:755-778) over the wave: lane r < 16 scores root r; the least
// (distance, Hamming, root) wins.
__device__ __forceinline__ int snap_wave(const Geo &g, const int32_t *x, int n, int lane) {
  uint32_t key = 0xffffffffu;
  if (lane < 16) {
    uint32_t dist = 0, ham = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const int32_t y = n * (int32_t)g.roots[lane][d];
      const int32_t e = x[d] - y;
      dist += (uint32_t)(e < 0 ? -e : e);
      ham += x[d] != y;
    }
    key = dist << 12 | ham << 8 | (uint32_t)lane;
  }
  return (int)(wave_min32(key) & 0xff);
}

// The same in one lane.
__device__ __forceinline__ int snap_lane(const Geo &g, const int32_t *x, int n) {
  uint32_t best = 0xffffffffu;
  for (int r = 0; r < 16; r++) {
    uint32_t dist = 0, ham = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const int32_t y = n * (int32_t)g.roots[r][d];
      const int32_t e = x[d] - y;
      dist += (uint32_t)(e < 0 ? -e : e);
      ham += x[d] != y;
    }
    best = min(best, dist << 12 | ham << 8 | (uint32_t)r);
  }
  return (int)(best & 0xff);
}

__device__ __forceinline__ uint64_t lower_bound64(const uint64_t *a, uint64_t n, uint64_t x) {
  uint64_t lo = 0, hi = n;
  while (lo < hi) {
    const uint64_t mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

__device__ void write_error(uor_d11_row_out *o, int status, int lane) {
  uint32_t *w = (uint32_t *)o;
  for (int i = lane; i < kRecWords; i += 64) w[i] = i == 0 ? (uint32_t)status : 0u;
}

// route_read (discrete_d11.rs:1337-1451) of block b; -1 when the route ends off a leaf. TR:
// the block's trace words at `tw` (header, then 6 words a stage, discrete_d11.rs:1369-1442).
template <bool TR>
__device__ int route_block(const DevModel &M, const Geo &g, const Plan &P, const WaveLds &w,
                           int len, int b, int lane, uint32_t *tw) {
  const int B = (int)M.blocks, S = (int)M.stages;
  const int qr0 = M.troot[(uint32_t)w.tok[len - 1] * B + b];
  if (M.knockout) {  // the last token's block, untransported (:1346-1361)
    if (TR)
      for (int i = lane; i < 4 + 6 * S; i += 64)
        tw[i] = i == 0 ? (uint32_t)P.frontier_len : i == 1 ? (uint32_t)qr0 : i == 2 ? 0u : 0xffffffffu;
    return qr0;
  }
  int node = 0, root = 0, total = 0;
  for (int stage = 0; stage < S; stage++) {
    const int frame = M.routes[b * S + stage];
    const int qr = g.act[frame][qr0];
    const int count = stage == 0 ? P.frontier_len : 3;
    uint32_t key = 0xffffffffu;
    if (lane < count) {
      const int r = stage == 0 ? lane : g.branch[root][lane];
      key = (uint32_t)g.dist[qr][r] << 16 | (uint32_t)g.ham[qr][r] << 8 | (uint32_t)lane;
    }
    const int best = (int)(wave_min32(key) & 0xff);
    const int goal = stage == 0 ? best : g.branch[root][best];
    const int from = root;
    total = g.compose[g.bfs[(root << 4) + goal]][total];
    root = goal;
    int next;
    if (stage == 0) {
      next = P.frontier[best];
    } else {
      const uint32_t nd = P.node[node];
      if (!(nd >> 30 & 1)) return -1;  // stepped past an atom leaf
      next = (int)(nd >> (9 * best) & kNone);
    }
    if (TR && lane < 6) {
      const uint32_t v[6] = {(uint32_t)frame, (uint32_t)from, (uint32_t)best, (uint32_t)goal,
                             (uint32_t)total, (uint32_t)next};
      uint32_t x = v[0];
#pragma unroll
      for (int k = 1; k < 6; k++) x = lane == k ? v[k] : x;
      tw[4 + 6 * stage + lane] = x;
    }
    const uint32_t nn = P.node[next];
    if (!(nn >> 30 & 1)) {
      const int carrier = M.troot[(uint32_t)w.tok[nn & kNone] * B + b];
      const int r = g.act[total][carrier];
      if (TR) {
        // The header, and the stages not taken.
        for (int i = lane; i < 6 * (S - stage - 1); i += 64) tw[4 + 6 * (stage + 1) + i] = 0xffffffffu;
        if (lane < 4)
          tw[lane] = lane == 0   ? (uint32_t)P.frontier_len
                     : lane == 1 ? (uint32_t)r
                     : lane == 2 ? (uint32_t)(stage + 1)
                                 : (nn & kNone);
      }
      return r;
    }
    node = next;
  }
  return -1;
}

// flock_or_relation_read (discrete_d11.rs:1453-1741) of block b. TR: the block's trace words
// at `tw` (header, then 28 words a level, every level visited whatever its gate, :1480-1738)
// and, for the relation read, its scores at `rw` padded to M.rel_stride (:1640-1644).
template <bool TR>
__device__ int flock_block(const DevModel &M, const Geo &g, const Plan &P, WaveLds &w, int len,
                           int b, bool relation, int lane, uint32_t *tw, uint32_t *rw) {
  const int B = (int)M.blocks, S = (int)M.stages;
  const int f = b == 0 ? B - 1 : 0;
  const uint32_t last = w.tok[len - 1];
  const int qf = M.troot[last * B + f];
  const int count = P.count;
  // Level by level: atoms take their token's roots; an inner node the snap of its children's
  // payloads carried into the first child's frame.
  for (int k = P.level_start[0] + lane; k < P.level_start[1]; k += 64) {
    const int i = P.order[k];
    const uint32_t t = w.tok[P.node[i] & kNone];
    w.frame[i] = M.troot[t * B + f];
    w.payload[i] = M.troot[t * B + b];
  }
  for (int l = 1; l < kMaxLevels && P.level_start[l] < P.level_start[l + 1]; l++) {
    wave_sync();
    for (int k = P.level_start[l] + lane; k < P.level_start[l + 1]; k += 64) {
      const int i = P.order[k];
      const uint32_t nd = P.node[i];
      const int c0 = nd & kNone, c1 = nd >> 9 & kNone, c2 = nd >> 18 & kNone;
      const int f0 = w.frame[c0];
      const int p0 = g.act[g.bfs[(f0 << 4) + f0]][w.payload[c0]];
      const int p1 = g.act[g.bfs[(w.frame[c1] << 4) + f0]][w.payload[c1]];
      const int p2 = g.act[g.bfs[(w.frame[c2] << 4) + f0]][w.payload[c2]];
      w.frame[i] = (uint8_t)f0;
      w.payload[i] = g.snap3[p0 << 8 | p1 << 4 | p2];
    }
  }
  wave_sync();
  if (relation) {
    const int8_t *rg = M.gates + B * S;
    for (int i = lane; i < count; i += 64) {
      w.prev[i] = 8 - (int32_t)g.dist[qf][w.frame[i]];
      w.rel[i] = 0;
    }
    // Previous node of the same level with the same frame (edge type 4, only on levels whose
    // gate uses it), 64 nodes at a time: the frame's four bit planes as ballots give each lane
    // the lanes holding its frame; the nearest lower one, else the level's last node with that
    // frame in earlier chunks (kept per frame in LDS).
    const uint64_t lt = (1ull << lane) - 1, gt_mask = ~lt & ~(1ull << lane);
    for (int l = 0; l < S && P.level_start[l] < P.level_start[l + 1]; l++) {
      if (rg[l * 5 + 4] == 0) continue;
      if (lane < 16) w.lastf[lane] = -1;
      wave_sync();
      for (int c = P.level_start[l]; c < P.level_start[l + 1]; c += 64) {
        const int k = c + lane;
        const bool valid = k < P.level_start[l + 1];
        const int i = valid ? P.order[k] : 0;
        const uint32_t fr = valid ? w.frame[i] : 0u;
        uint64_t planes[4];
#pragma unroll
        for (int bit = 0; bit < 4; bit++) planes[bit] = __ballot(fr >> bit & 1);
        const uint64_t same = same_as<4>(fr, planes, __ballot(valid));
        const uint64_t below = same & lt;
        const int src = below ? 63 - __clzll(below) : lane;
        const int from = __shfl(i, src, 64);
        const int seen = valid ? w.lastf[fr] : -1;
        if (valid) w.samef[i] = (int16_t)(below ? from : seen);
        wave_sync();
        if (valid && !(same & gt_mask)) w.lastf[fr] = (int16_t)i;
        wave_sync();
      }
    }
    wave_sync();
    for (uint32_t sw = 0; sw < M.read_sweeps; sw++) {
      for (int i = lane; i < count; i += 64) {
        const uint32_t nd = P.node[i], lk = P.link[i];
        const int li = nd >> 27 & 7;
        const bool inner = nd >> 30 & 1;
        const int parent = lk >> 16 & kNone, slot = lk >> 25 & 3;
        int32_t acc = w.rel[i];
#pragma unroll
        for (int e = 0; e < 5; e++) {
          const int gt = rg[li * 5 + e];
          if (gt == 0) continue;
          int32_t es = 0;
          if (e == 0) {
            if (inner) es = w.prev[nd & kNone] + w.prev[nd >> 9 & kNone] + w.prev[nd >> 18 & kNone];
            if (parent != (int)kNone) es += w.prev[parent];
          } else if (e == 1) {
            if (parent != (int)kNone) {
              const uint32_t pn = P.node[parent];
              const int a = pn & kNone, m1 = pn >> 9 & kNone, z = pn >> 18 & kNone;
              es = slot == 1 ? w.prev[a] + w.prev[z] : w.prev[m1];
            }
          } else if (e == 2) {
            const int j = P.left[i];
            if (j != 0xffff) es = w.prev[j];
          } else if (e == 3) {
            if (li == 0) {
              const int j = w.prevocc[nd & kNone];
              if (j >= 0) es = w.prev[j];
            }
          } else {
            const int j = w.samef[i];
            if (j >= 0) es = w.prev[j];
          }
          acc += gt > 0 ? es : -es;
        }
        w.rel[i] = acc;
      }
      wave_sync();
      for (int i = lane; i < count; i += 64) w.prev[i] = w.rel[i];
      wave_sync();
    }
    if (TR)
      for (int i = lane; i < (int)M.rel_stride; i += 64) rw[i] = i < count ? (uint32_t)w.rel[i] : 0xffffffffu;
  }
  // Per level with a gate: the kept nodes (best first) carried into the query frame.
  int32_t u[8];
  const int u0 = M.troot[last * B + b];
#pragma unroll
  for (int d = 0; d < 8; d++) u[d] = g.roots[u0][d];
  int terms = 1;
  const int kept = (int)M.read_kept;
  for (int l = 0; l < S; l++) {
    const int gate = M.gates[b * S + l];
    if (!TR && gate == 0) continue;
    uint64_t mk[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; j++) {
      mk[j] = 0;
      const int k = P.level_start[l] + lane + 64 * j;
      if (l < kMaxLevels && k < P.level_start[l + 1]) {
        const int i = P.order[k];
        const uint32_t lst = P.link[i] >> 8 & 0xff;
        if ((int)lst + 1 < len) {
          const int fr = w.frame[i];
          const uint32_t r = relation ? (uint32_t)w.rel[i] ^ 0x80000000u : 0x80000000u;
          mk[j] = (uint64_t)r << 32 | (uint64_t)(15 - g.dist[qf][fr]) << 28 |
                  (uint64_t)(15 - g.ham[qf][fr]) << 24 | (uint64_t)lst << 16 |
                  (uint64_t)(kNone - (uint32_t)i);
        }
      }
    }
    int32_t sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int found = 0;
    // Only the kept set enters the sum: when the eligible nodes fit, take them all.
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < kPerLane; j++) mine += mk[j] != 0;
    const uint32_t eligible = wave_sum32(mine);
    // The level's trace word this lane writes: kept nodes at 4 + k, their route states at 12 + k,
    // the carried roots at 20 + k, in selection order (the ordered selection always runs).
    uint32_t tv = 0xffffffffu;
    if (!TR && (int)eligible <= kept) {
#pragma unroll
      for (int j = 0; j < kPerLane; j++) {
        if (mk[j]) {
          const int node = (int)(kNone - (uint32_t)(mk[j] & kNone));
          const int cr = g.act[g.bfs[(w.frame[node] << 4) + qf]][w.payload[node]];
#pragma unroll
          for (int d = 0; d < 8; d++) sum[d] += g.roots[cr][d];
        }
      }
#pragma unroll
      for (int d = 0; d < 8; d++) sum[d] = (int32_t)wave_sum32((uint32_t)sum[d]);
      found = (int)eligible;
    }
    for (int r = 0; (TR || (int)eligible > kept) && r < kept; r++) {
      uint64_t loc = 0;
#pragma unroll
      for (int j = 0; j < kPerLane; j++) loc = mk[j] > loc ? mk[j] : loc;
      const uint64_t m = wave_max64(loc);
      if (m == 0) break;
#pragma unroll
      for (int j = 0; j < kPerLane; j++)
        if (mk[j] == m) mk[j] = 0;
      const int node = (int)(kNone - (uint32_t)(m & kNone));
      const int act = g.bfs[(w.frame[node] << 4) + qf];
      const int cr = g.act[act][w.payload[node]];
      if (TR) tv = lane == 4 + r ? (uint32_t)node : lane == 12 + r ? (uint32_t)act : lane == 20 + r ? (uint32_t)cr : tv;
#pragma unroll
      for (int d = 0; d < 8; d++) sum[d] += g.roots[cr][d];
      found++;
    }
    if (TR && lane < 28 && lane != 2)
      tw[4 + 28 * l + lane] = lane == 0 ? (uint32_t)(gate + 1) : lane == 1 ? (uint32_t)found
                              : lane == 3 ? eligible : tv;
    if (found == 0) {
      if (TR && lane == 2) tw[4 + 28 * l + 2] = 0xffffffffu;
      continue;
    }
    const int mroot = snap_wave(g, sum, found, lane);
    if (TR && lane == 2) tw[4 + 28 * l + 2] = (uint32_t)mroot;
    if (TR && gate == 0) continue;
#pragma unroll
    for (int d = 0; d < 8; d++) u[d] += gate > 0 ? g.roots[mroot][d] : -g.roots[mroot][d];
    terms++;
  }
  const int out = snap_wave(g, u, terms, lane);
  if (TR && lane < 4) tw[lane] = lane == 0 ? (uint32_t)qf : lane == 1 ? (uint32_t)out : lane == 2 ? (uint32_t)terms : (uint32_t)u0;
  return out;
}

// p / c for 0 <= p < 256 and 1 <= c <= 16 by restoring subtraction: the kernels divide by no
// variable with the compiler's `/`, whose expansion goes through a float reciprocal estimate.
__device__ __forceinline__ int div_small(int p, int c) {
  int q = 0;
#pragma unroll
  for (int k = 7; k >= 0; k--)
    if (p >= (c << k)) {
      p -= c << k;
      q |= 1 << k;
    }
  return q;
}

// The trunk's joint-pointer gate (discrete_d11.rs:463-685): the recurrence code from the
// products of step states over the prefix, the causal pointer successor, the best token of the
// sparse counts, and each read block carried to that token's root.
__device__ void trunk_gate(const DevModel &M, const Geo &g, WaveLds &w, int len, int lane) {
  uint8_t *qroot = w.qroot;
  const int last = len - 1, pprev = last > 0 ? last - 1 : 0, pmid = last / 2;
  uint32_t read_code = 0;
#pragma unroll
  for (int b = 0; b < 4; b++) read_code |= (uint32_t)qroot[b] << (4 * b);
  // compute_rec_code (:601-644): lanes 16 b .. 16 b + 15 hold block b, each a run of positions.
  const int seg = lane >> 4, sl = lane & 15;
  const int ch = (len + 15) >> 4;
  const int lo = sl * ch, hi = min(lo + ch, len);
  int acc = 0, part_prev = 0, part_mid = 0, part_last = 0;
  for (int p = lo; p < hi; p++) {
    const int r = M.code4[w.tok[p]] >> (4 * seg) & 15;
    acc = g.compose[M.step[(seg << 4) + r]][acc];
    if (p == pprev) part_prev = acc;
    if (p == pmid) part_mid = acc;
    if (p == last) part_last = acc;
  }
  int incl = acc;
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) {
    const int o = __shfl_up(incl, d, 16);
    if (sl >= d) incl = g.compose[incl][o];
  }
  int excl = __shfl_up(incl, 1, 16);
  if (sl == 0) excl = 0;
  const int a_prev = __shfl(g.compose[part_prev][excl], (seg << 4) + div_small(pprev, ch), 64);
  const int a_mid = __shfl(g.compose[part_mid][excl], (seg << 4) + div_small(pmid, ch), 64);
  const int f_last = __shfl(g.compose[part_last][excl], (seg << 4) + div_small(last, ch), 64);
  const int inv_prev = g.compose[a_prev][g.compose[a_prev][a_prev]];
  const int inv_mid = g.compose[a_mid][g.compose[a_mid][a_mid]];
  const int h_prev = g.compose[f_last][inv_prev], h_mid = g.compose[f_last][inv_mid];
  const int rl = M.code4[w.tok[last]] >> (4 * seg) & 15;
  const int rp = M.code4[w.tok[pprev]] >> (4 * seg) & 15;
  const int rm = M.code4[w.tok[pmid]] >> (4 * seg) & 15;
  const int rs = M.code4[w.tok[0]] >> (4 * seg) & 15;
  const int pr = g.act[h_prev][rp], mr = g.act[h_mid][rm], fr = g.act[f_last][rs];
  int32_t sum[8];
#pragma unroll
  for (int d = 0; d < 8; d++)
    sum[d] = g.roots[rl][d] + g.roots[pr][d] + g.roots[mr][d] + g.roots[fr][d];
  const int nr = g.act[M.norm[seg]][snap_lane(g, sum, 4)];
  uint32_t rec_code = 0;
#pragma unroll
  for (int b = 0; b < 4; b++) rec_code |= (uint32_t)__shfl(nr, 16 * b, 64) << (4 * b);
  // orbit_root_causal_successor (:470-498): the latest earlier position with the query's roots.
  const uint16_t qcode = M.code4[w.tok[last]];
  int pm = -1;
  for (int p = lane; p < last; p += 64)
    if (M.code4[w.tok[p]] == qcode) pm = p;
  pm = (int)wave_max32((uint32_t)(pm + 1)) - 1;
  const bool has_ptr = pm >= 0;
  const uint32_t ptr = has_ptr ? w.tok[pm + 1] : 0u;
  // select_level3_joint_pointer_global (:546-599): the candidates are the entries under the
  // query, read and recurrence keys, and the pointer successor. Each table is read under one key
  // per row, so lanes 0..11 first find the six keys' ranges; every count is then a search
  // within its key's range.
  const uint32_t qtok = w.tok[last];
  uint32_t key_of[kSparse];
  key_of[S_QUERY] = qtok;
  key_of[S_QUERY_READ] = qtok << 16 | read_code;
  key_of[S_READ] = read_code;
  key_of[S_QUERY_REC] = qtok << 16 | rec_code;
  key_of[S_READ_REC] = read_code << 16 | rec_code;
  key_of[S_REC] = rec_code;
  uint64_t bound = 0;
#pragma unroll
  for (int t = 0; t < kSparse; t++)
    if (lane == t || lane == t + kSparse) {
      const uint32_t b = key_of[t] >> kBucketShift[t];
      const uint64_t lo = M.bucket[t][b], hi = M.bucket[t][b + 1];
      if (kBucketShift[t] == 0) {
        bound = lane >= kSparse ? hi : lo;
      } else {
        const uint64_t x = ((uint64_t)key_of[t] + (lane >= kSparse ? 1 : 0)) << 32;
        bound = lo + lower_bound64(M.pairs[t] + lo, hi - lo, x);
      }
    }
  uint64_t beg[kSparse], end[kSparse];
#pragma unroll
  for (int t = 0; t < kSparse; t++) {
    beg[t] = lane64(bound, t);
    end[t] = lane64(bound, t + kSparse);
  }
  const uint64_t n0 = end[S_QUERY] - beg[S_QUERY], n1 = end[S_READ] - beg[S_READ];
  const uint64_t n2 = end[S_REC] - beg[S_REC];
  const uint64_t total = n0 + n1 + n2 + (has_ptr ? 1 : 0);
  uint64_t best_s = 0;
  uint32_t best_u = 0, best_t = 0xffffffffu;
  for (uint64_t c = lane; c < total; c += 64) {
    uint32_t tok;
    if (c < n0) tok = (uint32_t)M.pairs[S_QUERY][beg[S_QUERY] + c];
    else if (c < n0 + n1) tok = (uint32_t)M.pairs[S_READ][beg[S_READ] + c - n0];
    else if (c < n0 + n1 + n2) tok = (uint32_t)M.pairs[S_REC][beg[S_REC] + c - n0 - n1];
    else tok = ptr;
    if (tok >= M.vocab) continue;
    uint64_t cnt[5];
#pragma unroll
    for (int t = 0; t < 5; t++) {
      const uint64_t want = (uint64_t)key_of[t] << 32 | tok;
      const uint64_t i = beg[t] + lower_bound64(M.pairs[t] + beg[t], end[t] - beg[t], want);
      cnt[t] = i < end[t] && M.pairs[t][i] == want ? M.counts[t][i] : 0u;
    }
    const uint64_t s = (cnt[S_QUERY_READ] << 6) + (cnt[S_QUERY_REC] << 5) +
                       (cnt[S_READ_REC] << 3) + (cnt[S_READ] << 1) + cnt[S_QUERY] +
                       (has_ptr && ptr == tok ? 256u : 0u);
    const uint32_t uc = M.unigram[tok];
    if (s > 0 && (s > best_s || (s == best_s && (uc > best_u || (uc == best_u && tok < best_t))))) {
      best_s = s;
      best_u = uc;
      best_t = tok;
    }
  }
  const uint64_t ms = wave_max64(best_s);
  uint32_t chosen = M.unigram_best;
  if (ms > 0) {
    const uint32_t mu = wave_max32(best_s == ms ? best_u : 0u);
    chosen = wave_min32(best_s == ms && best_u == mu ? best_t : 0xffffffffu);
  }
  // apply_joint_pointer_gate (:646-684)
  const uint16_t target = M.code4[chosen];
  int moved[4];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int src_root = qroot[b], dst = target >> (4 * b) & 15;
    moved[b] = g.act[g.bfs[(src_root << 4) + dst]][src_root];  // an exact root: snap(., 1) keeps it
  }
  wave_sync();
  if (lane < 4) {
#pragma unroll
    for (int b = 0; b < 4; b++)
      if (b == lane) qroot[b] = (uint8_t)moved[b];
  }
  wave_sync();
}

// TR: evaluate_prefix_traced's words at `tw` (M.trace_block a block) and, for the relation
// read, the relation words at `rw` (M.rel_stride a block); unspecified for a row whose status
// is not 0 (the reference returns an error).
template <bool TR>
__device__ void score_row(const DevModel &M, const Geo &g, WaveLds &w, const uint32_t *prefix,
                          int len, uint32_t target, uint32_t stride, uor_d11_row_out *o,
                          int lane, uint32_t *tw, uint32_t *rw) {
  const int B = (int)M.blocks;
  int status = 0;
  if (len < 1 || len > (int)M.context || len > (int)stride) {
    status = UOR_D11_ROW_PREFIX_LENGTH;
  } else {
    bool bad = false;
    for (int i = lane; i < len; i += 64) {
      const uint32_t t = prefix[i];
      if (t >= M.vocab) bad = true;
      else w.tok[i] = (uint16_t)t;
    }
    if (__any(bad)) status = UOR_D11_ROW_PREFIX_TOKEN;
    else if (target >= M.vocab) status = UOR_D11_ROW_TARGET_TOKEN;
  }
  if (status) {
    write_error(o, status, lane);
    return;
  }
  wave_sync();
  const Plan &P = M.plans[len - 1];
  const bool relation = M.read_mode == UOR_D11_READ_RELATION;
  if (relation && M.gates[B * M.stages + 3] != 0) {
    // Edge type 3 (level 0 only): each atom's previous position holding the same token. Each
    // group of 64 positions keeps its tokens' 13 bit planes as ballots; a position's match in
    // group g is the AND of the planes its bits select, taken below its own lane in its group.
    const int groups = (len + 63) >> 6;
    for (int gi = 0; gi < groups; gi++) {
      const int a = gi * 64 + lane;
      const uint32_t t = a < len ? w.tok[a] : 0u;
#pragma unroll
      for (int bit = 0; bit < 13; bit++) {
        const uint64_t m = __ballot(t >> bit & 1);
        if (lane == 0) w.tokbits[gi][bit] = m;
      }
      const uint64_t vm = __ballot(a < len);
      if (lane == 0) w.tokbits[gi][13] = vm;
    }
    wave_sync();
    for (int gi = 0; gi < groups; gi++) {
      const int a = gi * 64 + lane;
      const uint32_t t = a < len ? w.tok[a] : 0u;
      int j = -1;
      for (int h = gi; h >= 0 && j < 0; h--) {
        uint64_t m = same_as<13>(t, w.tokbits[h], w.tokbits[h][13]);
        if (h == gi) m &= (1ull << lane) - 1;
        if (m) j = h * 64 + 63 - __clzll(m);
      }
      if (a < len) w.prevocc[a] = (int16_t)(j < 0 ? -1 : P.order[P.level_start[0] + j]);
    }
    wave_sync();
  }
  uint8_t *qroot = w.qroot;
  for (int b = 0; b < B; b++) {
    uint32_t *tb = TR ? tw + (uint64_t)b * M.trace_block : nullptr;
    uint32_t *rb = TR && relation ? rw + (uint64_t)b * M.rel_stride : nullptr;
    const int r = M.read_mode == UOR_D11_READ_ROUTE
                      ? route_block<TR>(M, g, P, w, len, b, lane, tb)
                      : flock_block<TR>(M, g, P, w, len, b, relation, lane, tb, rb);
    if (r < 0) {
      write_error(o, UOR_D11_ROW_ROUTE, lane);
      return;
    }
    if (lane == 0) qroot[b] = (uint8_t)r;
    wave_sync();
  }
  if (M.trunk && !M.knockout) trunk_gate(M, g, w, len, lane);  // not for a knockout (:1810-1814)
  // The writer (:1843-1888): admitted cells by (address distance, cell), then the top 8 of
  // their tokens by (token distance, token).
  const int q0 = qroot[0], ql = qroot[B - 1];
  uint32_t adk[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t c = (uint32_t)lane + 64u * j;
    const bool occ = M.occupied[c >> 5] >> (c & 31) & 1;
    adk[j] = occ ? ((uint32_t)(g.dist[q0][c >> 4] + g.dist[ql][c & 15]) << 8 | c) : 0xffffffffu;
  }
  const uint32_t adk0[4] = {adk[0], adk[1], adk[2], adk[3]};
  uint32_t *admitted = w.rec + 4, *ranked = w.rec + 20;
  if (lane < 24) w.rec[4 + lane] = 0;
  wave_sync();
  int na = 0;
  for (uint32_t r = 0; r < M.kept_cells; r++) {
    const uint32_t m = wave_min32(min(min(adk[0], adk[1]), min(adk[2], adk[3])));
    if (m == 0xffffffffu) break;
    const uint32_t c = m & 0xff;
    if ((int)(c & 63) == lane) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (j == (int)(c >> 6)) adk[j] = 0xffffffffu;
    }
    if (lane == 0) admitted[na] = c;
    na++;
  }
  wave_sync();
  // Candidate tokens: each lane keeps its best 8 (key = distance << 13 | token), then 8 rounds
  // of wave minima merge them. The same pass counts the target's token rivals.
  uint32_t top[8];
#pragma unroll
  for (int k = 0; k < 8; k++) top[k] = 0xffffffffu;
  uint32_t rivals = 0, rival_d = 0xffffffffu;
  for (int k = 0; k < na; k++) {
    const uint32_t c = admitted[k];
    for (uint32_t i = M.cell_off[c] + lane; i < M.cell_off[c + 1]; i += 64) {
      const uint32_t t = M.cell_tok[i];
      uint32_t td = 0;
      for (int b = 0; b < B; b++) td += g.dist[qroot[b]][M.troot[t * B + b]];
      if (t != target) {
        rivals++;
        rival_d = min(rival_d, td);
      }
      uint32_t x = td << 13 | t;
#pragma unroll
      for (int s = 0; s < 8; s++) {  // insertion into the sorted 8
        const uint32_t y = top[s];
        top[s] = min(x, y);
        x = max(x, y);
      }
    }
  }
  int found = 0;
  int head = 0;
  uint32_t first = 0;
  for (int r = 0; r < 8; r++) {
    uint32_t mine = 0xffffffffu;
#pragma unroll
    for (int s = 0; s < 8; s++)
      if (s == head) mine = top[s];
    const uint32_t m = wave_min32(mine);
    if (m == 0xffffffffu) break;
    if (mine == m) head++;
    if (lane == 0) ranked[found] = m & 0x1fff;
    if (found == 0) first = m & 0x1fff;
    found++;
  }
  if (found == 0) {
    write_error(o, UOR_D11_ROW_ZERO_TOKENS, lane);
    return;
  }
  // observe_target (:1892-1993)
  const uint32_t token_rivals = wave_sum32(rivals);
  const uint32_t rd = wave_min32(rival_d);
  const uint32_t tcell = M.cell[target];
  uint32_t td_t = 0;
  for (int b = 0; b < B; b++) td_t += g.dist[qroot[b]][M.troot[target * B + b]];
  const uint32_t ad_t = g.dist[q0][tcell >> 4] + g.dist[ql][tcell & 15];
  uint32_t address_rivals = 0, ra = 0xffffffffu;
  for (int k = 0; k < na; k++) {
    const uint32_t c = admitted[k];
    if (c != tcell) {
      address_rivals++;
      ra = min(ra, (uint32_t)(g.dist[q0][c >> 4] + g.dist[ql][c & 15]));
    }
  }
  uint32_t rank = 1;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t key = adk0[j];
    const uint32_t c = (uint32_t)lane + 64u * j;
    const bool before = key != 0xffffffffu && ((key >> 8) < ad_t || ((key >> 8) == ad_t && c < tcell));
    rank += __popcll(__ballot(before));
  }
  const uint32_t width = (uint32_t)B << 3;
  const uint32_t th = (rd == 0xffffffffu || width + td_t <= rd) ? 0u : width + td_t - rd;
  const uint32_t ah = (ra == 0xffffffffu || 8u + ad_t <= ra) ? 0u : 8u + ad_t - ra;
  const uint32_t rh = rank > M.kept_cells ? rank - M.kept_cells : 0u;
  const uint32_t loss_ta = th * 8u + ah * width, loss_tr = th * 8u + rh * width;
  // The rest of the record (admitted cells and top 8 are in place), stored whole.
  for (int i = lane; i < UOR_D11_MAX_BLOCKS * 8; i += 64) {
    const int b = i >> 3;
    w.rec[28 + i] = b < B ? (uint32_t)(int32_t)g.roots[qroot[b]][i & 7] : 0u;
  }
  if (lane == 0) {
    w.rec[0] = 0;
    w.rec[1] = (uint32_t)na;
    w.rec[2] = (uint32_t)found;
    w.rec[3] = first;
    w.rec[156] = th;
    w.rec[157] = ah;
    w.rec[158] = rh;
    w.rec[159] = loss_ta;
    w.rec[160] = loss_tr;
    w.rec[161] = token_rivals;
    w.rec[162] = address_rivals;
    w.rec[163] = M.policy == UOR_D11_POLICY_OCCUPIED_CELL_RANK ? loss_tr : loss_ta;
  }
  wave_sync();
  uint32_t *dst = (uint32_t *)o;
  for (int i = lane; i < kRecWords; i += 64) dst[i] = w.rec[i];
}

template <bool TR>
__device__ __forceinline__ void score_block(const DevModel &M, const uint32_t *prefixes,
                                            const int32_t *lengths, const uint32_t *targets,
                                            uint32_t rows, uint32_t stride, uor_d11_row_out *out,
                                            uint32_t *trace, uint32_t *rel_trace) {
  __shared__ Geo g;
  __shared__ WaveLds lds[kWaves];
  {
    const uint32_t *src = (const uint32_t *)M.geo;
    uint32_t *d = (uint32_t *)&g;
    for (uint32_t i = threadIdx.x; i < sizeof(Geo) / 4; i += kThreads) d[i] = src[i];
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kWaves + wave;
  if (row >= rows) return;
  score_row<TR>(M, g, lds[wave], prefixes + (uint64_t)row * stride, lengths[row], targets[row],
                stride, out + row, lane,
                TR ? trace + (uint64_t)row * M.blocks * M.trace_block : nullptr,
                TR && rel_trace ? rel_trace + (uint64_t)row * M.blocks * M.rel_stride : nullptr);
}

__global__ __launch_bounds__(kThreads) void d11_score_rows(DevModel M, const uint32_t *prefixes,
                                                           const int32_t *lengths,
                                                           const uint32_t *targets, uint32_t rows,
                                                           uint32_t stride, uor_d11_row_out *out) {
  score_block<false>(M, prefixes, lengths, targets, rows, stride, out, nullptr, nullptr);
}

// evaluate_prefix_traced for every row (discrete_d11.rs:1768-1770).
__global__ __launch_bounds__(kThreads) void d11_score_rows_traced(
    DevModel M, const uint32_t *prefixes, const int32_t *lengths, const uint32_t *targets,
    uint32_t rows, uint32_t stride, uor_d11_row_out *out, uint32_t *trace, uint32_t *rel_trace) {
  score_block<true>(M, prefixes, lengths, targets, rows, stride, out, trace, rel_trace);
}

// ---------------------------------------------------------------------------------------------
// Host side.

thread_local std::string g_error;

int fail(int code, const std::string &msg) {
  g_error = msg;
  return code;
}

struct Handle {
  int device = 0;
  DevModel dm{};
  std::vector<void *> bufs;
  ~Handle() {
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    for (void *p : bufs) (void)hipFree(p);
    (void)hipSetDevice(prev);
  }
  template <class T>
  const T *upload(const std::vector<T> &v) {
    void *p = nullptr;
    const size_t n = std::max<size_t>(v.size() * sizeof(T), 16);
    if (hipMalloc(&p, n) != hipSuccess) return nullptr;
    bufs.push_back(p);
    if (!v.empty() && hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
      return nullptr;
    return (const T *)p;
  }
};

int root_id(const int32_t *x) {
  for (int r = 0; r < 16; r++) {
    bool same = true;
    for (int d = 0; d < 8; d++) same &= x[d] == kD11Roots[r][d];
    if (same) return r;
  }
  return -1;
}

int host_snap(const int32_t *x, int n) {
  int best = 0;
  uint32_t bd = UINT32_MAX, bh = UINT32_MAX;
  for (int r = 0; r < 16; r++) {
    uint32_t dist = 0, ham = 0;
    for (int d = 0; d < 8; d++) {
      const int32_t y = n * kD11Roots[r][d], e = x[d] - y;
      dist += (uint32_t)(e < 0 ? -e : e);
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

Geo make_geo() {
  Geo g{};
  for (int a = 0; a < 64; a++)
    for (int r = 0; r < 16; r++) {
      int32_t y[8];
      for (int d = 0; d < 8; d++) {
        const int axis = kD11Axes[a * 8 + d];
        const int32_t v = kD11Roots[r][axis & 7];
        y[d] = axis & 8 ? -v : v;
      }
      g.act[a][r] = (uint8_t)root_id(y);  // the orbit is closed under the states
    }
  for (int i = 0; i < 16; i++)
    for (int j = 0; j < 16; j++) {
      uint32_t dist = 0, ham = 0;
      for (int d = 0; d < 8; d++) {
        const int e = kD11Roots[i][d] - kD11Roots[j][d];
        dist += (uint32_t)(e < 0 ? -e : e);
        ham += e != 0;
      }
      g.dist[i][j] = (uint8_t)dist;
      g.ham[i][j] = (uint8_t)ham;
      for (int k = 0; k < 16; k++) {
        int32_t s[8];
        for (int d = 0; d < 8; d++) s[d] = kD11Roots[i][d] + kD11Roots[j][d] + kD11Roots[k][d];
        g.snap3[i << 8 | j << 4 | k] = (uint8_t)host_snap(s, 3);
      }
    }
  for (int i = 0; i < 256; i++) g.bfs[i] = kD11Bfs[i];
  for (int r = 0; r < 16; r++)
    for (int p = 0; p < 3; p++) g.branch[r][p] = kD11Branch[r][p];
  for (int i = 0; i < 4096; i++) g.compose[i >> 6][i & 63] = kD11Compose[i];
  for (int r = 0; r < 16; r++)
    for (int d = 0; d < 8; d++) g.roots[r][d] = kD11Roots[r][d];
  return g;
}

// build_row_plan (discrete_d11.rs:813-884) with each node's parent and slot, its left
// neighbour (a same-level node j < i with last(j) + 1 == first(i): edge type 2's sum) and the
// level order. Returns false if a node had two left neighbours (never, for this tree).
bool make_plan(int length, Plan &p) {
  struct N {
    int c[3], atom, level, first, last, parent, slot;
  };
  std::vector<N> nodes;
  std::vector<int> frontier;
  for (int atom = 0; atom < length; atom++) {
    frontier.push_back((int)nodes.size());
    nodes.push_back({{-1, -1, -1}, atom, 0, atom, atom, -1, 0});
    for (;;) {
      const size_t n = frontier.size();
      if (n < 3) break;
      const int c0 = frontier[n - 3], c1 = frontier[n - 2], c2 = frontier[n - 1];
      const int lv = nodes[c0].level;
      if (nodes[c1].level != lv || nodes[c2].level != lv) break;
      const int parent = (int)nodes.size();
      nodes.push_back({{c0, c1, c2}, -1, lv + 1, nodes[c0].first, nodes[c2].last, -1, 0});
      for (int s = 0; s < 3; s++) {
        nodes[nodes[parent].c[s]].parent = parent;
        nodes[nodes[parent].c[s]].slot = s;
      }
      frontier.resize(n - 3);
      frontier.push_back(parent);
    }
  }
  memset(&p, 0, sizeof p);
  p.count = (uint16_t)nodes.size();
  p.frontier_len = (uint16_t)frontier.size();
  if (nodes.size() > (size_t)kMaxNodes || frontier.size() > 16) return false;
  for (size_t i = 0; i < frontier.size(); i++) p.frontier[i] = (uint16_t)frontier[i];
  int k = 0;
  for (int l = 0; l < kMaxLevels; l++) {
    p.level_start[l] = (uint16_t)k;
    for (size_t i = 0; i < nodes.size(); i++)
      if (nodes[i].level == l) p.order[k++] = (uint16_t)i;
  }
  p.level_start[kMaxLevels] = (uint16_t)k;
  for (size_t i = 0; i < nodes.size(); i++) {
    const N &n = nodes[i];
    const uint32_t inner = n.atom < 0;
    const uint32_t c0 = inner ? (uint32_t)n.c[0] : (uint32_t)n.atom;
    const uint32_t c1 = inner ? (uint32_t)n.c[1] : 0u, c2 = inner ? (uint32_t)n.c[2] : 0u;
    p.node[i] = c0 | c1 << 9 | c2 << 18 | (uint32_t)n.level << 27 | inner << 30;
    const uint32_t parent = n.parent < 0 ? kNone : (uint32_t)n.parent;
    p.link[i] = (uint32_t)n.first | (uint32_t)n.last << 8 | parent << 16 | (uint32_t)n.slot << 25;
    int left = -1, hits = 0;
    for (size_t j = 0; j < i; j++)
      if (nodes[j].level == n.level && nodes[j].last + 1 == n.first) {
        left = (int)j;
        hits++;
      }
    if (hits > 1) return false;
    p.left[i] = left < 0 ? 0xffff : (uint16_t)left;
  }
  return true;
}

int expected_stages(uint32_t context) {
  if (context < 1 || context > UOR_D11_MAX_CONTEXT) return -1;
  int stages = 1;
  uint32_t span = 3;
  while (span <= context) {
    stages++;
    span *= 3;
  }
  return stages;
}

}  // namespace d11

using namespace d11;

extern "C" uint32_t uor_d11_abi_version(void) { return UOR_D11_ABI_VERSION; }
extern "C" int64_t uor_d11_sizeof_model(void) { return (int64_t)sizeof(uor_d11_model); }
extern "C" int64_t uor_d11_sizeof_row_out(void) { return (int64_t)sizeof(uor_d11_row_out); }
extern "C" const char *uor_d11_last_error(void) { return g_error.c_str(); }

extern "C" int uor_d11_model_create(const uor_d11_model *m, int32_t device, void **handle) {
  if (!m || !handle) return fail(-1, "null argument");
  *handle = nullptr;
  const uint32_t V = m->vocabulary, B = m->blocks, S = m->stages;
  // The shape and section checks of from_bytes (discrete_d11.rs:972-1150).
  if (V < 2 || V > UOR_D11_MAX_VOCAB || B < 2 || B > UOR_D11_MAX_BLOCKS || m->context < 1 ||
      m->context > UOR_D11_MAX_CONTEXT || m->kept_cells < 1 || m->kept_cells > UOR_D11_MAX_KEPT_CELLS ||
      m->kept_cells > V || expected_stages(m->context) != (int)S)
    return fail(-1, "inconsistent or unsupported discrete shape");
  const bool ok_mode =
      (m->read_mode == UOR_D11_READ_ROUTE && m->read_kept == 0 && m->read_sweeps == 0) ||
      (m->read_mode == UOR_D11_READ_FLOCK && m->read_kept >= 1 && m->read_kept <= UOR_D11_MAX_KEPT &&
       m->read_sweeps == 0) ||
      (m->read_mode == UOR_D11_READ_RELATION && m->read_kept >= 1 &&
       m->read_kept <= UOR_D11_MAX_KEPT && m->read_sweeps >= 1 &&
       m->read_sweeps <= UOR_D11_MAX_SWEEPS);
  if (!ok_mode) return fail(-1, "unsupported discrete read mode or parameters");
  if (m->objective_policy > 1) return fail(-1, "unsupported discrete objective policy");
  if (m->flags & ~UOR_D11_FLAG_STATE_TRANSPORT_KNOCKOUT) return fail(-1, "unknown model flags");
  const bool knockout = (m->flags & UOR_D11_FLAG_STATE_TRANSPORT_KNOCKOUT) != 0;
  if (!m->table || !m->cells || !m->routes || !m->gates) return fail(-1, "null section");
  const uint32_t ngates = B * S + (m->read_mode == UOR_D11_READ_RELATION ? 5 * S : 0);
  for (uint32_t i = 0; i < B * S; i++)
    if (m->routes[i] >= 64) return fail(-1, "discrete.routes contains action index >= 64");
  for (uint32_t i = 0; i < ngates; i++)
    if (m->gates[i] < -1 || m->gates[i] > 1) return fail(-1, "discrete.gates contains trit outside -1..=1");
  std::vector<uint8_t> troot((size_t)V * B), cell(V);
  std::vector<uint16_t> code4(V);
  uint32_t occupied[8] = {0};
  for (uint32_t t = 0; t < V; t++) {
    for (uint32_t b = 0; b < B; b++) {
      const int r = root_id(m->table + ((size_t)t * B + b) * 8);
      if (r < 0) return fail(-1, "discrete.table block is outside the 16-root SpiralCore orbit");
      troot[(size_t)t * B + b] = (uint8_t)r;
    }
    const uint32_t c = (uint32_t)troot[(size_t)t * B] << 4 | troot[(size_t)t * B + B - 1];
    if (m->cells[t] != c) return fail(-1, "discrete.cells entry disagrees with discrete.table endpoint roots");
    cell[t] = (uint8_t)c;
    occupied[c >> 5] |= 1u << (c & 31);
    code4[t] = B >= 4 ? (uint16_t)(troot[(size_t)t * B] | troot[(size_t)t * B + 1] << 4 |
                                   troot[(size_t)t * B + 2] << 8 | troot[(size_t)t * B + 3] << 12)
                      : 0;
  }
  std::vector<uint32_t> cell_off(257, 0);
  for (uint32_t t = 0; t < V; t++) cell_off[cell[t] + 1]++;
  for (int c = 0; c < 256; c++) cell_off[c + 1] += cell_off[c];
  std::vector<uint16_t> cell_tok(V);
  {
    std::vector<uint32_t> fill(cell_off.begin(), cell_off.end() - 1);
    for (uint32_t t = 0; t < V; t++) cell_tok[fill[cell[t]]++] = (uint16_t)t;
  }
  // with_state_transport_knockout (discrete_d11.rs:1283-1304): identity routes (state 0), zero
  // level and relation gates.
  std::vector<uint8_t> routes(B * S);
  for (uint32_t i = 0; i < B * S; i++) routes[i] = knockout ? 0 : (uint8_t)m->routes[i];
  std::vector<int8_t> gates(ngates);
  for (uint32_t i = 0; i < ngates; i++) gates[i] = knockout ? 0 : (int8_t)m->gates[i];
  std::vector<Plan> plans(m->context);
  for (uint32_t n = 1; n <= m->context; n++)
    if (!make_plan((int)n, plans[n - 1])) return fail(-1, "row plan outside the kernel's limits");
  // The trunk (discrete_d11.rs:1196-1262).
  const uor_d11_trunk *tr = m->trunk;
  std::vector<uint8_t> step(64, 0), norm(4, 0);
  std::vector<uint32_t> unigram(V, 0);
  std::vector<uint64_t> pairs[kSparse];
  std::vector<uint32_t> counts[kSparse], bucket[kSparse];
  uint32_t unigram_best = 0;
  if (tr) {
    if (B != 4) return fail(-1, "the trunk requires 4 blocks");
    for (int i = 0; i < 64; i++) {
      if (tr->step_candidates[i] >= 16) return fail(-1, "discrete.trunk.step_candidates requires 64 candidates in 0..16");
      step[i] = (uint8_t)tr->step_candidates[i];
    }
    for (int i = 0; i < 4; i++) {
      if (tr->norm_candidates[i] >= 16) return fail(-1, "discrete.trunk.norm_candidates requires 4 candidates in 0..16");
      norm[i] = (uint8_t)tr->norm_candidates[i];
    }
    if (!tr->unigram || tr->unigram[0] >= V) return fail(-1, "discrete.trunk.unigram length, best_global, or counts invalid");
    bool any = false;
    for (uint32_t t = 0; t < V; t++) {
      unigram[t] = tr->unigram[1 + t];
      any |= unigram[t] != 0;
    }
    if (!any) return fail(-1, "discrete.trunk.unigram length, best_global, or counts invalid");
    unigram_best = tr->unigram[0];
    for (int i = 0; i < 12; i++) {  // every table is checked, six are read
      const uint64_t n = tr->sparse_rows[i];
      if (n && !tr->sparse[i]) return fail(-1, "null trunk table");
      std::vector<std::pair<uint64_t, uint32_t>> kv(n);
      for (uint64_t r = 0; r < n; r++) {
        const uint32_t *w = tr->sparse[i] + 3 * r;
        if (w[1] >= V || w[2] == 0) return fail(-1, "sparse trunk count table contains invalid token or zero count");
        kv[r] = {(uint64_t)w[0] << 32 | w[1], w[2]};
      }
      std::sort(kv.begin(), kv.end());
      for (uint64_t r = 1; r < n; r++)
        if (kv[r].first == kv[r - 1].first) return fail(-1, "duplicate (key, token) entry in sparse trunk count table");
      for (int s = 0; s < kSparse; s++)
        if (kSparseSource[s] == i) {
          pairs[s].resize(n);
          counts[s].resize(n);
          for (uint64_t r = 0; r < n; r++) {
            pairs[s][r] = kv[r].first;
            counts[s][r] = kv[r].second;
          }
        }
    }
  }
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (hipSetDevice(device) != hipSuccess) return fail(-2, "hipSetDevice failed");
  Handle *h = new Handle();
  h->device = device;
  DevModel &d = h->dm;
  d.vocab = V;
  d.blocks = B;
  d.context = m->context;
  d.kept_cells = m->kept_cells;
  d.stages = S;
  d.read_mode = m->read_mode;
  d.read_kept = m->read_kept;
  d.read_sweeps = m->read_sweeps;
  d.policy = m->objective_policy;
  d.trunk = tr != nullptr;
  d.unigram_best = unigram_best;
  d.knockout = knockout;
  d.trace_block = m->read_mode == UOR_D11_READ_ROUTE
                      ? UOR_D11_ROUTE_TRACE_HEADER_WORDS + S * UOR_D11_ROUTE_TRACE_STAGE_WORDS
                      : UOR_D11_ACTIVE_TRACE_HEADER_WORDS + S * UOR_D11_ACTIVE_TRACE_LEVEL_WORDS;
  d.rel_stride = m->read_mode == UOR_D11_READ_RELATION ? plans[m->context - 1].count : 0;
  for (int i = 0; i < 8; i++) d.occupied[i] = occupied[i];
  const std::vector<Geo> geo(1, make_geo());
  bool ok = (d.geo = h->upload(geo)) && (d.troot = h->upload(troot)) && (d.cell = h->upload(cell)) &&
            (d.cell_off = h->upload(cell_off)) && (d.cell_tok = h->upload(cell_tok)) &&
            (d.routes = h->upload(routes)) && (d.gates = h->upload(gates)) &&
            (d.plans = h->upload(plans)) && (d.unigram = h->upload(unigram)) &&
            (d.code4 = h->upload(code4)) && (d.step = h->upload(step)) && (d.norm = h->upload(norm));
  for (int s = 0; s < kSparse; s++) {
    bucket[s].assign(kBuckets + 1, 0);
    uint32_t i = 0;
    for (uint32_t b = 0; b < kBuckets; b++) {
      const uint64_t first = (uint64_t)b << (32 + kBucketShift[s]);  // below 2^64 for b < 2^16
      while (i < pairs[s].size() && pairs[s][i] < first) i++;
      bucket[s][b] = i;
    }
    if (kBucketShift[s] == 0)  // keys of 2^16 and above lie beyond every bucket
      while (i < pairs[s].size() && pairs[s][i] < ((uint64_t)kBuckets << 32)) i++;
    else
      i = (uint32_t)pairs[s].size();
    bucket[s][kBuckets] = i;
  }
  for (int s = 0; ok && s < kSparse; s++) {
    ok = (d.pairs[s] = h->upload(pairs[s])) && (d.counts[s] = h->upload(counts[s])) &&
         (d.bucket[s] = h->upload(bucket[s]));
    d.rows[s] = pairs[s].size();
  }
  (void)hipSetDevice(prev);
  if (!ok) {
    delete h;
    return fail(-2, "device allocation or copy failed");
  }
  *handle = h;
  return 0;
}

extern "C" void uor_d11_model_destroy(void *handle) { delete (Handle *)handle; }

extern "C" int uor_d11_score_rows_async(void *handle, const uint32_t *d_prefixes,
                                        const int32_t *d_lengths, const uint32_t *d_targets,
                                        uint32_t rows, uint32_t stride, uor_d11_row_out *d_out,
                                        void *stream) {
  if (!handle) return fail(-1, "null handle");
  if (rows == 0) return 0;
  if (!d_prefixes || !d_lengths || !d_targets || !d_out || stride == 0)
    return fail(-1, "null buffer or zero stride");
  Handle *h = (Handle *)handle;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(h->device);
  const uint32_t grid = (rows + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(d11_score_rows, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, h->dm,
                     d_prefixes, d_lengths, d_targets, rows, stride, d_out);
  const hipError_t e = hipGetLastError();
  (void)hipSetDevice(prev);
  return e == hipSuccess ? 0 : fail(-2, std::string("launch: ") + hipGetErrorString(e));
}

extern "C" uint32_t uor_d11_trace_words(void *handle, uint32_t *relation_words) {
  if (!handle) return 0;
  const DevModel &d = ((Handle *)handle)->dm;
  if (relation_words) *relation_words = d.blocks * d.rel_stride;
  return d.blocks * d.trace_block;
}

extern "C" int uor_d11_score_rows_traced_async(void *handle, const uint32_t *d_prefixes,
                                               const int32_t *d_lengths, const uint32_t *d_targets,
                                               uint32_t rows, uint32_t stride, uor_d11_row_out *d_out,
                                               uint32_t *d_trace, uint32_t *d_relation_trace,
                                               void *stream) {
  if (!handle) return fail(-1, "null handle");
  if (rows == 0) return 0;
  Handle *h = (Handle *)handle;
  if (!d_prefixes || !d_lengths || !d_targets || !d_out || !d_trace || stride == 0 ||
      (h->dm.rel_stride && !d_relation_trace))
    return fail(-1, "null buffer or zero stride");
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(h->device);
  const uint32_t grid = (rows + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(d11_score_rows_traced, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream,
                     h->dm, d_prefixes, d_lengths, d_targets, rows, stride, d_out, d_trace,
                     h->dm.rel_stride ? d_relation_trace : nullptr);
  const hipError_t e = hipGetLastError();
  (void)hipSetDevice(prev);
  return e == hipSuccess ? 0 : fail(-2, std::string("launch: ") + hipGetErrorString(e));
}

// The host-buffer form of either launch: copies in, one launch, copies out.
static int score_host(void *handle, const uint32_t *prefixes, const int32_t *lengths,
                      const uint32_t *targets, uint32_t rows, uint32_t stride, uor_d11_row_out *out,
                      uint32_t *trace, uint32_t *relation_trace) {
  if (!handle) return fail(-1, "null handle");
  if (rows == 0) return 0;
  if (!prefixes || !lengths || !targets || !out || stride == 0)
    return fail(-1, "null buffer or zero stride");
  for (uint32_t r = 0; r < rows; r++)
    if (lengths[r] < 0 || (uint32_t)lengths[r] > stride) return fail(-1, "a length exceeds the row stride");
  Handle *h = (Handle *)handle;
  uint32_t rel_words = 0;
  const uint32_t words = uor_d11_trace_words(handle, &rel_words);
  if (trace && rel_words && !relation_trace) return fail(-1, "a relation read needs the relation trace");
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(h->device);
  const size_t np = (size_t)rows * stride * 4, nr = (size_t)rows * 4, no = (size_t)rows * sizeof(uor_d11_row_out);
  const size_t nt = trace ? (size_t)rows * words * 4 : 0, nrel = trace ? (size_t)rows * rel_words * 4 : 0;
  const size_t at_out = (np + 2 * nr + 15) & ~(size_t)15, at_tr = (at_out + no + 15) & ~(size_t)15;
  const size_t at_rel = (at_tr + nt + 15) & ~(size_t)15;
  char *buf = nullptr;
  int rc = 0;
  if (hipMalloc((void **)&buf, at_rel + nrel + 64) != hipSuccess) {
    rc = fail(-2, "device allocation failed");
  } else {
    uint32_t *dp = (uint32_t *)buf;
    int32_t *dl = (int32_t *)(buf + np);
    uint32_t *dt = (uint32_t *)(buf + np + nr);
    uor_d11_row_out *dout = (uor_d11_row_out *)(buf + at_out);
    uint32_t *dtr = (uint32_t *)(buf + at_tr), *drel = (uint32_t *)(buf + at_rel);
    if (hipMemcpy(dp, prefixes, np, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dl, lengths, nr, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dt, targets, nr, hipMemcpyHostToDevice) != hipSuccess) {
      rc = fail(-2, "copy to the device failed");
    } else {
      rc = trace ? uor_d11_score_rows_traced_async(handle, dp, dl, dt, rows, stride, dout, dtr,
                                                   drel, nullptr)
                 : uor_d11_score_rows_async(handle, dp, dl, dt, rows, stride, dout, nullptr);
      if (rc == 0 && (hipDeviceSynchronize() != hipSuccess ||
                      hipMemcpy(out, dout, no, hipMemcpyDeviceToHost) != hipSuccess ||
                      (nt && hipMemcpy(trace, dtr, nt, hipMemcpyDeviceToHost) != hipSuccess) ||
                      (nrel && hipMemcpy(relation_trace, drel, nrel, hipMemcpyDeviceToHost) != hipSuccess)))
        rc = fail(-2, "scoring failed on the device");
    }
    (void)hipFree(buf);
  }
  (void)hipSetDevice(prev);
  return rc;
}

extern "C" int uor_d11_score_rows(void *handle, const uint32_t *prefixes, const int32_t *lengths,
                                  const uint32_t *targets, uint32_t rows, uint32_t stride,
                                  uor_d11_row_out *out) {
  return score_host(handle, prefixes, lengths, targets, rows, stride, out, nullptr, nullptr);
}

extern "C" int uor_d11_score_rows_traced(void *handle, const uint32_t *prefixes,
                                         const int32_t *lengths, const uint32_t *targets,
                                         uint32_t rows, uint32_t stride, uor_d11_row_out *out,
                                         uint32_t *trace, uint32_t *relation_trace) {
  if (!trace) return fail(-1, "null trace buffer");
  return score_host(handle, prefixes, lengths, targets, rows, stride, out, trace, relation_trace);
}
