// fbs_index.hip - the 256-cell CSR drawer index on the GPU: build, update, remove, validate,
// probe and full scan, the API of the reference's projects/uor-cuda-inverted-file
// (include/uor_inverted_file.hpp:41-50; host rules src/inverted_file.cpp:12-270; its CUDA
// kernels uor_if_build/update/probe/full_scan, src/kernels.cu:139-243, run one thread per
// index or per query row), and of the discrete crate's bucket build/update entries
// (crates/uor-r4-discrete/src/bucket_source.rs:1-12).
//
// A token's cell is r0 * 16 + r1 when the first 8 values of its row equal root r0 and the last
// 8 equal root r1 (the first matching root of 16), else ABSENT. The index lists each cell's
// tokens in ascending order (offsets[257], members), keeps every token's cell and counts the
// absent tokens. Status words hold uor_inverted_file::Status values
// (include/uor_inverted_file.hpp:29-37): 0 ok, 1 invalid argument, 2 non-root block,
// 3 CSR invariant.
//
// Build (three launches): cells and one histogram per tile (512 to 8,192 tokens: the largest
// that leaves about 256 tiles); one block per cell
// scanning that cell's tile counts; a stable scatter in which a token's place is its cell's
// offset + its tile's start in the cell + the earlier tokens of the tile in the same cell, the
// tile sorted in LDS first so that each cell's run is written contiguously.
// Update / remove (four launches): the structure check the reference runs first, spread over
// many blocks; one block moving the token with the reference's shifts (the members between
// the old and the new place move by one, in chunks that read before they write); then the
// check the reference runs after the move (structure for a removal, structure and every
// token's cell for an update), whose last block writes the status.
// Probe: one wave per query row (admission = the k nearest non-empty cells by endpoint L1,
// then the admitted cells' members ranked by row L1, top 8, ties to the lower id). Full scan:
// one block per query row over every token of the table.
//
// Every kernel bounds-checks what it indexes with values read from the index, so a corrupt
// index yields status 3 rather than an out-of-range access.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/uor_fbs.h"

namespace fbs_index {

constexpr uint32_t kAbsent = 0xffffffffu;
constexpr uint32_t kCells = 256;
constexpr uint32_t kSlots = kCells + 1;  // cells, then the absent tokens
constexpr uint32_t kThreads = 256;       // scan, verify and full-scan blocks
constexpr uint32_t kWaves = kThreads / 64;
constexpr uint32_t kBuildThreads = 512;  // cells and scatter blocks
constexpr uint32_t kBuildWaves = kBuildThreads / 64;
constexpr uint32_t kMaxPer = 16;  // rounds of kBuildThreads tokens per build tile
constexpr uint32_t kMaxTile = kBuildThreads * kMaxPer;
static_assert(kMaxTile <= 65536, "a token's place in its tile fits 16 bits");
constexpr uint32_t kMoveThreads = 1024;
constexpr uint32_t kShiftPer = 4;  // members per thread per shift chunk
constexpr uint32_t kMaxVerifyBlocks = 2048;
constexpr uint32_t kProbeWaves = 4;  // query rows per probe block
constexpr int32_t kOk = 0, kInvalid = 1, kNonRoot = 2, kCsr = 3;
constexpr int64_t kFar = INT64_MAX;
// Workspace words ahead of the build's tile counts.
constexpr uint32_t kBad = 0, kDone = 1, kTally = 2, kPost = 3, kHeader = 16;
static_assert(kThreads == kCells, "one thread per cell in the scans");
static_assert(kBuildThreads >= kCells, "a build block has a thread per cell");

// Rounds per build tile: the most (longer runs per cell, so the scatter's writes coalesce)
// that still leave about 256 tiles (one per CU) to spread the work.
__host__ __device__ inline uint32_t rounds_of(uint32_t count) {
  uint32_t per = 1;
  while (per < kMaxPer && (uint64_t)count >= (uint64_t)2 * per * kBuildThreads * 256) per *= 2;
  return per;
}
__host__ __device__ inline uint32_t tiles_of(uint32_t count) {
  const uint32_t tile = rounds_of(count) * kBuildThreads;
  return (count + tile - 1) / tile;
}

// ---- cells

__device__ __forceinline__ void load_roots(const int32_t *roots, int32_t *sroots) {
  for (uint32_t i = threadIdx.x; i < 128; i += blockDim.x) sroots[i] = roots[i];
}

// The first root (of 16, in LDS) equal to the 8 values at `block` (16-byte aligned).
__device__ __forceinline__ uint32_t root_id(const int32_t *block, const int32_t *sroots) {
  const int4 a = *(const int4 *)block, b = *(const int4 *)(block + 4);
  uint32_t id = kAbsent;
#pragma unroll
  for (int r = 15; r >= 0; r--) {
    const int4 x = *(const int4 *)(sroots + 8 * r), y = *(const int4 *)(sroots + 8 * r + 4);
    const bool same = a.x == x.x && a.y == x.y && a.z == x.z && a.w == x.w && b.x == y.x &&
                      b.y == y.y && b.z == y.z && b.w == y.w;
    id = same ? (uint32_t)r : id;
  }
  return id;
}

__device__ __forceinline__ uint32_t token_cell(const int32_t *row, uint32_t width,
                                               const int32_t *sroots) {
  const uint32_t a = root_id(row, sroots), b = root_id(row + width - 8, sroots);
  return a == kAbsent || b == kAbsent ? kAbsent : a * 16 + b;
}

// Inclusive scan over the block's N threads (buf: N words of LDS); every thread may read
// buf[N - 1], the block's total, on return.
template <uint32_t N>
__device__ uint32_t block_scan(uint32_t v, uint32_t *buf) {
  buf[threadIdx.x] = v;
  __syncthreads();
  for (uint32_t off = 1; off < N; off *= 2) {
    const uint32_t add = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
    __syncthreads();
    buf[threadIdx.x] += add;
    __syncthreads();
  }
  return buf[threadIdx.x];
}

// The cell holding position p of a CSR run list: the c with start[c] <= p < start[c + 1]
// (start non-decreasing, start[0] <= p < start[256]).
__device__ __forceinline__ uint32_t cell_at(const uint32_t *start, uint32_t p) {
  uint32_t lo = 0, hi = kCells;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (start[mid] <= p) lo = mid; else hi = mid;
  }
  return lo;
}

// ---- build

// Cells, and each tile's count of every cell (slot 256: absent tokens) as counts[slot][tile].
// Token t of a tile is t = tile * per * kBuildThreads + r * kBuildThreads + thread, r < per,
// in passes of up to 8 rows per thread (16 loads in flight each).
__global__ __launch_bounds__(kBuildThreads) void index_cells(const int32_t *__restrict__ table,
                                                             uint32_t count, uint32_t width,
                                                             const int32_t *__restrict__ roots,
                                                             uint32_t per, uint32_t tiles,
                                                             uint32_t *__restrict__ cells,
                                                             uint32_t *__restrict__ counts) {
  __shared__ __align__(16) int32_t sroots[128];
  __shared__ uint32_t hist[kSlots];
  load_roots(roots, sroots);
  for (uint32_t i = threadIdx.x; i < kSlots; i += kBuildThreads) hist[i] = 0;
  __syncthreads();
  // Four lanes a row, each loading one 16-byte piece of an endpoint block (the first block's
  // two, then the last block's two), so one load instruction covers 16 rows' endpoints instead
  // of one piece of 64 rows. Each lane matches its piece against its half of every root (a bit
  // per root); a lane pair's AND is the block's match, its lowest bit the first equal root.
  const uint32_t which = threadIdx.x & 3, half = which & 1;
  const uint32_t piece = which < 2 ? which : width / 4 - 4 + which;
  int4 R[16];
#pragma unroll
  for (int r = 0; r < 16; r++) R[r] = *(const int4 *)(sroots + 8 * r + 4 * half);
  constexpr uint32_t kRows = kBuildThreads / 4;  // rows a block reads per round
  // The rows are read once: non-temporal loads keep them from displacing what the caches hold
  // (measured 12 % faster at 16.8 M tokens).
  typedef int v4i __attribute__((ext_vector_type(4)));
  const uint32_t rounds = per * 4, first = blockIdx.x * per * kBuildThreads + (threadIdx.x >> 2);
  for (uint32_t round = 0; round < rounds; round += 8) {
    int4 v[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; u++) {
      const uint32_t t = first + (round + u) * kRows;
      v4i raw = {0, 0, 0, 0};
      if (round + u < rounds && t < count)
        raw = __builtin_nontemporal_load((const v4i *)(table + (uint64_t)t * width + 4 * piece));
      v[u] = make_int4(raw.x, raw.y, raw.z, raw.w);
    }
#pragma unroll
    for (uint32_t u = 0; u < 8; u++) {
      uint32_t m = 0;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int d = (v[u].x ^ R[r].x) | (v[u].y ^ R[r].y) | (v[u].z ^ R[r].z) | (v[u].w ^ R[r].w);
        m |= (uint32_t)(d == 0) << r;
      }
      m &= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xf, 0xf, false);  // lane ^ 1
      const uint32_t b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xf, 0xf, false);
      const uint32_t t = first + (round + u) * kRows;
      if (which == 0 && round + u < rounds && t < count) {
        const uint32_t c = m && b ? (uint32_t)__builtin_ctz(m) * 16 + (uint32_t)__builtin_ctz(b) : kAbsent;
        cells[t] = c;
        atomicAdd(&hist[c == kAbsent ? kCells : c], 1u);
      }
    }
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < kSlots; i += kBuildThreads)
    counts[(uint64_t)i * tiles + blockIdx.x] = hist[i];
}

// One block per slot: the exclusive scan of the slot's tile counts (in place: each tile's
// start within the slot) and the slot's total.
__global__ __launch_bounds__(kThreads) void index_scan_tiles(uint32_t *counts, uint32_t tiles,
                                                             uint32_t *totals) {
  __shared__ uint32_t buf[kThreads];
  uint32_t *row = counts + (uint64_t)blockIdx.x * tiles;
  uint32_t carry = 0;
  for (uint32_t base = 0; base < tiles; base += kThreads) {
    const uint32_t i = base + threadIdx.x;
    const uint32_t v = i < tiles ? row[i] : 0;
    const uint32_t incl = block_scan<kThreads>(v, buf);
    if (i < tiles) row[i] = carry + incl - v;
    carry += buf[kThreads - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// The lanes of this wave holding the same cell as this lane (a match of the cell's 8 bits over
// ballots), among the valid ones.
__device__ __forceinline__ uint64_t same_cell(uint32_t c, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; b++) {
    const bool bit = (c >> b) & 1;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stable scatter of one tile: its tokens are ordered by (cell, token) in LDS, then each cell's
// run is written to members contiguously (runs of tile/256 members on average, so the writes
// coalesce). Each wave takes a contiguous chunk of the tile: it counts its chunk's cells, one
// pass over the cells turns the counts into each wave's first place in every cell's run, and
// the wave walks its chunk again, a token's place being its wave's cursor for the cell plus the
// earlier lanes with the same cell; so the block meets three barriers a tile. Block 0 also
// writes offsets, the absent count and status.
__global__ __launch_bounds__(kBuildThreads) void index_scatter(
    const uint32_t *__restrict__ cells, uint32_t count, uint32_t per,
    const uint32_t *__restrict__ starts, uint32_t tiles, const uint32_t *__restrict__ totals,
    uint32_t allow_absent,
    uint32_t *__restrict__ offsets, uint32_t *__restrict__ members,
    uint32_t *__restrict__ absent_count, int32_t *__restrict__ status) {
  __shared__ uint32_t sorted[kMaxTile];  // cell << 16 | the token's place in the tile
  __shared__ uint32_t buf[kBuildThreads];
  __shared__ uint32_t lstart[kSlots];  // each cell's run within the tile's sorted tokens
  __shared__ uint32_t gbase[kCells];   // each cell's run within members
  __shared__ uint32_t wave_cnt[kBuildWaves][kCells];  // counts, then each wave's cursors
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64, tile = blockIdx.x;
  const bool is_cell = tid < kCells;
  // Cell offsets: the exclusive scan of the cells' totals.
  const uint32_t total = is_cell ? totals[tid] : 0;
  const uint32_t incl = block_scan<kBuildThreads>(total, buf);
  const uint32_t cell_base = incl - total;
  if (tile == 0 && is_cell) {
    offsets[tid] = cell_base;
    if (tid == kCells - 1) {
      offsets[kCells] = incl;
      const uint32_t absent = totals[kCells];
      *absent_count = absent;
      *status = absent && !allow_absent ? kNonRoot : kOk;
    }
  }
  // This tile's count of each cell, from its start and the next tile's.
  uint32_t here = 0;
  if (is_cell) {
    const uint32_t start = starts[(uint64_t)tid * tiles + tile];
    const uint32_t next = tile + 1 < tiles ? starts[(uint64_t)tid * tiles + tile + 1] : total;
    here = next - start;
    gbase[tid] = cell_base + start;
  }
  __syncthreads();  // buf is reused by the next scan
  const uint32_t lincl = block_scan<kBuildThreads>(here, buf);
  if (is_cell) lstart[tid] = lincl - here;
  if (tid == kCells - 1) lstart[kCells] = lincl;
  for (uint32_t i = tid; i < kBuildWaves * kCells; i += kBuildThreads) (&wave_cnt[0][0])[i] = 0;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1;
  // This wave's chunk: per rounds of 64 consecutive tokens, its cells loaded at once.
  const uint32_t local = wave * per * 64 + lane, tile_base = tile * per * kBuildThreads;
  uint32_t cv[kMaxPer];
#pragma unroll
  for (uint32_t r = 0; r < kMaxPer; r++) {
    const uint32_t t = tile_base + local + r * 64;
    cv[r] = r < per && t < count ? cells[t] : kAbsent;
  }
#pragma unroll
  for (uint32_t r = 0; r < kMaxPer; r++) {
    if (r >= per) break;
    const uint32_t c = cv[r];
    const bool valid = c != kAbsent;
    const uint64_t peers = same_cell(c, valid);
    if (valid && (peers & below) == 0) wave_cnt[wave][c] += __popcll(peers);
    wave_sync();
  }
  __syncthreads();
  // Each wave's first place in each cell's run: the run's start and the earlier waves' counts.
  if (is_cell) {
    uint32_t at = lstart[tid];
    for (uint32_t w = 0; w < kBuildWaves; w++) {
      const uint32_t n = wave_cnt[w][tid];
      wave_cnt[w][tid] = at;
      at += n;
    }
  }
  __syncthreads();
#pragma unroll
  for (uint32_t r = 0; r < kMaxPer; r++) {
    if (r >= per) break;
    const uint32_t c = cv[r];
    const bool valid = c != kAbsent;
    const uint64_t peers = same_cell(c, valid);
    if (valid) sorted[wave_cnt[wave][c] + __popcll(peers & below)] = c << 16 | (local + r * 64);
    wave_sync();
    if (valid && (peers & below) == 0) wave_cnt[wave][c] += __popcll(peers);
    wave_sync();
  }
  __syncthreads();
  const uint32_t n = lstart[kCells];
  for (uint32_t i = tid; i < n; i += kBuildThreads) {
    const uint32_t e = sorted[i], c = e >> 16;
    members[gbase[c] + (i - lstart[c])] = tile_base + (e & 0xffff);
  }
}

// ---- checks

__global__ void index_begin(uint32_t *ws, uint32_t post) {
  if (threadIdx.x < kHeader) ws[threadIdx.x] = threadIdx.x == kPost ? post : 0;
}

// validate_structure (inverted_file.cpp:141-162) and validate (:164-176), spread over the
// grid. phase 0: the structure, failures flagged in ws[kBad] (read by the move). phase 1: what
// ws[kPost] names (0 nothing, 1 the structure, 2 the structure and every token's cell against
// the table), the last block writing the status.
__global__ __launch_bounds__(kThreads) void index_verify(
    const int32_t *__restrict__ table, uint32_t count, uint32_t width,
    const int32_t *__restrict__ roots, const uint32_t *__restrict__ offsets,
    const uint32_t *__restrict__ members, const uint32_t *__restrict__ cells,
    const uint32_t *__restrict__ absent_count, uint32_t *ws, uint32_t phase,
    int32_t *__restrict__ status) {
  __shared__ __align__(16) int32_t sroots[128];
  __shared__ uint32_t soff[kSlots];
  __shared__ uint32_t bad, tally, last;
  const uint32_t what = phase == 0 ? 1 : ws[kPost];
  if (what == 0) return;
  const uint32_t tid = threadIdx.x;
  if (tid == 0) bad = tally = last = 0;
  for (uint32_t i = tid; i < kSlots; i += kThreads) soff[i] = offsets[i];
  if (what == 2) load_roots(roots, sroots);
  __syncthreads();
  const uint32_t absent = *absent_count, size = soff[kCells];
  if (tid == 0 && (soff[0] != 0 || size > count || (uint64_t)absent + size != count)) bad = 1;
  if (soff[tid] > soff[tid + 1] || soff[tid + 1] > size) bad = 1;
  __syncthreads();
  const uint32_t stride = gridDim.x * kThreads;
  if (!bad) {
    for (uint32_t p = blockIdx.x * kThreads + tid; p < size; p += stride) {
      const uint32_t m = members[p];
      if (m >= count || (p > soff[cell_at(soff, p)] && members[p - 1] >= m)) bad = 1;
    }
  }
  if (what == 2) {
    uint32_t gone = 0;
    for (uint32_t t = blockIdx.x * kThreads + tid; t < count; t += stride) {
      const uint32_t c = cells[t];
      if (c == kAbsent)
        gone++;
      else if (c != token_cell(table + (uint64_t)t * width, width, sroots))
        bad = 1;
    }
    atomicAdd(&tally, gone);
  }
  __syncthreads();
  if (tid == 0) {
    if (bad) atomicOr(&ws[kBad], 1u);
    if (what == 2) atomicAdd(&ws[kTally], tally);
    if (phase == 1) {
      __threadfence();
      last = atomicAdd(&ws[kDone], 1u) == gridDim.x - 1;
    }
  }
  __syncthreads();
  if (last && tid == 0) {
    __threadfence();
    const uint32_t b = atomicOr(&ws[kBad], 0u), g = atomicAdd(&ws[kTally], 0u);
    *status = b || (what == 2 && g != absent) ? kCsr : kOk;
  }
}

// ---- update / remove: one block

// members[p] = members[p + 1] for p in [from, to), in ascending chunks.
__device__ void shift_down(uint32_t *members, uint32_t from, uint32_t to) {
  constexpr uint32_t chunk = kMoveThreads * kShiftPer;
  for (uint32_t base = from; base < to; base += chunk) {
    uint32_t v[kShiftPer];
#pragma unroll
    for (uint32_t k = 0; k < kShiftPer; k++) {
      const uint32_t p = base + k * kMoveThreads + threadIdx.x;
      v[k] = p < to ? members[p + 1] : 0;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kShiftPer; k++) {
      const uint32_t p = base + k * kMoveThreads + threadIdx.x;
      if (p < to) members[p] = v[k];
    }
    __syncthreads();
  }
}

// members[p + 1] = members[p] for p in [from, to), in descending chunks.
__device__ void shift_up(uint32_t *members, uint32_t from, uint32_t to) {
  constexpr uint32_t chunk = kMoveThreads * kShiftPer;
  for (uint32_t top = to; top > from;) {
    const uint32_t lo = top - from < chunk ? from : top - chunk;
    uint32_t v[kShiftPer];
#pragma unroll
    for (uint32_t k = 0; k < kShiftPer; k++) {
      const uint32_t p = lo + k * kMoveThreads + threadIdx.x;
      v[k] = p < top ? members[p] : 0;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kShiftPer; k++) {
      const uint32_t p = lo + k * kMoveThreads + threadIdx.x;
      if (p < top) members[p + 1] = v[k];
    }
    __syncthreads();
    top = lo;
  }
}

// The first position in [lo, hi) whose member is not below `token` (members ascending there):
// where the reference's linear walk stops.
__device__ uint32_t lower_bound(const uint32_t *members, uint32_t lo, uint32_t hi,
                                uint32_t token) {
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (members[mid] < token) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// update (inverted_file.cpp:182-236, mode 0) and remove_token (:238-249, mode 1) after the
// structure check. Every decision is uniform over the block (all threads read the same words).
// Returns the status and, through `post`, the check to run after a move.
__device__ int32_t move_token(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, uint32_t moved, uint32_t mode,
                              uint32_t *offsets, uint32_t *members, uint32_t *cells,
                              uint32_t *absent_count, const uint32_t *ws, int32_t *sroots,
                              uint32_t *soff, uint32_t *remove_pos, uint32_t &post) {
  const uint32_t tid = threadIdx.x;
  if (moved >= count) return kInvalid;
  if (ws[kBad]) return kCsr;
  for (uint32_t i = tid; i < kSlots; i += kMoveThreads) soff[i] = offsets[i];
  if (mode == 0) load_roots(roots, sroots);
  if (tid == 0) *remove_pos = kAbsent;
  __syncthreads();
  const uint32_t absent = *absent_count, old_cell = cells[moved];
  uint32_t new_cell = kAbsent;
  if (mode == 0) {
    if (old_cell != kAbsent && old_cell >= kCells) return kCsr;
    new_cell = token_cell(table + (uint64_t)moved * width, width, sroots);
    if (new_cell == kAbsent) return kNonRoot;
    if (new_cell == old_cell) return kOk;
  } else {
    if (old_cell == kAbsent) return kOk;
    // remove_from_bucket (:84-100) reads the old cell's range; a cell past 255 has none.
    if (old_cell >= kCells) return kCsr;
  }
  if (old_cell != kAbsent) {
    for (uint32_t p = soff[old_cell] + tid; p < soff[old_cell + 1]; p += kMoveThreads)
      if (members[p] == moved) atomicMin(remove_pos, p);
    __syncthreads();
    if (*remove_pos == kAbsent) return kCsr;
  } else if (absent == 0) {
    return kCsr;
  }
  const uint32_t size = soff[kCells], rp = *remove_pos;
  uint32_t at = 0, lo_cell, hi_cell;
  int32_t delta;
  if (mode == 0) at = lower_bound(members, soff[new_cell], soff[new_cell + 1], moved);
  __syncthreads();  // every search has read before anything moves
  if (mode == 1) {  // out of old_cell: the later members move down
    shift_down(members, rp, size - 1);
    lo_cell = old_cell + 1, hi_cell = kCells, delta = -1;
  } else if (old_cell == kAbsent) {  // into new_cell: the later members move up
    shift_up(members, at, size);
    if (tid == 0) members[at] = moved;
    lo_cell = new_cell + 1, hi_cell = kCells, delta = 1;
  } else if (old_cell < new_cell) {
    shift_down(members, rp, at - 1);
    if (tid == 0) members[at - 1] = moved;
    lo_cell = old_cell + 1, hi_cell = new_cell, delta = -1;
  } else {
    shift_up(members, at, rp);
    if (tid == 0) members[at] = moved;
    lo_cell = new_cell + 1, hi_cell = old_cell, delta = 1;
  }
  for (uint32_t c = lo_cell + tid; c <= hi_cell; c += kMoveThreads)
    offsets[c] = (uint32_t)((int32_t)soff[c] + delta);
  if (tid == 0) {
    cells[moved] = mode == 1 ? kAbsent : new_cell;
    *absent_count = mode == 1 ? absent + 1 : old_cell == kAbsent ? absent - 1 : absent;
  }
  post = mode == 0 ? 2 : 1;
  return kOk;
}

__global__ __launch_bounds__(kMoveThreads) void index_move(
    const int32_t *table, uint32_t count, uint32_t width, const int32_t *roots, uint32_t moved,
    uint32_t mode, uint32_t *offsets, uint32_t *members, uint32_t *cells,
    uint32_t *absent_count, uint32_t *ws, int32_t *status) {
  __shared__ __align__(16) int32_t sroots[128];
  __shared__ uint32_t soff[kSlots];
  __shared__ uint32_t remove_pos;
  uint32_t post = 0;
  const int32_t st = move_token(table, count, width, roots, moved, mode, offsets, members, cells,
                                absent_count, ws, sroots, soff, &remove_pos, post);
  __syncthreads();
  if (threadIdx.x == 0) {
    ws[kBad] = ws[kDone] = ws[kTally] = 0;
    ws[kPost] = post;
    *status = st;
  }
}

// ---- probe and full scan

__device__ __forceinline__ uint64_t wave_min64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint64_t o = __shfl_xor(v, m, 64);
    v = o < v ? o : v;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_min32(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint32_t o = __shfl_xor(v, m, 64);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ bool before(int64_t d, uint32_t t, int64_t e, uint32_t u) {
  return d < e || (d == e && t < u);
}

// A lane's 8 best (distance, token), ascending.
struct Top8 {
  int64_t d[8];
  uint32_t t[8];
  __device__ void clear() {
#pragma unroll
    for (int i = 0; i < 8; i++) d[i] = kFar, t[i] = kAbsent;
  }
  __device__ void add(int64_t x, uint32_t y) {
    if (!before(x, y, d[7], t[7])) return;  // most candidates, once the list is full
    // From the bottom up: entry i takes entry i - 1 when the new pair sorts before that too,
    // else the new pair when it sorts before entry i.
#pragma unroll
    for (int i = 7; i > 0; i--) {
      if (before(x, y, d[i], t[i])) {
        const bool above = before(x, y, d[i - 1], t[i - 1]);
        d[i] = above ? d[i - 1] : x;
        t[i] = above ? t[i - 1] : y;
      }
    }
    if (before(x, y, d[0], t[0])) d[0] = x, t[0] = y;
  }
  // The wave's 8 best from every lane's 8: each round takes the smallest head, whose lane
  // drops it. Same result on every lane.
  __device__ void wave_best(uint32_t *out_t, int64_t *out_d) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const uint64_t dm = wave_min64((uint64_t)d[0]);
      const uint32_t tm = wave_min32((uint64_t)d[0] == dm ? t[0] : kAbsent);
      out_d[r] = (int64_t)dm;
      out_t[r] = dm == (uint64_t)kFar ? kAbsent : tm;
      if ((uint64_t)d[0] == dm && t[0] == tm) {
#pragma unroll
        for (int i = 0; i < 7; i++) d[i] = d[i + 1], t[i] = t[i + 1];
        d[7] = kFar, t[7] = kAbsent;
      }
    }
  }
};

__device__ __forceinline__ int64_t l1_8(const int32_t *q, const int32_t *r) {
  int64_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int64_t x = (int64_t)q[i] - r[i];
    s += x < 0 ? -x : x;
  }
  return s;
}

// |a - b| of two int32 values, exact in 32 unsigned bits.
__device__ __forceinline__ uint32_t absdiff32(int32_t a, int32_t b) {
  return a > b ? (uint32_t)a - (uint32_t)b : (uint32_t)b - (uint32_t)a;
}

// L1 between the query (LDS) and a table row, 16-byte loads; each difference in 32 bits, the
// sum in 64.
__device__ __forceinline__ int64_t row_l1(const int32_t *q, const int32_t *row, uint32_t width) {
  uint64_t s = 0;
  for (uint32_t i = 0; i < width; i += 4) {
    const int4 a = *(const int4 *)(row + i), b = *(const int4 *)(q + i);
    s += absdiff32(b.x, a.x);
    s += absdiff32(b.y, a.y);
    s += absdiff32(b.z, a.z);
    s += absdiff32(b.w, a.w);
  }
  return (int64_t)s;
}

// fill_admitted (inverted_file.cpp:83-96) on one wave: the k nearest non-empty cells by
// cell_distance (:38-47), ties to the lower cell; adm[0..16) on every lane, ABSENT-padded.
// rd: 32 words of LDS for this wave. Called by every wave of the block (it synchronises).
__device__ void admit_wave(const int32_t *sq, uint32_t width, const int32_t *sroots,
                           const uint32_t *offsets, uint32_t k, int64_t *rd, uint32_t *adm) {
  const uint32_t lane = threadIdx.x % 64;
  if (lane < 32) {
    const int32_t *part = lane < 16 ? sq : sq + width - 8;
    rd[lane] = l1_8(part, sroots + 8 * (lane % 16));
  }
  __syncthreads();
  uint64_t key[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t c = lane + 64 * j;
    const bool empty = offsets[c] == offsets[c + 1];
    key[j] = empty ? ~0ull : ((uint64_t)(rd[c / 16] + rd[16 + c % 16]) << 8) | c;
  }
#pragma unroll
  for (uint32_t i = 0; i < 16; i++) {
    uint64_t mine = key[0];
#pragma unroll
    for (int j = 1; j < 4; j++) mine = key[j] < mine ? key[j] : mine;
    const uint64_t m = i < k ? wave_min64(mine) : ~0ull;
    adm[i] = m == ~0ull ? kAbsent : (uint32_t)(m & 255);
#pragma unroll
    for (int j = 0; j < 4; j++) key[j] = key[j] == m ? ~0ull : key[j];
  }
}

// probe (inverted_file.cpp:250-258; kernel uor_if_probe, kernels.cu:198-213) for one query row
// per wave. The index is not validated here: callers validate it once per change.
__global__ __launch_bounds__(64 * kProbeWaves) void index_probe(
    const int32_t *__restrict__ table, uint32_t count, uint32_t width,
    const int32_t *__restrict__ roots, const int32_t *__restrict__ queries, uint32_t rows,
    uint32_t k, const uint32_t *__restrict__ offsets, const uint32_t *__restrict__ members,
    uint32_t *__restrict__ predictions, uint32_t *__restrict__ admitted,
    uint32_t *__restrict__ top8, int32_t *__restrict__ status) {
  __shared__ __align__(16) int32_t sroots[128];
  __shared__ __align__(16) int32_t sq[kProbeWaves][UOR_FBS_INDEX_MAX_WIDTH];
  __shared__ int64_t rd[kProbeWaves][32];
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint32_t row = blockIdx.x * kProbeWaves + wave;
  const uint32_t src = row < rows ? row : rows - 1;  // surplus waves repeat the last row, unwritten
  load_roots(roots, sroots);
  for (uint32_t i = lane; i < width; i += 64) sq[wave][i] = queries[(uint64_t)src * width + i];
  __syncthreads();
  uint32_t adm[16];
  admit_wave(sq[wave], width, sroots, offsets, k, rd[wave], adm);
  // The admitted cells' member ranges, concatenated; lane j takes positions j, j + 64, ...
  uint32_t lo[16], n[16], total = 0;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    lo[i] = n[i] = 0;
    if (adm[i] != kAbsent) {
      const uint32_t a = offsets[adm[i]], b = offsets[adm[i] + 1];
      if (b < a || b > count)
        bad = true;
      else
        lo[i] = a, n[i] = b - a;
    }
    total += n[i];
  }
  Top8 best;
  best.clear();
  for (uint32_t j = lane; j < total; j += 64) {
    uint32_t p = j, at = 0;
    bool found = false;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      if (!found && p < n[i]) at = lo[i] + p, found = true;
      if (!found) p -= n[i];
    }
    const uint32_t t = members[at];
    if (t >= count) {
      bad = true;
      continue;
    }
    best.add(row_l1(sq[wave], table + (uint64_t)t * width, width), t);
  }
  uint32_t out[8];
  int64_t dist[8];
  best.wave_best(out, dist);
  bad = __any(bad);
  if (row < rows && lane == 0) {
    predictions[row] = out[0];
#pragma unroll
    for (int i = 0; i < 8; i++) top8[(uint64_t)row * 8 + i] = out[i];
#pragma unroll
    for (int i = 0; i < 16; i++) admitted[(uint64_t)row * 16 + i] = adm[i];
    status[row] = bad ? kCsr : out[0] == kAbsent ? kInvalid : kOk;
  }
}

// full_scan (inverted_file.cpp:260-270; kernel uor_if_full_scan, kernels.cu:215-243) for one
// query row per block: cells admitted from `offsets` (an index of the table built with absent
// tokens allowed), then every token of the table whose cell is admitted, ranked.
__global__ __launch_bounds__(kThreads) void index_full_scan(
    const int32_t *__restrict__ table, uint32_t count, uint32_t width,
    const int32_t *__restrict__ roots, const int32_t *__restrict__ queries, uint32_t k,
    const uint32_t *__restrict__ offsets, uint32_t *__restrict__ predictions,
    uint32_t *__restrict__ admitted, uint32_t *__restrict__ top8,
    int32_t *__restrict__ status) {
  __shared__ __align__(16) int32_t sroots[128];
  __shared__ __align__(16) int32_t sq[UOR_FBS_INDEX_MAX_WIDTH];
  __shared__ int64_t rd[kWaves][32];
  __shared__ int64_t wd[kWaves][8];
  __shared__ uint32_t wt[kWaves][8];
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64, row = blockIdx.x;
  load_roots(roots, sroots);
  for (uint32_t i = tid; i < width; i += kThreads) sq[i] = queries[(uint64_t)row * width + i];
  __syncthreads();
  uint32_t adm[16];
  admit_wave(sq, width, sroots, offsets, k, rd[wave], adm);
  Top8 best;
  best.clear();
  for (uint32_t t = tid; t < count; t += kThreads) {
    const int32_t *r = table + (uint64_t)t * width;
    const uint32_t c = token_cell(r, width, sroots);
    bool in = false;
#pragma unroll
    for (int i = 0; i < 16; i++) in |= c != kAbsent && adm[i] == c;
    if (in) best.add(row_l1(sq, r, width), t);
  }
  uint32_t out[8];
  int64_t dist[8];
  best.wave_best(out, dist);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 8; i++) wd[wave][i] = dist[i], wt[wave][i] = out[i];
  }
  __syncthreads();
  if (wave == 0) {
    Top8 merged;
    merged.clear();
    if (lane < kWaves * 8) merged.add(wd[lane / 8][lane % 8], wt[lane / 8][lane % 8]);
    merged.wave_best(out, dist);
    if (lane == 0) {
      predictions[row] = out[0];
#pragma unroll
      for (int i = 0; i < 8; i++) top8[(uint64_t)row * 8 + i] = out[i];
#pragma unroll
      for (int i = 0; i < 16; i++) admitted[(uint64_t)row * 16 + i] = adm[i];
      status[row] = out[0] == kAbsent ? kInvalid : kOk;
    }
  }
}

}  // namespace fbs_index

using namespace fbs_index;

namespace {

bool table_ok(const int32_t *table, const int32_t *roots, uint32_t width) {
  return table && roots && width >= 16 && width <= UOR_FBS_INDEX_MAX_WIDTH && width % 4 == 0 &&
         ((uintptr_t)table & 15) == 0;
}

int launched() { return hipGetLastError() == hipSuccess ? UOR_FBS_OK : UOR_FBS_ERR_DEVICE; }

uint32_t verify_grid(uint32_t count) {
  const uint32_t g = (count + kThreads - 1) / kThreads;
  return g < 1 ? 1 : g > kMaxVerifyBlocks ? kMaxVerifyBlocks : g;
}

}  // namespace

extern "C" uint64_t uor_fbs_index_workspace_bytes(uint32_t count) {
  return ((uint64_t)kHeader + (uint64_t)kSlots * (tiles_of(count) + 1)) * sizeof(uint32_t);
}

extern "C" int uor_fbs_index_build_async(const int32_t *table, uint32_t count, uint32_t width,
                                         const int32_t *roots, uint32_t allow_absent,
                                         uint32_t *offsets, uint32_t *members, uint32_t *cells,
                                         uint32_t *absent_count, void *workspace, int32_t *status,
                                         void *stream) {
  if (!table_ok(table, roots, width) || !offsets || !members || !cells || !absent_count ||
      !workspace || !status || count == 0 || count > UOR_FBS_INDEX_MAX_TOKENS)
    return UOR_FBS_ERR_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  const uint32_t per = rounds_of(count), tiles = tiles_of(count);
  uint32_t *counts = (uint32_t *)workspace + kHeader;
  uint32_t *totals = counts + (uint64_t)kSlots * tiles;
  hipLaunchKernelGGL(index_cells, dim3(tiles), dim3(kBuildThreads), 0, s, table, count, width, roots,
                     per, tiles, cells, counts);
  hipLaunchKernelGGL(index_scan_tiles, dim3(kSlots), dim3(kThreads), 0, s, counts, tiles,
                     totals);
  hipLaunchKernelGGL(index_scatter, dim3(tiles), dim3(kBuildThreads), 0, s, cells, count, per,
                     counts, tiles, totals, allow_absent, offsets, members, absent_count, status);
  return launched();
}

static int index_change_async(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, uint32_t moved, uint32_t mode,
                              uint32_t *offsets, uint32_t *members, uint32_t *cells,
                              uint32_t *absent_count, void *workspace, int32_t *status,
                              void *stream) {
  if ((mode == 0 && !table_ok(table, roots, width)) || !offsets || !members || !cells ||
      !absent_count || !workspace || !status || count == 0 || count > UOR_FBS_INDEX_MAX_TOKENS)
    return UOR_FBS_ERR_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  uint32_t *ws = (uint32_t *)workspace;
  const uint32_t grid = verify_grid(count);
  hipLaunchKernelGGL(index_begin, dim3(1), dim3(64), 0, s, ws, 0u);
  hipLaunchKernelGGL(index_verify, dim3(grid), dim3(kThreads), 0, s, table, count, width, roots,
                     offsets, members, cells, absent_count, ws, 0u, status);
  hipLaunchKernelGGL(index_move, dim3(1), dim3(kMoveThreads), 0, s, table, count, width, roots,
                     moved, mode, offsets, members, cells, absent_count, ws, status);
  hipLaunchKernelGGL(index_verify, dim3(grid), dim3(kThreads), 0, s, table, count, width, roots,
                     offsets, members, cells, absent_count, ws, 1u, status);
  return launched();
}

extern "C" int uor_fbs_index_update_async(const int32_t *table, uint32_t count, uint32_t width,
                                          const int32_t *roots, uint32_t moved, uint32_t *offsets,
                                          uint32_t *members, uint32_t *cells,
                                          uint32_t *absent_count, void *workspace,
                                          int32_t *status, void *stream) {
  return index_change_async(table, count, width, roots, moved, 0, offsets, members, cells,
                            absent_count, workspace, status, stream);
}

extern "C" int uor_fbs_index_remove_async(uint32_t count, uint32_t moved, uint32_t *offsets,
                                          uint32_t *members, uint32_t *cells,
                                          uint32_t *absent_count, void *workspace,
                                          int32_t *status, void *stream) {
  return index_change_async(nullptr, count, 16, nullptr, moved, 1, offsets, members, cells,
                            absent_count, workspace, status, stream);
}

extern "C" int uor_fbs_index_validate_async(const int32_t *table, uint32_t count, uint32_t width,
                                            const int32_t *roots, const uint32_t *offsets,
                                            const uint32_t *members, const uint32_t *cells,
                                            const uint32_t *absent_count, void *workspace,
                                            int32_t *status, void *stream) {
  const bool full = table != nullptr;
  if ((full && !table_ok(table, roots, width)) || !offsets || !members || !cells ||
      !absent_count || !workspace || !status || count == 0 || count > UOR_FBS_INDEX_MAX_TOKENS)
    return UOR_FBS_ERR_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  uint32_t *ws = (uint32_t *)workspace;
  hipLaunchKernelGGL(index_begin, dim3(1), dim3(64), 0, s, ws, full ? 2u : 1u);
  hipLaunchKernelGGL(index_verify, dim3(verify_grid(count)), dim3(kThreads), 0, s, table, count,
                     width, roots, offsets, members, cells, absent_count, ws, 1u, status);
  return launched();
}

extern "C" int uor_fbs_index_probe_async(const int32_t *table, uint32_t count, uint32_t width,
                                         const int32_t *roots, const int32_t *queries,
                                         uint32_t rows, uint32_t k, const uint32_t *offsets,
                                         const uint32_t *members, uint32_t *predictions,
                                         uint32_t *admitted, uint32_t *top8, int32_t *status,
                                         void *stream) {
  if (!table_ok(table, roots, width) || !queries || !offsets ||
      !members || !predictions || !admitted || !top8 || !status || count == 0 ||
      count > UOR_FBS_INDEX_MAX_TOKENS || rows == 0 || k == 0 || k > 16)
    return UOR_FBS_ERR_ARGUMENT;
  hipLaunchKernelGGL(index_probe, dim3((rows + kProbeWaves - 1) / kProbeWaves),
                     dim3(64 * kProbeWaves), 0, (hipStream_t)stream, table, count, width, roots,
                     queries, rows, k, offsets, members, predictions, admitted, top8, status);
  return launched();
}

extern "C" int uor_fbs_index_full_scan_async(const int32_t *table, uint32_t count, uint32_t width,
                                             const int32_t *roots, const int32_t *queries,
                                             uint32_t rows, uint32_t k, const uint32_t *offsets,
                                             uint32_t *predictions, uint32_t *admitted,
                                             uint32_t *top8, int32_t *status, void *stream) {
  if (!table_ok(table, roots, width) || !queries || !offsets || !predictions || !admitted ||
      !top8 || !status || count == 0 || count > UOR_FBS_INDEX_MAX_TOKENS || rows == 0 || k == 0 ||
      k > 16)
    return UOR_FBS_ERR_ARGUMENT;
  hipLaunchKernelGGL(index_full_scan, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, table,
                     count, width, roots, queries, k, offsets, predictions, admitted, top8,
                     status);
  return launched();
}
