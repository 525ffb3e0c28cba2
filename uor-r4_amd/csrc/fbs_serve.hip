// fbs_serve.hip - the deferred writer of one-token serving launches: the drawer-major scan of
// every session's kept drawers, then the hand-out of each session's token.
//
// A serving launch steps every session by one token (serve_step, RS stack/session.rs:3405): the
// paired prefill kernel runs the step up to the writer's drawer selection and leaves a job per
// session (RunArgs::job_flag), and the session that opens a slice of 16 entries of a drawer's
// list appends that slice's work items. The writer's choice is the lowest (L1, token) over the
// members of the session's kept drawers (session.rs:4100-4121, twin fbs_core.h:606-623);
// sessions that keep the same drawer read the same member rows, so the scan here is laid out by
// drawer: a
// block holds 64 member rows of one drawer in registers, one row a lane, and scores them against
// the queries of up to 16 sessions that kept the drawer at a time (staged in LDS and read as
// broadcasts), each (row, session) L1 by packed v_sad_u16 over biased pairs. Each session's
// lowest (L1 << 32 | token) over a block's rows goes to its job by a 64-bit atomic minimum:
// the minimum of the packed pairs is the lexicographic one (the reference's lower token on equal
// L1), whatever order the blocks run in. A row is read once per 16 sessions instead of once per
// session, so the launch's candidate bytes shrink by the sessions a drawer serves.
#include <hip/hip_runtime.h>

#include "fbs_run.h"

namespace fbs {

// The blocks (a wavefront each) take the launch's items in turn: an item scores `rows` member
// rows from its first member index (one a lane, in registers) against the sessions of its
// slice of the drawer's list (16, or the rest of the list), whose query words are staged in LDS
// and read as broadcasts (every lane reads the same words), four sessions at a time. RW: the row
// words (biased 16-bit pairs) a lane holds at once; rows of more words are scored in segments of
// RW, the sessions' sums carried across. (Query words read as scalars straight from memory
// measured slower: each scalar load's wait lands on the sums' path.)
// T8: an int8 table, whose rows (code + 128 bytes) widen at the SADs as the fused writer's scan
// widens them (widen8), against queries published in that scan's scaled form.
template <int RW, bool T8>
__global__ __launch_bounds__(64) void fbs_serve_scan(DevModel M, ServeScan J) {
  __shared__ __align__(16) uint32_t qs[kServeSessions * RW];
  const uint32_t lane = threadIdx.x;
  uint32_t total = uniform32(J.item_count[0]);
  total = total < J.item_cap ? total : J.item_cap;
  const uint32_t words = M.d / 2;
  for (uint32_t it = blockIdx.x; it < total; it += gridDim.x) {
    const uint4 item = J.items[it];
    const uint32_t beg = uniform32(item.x), rows = uniform32(item.y);
    const uint32_t lbeg = uniform32(item.z), c = uniform32(item.w);
    uint32_t nc = uniform32(J.drawer_count[c]);
    nc = nc < J.list_stride ? nc : J.list_stride;  // a list holds at most list_stride sessions
    const uint32_t g = lbeg - c * J.list_stride;
    if (g >= nc) continue;
    const uint32_t ns = nc - g < kServeSessions ? nc - g : kServeSessions;
    const bool valid = lane < rows;
    const uint32_t tok = valid ? M.members[beg + lane] : 0u;
    const uint4 *row = T8 ? (const uint4 *)(M.table8 + (uint64_t)tok * M.d)
                          : (const uint4 *)((const uint32_t *)M.table_b + (uint64_t)tok * words);
    const uint32_t *list = J.drawer_list + lbeg;
    uint32_t sid[kServeSessions];
#pragma unroll
    for (uint32_t i = 0; i < kServeSessions; i++) sid[i] = i < ns ? uniform32(list[i]) : 0u;
    uint32_t acc[kServeSessions];
#pragma unroll
    for (uint32_t i = 0; i < kServeSessions; i++) acc[i] = 0;
    // The query quads this lane stages: 16-byte piece lane % (RW / 4) of session 64 j / (RW / 4)
    // + lane / (RW / 4), for each of the slice's kStage groups of 64 pieces.
    constexpr uint32_t kStage = kServeSessions * (RW / 4) / kWave;
    uint32_t stage_sid[kStage];
#pragma unroll
    for (uint32_t j = 0; j < kStage; j++) {
      const uint32_t i = (lane + kWave * j) / (RW / 4);
      stage_sid[j] = i < ns ? list[i] : list[0];
    }
    for (uint32_t seg = 0; seg < words; seg += RW) {
      // Once the last segment's (or item's) reads are done: the sessions' query words of this
      // segment go to LDS by direct loads (no registers), the rows' words to registers, every
      // load issued before the first is waited for.
      wave_sync();
#pragma unroll
      for (uint32_t j = 0; j < kStage; j++)
        if (kWave * j < ns * (RW / 4))
          __builtin_amdgcn_global_load_lds(
              (global_void *)(J.job_query + (uint64_t)stage_sid[j] * words + seg +
                              4 * (lane % (RW / 4))),
              (lds_void *)(qs + 4 * kWave * j), 16, 0, 0);
      // The row's quads of this segment: RW / 4 of biased 16-bit pairs, or RW / 8 of int8 codes.
      constexpr uint32_t kRowQuads = T8 ? RW / 8 : RW / 4;
      uint4 r[kRowQuads];
#pragma unroll
      for (uint32_t w = 0; w < kRowQuads; w++) r[w] = row[(T8 ? seg / 8 : seg / 4) + w];
      wait_lds_dma();
      // Four sessions at a time (four independent sums in flight), as many groups as the slice
      // fills; a group's sessions past ns read words never staged and are not used.
#pragma unroll
      for (uint32_t i0 = 0; i0 < kServeSessions; i0 += 4) {
        if (i0 < ns) {
          if constexpr (T8) {
#pragma unroll
            for (uint32_t w = 0; w < kRowQuads; w++) {
              uint32_t wd[8];  // the quad's 16 codes as eight widened words
              widen8(r[w].x, wd[0], wd[1]);
              widen8(r[w].y, wd[2], wd[3]);
              widen8(r[w].z, wd[4], wd[5]);
              widen8(r[w].w, wd[6], wd[7]);
#pragma unroll
              for (uint32_t i = i0; i < i0 + 4; i++) {
                const uint4 qa = *(const uint4 *)(qs + i * RW + 8 * w);
                const uint4 qb = *(const uint4 *)(qs + i * RW + 8 * w + 4);
                uint32_t a = acc[i];
                a = sad2_u16(qa.x, wd[0], a);
                a = sad2_u16(qa.y, wd[1], a);
                a = sad2_u16(qa.z, wd[2], a);
                a = sad2_u16(qa.w, wd[3], a);
                a = sad2_u16(qb.x, wd[4], a);
                a = sad2_u16(qb.y, wd[5], a);
                a = sad2_u16(qb.z, wd[6], a);
                a = sad2_u16(qb.w, wd[7], a);
                acc[i] = a;
              }
            }
          } else {
#pragma unroll
            for (uint32_t w = 0; w < kRowQuads; w++) {
#pragma unroll
              for (uint32_t i = i0; i < i0 + 4; i++) {
                const uint4 q = *(const uint4 *)(qs + i * RW + 4 * w);
                uint32_t a = acc[i];
                a = sad2_u16(q.x, r[w].x, a);
                a = sad2_u16(q.y, r[w].y, a);
                a = sad2_u16(q.z, r[w].z, a);
                a = sad2_u16(q.w, r[w].w, a);
                acc[i] = a;
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (uint32_t i = 0; i < kServeSessions; i++) {
      if (i < ns) {
        const uint64_t v = valid ? ((uint64_t)acc[i] << 32) | tok : ~0ull;
        const uint64_t best = wave_reduce64(v, OpMin());
        if (lane == 0 && best != ~0ull) atomicMin(J.job_best + sid[i], (unsigned long long)best);
      }
    }
  }
}

// Each job's token to the launch's output and to its slot cache's writer memory (the query and
// kept drawers are there already); the drawer counts, the item count and the job flags cleared
// for the next launch. (Run by the scan's last block instead, each block then ending with a
// device-scope release fence before its count, the scan measured 2.6 times slower.)
__global__ __launch_bounds__(256) void fbs_serve_finish(DevModel M, ServeScan J) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0) {
    for (uint32_t c = threadIdx.x; c < M.D; c += blockDim.x) J.drawer_count[c] = 0;
    if (threadIdx.x == 0) J.item_count[0] = 0;
  }
  if (i >= J.n) return;
  // The flag, the minimum and the slot loaded together (one wait), then used.
  const uint32_t flag = J.job_flag[i];
  const uint32_t tok = (uint32_t)J.job_best[i];
  const uint32_t slot = J.cache ? J.slots[i] : 0u;
  if (!flag) return;
  J.job_flag[i] = 0;
  J.out_tokens[(uint64_t)i * (J.gen + 1)] = tok;
  if (J.cache) {
    uint32_t *head = (uint32_t *)(J.cache + (uint64_t)slot * J.cache_stride);
    head[1] = M.writer_memory;
    head[2] = tok;
  }
}

// Sets n words to v (the job buffers' first state; no memset node in a captured launch).
__global__ __launch_bounds__(256) void fbs_fill_u32(uint32_t *p, uint64_t n, uint32_t v) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// The scan over `blocks` wavefronts, then the hand-out.
hipError_t launch_fbs_serve_scan(const DevModel &M, const ServeScan &J, uint32_t blocks,
                                 hipStream_t stream) {
  const uint32_t words = M.d / 2;
  if (words % 16 || blocks == 0) return hipErrorInvalidValue;  // widths are multiples of 32
  DevModel m = M;
  ServeScan j = J;
  void *args[] = {&m, &j};
  const bool t8 = M.table8 != nullptr;
  const void *f = words % 64 == 0   ? (t8 ? (const void *)fbs_serve_scan<64, true>
                                          : (const void *)fbs_serve_scan<64, false>)
                  : words % 32 == 0 ? (t8 ? (const void *)fbs_serve_scan<32, true>
                                          : (const void *)fbs_serve_scan<32, false>)
                                    : (t8 ? (const void *)fbs_serve_scan<16, true>
                                          : (const void *)fbs_serve_scan<16, false>);
  hipError_t e = hipLaunchKernel(f, dim3(blocks), dim3(kWave), args, 0, stream);
  if (e == hipSuccess) e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint32_t fin = (J.n + 255) / 256;
  e = hipLaunchKernel((const void *)fbs_serve_finish, dim3(fin ? fin : 1), dim3(256), args, 0, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

hipError_t launch_fbs_fill_u32(uint32_t *p, uint64_t n, uint32_t v, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint64_t blocks = (n + 255) / 256;
  fbs_fill_u32<<<dim3(blocks < 1024 ? (uint32_t)blocks : 1024u), dim3(256), 0, stream>>>(p, n, v);
  return hipGetLastError();
}

}  // namespace fbs
