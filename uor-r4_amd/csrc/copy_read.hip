// copy_read.hip - the copy heads' Hamming read on MI355X: for the last row of each token stream,
// every copy head picks earlier positions by the XOR-popcount distance between the row's query
// code and the positions' key codes under its rule, and the heads' margin-weighted mean of the
// table rows after those positions is the read (CopyHeads, crates/uor-r4-integer/src/stack/
// hamming.rs:266-538; nearest :690-701, latest_of :584-598, longest_of :601-615, mean_by
// :506-538).
//
// One wavefront reads one stream, four streams per block. Per head the lanes take the candidate
// positions 64 at a time: under the mean rule the distances are staged in LDS and the kept
// positions come out in (distance, position) order as successive wave minima of packed keys;
// the latest and longest rules are wave maxima over the matching positions. The weighted sums
// run with the lanes over the table row's coordinates, in 64-bit integers: a weight is at most
// 2^31 and a table value at most 2^15 in magnitude, so a head's sum over at most 32 positions
// stays below 2^51.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/uor_copy.h"
#include "fbs_int.h"

namespace copyread {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kPerLane = UOR_COPY_MAX_WIDTH / 64;
constexpr uint32_t kPosBits = 20;  // positions below UOR_COPY_MAX_STRIDE fit
constexpr uint32_t kPosMask = (1u << kPosBits) - 1;

struct Dev {
  uint32_t vocab, width, copy, kept, rule, has_marker, m0, m1;
  const uint64_t *codes;
  const int32_t *margins;
  const uint64_t *pair;
  const int16_t *table;
};

struct WaveLds {
  uint8_t dist[UOR_COPY_MAX_STRIDE];
  uint32_t pick[UOR_COPY_MAX_KEPT];  // s | distance << 24
};

template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t lane32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
// Wave minimum / maximum (DPP butterflies in each row of 16, then the rows as scalars).
__device__ __forceinline__ uint32_t wave_min32(uint32_t v) {
  v = min(v, dpp32<0xb1>(v));
  v = min(v, dpp32<0x4e>(v));
  v = min(v, dpp32<0x141>(v));
  v = min(v, dpp32<0x140>(v));
  return min(min(lane32(v, 0), lane32(v, 16)), min(lane32(v, 32), lane32(v, 48)));
}
__device__ __forceinline__ uint32_t wave_max32(uint32_t v) {
  v = max(v, dpp32<0xb1>(v));
  v = max(v, dpp32<0x4e>(v));
  v = max(v, dpp32<0x141>(v));
  v = max(v, dpp32<0x140>(v));
  return max(max(lane32(v, 0), lane32(v, 16)), max(lane32(v, 32), lane32(v, 48)));
}
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t code(const Dev &D, uint32_t token, uint32_t h) {
  return D.codes[(uint64_t)token * D.copy + h];
}
// joined (:379-385): under copy key 2 the near token's first half and the far token's second.
__device__ __forceinline__ uint64_t joined(const Dev &D, uint32_t near, uint32_t far, uint32_t h) {
  const uint64_t c = code(D, near, h), first = D.pair[h];
  return first ? (c & first) | (code(D, far, h) & ~first) : c;
}

// n / k rounded toward zero (Rust's i128 division), for k >= 1, in the integer division of
// fbs_int.h: the kernels divide by no variable with the compiler's `/`, whose expansion goes
// through a float reciprocal estimate.
__device__ __forceinline__ int64_t div_trunc(int64_t n, uint32_t k) {
  const uint64_t q = fbs::div128_64(fbs::uabs64(n), k);
  return n < 0 ? -(int64_t)q : (int64_t)q;
}

// copy_weight_q31 (:243-252), shared with the served step's reads.
__device__ __forceinline__ uint64_t weight_q31(int32_t margin, uint32_t d) {
  return fbs::copy_weight_q31(margin, d);
}

__global__ __launch_bounds__(kThreads) void copy_mean_rows(Dev D, const uint32_t *tokens,
                                                           const int32_t *lengths,
                                                           const uint8_t *opening, uint32_t rows,
                                                           uint32_t stride, int64_t *out,
                                                           uint8_t *found, int32_t *chosen) {
  __shared__ WaveLds lds[kWaves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kWaves + wave;
  if (row >= rows) return;
  WaveLds &w = lds[wave];
  const uint32_t *tok = tokens + (uint64_t)row * stride;
  int len = lengths[row];
  if (len < 0 || len > (int)stride) len = 0;  // outside the row: reads nothing
  bool bad = false;
  for (int i = lane; i < len; i += 64) bad |= tok[i] >= D.vocab;
  if (__any(bad)) len = 0;                     // a token outside the vocabulary: reads nothing
  const int t = len - 1;
  const bool opens = D.has_marker ? (len >= 2 && tok[t - 1] == D.m0 && tok[t] == D.m1)
                                  : (opening != nullptr && opening[row] != 0);
  int64_t sum[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; j++) sum[j] = 0;
  int heads_found = 0;
  for (uint32_t h = 0; h < D.copy; h++) {
    int n = 0;
    if (len >= 1) {
      const uint64_t q = joined(D, tok[t], tok[t > 0 ? t - 1 : 0], h);
      uint32_t rule = D.rule;
      if (rule == UOR_COPY_LONGEST_AFTER_OPENING)
        rule = opens ? UOR_COPY_LATEST_EXACT : UOR_COPY_LONGEST_EXACT;
      if (rule == UOR_COPY_MEAN) {
        for (int s = 1 + lane; s < t; s += 64)
          w.dist[s] = (uint8_t)__popcll(q ^ joined(D, tok[s - 1], tok[s >= 2 ? s - 2 : 0], h));
        wave_sync();
        uint32_t last = 0;  // every key is at least 1 (positions start at 1)
        for (uint32_t r = 0; r < D.kept; r++) {
          uint32_t loc = 0xffffffffu;
          for (int s = 1 + lane; s < t; s += 64) {
            const uint32_t k = (uint32_t)w.dist[s] << kPosBits | (uint32_t)s;
            if (k > last && k < loc) loc = k;
          }
          const uint32_t m = wave_min32(loc);
          if (m == 0xffffffffu) break;
          if (lane == 0) w.pick[r] = (m & kPosMask) | (m >> kPosBits) << 24;
          last = m;
          n++;
        }
      } else if (rule == UOR_COPY_LATEST_EXACT || rule == UOR_COPY_LATEST_NEAREST) {
        uint32_t best = 0xffffffffu;  // distance << 20 | (mask - s): least distance, latest s
        for (int s = 1 + lane; s < t; s += 64) {
          const uint32_t d = __popcll(q ^ joined(D, tok[s - 1], tok[s >= 2 ? s - 2 : 0], h));
          if (rule == UOR_COPY_LATEST_EXACT && d != 0) continue;
          best = min(best, d << kPosBits | (kPosMask - (uint32_t)s));
        }
        const uint32_t m = wave_min32(best);
        if (m != 0xffffffffu) {
          if (lane == 0) w.pick[0] = (kPosMask - (m & kPosMask)) | (m >> kPosBits) << 24;
          n = 1;
        }
      } else {  // longest exact (:601-615) with longer_at (:349-352)
        const int kd = D.pair[h] ? 2 : 1;
        uint32_t ex = 0, lg = 0;
        const uint64_t before = t >= kd ? code(D, tok[t - kd], h) : 0;
        for (int s = 1 + lane; s < t; s += 64) {
          if (joined(D, tok[s - 1], tok[s >= 2 ? s - 2 : 0], h) != q) continue;
          ex = max(ex, (uint32_t)s);
          if (s > kd && code(D, tok[s - 1 - kd], h) == before) lg = max(lg, (uint32_t)s);
        }
        ex = wave_max32(ex);
        lg = wave_max32(lg);
        const uint32_t pick = lg ? lg : ex;
        if (pick) {
          if (lane == 0) w.pick[0] = pick;
          n = 1;
        }
      }
    }
    wave_sync();
    if (chosen != nullptr && lane < (int)D.kept)
      chosen[((uint64_t)row * D.copy + h) * D.kept + lane] = lane < n ? (int32_t)w.pick[lane] : -1;
    int64_t head[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; j++) head[j] = 0;
    int count = 0;
    for (int k = 0; k < n; k++) {
      const uint32_t p = w.pick[k];
      const uint64_t wt = weight_q31(D.margins[h], p >> 24);
      if (wt == 0) continue;
      count++;
      const int16_t *trow = D.table + (uint64_t)tok[p & 0xffffff] * D.width;
#pragma unroll
      for (int j = 0; j < kPerLane; j++) {
        const uint32_t c = (uint32_t)lane + 64u * j;
        if (c < D.width) head[j] += (int64_t)trow[c] * (int64_t)wt;
      }
    }
    if (count) {
      heads_found++;
#pragma unroll
      for (int j = 0; j < kPerLane; j++) sum[j] += div_trunc(head[j], count);
    }
    wave_sync();
  }
#pragma unroll
  for (int j = 0; j < kPerLane; j++) {
    const uint32_t c = (uint32_t)lane + 64u * j;
    if (c < D.width) out[(uint64_t)row * D.width + c] = heads_found ? div_trunc(sum[j], heads_found) : 0;
  }
  if (lane == 0) found[row] = heads_found > 0;
}

// vocab_codes (hamming.rs:566-582): one thread per (token, copy head); the sign word of the
// token's table point through the head's unit rotations (stack_hamilton, the unit on the left;
// the products are exact: |unit| <= 2^31, |point| <= 2^15).
__global__ void copy_vocab_codes(const int64_t *units, const int16_t *table, uint32_t vocab,
                                 uint32_t width, uint32_t head_width, uint32_t copy,
                                 uint64_t *codes) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)vocab * copy) return;
  const uint32_t v = (uint32_t)fbs::div128_64(i, copy), h = (uint32_t)(i - (uint64_t)v * copy);
  const int16_t *row = table + (uint64_t)v * width;
  uint64_t word = 0;
  for (uint32_t c = 0; c < head_width; c += 4) {
    const uint32_t at = h * head_width + c;
    const int64_t *a = units + at;  // the quaternion at / 4
    const int64_t b0 = row[at], b1 = row[at + 1], b2 = row[at + 2], b3 = row[at + 3];
    const int64_t r[4] = {a[0] * b0 - a[1] * b1 - a[2] * b2 - a[3] * b3,
                          a[0] * b1 + a[1] * b0 + a[2] * b3 - a[3] * b2,
                          a[0] * b2 - a[1] * b3 + a[2] * b0 + a[3] * b1,
                          a[0] * b3 + a[1] * b2 - a[2] * b1 + a[3] * b0};
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (r[k] >= 0) word |= 1ull << (c + k);
  }
  codes[i] = word;
}

thread_local std::string g_error;
int fail(int code, const std::string &m) {
  g_error = m;
  return code;
}

struct Handle {
  int device = 0;
  Dev d{};
  void *buf = nullptr;
  ~Handle() {
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    (void)hipFree(buf);
    (void)hipSetDevice(prev);
  }
};

}  // namespace copyread

using namespace copyread;

extern "C" uint32_t uor_copy_abi_version(void) { return UOR_COPY_ABI_VERSION; }
extern "C" const char *uor_copy_last_error(void) { return g_error.c_str(); }

extern "C" int uor_copy_create(const uor_copy_heads *m, int32_t device, void **handle) {
  if (!m || !handle) return fail(-1, "null argument");
  *handle = nullptr;
  if (m->vocabulary < 1 || m->width < 1 || m->width > UOR_COPY_MAX_WIDTH || m->copy < 1 ||
      m->copy > UOR_COPY_MAX_HEADS || m->kept < 1 || m->kept > UOR_COPY_MAX_KEPT ||
      m->rule > UOR_COPY_LONGEST_AFTER_OPENING)
    return fail(-1, "copy heads outside the supported shape");
  if (!m->codes || !m->margins_q16 || !m->pair_first || !m->table) return fail(-1, "null table");
  if (m->has_marker && (m->marker[0] >= m->vocabulary || m->marker[1] >= m->vocabulary))
    return fail(-1, "reply marker outside the vocabulary");
  const size_t nc = (size_t)m->vocabulary * m->copy * 8, nm = (size_t)m->copy * 4,
               np = (size_t)m->copy * 8, nt = (size_t)m->vocabulary * m->width * 2;
  const size_t oc = 0, om = (oc + nc + 255) & ~(size_t)255, op = (om + nm + 255) & ~(size_t)255,
               ot = (op + np + 255) & ~(size_t)255, total = ot + nt;
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (hipSetDevice(device) != hipSuccess) return fail(-2, "hipSetDevice failed");
  Handle *h = new Handle();
  h->device = device;
  char *b = nullptr;
  bool ok = hipMalloc((void **)&b, total) == hipSuccess;
  if (ok) {
    h->buf = b;
    ok = hipMemcpy(b + oc, m->codes, nc, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(b + om, m->margins_q16, nm, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(b + op, m->pair_first, np, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(b + ot, m->table, nt, hipMemcpyHostToDevice) == hipSuccess;
  }
  (void)hipSetDevice(prev);
  if (!ok) {
    delete h;
    return fail(-2, "device allocation or copy failed");
  }
  h->d = Dev{m->vocabulary, m->width, m->copy, m->kept, m->rule, m->has_marker, m->marker[0],
             m->marker[1], (const uint64_t *)(b + oc), (const int32_t *)(b + om),
             (const uint64_t *)(b + op), (const int16_t *)(b + ot)};
  *handle = h;
  return 0;
}

extern "C" void uor_copy_destroy(void *handle) { delete (Handle *)handle; }

extern "C" int uor_copy_mean_rows_async(void *handle, const uint32_t *d_tokens,
                                        const int32_t *d_lengths, const uint8_t *d_opening,
                                        uint32_t rows, uint32_t stride, int64_t *d_out,
                                        uint8_t *d_found, int32_t *d_chosen, void *stream) {
  if (!handle) return fail(-1, "null handle");
  if (rows == 0) return 0;
  if (!d_tokens || !d_lengths || !d_out || !d_found || stride == 0 || stride > UOR_COPY_MAX_STRIDE)
    return fail(-1, "null buffer or stride outside 1..4096");
  Handle *h = (Handle *)handle;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(h->device);
  hipLaunchKernelGGL(copy_mean_rows, dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0,
                     (hipStream_t)stream, h->d, d_tokens, d_lengths, d_opening, rows, stride,
                     d_out, d_found, d_chosen);
  const hipError_t e = hipGetLastError();
  (void)hipSetDevice(prev);
  return e == hipSuccess ? 0 : fail(-2, std::string("launch: ") + hipGetErrorString(e));
}

extern "C" int uor_copy_mean_rows(void *handle, const uint32_t *tokens, const int32_t *lengths,
                                  const uint8_t *opening, uint32_t rows, uint32_t stride,
                                  int64_t *out, uint8_t *found, int32_t *chosen) {
  if (!handle) return fail(-1, "null handle");
  if (rows == 0) return 0;
  if (!tokens || !lengths || !out || !found || stride == 0 || stride > UOR_COPY_MAX_STRIDE)
    return fail(-1, "null buffer or stride outside 1..4096");
  Handle *h = (Handle *)handle;
  for (uint32_t r = 0; r < rows; r++) {
    if (lengths[r] < 0 || (uint32_t)lengths[r] > stride) return fail(-1, "a length exceeds the stride");
    for (int32_t i = 0; i < lengths[r]; i++)
      if (tokens[(size_t)r * stride + i] >= h->d.vocab) return fail(-1, "token outside the vocabulary");
  }
  const size_t nt = (size_t)rows * stride * 4, nl = (size_t)rows * 4, no = (size_t)rows * h->d.width * 8,
               nf = rows, nch = chosen ? (size_t)rows * h->d.copy * h->d.kept * 4 : 0;
  const size_t ot = 0, ol = (nt + 255) & ~(size_t)255, oo = (ol + nl + 255) & ~(size_t)255,
               of = (oo + no + 255) & ~(size_t)255, och = (of + nf + 255) & ~(size_t)255,
               oop = (och + nch + 255) & ~(size_t)255, total = oop + (opening ? rows : 0) + 16;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(h->device);
  char *b = nullptr;
  int rc = 0;
  if (hipMalloc((void **)&b, total) != hipSuccess) {
    rc = fail(-2, "device allocation failed");
  } else {
    if (hipMemcpy(b + ot, tokens, nt, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(b + ol, lengths, nl, hipMemcpyHostToDevice) != hipSuccess ||
        (opening && hipMemcpy(b + oop, opening, rows, hipMemcpyHostToDevice) != hipSuccess)) {
      rc = fail(-2, "copy to the device failed");
    } else {
      rc = uor_copy_mean_rows_async(handle, (const uint32_t *)(b + ot), (const int32_t *)(b + ol),
                                    opening ? (const uint8_t *)(b + oop) : nullptr, rows, stride,
                                    (int64_t *)(b + oo), (uint8_t *)(b + of),
                                    chosen ? (int32_t *)(b + och) : nullptr, nullptr);
      if (rc == 0 && (hipDeviceSynchronize() != hipSuccess ||
                      hipMemcpy(out, b + oo, no, hipMemcpyDeviceToHost) != hipSuccess ||
                      hipMemcpy(found, b + of, nf, hipMemcpyDeviceToHost) != hipSuccess ||
                      (chosen && hipMemcpy(chosen, b + och, nch, hipMemcpyDeviceToHost) != hipSuccess)))
        rc = fail(-2, "the read failed on the device");
    }
    (void)hipFree(b);
  }
  (void)hipSetDevice(prev);
  return rc;
}

extern "C" int uor_copy_vocab_codes(const int32_t *key_rotation, const int16_t *table,
                                    uint32_t vocab, uint32_t width, uint32_t heads_total,
                                    uint32_t copy, int32_t device, uint64_t *codes) {
  if (!key_rotation || !table || !codes) return fail(-1, "null buffer");
  if (vocab < 1 || width < 4 || width % 4 || heads_total < 1 || width % heads_total ||
      (width / heads_total) % 4 || width / heads_total > 64 || copy < 1 || copy > heads_total)
    return fail(-1, "codes need width / heads_total a multiple of 4 and at most 64");
  // The unit rotations g / |g| at Q31 (stack_rotation with lambda 2^31 and epsilon 0).
  std::vector<int64_t> units(width);
  for (uint32_t q = 0; q < width / 4; q++) fbs::rotation(key_rotation + 4 * q, 1ull << 31, 0, &units[4 * q]);
  const size_t nu = (size_t)width * 8, nt = (size_t)vocab * width * 2, nc = (size_t)vocab * copy * 8;
  const size_t ot = (nu + 255) & ~(size_t)255, oc = (ot + nt + 255) & ~(size_t)255;
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (hipSetDevice(device) != hipSuccess) return fail(-2, "hipSetDevice failed");
  char *b = nullptr;
  int rc = 0;
  if (hipMalloc((void **)&b, oc + nc) != hipSuccess) {
    rc = fail(-2, "device allocation failed");
  } else {
    const uint64_t n = (uint64_t)vocab * copy;
    if (hipMemcpy(b, units.data(), nu, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(b + ot, table, nt, hipMemcpyHostToDevice) != hipSuccess) {
      rc = fail(-2, "copy to the device failed");
    } else {
      hipLaunchKernelGGL(copy_vocab_codes, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr,
                         (const int64_t *)b, (const int16_t *)(b + ot), vocab, width,
                         width / heads_total, copy, (uint64_t *)(b + oc));
      if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
          hipMemcpy(codes, b + oc, nc, hipMemcpyDeviceToHost) != hipSuccess)
        rc = fail(-2, "the codes failed on the device");
    }
    (void)hipFree(b);
  }
  (void)hipSetDevice(prev);
  return rc;
}
