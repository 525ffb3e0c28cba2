// fbs_hamming.h - the Hamming reads of a lut-stack/6 stack inside the FBS step (gfx950): the
// copy heads, the type heads (payloads of the hook's input) and the ask heads (a question table
// with its carry), at the stream read after `depth` layers and on the readout
// (RS crates/uor-r4-integer/src/stack/hamming.rs: ServedHamming::stream :1831-1866 and
// readout :1883-1913; session.rs:4252-4276, 4296-4320). Included by fbs_run.h.
//
// One 64-lane wavefront runs a read; the session's tokens x_0..x_t sit in LDS. Each head in turn
// chooses its positions 1 <= s < t by the popcount distance between the row's query code and
// position s's key code (x_{s-1}'s code through the read's key rotation, precomputed per
// vocabulary entry at model creation): `nearest` (:690-701) from a histogram of the distances
// (staged in LDS with them) and one pass that keeps every position nearer than the threshold
// distance and the earliest ones at it, the latest and longest rules (:584-615) as one wave
// minimum or maximum. The chosen positions and their Q31 margin weights
// (`copy_weight_q31` :243-252) go to LDS, uniform for the wave; then every lane sums, for its
// own channels, the weighted values the positions bring back (the table point of the position's
// own token, or the payload kept at the position, which the same lane wrote), divides by the
// head's count, and after the last head by the number of heads that found a position, both
// quotients truncating toward zero (`mean_by` :506-538, :1282-1334). The sums at the hooks are
// formed exactly in 128 bits and rounded once (stream_sum, readout_sum, readout_ask_sum
// :1918-1953). Integer only: the quotients go through fbs_int.h's integer division.
#ifndef UOR_FBS_HAMMING_H
#define UOR_FBS_HAMMING_H

namespace fbs {

constexpr int32_t kCopyMeanExp = -43;       // COPY_MEAN_EXP, hamming.rs:175
constexpr int32_t kHammingWeightExp = -24;  // HAMMING_WEIGHT_EXP, format.rs:59
constexpr uint32_t kTypeMeanShift = 31;     // TYPE_MEAN_SHIFT, hamming.rs:1364
constexpr uint32_t kStreamShift = (uint32_t)(kResidualExp - kHammingWeightExp - kCopyMeanExp);
constexpr uint32_t kNormRaise = (uint32_t)(kNormFineExp - kCopyMeanExp);
constexpr uint32_t kReadoutShift = (uint32_t)(kNormFineExp - kHammingWeightExp - kCopyMeanExp);
constexpr uint32_t kStreamCopyRaise =
    (uint32_t)(kCopyMeanExp - kResidualExp + (int32_t)kTypeMeanShift);
constexpr uint32_t kReadoutTypeDrop =
    (uint32_t)(kCopyMeanExp - kNormFineExp + (int32_t)kTypeMeanShift);
constexpr uint32_t kPosBits = kHamPosBits;  // a packed pick: distance << 24 | position
constexpr uint32_t kPosMask = (1u << kPosBits) - 1;

FBS_HD i128 shl128(i128 v, uint32_t s) { return (i128)((u128)v << s); }

// `round_shift` (:1353-1360): v / 2^s rounded half away from zero, 1 <= s <= 126.
FBS_HD i128 round_shift128(i128 v, uint32_t s) {
  const i128 half = (i128)1 << (s - 1);
  return v >= 0 ? (v + half) >> s : -((half - v) >> s);
}

FBS_HD int64_t clamp_i64(i128 v) {
  return v > (i128)INT64_MAX ? INT64_MAX : v < (i128)INT64_MIN ? INT64_MIN : (int64_t)v;
}

// v / k rounded toward zero (Rust's integer division) by a prepared divisor k >= 1.
FBS_HD int64_t div_trunc64(int64_t v, const Divisor &k) {
  const uint64_t a = v < 0 ? 0 - (uint64_t)v : (uint64_t)v;
  const uint64_t q = divq((u128)a, k);
  return v < 0 ? (int64_t)(0 - q) : (int64_t)q;
}
FBS_HD i128 div_trunc128(i128 v, const Divisor &k) {
  const u128 a = v < 0 ? (u128)0 - (u128)v : (u128)v;
  const uint64_t hi = (uint64_t)(a >> 64), lo = (uint64_t)a;
  const uint64_t qh = divq((u128)hi, k), rh = hi - qh * k.d;
  const uint64_t ql = divq(((u128)rh << 64) | lo, k);  // rh < k, so the quotient fits
  const u128 q = ((u128)qh << 64) | ql;
  return v < 0 ? (i128)((u128)0 - q) : (i128)q;
}

// `stream_sum` (:1918-1925): x + w_c c + w_y y at Q16, formed exactly, rounded once.
FBS_HD int32_t ham_stream_sum(int32_t x, int32_t w_c, i128 c, int32_t w_y, i128 y) {
  constexpr uint32_t sh = kStreamShift + kStreamCopyRaise;
  const i128 sum = shl128(x, sh) + shl128((i128)w_c * c, kStreamCopyRaise) + (i128)w_y * y;
  const i128 r = round_shift128(sum, sh);
  return r > INT32_MAX ? INT32_MAX : r < INT32_MIN ? INT32_MIN : (int32_t)r;
}

// `readout_sum` (:1933-1940): n + [copy matched] w_c (c - n) + w_y y, the type term pre-rounded.
FBS_HD int64_t ham_readout_sum(int64_t n, int32_t w_c, bool has_c, i128 c, int32_t w_y, i128 y) {
  const i128 moved = has_c ? (i128)w_c * (c - shl128(n, kNormRaise)) : 0;
  const i128 typed = round_shift128((i128)w_y * y, kReadoutTypeDrop);
  return clamp_i64(round_shift128(shl128(n, kReadoutShift) + moved + typed, kReadoutShift));
}

// `readout_ask_sum` (:1946-1953): n + [copy matched] w_c (c - n) + [ask matched] w_y (y - n).
FBS_HD int64_t ham_readout_ask_sum(int64_t n, int32_t w_c, bool has_c, i128 c, int32_t w_y,
                                   bool has_y, i128 y) {
  const i128 raised = shl128(n, kNormRaise);
  const i128 copied = has_c ? (i128)w_c * (c - raised) : 0;
  const i128 asked = has_y ? (i128)w_y * (y - raised) : 0;
  return clamp_i64(round_shift128(shl128(n, kReadoutShift) + copied + asked, kReadoutShift));
}

// The sign nibble of unit (x) p (the unit on the left, `head_code` :550-564): bit i is 1 where
// coordinate i is at or above 0.
FBS_HD uint32_t ham_nibble(const int64_t *unit, const int64_t (&p)[4]) {
  const int64_t u[4] = {unit[0], unit[1], unit[2], unit[3]};
  i128 o[4];
  hamilton64(u, p, o);
  return (uint32_t)(o[0] >= 0) | (uint32_t)(o[1] >= 0) << 1 | (uint32_t)(o[2] >= 0) << 2 |
         (uint32_t)(o[3] >= 0) << 3;
}

// A load made a global load: the read's tables are reached through pointers read from memory
// (DevHamRead), which the compiler would otherwise load with flat instructions, and a flat load
// counts against the LDS counter as well, so every later wait for an LDS read would wait for it.
// 8- and 16-byte types load as plain integers and vectors (no constructor of a vector type takes
// a global-space reference).
template <class T>
__device__ __forceinline__ T gload(const T *p) {
  if constexpr (sizeof(T) == 8) {
    typedef __attribute__((address_space(1))) const unsigned long long *G8;
    return __builtin_bit_cast(T, *(G8)p);
  } else if constexpr (sizeof(T) == 16) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) const v4u *G16;
    return __builtin_bit_cast(T, *(G16)p);
  } else {
    typedef __attribute__((address_space(1))) const T *GP;
    return *(GP)p;
  }
}

// ham_nibble with the unit's words read by global loads (the read's tables are reached through
// pointers read from memory, which the compiler would otherwise load as flat).
__device__ __forceinline__ uint32_t ham_nibble_g(const int64_t *unit, const int64_t (&p)[4]) {
  const int64_t u[4] = {gload(unit), gload(unit + 1), gload(unit + 2), gload(unit + 3)};
  return ham_nibble(u, p);
}

// Head j's code word from the sign nibbles of its hw / 4 quaternions in LDS (uniform).
__device__ __forceinline__ uint64_t ham_word(const uint32_t *nib, uint32_t j, uint32_t hw) {
  uint64_t word = 0;
  for (uint32_t c = 0; c < hw; c += 4) word |= (uint64_t)nib[(j * hw + c) >> 2] << c;
  return word;
}

__device__ __forceinline__ uint64_t ham_code(const DevHamRead &R, uint32_t heads, uint32_t token,
                                             uint32_t head) {
  return gload(R.codes + (uint64_t)token * heads + head);
}

// One token's biased table words on the lane's four channels of quaternion q, and their Q12
// values.
__device__ __forceinline__ uint2 ham_point_raw(const DevModel &M, uint32_t token, uint32_t q) {
  return *(const uint2 *)(M.table_b + (uint64_t)token * M.d + 4 * q);
}
__device__ __forceinline__ void ham_point_of(uint2 w, int64_t (&v)[4]) {
  v[0] = (int16_t)(uint16_t)((w.x & 0xffffu) ^ 0x8000u);
  v[1] = (int16_t)(uint16_t)((w.x >> 16) ^ 0x8000u);
  v[2] = (int16_t)(uint16_t)((w.y & 0xffffu) ^ 0x8000u);
  v[3] = (int16_t)(uint16_t)((w.y >> 16) ^ 0x8000u);
}
__device__ __forceinline__ void ham_point(const DevModel &M, uint32_t token, uint32_t q,
                                          int64_t (&v)[4]) {
  const uint2 w = ham_point_raw(M, token, q);
  v[0] = (int16_t)(uint16_t)((w.x & 0xffffu) ^ 0x8000u);
  v[1] = (int16_t)(uint16_t)((w.x >> 16) ^ 0x8000u);
  v[2] = (int16_t)(uint16_t)((w.y & 0xffffu) ^ 0x8000u);
  v[3] = (int16_t)(uint16_t)((w.y >> 16) ^ 0x8000u);
}

// A head's positions at row t under `rule` (0 the mean's `nearest`, 1 latest exact, 2 latest
// nearest, 3 longest exact), position s's key from keyf(s), into S.hpick (position) and S.hwgt
// (Q31 weight): only the positions inside the margin (under the mean rule the `kept` nearest by
// (distance, position), in ascending position). `wd`: the head's weight of each distance
// 0..64 (`copy_weight_q31` of its margin, formed by the host), positive exactly below the
// margin. Returns their count, uniform. For the longest rule, longer(s) says whether one token
// more matches.
// The positions a lane visits are taken kHamBatch at a time, their keys (a token from LDS, then
// a code from the read's table) loaded together before any is used, so that a lane waits for one
// round trip per batch rather than one per position.
constexpr uint32_t kHamBatch = 8;

template <class KeyF, class LongerF>
__device__ __forceinline__ uint32_t ham_choose(const Lds &S, uint32_t rule, uint64_t q, uint32_t t,
                                               uint32_t kept, int32_t margin, const uint32_t *wd,
                                               uint32_t lane, KeyF keyf, LongerF longer) {
  if (t < 2) return 0;
  uint32_t n = 0;
  if (rule == 0) {
    // Distances inside the margin are those below dlim; the histogram and each distance's
    // weight go to LDS.
    const int64_t lim = ((int64_t)margin + 65535) >> 16;
    const uint32_t dlim = lim < 65 ? (uint32_t)lim : 65u;
    for (uint32_t i = lane; i < kHamBins; i += kWave) {
      S.hhist[i] = 0;
      S.hwd[i] = wd[i];
    }
    wave_sync();
    for (uint32_t s0 = 1 + lane; s0 < t; s0 += kHamBatch * kWave) {
      uint64_t key[kHamBatch];
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        key[u] = s < t ? keyf(s) : 0;
      }
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        if (s >= t) break;
        const uint32_t dd = (uint32_t)__popcll(q ^ key[u]);
        S.hdist[s] = (uint8_t)dd;
        if (dd < dlim) atomicAdd(&S.hhist[dd], 1u);
      }
    }
    wave_sync();
    // The threshold: the least distance th at which the positions nearer or equal reach `kept`
    // (then `need` positions at th are taken, the earliest first), else every position inside
    // the margin (th = dlim). Lane l holds distance l's count; a wave prefix sum of the counts
    // and a ballot of the lanes whose running count reaches `kept` find th at once, distance 64
    // (a lane short) after them.
    const uint32_t h = lane < dlim ? S.hhist[lane] : 0u;
    uint32_t cum = h;
#pragma unroll
    for (uint32_t off = 1; off < kWave; off <<= 1) {
      const uint32_t y = (uint32_t)__shfl_up((int)cum, off, kWave);
      cum += lane >= off ? y : 0u;
    }
    const uint64_t reach = __ballot(lane < dlim && cum >= kept);
    uint32_t th = dlim, need = 0;
    if (reach) {
      th = (uint32_t)__builtin_ctzll(reach);
      need = kept - ((uint32_t)__shfl((int)cum, (int)th, kWave) - (uint32_t)__shfl((int)h, (int)th, kWave));
    } else if (dlim > kWave) {
      const uint32_t below64 = (uint32_t)__shfl((int)cum, kWave - 1, kWave);
      if (below64 + S.hhist[kWave] >= kept) {
        th = kWave;
        need = kept - below64;
      }
    }
    // One pass in ascending position: positions nearer than th, and the first `need` at th.
    const uint64_t below = __lanemask_lt();
    uint32_t at = 0;
    for (uint32_t s1 = 1; s1 < t; s1 += 4 * kWave) {  // four rounds' distances read together
      uint32_t dv[4];
#pragma unroll
      for (uint32_t u = 0; u < 4; u++) {
        const uint32_t s = s1 + u * kWave + lane;
        dv[u] = s < t ? S.hdist[s] : 255u;
      }
#pragma unroll
      for (uint32_t u = 0; u < 4; u++) {
        const uint32_t s = s1 + u * kWave + lane, dd = dv[u];
        const uint64_t eq = __ballot(dd == th);
        const bool take = dd < th || (dd == th && at + (uint32_t)__popcll(eq & below) < need);
        const uint64_t tk = __ballot(take);
        if (take) {
          const uint32_t i = n + (uint32_t)__popcll(tk & below);
          S.hpick[i] = s;
          S.hwgt[i] = S.hwd[dd];
        }
        n += (uint32_t)__popcll(tk);
        at += (uint32_t)__popcll(eq);
      }
    }
  } else if (rule <= 2) {
    uint32_t best = UINT32_MAX;
    for (uint32_t s0 = 1 + lane; s0 < t; s0 += kHamBatch * kWave) {
      uint64_t key[kHamBatch];
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        key[u] = s < t ? keyf(s) : 0;
      }
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        const uint32_t dd = (uint32_t)__popcll(q ^ key[u]);
        const uint32_t k = dd << kPosBits | (kPosMask - s);
        best = s < t && (rule != 1 || dd == 0) && k < best ? k : best;
      }
    }
    const uint32_t m = wave_reduce32(best, OpMin());
    const uint32_t w = m == UINT32_MAX ? 0 : wd[m >> kPosBits];
    if (w) {
      if (lane == 0) {
        S.hpick[0] = kPosMask - (m & kPosMask);
        S.hwgt[0] = w;
      }
      n = 1;
    }
  } else {
    uint32_t ex = 0, lg = 0;
    for (uint32_t s0 = 1 + lane; s0 < t; s0 += kHamBatch * kWave) {
      uint64_t key[kHamBatch];
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        key[u] = s < t ? keyf(s) : ~q;
      }
#pragma unroll
      for (uint32_t u = 0; u < kHamBatch; u++) {
        const uint32_t s = s0 + u * kWave;
        if (s >= t || key[u] != q) continue;
        ex = s > ex ? s : ex;
        if (longer(s)) lg = s > lg ? s : lg;
      }
    }
    ex = wave_reduce32(ex, OpMax());
    lg = wave_reduce32(lg, OpMax());
    const uint32_t pick = lg ? lg : ex;
    const uint32_t w = pick ? wd[0] : 0;
    if (w) {
      if (lane == 0) {
        S.hpick[0] = pick;
        S.hwgt[0] = w;
      }
      n = 1;
    }
  }
  wave_sync();
  return n;
}

// The forced replay (Q5's, claude-249; HeadForce and `forcing`, :1397-1421, 1686-1740): head
// `head` of read `ri`'s forced query at step `step` (role 0) or candidate key (role 1), if any.
__device__ __forceinline__ bool dt_forced(const DtCtx *dc, const DevHam &H, uint32_t ri,
                                          uint32_t head, uint32_t step, uint32_t role,
                                          uint64_t &code) {
  if (!dc->mask) return false;
  const uint64_t at = ((uint64_t)step * H.nreads + ri) * H.heads + head;
  if (!((dc->mask[at] >> role) & 1u)) return false;
  code = dc->codes[2 * at + role];
  return true;
}

// One head's trace record at row t (`record`, :1787-1814): the query, the key at the row, and
// the kept positions as `nearest` keeps them (the kept nearest by (distance, position), every
// distance counted; :690-701) or the rule's one position (`latest_of`, `longest_of`), whatever
// the margin then weighs them. Run before the served choice, which overwrites the picks.
template <class KeyF, class LongerF>
__device__ __forceinline__ void ham_trace_head(const Lds &S, const DevHam &H, uint32_t rule,
                                               uint64_t q, uint64_t kt, uint32_t t, uint32_t lane,
                                               KeyF keyf, LongerF longer, uint8_t *rec) {
  const uint32_t n = ham_choose(S, rule, q, t, H.kept, INT32_MAX, H.ones, lane, keyf, longer);
  uint32_t *kept = (uint32_t *)(rec + 20);
  if (rule == 0) {
    for (uint32_t i = lane; i < n; i += kWave) {
      const uint32_t si = S.hpick[i], di = S.hdist[si];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < n; j++) {
        const uint32_t sj = S.hpick[j], dj = S.hdist[sj];
        rank += dj < di || (dj == di && sj < si) ? 1u : 0u;
      }
      kept[rank] = si;
    }
  } else if (lane == 0 && n) {
    kept[0] = S.hpick[0];
  }
  if (lane == 0) {
    *(uint64_t *)rec = q;
    *(uint64_t *)(rec + 8) = kt;
    *(uint32_t *)(rec + 16) = n;
  }
  wave_sync();
}

// The copy heads' mean at row t (`CopyHeads::mean_at` :482-504) on the lane's channels into cm
// (at 2^-43; |cm| < 2^53, so 64 bits hold it). Returns whether a head found a position.
// The copy heads h0, h0 + hs, ... below the copy count: each head that finds a position adds its
// mean (truncating toward zero) into cm; returns how many did. ham_copy_mean divides the sum by
// the count once every head has added (the sum of exact integers does not depend on the order).
template <int Q, bool DT = false>
__device__ __forceinline__ uint32_t ham_copy_part(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                                  const Lds &S, uint32_t t, uint32_t lane,
                                                  const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                                  int64_t (&cm)[Q][4], const DtCtx *dc,
                                                  uint32_t h0, uint32_t hs) {
  const DevHam &H = M.ham;
  const uint32_t *tk = S.tok;
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) cm[k][c] = 0;
  uint32_t rule = H.rule;
  if (rule == 4)  // longest after opening: the opening row is found from the marker
    rule = H.has_marker && t >= 1 && tk[t - 1] == H.m0 && tk[t] == H.m1 ? 1u : 3u;
  uint32_t found = 0;
  for (uint32_t h = h0; h < H.copy; h += hs) {
    const uint64_t first = H.pair[h];
    auto joined = [&](uint32_t near, uint32_t far) -> uint64_t {
      const uint64_t code = ham_code(R, H.heads, near, h);
      return first ? (code & first) | (ham_code(R, H.heads, far, h) & ~first) : code;
    };
    uint64_t q = joined(tk[t], tk[t ? t - 1 : 0]);
    if (DT) dt_forced(dc, H, ri, h, t, 0, q);
    const uint32_t kd = first ? 2 : 1;
    const uint64_t before = t >= kd ? ham_code(R, H.heads, tk[t - kd], h) : 0;
    auto keyf = [&](uint32_t s) {
      uint64_t k = joined(tk[s - 1], tk[s >= 2 ? s - 2 : 0]);
      if (DT) dt_forced(dc, H, ri, h, s, 1, k);
      return k;
    };
    // The longer test reads the tokens, which a replay does not force.
    auto longer = [&](uint32_t s) { return s > kd && ham_code(R, H.heads, tk[s - 1 - kd], h) == before; };
    if (DT && dc->rec) {
      const uint64_t kt = t ? keyf(t) : 0;
      ham_trace_head(S, H, rule, q, kt, t, lane, keyf, longer,
                     dc->rec + dc->reads_at + (R.heads_before + h) * decision_head_bytes(H.kept));
    }
    const uint32_t n = ham_choose(S, rule, q, t, H.kept, R.margin[h], R.wd + h * kHamBins, lane,
                                  keyf, longer);
    if (!n) continue;
    found++;
    const Divisor dv = make_divisor(n);
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) continue;
      int64_t acc[4] = {0, 0, 0, 0};
      for (uint32_t i0 = 0; i0 < n; i0 += 16) {  // sixteen positions' points loaded together
        uint2 raw[16];
#pragma unroll
        for (uint32_t u = 0; u < 16; u++) {
          const uint32_t i = i0 + u;
          raw[u] = i < n ? ham_point_raw(M, tk[S.hpick[i]], qi[k]) : make_uint2(0x80008000u, 0x80008000u);
        }
#pragma unroll
        for (uint32_t u = 0; u < 16; u++) {
          const uint32_t i = i0 + u;
          const int64_t w = i < n ? S.hwgt[i] : 0;
          int64_t v[4];
          ham_point_of(raw[u], v);
#pragma unroll
          for (int c = 0; c < 4; c++) acc[c] += v[c] * w;
        }
      }
#pragma unroll
      for (int c = 0; c < 4; c++) cm[k][c] += div_trunc64(acc[c], dv);
    }
    wave_sync();  // the picks are read before the next head writes them
  }
  return found;
}

template <int Q>
__device__ __forceinline__ void ham_finish64(int64_t (&cm)[Q][4], uint32_t found) {
  const Divisor dv = make_divisor(found);
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) cm[k][c] = div_trunc64(cm[k][c], dv);
}

template <int Q>
__device__ __forceinline__ void ham_finish128(i128 (&ym)[Q][4], uint32_t found) {
  const Divisor dv = make_divisor(found);
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) ym[k][c] = div_trunc128(ym[k][c], dv);
}

template <int Q, bool DT = false>
__device__ __forceinline__ bool ham_copy_mean(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                              const Lds &S, uint32_t t, uint32_t lane,
                                              const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                              int64_t (&cm)[Q][4], const DtCtx *dc = nullptr) {
  const uint32_t found = ham_copy_part<Q, DT>(M, R, ri, S, t, lane, qv, qi, cm, dc, 0, 1);
  if (!found) return false;
  ham_finish64<Q>(cm, found);
  return true;
}

// The type heads' mean at row t (`ServedHamming::type_mean` :1750-1783) into ym. A read that
// asks (`asked_point` :1161-1181, `ask_queries` :1185-1190) asks with the sign codes of
// (table + a)[x_t] 2^16 + sum_{s <= min(h, t)} c[x_{t-s}] (table + a)[x_{t-s}] through the key
// rotation and brings back the kept tokens' table points (ym at 2^-43); otherwise `point`'s
// payload (`payload` :1204-1215) is kept at row t of `pay` first, the query codes are `point`'s
// through the query rotation and the kept positions' payloads come back (ym at the point's
// exponent minus 31). Returns whether a head found a position.
// The type heads j0, j0 + js, ... below the head count (as ham_copy_part): the point's payload
// is kept at row t first where `write_pay` (one wavefront of a block writes it).
template <int Q, bool DT = false>
__device__ __forceinline__ uint32_t ham_type_part(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                                  const Lds &S, uint32_t t, uint32_t lane,
                                                  const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                                  const int64_t (&point)[Q][4], int64_t *pay,
                                                  i128 (&ym)[Q][4], const DtCtx *dc, uint32_t j0,
                                                  uint32_t js, bool write_pay) {
  const DevHam &H = M.ham;
  const uint32_t d = M.d, *tk = S.tok;
  const bool asks = R.ask != nullptr;
#pragma unroll
  for (int k = 0; k < Q; k++) {
#pragma unroll
    for (int c = 0; c < 4; c++) ym[k][c] = 0;
    if (!qv[k]) continue;
    const uint32_t q = qi[k];
    if (asks) {
      auto asked = [&](uint32_t v, int64_t (&o)[4]) {
        ham_point(M, v, q, o);
        const short4 a = gload((const short4 *)(R.ask + (uint64_t)v * d + 4 * q));
        o[0] += a.x;
        o[1] += a.y;
        o[2] += a.z;
        o[3] += a.w;
      };
      int64_t p[4];
      asked(tk[t], p);
#pragma unroll
      for (int c = 0; c < 4; c++) p[c] *= 65536;
      if (R.carry) {
        const uint32_t reach = R.carry_rows < t ? R.carry_rows : t;
        for (uint32_t s = 1; s <= reach; s++) {
          const uint32_t v = tk[t - s];
          const int64_t gain = gload(R.carry + v);
          int64_t o[4];
          asked(v, o);
#pragma unroll
          for (int c = 0; c < 4; c++) p[c] += gain * o[c];
        }
      }
      S.hnib[q] = ham_nibble_g(R.ku + 4 * q, p);
    } else {
      i128 o[4];
      const int64_t u[4] = {gload(R.vu + 4 * q), gload(R.vu + 4 * q + 1), gload(R.vu + 4 * q + 2),
                            gload(R.vu + 4 * q + 3)};
      hamilton64(u, point[k], o);
      if (write_pay) {
        int64_t *dst = pay + (uint64_t)t * d + 4 * q;
        *(longlong2 *)dst = make_longlong2(clamp_i64(round_shift128(o[0], 31)),
                                           clamp_i64(round_shift128(o[1], 31)));
        *(longlong2 *)(dst + 2) = make_longlong2(clamp_i64(round_shift128(o[2], 31)),
                                                 clamp_i64(round_shift128(o[3], 31)));
      }
      S.hnib[q] = ham_nibble_g(R.qu + 4 * q, point[k]);
    }
  }
  wave_sync();
  uint32_t found = 0;
  for (uint32_t j = j0; j < H.heads; j += js) {
    uint64_t q = ham_word(S.hnib, j, H.hw);
    if (DT) dt_forced(dc, H, ri, j, t, 0, q);
    auto keyf = [&](uint32_t s) {
      uint64_t k = ham_code(R, H.heads, tk[s - 1], j);
      if (DT) dt_forced(dc, H, ri, j, s, 1, k);
      return k;
    };
    auto never = [&](uint32_t) { return false; };
    if (DT && dc->rec) {
      const uint64_t kt = t ? keyf(t) : 0;
      ham_trace_head(S, H, 0, q, kt, t, lane, keyf, never,
                     dc->rec + dc->reads_at + (R.heads_before + j) * decision_head_bytes(H.kept));
    }
    const uint32_t n = ham_choose(S, 0, q, t, H.kept, R.margin[j], R.wd + j * kHamBins, lane,
                                  keyf, never);
    if (!n) continue;
    found++;
    const Divisor dv = make_divisor(n);
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) continue;
      i128 acc[4] = {0, 0, 0, 0};
      for (uint32_t i0 = 0; i0 < n; i0 += 4) {  // four positions' values loaded together
        int64_t v[4][4], w[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
          const uint32_t i = i0 + u;
          w[u] = i < n ? S.hwgt[i] : 0;
          v[u][0] = v[u][1] = v[u][2] = v[u][3] = 0;
          if (i >= n) continue;
          const uint32_t s = S.hpick[i];
          if (asks) {
            ham_point(M, tk[s], qi[k], v[u]);
          } else {
            const longlong2 *src = (const longlong2 *)(pay + (uint64_t)s * d + 4 * qi[k]);
            const longlong2 a = src[0], b = src[1];
            v[u][0] = a.x;
            v[u][1] = a.y;
            v[u][2] = b.x;
            v[u][3] = b.y;
          }
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; u++)
#pragma unroll
          for (int c = 0; c < 4; c++) acc[c] += (i128)v[u][c] * w[u];
      }
#pragma unroll
      for (int c = 0; c < 4; c++) ym[k][c] += div_trunc128(acc[c], dv);
    }
    wave_sync();
  }
  return found;
}

template <int Q, bool DT = false>
__device__ __forceinline__ bool ham_type_mean(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                              const Lds &S, uint32_t t, uint32_t lane,
                                              const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                              const int64_t (&point)[Q][4], int64_t *pay,
                                              i128 (&ym)[Q][4], const DtCtx *dc = nullptr) {
  const uint32_t found = ham_type_part<Q, DT>(M, R, ri, S, t, lane, qv, qi, point, pay, ym, dc,
                                              M.ham.copy, 1, true);
  if (!found) return false;
  ham_finish128<Q>(ym, found);
  return true;
}

// ---- The place read (fbs_snapshot.rs:2716-3135, served by hamming.rs:1510-1533 and 1625-1634) --
// The readout read's ask heads find a place in the session's finished user turns; the register
// over the session's tokens holds it from the reply's start, and a reply row it opens reads the
// token at the place (ham_readout). The sequence's register sits in LDS: kPlaceWords scalars
// (below), per position the end of the finished user turn that holds it (`uend`, 0 for none) and,
// at a row of a user turn's content whose token arms, the place its question found + 1 (`farm`;
// only an arming row's find can set the register, so no other row's is kept). Every lane runs the
// register's scalar program on the same values; lane 0 writes them back.
enum : uint32_t {
  kPlRole = 0,   // the turn being read: 0 none, 1 system, 2 user, 3 assistant
  kPlStart,      // its first content row
  kPlUsers,      // the document's finished user turns
  kPlLastA,      // the last of them: its content [a, b)
  kPlLastB,
  kPlDoc,        // the document's first row (positions before it belong to a forgotten one)
  kPlHas,        // the register is set: a place and the end of its turn's content
  kPlPlace,
  kPlEnd,
  kPlOffer,      // the place offered at the row read last, or kPlaceNone
  kPlOver,       // the reply being read reached its end mark
  kPlAnswered,   // a reply started since the last user turn did
};

// A fresh register (PlaceState::default) and empty per-position tables.
__device__ __forceinline__ void place_init(const DevModel &M, const Lds &S, uint32_t lane) {
  for (uint32_t i = lane; i < kPlaceWords; i += kWave) S.pst[i] = i == kPlOffer ? kPlaceNone : 0u;
  for (uint32_t i = lane; i < M.context; i += kWave) {
    S.uend[i] = 0;
    S.farm[i] = 0;
  }
  wave_sync();
}

// The find of the question at row t (ServedPlace::find, hamming.rs:1525-1533; place_find and
// place_pick, fbs_snapshot.rs:3093-3135): head j (a type head of the readout read) asks with the
// sign code of the ask point of x_t (the question table and carry, window from row 0) through
// the key rotation in the first half of its bits and x_{t-1}'s key code in the rest; its key at
// position s is x_{s-1}'s key code in the first half and x_{s-2}'s in the rest. Over the
// positions s >= 2 of the document's finished user turns, the nearest key (the later on ties)
// inside the head's margin (m > d 2^16); then the later of the heads' positions. Returns the
// place + 1, or 0. Uniform.
template <int Q>
__device__ __forceinline__ uint32_t place_find(const DevModel &M, const Lds &S, uint32_t t,
                                               uint32_t doc, uint32_t lane, const bool (&qv)[Q],
                                               const uint32_t (&qi)[Q]) {
  const DevHam &H = M.ham;
  const DevHamRead &R = H.reads[H.p_read];
  const uint32_t d = M.d, *tk = S.tok;
  if (t < 1) return 0;
#pragma unroll
  for (int k = 0; k < Q; k++) {
    if (!qv[k]) continue;
    const uint32_t q = qi[k];
    auto asked = [&](uint32_t v, int64_t (&o)[4]) {
      ham_point(M, v, q, o);
      const short4 a = *(const short4 *)(H.p_ask + (uint64_t)v * d + 4 * q);
      o[0] += a.x;
      o[1] += a.y;
      o[2] += a.z;
      o[3] += a.w;
    };
    int64_t p[4];
    asked(tk[t], p);
#pragma unroll
    for (int c = 0; c < 4; c++) p[c] *= 65536;
    if (H.p_carry) {
      const uint32_t reach = H.p_carry_rows < t ? H.p_carry_rows : t;
      for (uint32_t s = 1; s <= reach; s++) {
        const uint32_t v = tk[t - s];
        const int64_t gain = gload(H.p_carry + v);
        int64_t o[4];
        asked(v, o);
#pragma unroll
        for (int c = 0; c < 4; c++) p[c] += gain * o[c];
      }
    }
    S.hnib[q] = ham_nibble_g(R.ku + 4 * q, p);
  }
  wave_sync();
  const uint64_t first = (1ull << (H.hw / 2)) - 1;
  const uint32_t s0 = doc > 2 ? doc : 2u;
  uint32_t found = 0;
  for (uint32_t j = H.copy; j < H.heads; j++) {
    const uint64_t q = (ham_word(S.hnib, j, H.hw) & first) | (ham_code(R, H.heads, tk[t - 1], j) & ~first);
    uint32_t best = UINT32_MAX;
    for (uint32_t s = s0 + lane; s < t; s += kWave) {
      if (!S.uend[s]) continue;
      const uint64_t key = (ham_code(R, H.heads, tk[s - 1], j) & first) |
                           (ham_code(R, H.heads, tk[s - 2], j) & ~first);
      const uint32_t k = (uint32_t)__popcll(q ^ key) << kPosBits | (kPosMask - s);
      best = k < best ? k : best;
    }
    const uint32_t m = wave_reduce32(best, OpMin());
    if (m != UINT32_MAX && (int64_t)R.margin[j] > ((int64_t)(m >> kPosBits) << 16)) {
      const uint32_t s = kPosMask - (m & kPosMask);
      found = s + 1 > found ? s + 1 : found;
    }
  }
  return found;
}

// The register's step at row t (PlaceState::advance without a caller's asks,
// fbs_snapshot.rs:2937-3090, with PlaceTurns::push :2801-2837): the step of the place held by
// the row before, the turns, the arm at a reply's start, the find at an arming row of a user
// turn's content, the stop at the reply's end mark, and the offer of an open reply row.
template <int Q>
__device__ __forceinline__ void place_advance(const DevModel &M, const Lds &S, uint32_t t,
                                              uint32_t lane, const bool (&qv)[Q],
                                              const uint32_t (&qi)[Q]) {
  const DevHam &H = M.ham;
  const uint32_t *tk = S.tok;
  uint32_t *ps = S.pst;
  uint32_t role = ps[kPlRole], start = ps[kPlStart], users = ps[kPlUsers];
  uint32_t la = ps[kPlLastA], lb = ps[kPlLastB], doc = ps[kPlDoc];
  uint32_t place = ps[kPlPlace], pend = ps[kPlEnd];
  bool has = ps[kPlHas] != 0, over = ps[kPlOver] != 0, answered = ps[kPlAnswered] != 0;
  const uint32_t at = ps[kPlOffer], token = tk[t], len = t + 1;
  auto cls = [&](uint32_t v) -> uint32_t { return v < M.vocab ? (uint32_t)H.p_class[v] : 0u; };
  // The step: the row before was offered the token at the place, and this token is it.
  bool stepped = false;
  if (at != kPlaceNone && has && at == place && token == tk[place]) {
    const uint32_t next = place + 1;
    if (next >= pend || (cls(tk[next]) & kPlaceStop)) {
      has = false;
    } else {
      place = next;
      stepped = true;
    }
  }
  uint32_t pushed = 0;
  if (token == H.p_bos) {  // the start mark forgets the document
    has = false;
    answered = false;
    role = start = users = 0;
    doc = len;
  } else {
    const uint32_t sl = H.p_len[0];
    for (uint32_t r = 1; r <= 3 && !pushed; r++) {
      const uint32_t ml = H.p_len[r];
      if (!ml || ml > len) continue;
      const uint32_t *mk = H.p_marks + r * kPlaceMarkMax;
      bool ends = true;
      for (uint32_t i = 0; i < ml; i++) ends = ends && tk[len - ml + i] == mk[i];
      if (!ends) continue;
      const uint32_t m = len - ml;
      bool after = m >= sl;
      for (uint32_t i = 0; i < sl && after; i++) after = tk[m - sl + i] == H.p_marks[i];
      if (role == 0) {
        if (!(m > 0 && (tk[m - 1] == H.p_bos || after))) continue;
      } else {
        if (!(after && m >= start + sl)) continue;
        uint32_t b = m - sl;
        if (b > start && tk[b - 1] == H.p_eos) b--;
        if (role == 2) {
          for (uint32_t s = start + lane; s < b; s += kWave) S.uend[s] = (uint16_t)b;
          users++;
          la = start;
          lb = b;
        }
      }
      role = r;
      start = len;
      pushed = r;
    }
  }
  wave_sync();
  if (pushed == 2) {  // a user turn's start clears the register
    has = false;
    answered = false;
  } else if (pushed == 3) {  // a reply's start: the arm, once per user turn
    over = false;
    has = false;
    const bool asked = users > 0 && !answered;
    answered = true;
    if (asked) {
      uint32_t last = 0;  // the last arming row of the answered turn's content + 1
      for (uint32_t r = la + lane; r < lb; r += kWave)
        if (S.farm[r]) last = r + 1;
      last = wave_reduce32(last, OpMax());
      if (last) {
        const uint32_t pos = (uint32_t)S.farm[last - 1] - 1u;
        const uint32_t e = pos >= doc && pos < la ? (uint32_t)S.uend[pos] : 0u;
        if (e) {
          has = true;
          place = pos;
          pend = e;
        }
      }
    }
  }
  uint32_t offer = kPlaceNone;
  if (role == 2 && t >= start && users > 0) {
    if (cls(token) & kPlaceArm) {
      const uint32_t f = place_find<Q>(M, S, t, doc, lane, qv, qi);
      if (f && lane == 0) S.farm[t] = (uint16_t)f;
    }
  } else if (role == 3) {
    if (token == H.p_eos && t >= start) {
      over = true;
      has = false;
    }
    if (t + 1 >= start && !over && has && (stepped || (cls(token) & kPlaceOpen))) offer = place;
  }
  if (lane == 0) {
    ps[kPlRole] = role;
    ps[kPlStart] = start;
    ps[kPlUsers] = users;
    ps[kPlLastA] = la;
    ps[kPlLastB] = lb;
    ps[kPlDoc] = doc;
    ps[kPlHas] = has;
    ps[kPlPlace] = place;
    ps[kPlEnd] = pend;
    ps[kPlOffer] = offer;
    ps[kPlOver] = over;
    ps[kPlAnswered] = answered;
  }
  wave_sync();
}

// Both wavefronts of a paired block meet at a read: their LDS and global writes before it (the
// point, the partial sums, the payloads) are visible to the other after it.
__device__ __forceinline__ void hook_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Where a paired block's second wavefront reads and writes during a read (the LDS a read leaves
// unused): its distances, picks, weights, histogram and nibbles in the writer's staging list;
// the point it reads and the partial sums it returns (d i64, then d i128 as low and high i64
// halves) over the gather crossbar, the MLP outputs and the drawer scores, which lie contiguous
// (ham_pair_fits on the host).
__device__ __forceinline__ Lds ham_help_lds(const DevModel &M, const Lds &S0) {
  Lds S = S0;
  uint8_t *base = (uint8_t *)S0.list;
  S.hdist = base;
  base += (M.context + 15u) & ~15u;
  S.hpick = (uint32_t *)base;
  S.hwgt = S.hpick + kMaxHamKept;
  S.hhist = S.hwgt + kMaxHamKept;
  S.hwd = S.hhist + kHamBins;
  S.hnib = S.hwd + kHamBins;
  return S;
}

// A read's two means at row t (the copy heads' unless `skip_copy`, the type heads' where the read
// serves them; `point` the hook's input): on one wavefront, or (PAIR) with the paired block's
// second wavefront (ham_help), which takes the odd heads of each kind: the first publishes the
// request and the point, takes the even heads, and adds the second's partial sums and counts
// before the divisions; the sums are of exact integers, so the heads' order does not change them.
template <int Q, bool DT, bool PAIR>
__device__ __forceinline__ void ham_read_means(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                               const Lds &S, uint32_t t, int64_t *pay,
                                               uint32_t lane, const bool (&qv)[Q],
                                               const uint32_t (&qi)[Q],
                                               const int64_t (&point)[Q][4], bool skip_copy,
                                               int64_t (&cm)[Q][4], i128 (&ym)[Q][4],
                                               bool &has_c, bool &has_y, const DtCtx *dc) {
  int64_t *cache = R.typed && !R.ask ? pay + (uint64_t)R.slot * M.context * M.d : nullptr;
  if constexpr (PAIR) {
    static_assert(!DT, "the traced kernels run on one wavefront");
    int64_t *pc = (int64_t *)S.xbar;
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) pc[4 * qi[k] + c] = point[k][c];
    if (lane == 0) {
      S.hreq[0] = ri;
      S.hreq[1] = t;
      S.hreq[2] = skip_copy;
    }
    hook_sync();  // the request and the point
    uint32_t fc = 0, fy = 0;
    if (!skip_copy) {
      fc = ham_copy_part<Q>(M, R, ri, S, t, lane, qv, qi, cm, nullptr, 0, 2);
    } else {
#pragma unroll
      for (int k = 0; k < Q; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) cm[k][c] = 0;
    }
    if (R.typed) {
      fy = ham_type_part<Q>(M, R, ri, S, t, lane, qv, qi, point, cache, ym, nullptr, M.ham.copy, 2, true);
    } else {
#pragma unroll
      for (int k = 0; k < Q; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) ym[k][c] = 0;
    }
    hook_sync();  // the second wavefront's partial sums and counts
    const int64_t *py = pc + M.d;
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint32_t ch = 4 * qi[k] + c;
          cm[k][c] += pc[ch];
          ym[k][c] += (i128)(((u128)(uint64_t)py[M.d + ch] << 64) | (u128)(uint64_t)py[ch]);
        }
    fc += S.hreq[6];
    fy += S.hreq[7];
    has_c = fc != 0;
    has_y = fy != 0;
    if (has_c) ham_finish64<Q>(cm, fc);
    if (has_y) ham_finish128<Q>(ym, fy);
  } else {
    has_c = false;
    if (!skip_copy) {
      has_c = ham_copy_mean<Q, DT>(M, R, ri, S, t, lane, qv, qi, cm, dc);
    } else if (DT && dc->rec && M.ham.copy) {
      // The trace records the copy heads' choices at an open row too (`record` runs first).
      ham_copy_mean<Q, DT>(M, R, ri, S, t, lane, qv, qi, cm, dc);
    }
    has_y = R.typed && ham_type_mean<Q, DT>(M, R, ri, S, t, lane, qv, qi, point, cache, ym, dc);
  }
}

// The paired block's second wavefront at a read the first requests (ham_read_means): the odd
// copy and type heads over its own scratch (ham_help_lds), then its partial sums over the point it
// read and its counts in the request. Two hook barriers, as the first wavefront's.
template <int Q>
__device__ __forceinline__ void ham_help(const DevModel &M, const Lds &S0, int64_t *pay,
                                         uint32_t lane, const bool (&qv)[Q],
                                         const uint32_t (&qi)[Q]) {
  hook_sync();  // the request and the point
  const Lds S = ham_help_lds(M, S0);
  const uint32_t ri = S0.hreq[0], t = S0.hreq[1];
  const bool skip_copy = S0.hreq[2] != 0;
  const DevHamRead &R = M.ham.reads[ri];
  int64_t *pc = (int64_t *)S0.xbar, *py = pc + M.d;
  int64_t point[Q][4];
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) point[k][c] = qv[k] ? pc[4 * qi[k] + c] : 0;
  int64_t cm[Q][4];
  i128 ym[Q][4];
  uint32_t fc = 0, fy = 0;
  if (!skip_copy) {
    fc = ham_copy_part<Q>(M, R, ri, S, t, lane, qv, qi, cm, nullptr, 1, 2);
  } else {
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) cm[k][c] = 0;
  }
  if (R.typed) {
    int64_t *cache = R.ask ? nullptr : pay + (uint64_t)R.slot * M.context * M.d;
    fy = ham_type_part<Q>(M, R, ri, S, t, lane, qv, qi, point, cache, ym, nullptr, M.ham.copy + 1, 2,
                          false);
  } else {
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) ym[k][c] = 0;
  }
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k])
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const uint32_t ch = 4 * qi[k] + c;
        pc[ch] = cm[k][c];
        py[ch] = (int64_t)(uint64_t)(u128)ym[k][c];
        py[M.d + ch] = (int64_t)(uint64_t)((u128)ym[k][c] >> 64);
      }
  if (lane == 0) {
    S0.hreq[6] = fc;
    S0.hreq[7] = fy;
  }
  hook_sync();  // the partial sums and counts
}

// The stream read after `depth` layers (< the layer count) on the residual x, in place. `pay`:
// the sequence's payload caches, [slot][context][d].
template <int Q, bool DT = false, bool PAIR = false>
__device__ __forceinline__ void ham_stream(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                           const Lds &S, uint32_t t, int64_t *pay, uint32_t lane,
                                           const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                           int32_t (&x)[Q][4], const DtCtx *dc = nullptr) {
  int64_t cm[Q][4], point[Q][4];
  i128 ym[Q][4];
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) point[k][c] = x[k][c];
  bool has_c, has_y;
  ham_read_means<Q, DT, PAIR>(M, R, ri, S, t, pay, lane, qv, qi, point, false, cm, ym, has_c, has_y, dc);
  if (has_y && R.ask)
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) ym[k][c] = shl128(ym[k][c], kStreamCopyRaise);
  if (!has_c && !has_y) return;
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      const int4 wc = *(const int4 *)(R.w + 4 * qi[k]);
      const int4 wy = *(const int4 *)(R.w + M.d + 4 * qi[k]);
      const int32_t a[4] = {wc.x, wc.y, wc.z, wc.w}, b[4] = {wy.x, wy.y, wy.z, wy.w};
#pragma unroll
      for (int c = 0; c < 4; c++)
        x[k][c] = ham_stream_sum(x[k][c], a[c], has_c ? (i128)cm[k][c] : 0, b[c],
                                 has_y ? ym[k][c] : 0);
    }
}

// The readout read on the final norm's output n (at 2^-24), in place.
template <int Q, bool DT = false, bool PAIR = false>
__device__ __forceinline__ void ham_readout(const DevModel &M, const DevHamRead &R, uint32_t ri,
                                            const Lds &S, uint32_t t, int64_t *pay, uint32_t lane,
                                            const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                            int64_t (&n)[Q][4], const DtCtx *dc = nullptr) {
  int64_t cm[Q][4];
  i128 ym[Q][4];
  // At a row the place read opens, the table's point of the token at the place, at
  // 2^COPY_MEAN_EXP (a Q12 point at a Q31 weight of one), in place of the copy heads' mean
  // (hamming.rs:1895-1899).
  const uint32_t offer = M.ham.place ? S.pst[kPlOffer] : kPlaceNone;
  bool has_c, has_y;
  ham_read_means<Q, DT, PAIR>(M, R, ri, S, t, pay, lane, qv, qi, n, offer != kPlaceNone, cm, ym,
                              has_c, has_y, dc);
  if (offer != kPlaceNone) {
#pragma unroll
    for (int k = 0; k < Q; k++) {
      int64_t v[4] = {0, 0, 0, 0};
      if (qv[k]) ham_point(M, S.tok[offer], qi[k], v);
#pragma unroll
      for (int c = 0; c < 4; c++) cm[k][c] = v[c] * ((int64_t)1 << 31);
    }
    has_c = true;
  }
  if (!has_c && !has_y) return;
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      const int4 wc = *(const int4 *)(R.w + 4 * qi[k]);
      const int4 wy = *(const int4 *)(R.w + M.d + 4 * qi[k]);
      const int32_t a[4] = {wc.x, wc.y, wc.z, wc.w}, b[4] = {wy.x, wy.y, wy.z, wy.w};
#pragma unroll
      for (int c = 0; c < 4; c++)
        n[k][c] = R.ask ? ham_readout_ask_sum(n[k][c], a[c], has_c, cm[k][c], b[c], has_y, ym[k][c])
                        : ham_readout_sum(n[k][c], a[c], has_c, cm[k][c], b[c],
                                          has_y ? ym[k][c] : 0);
    }
}

}  // namespace fbs

#endif
