// fbs_kernel.hip - the SpiralCore/FBS integer decode step for gfx950 (MI355X).
//
// One 64-lane wavefront runs one sequence through every step of its run (teacher-forced
// sequences, greedy decode, or scoring). Per step (RS crates/uor-r4-integer/src/stack/
// session.rs:4129-4403 `stack_step_fbs`; twin fbs_core.h:635-675):
//   the token's writer row in; per layer the fine RMSNorm and gain, the FBS projections
//   (gathers through LDS by a precomputed per-lane program), the causal window read from the
//   sequence's ring in HBM, the quaternion recurrence with its output gate, the shared-exponent
//   requantize, the residual add, and the same for the Hamilton feed-forward gate; the final
//   norm, the Q12 query, and the drawer writer (drawer scores, P rounds of lowest (score, drawer),
//   then the lowest (L1, token) over the kept drawers' CSR members, scanned by lane groups of
//   d/32 lanes with packed v_sad_u16 on biased rows).
// The recurrence state of every layer stays in LDS for the whole run; only the window ring,
// the table rows and the outputs touch HBM. Every reduction is an exact integer max, sum or
// lexicographic min, so the outputs do not depend on lane order.
#include "fbs_device.h"
#include "fbs_int.h"

namespace fbs {

__device__ __forceinline__ uint32_t uniform32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  uint32_t lo = uniform32((uint32_t)v), hi = uniform32((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return uniform32(v);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t w = __shfl_xor(v, o);
    v = w < v ? w : v;
  }
  return uniform32(v);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor((unsigned long long)v, o);
    v = w > v ? w : v;
  }
  return uniform64(v);
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor((unsigned long long)v, o);
    v = w < v ? w : v;
  }
  return uniform64(v);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, o);
  return uniform64(v);
}

// Fine RMSNorm then the per-channel grid gain, for the lane's channels
// (RS stack/kernels.rs:569-620, session.rs:4057-4061).
template <int Q>
__device__ __forceinline__ void norm_gain(const DevModel &M, const int32_t (&x)[Q][4],
                                          const bool (&qv)[Q], const uint32_t (&qi)[Q],
                                          const int16_t *gain, int64_t (&out)[Q][4]) {
  uint32_t mx = 0;
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k])
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t a = uabs32(x[k][c]);
        mx = a > mx ? a : mx;
      }
  mx = wave_max_u32(mx);
  int32_t sh = bitlen64(mx) - 24;
  if (sh < 0) sh = 0;
  uint64_t sum = 0;
#pragma unroll
  for (int k = 0; k < Q; k++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int64_t y = qv[k] ? shift((int64_t)x[k][c], sh) : 0;
      out[k][c] = y;
      sum += uabs64(y) * uabs64(y);
    }
  sum = wave_sum_u64(sum);
  NormFactor f = norm_factor(sum, M.d, M.eps_int[sh]);
  f.r = uniform64(f.r);
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      short4 g = *(const short4 *)(gain + 4 * qi[k]);
      int16_t gc[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
      for (int c = 0; c < 4; c++) out[k][c] = grid_apply(norm_apply(f, out[k][c]), gc[c]);
    }
}

// Publish v (exponent -24) for the FBS gathers: word 2 i + s holds to_exp_i32 of v_i (s = 0)
// or of its saturating negation (s = 1), at exponent -16 (session.rs:4037-4053: the negation
// comes before the rounding shift).
template <int Q>
__device__ __forceinline__ void publish64(int32_t *xbar, const int64_t (&v)[Q][4],
                                          const bool (&qv)[Q], const uint32_t (&qi)[Q]) {
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      int4 p, n;
      p.x = to_exp_i32(v[k][0], kNormFineExp, kResidualExp);
      n.x = to_exp_i32(sat_neg64(v[k][0]), kNormFineExp, kResidualExp);
      p.y = to_exp_i32(v[k][1], kNormFineExp, kResidualExp);
      n.y = to_exp_i32(sat_neg64(v[k][1]), kNormFineExp, kResidualExp);
      p.z = to_exp_i32(v[k][2], kNormFineExp, kResidualExp);
      n.z = to_exp_i32(sat_neg64(v[k][2]), kNormFineExp, kResidualExp);
      p.w = to_exp_i32(v[k][3], kNormFineExp, kResidualExp);
      n.w = to_exp_i32(sat_neg64(v[k][3]), kNormFineExp, kResidualExp);
      int4 *dst = (int4 *)(xbar + 8 * qi[k]);
      dst[0] = make_int4(p.x, n.x, p.y, n.y);
      dst[1] = make_int4(p.z, n.z, p.w, n.w);
    }
}

// Publish 16-bit activations at exponent `exp` for gather16 (to_exp_i32 of +-a to -16).
__device__ __forceinline__ void publish16(int32_t *xbar, uint32_t channel0, const int32_t a[4],
                                          int32_t exp) {
  int32_t s = kResidualExp - exp;
  int4 *dst = (int4 *)(xbar + 2 * channel0);
  dst[0] = make_int4(to_exp_i32(a[0], exp, kResidualExp), to_exp_i32(-(int64_t)a[0], exp, kResidualExp),
                     to_exp_i32(a[1], exp, kResidualExp), to_exp_i32(-(int64_t)a[1], exp, kResidualExp));
  dst[1] = make_int4(to_exp_i32(a[2], exp, kResidualExp), to_exp_i32(-(int64_t)a[2], exp, kResidualExp),
                     to_exp_i32(a[3], exp, kResidualExp), to_exp_i32(-(int64_t)a[3], exp, kResidualExp));
  (void)s;
}

__device__ __forceinline__ int32_t gather1(const int32_t *xbar, const uint16_t *prog,
                                           uint32_t slot, uint32_t lane) {
  return xbar[prog[slot * kWave + lane]];
}

// A rotation of the gate kind (lambda 2^31, epsilon 0) applied to rhs: shift_wide(q (x) rhs, 15)
// (session.rs:4951-4968, :4005-4025). Raw gates use q = 2 u exactly, so the product is formed
// from u and shifted by 14.
__device__ __forceinline__ void gate_apply(const DevModel &M, const int32_t raw[4],
                                           const int64_t rhs[4], int64_t out[4]) {
  i128 prod[4];
  if (M.raw_gates) {
    int32_t u[4];
    unit_q30(raw, kGateEps, u);
    hamilton32(u, rhs, prod);
#pragma unroll
    for (int c = 0; c < 4; c++) out[c] = shift_wide(prod[c], 14);
  } else {
    int64_t q[4];
    snap_rotation(M.icosian, raw, 1ull << 31, q);
    hamilton64(q, rhs, prod);
#pragma unroll
    for (int c = 0; c < 4; c++) out[c] = shift_wide(prod[c], 15);
  }
}

// v_sad_u16 on gfx950 sums the absolute differences of both 16-bit halves:
// d = |a[15:0] - b[15:0]| + |a[31:16] - b[31:16]| + c (unsigned halves; measured on MI355X and
// held by the parity tests). Inline asm keeps the optimiser from reasoning about the halves.
__device__ __forceinline__ uint32_t sad2_u16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_sad_u16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// The candidate scan of the writer over members [beg, end) (or token ids beg..end for the
// nearest head): lane group g = lane / S scores one row per round, lane sub = lane % S its
// 32 channels (16 biased pairs against the packed biased query); the group sums its partial
// L1s and keeps the lowest (L1, token).
__device__ __forceinline__ uint64_t scan_rows(const DevModel &M, const uint32_t (&qpk)[16],
                                              uint32_t beg, uint32_t end, uint32_t S,
                                              uint32_t grp, uint32_t sub, bool seg_ok,
                                              uint32_t rows, uint64_t best) {
  const uint32_t d = M.d;
  for (uint32_t i0 = beg; i0 < end; i0 += rows) {
    uint32_t i = i0 + grp;
    bool ok = i < end;
    uint32_t t = ok ? (M.identity_rows ? i : M.members[i]) : 0u;
    uint32_t acc = 0;
    if (seg_ok) {
      const uint4 *row = (const uint4 *)(M.table_b + (uint64_t)t * d + 32u * sub);
      uint4 r[4];
#pragma unroll
      for (int w = 0; w < 4; w++) r[w] = row[w];
#pragma unroll
      for (int w = 0; w < 4; w++) {
        acc = sad2_u16(r[w].x, qpk[4 * w + 0], acc);
        acc = sad2_u16(r[w].y, qpk[4 * w + 1], acc);
        acc = sad2_u16(r[w].z, qpk[4 * w + 2], acc);
        acc = sad2_u16(r[w].w, qpk[4 * w + 3], acc);
      }
    }
    for (uint32_t o = 1; o < S; o <<= 1) acc += __shfl_xor(acc, (int)o);
    uint64_t cand = ((uint64_t)acc << 32) | t;
    if (ok && cand < best) best = cand;
  }
  return best;
}

// The native vector writer (RS stack/session.rs:4069-4121, TW 580-623) over keyed drawers,
// or the whole-table nearest head (session.rs:4418-4445). `q` holds the query (d words) in
// LDS. Returns the token (UINT32_MAX when no row was scored); writes the kept drawers in
// selection order to kept_out (nullable) from lane 0.
__device__ uint32_t writer(const DevModel &M, const int32_t *q, uint32_t *dscore, uint32_t lane,
                           uint32_t *kept_out) {
  const uint32_t d = M.d, segs = d >> 5;
  uint32_t S = 1;
  while (S < segs) S <<= 1;
  const uint32_t rows = kWave / S, grp = lane / S, sub = lane % S;
  const bool seg_ok = sub < segs;  // lanes past the row's last 32-channel segment add zero
  uint32_t qpk[16];  // biased query pairs: (q[2i] + 2^15) | (q[2i+1] + 2^15) << 16
#pragma unroll
  for (int i = 0; i < 16; i++)
    qpk[i] = seg_ok ? (uint32_t)(q[32 * sub + 2 * i] + 32768) |
                          ((uint32_t)(q[32 * sub + 2 * i + 1] + 32768) << 16)
                    : 0u;
  uint64_t best = UINT64_MAX;
  if (M.head == 1) {
    best = scan_rows(M, qpk, 0, M.vocab, S, grp, sub, seg_ok, rows, best);
    if (kept_out && lane < M.P) kept_out[lane] = 0;
  } else {
    int32_t qa[8], qb[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      qa[i] = q[i];
      qb[i] = q[d - 8 + i];
    }
    for (uint32_t c = lane; c < M.D; c += kWave) {
      const int16_t *key = M.keys + 16u * c;
      uint32_t s = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        s += uabs32(qa[i] - (int32_t)key[i]);
        s += uabs32(qb[i] - (int32_t)key[8 + i]);
      }
      dscore[c] = (s << 12) | c;
    }
    __syncthreads();
    for (uint32_t p = 0; p < M.P; p++) {
      uint32_t local = UINT32_MAX;
      for (uint32_t c = lane; c < M.D; c += kWave) local = dscore[c] < local ? dscore[c] : local;
      uint32_t pick = wave_min_u32(local) & 0xfffu;
      __syncthreads();
      if ((pick & (kWave - 1)) == lane) dscore[pick] = UINT32_MAX;
      if (kept_out && lane == 0) kept_out[p] = pick;
      uint32_t beg = M.offsets[pick], end = M.offsets[pick + 1];
      best = scan_rows(M, qpk, beg, end, S, grp, sub, seg_ok, rows, best);
      __syncthreads();
    }
  }
  best = wave_min_u64(best);
  return (uint32_t)best;
}

// One step of the session (RS stack/session.rs:4129-4403, TW 635-675) at position `pos` with
// ring slot `base`. Returns 0 or the reference's status code; the chosen token goes to *chosen
// when the writer runs.
template <int Q>
__device__ int step(const DevModel &M, int32_t *xbar, uint32_t *dscore, int64_t *st,
                    int32_t *ring, uint32_t base, uint32_t lane, const bool (&qv)[Q],
                    const uint32_t (&qi)[Q], uint32_t tok, bool want_writer, uint32_t *chosen,
                    uint32_t *kept_out, int32_t *query_out) {
  if (tok >= M.vocab) return 1;
  const uint32_t d = M.d, W = M.W, nq = M.nq;
  int32_t x[Q][4];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    if (qv[k]) {
      uint2 w = *(const uint2 *)(M.table_b + (uint64_t)tok * d + 4 * qi[k]);
      uint32_t ww[2] = {w.x, w.y};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int16_t v = (int16_t)(uint16_t)(((ww[c >> 1] >> (16 * (c & 1))) & 0xffffu) ^ 0x8000u);
        x[k][c] = (int32_t)v << 4;  // to_exp_i32(v, -12, -16)
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) x[k][c] = 0;
    }
  }
  for (uint32_t l = 0; l < M.L; l++) {
    const DevLayer ly = M.layers[l];
    int64_t v[Q][4];
    // ---- recurrence block
    norm_gain<Q>(M, x, qv, qi, ly.rec_gain, v);
    publish64<Q>(xbar, v, qv, qi);
    __syncthreads();
    int32_t drive[Q][4], gv[Q][4], rot[Q][4], dec[Q];
#pragma unroll
    for (int k = 0; k < Q; k++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        drive[k][c] = gather1(xbar, ly.prog, M.s_rec_in + 4 * k + c, lane);
        gv[k][c] = gather1(xbar, ly.prog, M.s_rec_in + 4 * Q + 4 * k + c, lane);
        rot[k][c] = gather1(xbar, ly.prog, M.s_rec_gate + Q + 4 * k + c, lane);
      }
      dec[k] = gather1(xbar, ly.prog, M.s_rec_gate + k, lane);
    }
    __syncthreads();
    int32_t *ring_l = ring + (uint64_t)l * W * d;
    int64_t sc[Q][4];
    uint64_t mx = 0;
#pragma unroll
    for (int k = 0; k < Q; k++) {
      if (!qv[k]) {
#pragma unroll
        for (int c = 0; c < 4; c++) sc[k][c] = 0;
        continue;
      }
      const uint32_t qq = qi[k], ch = 4 * qq;
      dec[k] = sat_add32(dec[k], ly.gate_bias[qq]);
#pragma unroll
      for (int c = 0; c < 4; c++) rot[k][c] = sat_add32(rot[k][c], ly.gate_bias[nq + ch + c]);
      // The causal window (session.rs:4842-4868): tap 0 on the drive, tap s on the drive s
      // positions back (ring slot base - s), then the drive enters slot base.
      int64_t wide[4];
      {
        int4 cb = *(const int4 *)(ly.conv_bias + ch);
        short4 t0 = *(const short4 *)(ly.taps + ch);
        wide[0] = wadd64(cb.x, grid_apply(drive[k][0], t0.x));
        wide[1] = wadd64(cb.y, grid_apply(drive[k][1], t0.y));
        wide[2] = wadd64(cb.z, grid_apply(drive[k][2], t0.z));
        wide[3] = wadd64(cb.w, grid_apply(drive[k][3], t0.w));
      }
      uint32_t slot = base;
      for (uint32_t s = 1; s <= W; s++) {
        slot = slot == 0 ? W - 1 : slot - 1;
        int4 h = *(const int4 *)(ring_l + (uint64_t)slot * d + ch);
        short4 t = *(const short4 *)(ly.taps + (uint64_t)s * d + ch);
        wide[0] = wadd64(wide[0], grid_apply(h.x, t.x));
        wide[1] = wadd64(wide[1], grid_apply(h.y, t.y));
        wide[2] = wadd64(wide[2], grid_apply(h.z, t.z));
        wide[3] = wadd64(wide[3], grid_apply(h.w, t.w));
      }
      *(int4 *)(ring_l + (uint64_t)base * d + ch) =
          make_int4(drive[k][0], drive[k][1], drive[k][2], drive[k][3]);
      // Lane weights (session.rs:4989-5026): geometric decay and keep from the 16-step table.
      int32_t sq = sat_add32(dec[k], ly.decay_offset[qq]);
      sq = sq < 0 ? 0 : sq > 65536 ? 65536 : sq;
      uint32_t idx = (uint32_t)sq >> 12;
      idx = idx > 15 ? 15 : idx;
      uint64_t lambda = 1ull << (30 - idx), keep = M.keep_q31[idx];
      // Transport (session.rs:5097-5145): h <- shift_wide(T (x) h + (keep wide) << 16, 31).
      int64_t *hp = st + (uint64_t)l * d + ch;
      int64_t h[4] = {hp[0], hp[1], hp[2], hp[3]};
      i128 moved[4];
      if (M.raw_transition) {
        int32_t u[4], T[4];
        unit_q30(rot[k], kRotationEps, u);
#pragma unroll
        for (int c = 0; c < 4; c++) T[c] = u[c] >> idx;  // (lambda u) >> 30, lambda = 2^(30-idx)
        hamilton32(T, h, moved);
      } else {
        int64_t T[4];
        snap_rotation(M.icosian, rot[k], lambda, T);
        hamilton64(T, h, moved);
      }
#pragma unroll
      for (int c = 0; c < 4; c++) {
        u128 drive_term = (u128)((i128)keep * (i128)wide[c]) << 16;
        h[c] = shift_wide((i128)((u128)moved[c] + drive_term), 31);
        hp[c] = h[c];
      }
      // Output gate on the moved state (session.rs:4951-4968).
      int64_t rhs[4], o[4];
#pragma unroll
      for (int c = 0; c < 4; c++) rhs[c] = shift(h[c], kResidualExp - kStateExp);
      gate_apply(M, gv[k], rhs, o);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        sc[k][c] = o[c];
        uint64_t a = uabs64(o[c]);
        mx = a > mx ? a : mx;
      }
    }
    // quantize16 over the d outputs (kernels.rs:545-553), then gather16 of rec_out.
    mx = wave_max_u64(mx);
    int32_t qs = bitlen64(mx) - 15;
    if (qs < 0) qs = 0;
    const int32_t act_exp = kProductExp + qs;
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k]) {
        int32_t a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) a[c] = quantize_elem(sc[k][c], qs);
        publish16(xbar, 4 * qi[k], a, act_exp);
      }
    __syncthreads();
    int32_t proj[Q][4];
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) proj[k][c] = gather1(xbar, ly.prog, M.s_rec_out + 4 * k + c, lane);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], proj[k][c]);
    // ---- feed-forward block: the Hamilton gate of mlp_gate on mlp_up (session.rs:4005-4025).
    norm_gain<Q>(M, x, qv, qi, ly.mlp_gain, v);
    publish64<Q>(xbar, v, qv, qi);
    __syncthreads();
    int64_t mo[kMaxMpl][4];
    uint64_t mmx = 0;
#pragma unroll
    for (int j = 0; j < (int)kMaxMpl; j++) {
      uint32_t mq = lane + kWave * j;
      if (j < (int)M.mpl && mq < M.nm) {
        int32_t g[4];
        int64_t up[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          g[c] = gather1(xbar, ly.prog, M.s_mlp_gate + 4 * j + c, lane);
          up[c] = gather1(xbar, ly.prog, M.s_mlp_up + 4 * j + c, lane);
        }
        gate_apply(M, g, up, mo[j]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          uint64_t a = uabs64(mo[j][c]);
          mmx = a > mmx ? a : mmx;
        }
      }
    }
    __syncthreads();
    mmx = wave_max_u64(mmx);
    qs = bitlen64(mmx) - 15;
    if (qs < 0) qs = 0;
    const int32_t mlp_exp = kProductExp + qs;
#pragma unroll
    for (int j = 0; j < (int)kMaxMpl; j++) {
      uint32_t mq = lane + kWave * j;
      if (j < (int)M.mpl && mq < M.nm) {
        int32_t a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) a[c] = quantize_elem(mo[j][c], qs);
        publish16(xbar, 4 * mq, a, mlp_exp);
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < Q; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) proj[k][c] = gather1(xbar, ly.prog, M.s_mlp_down + 4 * k + c, lane);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (qv[k])
#pragma unroll
        for (int c = 0; c < 4; c++) x[k][c] = sat_add32(x[k][c], proj[k][c]);
  }
  // Final norm, gain and the Q12 query (session.rs:4294-4295, 4364-4366).
  int64_t v[Q][4];
  norm_gain<Q>(M, x, qv, qi, M.final_gain, v);
#pragma unroll
  for (int k = 0; k < Q; k++)
    if (qv[k]) {
      int4 qq;
      int32_t qa[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int32_t y = to_exp_i32(v[k][c], kNormFineExp, kQ12Exp);
        qa[c] = y > 32767 ? 32767 : y < -32768 ? -32768 : y;
      }
      qq = make_int4(qa[0], qa[1], qa[2], qa[3]);
      *(int4 *)(xbar + 4 * qi[k]) = qq;
      if (query_out) *(int4 *)(query_out + 4 * qi[k]) = qq;
    }
  __syncthreads();
  if (want_writer) *chosen = writer(M, xbar, dscore, lane, kept_out);
  __syncthreads();
  return 0;
}

template <int Q>
__global__ __launch_bounds__(64) void fbs_run(DevModel M, RunArgs A) {
  extern __shared__ __align__(16) int32_t lds[];
  int32_t *xbar = lds;
  uint32_t *dscore = (uint32_t *)(lds + M.xbar_words);
  int64_t *st = (int64_t *)(lds + M.xbar_words + ((M.D + 3u) & ~3u));
  const uint32_t lane = threadIdx.x;
  const uint32_t d = M.d, L = M.L, W = M.W;
  int32_t *ring = A.ring + (uint64_t)blockIdx.x * L * W * d;
  bool qv[Q];
  uint32_t qi[Q];
#pragma unroll
  for (int k = 0; k < Q; k++) {
    qi[k] = lane + kWave * k;
    qv[k] = qi[k] < M.nq;
  }
  for (uint32_t s = blockIdx.x; s < A.n; s += gridDim.x) {
    // Fresh or resumed session: state, window rows (row r = the drive r + 1 positions back)
    // and position (LayerState::Recurrence, session.rs:1850).
    uint32_t pos = A.in_position ? A.in_position[s] : 0u;
    uint32_t base = pos % W;
    for (uint32_t l = 0; l < L; l++)
#pragma unroll
      for (int k = 0; k < Q; k++)
        if (qv[k]) {
          uint32_t ch = 4 * qi[k];
#pragma unroll
          for (int c = 0; c < 4; c++)
            st[(uint64_t)l * d + ch + c] =
                A.in_state ? A.in_state[((uint64_t)s * L + l) * d + ch + c] : 0;
          for (uint32_t r = 0; r < W; r++) {
            uint32_t slot = (base + 2 * W - 1 - r) % W;
            int4 h = make_int4(0, 0, 0, 0);
            if (A.in_history) h = *(const int4 *)(A.in_history + (((uint64_t)s * L + l) * W + r) * d + ch);
            *(int4 *)(ring + ((uint64_t)l * W + slot) * d + ch) = h;
          }
        }
    __syncthreads();
    int status = 0;
    uint32_t chosen = 0;
    if (A.mode == kModeDecode) {
      const uint32_t *prompt = A.tokens + (uint64_t)s * A.len;
      uint32_t *reply = A.out_tokens + (uint64_t)s * (A.gen + 1);
      for (uint32_t t = 0; t < A.len + A.gen && status == 0; t++) {
        uint32_t tok = t < A.len ? prompt[t] : chosen;
        if (pos >= M.context) {
          status = 2;
          break;
        }
        bool want = t + 1 >= A.len;  // the prompt's last step and every generated step
        status = step<Q>(M, xbar, dscore, st, ring, base, lane, qv, qi, tok, want, &chosen,
                         nullptr, nullptr);
        if (status) break;
        pos++;
        base = base + 1 == W ? 0 : base + 1;
        if (want && lane == 0) reply[t + 1 - A.len] = chosen;
      }
      if (status == 0) {
        for (uint32_t l = 0; l < L; l++)
#pragma unroll
          for (int k = 0; k < Q; k++)
            if (qv[k]) {
              uint32_t ch = 4 * qi[k];
              if (A.out_state)
#pragma unroll
                for (int c = 0; c < 4; c++)
                  A.out_state[((uint64_t)s * L + l) * d + ch + c] = st[(uint64_t)l * d + ch + c];
              if (A.out_history)
                for (uint32_t r = 0; r < W; r++) {
                  uint32_t slot = (base + 2 * W - 1 - r) % W;
                  *(int4 *)(A.out_history + (((uint64_t)s * L + l) * W + r) * d + ch) =
                      *(const int4 *)(ring + ((uint64_t)l * W + slot) * d + ch);
                }
            }
        if (A.out_position && lane == 0) A.out_position[s] = pos;
      }
    } else {
      const uint32_t *row = A.tokens + (uint64_t)s * A.len;
      unsigned long long hits = 0;
      for (uint32_t t = 0; t < A.len; t++) {
        if (pos >= M.context) {
          status = 2;
          break;
        }
        uint64_t at = (uint64_t)s * A.len + t;
        bool want = A.mode == kModeSequences || A.out_tokens || t + 1 < A.len;
        uint32_t *kept_out = (A.mode == kModeSequences && A.out_kept) ? A.out_kept + at * M.P : nullptr;
        int32_t *query_out = (A.mode == kModeSequences && A.out_query) ? A.out_query + at * d : nullptr;
        status = step<Q>(M, xbar, dscore, st, ring, base, lane, qv, qi, row[t], want, &chosen,
                         kept_out, query_out);
        if (status) break;
        pos++;
        base = base + 1 == W ? 0 : base + 1;
        if (A.out_tokens && lane == 0) A.out_tokens[at] = chosen;
        if (A.mode == kModeScore && t + 1 < A.len && chosen == row[t + 1]) hits++;
      }
      if (A.mode == kModeScore && lane == 0 && hits) atomicAdd(A.matches, hits);
    }
    if (lane == 0) A.status[s] = status;
    __syncthreads();
  }
}

template __global__ void fbs_run<1>(DevModel, RunArgs);
template __global__ void fbs_run<2>(DevModel, RunArgs);
template __global__ void fbs_run<4>(DevModel, RunArgs);

// Launch entry used by the host side (fbs_api.cpp).
hipError_t launch_run(const DevModel &M, const RunArgs &A, uint32_t grid, size_t lds_bytes,
                      hipStream_t stream) {
  dim3 g(grid), b(kWave);
  switch (M.qpl) {
    case 1:
      hipLaunchKernelGGL(fbs_run<1>, g, b, lds_bytes, stream, M, A);
      break;
    case 2:
      hipLaunchKernelGGL(fbs_run<2>, g, b, lds_bytes, stream, M, A);
      break;
    default:
      hipLaunchKernelGGL(fbs_run<4>, g, b, lds_bytes, stream, M, A);
      break;
  }
  return hipGetLastError();
}

}  // namespace fbs
