/*
 * fbs_oracle.h - CPU restatement of UOR-R4's SpiralCore/FBS integer step, for tests only.
 *
 * TEST INFRASTRUCTURE. This is the parity checker of the HIP path and the CPU baseline that
 * bench.py times beside it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product (libuor_fbs_hip.so) never links or calls it.
 *
 * It follows the Rust session (crates/uor-r4-integer/src/stack/session.rs,
 * stack/kernels.rs) and the reference's C++ twin
 * (docs/labs/d11-exporter-float-trunk/instrument/src/fbs_core.h) function by function; each
 * function in fbs_oracle.c names the lines it restates. It takes the same model image as the
 * product (include/uor_fbs.h), including the documented extensions (window W, D drawers with
 * keys and CSR members, int8 table, nearest head), which reduce to the reference's rules at
 * their defaults.
 *
 * Pinning (what checks each part): tests/test_oracle_golden.py compares every position's
 * token, kept cells and Q12 query with vectors written by the reference's own twin
 * (oracle/_ref, tests/golden/); tests/test_oracle_math.py checks the scalar routines against
 * closed forms and brute force (isqrt, floor division, the 120-root snap as an exact argmax,
 * rounding shifts, grid codes) and the extensions against their reference reductions.
 */
#ifndef FBS_ORACLE_H
#define FBS_ORACLE_H

#include <stdint.h>

#include "../include/uor_fbs.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Teacher-forced sequences from fresh sessions (fbs_core.h:681-695, host_kernel.cpp:16-29):
 * per position the token, the kept drawers (probes of them) and the width-long Q12 query.
 * Sequences are spread over `threads` POSIX threads (<= 0: one). */
int fbs_oracle_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *tokens,
                         uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                         uint32_t *out_kept, int32_t *out_query, int threads);

/* Greedy decode (fbs-toks.rs:1513-1533) of many sequences, with optional resume state and
 * export (layouts as uor_fbs_decode). `out_candidates` (nullable) gets, per sequence, the
 * number of writer candidate rows scored over all its steps. */
int fbs_oracle_decode(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *prompts,
                      uint32_t sequences, uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                      const int64_t *in_state, const int32_t *in_history,
                      const uint32_t *in_position, int64_t *out_state, int32_t *out_history,
                      uint32_t *out_position, uint64_t *out_candidates, int threads);

/* Teacher-forced scoring: matches of position t's choice with row[t+1]. */
int fbs_oracle_score(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *rows,
                     uint64_t n_rows, uint32_t len, uint32_t *out_argmin,
                     uint64_t *out_matches, int threads);

/* Greedy decode with the Hamming reads' session stream: the session's tokens ([n][context],
 * the first position of them valid) and the typed reads' payload caches
 * ([n][typed][context][width], typed = fbs_oracle_hamming_typed), resumed and exported beside the
 * state as IntegerStackSession keeps them (session.rs:2232-2252). */
/* The sequences with every position's snap trace (fbs_host_trace_sequences, TW
 * host_kernel.cpp:31-49): per position and layer, the transition's root per lane, the output
 * gate's per lane, the feed-forward gate's per 4 MLP channels; 255 where none was chosen. */
uint64_t fbs_oracle_trace_stride(const uor_fbs_model *m);
int fbs_oracle_trace_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *tokens,
                               uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                               uint32_t *out_kept, int32_t *out_query, uint8_t *out_trace,
                               int threads);
/* fbs_oracle_decode with the context slide on for every session (session.rs:2391-2402); a model
 * with Hamming reads is refused (UOR_FBS_ERR_SHAPE). */
int fbs_oracle_decode_slide(const uor_fbs_model *m, const uor_fbs_ext *ext, const uint32_t *prompts,
                            uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                            uint32_t *out_reply, const int64_t *in_state, const int32_t *in_history,
                            const uint32_t *in_position, int64_t *out_state, int32_t *out_history,
                            uint32_t *out_position, int threads);
int fbs_oracle_decode_stream(const uor_fbs_model *m, const uor_fbs_ext *ext,
                             const uint32_t *prompts, uint32_t sequences, uint32_t prompt_len,
                             uint32_t gen, uint32_t *out_reply, const int64_t *in_state,
                             const int32_t *in_history, const uint32_t *in_position,
                             const uint32_t *in_tokens, const int64_t *in_payloads,
                             int64_t *out_state, int32_t *out_history, uint32_t *out_position,
                             uint32_t *out_tokens, int64_t *out_payloads, int threads);
uint32_t fbs_oracle_hamming_typed(const uor_fbs_model *m, const uor_fbs_ext *ext);
/* One read at row t of tok (the stream read at depth < layers on x, the readout read on n). */
int fbs_oracle_hamming_row(const uor_fbs_model *m, const uor_fbs_ext *ext, uint32_t depth,
                           const uint32_t *tok, uint32_t t, int32_t *x, int64_t *n,
                           int64_t *payloads);
int fbs_oracle_hamming_codes(const uor_fbs_model *m, const uor_fbs_ext *ext, uint32_t r,
                             uint64_t *out);
/* The place read: teacher-forced sequences with every position's register after the step
 * (held, offered place; -1 for none), the register over a token stream with injected finds,
 * and the place pick over candidate ranges with per-position keys. */
int fbs_oracle_place_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext,
                               const uint32_t *tokens, uint32_t sequences, uint32_t len,
                               uint32_t *out_tokens, int32_t *out_query, int64_t *out_place,
                               int threads);
int fbs_oracle_place_rows(const uor_fbs_place *pm, uint32_t vocab, const uint32_t *tokens,
                          uint64_t n, const int64_t *finds, uint32_t nfinds, int64_t *out);
int64_t fbs_oracle_place_pick(const uint64_t *queries, const int32_t *margins, uint32_t heads,
                              const uint64_t *ranges, uint32_t nranges, const uint64_t *keys);
/* The Hamming trace and the decision trace with forced replay, teacher-forced from fresh
 * sessions: fbs_oracle_decision_stride bytes a position (layout in fbs_oracle.c). */
uint64_t fbs_oracle_decision_stride(const uor_fbs_model *m, const uor_fbs_ext *ext, int decisions);
int fbs_oracle_decision_sequences(const uor_fbs_model *m, const uor_fbs_ext *ext,
                                  const uint32_t *tokens, uint32_t sequences, uint32_t len,
                                  int decisions, const uint8_t *force_buckets,
                                  const uint64_t *force_codes, const uint8_t *force_mask,
                                  uint32_t *out_tokens, int32_t *out_query, uint8_t *out_trace,
                                  int threads);
/* stream_sum / readout_sum / readout_ask_sum (hamming.rs:1918-1953), 128-bit means as hi:lo. */
int32_t fbs_oracle_stream_sum(int32_t x, int32_t w_c, int64_t c_hi, uint64_t c_lo, int32_t w_y,
                              int64_t y_hi, uint64_t y_lo);
int64_t fbs_oracle_readout_sum(int64_t n, int32_t w_c, int has_c, int64_t c_hi, uint64_t c_lo,
                               int32_t w_y, int64_t y_hi, uint64_t y_lo);
int64_t fbs_oracle_readout_ask_sum(int64_t n, int32_t w_c, int has_c, int64_t c_hi, uint64_t c_lo,
                                   int32_t w_y, int has_y, int64_t y_hi, uint64_t y_lo);

/* Scalar routines, exported so the tests can check them against closed forms. */
int64_t fbs_oracle_shift(int64_t v, int32_t s);
int64_t fbs_oracle_shift_wide(int64_t hi, uint64_t lo, uint32_t s);
int64_t fbs_oracle_grid_apply(int64_t v, int16_t code);
void fbs_oracle_isqrt(uint64_t hi, uint64_t lo, uint64_t out[2]);
void fbs_oracle_div_u128(uint64_t nhi, uint64_t nlo, uint64_t dhi, uint64_t dlo, uint64_t out[2]);
uint32_t fbs_oracle_snap_select(const int8_t *icosian, const int32_t raw[4]);
int fbs_oracle_diff_positive(int64_t da, int64_t db);
void fbs_oracle_serve_rotation(const int8_t *icosian, uint32_t raw_form, const int32_t raw[4],
                               uint64_t lambda, uint64_t epsilon, int64_t out[4]);
int32_t fbs_oracle_quantize16(const int64_t *v, uint32_t n, int32_t exp, int16_t *out);
void fbs_oracle_rms_norm_fine(const int32_t *x, uint32_t n, int64_t eps_mantissa, int32_t eps_exp,
                              int64_t *out);
/* Writer on a given query: token, kept (probes of them); `candidates` = rows scored. */
uint32_t fbs_oracle_writer(const uor_fbs_model *m, const uor_fbs_ext *ext, const int32_t *query,
                           uint32_t *kept, uint64_t *candidates);

/* The 256-cell CSR drawer index (fbs_index_oracle.c; projects/uor-cuda-inverted-file/src/
 * inverted_file.cpp): table [count][width] int32, roots [16][8] int32, offsets[257],
 * members (offsets[256] used), cells[count]. Status 0 ok, 1 invalid argument, 2 non-root
 * block, 3 CSR invariant. */
uint32_t fbs_oracle_index_cell(const int32_t *row, uint32_t width, const int32_t *roots);
int fbs_oracle_index_build(const int32_t *table, uint32_t count, uint32_t width,
                           const int32_t *roots, int allow_absent, uint32_t *offsets,
                           uint32_t *members, uint32_t *cells, uint32_t *absent_count);
int fbs_oracle_index_update(const int32_t *table, uint32_t count, uint32_t width,
                            const int32_t *roots, uint32_t moved, uint32_t *offsets,
                            uint32_t *members, uint32_t *cells, uint32_t *absent_count);
int fbs_oracle_index_remove(uint32_t count, uint32_t moved, uint32_t *offsets, uint32_t *members,
                            uint32_t *cells, uint32_t *absent_count);
int fbs_oracle_index_validate_structure(const uint32_t *offsets, const uint32_t *members,
                                        const uint32_t *cells, uint32_t count,
                                        uint32_t absent_count);
int fbs_oracle_index_validate(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, const uint32_t *offsets,
                              const uint32_t *members, const uint32_t *cells,
                              uint32_t absent_count);
/* Probe and full scan of one query row [width]: admitted[16], top8[8], *prediction. */
int fbs_oracle_index_probe(const int32_t *table, uint32_t count, uint32_t width,
                           const int32_t *roots, const int32_t *query, uint32_t k,
                           const uint32_t *offsets, const uint32_t *members,
                           const uint32_t *cells, uint32_t absent_count, uint32_t *admitted,
                           uint32_t *top8, uint32_t *prediction);
int fbs_oracle_index_full_scan(const int32_t *table, uint32_t count, uint32_t width,
                               const int32_t *roots, const int32_t *query, uint32_t k,
                               uint32_t *admitted, uint32_t *top8, uint32_t *prediction);

#ifdef __cplusplus
}
#endif

#endif
