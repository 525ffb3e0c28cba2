/*
 * uor_copy.h - C ABI of the copy heads' Hamming read on MI355X (gfx950).
 *
 * Replaces the look-back read of the served Hamming copy heads, `CopyHeads`
 * (crates/uor-r4-integer/src/stack/hamming.rs:266-538): for the last row t of a token stream,
 * each copy head picks earlier positions 1 <= s < t by the XOR-popcount distance between the
 * row's query code and each position's key code (`nearest` :690-701, `latest_of` :584-598,
 * `longest_of` :601-615, the rule in force `CopyRule::at` :231-238, `choose_ruled` :356-371),
 * and the heads' margin-weighted mean of the table rows that followed those positions
 * (`copy_weight_q31` :243-252, `mean_by` :506-538) is the read. Batched: one read per stream.
 *
 * The caller passes the heads as `CopyHeads::new` holds them: every vocabulary entry's code per
 * copy head (the sign code of its table point through the key rotation, `vocab_codes`
 * :566-582, built at load), the margins, the copy-key-2 first-half masks, the kept count, the
 * rule and the artifact's reply marker. Integer only. One handle per device; a handle is not
 * safe to use from two threads at once.
 *
 * Return codes: 0 success, -1 invalid argument, -2 device error (uor_copy_last_error()).
 */
#ifndef UOR_COPY_H
#define UOR_COPY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UOR_COPY_ABI_VERSION 1u
#define UOR_COPY_MAX_HEADS 16u
#define UOR_COPY_MAX_KEPT 32u
#define UOR_COPY_MAX_WIDTH 1024u
#define UOR_COPY_MAX_STRIDE 4096u

/* CopyRule (hamming.rs:180-201) */
#define UOR_COPY_MEAN 0u
#define UOR_COPY_LATEST_EXACT 1u
#define UOR_COPY_LATEST_NEAREST 2u
#define UOR_COPY_LONGEST_EXACT 3u
#define UOR_COPY_LONGEST_AFTER_OPENING 4u

typedef struct {
  uint32_t vocabulary, width, copy, kept;
  uint32_t rule;
  uint32_t has_marker;   /* 1: a row opens a reply when its previous and own tokens are marker */
  uint32_t marker[2];
  const uint64_t *codes;        /* [vocabulary][copy] */
  const int32_t *margins_q16;   /* [copy], bits at Q16 */
  const uint64_t *pair_first;   /* [copy]: copy key 2's first-half bits, 0 for copy key 1 */
  const int16_t *table;         /* [vocabulary][width] */
} uor_copy_heads;

uint32_t uor_copy_abi_version(void);
const char *uor_copy_last_error(void);

int uor_copy_create(const uor_copy_heads *heads, int32_t device, void **handle);
void uor_copy_destroy(void *handle);

/* The heads' codes (`vocab_codes`, hamming.rs:541-582): for copy head h < copy of heads_total
 * heads over width / heads_total coordinates (at most 64), entry v's code is the sign word of
 * its table point through the head's key rotation, bit c set when coordinate c of
 * unit(key_rotation quaternion) (x) point is at or above 0, the unit at Q31 as `stack_rotation`
 * normalizes raw gates (epsilon 0). key_rotation holds width raw i32 values; codes receives
 * vocab x copy words. Host buffers; computed on `device`. */
int uor_copy_vocab_codes(const int32_t *key_rotation, const int16_t *table, uint32_t vocab,
                         uint32_t width, uint32_t heads_total, uint32_t copy, int32_t device,
                         uint64_t *codes);

/* For each of `rows` streams (tokens: rows x stride, row r's first lengths[r] tokens; opening:
 * one flag per row, the caller's reply mark, or NULL for none): the copy mean of its last row
 * into out[r][width] and found[r] = 1, or zeros and found[r] = 0 when no head kept a position
 * inside its margin (the reference's None). chosen (optional, rows x copy x kept int32): each
 * head's positions in the order read, s | distance << 24, -1 after the last. Host buffers. */
int uor_copy_mean_rows(void *handle, const uint32_t *tokens, const int32_t *lengths,
                       const uint8_t *opening, uint32_t rows, uint32_t stride, int64_t *out,
                       uint8_t *found, int32_t *chosen);

/* The same over device buffers on `stream` (a hipStream_t; NULL for the default stream). */
int uor_copy_mean_rows_async(void *handle, const uint32_t *d_tokens, const int32_t *d_lengths,
                             const uint8_t *d_opening, uint32_t rows, uint32_t stride,
                             int64_t *d_out, uint8_t *d_found, int32_t *d_chosen, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* UOR_COPY_H */
