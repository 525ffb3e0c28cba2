/* Test oracle (never shipped in the product path): a plain C restatement of the reference's
 * 256-cell CSR drawer index, projects/uor-cuda-inverted-file/src/inverted_file.cpp (the host
 * form of its uor_if_build/uor_if_update kernels, src/kernels.cu:139-196, and of the discrete
 * crate's discrete_bucket_build/update, crates/uor-r4-discrete/src/bucket_source.rs:1-12).
 *
 * A token's cell is r0 * 16 + r1 when the first 8 values of its row equal root r0 and the last
 * 8 equal root r1 (the first matching root; inverted_file.cpp:12-24), else ABSENT. The index
 * lists each cell's tokens in ascending order (offsets[257], members), keeps every token's
 * cell, and counts the absent ones. Status codes are uor_inverted_file::Status's
 * (include/uor_inverted_file.hpp:29-37): 0 ok, 1 invalid argument, 2 non-root block,
 * 3 CSR invariant.
 */
#include "fbs_oracle.h"

#include <string.h>

#define ABSENT 0xffffffffu

static uint32_t root_id(const int32_t *block, const int32_t *roots) {
  for (uint32_t r = 0; r < 16; r++)
    if (memcmp(block, roots + 8 * r, 8 * sizeof(int32_t)) == 0) return r;
  return ABSENT;
}

uint32_t fbs_oracle_index_cell(const int32_t *row, uint32_t width, const int32_t *roots) {
  const uint32_t first = root_id(row, roots), last = root_id(row + width - 8, roots);
  return first == ABSENT || last == ABSENT ? ABSENT : first * 16 + last;
}

/* inverted_file.cpp:141-162 `validate_structure` (members' length is offsets[256]). */
int fbs_oracle_index_validate_structure(const uint32_t *offsets, const uint32_t *members,
                                        const uint32_t *cells, uint32_t count,
                                        uint32_t absent_count) {
  (void)cells;
  if (offsets[0] != 0 || offsets[256] > count || absent_count + offsets[256] != count) return 3;
  for (uint32_t c = 0; c < 256; c++) {
    if (offsets[c] > offsets[c + 1] || offsets[c + 1] > offsets[256]) return 3;
    for (uint32_t p = offsets[c]; p < offsets[c + 1]; p++) {
      if (members[p] >= count) return 3;
      if (p > offsets[c] && members[p - 1] >= members[p]) return 3;
    }
  }
  return 0;
}

/* inverted_file.cpp:164-176 `validate`. */
int fbs_oracle_index_validate(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, const uint32_t *offsets,
                              const uint32_t *members, const uint32_t *cells,
                              uint32_t absent_count) {
  if (fbs_oracle_index_validate_structure(offsets, members, cells, count, absent_count)) return 3;
  uint32_t absent = 0;
  for (uint32_t t = 0; t < count; t++) {
    if (cells[t] == ABSENT) {
      absent++;
      continue;
    }
    if (cells[t] != fbs_oracle_index_cell(table + (size_t)t * width, width, roots)) return 3;
  }
  return absent == absent_count ? 0 : 3;
}

/* inverted_file.cpp:112-138 `build_index`: a counting sort by cell, tokens ascending. */
int fbs_oracle_index_build(const int32_t *table, uint32_t count, uint32_t width,
                           const int32_t *roots, int allow_absent, uint32_t *offsets,
                           uint32_t *members, uint32_t *cells, uint32_t *absent_count) {
  if (count == 0) return 1;
  memset(offsets, 0, 257 * sizeof(uint32_t));
  *absent_count = 0;
  for (uint32_t t = 0; t < count; t++) {
    const uint32_t c = fbs_oracle_index_cell(table + (size_t)t * width, width, roots);
    if (c == ABSENT && !allow_absent) return 2;
    cells[t] = c;
    if (c == ABSENT)
      ++*absent_count;
    else
      offsets[c + 1]++;
  }
  for (uint32_t c = 0; c < 256; c++) offsets[c + 1] += offsets[c];
  uint32_t cursor[256];
  memcpy(cursor, offsets, sizeof cursor);
  for (uint32_t t = 0; t < count; t++)
    if (cells[t] != ABSENT) members[cursor[cells[t]]++] = t;
  return fbs_oracle_index_validate(table, count, width, roots, offsets, members, cells,
                                   *absent_count);
}

/* inverted_file.cpp:182-236 `update`: the moved token's cell from its (new) row. */
int fbs_oracle_index_update(const int32_t *table, uint32_t count, uint32_t width,
                            const int32_t *roots, uint32_t moved, uint32_t *offsets,
                            uint32_t *members, uint32_t *cells, uint32_t *absent_count) {
  if (moved >= count) return 1;
  if (fbs_oracle_index_validate_structure(offsets, members, cells, count, *absent_count)) return 3;
  const uint32_t old_cell = cells[moved];
  if (old_cell != ABSENT && old_cell > 255) return 3;
  const uint32_t new_cell = fbs_oracle_index_cell(table + (size_t)moved * width, width, roots);
  if (new_cell == ABSENT) return 2;
  if (old_cell == new_cell) return 0;
  uint32_t remove_pos = ABSENT;
  if (old_cell != ABSENT) {
    for (uint32_t p = offsets[old_cell]; p < offsets[old_cell + 1]; p++)
      if (members[p] == moved) {
        remove_pos = p;
        break;
      }
    if (remove_pos == ABSENT) return 3;
  } else if (*absent_count == 0) {
    return 3;
  }
  const uint32_t size = offsets[256];
  if (old_cell == ABSENT) {
    uint32_t p = offsets[new_cell];
    while (p < offsets[new_cell + 1] && members[p] < moved) p++;
    memmove(members + p + 1, members + p, (size - p) * sizeof(uint32_t));
    members[p] = moved;
    for (uint32_t c = new_cell + 1; c <= 256; c++) offsets[c]++;
    --*absent_count;
  } else if (old_cell < new_cell) {
    uint32_t before = offsets[new_cell];
    while (before < offsets[new_cell + 1] && members[before] < moved) before++;
    const uint32_t target = before - 1;
    for (uint32_t p = remove_pos; p < target; p++) members[p] = members[p + 1];
    members[target] = moved;
    for (uint32_t c = old_cell + 1; c <= new_cell; c++) offsets[c]--;
  } else {
    uint32_t at = offsets[new_cell];
    while (at < offsets[new_cell + 1] && members[at] < moved) at++;
    for (uint32_t p = remove_pos; p > at; p--) members[p] = members[p - 1];
    members[at] = moved;
    for (uint32_t c = new_cell + 1; c <= old_cell; c++) offsets[c]++;
  }
  cells[moved] = new_cell;
  return fbs_oracle_index_validate(table, count, width, roots, offsets, members, cells,
                                   *absent_count);
}

/* inverted_file.cpp:238-249 `remove_token` (with remove_from_bucket, :84-100). */
int fbs_oracle_index_remove(uint32_t count, uint32_t moved, uint32_t *offsets, uint32_t *members,
                            uint32_t *cells, uint32_t *absent_count) {
  if (moved >= count) return 1;
  if (fbs_oracle_index_validate_structure(offsets, members, cells, count, *absent_count)) return 3;
  const uint32_t old_cell = cells[moved];
  if (old_cell == ABSENT) return 0;
  /* The reference reads offsets[old_cell] unchecked here (remove_from_bucket, :84-100); a
   * stored cell past 255 has no range, and is refused as a CSR invariant. */
  if (old_cell > 255) return 3;
  uint32_t remove_pos = ABSENT;
  for (uint32_t p = offsets[old_cell]; p < offsets[old_cell + 1]; p++)
    if (members[p] == moved) {
      remove_pos = p;
      break;
    }
  if (remove_pos == ABSENT) return 3;
  memmove(members + remove_pos, members + remove_pos + 1,
          (offsets[256] - remove_pos - 1) * sizeof(uint32_t));
  for (uint32_t c = old_cell + 1; c <= 256; c++) offsets[c]--;
  ++*absent_count;
  cells[moved] = ABSENT;
  return fbs_oracle_index_validate_structure(offsets, members, cells, count, *absent_count);
}

/* inverted_file.cpp:38-47 `cell_distance`: the query's first and last 8 values against the
 * cell's two roots. */
static int64_t cell_distance(const int32_t *query, uint32_t width, const int32_t *roots,
                             uint32_t cell) {
  const int32_t *first = roots + 8 * (cell / 16), *last = roots + 8 * (cell % 16);
  const int32_t *qlast = query + width - 8;
  int64_t d = 0;
  for (int i = 0; i < 8; i++) {
    const int64_t a = (int64_t)query[i] - first[i], b = (int64_t)qlast[i] - last[i];
    d += (a < 0 ? -a : a) + (b < 0 ? -b : b);
  }
  return d;
}

/* inverted_file.cpp:26-36 `l1` over the whole row. */
static int64_t row_l1(const int32_t *query, const int32_t *row, uint32_t width) {
  int64_t d = 0;
  for (uint32_t i = 0; i < width; i++) {
    const int64_t x = (int64_t)query[i] - row[i];
    d += x < 0 ? -x : x;
  }
  return d;
}

/* Keeps the n smallest (key, id) pairs, ascending, ties to the lower id: the first n of the
 * reference's sort by (distance, id). */
static void keep_smallest(int64_t key, uint32_t id, uint32_t n, int64_t *keys, uint32_t *ids) {
  for (uint32_t i = 0; i < n; i++) {
    if (key < keys[i] || (key == keys[i] && id < ids[i])) {
      for (uint32_t j = n - 1; j > i; j--) {
        keys[j] = keys[j - 1];
        ids[j] = ids[j - 1];
      }
      keys[i] = key;
      ids[i] = id;
      return;
    }
  }
}

/* inverted_file.cpp:83-96 `fill_admitted`: the k nearest non-empty cells. */
static void admit(const int32_t *query, uint32_t width, const int32_t *roots,
                  const uint32_t *offsets, uint32_t k, uint32_t *admitted) {
  int64_t dist[16];
  for (int i = 0; i < 16; i++) {
    admitted[i] = ABSENT;
    dist[i] = INT64_MAX;
  }
  for (uint32_t c = 0; c < 256; c++)
    if (offsets[c] != offsets[c + 1])
      keep_smallest(cell_distance(query, width, roots, c), c, k, dist, admitted);
}

/* inverted_file.cpp:250-258 `probe` (with rank_bucket, :49-64): members of the admitted
 * cells ranked by row L1, top 8, ties to the lower token. */
int fbs_oracle_index_probe(const int32_t *table, uint32_t count, uint32_t width,
                           const int32_t *roots, const int32_t *query, uint32_t k,
                           const uint32_t *offsets, const uint32_t *members,
                           const uint32_t *cells, uint32_t absent_count, uint32_t *admitted,
                           uint32_t *top8, uint32_t *prediction) {
  if (k == 0 || k > 16) return 1;
  if (fbs_oracle_index_validate(table, count, width, roots, offsets, members, cells, absent_count))
    return 3;
  admit(query, width, roots, offsets, k, admitted);
  int64_t dist[8];
  for (int i = 0; i < 8; i++) {
    top8[i] = ABSENT;
    dist[i] = INT64_MAX;
  }
  for (uint32_t i = 0; i < 16; i++) {
    const uint32_t c = admitted[i];
    if (c == ABSENT) continue;
    for (uint32_t p = offsets[c]; p < offsets[c + 1]; p++)
      keep_smallest(row_l1(query, table + (size_t)members[p] * width, width), members[p], 8, dist,
                    top8);
  }
  *prediction = top8[0];
  return top8[0] == ABSENT ? 1 : 0;
}

/* inverted_file.cpp:260-270 `full_scan` (with rank_full_scan, :66-81): cells admitted from an
 * index built over the table with absent tokens allowed, then every token of an admitted cell
 * ranked. */
int fbs_oracle_index_full_scan(const int32_t *table, uint32_t count, uint32_t width,
                               const int32_t *roots, const int32_t *query, uint32_t k,
                               uint32_t *admitted, uint32_t *top8, uint32_t *prediction) {
  if (k == 0 || k > 16) return 1;
  if (count == 0) return 1;
  uint32_t offsets[257] = {0};
  for (uint32_t t = 0; t < count; t++) {
    const uint32_t c = fbs_oracle_index_cell(table + (size_t)t * width, width, roots);
    if (c != ABSENT) offsets[c + 1]++;
  }
  for (uint32_t c = 0; c < 256; c++) offsets[c + 1] += offsets[c];
  admit(query, width, roots, offsets, k, admitted);
  int64_t dist[8];
  for (int i = 0; i < 8; i++) {
    top8[i] = ABSENT;
    dist[i] = INT64_MAX;
  }
  for (uint32_t t = 0; t < count; t++) {
    const int32_t *row = table + (size_t)t * width;
    const uint32_t c = fbs_oracle_index_cell(row, width, roots);
    if (c == ABSENT) continue;
    int in = 0;
    for (int i = 0; i < 16; i++) in |= admitted[i] == c;
    if (in) keep_smallest(row_l1(query, row, width), t, 8, dist, top8);
  }
  *prediction = top8[0];
  return top8[0] == ABSENT ? 1 : 0;
}
