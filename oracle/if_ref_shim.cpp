// Test infrastructure: a C entry layer over the reference's own inverted-file host library
// (projects/uor-cuda-inverted-file/src/inverted_file.cpp + codebook.cpp, compiled from where
// they lie into oracle/_ref/ by `make -C oracle ref`), so the tests can hold this build's index
// to the reference's on the same tables. Flat arrays in and out: table [count][32] int32 (four
// 8-value blocks, the reference's Token), offsets[257], members[count], cells[count].
#include <cstring>

#include "uor_inverted_file.hpp"

namespace ifr = uor_inverted_file;

namespace {

ifr::Table table_of(const int32_t *table, uint32_t count) {
  ifr::Table t;
  t.tokens.resize(count);
  for (uint32_t i = 0; i < count; i++)
    for (int b = 0; b < 4; b++)
      for (int d = 0; d < 8; d++) t.tokens[i][b][d] = table[(i * 4 + b) * 8 + d];
  return t;
}

ifr::Index index_of(const uint32_t *offsets, const uint32_t *members, const uint32_t *cells,
                    uint32_t count, uint32_t absent) {
  ifr::Index x;
  std::memcpy(x.offsets.data(), offsets, 257 * sizeof(uint32_t));
  x.members.assign(members, members + offsets[256]);
  x.cells.assign(cells, cells + count);
  x.absent_count = absent;
  return x;
}

void out(const ifr::Index &x, uint32_t *offsets, uint32_t *members, uint32_t *cells,
         uint32_t *absent) {
  std::memcpy(offsets, x.offsets.data(), 257 * sizeof(uint32_t));
  std::memcpy(members, x.members.data(), x.members.size() * sizeof(uint32_t));
  std::memcpy(cells, x.cells.data(), x.cells.size() * sizeof(uint32_t));
  *absent = x.absent_count;
}

}  // namespace

extern "C" {

void if_ref_codebook(int32_t *roots) {
  for (int r = 0; r < 16; r++)
    for (int d = 0; d < 8; d++) roots[r * 8 + d] = ifr::codebook[r][d];
}

int if_ref_build(const int32_t *table, uint32_t count, int allow_absent, uint32_t *offsets,
                 uint32_t *members, uint32_t *cells, uint32_t *absent) {
  ifr::Index x;
  const int st = (int)ifr::build(table_of(table, count), x, allow_absent != 0);
  if (st == 0) out(x, offsets, members, cells, absent);
  return st;
}

int if_ref_update(const int32_t *table, uint32_t count, uint32_t moved, uint32_t *offsets,
                  uint32_t *members, uint32_t *cells, uint32_t *absent) {
  ifr::Index x = index_of(offsets, members, cells, count, *absent);
  const int st = (int)ifr::update(table_of(table, count), moved, x);
  out(x, offsets, members, cells, absent);
  return st;
}

int if_ref_remove(const int32_t *table, uint32_t count, uint32_t moved, uint32_t *offsets,
                  uint32_t *members, uint32_t *cells, uint32_t *absent) {
  ifr::Index x = index_of(offsets, members, cells, count, *absent);
  const int st = (int)ifr::remove_token(table_of(table, count), moved, x);
  out(x, offsets, members, cells, absent);
  return st;
}

int if_ref_validate(const int32_t *table, uint32_t count, const uint32_t *offsets,
                    const uint32_t *members, const uint32_t *cells, uint32_t absent) {
  return (int)ifr::validate(table_of(table, count), index_of(offsets, members, cells, count, absent));
}

int if_ref_validate_structure(const uint32_t *offsets, const uint32_t *members,
                              const uint32_t *cells, uint32_t count, uint32_t absent) {
  return (int)ifr::validate_structure(index_of(offsets, members, cells, count, absent));
}

static void scan_out(const ifr::ScanResult &r, uint32_t *admitted, uint32_t *top8,
                     uint32_t *prediction) {
  std::memcpy(admitted, r.admitted.data(), 16 * sizeof(uint32_t));
  std::memcpy(top8, r.top8.data(), 8 * sizeof(uint32_t));
  *prediction = r.prediction;
}

static ifr::Query query_of(const int32_t *q) {
  ifr::Query x;
  for (int b = 0; b < 4; b++)
    for (int d = 0; d < 8; d++) x[b][d] = q[b * 8 + d];
  return x;
}

int if_ref_probe(const int32_t *table, uint32_t count, const int32_t *query, uint32_t k,
                 const uint32_t *offsets, const uint32_t *members, const uint32_t *cells,
                 uint32_t absent, uint32_t *admitted, uint32_t *top8, uint32_t *prediction) {
  ifr::ScanResult r;
  const int st = (int)ifr::probe(table_of(table, count), query_of(query), k,
                                 index_of(offsets, members, cells, count, absent), r);
  scan_out(r, admitted, top8, prediction);
  return st;
}

int if_ref_full_scan(const int32_t *table, uint32_t count, const int32_t *query, uint32_t k,
                     uint32_t *admitted, uint32_t *top8, uint32_t *prediction) {
  ifr::ScanResult r;
  const int st = (int)ifr::full_scan(table_of(table, count), query_of(query), k, r);
  scan_out(r, admitted, top8, prediction);
  return st;
}

}  // extern "C"
