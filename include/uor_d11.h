/*
 * uor_d11.h - C ABI of the discrete M1 row scorer on MI355X (gfx950).
 *
 * Replaces the reference's GPU panel scorer for the discrete `UORLUT01` container
 * (`uor-r4.lut-discrete/1` and the 19-table `uor-r4.lut-discrete-trunk/1`):
 *   - the kernel `d11_score_rows` (docs/labs/m1-d11-artifact-scorer/instrument/src/
 *     scorer.cu:12-41) and its host launcher `DeviceScorer::new` / `DeviceScorer::score`
 *     (instrument/src/device.rs:60-210), which evaluate
 *   - `IntegerDiscreteModel::evaluate_prefix` and `observe_target`
 *     (crates/uor-r4-integer/src/discrete_d11.rs:1761-1995) for every (prefix, target) row.
 *
 * The caller parses the container (the checks of `from_bytes`, discrete_d11.rs:931-1278) and
 * passes its sections as plain arrays; the library checks the model's shape and the trunk's
 * triples again, holds device copies, and builds the row plans (`build_row_plan`,
 * discrete_d11.rs:813-884) for every prefix length. Integer only. One handle per device; a
 * handle is not safe to use from two threads at once, distinct handles are.
 *
 * Return codes: 0 success, -1 invalid argument, -2 device error (uor_d11_last_error() names
 * it). Per-row statuses are in the records (UOR_D11_ROW_*), as the reference kernel's
 * (kernel_core.h:33-42).
 */
#ifndef UOR_D11_H
#define UOR_D11_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UOR_D11_ABI_VERSION 2u

#define UOR_D11_MAX_CONTEXT 243u
#define UOR_D11_MAX_BLOCKS 16u
#define UOR_D11_MAX_KEPT 8u
#define UOR_D11_MAX_KEPT_CELLS 16u
#define UOR_D11_MAX_SWEEPS 5u
#define UOR_D11_MAX_VOCAB 8192u

/* read_mode (discrete_d11.rs:286-290) */
#define UOR_D11_READ_ROUTE 0u
#define UOR_D11_READ_FLOCK 1u
#define UOR_D11_READ_RELATION 2u

/* The model's flags. STATE_TRANSPORT_KNOCKOUT: evaluate with_state_transport_knockout's copy
 * (discrete_d11.rs:1283-1304): the library (and the oracle) set every route to the identity
 * state 0 and zero the level and relation gates in their own copies of the tables; the route
 * read then returns the last token's blocks untransported (:1346-1361), and the trunk's pointer
 * gate is not applied (:1810-1814). */
#define UOR_D11_FLAG_STATE_TRANSPORT_KNOCKOUT 1u

/* Trace words of evaluate_prefix_traced (discrete_d11.rs:293-297, :1768-1770), per block of
 * the read, in block order:
 * - route read: a header (frontier length, the resolved root, stages taken, the atom) and per
 *   stage (route state, root before the stage, best port, goal root, composed state, next
 *   node) (:1369-1442);
 * - flock and relation reads: a header (query frame root, the block's output root, terms, the
 *   query payload's root) and per level (gate + 1, kept nodes found, their snapped root,
 *   eligible nodes, then 8 kept nodes best first, 8 route states carrying them into the query
 *   frame, 8 carried roots) (:1480-1738).
 * Words no step writes hold 0xffffffff. Relation reads also give each block's relation scores
 * (as u32) padded with 0xffffffff to the node count of a full context's plan (:1474-1478,
 * :1640-1644). */
#define UOR_D11_ROUTE_TRACE_HEADER_WORDS 4u
#define UOR_D11_ROUTE_TRACE_STAGE_WORDS 6u
#define UOR_D11_ACTIVE_TRACE_HEADER_WORDS 4u
#define UOR_D11_ACTIVE_TRACE_LEVEL_WORDS 28u

/* objective_policy (discrete_d11.rs:301-304): which loss `selected_loss` carries */
#define UOR_D11_POLICY_NEAREST_ADDRESS_MARGIN 0u /* loss_ta */
#define UOR_D11_POLICY_OCCUPIED_CELL_RANK 1u     /* loss_tr */

/* Row statuses (kernel_core.h:33-42). */
#define UOR_D11_ROW_OK 0
#define UOR_D11_ROW_PREFIX_LENGTH 1
#define UOR_D11_ROW_PREFIX_TOKEN 2
#define UOR_D11_ROW_PLAN 3
#define UOR_D11_ROW_ORBIT 4
#define UOR_D11_ROW_ROUTE 5
#define UOR_D11_ROW_ZERO_TOKENS 6
#define UOR_D11_ROW_SHAPE 7
#define UOR_D11_ROW_TARGET_TOKEN 8

/* The 15 trunk sections (discrete_d11.rs:500-518, loaded at :1196-1262). sparse[i] holds
 * sparse_rows[i] (key, token, count) triples of table i in the container's order: read, rec,
 * read_rec, rec_shuf, read_rec_shuf, rec_unit, read_rec_unit, query, query_read, query_rec,
 * query_rec_shuf, query_rec_unit. unigram holds 1 + vocabulary words: the global best token,
 * then every token's count. */
typedef struct {
  uint32_t step_candidates[64];
  uint32_t norm_candidates[4];
  const uint32_t *unigram;
  const uint32_t *sparse[12];
  uint64_t sparse_rows[12];
} uor_d11_trunk;

/* The model: DiscreteLutShape's integers (discrete_d11.rs:307-321) and the four base sections
 * (discrete.table i32 [vocabulary][blocks][8], every block one of the 16 orbit roots;
 * discrete.cells u32 [vocabulary]; discrete.routes u32 [blocks][stages]; discrete.gates i32
 * [blocks][stages] then, for the relation read, [stages][5]); trunk NULL for a 4-table model. */
typedef struct {
  uint32_t vocabulary, blocks, context, kept_cells, stages;
  uint32_t read_mode, read_kept, read_sweeps;
  uint32_t objective_policy;
  uint32_t flags; /* UOR_D11_FLAG_* */
  const int32_t *table;
  const uint32_t *cells;
  const uint32_t *routes;
  const int32_t *gates;
  const uor_d11_trunk *trunk;
} uor_d11_model;

/* One row's record: the fields of the reference kernel's D11RowOut (kernel_core.h:86-99) and
 * observe_target's rival counts and selected loss (discrete_d11.rs:403-415). read_vector holds
 * blocks * 8 coordinates. */
typedef struct {
  int32_t status;
  int32_t admitted_count;
  int32_t top8_count;
  uint32_t prediction;
  uint32_t admitted[UOR_D11_MAX_KEPT_CELLS];
  uint32_t top8[8];
  int32_t read_vector[UOR_D11_MAX_BLOCKS * 8];
  uint32_t token_hinge, address_hinge, rank_hinge;
  uint32_t loss_ta, loss_tr;
  uint32_t token_rivals, address_rivals;
  uint32_t selected_loss;
} uor_d11_row_out;

uint32_t uor_d11_abi_version(void);
int64_t uor_d11_sizeof_model(void);
int64_t uor_d11_sizeof_row_out(void);
/* The message of this thread's last failed call. */
const char *uor_d11_last_error(void);

/* Copies the model to `device` and builds the row plans (DeviceScorer::new, device.rs:60-118).
 * Refuses (-1) what from_bytes refuses of the shape, the tables' roots and cells, the routes,
 * the gates and the trunk's candidates and triples. */
int uor_d11_model_create(const uor_d11_model *m, int32_t device, void **handle);
void uor_d11_model_destroy(void *handle);

/* Scores `rows` rows (DeviceScorer::score, device.rs:120-210): prefixes holds rows x stride
 * tokens (row r's first lengths[r] are its prefix), targets one token per row; one record per
 * row in `out`. Host buffers; blocks until done. */
int uor_d11_score_rows(void *handle, const uint32_t *prefixes, const int32_t *lengths,
                       const uint32_t *targets, uint32_t rows, uint32_t stride,
                       uor_d11_row_out *out);

/* The same over device buffers, enqueued on `stream` (a hipStream_t; NULL for the default
 * stream); returns after the launch. */
int uor_d11_score_rows_async(void *handle, const uint32_t *d_prefixes, const int32_t *d_lengths,
                             const uint32_t *d_targets, uint32_t rows, uint32_t stride,
                             uor_d11_row_out *d_out, void *stream);

/* evaluate_prefix_traced (discrete_d11.rs:1768-1770, DiscreteTracedPrefixEvaluation :391-400)
 * for every row: the records as uor_d11_score_rows writes them, plus each row's trace words
 * (uor_d11_trace_words(handle, NULL) a row, the layout above) in `trace` and, for a relation
 * read, its relation words (`*relation_words` a row) in `relation_trace` (required then; ignored
 * otherwise). The reference's CPU evaluator returns these for one prefix; here they come from the
 * same kernels' traced instance. A row whose status is not 0 has unspecified trace words (the
 * reference returns an error and no trace). */
uint32_t uor_d11_trace_words(void *handle, uint32_t *relation_words);
int uor_d11_score_rows_traced(void *handle, const uint32_t *prefixes, const int32_t *lengths,
                              const uint32_t *targets, uint32_t rows, uint32_t stride,
                              uor_d11_row_out *out, uint32_t *trace, uint32_t *relation_trace);
int uor_d11_score_rows_traced_async(void *handle, const uint32_t *d_prefixes,
                                    const int32_t *d_lengths, const uint32_t *d_targets,
                                    uint32_t rows, uint32_t stride, uor_d11_row_out *d_out,
                                    uint32_t *d_trace, uint32_t *d_relation_trace, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* UOR_D11_H */
