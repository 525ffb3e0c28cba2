// fbs_device.h - the device image of a SpiralCore/FBS model and the launch arguments, shared by
// the kernels (fbs_run.h) and the host side that builds them (fbs_api.cpp).
//
// Layout in HBM (all tables uploaded once by uor_fbs_model_create, read by every sequence):
//   per layer: gains (d i16), window taps ((W+1) x d i16, tap s = s positions back) and their
//              descriptor forms (grid_desc for gains, tap_desc for taps; fbs_int.h),
//              conv_bias (d i32), gate_bias (d/4 + d i32), decay_offset (d/4 i32), and the
//              layer's gather program: [slot][64 lanes] u16 LDS word indices that carry out the
//              six FBS projections (stack_fbs_gather, session.rs:4037-4053) for this lane mapping;
//   writer: the table as biased u16 rows (v ^ 0x8000, vocab x d), drawer keys (D x 16 i16:
//           first-block key then last-block key), CSR drawer offsets (D + 1) and members;
//   per-sequence work (the library's, sized for the resident grid): the causal window ring,
//           [block][layer][W][d] i32.
// Lane mapping: one 64-lane wavefront runs one sequence. Lane j owns quaternions j + 64 k
// (k < QPL) of the recurrence, i.e. channels 4 q .. 4 q + 3, and MLP quaternions j + 64 k
// (k < mpl).
#ifndef UOR_FBS_DEVICE_H
#define UOR_FBS_DEVICE_H

#include <stddef.h>
#include <stdint.h>

namespace fbs {

constexpr uint32_t kWave = 64;
constexpr uint32_t kMaxMpl = 4;        // mlp <= 1024
constexpr uint32_t kMaxWidth = 1024;   // WRITER_MAX_WIDTH, format.rs:437
constexpr uint32_t kMaxDrawers = 4096;
constexpr uint32_t kMaxProbes = 64;
constexpr uint32_t kMaxWindow = 64;
constexpr int32_t kMaxKeyQ12 = 16384;  // |drawer key| bound that keeps a drawer score in 20 bits
constexpr uint32_t kListCap = 2048;    // member ids staged in LDS per scan segment
constexpr uint32_t kSeedWords = 384 + 256;  // the rsqrt and reciprocal seed tables (fbs_int.h)

struct DevLayer {
  const int16_t *rec_gain;
  const int16_t *mlp_gain;
  const int16_t *taps;          // (W + 1) * d, [tap][channel]
  const int32_t *conv_bias;     // d
  const int32_t *gate_bias;     // d/4 + d
  const int32_t *decay_offset;  // d/4
  const uint16_t *prog;         // nslots * 64
  const uint16_t *taps_desc;    // tap_desc of taps
  const uint16_t *rec_gain_desc;
  const uint16_t *mlp_gain_desc;
};

// The Hamming reads of a lut-stack/6 stack (fbs_hamming.h), one entry per read. Every table is
// the host's: the three rotations' unit quaternions at Q31 (`units`, hamming.rs:541-548) and
// each vocabulary entry's key code per head (`vocab_codes`, :566-582), copy heads first.
constexpr uint32_t kMaxHamKept = 64;        // positions a head keeps
constexpr uint32_t kHamPosBits = 24;        // positions below 2^24 (a pick packs its distance above)
constexpr uint32_t kHamBins = 68;            // distances 0..64 (a word per distance), padded
constexpr uint32_t kHamNoSlot = 0xffffffffu;
constexpr uint32_t kHamReqWords = 8;         // a read's request to a paired block's second wave

struct DevHamRead {
  const int64_t *qu, *ku, *vu;  // d each: query, key and value units
  const uint64_t *codes;        // vocab * heads
  const int32_t *margin;        // heads, bits at Q16
  const uint32_t *wd;           // heads * kHamBins: each distance's Q31 weight (copy_weight_q31)
  const int32_t *w;             // 2 d at 2^-24: w_c, then w_y
  const int16_t *ask;           // vocab * d question table (Q12), or null: the read does not ask
  const int32_t *carry;         // vocab carry gains (Q16), or null
  uint32_t carry_rows;          // the carry's reach
  uint32_t typed;               // type heads served (some w_y is not zero)
  uint32_t slot;                // payload cache of a typed read that does not ask, else kHamNoSlot
  uint32_t heads_before;        // the served heads of the earlier reads (a trace record's place)
};

// The readout read's place read (fbs_hamming.h's place register): the marks and the classes.
constexpr uint32_t kPlaceMarkMax = 16;     // ids a marker list holds (UOR_FBS_PLACE_MARK_MAX)
constexpr uint32_t kPlaceWords = 16;       // the register's scalars in LDS
constexpr uint32_t kPlaceNone = 0xffffffffu;
constexpr uint32_t kPlaceStop = 1, kPlaceArm = 2, kPlaceOpen = 4;  // the class bits

struct DevHam {
  uint32_t heads;               // 0: the model has no Hamming reads
  uint32_t copy, hw, kept;      // heads / 2 copy heads, d / heads coordinates a head
  uint32_t rule;                // the copy rule served (UOR_FBS_COPY_*, resolved)
  uint32_t has_marker, m0, m1;  // the longest rule's reply marker
  uint32_t slots;               // payload caches a session keeps
  uint32_t place;               // 1: the readout read's place read
  uint32_t p_read;              // the place read's index (the readout read)
  uint32_t p_bos, p_eos;        // the document's start and end marks
  uint32_t p_len[4];            // the separator's and the system, user, assistant markers' lengths
  uint32_t p_carry_rows;        // the place read's question carry reach
  uint32_t nreads;              // the reads
  const uint64_t *pair;         // copy: a copy key 2 head's first-half mask, else 0
  const int32_t *at;            // L + 1: the read index at each depth, or -1
  const DevHamRead *reads;
  const uint32_t *p_marks;      // 4 * kPlaceMarkMax: the separator, then the role markers
  const uint8_t *p_class;       // vocab: UOR_FBS_PLACE_STOP | _ARM | _OPEN
  const int16_t *p_ask;         // the place read's question table (vocab * d, Q12)
  const int32_t *p_carry;       // its carry gains (Q16), or null
  const uint32_t *ones;         // kHamBins ones: every distance kept (the trace's nearest)
};

struct DevModel {
  uint32_t vocab, d, m, L, W, D, P, head, context, raw_gates, raw_transition;
  uint32_t nq, nm, mpl, qpl;
  uint32_t nslots, s_rec_in, s_rec_gate, s_rec_out, s_mlp_gate, s_mlp_up, s_mlp_down;
  uint32_t xbar_words;      // 2 * max(d, m)
  uint32_t identity_rows;   // the nearest head: one drawer holding every token
  uint32_t taps_fast;       // every window tap has a descriptor (tap_desc != kGridDescSlow)
  uint32_t gains_fast;      // every norm gain (rec, mlp, final) has a descriptor (grid_desc)
  uint32_t log2d;           // log2(d) when d is a power of two, else 0xff
  uint32_t writer_memory;   // 1: a query equal to the writer's last one takes its result
  uint64_t w_recip;         // floor(2^32 / W): the ring slot of a position without division
  const DevLayer *layers;   // L entries
  const int16_t *final_gain;
  const uint16_t *final_gain_desc;
  const uint16_t *table_b;  // vocab * d, biased
  const int16_t *keys;      // D * 16
  const uint32_t *offsets;  // D + 1
  const uint32_t *members;  // offsets[D]
  const int8_t *icosian;    // 120 * 8
  const uint64_t *keep_q31; // 16
  const int64_t *eps_int;   // 9: the RMSNorm epsilon at each pre-shift 0..8
  DevHam ham;
  // An int8 table (uor_fbs_ext.table_i8): its codes biased, code + 128, vocab * d bytes, which
  // the writer's scan reads in place of table_b (half the bytes a candidate row moves); null
  // for an i16 table. Last, so that the other fields keep their kernel-argument offsets.
  const uint8_t *table8;
  uint32_t t8_shift;        // the int8 table's shift to Q12
  // Member ids the one-wavefront writer stages in LDS per scan segment: kListCap, or half of it
  // for a model with Hamming reads, so that four of their blocks share a CU's LDS at C3's shape.
  uint32_t list_cap;
  // eps_int[0] as a kernel argument: the pre-shift is 0 for almost every norm, whose epsilon is
  // then read from the argument segment instead of by a global load on the step's serial path.
  int64_t eps0;
};

// LDS bytes per block (the layout the kernels carve): the gather crossbar, the MLP outputs, the
// drawer scores, the kept drawers, the staged member list, the writer's last query and token,
// the seed tables, and every layer's recurrence state (i64).
inline size_t lds_bytes(const DevModel &M) {
  return 4ull * (M.xbar_words + 2 * M.m + ((M.D + 3u) & ~3u) + kMaxProbes + M.list_cap +
                 ((M.d + 3u) & ~3u) + 4 + kSeedWords) +
         8ull * M.L * M.d;
}

// Paired blocks (two wavefronts per sequence) add the window sums and gate quaternions handed
// from wave 1 to wave 0 (2 d i64), the kept drawers' ranges and four per-wave results.
// With two or more quaternions a lane, or Hamming reads, the state lives in global memory
// (kPairStateGlobal, pair_state_global).
inline size_t pair_lds_bytes(const DevModel &M) {
  return lds_bytes(M) + 4ull * (4 * M.d + 2 * kMaxProbes + 8) -
         (M.qpl >= 2 || M.ham.heads ? 8ull * M.L * M.d : 0);
}

// A Hamming model's kernels add the session's tokens (context u32), the distances (context
// bytes), one head's picks and weights (2 kMaxHamKept u32), its distance histogram and the
// weight of each distance (2 kHamBins u32) and the sign nibbles (d / 4 u32).
inline size_t place_lds_bytes(const DevModel &M) {
  // The register's scalars, then per position the end of its finished user turn (u16) and an
  // arming row's find + 1 (u16).
  return M.ham.place ? 4ull * kPlaceWords + 2 * ((2ull * M.context + 15ull) & ~15ull) : 0;
}

inline size_t ham_lds_bytes(const DevModel &M) {
  if (!M.ham.heads) return 0;
  return 4ull * M.context + ((M.context + 15ull) & ~15ull) + 8ull * kMaxHamKept + 8ull * kHamBins +
         4ull * (M.d / 4) + 4ull * kHamReqWords + place_lds_bytes(M);
}

// The paired Hamming kernels' second wavefront keeps its read scratch where a read leaves LDS
// unused (ham_help_lds): its distances, picks, weights, histogram and nibbles in the writer's
// staging list, the point and partial sums (3 d i64) over the gather crossbar, the MLP outputs
// and the drawer scores.
inline bool ham_pair_fits(const DevModel &M) {
  const uint64_t scratch = ((M.context + 15ull) & ~15ull) / 4 + 2ull * kMaxHamKept + 2ull * kHamBins + M.d / 4;
  const uint64_t pool = (uint64_t)M.xbar_words + 2ull * M.m + ((M.D + 3u) & ~3u);
  return scratch <= M.list_cap && pool >= 6ull * M.d;
}

// One serving slot's cache (uor_fbs_serve_slots_async), bytes from the entry's start: a u32 tag
// (the position + 1 the window sums hold for; 0: none), a u32 flag (the writer memory below
// holds a query), the memory's token, a u32 fingerprint of the slot's state the sums were formed
// beside (a launch that finds another state there sums the window afresh), then its query
// (d i32), its kept drawers (kMaxProbes u32) and, for paired blocks, the slot's window sums for
// its next step (L d i64).
struct SlotCacheLayout {
  uint32_t query, kept, sums, bytes;
};
__host__ __device__ inline SlotCacheLayout slot_cache_layout(const DevModel &M) {
  SlotCacheLayout c;
  c.query = 16;
  c.kept = c.query + 4 * ((M.d + 3u) & ~3u);
  c.sums = (c.kept + 4 * kMaxProbes + 15u) & ~15u;
  c.bytes = (c.sums + 8 * M.L * M.d + 255u) & ~255u;
  return c;
}

enum RunMode : uint32_t { kModeSequences = 0, kModeDecode = 1, kModeScore = 2 };

// Per-sequence status: 0, or the reference's codes (1 token, 2 context), or a slot past the
// slot arrays' capacity.
constexpr int32_t kStatusSlot = 3;

struct RunArgs {
  uint32_t mode;
  uint32_t n;          // sequences / rows
  uint32_t len;        // tokens per sequence (sequences, score) or the prompt length (decode)
  uint32_t gen;        // decode: generated steps
  const uint32_t *tokens;
  uint32_t *out_tokens;   // sequences: n*len; decode: n*(gen+1); score: n*len (nullable)
  uint32_t *out_kept;     // sequences: n*len*P (nullable)
  int32_t *out_query;     // sequences: n*len*d (nullable)
  const int64_t *in_state;
  const int32_t *in_history;
  const uint32_t *in_position;
  int64_t *out_state;
  int32_t *out_history;
  uint32_t *out_position;
  unsigned long long *matches;
  int32_t *status;        // n
  // Session slots: sequence s keeps its state and position at index slots[s] of the in/out
  // arrays (the same arrays, updated in place), and out_history's entry of that slot is the
  // sequence's window ring itself ([layer][W][d], row p mod W holding the drive of position
  // p), so nothing is copied between launches; null = index s, the rows exported newest first
  // through the block's own ring. A slot at or past `capacity` is refused with status
  // kStatusSlot. Slot sequences export their state and position also when a step is refused:
  // the session then holds the tokens stepped before it.
  const uint32_t *slots;
  uint32_t capacity;
  int32_t *ring;          // gridDim.x * L * W * d
  int64_t *hist;          // paired blocks: gridDim.x * L * d, the next step's window sums
  // Hamming models: the session's token stream ([n][context]: x_0..x_{position-1}) and its type
  // heads' payload caches ([n][slots][context][d]) in and out (null: a fresh stream, none
  // exported); `pay` the library's caches for sequences with no out_payloads, [gridDim.x][...].
  const uint32_t *in_stream;
  uint32_t *out_stream;
  const int64_t *in_payloads;
  int64_t *out_payloads;
  int64_t *pay;
  // Serving slots: each slot's cache (SlotCacheLayout, `cache_stride` bytes a slot; null: none)
  // and context slide flags (nonzero: the slot's session continues past a full context; null:
  // none slides).
  uint8_t *cache;
  uint32_t cache_stride;
  const uint8_t *slide;
  // One wavefront a sequence only: the snap trace, L (2 d/4 + m/4) bytes a position, of every
  // position (sequences) or of every step, len + gen a sequence (decode) (null: none).
  uint8_t *out_trace;
  // The part clocks' kernels only: kPartWords u64 a sequence (Part).
  uint64_t *out_parts;
  // The traced kernels only (uor_fbs_decision_sequences): every position's record, `dstride`
  // bytes (decision_layout), and the forced replay: rate buckets [n][len][L][d/4] (255: none),
  // codes [n][len][reads][heads][2] (query, key) with their mask [n][len][reads][heads] (bit 0
  // the query, bit 1 the key); null: nothing forced. `decisions`: the record holds the buckets.
  uint8_t *out_dtrace;
  uint32_t dstride, decisions;
  const uint8_t *force_buckets;
  const uint64_t *force_codes;
  const uint8_t *force_mask;
  // The deferred writer (one-token serving launches of the paired prefill kernels, keyed
  // drawers; null job_flag: the writer runs in the step). A step that does not take the
  // writer's remembered result ends at its drawer selection: sequence s's query goes to
  // job_query (d / 2 words of 16-bit pairs as the writer's scan packs them for the table),
  // each kept drawer c lists s in
  // drawer_list[c][.] (drawer_count[c] entries, list_stride a drawer), job_best[s] starts at
  // the largest (L1, token) and job_flag[s] at 1. The session that opens a slice of 16 entries
  // of c's list appends the slice's work items, one per 64 members of c (ServeScan::items).
  uint32_t *job_query;
  uint32_t *job_flag;
  unsigned long long *job_best;
  uint32_t *drawer_count;
  uint32_t *drawer_list;
  uint32_t list_stride;
  uint4 *items;
  uint32_t *item_count;
  uint32_t item_cap;
};

// The drawer-major scan of the deferred writer's jobs (fbs_serve.hip). A work item is one
// (drawer, 64 members) chunk and one slice of 16 sessions that kept the drawer:
// (first member index, rows, first drawer-list index, drawer). fbs_serve_scan's blocks take the
// items in turn, score every member row against the queries of the slice's sessions and
// combine each session's lowest (L1 << 32 | token) by a 64-bit atomic minimum; then
// fbs_serve_finish hands each job's token out (and to the slot cache's writer memory) and clears
// the drawer counts and the item count for the next launch.
constexpr uint32_t kServeRows = 64;       // member rows a scan block holds, one per lane
constexpr uint32_t kServeSessions = 16;   // sessions a scan block scores at once
struct ServeScan {
  uint4 *items;
  uint32_t *item_count;
  uint32_t item_cap;
  uint32_t n;                             // sequences of the launch
  uint32_t gen;                           // the launch's generated steps (the out_tokens stride)
  const uint32_t *job_query;
  uint32_t *job_flag;
  unsigned long long *job_best;
  uint32_t *drawer_count;
  const uint32_t *drawer_list;
  uint32_t list_stride;
  uint32_t *out_tokens;
  const uint32_t *slots;
  uint8_t *cache;                         // nullable
  uint32_t cache_stride;
};

// A traced position's record (uor_fbs_decision_sequences): with the decisions, each layer's rate
// scores (i32, [L][d/4]) then the entries used (u8, [L][d/4]), padded to 8 bytes; then each read
// in depth order, each served head (the copy heads, then the type heads where the read serves
// them): the query (u64), the key at the row (u64), the kept count (u32) and kept positions (u32,
// `kept` of them), padded to 8 bytes.
constexpr uint32_t decision_head_bytes(uint32_t kept) { return (20u + 4u * kept + 7u) & ~7u; }
constexpr uint32_t decision_bucket_bytes(uint32_t L, uint32_t lanes) { return (5u * L * lanes + 7u) & ~7u; }

// The part clocks (uor_fbs_decode_parts_async, after the reference's measure_fbs_step_parts,
// session.rs:4753): the phases of a paired block's step in the order they run, each wave's
// shader-clock cycles summed over a sequence's steps and layers. Wave 0 (the recurrence) and
// wave 1 (the window ring) share the numbering; a phase one wave does not run stays 0, and a
// barrier's entry is the time the wave waited there.
enum Part : uint32_t {
  kPartEmbed = 0,     // wave 0: the token's table row
  kPartLoads,         // the layer's parameters and gather words issued (wave 1: the window sums)
  kPartNormRec,       // wave 0: the recurrence block's norm, gain and publish
  kPartSync1,
  kPartTransition,    // wave 0: gathers, lane weights, the transition and its product with the
                      // state; wave 1: drive and gate gathers, tap 0, the ring write, the gates'
                      // quaternions
  kPartSync2,
  kPartTransport,     // wave 0: the transport and the output gate's product; wave 1: the next
                      // step's window sums
  kPartRequantRec,    // wave 0: quantize16 of the gate outputs and their publish
  kPartResidualRec,   // wave 0: the rec_out gathers and the residual add
  kPartNormMlp,       // wave 0: the feed-forward block's norm, gain and publish
  kPartSync3,
  kPartMlp,           // both: the waves' MLP quaternion groups
  kPartSync4,
  kPartRequantMlp,    // both: quantize16 of the waves' MLP groups
  kPartSync5,
  kPartResidualMlp,   // wave 0: the mlp_down gathers and the residual add
  kPartFinal,         // wave 0: the final norm, gain, Q12 query and the writer-memory check
  kPartSync6,
  kPartSelect,        // wave 0: drawer scores and the P kept drawers (or the remembered result)
  kPartSync7,
  kPartScan,          // both: the wave's half of the candidate rows
  kPartSync8,
  kPartStep,          // between steps: the token written out, the position advanced
  kParts
};
// Per sequence: cycles [wave][kParts], then the steps run and the sequence's wall time in ticks
// of the 100 MHz real-time counter (wave 0).
constexpr uint32_t kPartWords = 2 * kParts + 2;
// The part clocks' kernels add each wave's counters to the paired blocks' LDS (2 kParts u64).
inline size_t clock_lds_bytes() { return 16ull * kParts; }

}  // namespace fbs

#endif
