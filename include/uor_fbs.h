/*
 * uor_fbs.h - C ABI of the MI355X (gfx950) SpiralCore/FBS integer decode path.
 *
 * This is the drop-in boundary for UOR-R4's `lut-stack` FBS step
 * (`IntegerStackSession::step_native`, crates/uor-r4-integer/src/stack/session.rs:4129-4403)
 * and for the GPU evaluator that the reference drives through `#[repr(C)]` structs and
 * `extern "C"` entry points (docs/labs/d11-exporter-float-trunk/instrument/src/lib.rs:14-95,
 * host_kernel.cpp:8-49, evaluator.cu:8-34, device.rs:93-302).
 *
 * Plain C: fixed-width integers, raw pointers and sizes, no C++ or torch types. The host
 * keeps its own artifact loader (`IntegerStackModel::parse`) and hands the parsed integer
 * arrays over as a `uor_fbs_model` whose layout equals the reference's `CModel` /
 * `fbs_model` byte for byte, so an existing binding passes the same struct.
 *
 * Ownership: `uor_fbs_model_create` copies every table to the device; the caller may free
 * its arrays afterwards. Host-buffer entry points copy in and out and synchronise; the
 * `_async` entry points take device pointers and a HIP stream (as `void *`) and return once
 * the work is queued. A handle is not thread-safe; separate handles are.
 *
 * Status codes: 0 ok, 1 a token outside the vocabulary, 2 a sequence longer than the
 * context (fbs_core.h:625-628, mapped in lib.rs:269-274); the rest are this library's.
 */
#ifndef UOR_FBS_H
#define UOR_FBS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UOR_FBS_ABI_VERSION 3u

#define UOR_FBS_OK 0
#define UOR_FBS_ERR_TOKEN 1       /* token >= vocab (fbs_core.h:627) */
#define UOR_FBS_ERR_CONTEXT 2     /* position >= context (fbs_core.h:628) */
#define UOR_FBS_ERR_ARGUMENT 3    /* a null pointer, a zero or inconsistent size; as a
                                     per-sequence status: a slot past the capacity */
#define UOR_FBS_ERR_SHAPE 4       /* a model the reference's loader would refuse */
#define UOR_FBS_ERR_DEVICE 5      /* a HIP runtime error */
#define UOR_FBS_ERR_UNSUPPORTED 6 /* a shape this build has no kernel for */

/* One FBS projection (fbs_core.h:43-47, lib.rs:14-21): per output 8-block the input atom and
 * eight signed-axis codes (`code & 7` the source lane, `code & 8` negate). */
typedef struct uor_fbs_map {
  const uint16_t *atoms; /* blocks */
  const uint8_t *codes;  /* blocks * 8 */
  uint32_t blocks;
} uor_fbs_map;

/* One recurrence layer (fbs_core.h:49-57, lib.rs:23-39). */
typedef struct uor_fbs_layer {
  const int16_t *rec_gain; /* width grid codes */
  const int16_t *mlp_gain; /* width grid codes */
  uor_fbs_map rec_in;      /* width/8 atoms -> 2*width/8 blocks: drive, then output gate */
  uor_fbs_map rec_gate;    /* width/8 atoms -> (width/4 + width)/8 blocks: decays, rotations */
  uor_fbs_map rec_out;     /* width/8 atoms -> width/8 blocks */
  uor_fbs_map mlp_gate;    /* width/8 atoms -> mlp/8 blocks */
  uor_fbs_map mlp_up;      /* width/8 atoms -> mlp/8 blocks */
  uor_fbs_map mlp_down;    /* mlp/8 atoms -> width/8 blocks */
  const int16_t *taps;     /* 4 * width grid codes [tap][channel], tap s = s positions back */
  const int32_t *conv_bias;    /* width, exponent -16 */
  const int32_t *gate_bias;    /* width/4 + width, exponent -16 */
  const int32_t *decay_offset; /* width/4, Q16 */
} uor_fbs_layer;

/* The model (fbs_core.h:59-73, lib.rs:41-63; filled from `FbsImage`, session.rs:377-446). */
typedef struct uor_fbs_model {
  uint32_t vocab, width, mlp, context, kept, layer_count;
  int64_t eps_mantissa; /* RMSNorm epsilon = eps_mantissa * 2^eps_exp */
  int32_t eps_exp;
  const uor_fbs_layer *layers;
  const int16_t *final_gain;   /* width grid codes */
  const int16_t *writer_table; /* vocab * width, Q12: input embedding and writer rows */
  const int32_t *roots_q12;    /* 16 * 8: the Cl(0,6) orbit roots times 4096 */
  const int8_t *icosian;       /* 120 * 4 * 2: (a + b phi)/2 coefficient pairs */
  const uint64_t *keep_q31;    /* 16: isqrt(2^62 - 2^(60 - 2 i)) */
  uint32_t raw_gates;          /* nonzero: Hamilton gates served as unit quaternions */
  uint32_t raw_transition;     /* nonzero: transition served as lambda * unit quaternion */
} uor_fbs_model;

/* Extensions beyond the reference's loader limits (no counterpart in the reference). Every
 * zero/NULL field selects the reference's own rule, so `ext == NULL` is the reference model:
 *   window 0     -> 3 prior drive rows (CONVOLUTION_WIDTH 4, session.rs:85)
 *   drawers 0    -> 256 root-pair cells a*16+b scored by the query's first/last 8-blocks
 *   probes 0     -> model.kept cells kept per position
 *   keys NULL    -> key of drawer c = (roots_q12[c >> 4], roots_q12[c & 15]) (drawers 256)
 *   offsets NULL -> drawer of token t = t mod drawers, members ascending
 *   table_i8 NULL-> the i16 writer table; else row values are (code << table_shift) at Q12
 *   head 0       -> native writer; 1 -> whole-table L1 nearest (session.rs:4418-4445)     */
/* The Hamming reads of a `uor-r4.lut-stack/6` stack (the `hamming` record, StackHamming,
 * stack/format.rs:229-292, and one HammingReadImage per read, stack/hamming.rs:25-40, from the
 * sections `hamming.d{depth}.*`), served inside the step as the reference session serves them
 * (ServedHamming::stream after `depth` layers and ServedHamming::readout on the final norm's
 * output, session.rs:4252-4276, 4296-4320; hamming.rs:1551-1960), with the readout read's place
 * read when the record carries one (`hamming.place`, below). */
#define UOR_FBS_COPY_ARTIFACT 0xffffffffu /* serve the artifact's own copy rule */
#define UOR_FBS_COPY_MEAN 0u              /* CopyRule::Mean (hamming.rs:180-201) */
#define UOR_FBS_COPY_LATEST_EXACT 1u
#define UOR_FBS_COPY_LATEST_NEAREST 2u
#define UOR_FBS_COPY_LONGEST_EXACT 3u
#define UOR_FBS_COPY_LONGEST_AFTER_OPENING 4u

typedef struct uor_fbs_hamming_read {
  uint32_t depth;                /* after this many layers; the layer count: the readout read */
  uint32_t carry_rows;           /* the readout read's question carry reach h (0: none) */
  const int32_t *query_rotation; /* width raw values at 2^-24: the type heads' query */
  const int32_t *key_rotation;   /* width: the copy heads' and the type heads' keys */
  const int32_t *value_rotation; /* width: the type heads' payloads */
  const int32_t *margin;         /* heads margins in bits at Q16, each positive */
  const int32_t *weight;         /* 2 * width at 2^-24: the copy weights w_c, then w_y */
  const int16_t *ask;            /* vocab * width Q12 question table; NULL: the read does not ask */
  const int32_t *carry;          /* vocab carry gains at Q16 (with carry_rows), else NULL */
} uor_fbs_hamming_read;

/* The readout read's place read (the record's `place` marks, PlaceMarks, fbs_snapshot.rs:2725-
 * 2762, and the `hamming.d{depth}.place` class table, PlaceImage, :2772-2795): the ids that frame
 * a conversation and each vocabulary entry's class. The readout read's ask heads then find a
 * place in the session's finished user turns and bring nothing back themselves; a reply row the
 * register opens reads the token at the place in place of the copy heads' mean
 * (ServedHamming::place_advance and readout, hamming.rs:1510-1533, 1625-1634, 1883-1913;
 * PlaceState::advance, fbs_snapshot.rs:2893-3090). The caller's asks table (set_place_asks,
 * hamming.rs:1639) is not served. Each marker list holds at most UOR_FBS_PLACE_MARK_MAX ids. */
#define UOR_FBS_PLACE_STOP 1
#define UOR_FBS_PLACE_ARM 2
#define UOR_FBS_PLACE_OPEN 4
#define UOR_FBS_PLACE_MARK_MAX 16u
typedef struct uor_fbs_place {
  uint32_t bos, eos;               /* the document's start and end marks */
  uint32_t sep_len, system_len, user_len, assistant_len;
  const uint32_t *sep;             /* the turn separator, sep_len >= 1 ids */
  const uint32_t *system;          /* the role markers (system may be empty) */
  const uint32_t *user;
  const uint32_t *assistant;
  const int16_t *class_table;      /* vocab classes: STOP | ARM | OPEN bits */
} uor_fbs_place;

typedef struct uor_fbs_hamming {
  uint32_t heads;               /* per read: heads/2 copy heads, then the type (or ask) heads */
  uint32_t kept;                /* earlier positions each head keeps, >= 1 */
  uint32_t copy_key;            /* tokens a copy head's key names: 1 or 2 */
  uint32_t copy_latest;         /* nonzero: the copy heads read their latest exact match */
  const uint32_t *copy_keys;    /* heads/2 entries of 1 or 2 when they differ, else NULL */
  uint32_t copy_longest;        /* nonzero: the longest rule after the reply marker below */
  uint32_t marker[2];           /* the two ids before a reply's first token (copy_longest) */
  uint32_t rule;                /* the copy rule served: UOR_FBS_COPY_ARTIFACT or a rule */
  uint32_t read_count;
  const uor_fbs_hamming_read *reads; /* read_count reads, depths strictly increasing */
  const uor_fbs_place *place;        /* NULL: no place read */
} uor_fbs_hamming;

typedef struct uor_fbs_ext {
  uint32_t window;                 /* W prior rows of the causal window, 1..64 */
  uint32_t drawers;                /* D drawers, 1..4096 */
  uint32_t probes;                 /* P drawers kept per position, 1..min(D, 64) */
  uint32_t head;                   /* 0 writer, 1 nearest */
  const int16_t *const *wide_taps; /* per layer (W+1)*width grid codes [tap][channel] */
  const int32_t *drawer_keys;      /* D * 16 Q12 values: first-block key, last-block key */
  const uint32_t *drawer_offsets;  /* D + 1 CSR offsets into drawer_members */
  const uint32_t *drawer_members;  /* vocab token ids, each drawer's ascending */
  const int8_t *table_i8;          /* vocab * width codes */
  uint32_t table_shift;            /* 0..8 */
  uint32_t reserved;
  const uor_fbs_hamming *hamming;  /* NULL: no Hamming reads (every schema but lut-stack/6) */
} uor_fbs_ext;

typedef struct uor_fbs_handle uor_fbs_handle;

/* ABI checks, as fbs_host_sizeof_model / fbs_host_sizeof_layer (host_kernel.cpp:8-9). */
uint32_t uor_fbs_abi_version(void);
int64_t uor_fbs_sizeof_model(void);
int64_t uor_fbs_sizeof_layer(void);
int64_t uor_fbs_sizeof_ext(void);

/* The message of this thread's last failed call ("" if none). */
const char *uor_fbs_last_error(void);

/* Validate the model (the FBS rules of StackShape::validate, format.rs:616-752, and the route
 * and grid-code checks of fbs_model, session.rs:640-735), upload it to HIP device `device`
 * and prepare its lane tables. Replaces DeviceEvaluator::new (device.rs:93-170). */
int uor_fbs_model_create(const uor_fbs_model *model, const uor_fbs_ext *ext, int32_t device,
                         uor_fbs_handle **out);
void uor_fbs_model_destroy(uor_fbs_handle *handle);

/* Per-sequence state sizes for export/import: `state_words` int64 recurrence values
 * ([layer][width], exponent -32) and `history_words` int32 drive values
 * ([layer][window][width], row 0 the newest), as `LayerState::Recurrence` (session.rs:1850). */
uint64_t uor_fbs_state_words(const uor_fbs_handle *handle);
uint64_t uor_fbs_history_words(const uor_fbs_handle *handle);

/* Wavefronts per sequence of the kernels a run of n sequences launches: 2 (paired blocks, at
 * most one block per SIMD, each stepping its share of the sequences) unless
 * UOR_FBS_BLOCK_WAVES=1 was set at model creation or the model's paired LDS does not fit, then
 * 1 (one wavefront per sequence). The same for every n today; n is kept for a policy that
 * depends on the batch. No counterpart in the reference (its CPU decoder has no launch shape):
 * for profilers and tests. */
uint32_t uor_fbs_block_waves(const uor_fbs_handle *handle, uint32_t n);

/* Teacher-forced sequences from fresh sessions: every position's chosen token, kept drawers
 * (best first) and Q12 query. Same contract as fbs_host_sequences (host_kernel.cpp:16-29)
 * and fbs_eval_sequences (evaluator.cu:8-19): outputs S*len, S*len*probes, S*len*width.
 * Host buffers. Returns the first nonzero sequence status. */
int uor_fbs_sequences(uor_fbs_handle *handle, const uint32_t *tokens, uint32_t sequences,
                      uint32_t len, uint32_t *out_tokens, uint32_t *out_kept, int32_t *out_query);
/* The same on device buffers; `status` holds one int32 per sequence. */
int uor_fbs_sequences_async(uor_fbs_handle *handle, const uint32_t *tokens, uint32_t sequences,
                            uint32_t len, uint32_t *out_tokens, uint32_t *out_kept,
                            int32_t *out_query, int32_t *status, void *stream);

/* The snap trace (fbs_core.h:488-501, claude-134): uor_fbs_sequences with every position's trace,
 * `uor_fbs_trace_stride(handle)` bytes a position: per layer, the transition's chosen icosian root
 * per lane (width/4 bytes), the output gate's per lane, then the feed-forward gate's per 4 MLP
 * channels (mlp/4 bytes); 255 where a site is served unsnapped (raw gates or transition) or its
 * raw quaternion is zero. Same contract as fbs_trace_sequences (evaluator.cu:21-33) and
 * fbs_host_trace_sequences (host_kernel.cpp:31-49); the other outputs are those of
 * uor_fbs_sequences. Runs the one-wavefront kernels. Host buffers; `_async`: device buffers and
 * one int32 status per sequence. */
uint64_t uor_fbs_trace_stride(const uor_fbs_handle *handle);
int uor_fbs_trace_sequences(uor_fbs_handle *handle, const uint32_t *tokens, uint32_t sequences,
                            uint32_t len, uint32_t *out_tokens, uint32_t *out_kept,
                            int32_t *out_query, uint8_t *out_trace);
int uor_fbs_trace_sequences_async(uor_fbs_handle *handle, const uint32_t *tokens,
                                  uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                                  uint32_t *out_kept, int32_t *out_query, uint8_t *out_trace,
                                  int32_t *status, void *stream);

/* Batched greedy decode, the fbs-toks run (fbs-toks.rs:1513-1533) for many sequences: each
 * sequence steps its `prompt_len` prompt tokens, then `gen` more, each fed the previous
 * choice. `out_reply` gets gen+1 tokens per sequence: the prompt's last choice, then every
 * generated choice. Optional state: `in_*` resume a sequence (NULL = fresh session at
 * position 0), `out_*` export it after the last step (NULL = not wanted). Host buffers. */
int uor_fbs_decode(uor_fbs_handle *handle, const uint32_t *prompts, uint32_t sequences,
                   uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                   const int64_t *in_state, const int32_t *in_history,
                   const uint32_t *in_position, int64_t *out_state, int32_t *out_history,
                   uint32_t *out_position);
/* The same on device buffers; `status` holds one int32 per sequence. */
int uor_fbs_decode_async(uor_fbs_handle *handle, const uint32_t *prompts, uint32_t sequences,
                         uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                         const int64_t *in_state, const int32_t *in_history,
                         const uint32_t *in_position, int64_t *out_state,
                         int32_t *out_history, uint32_t *out_position, int32_t *status,
                         void *stream);

/* Part clocks, after measure_fbs_step_parts (session.rs:4721-4779, stack_step_fbs_timed :4456)
 * and `fbs-toks --parts`: uor_fbs_decode_async (gen > 0, a model the paired kernels serve) on an
 * instrumented copy of its kernel that reads the shader clock between the step's phases.
 * Outputs, state and statuses are the decode's. `out_parts` (device) gets per sequence
 * 2 * uor_fbs_part_count() + 2 uint64 words: for wave 0 (the recurrence chain) and then wave 1
 * (the window ring) the cycles spent in each part, summed over the sequence's steps and layers
 * (uor_fbs_part_name: the reference's parts of a step, the barriers between the two waves as
 * parts of their own), then the steps run, then the sequence's time in ticks of the 100 MHz
 * real-time counter. The clock reads cost time of their own: compare a plain decode's. */
uint32_t uor_fbs_part_count(void);
const char *uor_fbs_part_name(uint32_t part);
int uor_fbs_decode_parts_async(uor_fbs_handle *handle, const uint32_t *prompts,
                               uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                               uint32_t *out_reply, const int64_t *in_state,
                               const int32_t *in_history, const uint32_t *in_position,
                               int64_t *out_state, int32_t *out_history, uint32_t *out_position,
                               int32_t *status, uint64_t *out_parts, void *stream);

/* uor_fbs_decode_async without allocating: no hipMalloc, hipFree or allocating library call,
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops, hosts
 * that forbid allocation on their path). No counterpart in the reference. Same arguments,
 * outputs and statuses as uor_fbs_decode_async; the caller still passes every input and output
 * buffer. The window rings, window sums and (paired blocks) recurrence states live in a device array of
 * UOR_FBS_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the process ends:
 * the launch uses as many resident blocks as that holds (sequences loop within them; results do
 * not depend on the grid), and a model whose one sequence needs more is refused with
 * UOR_FBS_ERR_UNSUPPORTED. Every call on a GPU shares that GPU's array, and nothing in it needs
 * to start at zero: calls that overlap on one GPU (other streams, other threads, other handles)
 * race on it and must be serialised by the caller. */
#define UOR_FBS_NOALLOC_SCRATCH_BYTES (128u << 20)
int uor_fbs_decode_noalloc_async(uor_fbs_handle *handle, const uint32_t *prompts,
                                 uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                                 uint32_t *out_reply, const int64_t *in_state,
                                 const int32_t *in_history, const uint32_t *in_position,
                                 int64_t *out_state, int32_t *out_history,
                                 uint32_t *out_position, int32_t *status, void *stream);

/* Serving sessions held in caller-owned device arrays, one slot per session: `state`
 * [capacity][state_words] int64, `history` [capacity][history_words] int32 and `position`
 * [capacity] uint32, updated in place. A slot's history is its window ring, [layer][window]
 * [width] with row p mod window holding the drive of position p (exported row r, the drive
 * r + 1 positions back, is ring row (position - 1 - r) mod window), so no launch copies it.
 * Sequence i of the call is the session in slot
 * slots[i] < capacity (distinct within a call); it takes prompts[i*prompt_len ..] from its
 * slot's state, then `gen` greedy steps, as uor_fbs_decode_async: out_reply gets gen+1 tokens
 * per sequence. The serving loop of IntegerStackSession for a batch of sessions:
 * serve_step / step_native (session.rs:3356-3440, the browser's wasm_step,
 * wasm_serve.rs:140-152) with prompt_len 1 and gen 0, read_step (session.rs:3392) for all
 * prompt tokens but the last, which one call folds into prompt_len. Optional out_kept [n][P]
 * and out_query [n][width] receive the last step's kept drawers and Q12 query (step_native's
 * NativeStep, session.rs:484-493). A sequence refused with status 1 or 2 leaves its slot
 * holding the tokens stepped before the refused one, as the reference's session after its
 * error; status 3 (slots[i] >= capacity): nothing read or written. Device buffers. */
int uor_fbs_decode_slots_async(uor_fbs_handle *handle, const uint32_t *slots, uint32_t sequences,
                               uint32_t capacity, const uint32_t *prompts, uint32_t prompt_len,
                               uint32_t gen, uint32_t *out_reply, int64_t *state,
                               int32_t *history, uint32_t *position, uint32_t *out_kept,
                               int32_t *out_query, int32_t *status, void *stream);

/* ---- Hamming models (an ext with `hamming`): the session's token stream and payloads.
 * A Hamming read at row t reads the session's tokens x_0..x_t (IntegerStackSession::tokens) and,
 * for a read whose type heads bring back payloads, the payload it kept at every earlier row
 * (`hamming_payloads`, session.rs:1755-1759, 2232; ServedHamming::payload_caches,
 * hamming.rs:1680-1685), so a resumed session needs both besides its state. `stream_words`:
 * tokens a session keeps, the context (0 without Hamming reads); `payload_words`: int64 payload
 * values, [typed read][context][width] (0 without such reads). The other decode entry points
 * decode a Hamming model from fresh sessions and refuse `in_position` (resuming) on one with
 * UOR_FBS_ERR_UNSUPPORTED, as the reference refuses a saved session without its payloads
 * (session.rs:2885-2910); the slot and allocation-free entry points refuse Hamming models. */
uint64_t uor_fbs_stream_words(const uor_fbs_handle *handle);
uint64_t uor_fbs_payload_words(const uor_fbs_handle *handle);

/* uor_fbs_decode_async with the stream: `in_stream` [n][stream_words] (entries below the
 * position read) and `in_payloads` [n][payload_words] (rows below the position read) resume,
 * both required with `in_position` on a Hamming model; `out_stream` and `out_payloads` receive
 * them after the last step (rows at and past the position are left as found). `out_payloads`
 * may equal `in_payloads` (updated in place). On a model without Hamming reads the stream
 * arguments are ignored. Device buffers. */
int uor_fbs_decode_stream_async(uor_fbs_handle *handle, const uint32_t *prompts,
                                uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                                uint32_t *out_reply, const int64_t *in_state,
                                const int32_t *in_history, const uint32_t *in_position,
                                const uint32_t *in_stream, const int64_t *in_payloads,
                                int64_t *out_state, int32_t *out_history, uint32_t *out_position,
                                uint32_t *out_stream, int64_t *out_payloads, int32_t *status,
                                void *stream);
/* The same on host buffers. */
int uor_fbs_decode_stream(uor_fbs_handle *handle, const uint32_t *prompts, uint32_t sequences,
                          uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                          const int64_t *in_state, const int32_t *in_history,
                          const uint32_t *in_position, const uint32_t *in_stream,
                          const int64_t *in_payloads, int64_t *out_state, int32_t *out_history,
                          uint32_t *out_position, uint32_t *out_stream, int64_t *out_payloads);

/* ---- The serving loop with per-slot caches and the context slide.
 * uor_fbs_decode_slots_async's slots, plus two things a serving loop keeps between launches:
 * - `cache`: capacity * uor_fbs_slot_cache_bytes(handle) device bytes, zero-filled by the caller
 *   before its first use (a zero entry holds nothing). Each slot's entry keeps the window sums
 *   its last launch formed for the slot's next step, tagged with the position they hold for, so
 *   a launch that starts there does not sum the window again, and the writer's memory of its
 *   last query, which depends on the model alone. The sums are also tagged with a fingerprint of
 *   the slot's state as that launch left it: a launch that finds another state in the slot (a
 *   caller restored a session there at the same position) sums the window afresh. A caller
 *   that rewrites a slot's history alone, leaving its state and position, zeroes the slot's entry
 *   first (its first 4 bytes suffice); zeroing it on every write of a slot is always right. An
 *   entry belongs to this handle's model. NULL: no cache (as uor_fbs_decode_slots_async).
 * - `slide`: capacity bytes, nonzero for a slot whose session continues past a full context
 *   (IntegerStackSession::set_context_slide, session.rs:2391-2402, :4143-4151: the step does not
 *   refuse at the context, and the position keeps counting; nothing else in the step reads it
 *   beyond the window ring's slot). NULL: no slot slides. The reference refuses the slide for a
 *   model with Hamming reads or a turn memory; this entry refuses Hamming models and the caller
 *   (uor_fbs/session.py) the rest.
 * - `out_trace`: the snap trace of every step, sequences * (prompt_len + gen) *
 *   uor_fbs_trace_stride(handle) bytes, laid out as uor_fbs_trace_sequences' (per step, per
 *   layer: transition roots per lane, output gate roots, feed-forward gate roots). A session's
 *   opt-in snap trace (IntegerStackSession::enable_snap_trace, session.rs:2570-2620) records the
 *   transition roots (stack_lanes, session.rs:5097-5150); a zero raw quaternion, 255 here,
 *   selects root 0 there. Rows of steps a slot did not run are left as they were. NULL: no
 *   trace; otherwise the launch runs the one-wavefront kernels.
 * A launch of one token a session (prompt_len 1, gen 0) on a model with keyed drawers of skewed
 * sizes (the largest more than twice the mean) queues three kernels on
 * `stream`: the step up to the writer's drawer selection, a scan of every kept drawer's members
 * laid out by drawer over all the launch's sessions, and the hand-out of each session's token
 * (results those of the writer inside the step; the environment variable UOR_FBS_SERVE_SCAN=fused
 * or =drawer at model creation keeps the writer in the step or takes the scan whatever the sizes).
 * Its job buffers are the handle's, allocated on the first such launch of that many sessions.
 * No counterpart beyond those: the reference's sessions keep their window sums implicitly (a CPU
 * session steps one token at a time). Device buffers. */
uint64_t uor_fbs_slot_cache_bytes(const uor_fbs_handle *handle);
int uor_fbs_serve_slots_async(uor_fbs_handle *handle, const uint32_t *slots, uint32_t sequences,
                              uint32_t capacity, const uint32_t *prompts, uint32_t prompt_len,
                              uint32_t gen, uint32_t *out_reply, int64_t *state, int32_t *history,
                              uint32_t *position, void *cache, const uint8_t *slide,
                              uint32_t *out_kept, int32_t *out_query, uint8_t *out_trace,
                              int32_t *status, void *stream);

/* The serving loop for a model with Hamming reads (lut-stack/6): IntegerStackSession's
 * serve_step/step_native (session.rs:3356-3440) on sessions whose reads look back over their own
 * tokens and payloads (session.rs:4149-4152, 4252-4276, 4296-4320). uor_fbs_serve_slots_async's
 * slots, plus each slot's token stream and payload caches, updated in place:
 * - `stream`: capacity * uor_fbs_stream_words(handle) u32, the slot's tokens x_0..x_{position-1}
 *   (entries at and past the position are ignored and rewritten);
 * - `payloads`: capacity * uor_fbs_payload_words(handle) i64, each typed read's payload of every
 *   position, [typed read][context][width] (NULL for a model with none).
 * A fresh slot has position 0 (its stream and payloads are then not read). `cache` as
 * uor_fbs_serve_slots_async's (the writer's memory; these kernels keep no window sums there).
 * No context slide (the reference refuses it for Hamming reads) and no snap trace. A model
 * without Hamming reads is served as by uor_fbs_serve_slots_async (stream and payloads unused).
 * Device buffers. */
int uor_fbs_serve_slots_stream_async(uor_fbs_handle *handle, const uint32_t *slots,
                                     uint32_t sequences, uint32_t capacity,
                                     const uint32_t *prompts, uint32_t prompt_len, uint32_t gen,
                                     uint32_t *out_reply, int64_t *state, int32_t *history,
                                     uint32_t *position, uint32_t *stream, int64_t *payloads,
                                     void *cache, uint32_t *out_kept, int32_t *out_query,
                                     int32_t *status, void *hip_stream);

/* The Hamming trace and Q5's decision trace with the forced replay, teacher-forced from fresh
 * sessions: set_hamming_trace / take_hamming_trace (session.rs:2361-2370, HammingStepRead
 * hamming.rs:1378-1395, `record` :1787-1814) and set_decision_trace / take_decision_trace
 * (session.rs:2438-2515, DecisionStep fbs_snapshot.rs:643-703, ForcedBucket / ForcedCode
 * :754-797, BucketTrace::decide session.rs:2192-2215), as `fbs-toks --forced --decision-trace`
 * runs windows. Every position of `sequences` rows of `len` tokens gets a record of
 * uor_fbs_decision_stride(handle, decisions) bytes in `out_trace`:
 * - with `decisions`: each layer's rate scores clamp(decay + offset, 0, 2^16) (i32 [layer][lane],
 *   lane = width / 4) and the entries used (u8 [layer][lane]), padded to 8 bytes;
 * - then each Hamming read in depth order, each head it serves (the copy heads, then the type
 *   heads where the read serves them): the query code (u64), the key code at the row (u64, 0 at
 *   row 0), the kept count (u32) and the kept positions (u32 each, `kept` of them; the nearest by
 *   distance then position, or the rule's one position), padded to 8 bytes.
 * The forced replay (NULL: nothing forced): `force_buckets` [sequence][step][layer][lane] (255:
 * the score's own entry, else 0..15; needs `decisions`), `force_codes` [sequence][step][read]
 * [head][2] (the query, the key) with `force_mask` [sequence][step][read][head] (bit 0: the
 * query is forced at that step, bit 1: the key, which every later row reads for that candidate).
 * Refused as the reference refuses them: the decision trace on a snapped artifact or one whose
 * head is not the nearest; a forced bucket entry past 15; a forced code on a model without
 * Hamming reads, on a head its read does not serve, a key at step 0, or with a place read.
 * `out_tokens` and `out_query` (NULL: not wanted) as uor_fbs_sequences'. Host buffers. */
uint64_t uor_fbs_decision_stride(const uor_fbs_handle *handle, uint32_t decisions);
int uor_fbs_decision_sequences(uor_fbs_handle *handle, const uint32_t *tokens, uint32_t sequences,
                               uint32_t len, uint32_t decisions, const uint8_t *force_buckets,
                               const uint64_t *force_codes, const uint8_t *force_mask,
                               uint32_t *out_tokens, int32_t *out_query, uint8_t *out_trace);

/* Teacher-forced next-token scoring: for each row of `len` tokens, position t's choice is
 * compared with row[t+1] (t < len-1); `out_matches` gets the total count of equal pairs.
 * `out_argmin` (nullable) gets every position's choice, rows*len. Host buffers. */
int uor_fbs_score(uor_fbs_handle *handle, const uint32_t *rows, uint64_t n_rows, uint32_t len,
                  uint32_t *out_argmin, uint64_t *out_matches);
/* The same on device buffers: `matches` is one uint64 the kernel adds into (the caller
 * zeroes it), `status` one int32 per row. */
int uor_fbs_score_async(uor_fbs_handle *handle, const uint32_t *rows, uint64_t n_rows,
                        uint32_t len, uint32_t *out_argmin, uint64_t *matches,
                        int32_t *status, void *stream);

/* ---- The 256-cell CSR drawer index (the reference's uor_inverted_file API,
 * projects/uor-cuda-inverted-file/include/uor_inverted_file.hpp:41-50, which its CUDA
 * kernels uor_if_build/update/probe/full_scan, src/kernels.cu:139-243, serve; the discrete
 * crate's bucket build/update entries, crates/uor-r4-discrete/src/bucket_source.rs:1-12).
 *
 * table [count][width] int32 (16-byte aligned, width a multiple of 4 in 16..MAX_WIDTH; the
 * reference's Token is width 32: four 8-value blocks), roots [16][8] int32 (the reference's
 * codebook, src/codebook.cpp:5-14). A token's cell is r0*16 + r1 when its first 8 values equal
 * root r0 and its last 8 equal root r1 (first match), else ABSENT (0xffffffff). The index:
 * offsets [257], members [count] (offsets[256] of them used: each cell's tokens ascending),
 * cells [count], absent_count [1]. All device buffers; every call is asynchronous on `stream`
 * and writes one int32 `status` word, a uor_inverted_file::Status (hpp:29-37): 0 Ok,
 * 1 InvalidArgument, 2 NonRootBlock, 3 CsrInvariant. The return value is UOR_FBS_ERR_ARGUMENT
 * (nothing launched) for null pointers, count 0 or above MAX_TOKENS, a bad width or
 * alignment, k outside 1..16; UOR_FBS_ERR_DEVICE for a launch error. `workspace` holds
 * uor_fbs_index_workspace_bytes(count) bytes of device memory, needs no initialisation and
 * serialises the calls that share it (one stream). */
#define UOR_FBS_INDEX_ABSENT 0xffffffffu
#define UOR_FBS_INDEX_MAX_WIDTH 256u
#define UOR_FBS_INDEX_MAX_TOKENS (1u << 30)

uint64_t uor_fbs_index_workspace_bytes(uint32_t count);
/* build (inverted_file.cpp:112-138, 173-175): status 2 when a token has no cell and
 * allow_absent is 0 (the buffers then hold no valid index). */
int uor_fbs_index_build_async(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, uint32_t allow_absent, uint32_t *offsets,
                              uint32_t *members, uint32_t *cells, uint32_t *absent_count,
                              void *workspace, int32_t *status, void *stream);
/* update (inverted_file.cpp:182-236): token `moved`'s row changed; the index is checked first
 * (status 3, unchanged), then the token moves to its new cell (status 2 and unchanged when
 * the new row has no cell), and the whole index is validated against the table after a
 * move, as the reference returns validate(table, index). */
int uor_fbs_index_update_async(const int32_t *table, uint32_t count, uint32_t width,
                               const int32_t *roots, uint32_t moved, uint32_t *offsets,
                               uint32_t *members, uint32_t *cells, uint32_t *absent_count,
                               void *workspace, int32_t *status, void *stream);
/* remove_token (inverted_file.cpp:238-249): token `moved` leaves its cell for ABSENT. A stored
 * cell above 255, which the reference would index out of range, is refused with status 3. */
int uor_fbs_index_remove_async(uint32_t count, uint32_t moved, uint32_t *offsets,
                               uint32_t *members, uint32_t *cells, uint32_t *absent_count,
                               void *workspace, int32_t *status, void *stream);
/* validate (inverted_file.cpp:164-176) with a table, validate_structure (:141-162) when
 * `table` is null (roots and width then unused). */
int uor_fbs_index_validate_async(const int32_t *table, uint32_t count, uint32_t width,
                                 const int32_t *roots, const uint32_t *offsets,
                                 const uint32_t *members, const uint32_t *cells,
                                 const uint32_t *absent_count, void *workspace, int32_t *status,
                                 void *stream);
/* probe (inverted_file.cpp:250-258) for `rows` queries [rows][width]: admitted [rows][16]
 * (the k nearest non-empty cells by endpoint L1, ties to the lower cell, ABSENT-padded),
 * top8 [rows][8] (the admitted cells' members by row L1, ties to the lower token),
 * predictions [rows] = top8[0], status [rows]: 0, 1 when nothing was admitted, 3 when the
 * index pointed outside the table. The index is not validated (validate once per change; the
 * reference's probe validates on every call). */
int uor_fbs_index_probe_async(const int32_t *table, uint32_t count, uint32_t width,
                              const int32_t *roots, const int32_t *queries, uint32_t rows,
                              uint32_t k, const uint32_t *offsets, const uint32_t *members,
                              uint32_t *predictions, uint32_t *admitted, uint32_t *top8,
                              int32_t *status, void *stream);
/* full_scan (inverted_file.cpp:260-270): cells admitted from `offsets` of an index of the
 * same table built with allow_absent 1, then every token of the table in an admitted cell
 * ranked; outputs as the probe's. */
int uor_fbs_index_full_scan_async(const int32_t *table, uint32_t count, uint32_t width,
                                  const int32_t *roots, const int32_t *queries, uint32_t rows,
                                  uint32_t k, const uint32_t *offsets, uint32_t *predictions,
                                  uint32_t *admitted, uint32_t *top8, int32_t *status,
                                  void *stream);

#ifdef __cplusplus
}
#endif

#endif /* UOR_FBS_H */
