// fbs_api.cpp - the C ABI of include/uor_fbs.h: model validation and upload, the per-lane
// gather programs, device work buffers, and the sequences / decode / score entry points.
//
// Replaces the reference's GPU evaluator host side (docs/labs/d11-exporter-float-trunk/
// instrument/src/device.rs:93-302 `DeviceEvaluator::{new, run}`) and its FFI twin entry
// (host_kernel.cpp:16-29): the caller passes the parsed model image (`fbs_model` layout), the
// library validates it as the reference's loader would (session.rs:640-735 `fbs_model`,
// format.rs:616-752 `StackShape::validate`, kernels.rs:116-120 `grid_valid`) and keeps device
// copies laid out for the kernels (fbs_device.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/uor_fbs.h"
#include "fbs_device.h"
#include "fbs_int.h"

namespace fbs {
// The kernels: fbs_{prefill,decode,rows}{,_pair,_ham}.hip (phase x family).
#define FBS_LAUNCHER(NAME)                                                                     \
  hipError_t launch_##NAME(const DevModel &M, const RunArgs &A, uint32_t grid, size_t lds,    \
                           hipStream_t stream);
FBS_LAUNCHER(fbs_prefill)
FBS_LAUNCHER(fbs_prefill_pair)
FBS_LAUNCHER(fbs_prefill_ham)
FBS_LAUNCHER(fbs_decode)
FBS_LAUNCHER(fbs_decode_pair)
FBS_LAUNCHER(fbs_decode_ham)
FBS_LAUNCHER(fbs_rows)
FBS_LAUNCHER(fbs_rows_pair)
FBS_LAUNCHER(fbs_rows_ham)
FBS_LAUNCHER(fbs_prefill_8)
FBS_LAUNCHER(fbs_prefill_pair8)
FBS_LAUNCHER(fbs_decode_8)
FBS_LAUNCHER(fbs_decode_pair8)
FBS_LAUNCHER(fbs_rows_8)
FBS_LAUNCHER(fbs_rows_pair8)
FBS_LAUNCHER(fbs_decode_pair_clk)
FBS_LAUNCHER(fbs_rows_dt)
FBS_LAUNCHER(fbs_prefill_pair_ham)
FBS_LAUNCHER(fbs_decode_pair_ham)
FBS_LAUNCHER(fbs_rows_pair_ham)
#undef FBS_LAUNCHER
// The deferred writer's drawer-major scan and hand-out (fbs_serve.hip).
hipError_t launch_fbs_serve_scan(const DevModel &M, const ServeScan &J, uint32_t blocks,
                                 hipStream_t stream);
hipError_t launch_fbs_fill_u32(uint32_t *p, uint64_t n, uint32_t v, hipStream_t stream);
}

using namespace fbs;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(UOR_FBS_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

bool grid_valid(int16_t code) {  // kernels.rs:116-120
  uint32_t field = (uint32_t)(code < 0 ? -(int32_t)code : code) >> 4;
  return code == 0 || (field >= 1 && field <= 127);
}

}  // namespace

struct uor_fbs_handle {
  int device = 0;
  DevModel M{};
  std::vector<bool> ham_read_typed;  // per Hamming read: its type heads are served
  std::vector<void *> allocs;
  size_t lds_bytes = 0;
  uint32_t max_grid = 0;
  // Paired blocks (two wavefronts per sequence, two waves on every SIMD) run every launch unless
  // the environment asks for one wave or their LDS does not fit; their grid is at most one
  // block per SIMD, each block stepping its share of the batch's sequences in turn, so that
  // every block is resident from the start and each SIMD keeps wave 0 of one block beside
  // wave 1 of another.
  bool pair = false;
  size_t pair_lds = 0;
  uint32_t pair_grid = 0;
  uint32_t cus = 0;      // the device's compute units
  size_t lds_limit = 0;  // LDS bytes a block may take
  int32_t *ring = nullptr;
  int64_t *hist = nullptr;
  size_t ring_blocks = 0;
  // Hamming models: the type heads' payload caches of sequences whose caller takes none out.
  int64_t *pay = nullptr;
  size_t pay_blocks = 0;
  // This device's copy of the allocation-free decode's scratch array (null if its address could
  // not be read; that entry point then refuses).
  unsigned char *scratch = nullptr;
  // The deferred writer of one-token serving launches (fbs_serve.hip): the drawers' chunks of 64
  // members (all, and the most of one drawer), and the job buffers for `jobs_cap` sequences
  // (grown, never shrunk). Taken where the drawers' sizes are skewed (the largest more than
  // twice the mean), where a launch with the writer in the step waits for its sessions with the
  // largest drawers; UOR_FBS_SERVE_SCAN=drawer or =fused at model creation takes or refuses it
  // whatever the sizes.
  bool serve_drawer_major = true;
  uint32_t serve_nchunks = 0, serve_max_chunks = 0;
  uint32_t jobs_cap = 0, item_cap = 0;
  uint32_t *job_query = nullptr, *job_flag = nullptr, *drawer_count = nullptr,
           *drawer_list = nullptr, *item_count = nullptr;
  uint4 *items = nullptr;
  unsigned long long *job_best = nullptr;

  ~uor_fbs_handle() {
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    for (void *p : allocs) (void)hipFree(p);
    if (ring) (void)hipFree(ring);
    if (hist) (void)hipFree(hist);
    if (pay) (void)hipFree(pay);
    free_jobs();
    (void)hipSetDevice(prev);
  }

  void free_jobs() {
    for (void *p : {(void *)job_query, (void *)job_flag, (void *)drawer_count, (void *)drawer_list,
                    (void *)job_best, (void *)items, (void *)item_count})
      if (p) (void)hipFree(p);
    job_query = job_flag = drawer_count = drawer_list = item_count = nullptr;
    items = nullptr;
    job_best = nullptr;
    jobs_cap = item_cap = 0;
  }

  // The deferred writer's job buffers for n sequences: flags and drawer counts start at zero
  // (a fill kernel on `stream`; the hand-out kernel clears what a launch set).
  int ensure_jobs(uint32_t n, hipStream_t stream) {
    if (n <= jobs_cap) return 0;
    free_jobs();
    const size_t words = M.d / 2;
    // Items: a chunk's slices are at most its drawer's sessions / 16 + 1, and the sessions of all
    // drawers together n P.
    const uint64_t cap = serve_nchunks + (uint64_t)serve_max_chunks *
                                             (((uint64_t)n * M.P + kServeSessions - 1) / kServeSessions);
    if (cap > 0xffffffffull) return fail(UOR_FBS_ERR_UNSUPPORTED, "too many serving sessions");
    hipError_t e = hipMalloc((void **)&job_query, (size_t)n * words * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&job_flag, (size_t)n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&job_best, (size_t)n * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc((void **)&drawer_count, (size_t)M.D * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&drawer_list, (size_t)M.D * n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&items, (size_t)cap * sizeof(uint4));
    if (e == hipSuccess) e = hipMalloc((void **)&item_count, sizeof(uint32_t));
    if (e != hipSuccess) {
      free_jobs();
      return hip_fail(e, "hipMalloc(serving jobs)");
    }
    if ((e = launch_fbs_fill_u32(job_flag, n, 0, stream)) != hipSuccess ||
        (e = launch_fbs_fill_u32(drawer_count, M.D, 0, stream)) != hipSuccess ||
        (e = launch_fbs_fill_u32(item_count, 1, 0, stream)) != hipSuccess) {
      free_jobs();
      return hip_fail(e, "kernel launch");
    }
    jobs_cap = n;
    item_cap = (uint32_t)cap;
    return 0;
  }

  // Payload words (i64) one session keeps: slots x context x d.
  size_t payload_words() const { return (size_t)M.ham.slots * M.context * M.d; }

  int ensure_pay(size_t blocks) {
    if (blocks <= pay_blocks) return 0;
    if (pay) (void)hipFree(pay);
    pay = nullptr;
    pay_blocks = 0;
    hipError_t e = hipMalloc((void **)&pay, blocks * payload_words() * sizeof(int64_t));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(payload caches)");
    pay_blocks = blocks;
    return 0;
  }

  template <class T>
  int upload(const T *src, size_t count, const T **dst) {
    void *p = nullptr;
    size_t bytes = count * sizeof(T);
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    allocs.push_back(p);
    if (bytes) {
      e = hipMemcpy(p, src, bytes, hipMemcpyHostToDevice);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
    }
    *dst = (const T *)p;
    return 0;
  }

  // The window ring and the paired blocks' window sums, then their recurrence states (read by
  // the kernels of two or more quaternions a lane), for `blocks` resident sequences (grown,
  // never shrunk).
  int ensure_ring(size_t blocks) {
    if (blocks <= ring_blocks) return 0;
    if (ring) (void)hipFree(ring);
    if (hist) (void)hipFree(hist);
    ring = nullptr;
    hist = nullptr;
    ring_blocks = 0;
    size_t bytes = blocks * (size_t)M.L * M.W * M.d * sizeof(int32_t);
    hipError_t e = hipMalloc((void **)&ring, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(window ring)");
    e = hipMalloc((void **)&hist, 2 * blocks * (size_t)M.L * M.d * sizeof(int64_t));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(window sums)");
    ring_blocks = blocks;
    return 0;
  }
};

// The allocation-free decode (uor_fbs_decode_noalloc_async) keeps its window rings and window
// sums in this file-scope device array instead of memory from hipMalloc. Every GPU the library
// loads on holds its own copy, at its own address, until the process ends. In host code the
// array's name is not a device address: kernels and copies take the per-device address that
// hipGetSymbolAddress returns (scratch_address), read once per device at model creation.
static __device__ __align__(256) unsigned char scratch[UOR_FBS_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_ptr[kScratchDevices];
bool g_scratch_read[kScratchDevices];

// The scratch array's address on `device`, which must be current; read once per device (a
// failed read is not kept, so a later model creation on the device reads it again).
unsigned char *scratch_address(int device) {
  if (device < 0 || device >= kScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_read[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) {
      g_scratch_ptr[device] = (unsigned char *)p;
      g_scratch_read[device] = true;
    } else {
      (void)hipGetLastError();  // the entry point reports the missing address when called
    }
  }
  return g_scratch_ptr[device];
}

}  // namespace

extern "C" {

uint32_t uor_fbs_abi_version(void) { return UOR_FBS_ABI_VERSION; }
int64_t uor_fbs_sizeof_model(void) { return (int64_t)sizeof(uor_fbs_model); }
int64_t uor_fbs_sizeof_layer(void) { return (int64_t)sizeof(uor_fbs_layer); }
int64_t uor_fbs_sizeof_ext(void) { return (int64_t)sizeof(uor_fbs_ext); }
const char *uor_fbs_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"

namespace {

struct Resolved {
  uint32_t W, D, P, head;
  bool reference_writer;
};

int check_map(const uor_fbs_map &mp, uint32_t in_dim, uint32_t out_dim, const char *name,
              uint32_t layer) {
  if (mp.blocks != out_dim / 8)
    return fail(UOR_FBS_ERR_SHAPE, "l%u.%s: %u blocks, expected %u", layer, name, mp.blocks, out_dim / 8);
  if (!mp.atoms || !mp.codes) return fail(UOR_FBS_ERR_ARGUMENT, "l%u.%s: null table", layer, name);
  for (uint32_t o = 0; o < mp.blocks; o++) {
    if (mp.atoms[o] >= in_dim / 8)
      return fail(UOR_FBS_ERR_SHAPE, "l%u.%s: atom %u outside %u atoms", layer, name,
                  (unsigned)mp.atoms[o], in_dim / 8);
    for (int j = 0; j < 8; j++)
      if (mp.codes[8 * o + j] >= 16)
        return fail(UOR_FBS_ERR_SHAPE, "l%u.%s: code %u is not a signed axis", layer, name,
                    (unsigned)mp.codes[8 * o + j]);
  }
  return 0;
}

int check_codes(const int16_t *codes, size_t n, const char *name, uint32_t layer) {
  if (!codes) return fail(UOR_FBS_ERR_ARGUMENT, "l%u.%s: null table", layer, name);
  for (size_t i = 0; i < n; i++)
    if (!grid_valid(codes[i]))
      return fail(UOR_FBS_ERR_SHAPE, "l%u.%s: %d is not a grid code", layer, name, (int)codes[i]);
  return 0;
}

// The Hamming record and its reads, as the reference's loader refuses them
// (StackHamming::check, format.rs:336-430; hamming_image and AskImage::checked, hamming.rs:58-110,
// 1069-1095; check_payload_cache :1538-1549), and this build's own limits: a head keeps at most
// kMaxHamKept positions and positions fit 24 bits.
int check_hamming(const uor_fbs_model *m, const uor_fbs_hamming &hm) {
  const uint32_t d = m->width, heads = hm.heads;
  if (heads < 2 || heads % 2 || d % heads)
    return fail(UOR_FBS_ERR_SHAPE, "hamming: %u heads: an even count of at least 2 dividing the width", heads);
  const uint32_t hw = d / heads;
  if (hw % 4 || hw > 64)
    return fail(UOR_FBS_ERR_SHAPE, "hamming: heads of %u coordinates: whole 4-lane blocks, at most 64", hw);
  if (hm.copy_key != 1 && hm.copy_key != 2)
    return fail(UOR_FBS_ERR_SHAPE, "hamming: copy key %u names 1 or 2 tokens", hm.copy_key);
  bool any2 = hm.copy_key == 2, all_one = hm.copy_key == 1;
  if (hm.copy_keys) {
    bool differ = false;
    for (uint32_t k = 0; k < heads / 2; k++) {
      const uint32_t key = hm.copy_keys[k];
      if (key != 1 && key != 2) return fail(UOR_FBS_ERR_SHAPE, "hamming: copy key %u names 1 or 2 tokens", key);
      differ |= key != hm.copy_keys[0];
      any2 |= key == 2;
      all_one &= key == 1;
    }
    if (hm.copy_key != 1 || !differ)
      return fail(UOR_FBS_ERR_SHAPE, "hamming: mixed copy keys differ and leave copy_key at 1");
  }
  if (any2 && hw % 8)
    return fail(UOR_FBS_ERR_SHAPE, "hamming: copy key 2 needs heads of whole 8-coordinate blocks");
  if (hm.copy_longest && (!hm.copy_latest || !all_one || hm.marker[0] >= m->vocab || hm.marker[1] >= m->vocab))
    return fail(UOR_FBS_ERR_SHAPE,
                "hamming: the longest rule needs the latest exact rule, one-token copy keys and a "
                "marker of two vocabulary ids");
  if (hm.rule != UOR_FBS_COPY_ARTIFACT && hm.rule > UOR_FBS_COPY_LONGEST_AFTER_OPENING)
    return fail(UOR_FBS_ERR_ARGUMENT, "hamming: copy rule %u", hm.rule);
  if (hm.kept == 0) return fail(UOR_FBS_ERR_SHAPE, "hamming: a read keeps at least one position");
  if (hm.kept > kMaxHamKept)
    return fail(UOR_FBS_ERR_UNSUPPORTED, "hamming: %u kept positions (this build keeps at most %u)", hm.kept,
                kMaxHamKept);
  if (m->context >= (1u << kHamPosBits))
    return fail(UOR_FBS_ERR_UNSUPPORTED, "hamming: context %u past 2^24 - 1", m->context);
  if (hm.read_count == 0 || !hm.reads) return fail(UOR_FBS_ERR_SHAPE, "hamming: no reads");
  uint64_t typed = 0;
  for (uint32_t i = 0; i < hm.read_count; i++) {
    const uor_fbs_hamming_read &r = hm.reads[i];
    if (r.depth < 1 || r.depth > m->layer_count || (i && r.depth <= hm.reads[i - 1].depth))
      return fail(UOR_FBS_ERR_SHAPE, "hamming: read depths strictly increase from 1 to the layer count");
    if (!r.query_rotation || !r.key_rotation || !r.value_rotation || !r.margin || !r.weight)
      return fail(UOR_FBS_ERR_ARGUMENT, "hamming.d%u: null table", r.depth);
    for (uint32_t k = 0; k < heads; k++)
      if (r.margin[k] <= 0) return fail(UOR_FBS_ERR_SHAPE, "hamming.d%u.margin: a margin is not positive", r.depth);
    const bool last = i + 1 == hm.read_count;
    if (r.carry_rows || r.carry) {
      if (!last || r.depth != m->layer_count)
        return fail(UOR_FBS_ERR_SHAPE, "hamming: a question carry is served on the readout read only");
      if (!r.ask) return fail(UOR_FBS_ERR_SHAPE, "hamming: a question carry needs its read to ask");
      if (!r.carry || r.carry_rows == 0 || r.carry_rows > (1u << 12))
        return fail(UOR_FBS_ERR_SHAPE, "hamming: a question carry reaches 1 to 4096 rows with its gains");
    }
    bool ty = false;
    for (uint32_t c = 0; c < d; c++) ty |= r.weight[d + c] != 0;
    typed += ty && !r.ask;
  }
  if (typed * m->context * d * 8 > (1ull << 32))
    return fail(UOR_FBS_ERR_SHAPE, "hamming: the payload caches exceed 4 GiB a session");
  if (hm.place) {
    // StackHamming::check's place rules (format.rs:415-427) and PlaceImage::checked
    // (fbs_snapshot.rs:2779-2790, PlaceMarks::check :2741-2761).
    const uor_fbs_place &p = *hm.place;
    const uor_fbs_hamming_read &last = hm.reads[hm.read_count - 1];
    if (last.depth != m->layer_count || !last.ask)
      return fail(UOR_FBS_ERR_SHAPE, "hamming: a place read is served on a readout read that asks");
    if (hw % 8)
      return fail(UOR_FBS_ERR_SHAPE,
                  "hamming: a place read needs heads of whole 8-coordinate blocks, so each half is whole lanes");
    const uint32_t *lists[4] = {p.sep, p.system, p.user, p.assistant};
    const uint32_t lens[4] = {p.sep_len, p.system_len, p.user_len, p.assistant_len};
    for (int k = 0; k < 4; k++) {
      if (lens[k] > UOR_FBS_PLACE_MARK_MAX)
        return fail(UOR_FBS_ERR_UNSUPPORTED, "hamming: a place read's marker of %u ids (this build reads at most %u)",
                    lens[k], UOR_FBS_PLACE_MARK_MAX);
      if (lens[k] && !lists[k]) return fail(UOR_FBS_ERR_ARGUMENT, "hamming: a place read's null marker");
    }
    if (!p.class_table) return fail(UOR_FBS_ERR_ARGUMENT, "hamming: a place read's null class table");
    bool outside = p.bos >= m->vocab || p.eos >= m->vocab;
    for (int k = 0; k < 4; k++)
      for (uint32_t i = 0; i < lens[k]; i++) outside |= lists[k][i] >= m->vocab;
    if (outside) return fail(UOR_FBS_ERR_SHAPE, "hamming: a place read's mark is outside the vocabulary");
    if (!p.sep_len || !p.user_len || !p.assistant_len)
      return fail(UOR_FBS_ERR_SHAPE, "hamming: a place read needs a separator, a user marker and an assistant marker");
    if (p.bos == p.eos) return fail(UOR_FBS_ERR_SHAPE, "hamming: a place read's start mark and end mark are one token");
    for (int i = 1; i < 4; i++)
      for (int j = 1; j < 4; j++) {
        if (i == j || !lens[j] || lens[i] < lens[j]) continue;
        bool ends = true;
        for (uint32_t k = 0; k < lens[j]; k++) ends &= lists[i][lens[i] - lens[j] + k] == lists[j][k];
        if (ends) return fail(UOR_FBS_ERR_SHAPE, "hamming: one of a place read's role markers ends with another");
      }
    for (uint32_t v = 0; v < m->vocab; v++)
      if (p.class_table[v] & ~(UOR_FBS_PLACE_STOP | UOR_FBS_PLACE_ARM | UOR_FBS_PLACE_OPEN))
        return fail(UOR_FBS_ERR_SHAPE, "hamming: the place read's class table has a bit outside stop, arm and open");
    if (m->context > 0xffffu)
      return fail(UOR_FBS_ERR_UNSUPPORTED, "hamming: a place read over a context past 65535 positions");
  }
  return 0;
}

int validate(const uor_fbs_model *m, const uor_fbs_ext *e, Resolved *r) {
  if (!m) return fail(UOR_FBS_ERR_ARGUMENT, "null model");
  const uint32_t d = m->width, mlp = m->mlp;
  if (d < 32 || d > kMaxWidth || d % 32)
    return fail(UOR_FBS_ERR_SHAPE, "width %u: a multiple of 32 in 32..1024 (format.rs:724-729)", d);
  if (mlp < 32 || mlp > kMaxMpl * kWave * 4 || mlp % 32)
    return fail(UOR_FBS_ERR_SHAPE, "mlp %u: a multiple of 32 in 32..1024", mlp);
  if (m->vocab == 0 || m->vocab >= (1u << 24))
    return fail(UOR_FBS_ERR_SHAPE, "vocab %u: 1..2^24 - 1", m->vocab);
  if (m->context == 0) return fail(UOR_FBS_ERR_SHAPE, "zero context");
  if (m->layer_count == 0 || m->layer_count > 64)
    return fail(UOR_FBS_ERR_SHAPE, "layer count %u: 1..64", m->layer_count);
  if (m->kept == 0 || m->kept > 16)
    return fail(UOR_FBS_ERR_SHAPE, "kept cells %u: 1..16 (format.rs:436-439)", m->kept);
  if (!m->layers || !m->final_gain || !m->writer_table || !m->roots_q12 || !m->icosian || !m->keep_q31)
    return fail(UOR_FBS_ERR_ARGUMENT, "null model table");
  r->W = (e && e->window) ? e->window : 3;
  r->D = (e && e->drawers) ? e->drawers : 256;
  r->P = (e && e->probes) ? e->probes : m->kept;
  r->head = e ? e->head : 0;
  if (r->W > kMaxWindow) return fail(UOR_FBS_ERR_SHAPE, "window %u: 1..%u", r->W, kMaxWindow);
  if (r->D > kMaxDrawers) return fail(UOR_FBS_ERR_SHAPE, "drawers %u: 1..%u", r->D, kMaxDrawers);
  if (r->P > kMaxProbes || r->P > r->D)
    return fail(UOR_FBS_ERR_SHAPE, "probes %u: 1..min(drawers, %u)", r->P, kMaxProbes);
  if (r->head > 1) return fail(UOR_FBS_ERR_SHAPE, "head %u: 0 writer, 1 nearest", r->head);
  r->reference_writer = !(e && (e->drawer_keys || e->drawer_offsets)) && r->D == 256;
  if (r->D != 256 && !(e && e->drawer_keys))
    return fail(UOR_FBS_ERR_SHAPE, "%u drawers need drawer keys (root pairs make 256)", r->D);
  if (r->W != 3 && !(e && e->wide_taps))
    return fail(UOR_FBS_ERR_SHAPE, "window %u needs %u taps per channel (wide_taps)", r->W, r->W + 1);
  const uint32_t rows = d / 4 + d;
  for (uint32_t l = 0; l < m->layer_count; l++) {
    const uor_fbs_layer &ly = m->layers[l];
    int st;
    if ((st = check_codes(ly.rec_gain, d, "rec_norm_gain", l))) return st;
    if ((st = check_codes(ly.mlp_gain, d, "mlp_norm_gain", l))) return st;
    const int16_t *taps = (e && e->wide_taps) ? e->wide_taps[l] : ly.taps;
    if ((st = check_codes(taps, (size_t)(r->W + 1) * d, "conv_taps", l))) return st;
    if (!ly.conv_bias || !ly.gate_bias || !ly.decay_offset)
      return fail(UOR_FBS_ERR_ARGUMENT, "l%u: null bias table", l);
    if ((st = check_map(ly.rec_in, d, 2 * d, "rec_in.fbs", l))) return st;
    if ((st = check_map(ly.rec_gate, d, rows, "rec_gate.fbs", l))) return st;
    if ((st = check_map(ly.rec_out, d, d, "rec_out.fbs", l))) return st;
    if ((st = check_map(ly.mlp_gate, d, mlp, "mlp_gate.fbs", l))) return st;
    if ((st = check_map(ly.mlp_up, d, mlp, "mlp_up.fbs", l))) return st;
    if ((st = check_map(ly.mlp_down, mlp, d, "mlp_down.fbs", l))) return st;
  }
  int st;
  if ((st = check_codes(m->final_gain, d, "final_norm_gain", 0))) return st;
  if (e && e->table_i8 && e->table_shift > 8)
    return fail(UOR_FBS_ERR_SHAPE, "table_shift %u: 0..8", e->table_shift);
  if (e && e->drawer_keys)
    for (size_t i = 0; i < (size_t)r->D * 16; i++)
      if (e->drawer_keys[i] > kMaxKeyQ12 || e->drawer_keys[i] < -kMaxKeyQ12)
        return fail(UOR_FBS_ERR_UNSUPPORTED, "drawer key %d outside +-%d", e->drawer_keys[i], kMaxKeyQ12);
  if (e && e->drawer_offsets) {
    if (!e->drawer_members) return fail(UOR_FBS_ERR_ARGUMENT, "drawer offsets without members");
    for (uint32_t c = 0; c < r->D; c++)
      if (e->drawer_offsets[c + 1] < e->drawer_offsets[c])
        return fail(UOR_FBS_ERR_SHAPE, "drawer offsets decrease at %u", c);
    for (uint32_t i = e->drawer_offsets[0]; i < e->drawer_offsets[r->D]; i++)
      if (e->drawer_members[i] >= m->vocab)
        return fail(UOR_FBS_ERR_SHAPE, "drawer member %u outside the vocabulary", e->drawer_members[i]);
  }
  if (e && e->hamming && (st = check_hamming(m, *e->hamming))) return st;
  return 0;
}

// Gather program word of output `o` of `mp` (source words: 2 channel + negate).
uint16_t prog_word(const uor_fbs_map &mp, uint32_t o) {
  uint8_t code = mp.codes[o];
  uint32_t src = 8u * mp.atoms[o / 8] + (code & 7u);
  return (uint16_t)(2 * src + ((code >> 3) & 1u));
}

}  // namespace

namespace {

// The served reads (ServedHamming::new, hamming.rs:1571-1609, with CopyHeads::new :287-313 and
// TypeHeads::new :1130-1145): each read's three rotations as unit quaternions at Q31 (`units`
// :541-548, stack_rotation at lambda 2^31 and epsilon 0), every vocabulary entry's key code per
// head through the key rotation (`head_code`, `vocab_codes` :550-582), the copy heads' pair masks
// and rule, and the payload cache slot of each typed read that does not ask.
int upload_hamming(uor_fbs_handle *h, const uor_fbs_model *m, const uor_fbs_ext &e,
                   const uor_fbs_hamming &hm) {
  DevModel &M = h->M;
  DevHam &H = M.ham;
  const uint32_t d = m->width, V = m->vocab, heads = hm.heads, hw = d / heads;
  H.heads = heads;
  H.copy = heads / 2;
  H.hw = hw;
  H.kept = hm.kept;
  H.rule = hm.rule != UOR_FBS_COPY_ARTIFACT ? hm.rule
           : hm.copy_longest                ? UOR_FBS_COPY_LONGEST_AFTER_OPENING
           : hm.copy_latest                 ? UOR_FBS_COPY_LATEST_EXACT
                                            : UOR_FBS_COPY_MEAN;
  H.has_marker = hm.copy_longest != 0;
  H.m0 = hm.marker[0];
  H.m1 = hm.marker[1];
  std::vector<uint64_t> pair(H.copy);
  for (uint32_t k = 0; k < H.copy; k++) {
    const uint32_t key = hm.copy_keys ? hm.copy_keys[k] : hm.copy_key;
    pair[k] = key == 2 ? (1ull << (hw / 2)) - 1 : 0;
  }
  std::vector<int32_t> at(M.L + 1, -1);
  std::vector<DevHamRead> reads(hm.read_count);
  // The writer table's value of token v, channel c, at Q12: what the reads see.
  auto row_q12 = [&](uint32_t v, uint32_t c) -> int64_t {
    const size_t i = (size_t)v * d + c;
    return e.table_i8 ? (int64_t)e.table_i8[i] * (1 << e.table_shift) : m->writer_table[i];
  };
  int st;
  for (uint32_t i = 0; i < hm.read_count; i++) {
    const uor_fbs_hamming_read &r = hm.reads[i];
    DevHamRead &R = reads[i];
    at[r.depth] = (int32_t)i;
    std::vector<int64_t> units[3];
    const int32_t *raw[3] = {r.query_rotation, r.key_rotation, r.value_rotation};
    for (int k = 0; k < 3; k++) {
      units[k].resize(d);
      for (uint32_t q = 0; q < d / 4; q++) rotation(raw[k] + 4 * q, 1ull << 31, kGateEps, units[k].data() + 4 * q);
    }
    const int64_t **dst[3] = {&R.qu, &R.ku, &R.vu};
    for (int k = 0; k < 3; k++)
      if ((st = h->upload(units[k].data(), d, dst[k]))) return st;
    std::vector<uint64_t> codes((size_t)V * heads, 0);
    for (uint32_t v = 0; v < V; v++)
      for (uint32_t q = 0; q < d / 4; q++) {
        int64_t p[4];
        for (int c = 0; c < 4; c++) p[c] = row_q12(v, 4 * q + c);
        i128 o[4];
        hamilton64(units[1].data() + 4 * q, p, o);
        const uint32_t head = 4 * q / hw, bit = 4 * q % hw;
        for (int c = 0; c < 4; c++)
          if (o[c] >= 0) codes[(size_t)v * heads + head] |= 1ull << (bit + c);
      }
    if ((st = h->upload(codes.data(), codes.size(), &R.codes))) return st;
    if ((st = h->upload(r.margin, heads, &R.margin))) return st;
    std::vector<uint32_t> wd((size_t)heads * kHamBins, 0);
    for (uint32_t k = 0; k < heads; k++)
      for (uint32_t dd = 0; dd <= 64; dd++) wd[(size_t)k * kHamBins + dd] = copy_weight_q31(r.margin[k], dd);
    if ((st = h->upload(wd.data(), wd.size(), &R.wd))) return st;
    if ((st = h->upload(r.weight, 2 * (size_t)d, &R.w))) return st;
    R.ask = nullptr;
    R.carry = nullptr;
    if (r.ask && (st = h->upload(r.ask, (size_t)V * d, &R.ask))) return st;
    if (r.carry && (st = h->upload(r.carry, V, &R.carry))) return st;
    R.carry_rows = r.carry ? r.carry_rows : 0;
    R.typed = 0;
    for (uint32_t c = 0; c < d; c++) R.typed |= r.weight[d + c] != 0;
    R.slot = R.typed && !r.ask ? H.slots++ : kHamNoSlot;
  }
  H.place = 0;
  if (hm.place) {
    // The place read's ask heads find a place and bring nothing back: its read serves no type
    // heads and reads as a read that does not ask (`typed = places.is_none() && ...`,
    // hamming.rs:1580-1600); the question table and carry serve the find.
    const uor_fbs_place &p = *hm.place;
    H.place = 1;
    H.p_read = hm.read_count - 1;
    H.p_bos = p.bos;
    H.p_eos = p.eos;
    const uint32_t *lists[4] = {p.sep, p.system, p.user, p.assistant};
    const uint32_t lens[4] = {p.sep_len, p.system_len, p.user_len, p.assistant_len};
    std::vector<uint32_t> marks(4 * kPlaceMarkMax, 0);
    for (int k = 0; k < 4; k++) {
      H.p_len[k] = lens[k];
      for (uint32_t i = 0; i < lens[k]; i++) marks[k * kPlaceMarkMax + i] = lists[k][i];
    }
    if ((st = h->upload(marks.data(), marks.size(), &H.p_marks))) return st;
    std::vector<uint8_t> cls(V);
    for (uint32_t v = 0; v < V; v++) cls[v] = (uint8_t)p.class_table[v];
    if ((st = h->upload(cls.data(), cls.size(), &H.p_class))) return st;
    DevHamRead &R = reads[H.p_read];
    H.p_ask = R.ask;
    H.p_carry = R.carry;
    H.p_carry_rows = R.carry_rows;
    R.ask = nullptr;
    R.carry = nullptr;
    R.carry_rows = 0;
    R.typed = 0;
  }
  // A trace record's heads: each read's copy heads, then its type heads where it serves them.
  uint32_t before = 0;
  h->ham_read_typed.clear();
  for (DevHamRead &R : reads) {
    R.heads_before = before;
    before += H.copy + (R.typed ? heads - H.copy : 0);
    h->ham_read_typed.push_back(R.typed != 0);
  }
  H.nreads = hm.read_count;
  std::vector<uint32_t> ones(kHamBins, 1);
  if ((st = h->upload(ones.data(), ones.size(), &H.ones))) return st;
  if ((st = h->upload(pair.data(), pair.size(), &H.pair))) return st;
  if ((st = h->upload(at.data(), at.size(), &H.at))) return st;
  if ((st = h->upload(reads.data(), reads.size(), &H.reads))) return st;
  return 0;
}

}  // namespace

extern "C" int uor_fbs_model_create(const uor_fbs_model *m, const uor_fbs_ext *e, int32_t device,
                                    uor_fbs_handle **out) {
  if (!out) return fail(UOR_FBS_ERR_ARGUMENT, "null output handle");
  *out = nullptr;
  Resolved r;
  int st = validate(m, e, &r);
  if (st) return st;
  int count = 0;
  hipError_t he = hipGetDeviceCount(&count);
  if (he != hipSuccess || count == 0) return fail(UOR_FBS_ERR_DEVICE, "no HIP device");
  if (device < 0 || device >= count) return fail(UOR_FBS_ERR_ARGUMENT, "device %d of %d", device, count);
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(device);
  uor_fbs_handle *h = new uor_fbs_handle();
  h->device = device;
  h->scratch = scratch_address(device);
  DevModel &M = h->M;
  const uint32_t d = m->width, mlp = m->mlp, L = m->layer_count;
  M.vocab = m->vocab;
  M.d = d;
  M.m = mlp;
  M.L = L;
  M.W = r.W;
  M.D = r.D;
  M.P = r.P;
  M.head = r.head;
  M.context = m->context;
  M.raw_gates = m->raw_gates != 0;
  M.raw_transition = m->raw_transition != 0;
  M.nq = d / 4;
  M.nm = mlp / 4;
  M.qpl = (M.nq + kWave - 1) / kWave;
  if (M.qpl == 3) M.qpl = 4;
  M.mpl = (M.nm + kWave - 1) / kWave;
  const uint32_t Q = M.qpl, MP = M.mpl;
  M.s_rec_in = 0;
  M.s_rec_gate = 8 * Q;
  M.s_rec_out = 13 * Q;
  M.s_mlp_gate = 17 * Q;
  M.s_mlp_up = 17 * Q + 4 * MP;
  M.s_mlp_down = 17 * Q + 8 * MP;
  M.nslots = 21 * Q + 8 * MP;
  M.xbar_words = 2 * (d > mlp ? d : mlp);
  M.identity_rows = r.head == 1;
  M.taps_fast = 1;
  M.gains_fast = 1;
  M.log2d = (d & (d - 1)) == 0 ? (uint32_t)__builtin_ctz(d) : 0xffu;
  // UOR_FBS_WRITER_MEMORY=0 turns the writer's memory of its last query off (for measurement:
  // every step then scans its candidates; the results are the same either way).
  const char *wm = getenv("UOR_FBS_WRITER_MEMORY");
  M.writer_memory = (wm && wm[0] == '0' && !wm[1]) ? 0u : 1u;
  // UOR_FBS_SERVE_SCAN=fused keeps the writer inside one-token serving launches, =drawer takes
  // the drawer-major scan; otherwise the drawers' sizes choose (below). The results are the same
  // either way.
  const char *ss = getenv("UOR_FBS_SERVE_SCAN");
  const int serve_mode = ss && std::strcmp(ss, "fused") == 0    ? 2
                         : ss && std::strcmp(ss, "drawer") == 0 ? 1
                                                                 : 0;
  M.w_recip = (1ull << 32) / M.W;
  int64_t eps_int[9];
  for (int sh = 0; sh <= 8; sh++) eps_int[sh] = norm_eps(m->eps_mantissa, m->eps_exp, sh);

  auto done = [&](int code) {
    if (code) delete h;
    else *out = h;
    (void)hipSetDevice(prev);
    return code;
  };

  // Layers: gains, taps, biases and the gather program.
  std::vector<DevLayer> layers(L);
  for (uint32_t l = 0; l < L; l++) {
    const uor_fbs_layer &ly = m->layers[l];
    DevLayer &dl = layers[l];
    if ((st = h->upload(ly.rec_gain, d, &dl.rec_gain))) return done(st);
    if ((st = h->upload(ly.mlp_gain, d, &dl.mlp_gain))) return done(st);
    const int16_t *taps = (e && e->wide_taps) ? e->wide_taps[l] : ly.taps;
    if ((st = h->upload(taps, (size_t)(r.W + 1) * d, &dl.taps))) return done(st);
    {
      std::vector<uint16_t> td((size_t)(r.W + 1) * d), rg(d), mg(d);
      for (size_t i = 0; i < td.size(); i++) {
        td[i] = tap_desc(taps[i]);
        if (td[i] == kGridDescSlow) M.taps_fast = 0;
      }
      for (uint32_t i = 0; i < d; i++) {
        rg[i] = grid_desc(ly.rec_gain[i]);
        mg[i] = grid_desc(ly.mlp_gain[i]);
        if (rg[i] == kGridDescSlow || mg[i] == kGridDescSlow) M.gains_fast = 0;
      }
      if ((st = h->upload(td.data(), td.size(), &dl.taps_desc))) return done(st);
      if ((st = h->upload(rg.data(), rg.size(), &dl.rec_gain_desc))) return done(st);
      if ((st = h->upload(mg.data(), mg.size(), &dl.mlp_gain_desc))) return done(st);
    }
    if ((st = h->upload(ly.conv_bias, d, &dl.conv_bias))) return done(st);
    if ((st = h->upload(ly.gate_bias, d / 4 + d, &dl.gate_bias))) return done(st);
    if ((st = h->upload(ly.decay_offset, d / 4, &dl.decay_offset))) return done(st);
    std::vector<uint16_t> prog((size_t)M.nslots * kWave, 0);
    auto put = [&](uint32_t slot, uint32_t lane, uint16_t w) { prog[(size_t)slot * kWave + lane] = w; };
    for (uint32_t lane = 0; lane < kWave; lane++) {
      for (uint32_t k = 0; k < Q; k++) {
        uint32_t q = lane + kWave * k;
        if (q >= M.nq) continue;
        for (uint32_t c = 0; c < 4; c++) {
          put(M.s_rec_in + 4 * k + c, lane, prog_word(ly.rec_in, 4 * q + c));
          put(M.s_rec_in + 4 * Q + 4 * k + c, lane, prog_word(ly.rec_in, d + 4 * q + c));
          put(M.s_rec_gate + Q + 4 * k + c, lane, prog_word(ly.rec_gate, M.nq + 4 * q + c));
          put(M.s_rec_out + 4 * k + c, lane, prog_word(ly.rec_out, 4 * q + c));
          put(M.s_mlp_down + 4 * k + c, lane, prog_word(ly.mlp_down, 4 * q + c));
        }
        put(M.s_rec_gate + k, lane, prog_word(ly.rec_gate, q));
      }
      for (uint32_t j = 0; j < MP; j++) {
        uint32_t mq = lane + kWave * j;
        if (mq >= M.nm) continue;
        for (uint32_t c = 0; c < 4; c++) {
          put(M.s_mlp_gate + 4 * j + c, lane, prog_word(ly.mlp_gate, 4 * mq + c));
          put(M.s_mlp_up + 4 * j + c, lane, prog_word(ly.mlp_up, 4 * mq + c));
        }
      }
    }
    if ((st = h->upload(prog.data(), prog.size(), &dl.prog))) return done(st);
  }
  if ((st = h->upload(layers.data(), layers.size(), &M.layers))) return done(st);
  if ((st = h->upload(m->final_gain, d, &M.final_gain))) return done(st);
  {
    std::vector<uint16_t> fg(d);
    for (uint32_t i = 0; i < d; i++) {
      fg[i] = grid_desc(m->final_gain[i]);
      if (fg[i] == kGridDescSlow) M.gains_fast = 0;
    }
    if ((st = h->upload(fg.data(), fg.size(), &M.final_gain_desc))) return done(st);
  }

  // Writer table, biased for the unsigned SAD (row value v stored as v ^ 0x8000).
  {
    size_t n = (size_t)m->vocab * d;
    std::vector<uint16_t> tb(n);
    if (e && e->table_i8) {
      for (size_t i = 0; i < n; i++)
        tb[i] = (uint16_t)((uint16_t)((int32_t)e->table_i8[i] * (1 << e->table_shift)) ^ 0x8000u);
    } else {
      for (size_t i = 0; i < n; i++) tb[i] = (uint16_t)((uint16_t)m->writer_table[i] ^ 0x8000u);
    }
    if ((st = h->upload(tb.data(), n, &M.table_b))) return done(st);
    M.table8 = nullptr;
    M.t8_shift = 0;
    if (e && e->table_i8) {  // the writer's scan reads the codes themselves, biased
      std::vector<uint8_t> t8(n);
      for (size_t i = 0; i < n; i++) t8[i] = (uint8_t)((int32_t)e->table_i8[i] + 128);
      if ((st = h->upload(t8.data(), n, &M.table8))) return done(st);
      M.t8_shift = e->table_shift;
    }
  }
  // Drawer keys: the extension's, or the 256 root pairs (cell c = a * 16 + b scores the first
  // 8-block against root a and the last against root b, session.rs:4069-4090).
  {
    std::vector<int16_t> keys((size_t)r.D * 16);
    for (uint32_t c = 0; c < r.D; c++)
      for (int i = 0; i < 8; i++) {
        int32_t ka, kb;
        if (e && e->drawer_keys) {
          ka = e->drawer_keys[16ull * c + i];
          kb = e->drawer_keys[16ull * c + 8 + i];
        } else {
          ka = m->roots_q12[8 * (c >> 4) + i];
          kb = m->roots_q12[8 * (c & 15) + i];
          if (ka > kMaxKeyQ12 || ka < -kMaxKeyQ12 || kb > kMaxKeyQ12 || kb < -kMaxKeyQ12)
            return done(fail(UOR_FBS_ERR_UNSUPPORTED, "root coordinate outside +-%d", kMaxKeyQ12));
        }
        keys[16ull * c + i] = (int16_t)ka;
        keys[16ull * c + 8 + i] = (int16_t)kb;
      }
    if ((st = h->upload(keys.data(), keys.size(), &M.keys))) return done(st);
  }
  // Drawer membership as CSR: the extension's, or token t in drawer t mod D (ascending).
  {
    std::vector<uint32_t> off(r.D + 1), mem;
    if (e && e->drawer_offsets) {
      uint32_t b0 = e->drawer_offsets[0];
      for (uint32_t c = 0; c <= r.D; c++) off[c] = e->drawer_offsets[c] - b0;
      mem.assign(e->drawer_members + b0, e->drawer_members + e->drawer_offsets[r.D]);
    } else {
      mem.reserve(m->vocab);
      for (uint32_t c = 0; c < r.D; c++) {
        off[c] = (uint32_t)mem.size();
        for (uint32_t t = c; t < m->vocab; t += r.D) mem.push_back(t);
      }
      off[r.D] = (uint32_t)mem.size();
    }
    if (mem.empty()) mem.push_back(0);
    if ((st = h->upload(off.data(), off.size(), &M.offsets))) return done(st);
    if ((st = h->upload(mem.data(), mem.size(), &M.members))) return done(st);
    // The deferred writer's scan chunks: each drawer's members, 64 at a time; and whether the
    // drawers' sizes are skewed enough for it (measured: C3's Zipf drawers, largest 512 against
    // a mean of 128, 0.105 against 0.159 ms a serving launch; C2's uniform ones 0.095-0.115
    // against 0.075-0.083 ms).
    uint32_t largest = 0;
    for (uint32_t c = 0; c < r.D; c++) {
      const uint32_t size = off[c + 1] - off[c], nch = (size + kServeRows - 1) / kServeRows;
      h->serve_nchunks += nch;
      h->serve_max_chunks = nch > h->serve_max_chunks ? nch : h->serve_max_chunks;
      largest = size > largest ? size : largest;
    }
    const bool skewed = (uint64_t)largest * r.D > 2ull * off[r.D];
    h->serve_drawer_major = serve_mode == 1 || (serve_mode == 0 && skewed);
  }
  if ((st = h->upload(m->icosian, 120 * 8, &M.icosian))) return done(st);
  if ((st = h->upload(m->keep_q31, 16, &M.keep_q31))) return done(st);
  if ((st = h->upload(eps_int, 9, &M.eps_int))) return done(st);
  M.eps0 = eps_int[0];

  if (e && e->hamming && (st = upload_hamming(h, m, *e, *e->hamming))) return done(st);

  hipDeviceProp_t prop;
  he = hipGetDeviceProperties(&prop, device);
  if (he != hipSuccess) return done(hip_fail(he, "hipGetDeviceProperties"));
  M.list_cap = M.ham.heads ? kListCap / 2 : kListCap;  // the paired kernels split kListCap
  h->lds_bytes = fbs::lds_bytes(M) + fbs::ham_lds_bytes(M);
  if (h->lds_bytes > prop.sharedMemPerBlock)
    return done(fail(UOR_FBS_ERR_UNSUPPORTED, "%zu bytes of LDS per sequence exceed %zu",
                     h->lds_bytes, (size_t)prop.sharedMemPerBlock));
  h->max_grid = (uint32_t)prop.multiProcessorCount * 8;
  // UOR_FBS_BLOCK_WAVES=1 fixes one wavefront per sequence (default: paired blocks).
  const char *bw = getenv("UOR_FBS_BLOCK_WAVES");
  // A model with Hamming reads pairs at one quaternion a lane (wider, the paired reads spill
  // their registers) where wave 1's read scratch fits the LDS a read leaves unused
  // (ham_pair_fits); its blocks add the reads' LDS to the paired layout.
  h->pair_lds = fbs::pair_lds_bytes(M) + fbs::ham_lds_bytes(M);
  h->pair = !(bw && bw[0] == '1' && !bw[1]) && h->pair_lds <= prop.sharedMemPerBlock &&
            (!M.ham.heads || (M.qpl == 1 && fbs::ham_pair_fits(M)));
  h->pair_grid = (uint32_t)prop.multiProcessorCount * 4;  // four SIMDs per CU
  h->cus = (uint32_t)prop.multiProcessorCount;
  h->lds_limit = prop.sharedMemPerBlock;
  return done(0);
}

extern "C" void uor_fbs_model_destroy(uor_fbs_handle *h) { delete h; }

extern "C" uint64_t uor_fbs_state_words(const uor_fbs_handle *h) {
  return h ? (uint64_t)h->M.L * h->M.d : 0;
}
extern "C" uint64_t uor_fbs_history_words(const uor_fbs_handle *h) {
  return h ? (uint64_t)h->M.L * h->M.W * h->M.d : 0;
}
extern "C" uint32_t uor_fbs_block_waves(const uor_fbs_handle *h, uint32_t n) {
  (void)n;
  return h && h->pair ? 2u : 1u;
}

namespace {

// `noalloc`: the window rings and sums come from the device's scratch array, whose size bounds
// the grid (sequences loop within the blocks), and nothing is allocated. `one_wave`: the
// one-wavefront kernels whatever the model's default (the snap trace is recorded there).
int launch(uor_fbs_handle *h, RunArgs &A, hipStream_t stream, bool noalloc = false,
           bool one_wave = false) {
  if (A.n == 0) return 0;
  const bool clocks = A.out_parts != nullptr;
  if (clocks && (!h->pair || one_wave || noalloc || h->M.ham.heads || A.mode != kModeDecode ||
                 A.gen == 0 || A.slots))
    return fail(UOR_FBS_ERR_UNSUPPORTED,
                "the part clocks time the paired decode kernels (a model they serve, gen > 0)");
  if (!A.slots) A.capacity = A.n;
  const bool pair = h->pair && !one_wave;
  const uint32_t cap = pair ? h->pair_grid : h->max_grid;
  uint32_t grid = A.n < cap ? A.n : cap;
  if (noalloc && h->M.ham.heads)
    return fail(UOR_FBS_ERR_UNSUPPORTED,
                "the allocation-free decode serves no Hamming reads (their token streams and payload "
                "caches are the caller's: uor_fbs_decode_stream_async)");
  if (h->M.ham.slots && !A.out_payloads) {
    // The library's payload caches, one per resident block, within 16 GiB (blocks loop over
    // their sequences).
    const size_t per = h->payload_words() * sizeof(int64_t), fit = ((size_t)16 << 30) / per;
    if (fit == 0) return fail(UOR_FBS_ERR_UNSUPPORTED, "one session's payload caches exceed 16 GiB");
    grid = grid < fit ? grid : (uint32_t)fit;
    int st = h->ensure_pay(grid);
    if (st) return st;
    A.pay = h->pay;
  }
  if (noalloc) {
    if (!h->scratch)
      return fail(UOR_FBS_ERR_DEVICE, "the scratch array's device address could not be read");
    const size_t ring = (size_t)h->M.L * h->M.W * h->M.d * sizeof(int32_t);
    const size_t sums = pair ? 2 * (size_t)h->M.L * h->M.d * sizeof(int64_t) : 0;  // and states
    const size_t fit = (UOR_FBS_NOALLOC_SCRATCH_BYTES - 256) / (ring + sums);
    if (fit == 0)
      return fail(UOR_FBS_ERR_UNSUPPORTED,
                  "one sequence's window ring, sums and state (%zu bytes) exceed the %zu-byte scratch",
                  ring + sums, (size_t)UOR_FBS_NOALLOC_SCRATCH_BYTES);
    grid = grid < fit ? grid : (uint32_t)fit;
    A.ring = (int32_t *)h->scratch;
    A.hist = (int64_t *)(h->scratch + ((grid * ring + 255) & ~(size_t)255));
  } else {
    int st = h->ensure_ring(grid);
    if (st) return st;
    A.ring = h->ring;
    A.hist = h->hist;
  }
  const bool decode = A.mode == kModeDecode;
  const uint32_t waves = pair ? 2 : 1;
  const size_t lds = pair ? h->pair_lds + (clocks ? clock_lds_bytes() : 0) : h->lds_bytes;
  if (clocks) {
    if (lds > h->lds_limit)
      return fail(UOR_FBS_ERR_UNSUPPORTED, "the part clocks' LDS (%zu bytes) does not fit", lds);
    hipError_t e = launch_fbs_decode_pair_clk(h->M, A, grid, lds, stream);
    return e != hipSuccess ? hip_fail(e, "kernel launch") : 0;
  }
  if (A.out_dtrace) {  // the traced teacher-forced kernels (one wavefront a sequence)
    if (pair || A.mode != kModeSequences)
      return fail(UOR_FBS_ERR_UNSUPPORTED, "the traces run teacher-forced on one wavefront");
    hipError_t e = launch_fbs_rows_dt(h->M, A, grid, lds, stream);
    return e != hipSuccess ? hip_fail(e, "kernel launch") : 0;
  }
  using Launcher = hipError_t (*)(const DevModel &, const RunArgs &, uint32_t, size_t, hipStream_t);
  // Families: one wavefront, paired, Hamming reads, then the first two for an int8 table, then
  // the paired Hamming reads.
  static const Launcher table[3][6] = {
      {launch_fbs_prefill, launch_fbs_prefill_pair, launch_fbs_prefill_ham, launch_fbs_prefill_8,
       launch_fbs_prefill_pair8, launch_fbs_prefill_pair_ham},
      {launch_fbs_decode, launch_fbs_decode_pair, launch_fbs_decode_ham, launch_fbs_decode_8,
       launch_fbs_decode_pair8, launch_fbs_decode_pair_ham},
      {launch_fbs_rows, launch_fbs_rows_pair, launch_fbs_rows_ham, launch_fbs_rows_8,
       launch_fbs_rows_pair8, launch_fbs_rows_pair_ham}};
  const int phase = decode && A.gen == 0 ? 0 : decode ? 1 : 2;
  const int family = h->M.ham.heads ? (waves == 2 ? 5 : 2) : (waves == 2 ? 1 : 0) + (h->M.table8 ? 3 : 0);
  hipError_t e = table[phase][family](h->M, A, grid, lds, stream);
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return 0;
}

// Device buffers for the host-buffer entry points.
struct DevBuf {
  std::vector<void *> ptrs;
  ~DevBuf() {
    for (void *p : ptrs) (void)hipFree(p);
  }
  template <class T>
  int alloc(T **p, size_t count) {
    *p = nullptr;
    if (count == 0) return 0;
    hipError_t e = hipMalloc((void **)p, count * sizeof(T));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    ptrs.push_back(*p);
    return 0;
  }
  template <class T>
  int in(T **p, const T *src, size_t count) {
    if (!src) {
      *p = nullptr;
      return 0;
    }
    int st = alloc(p, count);
    if (st) return st;
    hipError_t e = hipMemcpy(*p, src, count * sizeof(T), hipMemcpyHostToDevice);
    return e == hipSuccess ? 0 : hip_fail(e, "hipMemcpy");
  }
};

template <class T>
int copy_out(T *dst, const T *src, size_t count) {
  if (!dst || !src || count == 0) return 0;
  hipError_t e = hipMemcpy(dst, src, count * sizeof(T), hipMemcpyDeviceToHost);
  return e == hipSuccess ? 0 : hip_fail(e, "hipMemcpy");
}

int first_status(const std::vector<int32_t> &status) {
  for (int32_t s : status)
    if (s) return fail(s, "a sequence failed with status %d (1 token, 2 context, 3 slot)", s);
  return 0;
}

// A Hamming model's session reads its earlier tokens (and payloads): resuming one needs them.
int refuse_streamless() {
  return fail(UOR_FBS_ERR_UNSUPPORTED,
              "a Hamming model resumes a session only with its token stream "
              "(uor_fbs_decode_stream_async)");
}

struct DeviceScope {
  int prev = 0;
  explicit DeviceScope(int dev) {
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(dev);
  }
  ~DeviceScope() { (void)hipSetDevice(prev); }
};

}  // namespace

extern "C" int uor_fbs_sequences_async(uor_fbs_handle *h, const uint32_t *tokens, uint32_t sequences,
                                       uint32_t len, uint32_t *out_tokens, uint32_t *out_kept,
                                       int32_t *out_query, int32_t *status, void *stream) {
  if (!h || (!tokens && sequences && len) || !status || !out_tokens)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeSequences;
  A.n = sequences;
  A.len = len;
  A.tokens = tokens;
  A.out_tokens = out_tokens;
  A.out_kept = out_kept;
  A.out_query = out_query;
  A.status = status;
  return launch(h, A, (hipStream_t)stream);
}

extern "C" uint64_t uor_fbs_trace_stride(const uor_fbs_handle *h) {
  return h ? (uint64_t)h->M.L * (2 * h->M.nq + h->M.nm) : 0;
}

extern "C" int uor_fbs_trace_sequences_async(uor_fbs_handle *h, const uint32_t *tokens,
                                             uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                                             uint32_t *out_kept, int32_t *out_query,
                                             uint8_t *out_trace, int32_t *status, void *stream) {
  if (!h || (!tokens && sequences && len) || !status || !out_tokens || !out_trace)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeSequences;
  A.n = sequences;
  A.len = len;
  A.tokens = tokens;
  A.out_tokens = out_tokens;
  A.out_kept = out_kept;
  A.out_query = out_query;
  A.out_trace = out_trace;
  A.status = status;
  return launch(h, A, (hipStream_t)stream, false, true);
}

extern "C" int uor_fbs_trace_sequences(uor_fbs_handle *h, const uint32_t *tokens,
                                       uint32_t sequences, uint32_t len, uint32_t *out_tokens,
                                       uint32_t *out_kept, int32_t *out_query,
                                       uint8_t *out_trace) {
  if (!h || !tokens || !out_tokens || !out_trace) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (sequences == 0 || len == 0) return 0;
  DeviceScope scope(h->device);
  const size_t n = (size_t)sequences * len, stride = uor_fbs_trace_stride(h);
  DevBuf b;
  uint32_t *dt, *dot, *dk = nullptr;
  int32_t *dq = nullptr, *ds;
  uint8_t *dtr;
  int st;
  if ((st = b.in(&dt, tokens, n)) || (st = b.alloc(&dot, n)) || (st = b.alloc(&ds, sequences)) ||
      (st = b.alloc(&dtr, n * stride)))
    return st;
  if (out_kept && (st = b.alloc(&dk, n * h->M.P))) return st;
  if (out_query && (st = b.alloc(&dq, n * h->M.d))) return st;
  if ((st = uor_fbs_trace_sequences_async(h, dt, sequences, len, dot, dk, dq, dtr, ds, nullptr)))
    return st;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(sequences);
  if ((st = copy_out(status.data(), ds, sequences)) || (st = copy_out(out_tokens, dot, n)) ||
      (st = copy_out(out_kept, dk, n * h->M.P)) || (st = copy_out(out_query, dq, n * h->M.d)) ||
      (st = copy_out(out_trace, dtr, n * stride)))
    return st;
  return first_status(status);
}

extern "C" uint64_t uor_fbs_decision_stride(const uor_fbs_handle *h, uint32_t decisions) {
  if (!h) return 0;
  const DevModel &M = h->M;
  uint64_t at = decisions ? decision_bucket_bytes(M.L, M.nq) : 0;
  if (M.ham.heads) {
    uint32_t heads = 0;
    const uint32_t copy = M.ham.heads / 2;
    for (uint32_t i = 0; i < h->ham_read_typed.size(); i++)
      heads += copy + (h->ham_read_typed[i] ? M.ham.heads - copy : 0);
    at += (uint64_t)heads * decision_head_bytes(M.ham.kept);
  }
  return at;
}

extern "C" int uor_fbs_decision_sequences(uor_fbs_handle *h, const uint32_t *tokens,
                                          uint32_t sequences, uint32_t len, uint32_t decisions,
                                          const uint8_t *force_buckets, const uint64_t *force_codes,
                                          const uint8_t *force_mask, uint32_t *out_tokens,
                                          int32_t *out_query, uint8_t *out_trace) {
  if (!h || !tokens || !out_tokens || !out_trace) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (sequences == 0 || len == 0) return 0;
  const DevModel &M = h->M;
  // set_decision_trace's refusals (session.rs:2438-2500).
  if (decisions && (!M.raw_gates || !M.raw_transition))
    return fail(UOR_FBS_ERR_SHAPE,
                "the decision trace reads an unsnapped artifact: the snap is not a decision it records");
  if (decisions && M.head != 1)
    return fail(UOR_FBS_ERR_SHAPE,
                "the decision trace reads the Hamilton gate and the nearest head, with no point key");
  if (force_buckets && !decisions)
    return fail(UOR_FBS_ERR_ARGUMENT, "forced buckets need the decision trace");
  if (!force_codes != !force_mask) return fail(UOR_FBS_ERR_ARGUMENT, "forced codes come with their mask");
  if (len > M.context) return fail(UOR_FBS_ERR_SHAPE, "a window past the context");
  const size_t n = (size_t)sequences * len, lanes = (size_t)M.L * M.nq;
  if (force_buckets)
    for (size_t i = 0; i < n * lanes; i++)
      if (force_buckets[i] != 255 && force_buckets[i] > 15)
        return fail(UOR_FBS_ERR_SHAPE, "a forced bucket names a step, layer, lane or entry outside the model");
  const uint32_t R = M.ham.heads ? M.ham.nreads : 0, H = M.ham.heads, copy = H / 2;
  if (force_mask) {
    if (!M.ham.heads) return fail(UOR_FBS_ERR_SHAPE, "a forced code names a read the model does not have");
    bool any = false;
    for (size_t i = 0; i < n * R * H; i++) {
      const uint8_t f = force_mask[i];
      if (!f) continue;
      any = true;
      const size_t head = i % H, r = (i / H) % R, step = (i / H / R) % len;
      if (f & ~3u) return fail(UOR_FBS_ERR_ARGUMENT, "a forced code's mask holds bits 0 and 1");
      if (head >= copy && !h->ham_read_typed[r])
        return fail(UOR_FBS_ERR_SHAPE, "a forced code names a head its read does not serve");
      if ((f & 2u) && step == 0) return fail(UOR_FBS_ERR_SHAPE, "a forced key at step 0 names no candidate");
    }
    if (any && M.ham.place) return fail(UOR_FBS_ERR_SHAPE, "forced codes are not served with a place read");
  }
  DeviceScope scope(h->device);
  const uint64_t stride = uor_fbs_decision_stride(h, decisions);
  DevBuf b;
  uint32_t *dt, *dot;
  int32_t *dq = nullptr, *ds;
  uint8_t *dtr, *dfb = nullptr, *dfm = nullptr;
  uint64_t *dfc = nullptr;
  int st;
  if ((st = b.in(&dt, tokens, n)) || (st = b.alloc(&dot, n)) || (st = b.alloc(&ds, sequences)) ||
      (st = b.alloc(&dtr, n * stride)) || (st = b.in(&dfb, force_buckets, n * lanes)) ||
      (st = b.in(&dfc, force_codes, n * R * H * 2)) || (st = b.in(&dfm, force_mask, n * R * H)))
    return st;
  if (out_query && (st = b.alloc(&dq, n * M.d))) return st;
  if (stride) {
    hipError_t e = hipMemset(dtr, 0, n * stride);
    if (e != hipSuccess) return hip_fail(e, "hipMemset");
  }
  RunArgs A{};
  A.mode = kModeSequences;
  A.n = sequences;
  A.len = len;
  A.tokens = dt;
  A.out_tokens = dot;
  A.out_query = dq;
  A.status = ds;
  A.out_dtrace = dtr;
  A.dstride = (uint32_t)stride;
  A.decisions = decisions ? 1u : 0u;
  A.force_buckets = dfb;
  A.force_codes = dfc;
  A.force_mask = dfm;
  if ((st = launch(h, A, nullptr, false, true))) return st;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(sequences);
  if ((st = copy_out(status.data(), ds, sequences)) || (st = copy_out(out_tokens, dot, n)) ||
      (st = copy_out(out_query, dq, n * M.d)) || (st = copy_out(out_trace, dtr, n * stride)))
    return st;
  return first_status(status);
}

extern "C" int uor_fbs_sequences(uor_fbs_handle *h, const uint32_t *tokens, uint32_t sequences,
                                 uint32_t len, uint32_t *out_tokens, uint32_t *out_kept,
                                 int32_t *out_query) {
  if (!h || !tokens || !out_tokens) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (sequences == 0 || len == 0) return 0;
  DeviceScope scope(h->device);
  size_t n = (size_t)sequences * len;
  DevBuf b;
  uint32_t *dt, *dot, *dk = nullptr;
  int32_t *dq = nullptr, *ds;
  int st;
  if ((st = b.in(&dt, tokens, n)) || (st = b.alloc(&dot, n)) || (st = b.alloc(&ds, sequences)))
    return st;
  if (out_kept && (st = b.alloc(&dk, n * h->M.P))) return st;
  if (out_query && (st = b.alloc(&dq, n * h->M.d))) return st;
  if ((st = uor_fbs_sequences_async(h, dt, sequences, len, dot, dk, dq, ds, nullptr))) return st;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(sequences);
  if ((st = copy_out(status.data(), ds, sequences)) || (st = copy_out(out_tokens, dot, n)) ||
      (st = copy_out(out_kept, dk, n * h->M.P)) || (st = copy_out(out_query, dq, n * h->M.d)))
    return st;
  return first_status(status);
}

extern "C" int uor_fbs_decode_async(uor_fbs_handle *h, const uint32_t *prompts, uint32_t sequences,
                                    uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                                    const int64_t *in_state, const int32_t *in_history,
                                    const uint32_t *in_position, int64_t *out_state,
                                    int32_t *out_history, uint32_t *out_position, int32_t *status,
                                    void *stream) {
  if (!h || !prompts || !out_reply || !status) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  if (in_position && h->M.ham.heads) return refuse_streamless();
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = in_state;
  A.in_history = in_history;
  A.in_position = in_position;
  A.out_state = out_state;
  A.out_history = out_history;
  A.out_position = out_position;
  A.status = status;
  return launch(h, A, (hipStream_t)stream);
}

extern "C" uint32_t uor_fbs_part_count(void) { return kParts; }

extern "C" const char *uor_fbs_part_name(uint32_t part) {
  static const char *const names[kParts] = {
      "embed",        "loads",          "norm_rec",     "sync1",          "transition",
      "sync2",        "transport",      "requant_rec",  "residual_rec",   "norm_mlp",
      "sync3",        "mlp",            "sync4",        "requant_mlp",    "sync5",
      "residual_mlp", "final",          "sync6",        "select",         "sync7",
      "scan",         "sync8",          "step"};
  return part < kParts ? names[part] : nullptr;
}

extern "C" int uor_fbs_decode_parts_async(uor_fbs_handle *h, const uint32_t *prompts,
                                          uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                                          uint32_t *out_reply, const int64_t *in_state,
                                          const int32_t *in_history, const uint32_t *in_position,
                                          int64_t *out_state, int32_t *out_history,
                                          uint32_t *out_position, int32_t *status,
                                          uint64_t *out_parts, void *stream) {
  if (!h || !prompts || !out_reply || !status || !out_parts)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = in_state;
  A.in_history = in_history;
  A.in_position = in_position;
  A.out_state = out_state;
  A.out_history = out_history;
  A.out_position = out_position;
  A.status = status;
  A.out_parts = out_parts;
  return launch(h, A, (hipStream_t)stream);
}

extern "C" int uor_fbs_decode_noalloc_async(uor_fbs_handle *h, const uint32_t *prompts,
                                            uint32_t sequences, uint32_t prompt_len, uint32_t gen,
                                            uint32_t *out_reply, const int64_t *in_state,
                                            const int32_t *in_history, const uint32_t *in_position,
                                            int64_t *out_state, int32_t *out_history,
                                            uint32_t *out_position, int32_t *status, void *stream) {
  if (!h || !prompts || !out_reply || !status) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  if (in_position && h->M.ham.heads) return refuse_streamless();
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = in_state;
  A.in_history = in_history;
  A.in_position = in_position;
  A.out_state = out_state;
  A.out_history = out_history;
  A.out_position = out_position;
  A.status = status;
  return launch(h, A, (hipStream_t)stream, true);
}

extern "C" int uor_fbs_decode_slots_async(uor_fbs_handle *h, const uint32_t *slots,
                                          uint32_t sequences, uint32_t capacity,
                                          const uint32_t *prompts, uint32_t prompt_len,
                                          uint32_t gen, uint32_t *out_reply, int64_t *state,
                                          int32_t *history, uint32_t *position, uint32_t *out_kept,
                                          int32_t *out_query, int32_t *status, void *stream) {
  if (!h || !slots || !prompts || !out_reply || !state || !history || !position || !status)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a step needs at least one token");
  if (h->M.ham.heads)
    return fail(UOR_FBS_ERR_UNSUPPORTED,
                "session slots serve no Hamming reads yet (uor_fbs_decode_stream_async resumes them)");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = state;
  A.in_history = history;
  A.in_position = position;
  A.out_state = state;
  A.out_history = history;
  A.out_position = position;
  A.out_kept = out_kept;
  A.out_query = out_query;
  A.slots = slots;
  A.capacity = capacity;
  A.status = status;
  return launch(h, A, (hipStream_t)stream);
}

extern "C" uint64_t uor_fbs_slot_cache_bytes(const uor_fbs_handle *h) {
  return h ? slot_cache_layout(h->M).bytes : 0;
}

extern "C" int uor_fbs_serve_slots_async(uor_fbs_handle *h, const uint32_t *slots,
                                         uint32_t sequences, uint32_t capacity,
                                         const uint32_t *prompts, uint32_t prompt_len, uint32_t gen,
                                         uint32_t *out_reply, int64_t *state, int32_t *history,
                                         uint32_t *position, void *cache, const uint8_t *slide,
                                         uint32_t *out_kept, int32_t *out_query, uint8_t *out_trace,
                                         int32_t *status, void *stream) {
  if (!h || !slots || !prompts || !out_reply || !state || !history || !position || !status)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a step needs at least one token");
  if (h->M.ham.heads)
    return fail(UOR_FBS_ERR_UNSUPPORTED,
                "session slots serve no Hamming reads yet (uor_fbs_decode_stream_async resumes them)");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = state;
  A.in_history = history;
  A.in_position = position;
  A.out_state = state;
  A.out_history = history;
  A.out_position = position;
  A.out_kept = out_kept;
  A.out_query = out_query;
  A.slots = slots;
  A.capacity = capacity;
  A.status = status;
  A.cache = (uint8_t *)cache;
  A.cache_stride = slot_cache_layout(h->M).bytes;
  A.slide = slide;
  A.out_trace = out_trace;
  // One token a session on the paired kernels with keyed drawers (of skewed sizes, or as the
  // environment asked at model creation): the step stops at the drawer selection and the
  // drawer-major scan (fbs_serve.hip) chooses the tokens.
  const bool deferred = h->serve_drawer_major && h->pair && !h->M.ham.heads &&
                        h->M.head != 1 && h->M.d % 32 == 0 && prompt_len == 1 && gen == 0 &&
                        !out_trace && sequences > 0 &&
                        (uint64_t)h->M.D * sequences < (1ull << 32);  // drawer-list indices
  hipStream_t st = (hipStream_t)stream;
  if (deferred) {
    int e = h->ensure_jobs(sequences, st);
    if (e) return e;
    A.job_query = h->job_query;
    A.job_flag = h->job_flag;
    A.job_best = h->job_best;
    A.drawer_count = h->drawer_count;
    A.drawer_list = h->drawer_list;
    A.list_stride = h->jobs_cap;
    A.items = h->items;
    A.item_count = h->item_count;
    A.item_cap = h->item_cap;
  }
  // The trace is recorded by the one-wavefront kernels.
  int rc = launch(h, A, st, false, out_trace != nullptr);
  if (rc || !deferred) return rc;
  ServeScan J{};
  J.items = h->items;
  J.item_count = h->item_count;
  J.item_cap = h->item_cap;
  J.n = sequences;
  J.gen = gen;
  J.job_query = h->job_query;
  J.job_flag = h->job_flag;
  J.job_best = h->job_best;
  J.drawer_count = h->drawer_count;
  J.drawer_list = h->drawer_list;
  J.list_stride = h->jobs_cap;
  J.out_tokens = out_reply;
  J.slots = slots;
  J.cache = (uint8_t *)cache;
  J.cache_stride = A.cache_stride;
  // The scan's wavefronts take the items in turn: two a SIMD, or one an item.
  uint32_t blocks = h->item_cap < 8 * h->cus ? h->item_cap : 8 * h->cus;
  blocks = blocks ? blocks : 1;
  const hipError_t e = launch_fbs_serve_scan(h->M, J, blocks, st);
  return e != hipSuccess ? hip_fail(e, "kernel launch") : 0;
}

extern "C" int uor_fbs_serve_slots_stream_async(
    uor_fbs_handle *h, const uint32_t *slots, uint32_t sequences, uint32_t capacity,
    const uint32_t *prompts, uint32_t prompt_len, uint32_t gen, uint32_t *out_reply, int64_t *state,
    int32_t *history, uint32_t *position, uint32_t *stream, int64_t *payloads, void *cache,
    uint32_t *out_kept, int32_t *out_query, int32_t *status, void *hip_stream) {
  if (!h || !slots || !prompts || !out_reply || !state || !history || !position || !status)
    return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a step needs at least one token");
  if (h->M.ham.heads && !stream)
    return fail(UOR_FBS_ERR_ARGUMENT, "a Hamming model's slots need their token streams");
  if (h->M.ham.slots && !payloads)
    return fail(UOR_FBS_ERR_ARGUMENT, "a Hamming model's typed reads need their payload caches");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = state;
  A.in_history = history;
  A.in_position = position;
  A.out_state = state;
  A.out_history = history;
  A.out_position = position;
  A.out_kept = out_kept;
  A.out_query = out_query;
  A.slots = slots;
  A.capacity = capacity;
  A.status = status;
  A.cache = (uint8_t *)cache;
  A.cache_stride = slot_cache_layout(h->M).bytes;
  if (h->M.ham.heads) {
    A.in_stream = stream;
    A.out_stream = stream;
    A.in_payloads = payloads;
    A.out_payloads = payloads;
  }
  return launch(h, A, (hipStream_t)hip_stream);
}

extern "C" int uor_fbs_decode(uor_fbs_handle *h, const uint32_t *prompts, uint32_t sequences,
                              uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                              const int64_t *in_state, const int32_t *in_history,
                              const uint32_t *in_position, int64_t *out_state,
                              int32_t *out_history, uint32_t *out_position) {
  if (!h || !prompts || !out_reply) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  if (sequences == 0) return 0;
  DeviceScope scope(h->device);
  const size_t sw = uor_fbs_state_words(h), hw = uor_fbs_history_words(h);
  DevBuf b;
  uint32_t *dp, *dr, *dip = nullptr, *dop = nullptr;
  int64_t *dis = nullptr, *dos = nullptr;
  int32_t *dih = nullptr, *doh = nullptr, *ds;
  int st;
  if ((st = b.in(&dp, prompts, (size_t)sequences * prompt_len)) ||
      (st = b.alloc(&dr, (size_t)sequences * (gen + 1))) || (st = b.alloc(&ds, sequences)) ||
      (st = b.in(&dis, in_state, sequences * sw)) || (st = b.in(&dih, in_history, sequences * hw)) ||
      (st = b.in(&dip, in_position, sequences)))
    return st;
  if (out_state && (st = b.alloc(&dos, sequences * sw))) return st;
  if (out_history && (st = b.alloc(&doh, sequences * hw))) return st;
  if (out_position && (st = b.alloc(&dop, sequences))) return st;
  if ((st = uor_fbs_decode_async(h, dp, sequences, prompt_len, gen, dr, dis, dih, dip, dos, doh,
                                 dop, ds, nullptr)))
    return st;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(sequences);
  if ((st = copy_out(status.data(), ds, sequences)) ||
      (st = copy_out(out_reply, dr, (size_t)sequences * (gen + 1))) ||
      (st = copy_out(out_state, dos, sequences * sw)) ||
      (st = copy_out(out_history, doh, sequences * hw)) ||
      (st = copy_out(out_position, dop, sequences)))
    return st;
  return first_status(status);
}

extern "C" uint64_t uor_fbs_stream_words(const uor_fbs_handle *h) {
  return h && h->M.ham.heads ? h->M.context : 0;
}
extern "C" uint64_t uor_fbs_payload_words(const uor_fbs_handle *h) {
  return h && h->M.ham.heads ? h->payload_words() : 0;
}

extern "C" int uor_fbs_decode_stream_async(
    uor_fbs_handle *h, const uint32_t *prompts, uint32_t sequences, uint32_t prompt_len,
    uint32_t gen, uint32_t *out_reply, const int64_t *in_state, const int32_t *in_history,
    const uint32_t *in_position, const uint32_t *in_stream, const int64_t *in_payloads,
    int64_t *out_state, int32_t *out_history, uint32_t *out_position, uint32_t *out_stream,
    int64_t *out_payloads, int32_t *status, void *stream) {
  if (!h || !prompts || !out_reply || !status) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  if (in_position && h->M.ham.heads && (!in_stream || (h->M.ham.slots && !in_payloads)))
    return fail(UOR_FBS_ERR_ARGUMENT, "a resumed session needs its token stream%s",
                h->M.ham.slots ? " and payload caches" : "");
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeDecode;
  A.n = sequences;
  A.len = prompt_len;
  A.gen = gen;
  A.tokens = prompts;
  A.out_tokens = out_reply;
  A.in_state = in_state;
  A.in_history = in_history;
  A.in_position = in_position;
  A.out_state = out_state;
  A.out_history = out_history;
  A.out_position = out_position;
  A.status = status;
  if (h->M.ham.heads) {
    A.in_stream = in_stream;
    A.out_stream = out_stream;
    A.in_payloads = h->M.ham.slots ? in_payloads : nullptr;
    A.out_payloads = h->M.ham.slots ? out_payloads : nullptr;
  }
  return launch(h, A, (hipStream_t)stream);
}

extern "C" int uor_fbs_decode_stream(uor_fbs_handle *h, const uint32_t *prompts, uint32_t sequences,
                                     uint32_t prompt_len, uint32_t gen, uint32_t *out_reply,
                                     const int64_t *in_state, const int32_t *in_history,
                                     const uint32_t *in_position, const uint32_t *in_stream,
                                     const int64_t *in_payloads, int64_t *out_state,
                                     int32_t *out_history, uint32_t *out_position,
                                     uint32_t *out_stream, int64_t *out_payloads) {
  if (!h || !prompts || !out_reply) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (prompt_len == 0) return fail(UOR_FBS_ERR_ARGUMENT, "a decode needs at least one prompt token");
  if (sequences == 0) return 0;
  DeviceScope scope(h->device);
  const size_t sw = uor_fbs_state_words(h), hw = uor_fbs_history_words(h);
  const size_t tw = uor_fbs_stream_words(h), pw = uor_fbs_payload_words(h);
  DevBuf b;
  uint32_t *dp, *dr, *dip = nullptr, *dop = nullptr, *dit = nullptr, *dot = nullptr;
  int64_t *dis = nullptr, *dos = nullptr, *dipl = nullptr, *dopl = nullptr;
  int32_t *dih = nullptr, *doh = nullptr, *ds;
  int st;
  if ((st = b.in(&dp, prompts, (size_t)sequences * prompt_len)) ||
      (st = b.alloc(&dr, (size_t)sequences * (gen + 1))) || (st = b.alloc(&ds, sequences)) ||
      (st = b.in(&dis, in_state, sequences * sw)) || (st = b.in(&dih, in_history, sequences * hw)) ||
      (st = b.in(&dip, in_position, sequences)) ||
      (tw && (st = b.in(&dit, in_stream, sequences * tw))) ||
      (pw && (st = b.in(&dipl, in_payloads, sequences * pw))))
    return st;
  if (out_state && (st = b.alloc(&dos, sequences * sw))) return st;
  if (out_history && (st = b.alloc(&doh, sequences * hw))) return st;
  if (out_position && (st = b.alloc(&dop, sequences))) return st;
  if (out_stream && tw && (st = b.alloc(&dot, sequences * tw))) return st;
  if (out_payloads && pw && (st = b.alloc(&dopl, sequences * pw))) return st;
  if ((st = uor_fbs_decode_stream_async(h, dp, sequences, prompt_len, gen, dr, dis, dih, dip, dit,
                                        dipl, dos, doh, dop, dot, dopl, ds, nullptr)))
    return st;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(sequences);
  if ((st = copy_out(status.data(), ds, sequences)) ||
      (st = copy_out(out_reply, dr, (size_t)sequences * (gen + 1))) ||
      (st = copy_out(out_state, dos, sequences * sw)) ||
      (st = copy_out(out_history, doh, sequences * hw)) ||
      (st = copy_out(out_position, dop, sequences)) ||
      (st = copy_out(out_stream, dot, sequences * tw)) ||
      (st = copy_out(out_payloads, dopl, sequences * pw)))
    return st;
  return first_status(status);
}

extern "C" int uor_fbs_score_async(uor_fbs_handle *h, const uint32_t *rows, uint64_t n_rows,
                                   uint32_t len, uint32_t *out_argmin, uint64_t *matches,
                                   int32_t *status, void *stream) {
  if (!h || !rows || !matches || !status) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  if (n_rows >= (1ull << 31)) return fail(UOR_FBS_ERR_ARGUMENT, "%llu rows: below 2^31 per call",
                                          (unsigned long long)n_rows);
  DeviceScope scope(h->device);
  RunArgs A{};
  A.mode = kModeScore;
  A.n = (uint32_t)n_rows;
  A.len = len;
  A.tokens = rows;
  A.out_tokens = out_argmin;
  A.matches = (unsigned long long *)matches;
  A.status = status;
  return launch(h, A, (hipStream_t)stream);
}

extern "C" int uor_fbs_score(uor_fbs_handle *h, const uint32_t *rows, uint64_t n_rows, uint32_t len,
                             uint32_t *out_argmin, uint64_t *out_matches) {
  if (!h || !rows || !out_matches) return fail(UOR_FBS_ERR_ARGUMENT, "null argument");
  *out_matches = 0;
  if (n_rows == 0 || len == 0) return 0;
  DeviceScope scope(h->device);
  size_t n = (size_t)n_rows * len;
  DevBuf b;
  uint32_t *dr, *da = nullptr;
  uint64_t *dm;
  int32_t *ds;
  int st;
  if ((st = b.in(&dr, rows, n)) || (st = b.alloc(&dm, 1)) || (st = b.alloc(&ds, n_rows))) return st;
  if (out_argmin && (st = b.alloc(&da, n))) return st;
  hipError_t e = hipMemset(dm, 0, sizeof(uint64_t));
  if (e != hipSuccess) return hip_fail(e, "hipMemset");
  if ((st = uor_fbs_score_async(h, dr, n_rows, len, da, dm, ds, nullptr))) return st;
  e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, "kernel");
  std::vector<int32_t> status(n_rows);
  if ((st = copy_out(status.data(), ds, n_rows)) || (st = copy_out(out_matches, dm, 1)) ||
      (st = copy_out(out_argmin, da, n)))
    return st;
  return first_status(status);
}
