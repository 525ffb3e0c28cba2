"""Seeded synthetic SpiralCore/FBS artifacts and prompts, written directly in integers.

The reference builds its synthetic trunks from floats through its exporter
(crates/uor-r4-integer/src/stack/synthetic.rs:101-162, format.rs:2327-2460). This generator
draws the served integers themselves from the reference's test LCG
(``x <- x * 6364136223846793005 + 1442695040888963407``, output ``x >> 33``,
synthetic.rs:12-23), so any shape BASELINE names can be produced without a float path:

- writer table: i16 uniform in [-2^15, 2^15) (or int8 codes uniform in [-128, 128));
- route words: atom uniform below the input blocks, state uniform below 64, codes from AXES;
- grid codes: gains about [0.5, 2), taps about +-[2^-5, 2^-1] with a few zeros;
- biases: i32 at exponent -16 in about +-0.25; decay offsets spread over the 16 rates;
- RMSNorm epsilon 1e-5 as ``round(1e-5 * 2^48) * 2^-48`` (format.rs:2572-2582).

Drawers beyond the reference's 256 root-pair cells get seeded Q12 keys and Zipf-skewed CSR
membership (sizes proportional to 1/(j+1)^s, capped, every token in exactly one drawer,
members ascending).
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

from . import tables

LCG_A = 6364136223846793005
LCG_C = 1442695040888963407
MASK64 = (1 << 64) - 1


def _lcg_jump(k: int) -> tuple[int, int]:
    """(A, C) with x_{n+k} = A x_n + C mod 2^64."""
    a, c = 1, 0
    base_a, base_c = LCG_A, LCG_C
    while k:
        if k & 1:
            a, c = (a * base_a) & MASK64, (c * base_a + base_c) & MASK64
        base_a, base_c = (base_a * base_a) & MASK64, (base_c * base_a + base_c) & MASK64
        k >>= 1
    return a, c


class Lcg:
    """The reference's test generator; ``take(n)`` returns the next n outputs at once."""

    BLOCK = 1 << 16

    def __init__(self, seed: int):
        self.x = seed & MASK64
        mults = np.empty(self.BLOCK, dtype=np.uint64)
        adds = np.empty(self.BLOCK, dtype=np.uint64)
        for k in range(self.BLOCK):  # x_{n+k+1} = A_{k+1} x_n + C_{k+1}
            a, c = _lcg_jump(k + 1)
            mults[k], adds[k] = a, c
        self._mults, self._adds = mults, adds
        self._block_a, self._block_c = _lcg_jump(self.BLOCK)

    def next(self) -> int:
        self.x = (self.x * LCG_A + LCG_C) & MASK64
        return self.x >> 33

    def take(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint64)
        done = 0
        with np.errstate(over="ignore"):
            while done < n:
                k = min(self.BLOCK, n - done)
                xs = self._mults[:k] * np.uint64(self.x) + self._adds[:k]
                out[done:done + k] = xs >> np.uint64(33)
                self.x = int(xs[k - 1])
                done += k
        return out


_LCG_CACHE: dict[int, Lcg] = {}


def lcg(seed: int) -> Lcg:
    """A fresh generator at ``seed`` (the jump tables are shared)."""
    proto = _LCG_CACHE.get(0)
    if proto is None:
        proto = _LCG_CACHE[0] = Lcg(0)
    g = Lcg.__new__(Lcg)
    g.__dict__.update(proto.__dict__)
    g.x = seed & MASK64
    return g


PLACE_STOP, PLACE_ARM, PLACE_OPEN = 1, 2, 4  # fbs_snapshot.rs:2762-2766
PLACE_MARK_MAX = 16  # ids a marker list may hold on this build


@dataclass(frozen=True)
class PlaceMarks:
    """The ids that frame a conversation for the place read (PlaceMarks, fbs_snapshot.rs:2725-
    2732): the document's start and end marks, the turn separator and the three role markers."""

    bos: int
    eos: int
    sep: tuple
    system: tuple
    user: tuple
    assistant: tuple

    def check(self, vocab: int) -> str | None:
        """PlaceMarks::check (fbs_snapshot.rs:2741-2761): the reason marks are refused, or None.
        This build also refuses a marker list over PLACE_MARK_MAX ids."""
        lists = (self.sep, self.system, self.user, self.assistant)
        if any(not 0 <= int(i) < vocab for i in (self.bos, self.eos, *[x for l in lists for x in l])):
            return "a place read's mark is outside the vocabulary"
        if not self.sep or not self.user or not self.assistant:
            return "a place read needs a separator, a user marker and an assistant marker"
        if self.bos == self.eos:
            return "a place read's start mark and end mark are one token"
        roles = (tuple(self.system), tuple(self.user), tuple(self.assistant))
        for i, a in enumerate(roles):
            for j, b in enumerate(roles):
                if i != j and b and len(a) >= len(b) and a[len(a) - len(b):] == b:
                    return "one of a place read's role markers ends with another"
        if any(len(l) > PLACE_MARK_MAX for l in lists):
            return f"a place read's marker list holds more than {PLACE_MARK_MAX} ids on this build"
        return None

    def to_json(self) -> dict:
        return dict(bos=int(self.bos), eos=int(self.eos), sep=[int(x) for x in self.sep],
                    system=[int(x) for x in self.system], user=[int(x) for x in self.user],
                    assistant=[int(x) for x in self.assistant])


@dataclass(frozen=True)
class HammingSpec:
    """Seeded Hamming reads of a lut-stack/6 stack (StackHamming, stack/format.rs:229-292)."""

    heads: int = 4
    depths: tuple = (1,)          # after these many layers; the layer count is the readout read
    kept: int = 16                # HAMMING_KEPT (format.rs:61)
    copy_key: int = 1
    copy_keys: tuple | None = None
    copy_latest: bool = False
    copy_longest: tuple | None = None   # the reply marker (two ids)
    asks: tuple | None = None     # one flag per read
    carry_rows: int = 0           # the readout read's question carry reach
    typed: bool = True            # nonzero type weights w_y (type heads served)
    margin_bits: tuple = (2, 12)  # margins drawn in this many bits (at Q16)
    rule: int = 0xFFFFFFFF        # the copy rule served (UOR_FBS_COPY_*; default: the artifact's)
    place: PlaceMarks | None = None  # the readout read's place read (its read must ask)


@dataclass(frozen=True)
class Spec:
    """Shape of a synthetic artifact. Zero extension fields mean the reference's rule."""

    vocab: int
    width: int
    mlp: int
    layers: int
    context: int
    kept: int                 # the reference's kept cells (and the default probes)
    window: int = 3           # W prior rows of the causal window (reference 3)
    drawers: int = 0          # 0: the 256 root-pair cells, token t in cell t mod 256
    probes: int = 0           # 0: kept
    zipf_drawers: float = 0.0 # > 0: Zipf(s) drawer sizes over CSR members
    max_drawer: int = 0       # cap on a drawer's size (0: none)
    table: str = "i16"        # "i16" or "i8"
    table_shift: int = 8      # i8 row value at Q12 = code << shift
    head: int = 0             # 0 writer, 1 whole-table nearest
    raw_gates: bool = True
    raw_transition: bool = True
    gain_fields: tuple = (63, 64)
    tap_fields: tuple = (59, 62)
    bias_range: int = 1 << 14
    hamming: HammingSpec | None = None

    @property
    def reference_shape(self) -> bool:
        return (self.window == 3 and self.drawers in (0, 256) and self.zipf_drawers == 0
                and self.table == "i16" and self.probes in (0, self.kept))


@dataclass
class HammingRead:
    """One read's integers (HammingReadImage, stack/hamming.rs:25-40)."""

    depth: int
    query_rotation: np.ndarray  # width i32 at 2^-24
    key_rotation: np.ndarray
    value_rotation: np.ndarray
    margin: np.ndarray          # heads i32 at Q16, positive
    weight: np.ndarray          # 2 * width i32 at 2^-24: w_c then w_y
    ask: np.ndarray | None = None    # vocab * width i16 Q12
    carry: np.ndarray | None = None  # vocab i32 Q16


@dataclass
class Layer:
    rec_gain: np.ndarray
    mlp_gain: np.ndarray
    maps: dict            # name -> (atoms u16 [blocks], codes u8 [blocks*8])
    taps: np.ndarray      # 4 * width (the reference's four taps)
    wide_taps: np.ndarray | None  # (W+1) * width when W != 3
    conv_bias: np.ndarray
    gate_bias: np.ndarray
    decay_offset: np.ndarray


@dataclass
class Artifact:
    spec: Spec
    seed: int
    layers: list
    final_gain: np.ndarray
    writer_table: np.ndarray          # vocab * width i16 (always present: the i8 table widened)
    table_i8: np.ndarray | None
    eps_mantissa: int
    eps_exp: int
    roots_q12: np.ndarray = field(default_factory=tables.roots_q12)
    icosian: np.ndarray = field(default_factory=tables.icosian_coefficients)
    keep_q31: np.ndarray = field(default_factory=tables.keep_q31)
    drawer_keys: np.ndarray | None = None
    drawer_offsets: np.ndarray | None = None
    drawer_members: np.ndarray | None = None
    # SHA-256 (hex) of the container bytes a served artifact was read from (format.rs:1493);
    # None for a generated one.
    sha256: str | None = None
    # A container with a turn memory (`memory` record, lut-stack/7 and /8): the plain step does not
    # apply it, but it rules out the context slide (session.rs:1146-1151).
    turn_memory: bool = False
    # The Hamming reads (lut-stack/6): the record's fields and one HammingRead per depth.
    hamming: HammingSpec | None = None
    hamming_reads: list | None = None
    # The place read's class table (vocab i16: PLACE_STOP | PLACE_ARM | PLACE_OPEN), with
    # hamming.place.
    hamming_place: np.ndarray | None = None

    @property
    def window(self) -> int:
        return self.spec.window

    @property
    def probes(self) -> int:
        return self.spec.probes or self.spec.kept

    @property
    def drawers(self) -> int:
        return self.spec.drawers or 256

    def drawer_sizes(self) -> np.ndarray:
        if self.drawer_offsets is not None:
            return np.diff(self.drawer_offsets.astype(np.int64))
        d = self.drawers
        v = self.spec.vocab
        return np.array([(v - c + d - 1) // d for c in range(d)], dtype=np.int64)


def _grid_codes(g: Lcg, n: int, fields: tuple, signed: bool, zero_every: int = 0) -> np.ndarray:
    r = g.take(3 * n).reshape(3, n)
    lo, hi = fields
    f = lo + (r[0] % np.uint64(hi - lo + 1)).astype(np.int64)
    mant = (r[1] % np.uint64(16)).astype(np.int64)
    code = (f << 4) | mant
    if signed:
        code = np.where(r[2] & np.uint64(1), -code, code)
    if zero_every:
        code = np.where((r[2] >> np.uint64(1)) % np.uint64(zero_every) == 0, 0, code)
    return code.astype(np.int16)


def _uniform_i32(g: Lcg, n: int, half: int) -> np.ndarray:
    return ((g.take(n) % np.uint64(2 * half + 1)).astype(np.int64) - half).astype(np.int32)


def _route(g: Lcg, in_dim: int, out_dim: int):
    in_blocks, out_blocks = in_dim // 8, out_dim // 8
    r = g.take(2 * out_blocks).reshape(2, out_blocks)
    atoms = (r[0] % np.uint64(in_blocks)).astype(np.uint16)
    states = (r[1] % np.uint64(64)).astype(np.int64)
    codes = tables.AXES.reshape(64, 8)[states].reshape(-1).astype(np.uint8)
    return atoms, codes


def zipf_sizes(total: int, n: int, s: float, cap: int) -> np.ndarray:
    """Integer sizes summing to ``total``, proportional to 1/(j+1)^s, each in [1, cap]."""
    w = 1.0 / np.arange(1, n + 1, dtype=np.float64) ** s
    cap = cap or total
    if cap * n < total:
        raise ValueError("drawer cap too small for the vocabulary")
    sizes = np.zeros(n)
    fixed = np.zeros(n, dtype=bool)
    remaining = float(total - n)  # every drawer holds at least one token
    for _ in range(64):
        free = ~fixed
        share = w * free
        share = share / share.sum() * remaining
        over = free & (share > cap - 1)
        if not over.any():
            sizes = np.where(fixed, cap - 1, share)
            break
        fixed |= over
        remaining = float(total - n) - (cap - 1) * fixed.sum()
    base = np.floor(sizes).astype(np.int64)
    left = (total - n) - int(base.sum())
    order = np.argsort(-(sizes - base), kind="stable")
    for j in order:
        if left <= 0:
            break
        if base[j] + 1 <= cap - 1:
            base[j] += 1
            left -= 1
    out = base + 1
    assert out.sum() == total and out.max() <= cap and out.min() >= 1
    return out


def make_artifact(spec: Spec, seed: int) -> Artifact:
    """A seeded artifact of ``spec``: every table drawn in a fixed order from one LCG."""
    g = lcg(seed)
    d, m = spec.width, spec.mlp
    lanes = d // 4
    gate_rows = lanes + d
    if d % 32 or m % 32:
        raise ValueError("width and mlp must be multiples of 32 (format.rs:724-729)")
    layers = []
    for _ in range(spec.layers):
        rec_gain = _grid_codes(g, d, spec.gain_fields, False)
        mlp_gain = _grid_codes(g, d, spec.gain_fields, False)
        maps = {}
        for name, i, o in (("rec_in", d, 2 * d), ("rec_gate", d, gate_rows), ("rec_out", d, d),
                           ("mlp_gate", d, m), ("mlp_up", d, m), ("mlp_down", m, d)):
            maps[name] = _route(g, i, o)
        ntaps = spec.window + 1
        all_taps = _grid_codes(g, ntaps * d, spec.tap_fields, True, zero_every=16)
        taps = all_taps[: 4 * d].copy() if ntaps >= 4 else np.concatenate(
            [all_taps, np.zeros((4 - ntaps) * d, np.int16)])
        wide = None if spec.window == 3 else all_taps
        conv_bias = _uniform_i32(g, d, spec.bias_range)
        gate_bias = _uniform_i32(g, gate_rows, spec.bias_range)
        jitter = _uniform_i32(g, lanes, 1 << 11).astype(np.int64)
        decay = (np.arange(lanes, dtype=np.int64) * 65536) // lanes + 2048 + jitter
        layers.append(Layer(rec_gain, mlp_gain, maps, taps, wide, conv_bias, gate_bias,
                            decay.astype(np.int32)))
    final_gain = _grid_codes(g, d, spec.gain_fields, False)
    n = spec.vocab * d
    if spec.table == "i8":
        table_i8 = ((g.take(n) % np.uint64(256)).astype(np.int64) - 128).astype(np.int8)
        writer = (table_i8.astype(np.int32) << spec.table_shift).astype(np.int16)
    else:
        table_i8 = None
        writer = ((g.take(n) % np.uint64(65536)).astype(np.int64) - 32768).astype(np.int16)
    art = Artifact(spec=spec, seed=seed, layers=layers, final_gain=final_gain,
                   writer_table=writer, table_i8=table_i8,
                   eps_mantissa=int(round(1e-5 * 2.0 ** 48)), eps_exp=-48)
    D = spec.drawers or 256
    if D != 256:
        art.drawer_keys = _uniform_i32(g, D * 16, 8192)
    if spec.zipf_drawers > 0:
        sizes = zipf_sizes(spec.vocab, D, spec.zipf_drawers, spec.max_drawer)
        perm = np.argsort(g.take(spec.vocab), kind="stable").astype(np.uint32)
        offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint32)
        members = np.empty(spec.vocab, dtype=np.uint32)
        for c in range(D):
            members[offsets[c]:offsets[c + 1]] = np.sort(perm[offsets[c]:offsets[c + 1]])
        art.drawer_offsets, art.drawer_members = offsets, members
    if spec.hamming is not None:
        art.hamming, art.hamming_reads = spec.hamming, _hamming_reads(g, spec)
        if spec.hamming.place is not None:
            art.hamming_place = place_classes(g, spec.vocab, spec.hamming.place)
    return art


def place_classes(g: Lcg, vocab: int, marks: PlaceMarks) -> np.ndarray:
    """A seeded class table: each entry stops with probability 1/8, arms with 1/16 and opens
    with 1/8 (independently); the marks themselves have no class."""
    r = g.take(vocab)
    cls = (np.where(r % np.uint64(8) == 0, PLACE_STOP, 0) | np.where((r >> np.uint64(3)) % np.uint64(16) == 0, PLACE_ARM, 0)
           | np.where((r >> np.uint64(7)) % np.uint64(8) == 0, PLACE_OPEN, 0)).astype(np.int16)
    for i in (marks.bos, marks.eos, *marks.sep, *marks.system, *marks.user, *marks.assistant):
        cls[int(i)] = 0
    return cls


def _hamming_reads(g: Lcg, spec: Spec) -> list:
    """Seeded reads for spec.hamming, drawn after every other table (so an artifact without reads
    is unchanged): raw rotations in +-2^24 (about +-1 at 2^-24), margins between the record's
    bit bounds at Q16, weights in +-2^24, and ask tables in +-2^12 at Q12 with carry gains in
    +-2^16 at Q16."""
    h, d, V = spec.hamming, spec.width, spec.vocab
    if h.heads < 2 or h.heads % 2 or d % h.heads or (d // h.heads) % 4 or d // h.heads > 64:
        raise ValueError("heads: even, at least 2, dividing the width into 4..64-coordinate heads")
    reads = []
    lo, hi = h.margin_bits
    for r, depth in enumerate(h.depths):
        rot = [_uniform_i32(g, d, 1 << 24) for _ in range(3)]
        margin = (((g.take(h.heads) % np.uint64((hi - lo) * 65536 + 1)).astype(np.int64)
                   + lo * 65536)).astype(np.int32)
        margin = np.maximum(margin, 1)
        weight = _uniform_i32(g, 2 * d, 1 << 24)
        if not h.typed:
            weight[d:] = 0
        asks = h.asks is not None and h.asks[r]
        ask = _uniform_i32(g, V * d, 1 << 12).astype(np.int16) if asks else None
        last = r + 1 == len(h.depths)
        carry = _uniform_i32(g, V, 1 << 16) if (asks and last and h.carry_rows) else None
        reads.append(HammingRead(depth, rot[0], rot[1], rot[2], margin, weight, ask, carry))
    return reads


def hamming_reads(spec: Spec, hamming: HammingSpec, seed: int) -> list:
    """Seeded reads for `hamming` over `spec`'s shape, drawn on their own (to add to an artifact
    read from a container, uorlut.add_hamming)."""
    return _hamming_reads(lcg(seed), replace(spec, hamming=hamming))


def uniform_prompts(vocab: int, count: int, length: int, seed: int) -> np.ndarray:
    """``count`` rows of ``length`` ids ``next() % vocab`` (tests/parity.rs:25-34's sequences)."""
    return (lcg(seed).take(count * length) % np.uint64(vocab)).astype(np.uint32).reshape(count, length)


def zipf_prompts(vocab: int, count: int, length: int, seed: int, s: float = 1.1) -> np.ndarray:
    """Zipf(s) ids by inverse CDF over an integer cumulative table (2^31 scale): id = rank."""
    w = 1.0 / np.arange(1, vocab + 1, dtype=np.float64) ** s
    cum = np.floor(np.cumsum(w) / w.sum() * float(1 << 31)).astype(np.int64)
    cum[-1] = 1 << 31
    u = lcg(seed).take(count * length).astype(np.int64)  # 31-bit outputs
    ids = np.searchsorted(cum, u, side="right")
    return np.minimum(ids, vocab - 1).astype(np.uint32).reshape(count, length)


# The reference's own synthetic shapes (synthetic.rs:44-99) and BASELINE's configs.
SMALL = Spec(vocab=256, width=32, mlp=32, layers=2, context=8, kept=2)
NON_SQUARE = Spec(vocab=512, width=64, mlp=96, layers=3, context=16, kept=8)
TINY = Spec(vocab=512, width=64, mlp=64, layers=1, context=8, kept=8)

CONFIGS = {
    # C1/C2: width 128, vocab 8192, window 8, 64 drawers probing 4 (uniform membership).
    "c1": Spec(vocab=8192, width=128, mlp=192, layers=6, context=512, kept=4, window=8,
               drawers=64, probes=4),
    "c2": Spec(vocab=8192, width=128, mlp=192, layers=6, context=1024, kept=4, window=8,
               drawers=64, probes=4),
    # C3/C4: width 256, vocab 32768, window 16, 256 Zipf drawers (max 512) probing 8.
    "c3": Spec(vocab=32768, width=256, mlp=384, layers=6, context=2048, kept=8, window=16,
               drawers=256, probes=8, zipf_drawers=1.1, max_drawer=512),
    "c4": Spec(vocab=32768, width=256, mlp=384, layers=6, context=128, kept=8, window=16,
               drawers=256, probes=8, zipf_drawers=1.1, max_drawer=512),
    # C5: width 512, vocab 65536, window 32, 1024 Zipf drawers (max 1024) probing 16, int8.
    "c5": Spec(vocab=65536, width=512, mlp=768, layers=6, context=8192, kept=16, window=32,
               drawers=1024, probes=16, zipf_drawers=1.1, max_drawer=1024, table="i8"),
}


def reference_twin(spec: Spec) -> Spec:
    """The reference-exact twin of a config: 256 root-pair cells (t mod 256), window 3,
    i16 table, vocab capped at 8192 (format.rs:436-439)."""
    return replace(spec, vocab=min(spec.vocab, 8192), window=3, drawers=0, probes=0,
                   zipf_drawers=0.0, max_drawer=0, table="i16", kept=spec.probes or spec.kept)
