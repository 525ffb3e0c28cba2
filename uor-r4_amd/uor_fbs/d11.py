"""The discrete M1 container (``uor-r4.lut-discrete/1`` and the 19-table
``uor-r4.lut-discrete-trunk/1``) and its GPU row scorer.

Mirrors ``IntegerDiscreteModel`` (crates/uor-r4-integer/src/discrete_d11.rs:687-1995):
``from_bytes`` (:931-1278) parses and checks a ``UORLUT01`` container, ``evaluate_prefix``
(:1761) reads a causal prefix into one orbit root per block and ranks the writer's tokens, and
``observe_target`` (:1892-1995) adds the target's hinges and losses. ``score_rows`` is the panel
scorer of docs/labs/m1-d11-artifact-scorer (``d11_score_rows``, ``DeviceScorer::score``,
device.rs:120-210): every (prefix, target) row in one launch, one record per row.

Parsing and the container checks run here on the host, as the reference's loader does; every
evaluation runs in the HIP library (``uor_d11_*`` in include/uor_d11.h). There is no host
evaluation path. ``build_container`` writes containers in the reference's layout (the test
builder of discrete_d11.rs:2006-2086) and ``synthetic`` makes M1-shaped models.
"""

from __future__ import annotations

import ctypes as C
import json
from dataclasses import asdict, dataclass, field

import numpy as np

from . import tables

MAGIC = b"UORLUT01"
SCHEMA = "uor-r4.lut-discrete/1"
TRUNK_SCHEMA = "uor-r4.lut-discrete-trunk/1"
SNAPSHOT_SCHEMA = "uor-r4.discrete-spiralcore-fbs/2"
OPERATOR_KAPPA = "blake3:a0ea3a10dd10c5f4856b0d881d33d94c3293bad0e68bd07a47918e2bb82c819b"
COMPOSITION_KAPPA = "blake3:f2986c8e68dcb30a9cb511a42547179a87b66ef212a87b728765d03e70e640b0"
ALIGN = 64
MAX_HEADER = 64 << 20
MAX_CONTEXT = 243
MAX_KEPT = 8
MAX_SWEEPS = 5
EDGE_TYPES = 5
READ_MODES = {"route": 0, "flock": 1, "relation": 2}
POLICIES = {"nearest_address_margin_v1": 0, "occupied_cell_rank_hinge_v1": 1}
# The 15 trunk sections after the four base tables, in container order (discrete_d11.rs:1196-1260).
TRUNK_SPARSE = (
    "read_table", "rec_table", "read_rec_table", "rec_shuf_table", "read_rec_shuf_table",
    "rec_unit_table", "read_rec_unit_table", "query_table", "query_read_table", "query_rec_table",
    "query_rec_shuf_table", "query_rec_unit_table",
)
TRUNK_SECTIONS = ("step_candidates", "norm_candidates", "unigram") + TRUNK_SPARSE

# Row status codes of the scorer (the reference kernel's, kernel_core.h:33-42).
STATUS = {0: "ok", 1: "prefix length must be in 1..=context", 2: "prefix token ID outside vocabulary",
          3: "row plan invalid", 4: "block outside the SpiralCore orbit",
          5: "route did not reach an atom leaf", 6: "writer admitted zero tokens", 7: "shape",
          8: "target token ID outside vocabulary"}


class DiscreteError(ValueError):
    """A refused container or prefix (the reference's ``StackError::invalid``)."""


@dataclass
class Shape:
    """``DiscreteLutShape`` (discrete_d11.rs:307-321)."""
    vocabulary: int
    blocks: int
    context: int
    kept_cells: int
    stages: int
    read_mode: str = "route"
    read_kept: int = 0
    read_sweeps: int = 0
    objective_policy: str = "nearest_address_margin_v1"
    read_initialization: str = "zero_gates_v1"
    seed: int = 7
    epoch: int = 0


@dataclass
class Trunk:
    """The trunk sections: 64 step and 4 norm candidates, the unigram table (its first word the
    global best token) and twelve sparse (key, token, count) triple tables."""
    step_candidates: np.ndarray
    norm_candidates: np.ndarray
    unigram: np.ndarray
    sparse: dict = field(default_factory=dict)   # name -> (n, 3) uint32


@dataclass
class Artifact:
    shape: Shape
    table: np.ndarray           # (vocab, blocks, 8) int32, every block an orbit root
    cells: np.ndarray           # (vocab,) uint32
    routes: np.ndarray          # (blocks * stages,) uint32
    gates: np.ndarray           # (blocks * stages [+ stages * 5],) int32
    trunk: Trunk | None = None


def expected_stages(context: int) -> int | None:
    """1 + the number of spans 3, 9, 27, ... within the context (discrete_d11.rs:712-723)."""
    if not 1 <= context <= MAX_CONTEXT:
        return None
    stages, span = 1, 3
    while span <= context:
        stages += 1
        span *= 3
    return stages


def plan_nodes(length: int) -> int:
    """build_row_plan's node count (discrete_d11.rs:813-884): every atom, and a node for each
    merge of the frontier's last three nodes while they share a level."""
    levels, count = [], 0
    for _ in range(length):
        levels.append(0)
        count += 1
        while len(levels) >= 3 and levels[-1] == levels[-2] == levels[-3]:
            levels[-3:] = [levels[-1] + 1]
            count += 1
    return count


def root_ids(table: np.ndarray) -> np.ndarray:
    """Orbit root of every 8-block (-1 where a block is none of the 16)."""
    t = np.asarray(table, np.int64).reshape(-1, 8)
    eq = (t[:, None, :] == tables.ROOTS[None, :, :].astype(np.int64)).all(-1)
    out = np.where(eq.any(1), eq.argmax(1), -1)
    return out.reshape(np.asarray(table).shape[:-1])


def endpoint_cells(table: np.ndarray) -> np.ndarray:
    r = root_ids(table)
    return ((r[:, 0] << 4) + r[:, -1]).astype(np.uint32)


# ---------------------------------------------------------------------------------------------
# Container writing and reading.

def _section(blob: bytearray, data: bytes) -> dict:
    blob.extend(b"\0" * ((ALIGN - len(blob) % ALIGN) % ALIGN))
    span = {"offset": len(blob), "bytes": len(data)}
    blob.extend(data)
    return span


def build_container(shape: Shape, table, routes, gates, trunk: Trunk | None = None,
                    cells=None) -> bytes:
    """A ``UORLUT01`` discrete container in the reference's layout: magic, u64 header length,
    the JSON header, zero padding to 64 bytes, then each section 64-byte aligned."""
    table = np.ascontiguousarray(table, np.int32)
    cells = endpoint_cells(table) if cells is None else np.asarray(cells, np.uint32)
    blob = bytearray()
    specs = []

    def push(name, kind, arr):
        arr = np.ascontiguousarray(arr, "<i4" if kind == "i32" else "<u4").reshape(-1)
        specs.append({"name": name, "kind": kind, "len": int(arr.size),
                      "span": _section(blob, arr.tobytes())})

    push("discrete.table", "i32", table)
    push("discrete.cells", "u32", cells)
    push("discrete.routes", "u32", routes)
    push("discrete.gates", "i32", gates)
    if trunk is not None:
        push("discrete.trunk.step_candidates", "u32", trunk.step_candidates)
        push("discrete.trunk.norm_candidates", "u32", trunk.norm_candidates)
        push("discrete.trunk.unigram", "u32", trunk.unigram)
        for name in TRUNK_SPARSE:
            push("discrete.trunk." + name, "u32",
                 trunk.sparse.get(name, np.zeros((0, 3), np.uint32)))
    header = {
        "schema": TRUNK_SCHEMA if trunk is not None else SCHEMA,
        "shape": asdict(shape), "matrices": [], "tables": specs,
        "source": {"snapshot_schema": SNAPSHOT_SCHEMA, "snapshot_sha256": "00" * 32,
                   "operator_kappa": OPERATOR_KAPPA, "composition_kappa": COMPOSITION_KAPPA,
                   "kernel_sha256": "11" * 32, "source_sha256": "22" * 32,
                   "geometry_sha256": "33" * 32},
    }
    js = json.dumps(header, separators=(",", ":")).encode()
    out = bytearray(MAGIC + len(js).to_bytes(8, "little") + js)
    out.extend(b"\0" * ((ALIGN - len(out) % ALIGN) % ALIGN))
    out.extend(blob)
    return bytes(out)


def parse_container(data: bytes) -> Artifact:
    """The checks of ``from_bytes`` (discrete_d11.rs:931-1278), in its order; DiscreteError on
    the first that fails."""
    if len(data) < 16 or data[:8] != MAGIC:
        raise DiscreteError("missing UORLUT01 magic")
    hlen = int.from_bytes(data[8:16], "little")
    if hlen > MAX_HEADER or 16 + hlen > len(data):
        raise DiscreteError("UORLUT01 header length out of bounds")
    try:
        header = json.loads(data[16:16 + hlen])
        schema, shape_d, tabs, source = (header["schema"], header["shape"], header["tables"],
                                         header["source"])
        matrices = header["matrices"]
        shape = Shape(**{k: shape_d[k] for k in Shape.__dataclass_fields__})
    except (ValueError, KeyError, TypeError) as e:
        raise DiscreteError(f"header: {e}") from None
    if schema not in (SCHEMA, TRUNK_SCHEMA):
        raise DiscreteError("discrete UORLUT01 artifact requires schema uor-r4.lut-discrete/1 "
                            "or uor-r4.lut-discrete-trunk/1")
    is_trunk = schema == TRUNK_SCHEMA
    if matrices:
        raise DiscreteError("discrete UORLUT01 artifact requires empty matrices")
    if (source.get("snapshot_schema") != SNAPSHOT_SCHEMA
            or source.get("operator_kappa") != OPERATOR_KAPPA
            or source.get("composition_kappa") != COMPOSITION_KAPPA):
        raise DiscreteError("discrete UORLUT01 snapshot_schema or geometry kappa mismatch")
    unaligned = 16 + hlen
    start = unaligned + (ALIGN - unaligned % ALIGN) % ALIGN
    if start > len(data) or any(data[unaligned:start]):
        raise DiscreteError("UORLUT01 header padding is missing or non-zero")
    body = data[start:]
    s = shape
    if (not 2 <= s.vocabulary <= 8192 or not 2 <= s.blocks <= 16
            or not 1 <= s.context <= MAX_CONTEXT or not 1 <= s.kept_cells <= 16
            or s.kept_cells > s.vocabulary or expected_stages(s.context) != s.stages):
        raise DiscreteError("inconsistent or unsupported discrete shape")
    mode = s.read_mode
    if not ((mode == "route" and s.read_kept == 0 and s.read_sweeps == 0)
            or (mode == "flock" and 1 <= s.read_kept <= MAX_KEPT and s.read_sweeps == 0)
            or (mode == "relation" and 1 <= s.read_kept <= MAX_KEPT
                and 1 <= s.read_sweeps <= MAX_SWEEPS)):
        raise DiscreteError("unsupported discrete read mode or parameters")
    if s.objective_policy not in POLICIES:
        raise DiscreteError("unsupported discrete objective policy")
    if not (s.read_initialization == "zero_gates_v1"
            or (s.read_initialization == "active_leaf_v1" and mode != "route")):
        raise DiscreteError("unsupported discrete read initialization")
    if (not is_trunk and len(tabs) != 4) or (is_trunk and (len(tabs) != 19 or s.blocks != 4)):
        raise DiscreteError("discrete UORLUT01 requires 4 tables (uor-r4.lut-discrete/1) or 19 "
                            "tables with 4 blocks (uor-r4.lut-discrete-trunk/1)")
    if is_trunk:
        prev_end = 0
        for t in tabs:
            o, n = int(t["span"]["offset"]), int(t["span"]["bytes"])
            end = o + n
            if (o % ALIGN or o < prev_end or o - prev_end >= ALIGN or end > len(body)
                    or any(body[prev_end:o])):
                raise DiscreteError("discrete UORLUT01 section ordering, alignment gap, or "
                                    "zero-padding invalid")
            prev_end = end
        if prev_end != len(body):
            raise DiscreteError("discrete UORLUT01 has unexpected trailing bytes")

    def read(name, kind, length):
        t = next((t for t in tabs if t["name"] == name), None)
        if t is None:
            raise DiscreteError(f"missing table {name}")
        if t["kind"] != kind or t["len"] != length:
            raise DiscreteError(f"table {name} kind or length mismatch")
        o, n = int(t["span"]["offset"]), int(t["span"]["bytes"])
        if o % ALIGN or n != 4 * length:
            raise DiscreteError(f"table {name} alignment or byte span mismatch")
        if o + n > len(body):
            raise DiscreteError(f"table {name} span out of bounds")
        return np.frombuffer(body, "<i4" if kind == "i32" else "<u4", length, o)

    V, B, S = s.vocabulary, s.blocks, s.stages
    base = B * S
    total = base + EDGE_TYPES * S if mode == "relation" else base
    table = read("discrete.table", "i32", V * B * 8).astype(np.int32).reshape(V, B, 8)
    cells = read("discrete.cells", "u32", V).astype(np.uint32)
    routes = read("discrete.routes", "u32", base).astype(np.uint32)
    gates = read("discrete.gates", "i32", total).astype(np.int32)
    if (routes >= 64).any():
        raise DiscreteError("discrete.routes contains action index >= 64")
    if ((gates < -1) | (gates > 1)).any():
        raise DiscreteError("discrete.gates contains trit outside -1..=1")
    roots = root_ids(table)
    for tok in range(V):  # the reference checks token by token: orbit first, then the cell
        if (roots[tok] < 0).any():
            raise DiscreteError("discrete.table block is outside the 16-root SpiralCore orbit")
        if cells[tok] != (int(roots[tok, 0]) << 4) + int(roots[tok, -1]):
            raise DiscreteError("discrete.cells entry disagrees with discrete.table endpoint roots")
    trunk = None
    if is_trunk:
        def read_any(idx, name):
            t = tabs[idx]
            if t["name"] != "discrete.trunk." + name or t["kind"] != "u32":
                raise DiscreteError(f"trunk table discrete.trunk.{name} name or kind mismatch")
            o, n = int(t["span"]["offset"]), int(t["span"]["bytes"])
            if o % ALIGN or n != 4 * int(t["len"]):
                raise DiscreteError(f"trunk table discrete.trunk.{name} alignment or byte span mismatch")
            if o + n > len(body):
                raise DiscreteError(f"trunk table discrete.trunk.{name} out of bounds")
            return np.frombuffer(body, "<u4", int(t["len"]), o).astype(np.uint32)
        step = read_any(4, "step_candidates")
        if len(step) != 64 or (step >= 16).any():
            raise DiscreteError("discrete.trunk.step_candidates requires 64 candidates in 0..16")
        norm = read_any(5, "norm_candidates")
        if len(norm) != 4 or (norm >= 16).any():
            raise DiscreteError("discrete.trunk.norm_candidates requires 4 candidates in 0..16")
        uni = read_any(6, "unigram")
        if len(uni) != 1 + V or uni[0] >= V or not uni[1:].any():
            raise DiscreteError("discrete.trunk.unigram length, best_global, or counts invalid")
        sparse = {}
        for i, name in enumerate(TRUNK_SPARSE):
            w = read_any(7 + i, name)
            if len(w) % 3:
                raise DiscreteError("sparse trunk count table word length must be a multiple of 3")
            tri = w.reshape(-1, 3)
            if ((tri[:, 1] >= V) | (tri[:, 2] == 0)).any():
                raise DiscreteError("sparse trunk count table contains invalid token or zero count")
            pairs = tri[:, 0].astype(np.uint64) << np.uint64(32) | tri[:, 1]
            if len(np.unique(pairs)) != len(pairs):
                raise DiscreteError("duplicate (key, token) entry in sparse trunk count table")
            sparse[name] = tri
        trunk = Trunk(step, norm, uni, sparse)
    return Artifact(shape, table, cells, routes, gates, trunk)


# ---------------------------------------------------------------------------------------------
# Synthetic models of the M1 shape.

def synthetic(vocabulary=4096, blocks=4, context=192, kept_cells=8, read_mode="relation",
              read_kept=8, read_sweeps=1, seed=1, trunk=True, gate_density=0.5,
              trunk_entries=200_000) -> Artifact:
    """A random model: token blocks uniform over the 16 roots, route states uniform below 64,
    gates -1/0/+1, and (trunk) random sparse tables keyed as the joint pointer reads them."""
    rng = np.random.default_rng(seed)
    S = expected_stages(context)
    roots = rng.integers(0, 16, (vocabulary, blocks))
    table = tables.ROOTS[roots].astype(np.int32)
    routes = rng.integers(0, 64, blocks * S).astype(np.uint32)
    ng = blocks * S + (EDGE_TYPES * S if read_mode == "relation" else 0)
    gates = np.where(rng.random(ng) < gate_density, rng.choice([-1, 1], ng), 0).astype(np.int32)
    shape = Shape(vocabulary, blocks, context, kept_cells, S, read_mode,
                  0 if read_mode == "route" else read_kept,
                  read_sweeps if read_mode == "relation" else 0,
                  read_initialization="zero_gates_v1")
    tr = None
    if trunk:
        assert blocks == 4
        codes = (roots[:, 0] | roots[:, 1] << 4 | roots[:, 2] << 8 | roots[:, 3] << 12)
        sparse = {}
        for name in TRUNK_SPARSE:
            n = trunk_entries if name in ("query_table", "read_table", "rec_table",
                                          "query_read_table", "query_rec_table",
                                          "read_rec_table") else 64
            if name.startswith("query_read") or name.startswith("query_rec"):
                key = (rng.integers(0, vocabulary, n) << 16) | codes[rng.integers(0, vocabulary, n)]
            elif name.startswith("read_rec"):
                key = (codes[rng.integers(0, vocabulary, n)] << 16) | codes[rng.integers(0, vocabulary, n)]
            elif name.startswith("query"):
                key = rng.integers(0, vocabulary, n)
            else:
                key = codes[rng.integers(0, vocabulary, n)]
            tri = np.stack([key, rng.integers(0, vocabulary, n), rng.integers(1, 50, n)], 1)
            tri = tri.astype(np.uint32)
            _, keep = np.unique(tri[:, 0].astype(np.uint64) << np.uint64(32) | tri[:, 1],
                                return_index=True)
            sparse[name] = tri[np.sort(keep)]
        uni = np.concatenate([[rng.integers(0, vocabulary)],
                              rng.integers(0, 1000, vocabulary)]).astype(np.uint32)
        tr = Trunk(rng.integers(0, 16, 64).astype(np.uint32),
                   rng.integers(0, 16, 4).astype(np.uint32), uni, sparse)
    return Artifact(shape, table, endpoint_cells(table), routes, gates, tr)


def panel_rows(art: Artifact, rows: int, seed: int, min_len: int = 1):
    """(prefixes (rows, context) uint32 zero-padded, lengths, targets): lengths uniform in
    [min_len, context], tokens uniform, each row's target the token after its prefix."""
    rng = np.random.default_rng(seed)
    V, ctx = art.shape.vocabulary, art.shape.context
    seq = rng.integers(0, V, (rows, ctx + 1)).astype(np.uint32)
    lengths = rng.integers(min_len, ctx + 1, rows).astype(np.int32)
    prefixes = np.where(np.arange(ctx)[None, :] < lengths[:, None], seq[:, :ctx], 0).astype(np.uint32)
    targets = seq[np.arange(rows), lengths].astype(np.uint32)
    return prefixes, lengths, targets


def tables_header_arrays() -> dict:
    """The arrays csrc/d11_tables.h must hold (checked by a CPU test)."""
    return {"kD11Axes": tables.AXES, "kD11Roots": tables.ROOTS, "kD11Bfs": tables.BFS,
            "kD11Branch": tables.BRANCH, "kD11Compose": tables.compose_table()}


# ---------------------------------------------------------------------------------------------
# The C ABI (include/uor_d11.h).

SYMBOLS = ("uor_d11_abi_version", "uor_d11_sizeof_model", "uor_d11_sizeof_row_out",
           "uor_d11_last_error", "uor_d11_model_create", "uor_d11_model_destroy",
           "uor_d11_score_rows", "uor_d11_score_rows_async", "uor_d11_trace_words",
           "uor_d11_score_rows_traced", "uor_d11_score_rows_traced_async")

MAX_BLOCKS = 16
MAX_KEPT_CELLS = 16


class CTrunk(C.Structure):
    _fields_ = [("step_candidates", C.c_uint32 * 64), ("norm_candidates", C.c_uint32 * 4),
                ("unigram", C.c_void_p), ("sparse", C.c_void_p * 12),
                ("sparse_rows", C.c_uint64 * 12)]


class CModel(C.Structure):
    _fields_ = [("vocabulary", C.c_uint32), ("blocks", C.c_uint32), ("context", C.c_uint32),
                ("kept_cells", C.c_uint32), ("stages", C.c_uint32), ("read_mode", C.c_uint32),
                ("read_kept", C.c_uint32), ("read_sweeps", C.c_uint32),
                ("objective_policy", C.c_uint32), ("flags", C.c_uint32),
                ("table", C.c_void_p), ("cells", C.c_void_p), ("routes", C.c_void_p),
                ("gates", C.c_void_p), ("trunk", C.POINTER(CTrunk))]


class CRowOut(C.Structure):
    _fields_ = [("status", C.c_int32), ("admitted_count", C.c_int32), ("top8_count", C.c_int32),
                ("prediction", C.c_uint32), ("admitted", C.c_uint32 * MAX_KEPT_CELLS),
                ("top8", C.c_uint32 * 8), ("read_vector", C.c_int32 * (MAX_BLOCKS * 8)),
                ("token_hinge", C.c_uint32), ("address_hinge", C.c_uint32),
                ("rank_hinge", C.c_uint32), ("loss_ta", C.c_uint32), ("loss_tr", C.c_uint32),
                ("token_rivals", C.c_uint32), ("address_rivals", C.c_uint32),
                ("selected_loss", C.c_uint32)]


ROW_DTYPE = np.dtype([("status", "<i4"), ("admitted_count", "<i4"), ("top8_count", "<i4"),
                      ("prediction", "<u4"), ("admitted", "<u4", MAX_KEPT_CELLS),
                      ("top8", "<u4", 8), ("read_vector", "<i4", MAX_BLOCKS * 8),
                      ("token_hinge", "<u4"), ("address_hinge", "<u4"), ("rank_hinge", "<u4"),
                      ("loss_ta", "<u4"), ("loss_tr", "<u4"), ("token_rivals", "<u4"),
                      ("address_rivals", "<u4"), ("selected_loss", "<u4")])
assert ROW_DTYPE.itemsize == C.sizeof(CRowOut)


FLAG_STATE_TRANSPORT_KNOCKOUT = 1


def c_model(art: Artifact, knockout: bool = False):
    """The ``uor_d11_model`` image of an artifact and the arrays it points into (keep both);
    `knockout`: its state-transport knockout (the flag; the library zeroes the tables itself)."""
    s = art.shape
    keep = [np.ascontiguousarray(art.table, np.int32), np.ascontiguousarray(art.cells, np.uint32),
            np.ascontiguousarray(art.routes, np.uint32), np.ascontiguousarray(art.gates, np.int32)]
    m = CModel(s.vocabulary, s.blocks, s.context, s.kept_cells, s.stages, READ_MODES[s.read_mode],
               s.read_kept, s.read_sweeps, POLICIES[s.objective_policy],
               FLAG_STATE_TRANSPORT_KNOCKOUT if knockout else 0,
               *(a.ctypes.data for a in keep), None)
    if art.trunk is not None:
        t = CTrunk()
        t.step_candidates[:] = [int(v) for v in art.trunk.step_candidates]
        t.norm_candidates[:] = [int(v) for v in art.trunk.norm_candidates]
        uni = np.ascontiguousarray(art.trunk.unigram, np.uint32)
        keep.append(uni)
        t.unigram = uni.ctypes.data
        for i, name in enumerate(TRUNK_SPARSE):
            tri = np.ascontiguousarray(art.trunk.sparse.get(name, np.zeros((0, 3))), np.uint32)
            keep.append(tri)
            t.sparse[i] = tri.ctypes.data if len(tri) else None
            t.sparse_rows[i] = len(tri)
        keep.append(t)
        m.trunk = C.pointer(t)
    return m, keep


_lib = None


def lib():
    global _lib
    if _lib is None:
        from . import hip
        L = hip.lib()
        P = C.c_void_p
        L.uor_d11_abi_version.restype = C.c_uint32
        L.uor_d11_sizeof_model.restype = C.c_int64
        L.uor_d11_sizeof_row_out.restype = C.c_int64
        L.uor_d11_last_error.restype = C.c_char_p
        L.uor_d11_model_create.argtypes = [C.POINTER(CModel), C.c_int32, C.POINTER(P)]
        L.uor_d11_model_destroy.argtypes = [P]
        L.uor_d11_model_destroy.restype = None
        L.uor_d11_score_rows.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P]
        L.uor_d11_score_rows_async.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P]
        L.uor_d11_trace_words.argtypes = [P, P]
        L.uor_d11_trace_words.restype = C.c_uint32
        L.uor_d11_score_rows_traced.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P]
        L.uor_d11_score_rows_traced_async.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P,
                                                      P]
        assert L.uor_d11_sizeof_row_out() == ROW_DTYPE.itemsize
        assert L.uor_d11_sizeof_model() == C.sizeof(CModel)
        _lib = L
    return _lib


def _check(code: int):
    if code != 0:
        raise DiscreteError(f"uor_d11 status {code}: {lib().uor_d11_last_error().decode()}")


@dataclass
class Evaluation:
    """``DiscretePrefixEvaluation`` (discrete_d11.rs:376-389) plus the target's observation."""
    read_vector: list
    admitted_cells: list
    top8: list
    prediction: int
    token_rivals: int = 0
    address_rivals: int = 0
    token_hinge: int = 0
    address_hinge: int = 0
    rank_hinge: int = 0
    loss_ta: int = 0
    loss_tr: int = 0
    selected_loss: int = 0
    relation_scores: list | None = None  # blocks * nodes of the row's plan (relation reads)


@dataclass
class TracedEvaluation:
    """``DiscreteTracedPrefixEvaluation`` (discrete_d11.rs:391-400): the evaluation and the read's
    decision words (layout in include/uor_d11.h), the relation scores padded to a full context's
    node count with 0xffffffff (relation reads)."""
    evaluation: Evaluation
    trace_words: list
    relation_trace_words: list | None


class IntegerDiscreteModel:
    """A discrete model resident on one GPU (the reference's API names)."""

    def __init__(self, art: Artifact, device: int = 0, knockout: bool = False):
        self.art = art
        self.shape = art.shape
        self.device = device
        self.knockout = knockout
        m, keep = c_model(art, knockout=knockout)
        h = C.c_void_p()
        _check(lib().uor_d11_model_create(C.byref(m), device, C.byref(h)))
        self.handle = h

    def with_state_transport_knockout(self) -> "IntegerDiscreteModel":
        """``with_state_transport_knockout`` (discrete_d11.rs:1283-1304): a model whose binder
        routes are the identity state and whose level and relation gates are zero; its route read
        returns the last token's blocks untransported and the trunk's pointer gate is skipped."""
        return IntegerDiscreteModel(self.art, self.device, knockout=True)

    def is_state_transport_knocked_out(self) -> bool:
        return self.knockout

    @classmethod
    def from_bytes(cls, data: bytes, device: int = 0):
        return cls(parse_container(data), device)

    def is_trunk_d11(self) -> bool:
        return self.art.trunk is not None

    def close(self):
        if getattr(self, "handle", None):
            lib().uor_d11_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def score_rows(self, prefixes, lengths, targets) -> np.ndarray:
        """One record (``ROW_DTYPE``) per row; prefixes (rows, stride) zero-padded."""
        prefixes = np.ascontiguousarray(prefixes, np.uint32)
        if prefixes.ndim != 2:
            raise ValueError("prefixes must be (rows, stride)")
        rows, stride = prefixes.shape
        lengths = np.ascontiguousarray(lengths, np.int32)
        targets = np.ascontiguousarray(targets, np.uint32)
        if lengths.shape != (rows,) or targets.shape != (rows,):
            raise ValueError("lengths and targets need one entry per row")
        if rows and ((lengths < 0) | (lengths > stride)).any():
            raise ValueError("a length exceeds the row stride")
        out = np.zeros(rows, ROW_DTYPE)
        if rows:
            _check(lib().uor_d11_score_rows(self.handle, prefixes.ctypes.data, lengths.ctypes.data,
                                            targets.ctypes.data, rows, stride, out.ctypes.data))
        return out

    def trace_words(self) -> tuple[int, int]:
        """(trace words, relation trace words) of one row."""
        rw = C.c_uint32()
        return int(lib().uor_d11_trace_words(self.handle, C.byref(rw))), rw.value

    def score_rows_traced(self, prefixes, lengths, targets):
        """``score_rows`` with every row's trace: (records, trace [rows, words], relation trace
        [rows, blocks, a full context's node count] or None)."""
        prefixes = np.ascontiguousarray(prefixes, np.uint32)
        if prefixes.ndim != 2:
            raise ValueError("prefixes must be (rows, stride)")
        rows, stride = prefixes.shape
        lengths = np.ascontiguousarray(lengths, np.int32)
        targets = np.ascontiguousarray(targets, np.uint32)
        if lengths.shape != (rows,) or targets.shape != (rows,):
            raise ValueError("lengths and targets need one entry per row")
        if rows and ((lengths < 0) | (lengths > stride)).any():
            raise ValueError("a length exceeds the row stride")
        words, rwords = self.trace_words()
        out = np.zeros(rows, ROW_DTYPE)
        trace = np.zeros((rows, words), np.uint32)
        rel = np.zeros((rows, rwords), np.uint32) if rwords else None
        if rows:
            _check(lib().uor_d11_score_rows_traced(
                self.handle, prefixes.ctypes.data, lengths.ctypes.data, targets.ctypes.data, rows,
                stride, out.ctypes.data, trace.ctypes.data, None if rel is None else rel.ctypes.data))
        if rel is not None:
            rel = rel.reshape(rows, self.shape.blocks, -1)
        return out, trace, rel

    def _one(self, prefix, target, traced=False):
        prefix = np.asarray(prefix, np.uint32).reshape(-1)
        if len(prefix) == 0 or len(prefix) > self.shape.context:
            raise DiscreteError("prefix length must be in 1..=context")
        if (prefix >= self.shape.vocabulary).any():
            raise DiscreteError("prefix token ID outside vocabulary")
        if traced:
            out, trace, rel = self.score_rows_traced(prefix[None, :], [len(prefix)], [target])
            row, trace, rel = out[0], trace[0], None if rel is None else rel[0]
        else:
            row = self.score_rows(prefix[None, :], [len(prefix)], [target])[0]
        if row["status"] != 0:
            raise DiscreteError(STATUS.get(int(row["status"]), str(row["status"])))
        return (row, trace, rel) if traced else row

    def _relation(self) -> bool:
        return READ_MODES[self.shape.read_mode] == 2

    def _evaluation(self, row, observed: bool, rel=None, length=0) -> Evaluation:
        B = self.shape.blocks
        ev = Evaluation(row["read_vector"][:8 * B].tolist(),
                        row["admitted"][:row["admitted_count"]].tolist(),
                        row["top8"][:row["top8_count"]].tolist(), int(row["prediction"]))
        if rel is not None:  # the row plan's nodes of each block, as i32 (:386-388)
            n = plan_nodes(length)
            ev.relation_scores = rel[:, :n].view(np.int32).reshape(-1).tolist()
        if observed:
            for k in ("token_rivals", "address_rivals", "token_hinge", "address_hinge",
                      "rank_hinge", "loss_ta", "loss_tr", "selected_loss"):
                setattr(ev, k, int(row[k]))
        return ev

    def evaluate_prefix(self, prefix) -> Evaluation:
        """``evaluate_prefix`` (discrete_d11.rs:1761): the read, admitted cells and top 8, and a
        relation read's scores (taken from the traced launch)."""
        if self._relation():
            return self.evaluate_prefix_traced(prefix).evaluation
        return self._evaluation(self._one(prefix, 0), False)

    def evaluate_prefix_traced(self, prefix) -> TracedEvaluation:
        """``evaluate_prefix_traced`` (discrete_d11.rs:1768): the evaluation with the read's
        decision words."""
        row, trace, rel = self._one(prefix, 0, traced=True)
        n = len(np.asarray(prefix).reshape(-1))
        return TracedEvaluation(self._evaluation(row, False, rel, n), trace.tolist(),
                                None if rel is None else rel.reshape(-1).tolist())

    def observe_target(self, prefix, target: int) -> Evaluation:
        """``observe_target`` (discrete_d11.rs:1892): the evaluation plus hinges and losses."""
        if not 0 <= int(target) < self.shape.vocabulary:
            raise DiscreteError("target token ID outside vocabulary")
        if self._relation():
            row, _, rel = self._one(prefix, int(target), traced=True)
            return self._evaluation(row, True, rel, len(np.asarray(prefix).reshape(-1)))
        return self._evaluation(self._one(prefix, int(target)), True)
