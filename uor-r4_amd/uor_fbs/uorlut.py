"""Reader of the reference's `UORLUT01` stack container for the SpiralCore/FBS stacks this path
serves, producing the same `Artifact` the seeded generator does (so `cabi.Image`, the HIP model
and the oracle take trained weights unchanged).

Container layout (crates/uor-r4-integer/src/stack/format.rs:1-16, `Container::parse`
:1202-1518): the 8-byte magic `UORLUT01`, a little-endian u64 header length, the JSON header,
zero padding to a multiple of 64 bytes, then the data; every table is named in the header with
its kind (`i16`, `i32`, `u32`, little-endian), length and byte span relative to the data start.

The FBS image (`fbs_model`, session.rs:640-735): per layer `l{l}.rec_in.fbs` .. `mlp_down.fbs`
route words (atom in the low 16 bits, axis state in the high 16 bits, codes = `cl06_axes(state)`,
discrete_d11.rs:857-913), `rec_norm_gain`, `mlp_norm_gain`, `conv_taps` (4 x width grid codes),
`conv_bias`, `gate_bias`, `decay_offset`; then `final_norm_gain` and `writer.table`.

Served schemas: `uor-r4.lut-stack/4` and `/5` (FBS, snapped or raw gates/transition), and the
turn-memory `/7` and point-key `/8` stacks, whose extra records `step_native` does not apply
(session.rs:4327-4392 applies them only after `mark_reply_start`); the reference's loader
accepts them for the plain step, and so does this one. Hamming reads, memory chains, bound
contracts, address tables, Q31 records and pair rows are refused by schema, as a reader that
does not serve them must.

Loading is host code outside the served path: it reads JSON and raw little-endian arrays and
executes nothing from the file.
"""

from __future__ import annotations

import hashlib
import json
import struct

import numpy as np

from . import tables
from .synth import Artifact, Layer, Spec

MAGIC = b"UORLUT01"
ALIGN = 64                 # format.rs:443
GROUP = 32                 # format.rs:441
MAX_HEADER = 64 << 20      # format.rs:445
KINDS = {"i16": np.dtype("<i2"), "i32": np.dtype("<i4"), "u32": np.dtype("<u4")}
SERVED = {
    "uor-r4.lut-stack/4",  # FBS, snapped gates and transition
    "uor-r4.lut-stack/5",  # FBS with raw gates or transition
    "uor-r4.lut-stack/7",  # + turn memory (not applied by step_native)
    "uor-r4.lut-stack/8",  # + point key (not applied by step_native)
}
REFUSED_RECORDS = ("hamming", "memory_chain", "address", "pair_rows", "q31", "q31_lanes", "q31_read")


class UorlutError(ValueError):
    """A container this reader refuses, with the reference loader's reason where it has one."""


def _grid_valid(codes: np.ndarray) -> bool:
    """`grid_valid` (kernels.rs:116-120): zero, or |code| >> 4 in 1..127."""
    field = np.abs(codes.astype(np.int32)) >> 4
    return bool(np.all((codes == 0) | ((field >= 1) & (field <= 127))))


def parse(data: bytes) -> tuple[dict, dict]:
    """The header and every table as a numpy array, with the container's bounds checks."""
    if len(data) < 16 or data[:8] != MAGIC:
        raise UorlutError("not a UORLUT01 container (magic)")
    (declared,) = struct.unpack("<Q", data[8:16])
    if declared > MAX_HEADER or 16 + declared > len(data):
        raise UorlutError(f"header length {declared} exceeds the {len(data)}-byte container")
    end = 16 + declared
    try:
        header = json.loads(data[16:end].decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise UorlutError(f"header: {e}") from None
    start = end + (ALIGN - end % ALIGN) % ALIGN
    if start > len(data):
        raise UorlutError("no data section")
    body = memoryview(data)[start:]
    out = {}
    for t in header.get("tables", []):
        name, kind, n = t["name"], t["kind"], int(t["len"])
        if name in out:
            raise UorlutError(f"duplicate section {name}")
        if kind not in KINDS:
            raise UorlutError(f"{name}: table kind {kind} is not served")
        off, size = int(t["span"]["offset"]), int(t["span"]["bytes"])
        if n * KINDS[kind].itemsize != size or off < 0 or off + size > len(body):
            raise UorlutError(f"{name}: table span out of bounds")
        out[name] = np.frombuffer(body[off:off + size], dtype=KINDS[kind]).copy()
    return header, out


def _check_shape(header: dict) -> dict:
    schema = header.get("schema")
    if schema not in SERVED:
        raise UorlutError(f"schema {schema} is not served by this path")
    for rec in REFUSED_RECORDS:
        if header.get(rec) is not None:
            raise UorlutError(f"the {rec} record is not served by this path")
    if header.get("group") != GROUP:
        raise UorlutError(f"group {header.get('group')} (expected {GROUP})")
    s = header["shape"]
    raw = bool(s.get("raw_gates")) or bool(s.get("raw_transition"))
    memory, point = header.get("memory") is not None, header.get("point") is not None
    expected = ("uor-r4.lut-stack/8" if point else "uor-r4.lut-stack/7" if memory
                else "uor-r4.lut-stack/5" if raw else "uor-r4.lut-stack/4")
    if schema != expected:
        raise UorlutError(f"schema {schema} does not match its records (expected {expected})")
    reasons = [
        (s.get("projection") != "spiralcore_fbs", "projection is not spiralcore_fbs"),
        (any(c != "r" for c in s.get("pattern", "")) or not s.get("pattern"),
         "an FBS stack's layers are all recurrence layers (pattern of r)"),
        (s.get("rec_gates") != "geometric", "rec_gates must be geometric"),
        (not s.get("rotation"), "rec_gates=geometric needs learned rotations"),
        (s.get("head") not in ("native_vector", "native_vector_nearest"),
         "the head must be native_vector or native_vector_nearest"),
        (s.get("kept_cells") is None or not 1 <= s["kept_cells"] <= 16, "kept cells 1..16"),
        (s.get("heads", 1) != 1, "one head"),
    ]
    for bad, why in reasons:
        if bad:
            raise UorlutError(why)
    snap = header.get("transport_snap")
    if not s.get("raw_transition"):
        if not snap or snap.get("name") != "icosian" or snap.get("roots") != 120:
            raise UorlutError("a snapped transition needs transport_snap=icosian with 120 roots")
    return s


def load(source) -> Artifact:
    """A served FBS artifact from a path or the container's bytes."""
    data = source if isinstance(source, (bytes, bytearray)) else open(source, "rb").read()
    header, tabs = parse(bytes(data))
    s = _check_shape(header)
    d, m, V = int(s["width"]), int(s["mlp"]), int(s["vocab"])
    L, lanes = len(s["pattern"]), d // 4
    rows = lanes + d

    def table(name, kind, n):
        if name not in tabs:
            raise UorlutError(f"missing section {name}")
        t = tabs[name]
        if t.dtype != KINDS[kind] or len(t) != n:
            raise UorlutError(f"{name}: {len(t)} {t.dtype} values, expected {n} {kind}")
        return t

    def codes(name, n):
        t = table(name, "i16", n).astype(np.int16)
        if not _grid_valid(t):
            raise UorlutError(f"{name}: not grid codes")
        return t

    def route(name, in_blocks, out_blocks):
        w = table(name, "u32", out_blocks)
        atoms, states = w & 0xFFFF, w >> 16
        if np.any(atoms >= in_blocks) or np.any(states >= 64):
            raise UorlutError(f"{name}: a route entry lies outside {in_blocks} atoms or 64 states")
        return atoms.astype(np.uint16), tables.AXES.reshape(64, 8)[states].reshape(-1).astype(np.uint8)

    layers = []
    for l in range(L):
        p = f"l{l}."
        maps = {}
        for name, i, o in (("rec_in", d, 2 * d), ("rec_gate", d, rows), ("rec_out", d, d),
                           ("mlp_gate", d, m), ("mlp_up", d, m), ("mlp_down", m, d)):
            maps[name] = route(p + name + ".fbs", i // 8, o // 8)
        layers.append(Layer(
            rec_gain=codes(p + "rec_norm_gain", d), mlp_gain=codes(p + "mlp_norm_gain", d),
            maps=maps, taps=codes(p + "conv_taps", 4 * d), wide_taps=None,
            conv_bias=table(p + "conv_bias", "i32", d).astype(np.int32),
            gate_bias=table(p + "gate_bias", "i32", rows).astype(np.int32),
            decay_offset=table(p + "decay_offset", "i32", lanes).astype(np.int32)))
    eps = header["numerics"]["rms_eps"]
    spec = Spec(vocab=V, width=d, mlp=m, layers=L, context=int(s["context"]),
                kept=int(s["kept_cells"]), head=1 if s["head"] == "native_vector_nearest" else 0,
                raw_gates=bool(s.get("raw_gates")), raw_transition=bool(s.get("raw_transition")))
    return Artifact(spec=spec, seed=-1, layers=layers, final_gain=codes("final_norm_gain", d),
                    writer_table=table("writer.table", "i16", V * d).astype(np.int16),
                    table_i8=None, eps_mantissa=int(eps["mantissa"]), eps_exp=int(eps["exp"]),
                    sha256=hashlib.sha256(data).hexdigest())
