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

Served schemas: `uor-r4.lut-stack/4` and `/5` (FBS, snapped or raw gates/transition), `/6`
(FBS with Hamming reads: the `hamming` record and its `hamming.d{depth}.*` sections,
StackHamming, format.rs:229-430, read as hamming_image does, hamming.rs:58-110), and the
turn-memory `/7` and point-key `/8` stacks (with or without Hamming reads), whose turn memory
`step_native` does not apply (session.rs:4327-4392 applies it only after `mark_reply_start`);
the reference's loader accepts them for the plain step, and so does this one. The Hamming place
read (`hamming.place`), memory chains, bound contracts, address tables, Q31 records and pair
rows are refused, as a reader that does not serve them must.

Loading is host code outside the served path: it reads JSON and raw little-endian arrays and
executes nothing from the file.
"""

from __future__ import annotations

import hashlib
import json
import struct

import numpy as np

from . import tables
from .synth import (PLACE_ARM, PLACE_OPEN, PLACE_STOP, Artifact, HammingRead, HammingSpec, Layer,
                    PlaceMarks, Spec)

MAGIC = b"UORLUT01"
ALIGN = 64                 # format.rs:443
GROUP = 32                 # format.rs:441
MAX_HEADER = 64 << 20      # format.rs:445
KINDS = {"i16": np.dtype("<i2"), "i32": np.dtype("<i4"), "u32": np.dtype("<u4")}
SERVED = {
    "uor-r4.lut-stack/4",  # FBS, snapped gates and transition
    "uor-r4.lut-stack/5",  # FBS with raw gates or transition
    "uor-r4.lut-stack/6",  # FBS with Hamming reads
    "uor-r4.lut-stack/7",  # + turn memory (not applied by step_native)
    "uor-r4.lut-stack/8",  # + point key (not applied by step_native)
}
REFUSED_RECORDS = ("memory_chain", "address", "pair_rows", "q31", "q31_lanes", "q31_read")
# The Hamming record's fields (StackHamming, format.rs:229-292, deny_unknown_fields) and the
# exponents this engine reads (format.rs:55-59).
HAMMING_FIELDS = {"heads", "depths", "kept", "rotation_exp", "margin_exp", "weight_exp", "copy_key",
                  "copy_keys", "copy_latest", "copy_longest", "asks", "carry_rows", "place"}
HAMMING_EXPS = {"rotation_exp": -24, "margin_exp": -16, "weight_exp": -24}
ASK_CARRY_MAX = 1 << 12            # hamming.rs:1052
MAX_READ_CACHE_BYTES = 1 << 32     # format.rs:456


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
    hamming = header.get("hamming") is not None
    expected = ("uor-r4.lut-stack/8" if point else "uor-r4.lut-stack/7" if memory
                else "uor-r4.lut-stack/6" if hamming
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


def _place_marks(rec) -> PlaceMarks:
    """The record's `place` marks (PlaceMarks, fbs_snapshot.rs:2725-2732, deny_unknown_fields)."""
    fields = {"bos", "eos", "sep", "system", "user", "assistant"}
    if not isinstance(rec, dict) or set(rec) != fields:
        raise UorlutError(f"hamming.place: the fields are {sorted(fields)}")
    try:
        lists = {k: tuple(int(x) for x in rec[k]) for k in ("sep", "system", "user", "assistant")}
        return PlaceMarks(bos=int(rec["bos"]), eos=int(rec["eos"]), **lists)
    except (TypeError, ValueError):
        raise UorlutError("hamming.place: marks are vocabulary ids") from None


def _check_hamming(rec: dict, s: dict) -> HammingSpec:
    """`StackHamming::check` (format.rs:336-430) on the header's record."""
    if not isinstance(rec, dict) or set(rec) - HAMMING_FIELDS:
        raise UorlutError(f"hamming: unknown fields {sorted(set(rec) - HAMMING_FIELDS)}")
    missing = {"heads", "depths", "kept", *HAMMING_EXPS} - set(rec)
    if missing:
        raise UorlutError(f"hamming: missing fields {sorted(missing)}")
    d, V, L = int(s["width"]), int(s["vocab"]), len(s["pattern"])
    heads, depths, kept = int(rec["heads"]), [int(x) for x in rec["depths"]], int(rec["kept"])
    if heads < 2 or heads % 2 or d % heads:
        raise UorlutError("a Hamming read needs an even head count of at least 2 that divides the width")
    hw = d // heads
    if hw % 4 or hw > 64:
        raise UorlutError("a Hamming head needs whole 4-lane blocks and at most 64 coordinates")
    copy_key = int(rec.get("copy_key", 1))
    if copy_key not in (1, 2):
        raise UorlutError("a Hamming copy key names 1 or 2 tokens")
    keys = rec.get("copy_keys")
    if keys is not None:
        keys = [int(k) for k in keys]
        if (copy_key != 1 or len(keys) != heads // 2 or any(k not in (1, 2) for k in keys)
                or all(k == keys[0] for k in keys)):
            raise UorlutError("mixed Hamming copy keys name 1 or 2 tokens for each copy head, differ, "
                              "and leave copy_key at 1")
    per_head = keys or [copy_key] * (heads // 2)
    if 2 in per_head and hw % 8:
        raise UorlutError("copy key 2 needs heads of whole 8-coordinate blocks")
    latest, longest = bool(rec.get("copy_latest", False)), rec.get("copy_longest")
    if longest is not None:
        longest = tuple(int(x) for x in longest)
        if not latest or any(k != 1 for k in per_head) or len(longest) != 2 or max(longest) >= V:
            raise UorlutError("the longest rule needs the latest exact rule, one-token copy keys and "
                              "a marker of two vocabulary ids")
    if not depths or any(b <= a for a, b in zip(depths, depths[1:])) or not all(1 <= x <= L for x in depths):
        raise UorlutError("Hamming read depths must be strictly increasing, from 1 to the layer count")
    if kept == 0:
        raise UorlutError("a Hamming read keeps at least one position")
    asks = rec.get("asks")
    if asks is not None:
        asks = tuple(bool(a) for a in asks)
        if len(asks) != len(depths) or not any(asks):
            raise UorlutError("Hamming ask heads name one flag per read, not all off")
    reach = rec.get("carry_rows")
    if reach is not None:
        reach = int(reach)
        if depths[-1] != L:
            raise UorlutError("a Hamming question carry is served on the readout read only")
        if not (asks and asks[-1]):
            raise UorlutError("a Hamming question carry needs its read to ask")
        if not 1 <= reach <= ASK_CARRY_MAX:
            raise UorlutError("a Hamming question carry reaches from 1 to ASK_CARRY_MAX rows")
    place = rec.get("place")
    if place is not None:
        place = _place_marks(place)
        if depths[-1] != L or not (asks and asks[-1]):
            raise UorlutError("a Hamming place read is served on a readout read that asks")
        if hw % 8:
            raise UorlutError("a Hamming place read needs heads of whole 8-coordinate blocks, so "
                              "each half is whole lanes")
        why = place.check(V)
        if why:
            raise UorlutError(why)
    for k, v in HAMMING_EXPS.items():
        if rec.get(k) != v:
            raise UorlutError("the Hamming read's exponents are not this engine's")
    return HammingSpec(heads=heads, depths=tuple(depths), kept=kept, copy_key=copy_key,
                       copy_keys=None if keys is None else tuple(keys), copy_latest=latest,
                       copy_longest=longest, asks=asks, carry_rows=reach or 0, place=place)


def _place_classes(h: HammingSpec, tabs: dict, V: int) -> np.ndarray | None:
    """The readout read's `hamming.d{depth}.place` class table (PlaceImage::checked,
    fbs_snapshot.rs:2779-2790), present exactly when the record carries the marks
    (hamming.rs:113-122)."""
    name = f"hamming.d{h.depths[-1]}.place"
    if h.place is None:
        if name in tabs:
            raise UorlutError(f"{name}: present, but the record names no place read")
        return None
    if name not in tabs:
        raise UorlutError(f"missing section {name}")
    t = tabs[name]
    if t.dtype != KINDS["i16"]:
        raise UorlutError(f"{name}: {t.dtype} values, expected i16")
    if len(t) != V:
        raise UorlutError(f"the place read's class table has {len(t)} entries for a vocabulary of {V}")
    cls = np.asarray(t, np.int16)
    if np.any(cls & ~np.int16(PLACE_STOP | PLACE_ARM | PLACE_OPEN)):
        raise UorlutError("the place read's class table has a bit outside stop, arm and open")
    return cls


def _hamming_reads(h: HammingSpec, tabs: dict, V: int, d: int, context: int) -> list:
    """Every read's sections at the lengths its record implies (hamming_image, hamming.rs:58-110;
    AskImage::checked :1069-1095), margins positive, and the payload caches within the session
    read cache (check_payload_cache :1538-1549)."""
    reads, typed = [], 0
    for r, depth in enumerate(h.depths):
        def section(part, kind, n, present=True):
            name = f"hamming.d{depth}.{part}"
            if name not in tabs:
                if present:
                    raise UorlutError(f"missing section {name}")
                return None
            if not present:
                raise UorlutError(f"{name}: present, but the record does not name it")
            t = tabs[name]
            if t.dtype != KINDS[kind] or len(t) != n:
                raise UorlutError(f"{name}: {len(t)} {t.dtype} values, expected {n} {kind}")
            return t
        margin = section("margin", "i32", h.heads).astype(np.int32)
        if np.any(margin <= 0):
            raise UorlutError(f"hamming.d{depth}.margin: a margin is not positive")
        asks = bool(h.asks and h.asks[r])
        carries = bool(h.carry_rows) and r + 1 == len(h.depths)
        ask = section("ask", "i16", V * d, asks)
        carry = section("carry", "i32", V, carries)
        weight = section("weight", "i32", 2 * d).astype(np.int32)
        typed += int(not asks and np.any(weight[d:] != 0))
        reads.append(HammingRead(
            depth=depth, query_rotation=section("query_rotation", "i32", d).astype(np.int32),
            key_rotation=section("key_rotation", "i32", d).astype(np.int32),
            value_rotation=section("value_rotation", "i32", d).astype(np.int32), margin=margin,
            weight=weight, ask=None if ask is None else ask.astype(np.int16),
            carry=None if carry is None else carry.astype(np.int32)))
    if typed * context * d * 8 > MAX_READ_CACHE_BYTES:
        raise UorlutError("the Hamming type heads' payload cache exceeds the session read cache's 4 GiB")
    return reads


def add_hamming(source, h: HammingSpec, reads: list) -> bytes:
    """A container with Hamming reads added: every section of `source` byte for byte, each read's
    `hamming.d{depth}.*` sections appended, the header's `hamming` record written and its schema
    moved to `/6` when it has no turn memory (as the reference's exporter names a Hamming stack,
    format.rs:2595-2607, and its section adders append, :2730-2783). The result is read back."""
    data = bytes(source if isinstance(source, (bytes, bytearray)) else open(source, "rb").read())
    header, _ = parse(data)
    if header.get("hamming") is not None:
        raise UorlutError("the container already has Hamming reads")
    if h.place is not None:
        raise UorlutError("a place read is added after the reads (add_hamming_place)")
    (declared,) = struct.unpack("<Q", data[8:16])
    end = 16 + declared
    body = bytearray(data[end + (ALIGN - end % ALIGN) % ALIGN:])
    tables_ = list(header["tables"])

    def push(name, arr, kind):
        nonlocal body
        body += b"\0" * ((ALIGN - len(body) % ALIGN) % ALIGN)
        raw = np.ascontiguousarray(arr, KINDS[kind]).tobytes()
        tables_.append({"name": name, "kind": kind, "len": int(np.asarray(arr).size),
                        "span": {"offset": len(body), "bytes": len(raw)}})
        body += raw

    for r in reads:
        p = f"hamming.d{r.depth}."
        for part in ("query_rotation", "key_rotation", "value_rotation", "margin", "weight"):
            push(p + part, getattr(r, part), "i32")
        if r.ask is not None:
            push(p + "ask", r.ask, "i16")
        if r.carry is not None:
            push(p + "carry", r.carry, "i32")
    rec = {"heads": h.heads, "depths": list(h.depths), "kept": h.kept, **HAMMING_EXPS}
    if h.copy_key != 1:
        rec["copy_key"] = h.copy_key
    if h.copy_keys is not None:
        rec["copy_keys"] = list(h.copy_keys)
    if h.copy_latest:
        rec["copy_latest"] = True
    if h.copy_longest is not None:
        rec["copy_longest"] = list(h.copy_longest)
    if h.asks is not None:
        rec["asks"] = list(h.asks)
    if h.carry_rows:
        rec["carry_rows"] = h.carry_rows
    header = dict(header, tables=tables_, hamming=rec)
    if header.get("memory") is None and header.get("point") is None:
        header["schema"] = "uor-r4.lut-stack/6"
    hb = json.dumps(header).encode()
    out = MAGIC + struct.pack("<Q", len(hb)) + hb
    out += b"\0" * ((ALIGN - len(out) % ALIGN) % ALIGN) + bytes(body)
    load(out)
    return out


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
    art = Artifact(spec=spec, seed=-1, layers=layers, final_gain=codes("final_norm_gain", d),
                   writer_table=table("writer.table", "i16", V * d).astype(np.int16),
                   table_i8=None, eps_mantissa=int(eps["mantissa"]), eps_exp=int(eps["exp"]),
                   sha256=hashlib.sha256(data).hexdigest(),
                   turn_memory=header.get("memory") is not None)
    if header.get("hamming") is not None:
        art.hamming = _check_hamming(header["hamming"], s)
        art.hamming_reads = _hamming_reads(art.hamming, tabs, V, d, int(s["context"]))
        art.hamming_place = _place_classes(art.hamming, tabs, V)
    return art


def add_hamming_place(source, marks: PlaceMarks, classes) -> bytes:
    """A Hamming stack whose readout read asks, with the place read added
    (add_hamming_place_uorlut01, format.rs:2780-2819): every section byte for byte, then
    `hamming.d{depth}.place` (i16 classes of the vocabulary) on the readout read, the record's
    `place` carrying the marks. Refused: a stack without Hamming reads or with a place read
    already, marks or classes PlaceImage::checked refuses, and a readout read that does not ask.
    The result is read back."""
    data = bytes(source if isinstance(source, (bytes, bytearray)) else open(source, "rb").read())
    header, _ = parse(data)
    rec = header.get("hamming")
    if rec is None:
        raise UorlutError("a place read is added to a stack with Hamming reads")
    if rec.get("place") is not None:
        raise UorlutError("a place read is added to a stack without one")
    V = int(header["shape"]["vocab"])
    cls = np.asarray(classes, np.int16)
    why = marks.check(V)
    if why:
        raise UorlutError(why)
    if len(cls) != V:
        raise UorlutError(f"the place read's class table has {len(cls)} entries for a vocabulary of {V}")
    if np.any(cls & ~np.int16(PLACE_STOP | PLACE_ARM | PLACE_OPEN)):
        raise UorlutError("the place read's class table has a bit outside stop, arm and open")
    (declared,) = struct.unpack("<Q", data[8:16])
    end = 16 + declared
    body = bytearray(data[end + (ALIGN - end % ALIGN) % ALIGN:])
    body += b"\0" * ((ALIGN - len(body) % ALIGN) % ALIGN)
    raw = cls.tobytes()
    name = f"hamming.d{int(rec['depths'][-1])}.place"
    tables_ = list(header["tables"]) + [{"name": name, "kind": "i16", "len": int(cls.size),
                                         "span": {"offset": len(body), "bytes": len(raw)}}]
    body += raw
    header = dict(header, tables=tables_, hamming=dict(rec, place=marks.to_json()))
    hb = json.dumps(header).encode()
    out = MAGIC + struct.pack("<Q", len(hb)) + hb
    out += b"\0" * ((ALIGN - len(out) % ALIGN) % ALIGN) + bytes(body)
    load(out)
    return out
