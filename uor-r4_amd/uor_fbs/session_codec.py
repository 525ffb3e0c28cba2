"""The reference's session snapshot and its two encodings: the integer-safe byte stream
`UR4SESS1`/`2`/`3` with the `UORMEM01` durable-scope envelope (crates/uor-r4-integer/src/
session_codec.rs), and the JSON form `save_session_to_file` writes (serde_json of
`SerializedStackSession`, stack/session.rs:1872-1960, 3202-3290).

The snapshot classes carry the reference's fields in its order; the byte layout, the varint,
the magic chosen by content, and the refusals (bad magic, truncation, counts longer than the
remaining bytes, trailing bytes, bad tags, invalid UTF-8) follow session_codec.rs:12-380.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field

STACK_SESSION_SCHEMA = "uor-r4.stack-session/1"   # session.rs:1872

MAGIC = b"UR4SESS1"            # session_codec.rs:47-52
MAGIC_CONTENT = b"UR4SESS2"
MAGIC_PAYLOADS = b"UR4SESS3"
DURABLE_SCOPE_MAGIC = b"UORMEM01"   # session_codec.rs:382-386
DURABLE_SCOPE_VERSION = 1


class CodecError(ValueError):
    """A byte stream the reference's decoder refuses."""


@dataclass
class RecurrenceLayer:
    """`SerializedStackLayerState::Recurrence` (session.rs:1876-1884): state [width] i64 at
    exponent -32, history [window][width] i32 (row 0 the newest drive) at exponent -16."""
    state: list
    history: list


@dataclass
class ReadLayer:
    """`SerializedStackLayerState::Read` (session.rs:1885-1894); a dense stack's read cache.
    The FBS path has no read layers, but snapshots that carry them encode and decode."""
    keys: list
    values: list
    lifts: list


@dataclass
class SerializedStackSession:
    """`SerializedStackSession` (session.rs:1900-1960), field for field."""
    schema: str
    version: int
    artifact_sha256: str
    position: int
    cache_at: int
    lift_at: int
    copy_scale_q16: int = 0
    logits: list = field(default_factory=list)
    tokens: list = field(default_factory=list)
    hamming_payloads: list = field(default_factory=list)
    snap_trace: list | None = None
    pointer_keys: list = field(default_factory=list)
    pointer_lifts: list = field(default_factory=list)
    mixture: list = field(default_factory=list)
    content_readout_sha256: str | None = None
    layers: list = field(default_factory=list)


# ---- the byte stream ------------------------------------------------------------------------

def _v64(out: bytearray, v: int):
    if not 0 <= v < 1 << 64:
        raise CodecError("session codec: a count outside u64")
    while True:
        b = v & 0x7F
        v >>= 7
        if v == 0:
            out.append(b)
            return
        out.append(b | 0x80)


def _str(out: bytearray, s: str):
    b = s.encode("utf-8")
    out += struct.pack("<I", len(b))
    out += b


def _vec(out: bytearray, fmt: str, xs):
    _v64(out, len(xs))
    if len(xs):
        out += struct.pack(f"<{len(xs)}{fmt}", *xs)


def encode(s: SerializedStackSession) -> bytes:
    """`session_codec::encode` (session_codec.rs:114-190): the magic by content (payloads ->
    UR4SESS3, a content-readout hash -> UR4SESS2, else UR4SESS1), then the fields in order."""
    out = bytearray()
    payloads = len(s.hamming_payloads) > 0
    out += MAGIC_PAYLOADS if payloads else MAGIC_CONTENT if s.content_readout_sha256 is not None else MAGIC
    _str(out, s.schema)
    out += struct.pack("<I", s.version)
    _str(out, s.artifact_sha256)
    out += struct.pack("<QQQi", s.position, s.cache_at, s.lift_at, s.copy_scale_q16)
    _vec(out, "i", s.logits)
    _vec(out, "I", s.tokens)
    if s.snap_trace is None:
        out.append(0)
    else:
        out.append(1)
        _vec(out, "I", s.snap_trace)
    _vec(out, "i", s.pointer_keys)
    _vec(out, "Q", s.pointer_lifts)
    _vec(out, "i", s.mixture)
    if payloads:
        out.append(1 if s.content_readout_sha256 is not None else 0)
        if s.content_readout_sha256 is not None:
            _str(out, s.content_readout_sha256)
        _v64(out, len(s.hamming_payloads))
        for p in s.hamming_payloads:
            _vec(out, "q", p)
    elif s.content_readout_sha256 is not None:
        _str(out, s.content_readout_sha256)
    _v64(out, len(s.layers))
    for layer in s.layers:
        if isinstance(layer, RecurrenceLayer):
            out.append(0)
            _vec(out, "q", layer.state)
            _vec(out, "i", layer.history)
        elif isinstance(layer, ReadLayer):
            out.append(1)
            _vec(out, "i", layer.keys)
            _vec(out, "i", layer.values)
            _vec(out, "Q", layer.lifts)
        else:
            raise CodecError(f"session codec: unknown layer {type(layer).__name__}")
    return bytes(out)


class _Reader:
    def __init__(self, buf: bytes):
        self.buf, self.at = buf, 0

    def take(self, n: int) -> bytes:
        end = self.at + n
        if end > len(self.buf):
            raise CodecError("session codec: truncated input")
        b = self.buf[self.at:end]
        self.at = end
        return b

    def unpack(self, fmt: str):
        return struct.unpack("<" + fmt, self.take(struct.calcsize("<" + fmt)))[0]

    def v64(self) -> int:
        acc, shift = 0, 0
        while True:
            b = self.take(1)[0]
            acc |= (b & 0x7F) << shift
            if not b & 0x80:
                return acc
            shift += 7
            if shift >= 64:
                raise CodecError("session codec: varint overflow")

    def count(self, elem_shift: int) -> int:
        n = self.v64()
        if n > (len(self.buf) - self.at) >> elem_shift:
            raise CodecError("session codec: truncated input")
        return n

    def string(self) -> str:
        n = self.unpack("I")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError:
            raise CodecError("session codec: invalid utf-8") from None

    def vec(self, fmt: str, shift: int) -> list:
        n = self.count(shift)
        return list(struct.unpack(f"<{n}{fmt}", self.take(n << shift))) if n else []

    def tag(self, what: str, allowed=(0, 1)) -> int:
        t = self.take(1)[0]
        if t not in allowed:
            raise CodecError(f"session codec: bad {what} tag {t}")
        return t


def decode(data: bytes) -> SerializedStackSession:
    """`session_codec::decode` (session_codec.rs:282-378)."""
    r = _Reader(bytes(data))
    magic = r.take(8)
    if magic not in (MAGIC, MAGIC_CONTENT, MAGIC_PAYLOADS):
        raise CodecError("session codec: bad magic")
    schema = r.string()
    version = r.unpack("I")
    sha = r.string()
    position, cache_at, lift_at = r.unpack("Q"), r.unpack("Q"), r.unpack("Q")
    copy_scale = r.unpack("i")
    logits = r.vec("i", 2)
    tokens = r.vec("I", 2)
    snap = r.vec("I", 2) if r.tag("snap_trace") else None
    pointer_keys = r.vec("i", 2)
    pointer_lifts = r.vec("Q", 3)
    mixture = r.vec("i", 2)
    content, payloads = None, []
    if magic == MAGIC_PAYLOADS:
        if r.tag("content"):
            content = r.string()
        payloads = [r.vec("q", 3) for _ in range(r.count(0))]
    elif magic == MAGIC_CONTENT:
        content = r.string()
    layers = []
    for _ in range(r.count(0)):
        if r.tag("layer") == 0:
            layers.append(RecurrenceLayer(r.vec("q", 3), r.vec("i", 2)))
        else:
            layers.append(ReadLayer(r.vec("i", 2), r.vec("i", 2), r.vec("Q", 3)))
    if r.at != len(r.buf):
        raise CodecError("session codec: trailing bytes")
    return SerializedStackSession(schema, version, sha, position, cache_at, lift_at, copy_scale,
                                  logits, tokens, payloads, snap, pointer_keys, pointer_lifts,
                                  mixture, content, layers)


# ---- the durable-scope envelope -------------------------------------------------------------

@dataclass(frozen=True)
class ScopedSessionIdent:
    """`ScopedSessionIdent` (session_codec.rs:390-427): trimmed, each 1..256 bytes."""
    user_id: str
    project_id: str
    session_id: str

    @staticmethod
    def new(user_id: str, project_id: str, session_id: str) -> "ScopedSessionIdent":
        u, p, s = user_id.strip(), project_id.strip(), session_id.strip()
        if not u or not p or not s or len(u) > 256 or len(p) > 256 or len(s) > 256:
            raise CodecError("session codec: invalid identity scope")
        return ScopedSessionIdent(u, p, s)


def export_scope(scope: ScopedSessionIdent, state: SerializedStackSession) -> bytes:
    """`export_scope` (session_codec.rs:431-452): the UORMEM01 envelope around the snapshot."""
    ScopedSessionIdent.new(scope.user_id, scope.project_id, scope.session_id)
    snap = encode(state)
    out = bytearray(DURABLE_SCOPE_MAGIC)
    out += struct.pack("<I", DURABLE_SCOPE_VERSION)
    for s in (scope.user_id, scope.project_id, scope.session_id):
        _str(out, s)
    out += bytes([0, 1])  # no last entity; the snapshot present
    out += struct.pack("<I", len(snap))
    out += snap
    out += struct.pack("<II", 0, 0)  # no facts, no non-memory turns
    return bytes(out)


def import_scope(data: bytes) -> tuple[ScopedSessionIdent, SerializedStackSession]:
    """`import_scope` (session_codec.rs:456-490)."""
    r = _Reader(bytes(data))
    if r.take(8) != DURABLE_SCOPE_MAGIC:
        raise CodecError("session codec: bad UORMEM01 magic")
    if r.unpack("I") != DURABLE_SCOPE_VERSION:
        raise CodecError("session codec: unsupported UORMEM01 version")
    scope = ScopedSessionIdent.new(r.string(), r.string(), r.string())
    t = r.take(1)[0]
    if t == 1:
        r.string()
    elif t != 0:
        raise CodecError("session codec: bad last_entity tag")
    if r.take(1)[0] != 1:
        raise CodecError("session codec: missing UR4SESS1 snapshot in UORMEM01")
    state = decode(r.take(r.unpack("I")))
    facts, prose = r.unpack("I"), r.unpack("I")
    if facts or prose or r.at != len(r.buf):
        raise CodecError("session codec: unexpected trailing or fact sections")
    return scope, state


# ---- the JSON form --------------------------------------------------------------------------

def to_json(s: SerializedStackSession) -> bytes:
    """serde_json of `SerializedStackSession` (session.rs:1898-1960): the fields in declaration
    order, compact; the empty vectors and absent options that carry `skip_serializing_if` left
    out; the layer enum externally tagged (`{"Recurrence": {"state": .., "history": ..}}`)."""
    d = {"schema": s.schema, "version": s.version, "artifact_sha256": s.artifact_sha256,
         "position": s.position, "cache_at": s.cache_at, "lift_at": s.lift_at,
         "copy_scale_q16": s.copy_scale_q16}
    for name in ("logits", "tokens", "hamming_payloads"):
        if getattr(s, name):
            d[name] = list(getattr(s, name))
    if s.snap_trace is not None:
        d["snap_trace"] = list(s.snap_trace)
    for name in ("pointer_keys", "pointer_lifts", "mixture"):
        if getattr(s, name):
            d[name] = list(getattr(s, name))
    if s.content_readout_sha256 is not None:
        d["content_readout_sha256"] = s.content_readout_sha256
    layers = []
    for layer in s.layers:
        if isinstance(layer, RecurrenceLayer):
            layers.append({"Recurrence": {"state": list(layer.state), "history": list(layer.history)}})
        else:
            layers.append({"Read": {"keys": list(layer.keys), "values": list(layer.values),
                                    "lifts": list(layer.lifts)}})
    d["layers"] = layers
    return json.dumps(d, separators=(",", ":")).encode()


def from_json(data: bytes) -> SerializedStackSession:
    """The reverse of `to_json`, with serde's defaults for the fields it may leave out."""
    try:
        d = json.loads(data)
    except (ValueError, UnicodeDecodeError) as e:
        raise CodecError(f"invalid session JSON: {e}") from None
    if not isinstance(d, dict):
        raise CodecError("invalid session JSON: not an object")
    for name in ("schema", "version", "artifact_sha256", "position", "cache_at", "lift_at", "layers"):
        if name not in d:
            raise CodecError(f"invalid session JSON: missing field `{name}`")
    layers = []
    for entry in d["layers"]:
        if not isinstance(entry, dict) or len(entry) != 1:
            raise CodecError("invalid session JSON: a layer is not one tagged variant")
        (kind, body), = entry.items()
        if kind == "Recurrence":
            layers.append(RecurrenceLayer(list(body["state"]), list(body["history"])))
        elif kind == "Read":
            layers.append(ReadLayer(list(body["keys"]), list(body["values"]), list(body["lifts"])))
        else:
            raise CodecError(f"invalid session JSON: unknown variant `{kind}`")
    return SerializedStackSession(
        d["schema"], d["version"], d["artifact_sha256"], d["position"], d["cache_at"], d["lift_at"],
        d.get("copy_scale_q16", 0), list(d.get("logits", [])), list(d.get("tokens", [])),
        [list(p) for p in d.get("hamming_payloads", [])], d.get("snap_trace"),
        list(d.get("pointer_keys", [])), list(d.get("pointer_lifts", [])),
        list(d.get("mixture", [])), d.get("content_readout_sha256"), layers)
