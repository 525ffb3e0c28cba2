"""The session snapshot encodings against the reference's committed contract fixture and its own
codec tests (crates/uor-r4-integer/src/session_codec.rs:462-608,
crates/uor-r4-integer/tests/session_codec_interop_fixture.rs,
crates/uor-r4-object-store/tests/integer_session_interop.rs).

`tests/golden/session/integer_ur4sess1_v1.hex` is the reference's fixture file
(crates/uor-r4-object-store/tests/fixtures/integer_ur4sess1_v1.hex), copied as data: the
bytes its integer codec emits for the contract state below, pinned there by SHA-256
ef0ffeee...78b1 on both sides of the reference's crate boundary.
"""

import hashlib
import os
import struct

import pytest

from conftest import GOLDEN
from uor_fbs.session_codec import (DURABLE_SCOPE_MAGIC, DURABLE_SCOPE_VERSION, MAGIC, MAGIC_CONTENT,
                                   MAGIC_PAYLOADS, STACK_SESSION_SCHEMA, CodecError, ReadLayer,
                                   RecurrenceLayer, ScopedSessionIdent, SerializedStackSession,
                                   decode, encode, export_scope, from_json, import_scope, to_json)

FIXTURE_SHA256 = "ef0ffeeeeb82baa7fa83186a6fc3416cfc660a5d993f2d990f8a5c2893e478b1"
I32_MIN, I32_MAX = -(1 << 31), (1 << 31) - 1
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1
U64_MAX = (1 << 64) - 1


def fixture() -> bytes:
    text = open(os.path.join(GOLDEN, "session", "integer_ur4sess1_v1.hex")).read()
    return bytes.fromhex("".join(text.split()))


def sample() -> SerializedStackSession:
    """The reference tests' contract state (session_codec.rs:466-497)."""
    return SerializedStackSession(
        schema=STACK_SESSION_SCHEMA, version=1, artifact_sha256="ab" * 32, position=7,
        cache_at=7 * 288, lift_at=7 * 6, copy_scale_q16=65536,
        logits=[-3, 0, 65536, I32_MIN, I32_MAX], tokens=[0, 5, 77, 4095], hamming_payloads=[],
        snap_trace=[0, 119], pointer_keys=[1, -2, 3], pointer_lifts=[U64_MAX, 0, 1 << 62],
        mixture=[9, -9], content_readout_sha256=None,
        layers=[RecurrenceLayer([I64_MIN, -1, 0, 1, I64_MAX], [4, -4, 16]),
                ReadLayer([11, 12], [-11, -12], [1, 2, 3, 4])])


def test_fixture_is_the_reference_contract():
    assert hashlib.sha256(fixture()).hexdigest() == FIXTURE_SHA256
    assert encode(sample()) == fixture()
    assert decode(fixture()) == sample()


def test_fixture_header_fields():
    # integer_session_interop.rs:44-52: the store's header view of the same bytes.
    s = decode(fixture())
    assert s.position == 7 and s.tokens == [0, 5, 77, 4095]
    assert s.logits == [-3, 0, 65536, I32_MIN, I32_MAX]
    assert fixture()[:8] == MAGIC


def test_round_trip_and_magic_by_content():
    s = sample()
    assert decode(encode(s)) == s
    s.content_readout_sha256 = "cd" * 32
    b = encode(s)
    assert b[:8] == MAGIC_CONTENT and decode(b) == s
    s.hamming_payloads = [[1, -2, I64_MIN], [], [I64_MAX]]
    b = encode(s)
    assert b[:8] == MAGIC_PAYLOADS and decode(b) == s
    s.content_readout_sha256 = None
    assert decode(encode(s)) == s


def test_empty_vectors_round_trip():
    s = sample()
    s.logits, s.tokens, s.snap_trace = [], [], None
    s.pointer_keys, s.pointer_lifts, s.mixture, s.layers = [], [], [], []
    assert decode(encode(s)) == s


def test_refuses_bad_magic_trailing_and_truncation():
    b = bytearray(encode(sample()))
    b[0] ^= 1
    with pytest.raises(CodecError, match="bad magic"):
        decode(bytes(b))
    with pytest.raises(CodecError, match="trailing"):
        decode(encode(sample()) + b"\0")
    full = encode(sample())
    for cut in (1, 9, 40, len(full) // 2, len(full) - 1):
        with pytest.raises(CodecError, match="truncated"):
            decode(full[:cut])


def test_refuses_an_oversized_count_without_allocating():
    # session_codec.rs:568-583: a u64::MAX varint count for the logits.
    out = bytearray(MAGIC)
    for s in (STACK_SESSION_SCHEMA,):
        out += struct.pack("<I", len(s)) + s.encode()
    out += struct.pack("<I", 1)
    out += struct.pack("<I", 64) + b"ab" * 32
    out += struct.pack("<QQQi", 1, 288, 6, 65536)
    out += bytes([0xFF] * 9 + [0x01])  # v64 u64::MAX
    with pytest.raises(CodecError):
        decode(bytes(out))
    # A varint longer than 64 bits.
    with pytest.raises(CodecError, match="overflow|truncated"):
        decode(bytes(out[:-10]) + bytes([0xFF] * 10 + [0x01]))


def test_refuses_bad_tags_and_utf8():
    full = bytearray(encode(sample()))
    # The snap-trace tag follows the tokens: locate it from the layout.
    at = 8 + 4 + len(STACK_SESSION_SCHEMA) + 4 + 4 + 64 + 8 * 3 + 4
    at += 1 + 5 * 4 + 1 + 4 * 4
    assert full[at] == 1
    bad = bytearray(full)
    bad[at] = 2
    with pytest.raises(CodecError, match="snap_trace tag"):
        decode(bytes(bad))
    bad = bytearray(full)
    bad[12] = 0xFF  # first schema byte
    with pytest.raises(CodecError, match="utf-8"):
        decode(bytes(bad))


def test_durable_scope_envelope():
    # session_codec.rs:586-606 and session_codec_interop_fixture.rs:78-99.
    scope = ScopedSessionIdent.new("alice", "uor-r4", "s1")
    env = export_scope(scope, sample())
    assert env[:8] == DURABLE_SCOPE_MAGIC and DURABLE_SCOPE_MAGIC == b"UORMEM01"
    assert struct.unpack("<I", env[8:12])[0] == DURABLE_SCOPE_VERSION == 1
    assert fixture() in env  # the envelope embeds the exact snapshot bytes
    got_scope, got = import_scope(env)
    assert got_scope == scope and got == sample()
    with pytest.raises(CodecError):
        import_scope(bytes([env[0] ^ 1]) + env[1:])
    with pytest.raises(CodecError):
        import_scope(env + b"\0")
    with pytest.raises(CodecError):
        ScopedSessionIdent.new("", "proj", "sess")
    with pytest.raises(CodecError):
        ScopedSessionIdent.new("u" * 257, "p", "s")
    assert ScopedSessionIdent.new("  u ", "p", "s").user_id == "u"


def test_json_form():
    s = sample()
    text = to_json(s)
    assert from_json(text) == s
    head = text[:120].decode()
    # serde's order and compact form: the schema first, no spaces.
    assert head.startswith('{"schema":"uor-r4.stack-session/1","version":1,"artifact_sha256":"abab')
    assert b'"layers":[{"Recurrence":{"state":[-9223372036854775808,-1,0,1,9223372036854775807]' in text
    assert b'{"Read":{"keys":[11,12],"values":[-11,-12],"lifts":[1,2,3,4]}}' in text
    # Empty vectors and absent options are left out (skip_serializing_if), and read back as
    # serde's defaults.
    e = sample()
    e.logits, e.tokens, e.snap_trace, e.pointer_keys, e.pointer_lifts, e.mixture = [], [], None, [], [], []
    t = to_json(e)
    for name in (b'"logits"', b'"tokens"', b'"snap_trace"', b'"pointer_keys"', b'"mixture"',
                 b'"hamming_payloads"', b'"content_readout_sha256"'):
        assert name not in t
    assert b'"copy_scale_q16":65536' in t
    assert from_json(t) == e
    with pytest.raises(CodecError):
        from_json(b'{"schema":"x"}')
    with pytest.raises(CodecError):
        from_json(b"not json")
