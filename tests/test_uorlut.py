"""The UORLUT01 reader on trained artifacts the reference holds (copied as data fixtures under
tests/golden/trained/, with their SHA-256 and source path): the oracle against the reference
twin's golden vectors on trained weights, and the reader's refusals, which follow the reference
loader's checks (crates/uor-r4-integer/src/stack/format.rs:1202-1518, session.rs:640-735)."""

import glob
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from uor_fbs import synth, uorlut

TRAINED = os.path.join(GOLDEN, "trained")
MANIFEST = json.load(open(os.path.join(TRAINED, "manifest.json")))


def fixture(name):
    entry = MANIFEST[name]
    data = open(os.path.join(TRAINED, entry["artifact"]), "rb").read()
    return entry, data, np.load(os.path.join(TRAINED, f"{name}.npz"))


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_trained_fixture_digest_and_shape(name):
    entry, data, _ = fixture(name)
    assert hashlib.sha256(data).hexdigest() == entry["artifact_sha256"]
    art = uorlut.load(data)
    s = art.spec
    assert (s.vocab, s.width, s.mlp, s.layers, s.context, s.kept) == (4096, 256, 384, 6, 192, 8)
    assert s.raw_gates and s.raw_transition and s.head == 0 and s.reference_shape


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_oracle_matches_twin_on_trained_weights(name):
    entry, data, g = fixture(name)
    art = uorlut.load(data)
    st, tok, kept, query = oracle.sequences(art, g["tokens"], threads=6)
    assert st == 0
    np.testing.assert_array_equal(tok, g["out_tokens"])
    np.testing.assert_array_equal(kept, g["out_kept"])
    assert [hashlib.sha256(q.tobytes()).hexdigest() for q in query] == entry["query_sha256"]


def _split(data):
    n = struct.unpack("<Q", data[8:16])[0]
    header = json.loads(data[16:16 + n])
    end = 16 + n
    start = end + (64 - end % 64) % 64
    return header, data[start:]


def _build(header, body):
    h = json.dumps(header).encode()
    end = 16 + len(h)
    return uorlut.MAGIC + struct.pack("<Q", len(h)) + h + b"\0" * ((64 - end % 64) % 64) + body


def test_rebuilt_container_loads_identically():
    _, data, _ = fixture(sorted(MANIFEST)[0])
    a = uorlut.load(data)
    b = uorlut.load(_build(*_split(data)))
    np.testing.assert_array_equal(a.writer_table, b.writer_table)
    np.testing.assert_array_equal(a.layers[3].maps["mlp_up"][1], b.layers[3].maps["mlp_up"][1])


def _mutant(data, fn):
    header, body = _split(data)
    body = bytearray(body)
    fn(header, body)
    return _build(header, bytes(body))


def _table(header, name):
    return next(t for t in header["tables"] if t["name"] == name)


@pytest.mark.parametrize("case", [
    "magic", "header_length", "schema", "record", "projection", "pattern", "span", "length",
    "duplicate", "missing", "route_atom", "route_state", "grid_code", "snap"])
def test_refuses_malformed_containers(case):
    _, data, _ = fixture(sorted(MANIFEST)[0])
    if case == "magic":
        bad = b"UORLUT02" + data[8:]
    elif case == "header_length":
        bad = data[:8] + struct.pack("<Q", len(data)) + data[16:]
    else:
        def edit(h, body):
            if case == "schema":
                h["schema"] = "uor-r4.lut-stack/6"
            elif case == "record":
                h["hamming"] = {}
            elif case == "projection":
                h["shape"]["projection"] = "dense"
            elif case == "pattern":
                h["shape"]["pattern"] = "rrarrr"
            elif case == "span":
                _table(h, "writer.table")["span"]["offset"] = len(body)
            elif case == "length":
                _table(h, "l0.conv_bias")["len"] -= 1
            elif case == "duplicate":
                h["tables"].append(dict(_table(h, "l0.conv_bias")))
            elif case == "missing":
                h["tables"] = [t for t in h["tables"] if t["name"] != "l2.gate_bias"]
            elif case in ("route_atom", "route_state"):
                off = _table(h, "l1.rec_out.fbs")["span"]["offset"]
                word = 0x7FFF if case == "route_atom" else (64 << 16)
                body[off:off + 4] = struct.pack("<I", word)
            elif case == "grid_code":
                off = _table(h, "l0.rec_norm_gain")["span"]["offset"]
                body[off:off + 2] = struct.pack("<h", 8)  # exponent field 0
            elif case == "snap":
                h["shape"]["raw_transition"] = False
        bad = _mutant(data, edit)
    with pytest.raises(uorlut.UorlutError):
        uorlut.load(bad)


@pytest.mark.skipif(not os.path.isdir("/root/reference/docs"), reason="reference checkout absent")
def test_every_trained_artifact_in_the_reference_loads():
    files = sorted(glob.glob("/root/reference/docs/**/*.uorlut", recursive=True))
    assert len(files) >= 50
    for f in files:
        art = uorlut.load(f)
        assert art.spec.width == 256 and art.spec.layers == 6


# ---- Hamming reads (lut-stack/6, and /7 or /8 with a `hamming` record) ---------------------
# No container the reference holds has Hamming reads, so they are added to a trained fixture
# (uorlut.add_hamming, as the reference's section adders append, format.rs:2730-2783) with
# seeded reads; the reader's refusals follow StackHamming::check (format.rs:336-430) and
# hamming_image (hamming.rs:58-110).

HAM = synth.HammingSpec(heads=8, depths=(2, 6), kept=16, asks=(False, True), carry_rows=4)


def hamming_fixture(h=HAM):
    _, data, _ = fixture(sorted(MANIFEST)[0])
    reads = synth.hamming_reads(uorlut.load(data).spec, h, 7)
    return data, uorlut.add_hamming(data, h, reads), reads


def test_hamming_reads_load_as_added():
    data, added, reads = hamming_fixture()
    art = uorlut.load(added)
    assert json.loads(added[16:16 + struct.unpack("<Q", added[8:16])[0]])["schema"] == "uor-r4.lut-stack/7"
    h = art.hamming
    assert (h.heads, h.depths, h.kept, h.asks, h.carry_rows, h.copy_key) == (8, (2, 6), 16, (False, True), 4, 1)
    for a, b in zip(art.hamming_reads, reads):
        assert a.depth == b.depth
        for part in ("query_rotation", "key_rotation", "value_rotation", "margin", "weight", "ask", "carry"):
            x, y = getattr(a, part), getattr(b, part)
            assert (x is None) == (y is None) and (x is None or np.array_equal(x, y)), part
    # The reads change what the model decodes (the oracle, a few steps).
    plain = uorlut.load(data)
    prompts = (np.arange(24, dtype=np.uint32).reshape(2, 12) * 37) % 50
    assert not np.array_equal(oracle.decode(art, prompts, 6)["reply"], oracle.decode(plain, prompts, 6)["reply"])


def test_a_stack_without_memory_names_schema_6():
    _, data, _ = fixture(sorted(MANIFEST)[0])
    header, body = _split(data)
    del header["memory"]
    header["schema"] = "uor-r4.lut-stack/5"
    plain = _build(header, body)
    uorlut.load(plain)
    reads = synth.hamming_reads(uorlut.load(plain).spec, HAM, 3)
    added = uorlut.add_hamming(plain, HAM, reads)
    assert _split(added)[0]["schema"] == "uor-r4.lut-stack/6"
    assert uorlut.load(added).hamming.depths == (2, 6)


@pytest.mark.parametrize("case", [
    "place", "unknown", "missing_field", "exponent", "depth_zero", "depth_order", "depth_past",
    "odd_heads", "wide_heads", "copy_keys_equal", "longest_without_latest", "kept_zero",
    "asks_all_off", "carry_without_ask", "carry_reach", "ask_unnamed", "ask_missing",
    "margin_zero", "section_length", "schema_6_with_memory"])
def test_refuses_malformed_hamming_reads(case):
    _, added, _ = hamming_fixture()

    def edit(h, body):
        r = h["hamming"]
        if case == "place":
            r["place"] = {"stop": [1], "arm": [2], "open": [3]}
        elif case == "unknown":
            r["bogus"] = 1
        elif case == "missing_field":
            del r["kept"]
        elif case == "exponent":
            r["margin_exp"] = -15
        elif case == "depth_zero":
            r["depths"] = [0, 6]
        elif case == "depth_order":
            r["depths"] = [6, 2]
        elif case == "depth_past":
            r["depths"] = [2, 7]
        elif case == "odd_heads":
            r["heads"] = 7
        elif case == "wide_heads":
            r["heads"] = 2  # 128 coordinates a head
        elif case == "copy_keys_equal":
            r["copy_keys"] = [1, 1, 1, 1]
        elif case == "longest_without_latest":
            r["copy_longest"] = [1, 2]
        elif case == "kept_zero":
            r["kept"] = 0
        elif case == "asks_all_off":
            r["asks"] = [False, False]
            del r["carry_rows"]
        elif case == "carry_without_ask":
            r["asks"] = [True, False]
        elif case == "carry_reach":
            r["carry_rows"] = 4097
        elif case == "ask_unnamed":
            del r["asks"]
            del r["carry_rows"]
        elif case == "ask_missing":
            h["tables"] = [t for t in h["tables"] if t["name"] != "hamming.d6.ask"]
        elif case == "margin_zero":
            off = _table(h, "hamming.d2.margin")["span"]["offset"]
            body[off:off + 4] = struct.pack("<i", 0)
        elif case == "section_length":
            t = _table(h, "hamming.d2.weight")
            t["len"] -= 1
            t["span"]["bytes"] -= 4
        elif case == "schema_6_with_memory":
            h["schema"] = "uor-r4.lut-stack/6"
    with pytest.raises(uorlut.UorlutError):
        uorlut.load(_mutant(added, edit))
