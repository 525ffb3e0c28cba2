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
from uor_fbs import uorlut

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
