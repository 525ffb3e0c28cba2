"""The oracle equals the reference's own C++ twin at every position of the golden cases.

The vectors in tests/golden/ were written by the twin compiled from the reference's sources
(tests/golden/make_golden.py, fbs_host_sequences at
docs/labs/d11-exporter-float-trunk/instrument/src/host_kernel.cpp:16-29): per position the
chosen token, the kept cells and the Q12 query. The artifacts are rebuilt from their spec and
seed; their table digest guards against generator drift.
"""

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from uor_fbs import synth

MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))


def load_case(name):
    entry = MANIFEST[name]
    spec = synth.Spec(**{k: tuple(v) if isinstance(v, list) else v for k, v in entry["spec"].items()})
    art = synth.make_artifact(spec, entry["seed"])
    data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    return entry, art, data


def check_outputs(entry, data, tok, kept, query):
    np.testing.assert_array_equal(tok, data["out_tokens"])
    np.testing.assert_array_equal(kept, data["out_kept"])
    if "out_query" in data:
        np.testing.assert_array_equal(query, data["out_query"])
    else:
        got = [hashlib.sha256(np.ascontiguousarray(q).tobytes()).hexdigest() for q in query]
        assert got == entry["query_sha256"]


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_oracle_matches_twin_golden(name):
    from make_golden_digest import artifact_digest
    entry, art, data = load_case(name)
    assert artifact_digest(art) == entry["artifact_sha256"], "generator drifted"
    st, tok, kept, query = oracle.sequences(art, data["tokens"], threads=4)
    assert st == 0
    check_outputs(entry, data, tok, kept, query)


def test_golden_cases_are_not_degenerate():
    """Each case chooses many distinct tokens and the snap choices change the outputs."""
    for name in MANIFEST:
        data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
        assert len(np.unique(data["out_tokens"])) >= 20, name
    for base in ("small", "non_square", "tiny_gain"):
        outs = [np.load(os.path.join(GOLDEN, f"{base}_{s}_seq.npz"))["out_tokens"]
                for s in ("g1t1", "g0t0", "g1t0", "g0t1")]
        assert not np.array_equal(outs[0], outs[1])


TRACE = json.load(open(os.path.join(GOLDEN, "trace", "manifest.json")))


@pytest.mark.parametrize("name", sorted(TRACE))
def test_oracle_snap_trace_matches_twin_golden(name):
    """The snap trace (fbs_host_trace_sequences, host_kernel.cpp:31-49, written by
    tests/golden/make_golden_trace.py): every position's roots per layer, 255 where a site is
    served unsnapped or its raw quaternion is zero; the outputs beside it are the golden ones."""
    entry, art, data = load_case(name)
    rec = TRACE[name]
    st, tok, kept, query, trace = oracle.trace_sequences(art, data["tokens"], threads=4)
    assert st == 0 and trace.shape[-1] == rec["stride"]
    check_outputs(entry, data, tok, kept, query)
    if "trace_sha256" in rec:
        assert [hashlib.sha256(t.tobytes()).hexdigest() for t in trace] == rec["trace_sha256"]
    else:
        np.testing.assert_array_equal(trace, np.load(os.path.join(GOLDEN, "trace", f"{name}.npz"))["trace"])
    if oracle.twin_available():
        t2 = oracle.twin_trace_sequences(art, data["tokens"])[4]
        np.testing.assert_array_equal(trace, t2)
