"""The HIP path (libuor_fbs_hip.so through its C ABI) against the reference twin's golden vectors
and the oracle, bit for bit: every position's chosen token, kept drawers and Q12 query, greedy
decode replies, exported state and window, score counts, and the reference's status codes.

Cases follow the reference's own parity tests (docs/labs/d11-exporter-float-trunk/instrument/
tests/parity.rs:50-183: single tokens over the whole vocabulary, LCG sequences of full context,
all four snap choices) plus BASELINE's configurations at reduced batch and length, whose
extended semantics (window W, keyed Zipf drawers, int8 table, nearest head) the oracle defines.
"""

import hashlib
import json
import os
from dataclasses import replace

import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from uor_fbs import synth
from uor_fbs.hip import FbsError, Model

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("block_waves")]

MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))


def load_case(name):
    entry = MANIFEST[name]
    spec = synth.Spec(**{k: tuple(v) if isinstance(v, list) else v for k, v in entry["spec"].items()})
    return entry, synth.make_artifact(spec, entry["seed"]), np.load(os.path.join(GOLDEN, f"{name}.npz"))


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_golden_twin_vectors(name):
    entry, art, data = load_case(name)
    print(f"case {name} tokens {data['tokens'].shape}", flush=True)
    model = Model(art)
    tok, kept, query = model.sequences(data["tokens"])
    np.testing.assert_array_equal(tok, data["out_tokens"])
    np.testing.assert_array_equal(kept, data["out_kept"])
    if "out_query" in data:
        np.testing.assert_array_equal(query, data["out_query"])
    else:
        got = [hashlib.sha256(np.ascontiguousarray(q).tobytes()).hexdigest() for q in query]
        assert got == entry["query_sha256"]


def reduced(name, **kw):
    spec = synth.CONFIGS[name]
    return replace(spec, **kw)


EXTENDED = {
    # BASELINE C1/C2 semantics: width 128, window 8, 64 keyed drawers (uniform) probing 4.
    "c2_ext": (reduced("c2", context=48), 31, lambda s: synth.uniform_prompts(s.vocab, 6, 40, 41)),
    # C3/C4: width 256, window 16, 256 Zipf drawers (max 512) probing 8, vocab 32768.
    "c3_ext": (reduced("c3", context=24), 33, lambda s: synth.zipf_prompts(s.vocab, 4, 20, 43)),
    # C5: width 512, window 32, 1024 Zipf drawers probing 16, int8 table (2 layers to keep the
    # oracle quick).
    "c5_ext": (reduced("c5", context=16, layers=2), 35, lambda s: synth.uniform_prompts(s.vocab, 2, 12, 45)),
    # Snapped gates and transition on an extended shape.
    "c2_snapped": (replace(reduced("c2", context=24, layers=2), raw_gates=False, raw_transition=False),
                   37, lambda s: synth.uniform_prompts(s.vocab, 3, 16, 47)),
    # Mixed snap choices, nearest head, a width that is not a power of two.
    "nearest": (replace(synth.NON_SQUARE, head=1, raw_gates=False), 39,
                lambda s: synth.uniform_prompts(s.vocab, 4, 16, 49)),
    "width96": (synth.Spec(vocab=700, width=96, mlp=160, layers=2, context=20, kept=3, window=5,
                           drawers=48, probes=6, zipf_drawers=1.3, max_drawer=40), 40,
                lambda s: synth.uniform_prompts(s.vocab, 5, 20, 50)),
    "width768": (synth.Spec(vocab=1024, width=768, mlp=96, layers=1, context=8, kept=4), 41,
                 lambda s: synth.uniform_prompts(s.vocab, 2, 8, 51)),
}


@pytest.mark.parametrize("name", sorted(EXTENDED))
def test_extended_shapes_match_oracle(name):
    spec, seed, make_tokens = EXTENDED[name]
    art = synth.make_artifact(spec, seed)
    tokens = make_tokens(spec)
    print(f"case {name} spec {spec} tokens {tokens.shape}", flush=True)
    st, want_t, want_k, want_q = oracle.sequences(art, tokens, threads=8)
    assert st == 0
    tok, kept, query = Model(art).sequences(tokens)
    np.testing.assert_array_equal(query, want_q)
    np.testing.assert_array_equal(kept, want_k)
    np.testing.assert_array_equal(tok, want_t)
    assert len(np.unique(tok)) > 4  # the case is not degenerate


def test_block_waves_follow_the_setting(block_waves, monkeypatch):
    art = synth.make_artifact(synth.SMALL, 1)
    assert Model(art).block_waves(64) == (2 if block_waves == "paired" else 1)
    monkeypatch.delenv("UOR_FBS_BLOCK_WAVES")
    model = Model(art)  # the library's choice: paired blocks at every batch size
    assert model.block_waves(1024) == 2 and model.block_waves(1 << 20) == 2


def test_decode_matches_oracle_and_resumes():
    spec = reduced("c2", context=64, layers=3)
    art = synth.make_artifact(spec, 51)
    prompts = synth.uniform_prompts(spec.vocab, 7, 12, 61)
    print("decode c2 layers 3", flush=True)
    model = Model(art)
    want = oracle.decode(art, prompts, gen=30, threads=8)
    got = model.decode(prompts, gen=30)
    np.testing.assert_array_equal(got["reply"], want["reply"])
    np.testing.assert_array_equal(got["state"], want["state"])
    np.testing.assert_array_equal(got["history"], want["history"])
    np.testing.assert_array_equal(got["position"], want["position"])
    # Split in two halves through the exported state (save_state/restore_state, session.rs:2777).
    first = model.decode(prompts, gen=9)
    second = model.decode(first["reply"][:, -1:], gen=20, in_state=first["state"],
                          in_history=first["history"], in_position=first["position"])
    np.testing.assert_array_equal(second["reply"][:, 1:], want["reply"][:, 11:])
    np.testing.assert_array_equal(second["state"], want["state"])
    np.testing.assert_array_equal(second["history"], want["history"])


def test_score_matches_oracle():
    spec = reduced("c3", context=16, layers=2)
    art = synth.make_artifact(spec, 53)
    rows = synth.zipf_prompts(spec.vocab, 9, 16, 63)
    # Rows that follow the model's own choices score every position.
    st, tok, _, _ = oracle.sequences(art, rows[:1], threads=1)
    print("score c3 layers 2", flush=True)
    model = Model(art)
    want_st, want_matches, want_argmin = oracle.score(art, rows, threads=8)
    matches, argmin = model.score(rows)
    np.testing.assert_array_equal(argmin, want_argmin)
    assert matches == want_matches
    matches2, none = model.score(rows, want_argmin=False)
    assert matches2 == matches and none is None


def test_status_codes():
    art = synth.make_artifact(synth.SMALL, 1)
    model = Model(art)
    print("status codes", flush=True)
    with pytest.raises(FbsError) as e:
        model.sequences(np.array([[1, 2, 256]], np.uint32))
    assert e.value.code == 1
    with pytest.raises(FbsError) as e:
        model.sequences(np.zeros((1, 9), np.uint32))
    assert e.value.code == 2
    with pytest.raises(FbsError) as e:
        model.decode(np.zeros((1, 4), np.uint32), gen=5)
    assert e.value.code == 2
    # The sequences before and after a failing one still run.
    ok = model.sequences(np.array([[3, 4, 5]], np.uint32))[0]
    assert ok.shape == (1, 3)


def test_run_twice_is_identical_and_batch_independent():
    spec = reduced("c2", context=32, layers=2)
    art = synth.make_artifact(spec, 55)
    tokens = synth.uniform_prompts(spec.vocab, 40, 32, 65)
    model = Model(art)
    a = model.sequences(tokens)
    b = model.sequences(tokens)
    one = model.sequences(tokens[17:18])
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    for x, y in zip(a, one):
        np.testing.assert_array_equal(x[17:18], y)


def test_decode_batch_above_the_grid_matches_oracle():
    # More sequences than resident blocks (at most one paired block per SIMD, 1,024 on MI355X):
    # each block decodes several sequences in turn, each from its own fresh session. Sequences
    # on both sides of the block boundaries must equal the oracle's, state and window included.
    spec = reduced("c2", context=24, layers=2)
    art = synth.make_artifact(spec, 58)
    prompts = synth.uniform_prompts(spec.vocab, 2600, 8, 68)
    model = Model(art)
    out = model.decode(prompts, gen=12)
    pick = np.array([0, 1, 1023, 1024, 1025, 2047, 2048, 2049, 2599])
    ref = oracle.decode(art, prompts[pick], 12, threads=4)
    assert ref["status"] == 0
    np.testing.assert_array_equal(out["reply"][pick], ref["reply"])
    np.testing.assert_array_equal(out["state"][pick], ref["state"])
    np.testing.assert_array_equal(out["history"][pick], ref["history"])
    np.testing.assert_array_equal(out["position"][pick], ref["position"])


def test_repeated_queries_reuse_the_writer_exactly():
    # A token fed again and again settles the state, so consecutive queries repeat exactly and
    # the kernel takes the writer's last result instead of scanning again. Every position's
    # token, kept drawers and query must still equal the oracle's.
    spec = reduced("c3", context=96, layers=2)
    art = synth.make_artifact(spec, 57)
    rows = np.repeat(np.array([[11], [4703], [9200], [31000]], np.uint32), 96, axis=1)
    print("repeated tokens c3 layers 2", flush=True)
    st, want_t, want_k, want_q = oracle.sequences(art, rows, threads=4)
    assert st == 0
    tok, kept, query = Model(art).sequences(rows)
    repeats = (query[:, 1:] == query[:, :-1]).all(-1).sum()
    assert repeats > 20, repeats  # the reuse path runs
    np.testing.assert_array_equal(query, want_q)
    np.testing.assert_array_equal(kept, want_k)
    np.testing.assert_array_equal(tok, want_t)


TRACE = json.load(open(os.path.join(GOLDEN, "trace", "manifest.json")))


@pytest.mark.parametrize("name", sorted(TRACE))
def test_snap_trace_matches_the_golden_twin(name):
    """uor_fbs_trace_sequences against the twin's fbs_host_trace_sequences (host_kernel.cpp:31-49,
    tests/golden/make_golden_trace.py): every position's roots, and the outputs beside them."""
    entry, art, data = load_case(name)
    rec = TRACE[name]
    print(f"trace {name} tokens {data['tokens'].shape}", flush=True)
    tok, kept, query, trace = Model(art).trace_sequences(data["tokens"])
    np.testing.assert_array_equal(tok, data["out_tokens"])
    np.testing.assert_array_equal(kept, data["out_kept"])
    assert trace.shape[-1] == rec["stride"]
    if "trace_sha256" in rec:
        assert [hashlib.sha256(t.tobytes()).hexdigest() for t in trace] == rec["trace_sha256"]
    else:
        np.testing.assert_array_equal(trace, np.load(os.path.join(GOLDEN, "trace", f"{name}.npz"))["trace"])
