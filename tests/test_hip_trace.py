"""The traced kernels (uor_fbs_decision_sequences: the Hamming trace and the decision trace with
the forced replay, session.rs:2361-2370, 2438-2515) against the oracle, record for record and
byte for byte: every head's query, key and kept set, every layer's rate scores and entries,
under forced buckets and codes, at one, two and four quaternions a lane, with copy, type and ask
heads, the rules and the place read; and the reference's refusals through the C ABI.
"""

from dataclasses import replace

import ctypes as C
import numpy as np
import pytest

import oracle
from test_place_oracle import P_TALK, place_trunk
from uor_fbs import hip, synth
from uor_fbs.hip import FbsError, Model
from uor_fbs.trace import DecisionForceWindow, ForcedBucket, ForcedCode, TraceLayout

pytestmark = pytest.mark.gpu

H = synth.HammingSpec
CASES = {
    "w64_copy_type": (synth.Spec(vocab=96, width=64, mlp=64, layers=3, context=48, kept=4, head=1),
                      H(heads=4, depths=(1, 3), kept=4)),
    "w64_rules_ask": (synth.Spec(vocab=96, width=64, mlp=96, layers=3, context=48, kept=4, head=1),
                      H(heads=8, depths=(2, 3), kept=6, asks=(False, True), carry_rows=2,
                        copy_keys=(1, 2, 1, 2), copy_latest=True)),
    "w512": (synth.Spec(vocab=256, width=512, mlp=128, layers=2, context=40, kept=4, head=1),
             H(heads=16, depths=(1, 2), kept=8, asks=(True, False))),
    "w1024_writer": (synth.Spec(vocab=256, width=1024, mlp=128, layers=2, context=32, kept=8),
                     H(heads=16, depths=(1, 2), kept=5, rule=3)),
    "plain_nearest": (synth.Spec(vocab=300, width=128, mlp=128, layers=3, context=40, kept=8,
                                 head=1, window=5), None),
}


def case(name, seed=13):
    spec, ham = CASES[name]
    art = synth.make_artifact(replace(spec, hamming=ham), seed)
    toks = (synth.uniform_prompts(spec.vocab, 3, spec.context - 4, seed + 1) % 14).astype(np.uint32)
    return art, toks


def check(art, toks, decisions, force=None):
    got = Model(art).decision_trace(toks, decisions, force)
    st, t2, q2, raw2 = oracle.decision_sequences(art, toks, decisions, force, threads=4)
    assert st == 0
    np.testing.assert_array_equal(got["tokens"], t2)
    np.testing.assert_array_equal(got["query"], q2)
    np.testing.assert_array_equal(got["raw"], raw2)
    return got


@pytest.mark.parametrize("name", sorted(CASES))
def test_the_traces_match_the_oracle(name):
    art, toks = case(name)
    print(f"trace {name} {toks.shape}", flush=True)
    decisions = art.spec.head == 1
    got = check(art, toks, decisions)
    if art.hamming is None:
        return
    check(art, toks, False)
    # The trace changes nothing the step serves.
    tok, _, query = Model(art).sequences(toks)
    np.testing.assert_array_equal(got["tokens"], tok)
    np.testing.assert_array_equal(got["query"], query)


@pytest.mark.parametrize("name", ["w64_copy_type", "w64_rules_ask", "w512", "plain_nearest"])
def test_the_forced_replay_matches_the_oracle(name):
    art, toks = case(name)
    print(f"forced {name}", flush=True)
    lay = TraceLayout.of(art, True)
    rng = np.random.default_rng(3)
    windows = []
    for i in range(len(toks)):
        w = DecisionForceWindow(position=i)
        for _ in range(6):
            w.buckets.append(ForcedBucket(int(rng.integers(0, toks.shape[1])), int(rng.integers(0, lay.layers)),
                                          int(rng.integers(0, lay.lanes)), int(rng.integers(0, 16))))
        w.buckets = list({(b.step, b.layer, b.lane): b for b in w.buckets}.values())
        if lay.depths:
            seen = set()
            for _ in range(8):
                r = int(rng.integers(0, len(lay.depths)))
                hh = int(rng.integers(0, lay.served[r]))
                role = "query" if rng.random() < 0.5 else "key"
                step = int(rng.integers(1, toks.shape[1]))
                if (step, r, hh, role) in seen:
                    continue
                seen.add((step, r, hh, role))
                w.codes.append(ForcedCode(step, lay.depths[r], hh, role, int(rng.integers(0, 1 << 62))))
        windows.append(w)
    got = check(art, toks, True, windows)
    assert not np.array_equal(got["query"], Model(art).sequences(toks)[2])


def test_the_place_read_is_traced_at_its_open_rows():
    _, placed = place_trunk()
    toks = np.asarray([P_TALK], np.uint32)
    check(placed, toks, False)


def test_the_reference_refusals():
    art, toks = case("w64_copy_type")
    snapped = synth.make_artifact(replace(CASES["w64_copy_type"][0], raw_transition=False,
                                          hamming=CASES["w64_copy_type"][1]), 13)
    with pytest.raises(FbsError, match="unsnapped"):
        Model(snapped).decision_trace(toks, True)
    writer, toks_w = case("w1024_writer")
    with pytest.raises(FbsError, match="nearest head"):
        Model(writer).decision_trace(toks_w, True)
    # The C ABI's own checks, past the host's: a key at step 0, a code with a place read.
    model = Model(art)
    L = hip.lib()
    S, n = toks.shape
    lay = TraceLayout.of(art, True)
    R, Hh = len(lay.depths), lay.heads
    codes = np.zeros((S, n, R, Hh, 2), np.uint64)
    mask = np.zeros((S, n, R, Hh), np.uint8)
    mask[0, 0, 0, 0] = 2
    out_t = np.zeros((S, n), np.uint32)
    raw = np.zeros((S, n, lay.stride), np.uint8)
    vp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    assert L.uor_fbs_decision_sequences(model.handle, vp(toks), S, n, 1, None, vp(codes), vp(mask),
                                        vp(out_t), None, vp(raw)) != 0
    assert b"step 0" in L.uor_fbs_last_error()
    _, placed = place_trunk()
    pm = Model(placed)
    pl = TraceLayout.of(placed, False)
    codes = np.zeros((1, 8, len(pl.depths), pl.heads, 2), np.uint64)
    mask = np.zeros((1, 8, len(pl.depths), pl.heads), np.uint8)
    mask[0, 3, 0, 0] = 1
    t8 = np.asarray([P_TALK[:8]], np.uint32)
    raw = np.zeros((1, 8, pl.stride), np.uint8)
    out_t = np.zeros((1, 8), np.uint32)
    assert L.uor_fbs_decision_sequences(pm.handle, vp(t8), 1, 8, 0, None, vp(codes), vp(mask),
                                        vp(out_t), None, vp(raw)) != 0
    assert b"place read" in L.uor_fbs_last_error()


def test_a_session_records_the_traces_of_its_served_steps():
    # The session's traces (session.rs:2361-2370, 2438-2515): the Hamming trace from the step
    # after it is turned on, taken and still on; the decision trace from a fresh session, taken
    # and off; both the records of the teacher-forced window over the same tokens.
    from uor_fbs.session import Session, SessionError, SessionPool
    art, toks = case("w64_copy_type")
    row = toks[0]
    want = Model(art).decision_trace(toks[:1], False)["steps"][0]
    pool = SessionPool(Model(art), capacity=2)
    s = Session(pool)
    assert s.take_hamming_trace() is None
    s.feed(row[:5])
    s.set_hamming_trace(True)
    s.feed(row[5:9])
    for tok in row[9:12]:
        s.serve_step(int(tok))
    got = s.take_hamming_trace()
    assert got == [r for step in want[5:12] for r in step]
    assert s.take_hamming_trace() == []
    d = Session(pool)
    d.set_decision_trace()
    d.feed(row[:7])
    d.serve_step(int(row[7]))
    steps = d.take_decision_trace()
    full = Model(art).decision_trace(toks[:1], True)["steps"][0][:8]
    for st in full:
        st.nearest = None
    assert steps == full
    assert d.take_decision_trace() is None
    with pytest.raises(SessionError):
        d.set_decision_trace()  # the session has stepped
