"""The serving session's snap-trace bookkeeping (uor_fbs/session.py: enable_snap_trace, snap_trace,
save_state, restore_state, reset; stack/session.rs:2570-2620, :2728-2737, :2827-2845,
:3172-3190) on the CPU: `Session` runs over a stand-in pool whose launches come from the oracle's
teacher-forced trace (the GPU test in test_hip_session.py runs the same calls on the device)."""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import session_codec, synth
from uor_fbs.session import ModelInfo, Session, serve_steps, transition_roots

SPEC = replace(synth.CONFIGS["c2"], context=40, layers=2, raw_transition=False, raw_gates=False)


class OraclePool:
    """The pool surface Session uses, each launch answered by the oracle over the slot's whole
    token history (a session's state is a function of its tokens)."""

    def __init__(self, art, capacity=4):
        self.model = type("M", (), {"art": art})()
        self.info = ModelInfo.of(art)
        self.hist = {k: [] for k in range(capacity)}
        self.free = list(range(capacity))

    def acquire(self, slot=None):
        return self.free.pop(0) if slot is None else (self.free.remove(slot), slot)[1]

    def release(self, slot):
        self.free.append(slot)

    def set_slide(self, slot, on):
        pass

    def clear(self, slots):
        for s in slots:
            self.hist[s] = []

    def run(self, slots, tokens, gen=0, native=False, trace=False):
        assert gen == 0
        out = dict(reply=[], status=[], kept=[], query=[], trace=[])
        for s, row in zip(slots, np.asarray(tokens)):
            start = len(self.hist[s])
            self.hist[s] += [int(t) for t in row]
            st, tok, kept, query, tr = oracle.trace_sequences(
                self.model.art, np.asarray([self.hist[s]], np.uint32))
            assert st == 0
            out["reply"].append(tok[0, -1:])
            out["status"].append(0)
            out["kept"].append(kept[0, -1])
            out["query"].append(query[0, -1])
            out["trace"].append(tr[0, start:])
        return out

    def read(self, slot):
        i = self.info
        return (np.zeros(i.state_words, np.int64), np.zeros(i.history_words, np.int32),
                len(self.hist[slot]))

    def write(self, slot, state, history, position):
        self.hist[slot] = list(self.restored)


@pytest.fixture(scope="module")
def art():
    return synth.make_artifact(SPEC, 41)


def test_trace_records_the_transition_roots(art):
    tokens = synth.uniform_prompts(SPEC.vocab, 1, 16, 43)[0]
    _, _, _, _, tr = oracle.trace_sequences(art, tokens[None])
    lanes, per = SPEC.width // 4, SPEC.layers * SPEC.width // 4
    want = transition_roots(tr[0], SPEC.layers, lanes)
    assert (want < 120).all()
    pool = OraclePool(art)
    a = Session(pool)
    assert a.snap_trace() is None
    a.feed(tokens[:3])
    a.enable_snap_trace()                       # from position 3
    a.feed(tokens[3:7])
    for t in tokens[7:10]:
        a.serve_step(int(t))
    got = a.snap_trace()
    assert [e.root for e in got] == want[3 * per:10 * per].tolist()
    assert [(e.layer, e.position, e.lane) for e in got[:lanes + 1]] == \
        [(0, 3, k) for k in range(lanes)] + [(1, 3, 0)]
    assert got[-1].position == 9 and got[-1].layer == SPEC.layers - 1
    assert a.save_state().snap_trace is None    # not traced from position 0

    b = Session(pool)
    b.enable_snap_trace()
    b.feed(tokens[:6])
    snap = b.save_state()
    assert snap.snap_trace == want[:6 * per].tolist()
    # A traced snapshot continues its trace; serve_steps traces the sessions that trace.
    c = Session(pool)
    pool.restored = tokens[:6]
    c.restore_state(session_codec.decode(session_codec.encode(snap)))
    serve_steps([c, a], [int(tokens[6]), int(tokens[10])])
    for t in tokens[7:16]:
        c.serve_step(int(t))
    assert c.save_state().snap_trace == want.tolist()
    # An untraced snapshot turns tracing off.
    untraced = a.save_state()
    pool.restored = tokens[:11]
    c.restore_state(untraced)
    assert c.snap_trace() is None and c.save_state().snap_trace is None
    # reset keeps tracing on and starts it over at position 0.
    b.reset()
    b.feed(tokens[:4])
    assert [e.root for e in b.snap_trace()] == want[:4 * per].tolist()
    assert b.save_state().snap_trace == want[:4 * per].tolist()


def test_unsnapped_model_records_nothing():
    art = synth.make_artifact(replace(SPEC, raw_transition=True), 47)
    pool = OraclePool(art)
    a = Session(pool)
    a.enable_snap_trace()
    a.feed(synth.uniform_prompts(SPEC.vocab, 1, 5, 49)[0])
    assert a.snap_trace() == [] and a.save_state().snap_trace is None
