"""The Hamming trace and the decision trace with the forced replay in the oracle, held to what the
reference's own tests hold them to (the_hamming_trace_records_each_reads_choices_and_changes_no_step,
stack/tests.rs:7586-7640; a replay that forces nothing is the served read, :4900-4935) and to
what the traces mean, by brute force over the records themselves: every head's kept set is the
`nearest` of its query over the keys the earlier rows recorded (ascending distance, then
position; hamming.rs:690-701), a copy head's query and key are its vocabulary codes, a type
head's key its code of the token before, every rate entry the score's bucket
min(score >> 12, 15) (session.rs:4998-5006) unless forced, and a forced code or bucket is used
exactly where it is named (BucketTrace::decide :2192-2215, HeadForce :1397-1421).
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import synth
from uor_fbs.trace import (DecisionForceWindow, ForcedBucket, ForcedCode, TraceError,
                           TraceLayout)

H = synth.HammingSpec
SPEC = synth.Spec(vocab=96, width=64, mlp=64, layers=3, context=40, kept=4, head=1)


def art_of(hamming, spec=SPEC, seed=5):
    return synth.make_artifact(replace(spec, hamming=hamming), seed)


def rows(art, n=2, length=30, seed=9):
    return (synth.uniform_prompts(art.spec.vocab, n, length, seed) % 12).astype(np.uint32)


def parsed(art, raw, decisions):
    lay = TraceLayout.of(art, decisions)
    return lay, [[lay.step(r.tobytes()) if decisions else lay.reads(r.tobytes()) for r in row]
                 for row in raw]


def reads_of(step, decisions):
    if not decisions:
        return step
    return [l.read for l in step.layers if l.read is not None] + ([step.readout] if step.readout else [])


def brute_nearest(query, keys, t, kept):
    cand = sorted((bin(int(query) ^ int(keys[s])).count("1"), s) for s in range(1, t))
    return [s for _, s in cand[:kept]]


@pytest.mark.parametrize("decisions", [False, True])
def test_the_trace_records_each_reads_choices_and_changes_no_step(decisions):
    art = art_of(H(heads=4, depths=(1, 3), kept=4))
    toks = rows(art)
    st, t0, _, q0 = oracle.sequences(art, toks)
    st2, t1, q1, raw = oracle.decision_sequences(art, toks, decisions)
    assert st == st2 == 0
    np.testing.assert_array_equal(t1, t0)
    np.testing.assert_array_equal(q1, q0)
    lay, steps = parsed(art, raw, decisions)
    h, copy, kept = art.hamming.heads, art.hamming.heads // 2, art.hamming.kept
    full = 0
    for ri, read in enumerate(art.hamming_reads):
        codes = oracle.hamming_codes(art, ri)
        for i in range(len(toks)):
            recs = [reads_of(steps[i][t], decisions)[ri] for t in range(toks.shape[1])]
            assert all(r.depth == read.depth for r in recs)
            for head in range(h):
                keys = [recs[t].heads[head].key for t in range(len(recs))]
                for t, r in enumerate(recs):
                    hd = r.heads[head]
                    want = min(kept, max(t - 1, 0))
                    assert len(hd.kept) == want, (ri, head, t)
                    assert hd.kept == brute_nearest(hd.query, keys, t, kept), (ri, head, t)
                    assert hd.key == (0 if t == 0 else int(codes[toks[i, t - 1], head]))
                    if head < copy:
                        assert hd.query == int(codes[toks[i, t], head])
                    full += want == kept
    assert full > 0


def test_copy_key_2_rules_and_asks_record_what_they_serve():
    # Pair keys join the token two back; the latest-exact rule keeps its one exact match; an
    # asking read's type heads ask from the question table. Each kept set is the rule's own
    # choice over the recorded keys.
    art = art_of(H(heads=4, depths=(1, 3), kept=4, copy_keys=(1, 2), copy_latest=True,
                   asks=(False, True)))
    toks = rows(art, 2, 32, 3)
    st, _, _, raw = oracle.decision_sequences(art, toks, False)
    assert st == 0
    _, steps = parsed(art, raw, False)
    copy = art.hamming.heads // 2
    for i in range(len(toks)):
        for ri in range(2):
            recs = [steps[i][t][ri] for t in range(toks.shape[1])]
            for head in range(copy):
                keys = [r.heads[head].key for r in recs]
                for t, r in enumerate(recs):
                    hd = r.heads[head]
                    exact = [s for s in range(1, t) if keys[s] == hd.query]
                    assert hd.kept == ([max(exact)] if exact else []), (ri, head, t)


def test_a_replay_that_forces_nothing_is_the_served_read_and_forced_codes_are_used():
    art = art_of(H(heads=4, depths=(1, 3), kept=4))
    toks = rows(art, 1, 24, 4)
    st, t0, q0, raw0 = oracle.decision_sequences(art, toks, True)
    st1, t1, q1, raw1 = oracle.decision_sequences(art, toks, True, DecisionForceWindow())
    assert st == st1 == 0
    np.testing.assert_array_equal(raw1, raw0)
    np.testing.assert_array_equal(q1, q0)
    lay, steps = parsed(art, raw0, True)
    # Forcing every recorded code and bucket to what it was changes nothing.
    same = DecisionForceWindow()
    for t, step in enumerate(steps[0]):
        for l, layer in enumerate(step.layers):
            for lane, e in enumerate(layer.entry):
                same.buckets.append(ForcedBucket(t, l, lane, e))
        for r in reads_of(step, True):
            for hh, hd in enumerate(r.heads):
                same.codes.append(ForcedCode(t, r.depth, hh, "query", hd.query))
                if t:
                    same.codes.append(ForcedCode(t, r.depth, hh, "key", hd.key))
    st2, t2, q2, raw2 = oracle.decision_sequences(art, toks, True, same)
    assert st2 == 0
    np.testing.assert_array_equal(raw2, raw0)
    np.testing.assert_array_equal(q2, q0)
    # A forced query at one row replaces that row's query only; a forced key at step s is every
    # later row's candidate key there.
    t, s = 20, 7
    forced = DecisionForceWindow(codes=[ForcedCode(t, 1, 0, "query", 0x5A5A),
                                        ForcedCode(s, 1, 0, "key", 0x5A5A)])
    st3, _, _, raw3 = oracle.decision_sequences(art, toks, True, forced)
    assert st3 == 0
    _, steps3 = parsed(art, raw3, True)
    recs = [reads_of(x, True)[0] for x in steps3[0]]
    keys = [r.heads[0].key for r in recs]
    assert recs[t].heads[0].query == 0x5A5A and keys[s] == 0x5A5A
    assert recs[t].heads[0].kept == brute_nearest(0x5A5A, keys, t, art.hamming.kept)
    assert s in recs[t].heads[0].kept  # the forced key equals the forced query: distance 0
    for u in range(s + 1, len(recs)):
        assert recs[u].heads[0].kept == brute_nearest(recs[u].heads[0].query, keys, u, art.hamming.kept)


def test_the_rate_buckets_are_the_scores_unless_forced():
    art = art_of(H(heads=4, depths=(1, 3), kept=4))
    toks = rows(art, 2, 20, 6)
    st, _, q0, raw = oracle.decision_sequences(art, toks, True)
    assert st == 0
    _, steps = parsed(art, raw, True)
    for row in steps:
        for step in row:
            assert len(step.layers) == art.spec.layers
            for layer in step.layers:
                sc = np.asarray(layer.score_q16)
                assert ((sc >= 0) & (sc <= 65536)).all()
                np.testing.assert_array_equal(layer.entry, np.minimum(sc >> 12, 15))
    # A forced entry is the one used, and moves what follows.
    e = steps[0][3].layers[1].entry[2]
    force = DecisionForceWindow(buckets=[ForcedBucket(3, 1, 2, (e + 7) % 16)])
    st2, _, q2, raw2 = oracle.decision_sequences(art, toks, True, [force, None])
    assert st2 == 0
    _, steps2 = parsed(art, raw2, True)
    assert steps2[0][3].layers[1].entry[2] == (e + 7) % 16
    assert steps2[0][3].layers[1].score_q16 == steps[0][3].layers[1].score_q16
    np.testing.assert_array_equal(q2[1], q0[1])  # the other row forced nothing
    np.testing.assert_array_equal(q2[0, :3], q0[0, :3])
    assert not np.array_equal(q2[0, 3:], q0[0, 3:])


def test_the_nearest_and_the_forced_set_refusals():
    from uor_fbs.trace import nearest
    table = np.array([[0, 0], [3, 1], [1, 3], [10, 10]], np.int16)
    n = nearest([2, 2], table)
    assert (n.pick, n.score_q12, n.runner_up, n.runner_score_q12) == (1, -2, 2, -2)
    art = art_of(H(heads=4, depths=(1, 3), kept=4))
    lay = TraceLayout.of(art, True)
    bad = [[ForcedBucket(40, 0, 0, 1)], [ForcedBucket(0, 3, 0, 1)], [ForcedBucket(0, 0, 16, 1)],
           [ForcedBucket(0, 0, 0, 16)], [ForcedBucket(0, 0, 0, 1), ForcedBucket(0, 0, 0, 2)]]
    for b in bad:
        with pytest.raises(TraceError):
            lay.force_arrays([DecisionForceWindow(buckets=b)], 1, 40)
    for c in ([ForcedCode(1, 2, 0, "query", 1)], [ForcedCode(1, 1, 4, "query", 1)],
              [ForcedCode(0, 1, 0, "key", 1)], [ForcedCode(40, 1, 0, "query", 1)],
              [ForcedCode(1, 1, 0, "key", 1), ForcedCode(1, 1, 0, "key", 2)]):
        with pytest.raises(TraceError):
            lay.force_arrays([DecisionForceWindow(codes=c)], 1, 40)
    with pytest.raises(TraceError):
        TraceLayout.of(art, False).force_arrays([DecisionForceWindow(buckets=[ForcedBucket(0, 0, 0, 1)])], 1, 40)
