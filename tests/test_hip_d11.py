"""The HIP discrete M1 row scorer (uor_d11_score_rows) against the oracle, record for record
and bit for bit: the reference's witness models with their literal expectations
(discrete_d11.rs:2088-2458), random models of every read mode, sweep count and trunk choice,
the row statuses, and panels of the M1 shape (vocabulary 4,096, 4 blocks, context 192, relation
read keeping 8 with the 19-table trunk) larger than one launch's resident waves."""

import numpy as np
import pytest

import d11_cases as W
import oracle
from uor_fbs import d11

pytestmark = pytest.mark.gpu


def gpu_rows(art, pre, lens, tg):
    model = d11.IntegerDiscreteModel(art)
    try:
        return model.score_rows(pre, lens, tg)
    finally:
        model.close()


def assert_same(got, want):
    gw = got.view(np.uint32).reshape(len(got), -1)
    ww = want.view(np.uint32).reshape(len(want), -1)
    bad = np.nonzero((gw != ww).any(1))[0]
    if len(bad):
        i = bad[0]
        fields = [f for f in d11.ROW_DTYPE.names if not np.array_equal(got[i][f], want[i][f])]
        raise AssertionError(f"{len(bad)} rows differ; first row {i}: {fields} "
                             f"got {[got[i][f] for f in fields]} want {[want[i][f] for f in fields]}")


def test_witnesses_on_the_gpu():
    print("d11 witnesses", flush=True)
    art, _ = W.model(W.SHAPE_2, *W.WRITER_2)
    out = gpu_rows(art, *W.rows_of(list(W.WRITER_2_EXPECT)))
    for rec, (pred, admitted, top8, trivals, arivals, loss) in zip(out, W.WRITER_2_EXPECT.values()):
        assert rec["status"] == 0 and rec["prediction"] == pred
        assert rec["admitted"][:rec["admitted_count"]].tolist() == admitted
        assert rec["top8"][:rec["top8_count"]].tolist() == top8
        assert (rec["token_rivals"], rec["address_rivals"], rec["selected_loss"]) == (trivals, arivals, loss)
    art, _ = W.model(W.SHAPE_3, *W.TRANSPORT_3)
    out = gpu_rows(art, *W.rows_of([(p, 0) for p in W.TRANSPORT_3_EXPECT]))
    for rec, want in zip(out, W.TRANSPORT_3_EXPECT.values()):
        assert rec["read_vector"][:16].tolist() == want
    for shape, gates, read, loss in ((W.FLOCK_SHAPE, W.FLOCK_GATES, W.COPY_BASE_READ, 640),
                                     (W.REL_SHAPE, W.REL_BASE_GATES, W.COPY_BASE_READ, 640),
                                     (W.REL_SHAPE, W.REL_ACTIVE_GATES, W.COPY_ACTIVE_READ, 448)):
        art, _ = W.model(shape, W.COPY_TOKENS, [0, 0, 0, 0], gates)
        rec = gpu_rows(art, *W.rows_of([(W.COPY_PREFIX, 2)]))[0]
        assert rec["read_vector"][:16].tolist() == read and rec["selected_loss"] == loss
    art, _ = W.model(W.TRUNK_SHAPE, W.TRUNK_TOKENS, [0] * 8, [0] * 8, W.trunk_witness())
    out = gpu_rows(art, *W.rows_of([(p, 0) for p in W.TRUNK_EXPECT]))
    for rec, (read, pred) in zip(out, W.TRUNK_EXPECT.values()):
        assert rec["read_vector"][:32].tolist() == read and rec["prediction"] == pred


CASES = [
    # mode, blocks, vocab, context, kept_cells, kept, sweeps, trunk, seed
    ("route", 2, 300, 30, 4, 0, 0, False, 11),
    ("route", 4, 4096, 192, 8, 0, 0, True, 12),
    ("flock", 3, 700, 81, 6, 3, 0, False, 13),
    ("flock", 4, 4096, 192, 8, 8, 0, True, 14),
    ("relation", 2, 200, 27, 3, 1, 1, False, 15),
    ("relation", 5, 1000, 100, 16, 5, 3, False, 16),
    ("relation", 4, 4096, 192, 8, 8, 1, True, 17),
    ("relation", 4, 8192, 243, 16, 8, 5, True, 18),
    ("relation", 16, 2000, 60, 12, 2, 2, False, 19),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-b{c[1]}-v{c[2]}-ctx{c[3]}-s{c[6]}-t{int(c[7])}" for c in CASES])
def test_random_models_match_the_oracle(case):
    mode, blocks, V, ctx, kc, kept, sweeps, trunk, seed = case
    art = d11.synthetic(vocabulary=V, blocks=blocks, context=ctx, kept_cells=kc, read_mode=mode,
                        read_kept=kept, read_sweeps=sweeps, seed=seed, trunk=trunk,
                        trunk_entries=20000)
    pre, lens, tg = d11.panel_rows(art, 300, seed + 100)
    lens[:3] = [1, 2, ctx]
    print(f"d11 {case}", flush=True)
    got = gpu_rows(art, pre, lens, tg)
    want = oracle.d11_score_rows(art, pre, lens, tg, threads=8)
    assert (want["status"] == 0).all()
    assert_same(got, want)


def test_row_statuses_match_the_oracle():
    art = d11.synthetic(vocabulary=500, context=40, seed=21, trunk_entries=1000)
    pre, lens, tg = d11.panel_rows(art, 12, 22)
    lens[0], lens[1] = 0, 41            # length outside 1..=context
    pre[2, 5] = 500                     # a token outside the vocabulary
    lens[2] = max(lens[2], 6)
    tg[3] = 777                         # a target outside the vocabulary
    print("d11 statuses", flush=True)
    pre = np.pad(pre, ((0, 0), (0, 1)))
    got = gpu_rows(art, pre, lens, tg)
    want = oracle.d11_score_rows(art, pre, lens, tg, threads=2)
    assert got["status"][:4].tolist() == [1, 1, 2, 8]
    assert_same(got, want)


def test_m1_panel_beyond_one_launch_of_resident_waves():
    # 20,000 rows of the M1 shape: more rows than the chip holds waves at once, so waves start
    # as others finish; rows on both sides of every block boundary are checked.
    art = d11.synthetic(seed=31, trunk_entries=200_000)
    pre, lens, tg = d11.panel_rows(art, 20000, 32, min_len=150)
    print("d11 M1 panel 20000 rows", flush=True)
    got = gpu_rows(art, pre, lens, tg)
    pick = np.unique(np.concatenate([np.arange(0, 20000, 997), np.arange(4090, 4100),
                                     np.arange(19990, 20000)]))
    want = oracle.d11_score_rows(art, pre[pick], lens[pick], tg[pick], threads=8)
    assert_same(got[pick], want)
    assert (got["status"] == 0).all()
    assert len(np.unique(got["prediction"])) > 100


TRACE_CASES = [c for c in CASES if c[3] <= 192] + [("relation", 4, 8192, 243, 16, 8, 5, True, 18)]


@pytest.mark.parametrize("knockout", [False, True], ids=["model", "knockout"])
@pytest.mark.parametrize("case", TRACE_CASES, ids=[f"{c[0]}-b{c[1]}-ctx{c[3]}-s{c[6]}-t{int(c[7])}" for c in TRACE_CASES])
def test_traced_rows_match_the_oracle(case, knockout):
    """uor_d11_score_rows_traced (evaluate_prefix_traced, discrete_d11.rs:1768) and the
    state-transport knockout (:1283-1304) against the oracle: records, trace words and relation
    words, word for word."""
    mode, blocks, V, ctx, kc, kept, sweeps, trunk, seed = case
    art = d11.synthetic(vocabulary=V, blocks=blocks, context=ctx, kept_cells=kc, read_mode=mode,
                        read_kept=kept, read_sweeps=sweeps, seed=seed, trunk=trunk,
                        trunk_entries=20000)
    pre, lens, tg = d11.panel_rows(art, 200, seed + 200)
    lens[:3] = [1, 2, ctx]
    print(f"d11 traced {case} knockout={knockout}", flush=True)
    model = d11.IntegerDiscreteModel(art, knockout=knockout)
    try:
        got, tr, rel = model.score_rows_traced(pre, lens, tg)
        plain = model.score_rows(pre, lens, tg)
    finally:
        model.close()
    want, wtr, wrel = oracle.d11_score_rows_traced(art, pre, lens, tg, knockout=knockout, threads=8)
    assert (want["status"] == 0).all()
    assert_same(got, want)
    assert_same(plain, want)
    np.testing.assert_array_equal(tr, wtr)
    assert (rel is None) == (wrel is None)
    if rel is not None:
        np.testing.assert_array_equal(rel, wrel)


def test_traced_evaluation_api():
    """evaluate_prefix_traced, a relation read's relation_scores from evaluate_prefix, and
    with_state_transport_knockout through the Python face, against the oracle."""
    art = d11.synthetic(vocabulary=1500, context=100, read_mode="relation", read_kept=8,
                        read_sweeps=2, seed=41, trunk_entries=5000)
    prefix = d11.panel_rows(art, 1, 42, min_len=60)[0][0][:77]
    print("d11 traced api", flush=True)
    model = d11.IntegerDiscreteModel(art)
    ko = model.with_state_transport_knockout()
    try:
        assert ko.is_state_transport_knocked_out() and not model.is_state_transport_knocked_out()
        t = model.evaluate_prefix_traced(prefix)
        _, wtr, wrel = oracle.d11_score_rows_traced(art, prefix[None], [77], [0])
        assert t.trace_words == wtr[0].tolist()
        assert t.relation_trace_words == wrel[0].reshape(-1).tolist()
        _, rel = oracle.d11_row_relation(art, prefix, 0)
        assert t.evaluation.relation_scores == rel.reshape(-1).tolist()
        assert model.evaluate_prefix(prefix).relation_scores == rel.reshape(-1).tolist()
        k = ko.evaluate_prefix(prefix)
        want, _, _ = oracle.d11_score_rows_traced(art, prefix[None], [77], [0], knockout=True)
        assert k.read_vector == want[0]["read_vector"][:32].tolist()
        assert k.read_vector == art.table.reshape(1500, 4, 8)[prefix[-1]].reshape(-1).tolist()
    finally:
        ko.close()
        model.close()
