"""CPU tests of the CSR drawer index oracle (oracle/fbs_index_oracle.c).

The oracle is held to an independent numpy restatement (tests/index_cases.py), to the
reference's own cases (projects/uor-cuda-inverted-file/tests/inverted_file_test.cpp:140-300:
seeded parity, single-cell collapse, fewer than K cells, refusals, 64 incremental updates
equal to fresh builds, removal and reinsertion, draining, ties, stale and corrupt indexes,
middle-block sensitivity, extreme distances) and, where the reference checkout exists, to the
reference's inverted-file library itself (oracle/_ref/libif_ref.so) on every call.
"""

import numpy as np
import pytest

import oracle
from index_cases import (ABSENT, R, cell_table, np_build, np_probe, query_at, random_table,
                         table_of, zero_query_at, zero_table_of)
from uor_fbs.index import HostIndex

needs_ref = pytest.mark.skipif(not oracle.if_ref_available(),
                               reason="the reference's inverted file is not built here")


def host(t) -> HostIndex:
    return HostIndex(*t)


def built(table, allow_absent=False) -> HostIndex:
    st, idx = oracle.index_build(table, R, allow_absent)
    assert st == 0
    return idx


def probe_all(table, idx, query, k):
    """Oracle probe == oracle full scan == numpy; returns the probe."""
    st, adm, top, pred = oracle.index_probe(table, R, query, k, idx)
    fs = oracle.index_full_scan(table, R, query, k)
    assert st == fs[0]
    np.testing.assert_array_equal(adm, fs[1])
    np.testing.assert_array_equal(top, fs[2])
    assert pred == fs[3]
    if st == 0:
        want_adm, want_top = np_probe(table, query, k, idx.offsets, idx.members)
        np.testing.assert_array_equal(adm, want_adm)
        np.testing.assert_array_equal(top, want_top)
        assert pred == top[0]
    return st, adm, top, pred


@needs_ref
def test_codebook_fixture_is_the_reference_codebook():
    np.testing.assert_array_equal(oracle.ref_codebook(), R)


def test_inputs_match_the_package_generators():
    """The package's codebook and seeded generators (bench.py's inputs) are these inputs."""
    from uor_fbs import index as ix
    np.testing.assert_array_equal(ix.CODEBOOK, R)
    np.testing.assert_array_equal(ix.seeded_table(300), table_of(300))
    for s in range(40):
        np.testing.assert_array_equal(ix.seeded_query(s), query_at(s))


@pytest.mark.parametrize("v", [1, 64, 256, 4096])
def test_build_matches_numpy_and_construction(v):
    t = table_of(v)
    idx = built(t)
    assert idx.same(host(np_build(t)))
    i = np.arange(v)
    np.testing.assert_array_equal(idx.cells, ((i * 7 + 1) % 16) * 16 + (i * 11 + 3) % 16)
    assert oracle.index_validate(t, R, idx) == 0


@pytest.mark.parametrize("width", [16, 32, 64])
def test_build_random_tables_with_absent_tokens(width):
    rng = np.random.default_rng(width)
    t = random_table(rng, 5000, width, absent_frac=0.1)
    assert oracle.index_build(t, R)[0] == 2  # NonRootBlock without allow_absent
    idx = built(t, allow_absent=True)
    assert idx.same(host(np_build(t)))
    assert idx.absent_count == int((np_build(t)[2] == ABSENT).sum()) > 0
    for seed in range(4):
        q = rng.integers(-50, 50, size=width).astype(np.int32)
        q[:8], q[-8:] = R[seed], R[(seed * 3 + 5) % 16]
        assert probe_all(t, idx, q, 8)[0] == 0


def test_cell_is_the_first_matching_root():
    roots = R.copy()
    roots[9] = roots[2]  # a duplicate root: the first one wins
    row = np.zeros(32, np.int32)
    row[:8], row[-8:] = R[2], R[5]
    assert oracle.index_cell(row, roots) == 2 * 16 + 5
    row[-8:] = 1
    assert oracle.index_cell(row, roots) == ABSENT


@pytest.mark.parametrize("v", [1, 64, 256, 4096])
@pytest.mark.parametrize("k", [1, 8, 16])
def test_seeded_parity(v, k):
    t = table_of(v)
    idx = built(t)
    for seed in (7, 0, 3, 12):
        assert probe_all(t, idx, query_at(seed), k)[0] == 0


def test_single_cell_collapse_and_few_cells():
    single = cell_table([0] * 256, [0] * 256)
    idx = built(single)
    np.testing.assert_array_equal(idx.members, np.arange(256))
    assert idx.offsets[0] == 0 and (idx.offsets[1:] == 256).all()
    st, adm, top, pred = probe_all(single, idx, query_at(7), 8)
    assert st == 0 and adm[0] == 0 and (adm[1:] == ABSENT).all()
    np.testing.assert_array_equal(top, np.arange(8))  # equal distances: lowest ids
    few = cell_table([0, 1, 2], [0, 1, 2])
    idx = built(few)
    st, adm, top, pred = probe_all(few, idx, query_at(7), 16)
    assert st == 0
    assert sorted(adm[:3].tolist()) == [0, 17, 34] and (adm[3:] == ABSENT).all()
    assert sorted(top[:3].tolist()) == [0, 1, 2] and (top[3:] == ABSENT).all()


def test_refusals():
    few = cell_table([0, 1, 2], [0, 1, 2])
    idx = built(few)
    assert oracle.index_probe(few, R, query_at(0), 0, idx)[0] == 1
    assert oracle.index_probe(few, R, query_at(0), 17, idx)[0] == 1
    assert oracle.index_full_scan(few, R, query_at(0), 0)[0] == 1
    invalid = few.copy()
    invalid[0, :8] = 0
    assert oracle.index_build(invalid, R)[0] == 2
    assert oracle.index_build(np.zeros((0, 32), np.int32), R)[0] == 1
    assert oracle.index_update(few, R, 3, idx)[0] == 1  # moved out of range
    assert oracle.index_remove(3, 3, idx)[0] == 1


def test_incremental_updates_equal_fresh_builds():
    moving = table_of(256)
    idx = built(moving)
    st, same = oracle.index_update(moving, R, 0, idx)
    assert st == 0 and same.same(idx)  # no-op update preserves the index
    for step in range(64):
        moved = (step * 17) % 256
        moving[moved, :8] = R[(step + 3) % 16]
        moving[moved, -8:] = R[(step * 5 + 1) % 16]
        st, idx = oracle.index_update(moving, R, moved, idx)
        assert st == 0
        assert oracle.index_validate(moving, R, idx) == 0
        assert idx.same(built(moving))
        assert probe_all(moving, idx, query_at(step), 8)[0] == 0


def test_random_moves_against_fresh_builds():
    """Moves between every pair of cell orders, into and out of ABSENT, with absent tokens."""
    rng = np.random.default_rng(5)
    t = random_table(rng, 700, absent_frac=0.05, cells=40)
    idx = built(t, allow_absent=True)
    for step in range(300):
        moved = int(rng.integers(0, len(t)))
        action = rng.random()
        if action < 0.15:
            st, after = oracle.index_remove(len(t), moved, idx)
            t[moved, :8] = 0
            assert st == 0
        else:
            c = int(rng.integers(0, 256))
            t[moved, :8], t[moved, -8:] = R[c // 16], R[c % 16]
            st, after = oracle.index_update(t, R, moved, idx)
            assert st == 0
        idx = after
        assert idx.same(built(t, allow_absent=True)), step


def test_removal_and_reinsertion():
    removal = cell_table([0, 1, 2], [0, 1, 2])
    idx = built(removal)
    removal[0, :8] = 0
    st, after = oracle.index_update(removal, R, 0, idx)
    assert st == 2 and after.same(idx)  # refused without mutation
    st, idx = oracle.index_remove(3, 0, idx)
    assert st == 0 and idx.absent_count == 1 and idx.cells[0] == ABSENT
    assert oracle.index_validate(removal, R, idx) == 0
    removal[0, :8] = R[0]
    st, idx = oracle.index_update(removal, R, 0, idx)
    assert st == 0 and idx.absent_count == 0
    assert idx.same(built(removal))


def test_drained_index():
    drained = cell_table([0, 1, 2], [0, 1, 2])
    idx = built(drained)
    drained[:, :8] = 0
    for tok in range(3):
        st, idx = oracle.index_remove(3, tok, idx)
        assert st == 0
    assert idx.absent_count == 3 and len(idx.members) == 0
    assert oracle.index_probe(drained, R, query_at(0), 1, idx)[0] == 1
    assert oracle.index_full_scan(drained, R, query_at(0), 1)[0] == 1
    assert oracle.index_remove(3, 1, idx)[0] == 0  # removing an absent token is a no-op


def test_ties_stale_and_corrupt():
    ties = cell_table([0, 0], [0, 0])
    idx = built(ties)
    st, adm, top, pred = probe_all(ties, idx, query_at(0), 1)
    assert st == 0 and pred == 0
    stale = idx.copy()
    stale.cells[0] = 7
    assert oracle.index_validate(ties, R, stale) == 3
    corrupt = idx.copy()
    corrupt.offsets[1] = 99
    assert oracle.index_validate(ties, R, corrupt) == 3
    assert oracle.index_probe(ties, R, query_at(0), 1, corrupt)[0] == 3
    assert oracle.index_update(ties, R, 0, corrupt)[0] == 3
    out_of_range = idx.copy()
    out_of_range.cells[0] = 999
    assert oracle.index_update(ties, R, 0, out_of_range)[0] == 3
    assert oracle.index_remove(2, 0, out_of_range)[0] == 3
    descending = idx.copy()
    descending.members[:] = [1, 0]
    assert oracle.index_validate_structure(descending) == 3
    miscount = idx.copy()
    miscount.absent_count = 1
    assert oracle.index_validate_structure(miscount) == 3


def test_middle_blocks_change_rankings():
    top_changes = prediction_changes = 0
    for v in (64, 256):
        varied, zero = table_of(v), zero_table_of(v)
        for k in (1, 8, 16):
            for seed in range(4):
                a = oracle.index_full_scan(varied, R, query_at(seed), k)
                b = oracle.index_full_scan(zero, R, zero_query_at(seed), k)
                assert a[0] == 0 and b[0] == 0
                top_changes += not np.array_equal(a[2], b[2])
                prediction_changes += a[3] != b[3]
    assert top_changes >= 3 and prediction_changes >= 1


def test_extreme_distances_use_64_bits():
    extreme = table_of(2)
    extreme[:, 8:24] = np.iinfo(np.int32).max
    q = query_at(0)
    q[8:24] = np.iinfo(np.int32).min
    idx = built(extreme)
    st, adm, top, pred = probe_all(extreme, idx, q, 1)
    assert st == 0


# ---- the oracle against the reference's own library, call by call

def same_result(a, b):
    assert a[0] == b[0]
    if a[0] == 0:
        for x, y in zip(a[1:], b[1:]):
            np.testing.assert_array_equal(x, y)


@needs_ref
@pytest.mark.parametrize("v", [1, 64, 256, 4096])
def test_oracle_equals_reference_build_and_scans(v):
    t = table_of(v)
    st, idx = oracle.index_build(t, R)
    rst, ridx = oracle.ref_build(t)
    assert st == rst == 0 and idx.same(ridx)
    for k in (1, 8, 16):
        for seed in (0, 7, 11):
            same_result(oracle.index_probe(t, R, query_at(seed), k, idx),
                        oracle.ref_probe(t, query_at(seed), k, ridx))
            same_result(oracle.index_full_scan(t, R, query_at(seed), k),
                        oracle.ref_full_scan(t, query_at(seed), k))


@needs_ref
def test_oracle_equals_reference_on_random_changes():
    rng = np.random.default_rng(11)
    t = random_table(rng, 500, absent_frac=0.05, cells=30)
    st, idx = oracle.index_build(t, R, True)
    rst, ridx = oracle.ref_build(t, True)
    assert st == rst == 0 and idx.same(ridx)
    for step in range(250):
        moved = int(rng.integers(0, len(t)))
        r = rng.random()
        if r < 0.1:
            a, b = oracle.index_remove(len(t), moved, idx), oracle.ref_remove(t, moved, ridx)
        else:
            if r < 0.2:
                t[moved, :8] = 0  # a non-root row: refused
            else:
                c = int(rng.integers(0, 256))
                t[moved, :8], t[moved, -8:] = R[c // 16], R[c % 16]
            a, b = oracle.index_update(t, R, moved, idx), oracle.ref_update(t, moved, ridx)
        assert a[0] == b[0], step
        assert a[1].same(b[1]), step
        idx, ridx = a[1], b[1]
        if step % 25 == 0:
            q = query_at(step)
            same_result(oracle.index_probe(t, R, q, 8, idx), oracle.ref_probe(t, q, 8, ridx))


@needs_ref
def test_oracle_equals_reference_on_refusals():
    ties = cell_table([0, 0], [0, 0])
    _, idx = oracle.ref_build(ties)
    for mutate in ("stale", "offsets", "range", "order"):
        bad = idx.copy()
        if mutate == "stale":
            bad.cells[0] = 7
        elif mutate == "offsets":
            bad.offsets[1] = 99
        elif mutate == "range":
            bad.cells[0] = 999
        else:
            bad.members[:] = [1, 0]
        assert oracle.index_validate(ties, R, bad) == oracle.ref_validate(ties, bad)
        assert oracle.index_update(ties, R, 0, bad)[0] == oracle.ref_update(ties, 0, bad)[0]
        if mutate != "range":  # the reference's remove would index past its offsets there
            assert oracle.index_remove(2, 0, bad)[0] == oracle.ref_remove(ties, 0, bad)[0]
    for k in (0, 17):
        assert oracle.index_probe(ties, R, query_at(0), k, idx)[0] == \
            oracle.ref_probe(ties, query_at(0), k, idx)[0]
