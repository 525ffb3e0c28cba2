"""GPU parity of the CSR drawer index (uor-r4_amd/csrc/fbs_index.hip through uor_fbs.index)
against the oracle (oracle/fbs_index_oracle.c, itself held to the reference's inverted-file
library): builds at every tile boundary and skew, the reference's update, removal, refusal and
corruption cases (projects/uor-cuda-inverted-file/tests/inverted_file_test.cpp:140-300),
random move sequences, long shifts, and batched probes and full scans. Bit-exact: every
offset, member, cell, absent count, admitted cell, top-8 token and status.
"""

import numpy as np
import pytest

import oracle
from index_cases import (ABSENT, R, cell_table, query_at, random_table, table_of,
                         zero_query_at, zero_table_of)
from uor_fbs import index as ix

pytestmark = pytest.mark.gpu


def device(table):
    t = ix.Table(table, R)
    return t, ix.Index(t.count)


def oracle_built(table, allow_absent=False):
    st, idx = oracle.index_build(table, R, allow_absent)
    assert st == 0
    return idx


def check_scan(res: ix.ScanResult, table, queries, k, host_index=None):
    for r, q in enumerate(queries):
        if host_index is None:
            want = oracle.index_full_scan(table, R, q, k)
        else:
            want = oracle.index_probe(table, R, q, k, host_index)
        assert res.status[r] == want[0], r
        np.testing.assert_array_equal(res.admitted[r], want[1], err_msg=f"row {r}")
        np.testing.assert_array_equal(res.top8[r], want[2], err_msg=f"row {r}")
        assert res.prediction[r] == want[3], r


@pytest.mark.parametrize("count,width", [(1, 32), (64, 32), (511, 32), (512, 32), (513, 16),
                                         (4096, 32), (65536, 32), (300001, 64), (5000, 256),
                                         ((1 << 20) + 1, 32), ((1 << 22) + 3, 16)])
def test_build_matches_oracle(count, width):
    rng = np.random.default_rng(count)
    table = table_of(count) if width == 32 and count <= 4096 else random_table(rng, count, width)
    t, idx = device(table)
    assert ix.build(t, idx) == ix.Status.Ok
    assert idx.to_host().same(oracle_built(table))
    assert ix.validate(t, idx) == ix.Status.Ok
    assert ix.validate_structure(idx) == ix.Status.Ok


@pytest.mark.parametrize("cells", [1, 3, 256])
def test_build_with_absent_tokens_and_skew(cells):
    rng = np.random.default_rng(cells)
    table = random_table(rng, 100_000, 32, absent_frac=0.2, cells=cells)
    t, idx = device(table)
    assert ix.build(t, idx) == ix.Status.NonRootBlock
    assert ix.build(t, idx, allow_absent=True) == ix.Status.Ok
    want = oracle_built(table, True)
    assert idx.to_host().same(want)
    assert want.absent_count > 0
    assert ix.validate(t, idx) == ix.Status.Ok


def test_rebuild_reuses_buffers():
    rng = np.random.default_rng(3)
    a, b = random_table(rng, 9000, 32, 0.1), random_table(rng, 9000, 32, 0.0, cells=7)
    t, idx = device(a)
    assert ix.build(t, idx, True) == ix.Status.Ok
    t2 = ix.Table(b, R)
    assert ix.build(t2, idx) == ix.Status.Ok
    assert idx.to_host().same(oracle_built(b))


def test_incremental_updates_equal_oracle_and_fresh_builds():
    moving = table_of(256)
    t, idx = device(moving)
    assert ix.build(t, idx) == ix.Status.Ok
    before = idx.to_host()
    assert ix.update(t, 0, idx) == ix.Status.Ok
    assert idx.to_host().same(before)  # no-op update
    host = before
    for step in range(64):
        moved = (step * 17) % 256
        moving[moved, :8] = R[(step + 3) % 16]
        moving[moved, -8:] = R[(step * 5 + 1) % 16]
        t.set_row(moved, moving[moved])
        assert ix.update(t, moved, idx) == ix.Status.Ok
        st, host = oracle.index_update(moving, R, moved, host)
        assert st == 0
        got = idx.to_host()
        assert got.same(host), step
        assert got.same(oracle_built(moving)), step
        res = ix.probe(t, query_at(step)[None], 8, idx)
        check_scan(res, moving, query_at(step)[None], 8, host)


@pytest.mark.parametrize("count,cells", [(5000, 256), (700, 30)])
def test_random_moves_match_oracle(count, cells):
    rng = np.random.default_rng(count)
    table = random_table(rng, count, 32, absent_frac=0.05, cells=cells)
    t, idx = device(table)
    assert ix.build(t, idx, True) == ix.Status.Ok
    host = oracle_built(table, True)
    for step in range(200):
        moved = int(rng.integers(0, count))
        r = rng.random()
        if r < 0.12:
            got = ix.remove_token(t, moved, idx)
            st, host2 = oracle.index_remove(count, moved, host)
        else:
            if r < 0.2:
                table[moved, :8] = 0  # no cell: refused, nothing changes
            else:
                c = int(rng.integers(0, 256))
                table[moved, :8], table[moved, -8:] = R[c // 16], R[c % 16]
            t.set_row(moved, table[moved])
            got = ix.update(t, moved, idx)
            st, host2 = oracle.index_update(table, R, moved, host)
        assert int(got) == st, step
        host = host2
        assert idx.to_host().same(host), step


def test_long_shifts_between_far_cells():
    """Moves between cell 0 and cell 255 of a 120k-token index shift ~60k members each way."""
    n = 120_000
    first = np.where(np.arange(n) % 2 == 0, 0, 15)
    table = cell_table(first, first)  # cells 0 and 255
    t, idx = device(table)
    assert ix.build(t, idx) == ix.Status.Ok
    host = oracle_built(table)
    for moved, cell in ((0, 255), (n - 1, 0), (n // 2, 255), (7, 0), (n - 2, 17)):
        table[moved, :8], table[moved, -8:] = R[cell // 16], R[cell % 16]
        t.set_row(moved, table[moved])
        assert ix.update(t, moved, idx) == ix.Status.Ok
        st, host = oracle.index_update(table, R, moved, host)
        assert st == 0
        assert idx.to_host().same(host)
    for moved in (1, n - 3):
        assert ix.remove_token(t, moved, idx) == ix.Status.Ok
        st, host = oracle.index_remove(n, moved, host)
        assert st == 0
        assert idx.to_host().same(host)
    table[1, :8] = R[0]
    table[1, -8:] = R[0]
    t.set_row(1, table[1])
    assert ix.update(t, 1, idx) == ix.Status.Ok  # back in from ABSENT
    st, host = oracle.index_update(table, R, 1, host)
    assert idx.to_host().same(host)


def test_removal_reinsertion_and_draining():
    removal = cell_table([0, 1, 2], [0, 1, 2])
    t, idx = device(removal)
    assert ix.build(t, idx) == ix.Status.Ok
    before = idx.to_host()
    removal[0, :8] = 0
    t.set_row(0, removal[0])
    assert ix.update(t, 0, idx) == ix.Status.NonRootBlock
    assert idx.to_host().same(before)  # refused without mutation
    assert ix.remove_token(t, 0, idx) == ix.Status.Ok
    got = idx.to_host()
    assert got.absent_count == 1 and got.cells[0] == ABSENT
    assert ix.validate(t, idx) == ix.Status.Ok
    removal[0, :8] = R[0]
    t.set_row(0, removal[0])
    assert ix.update(t, 0, idx) == ix.Status.Ok
    assert idx.to_host().same(oracle_built(removal))
    drained = removal.copy()
    drained[:, :8] = 0
    for tok in range(3):
        t.set_row(tok, drained[tok])
        assert ix.remove_token(t, tok, idx) == ix.Status.Ok
    got = idx.to_host()
    assert got.absent_count == 3 and len(got.members) == 0
    assert ix.remove_token(t, 1, idx) == ix.Status.Ok  # already absent
    res = ix.probe(t, query_at(0)[None], 1, idx)
    assert res.status[0] == ix.Status.InvalidArgument and res.prediction[0] == ABSENT
    res = ix.full_scan(t, query_at(0)[None], 1)
    assert res.status[0] == ix.Status.InvalidArgument
    assert ix.update(t, 3, idx) == ix.Status.InvalidArgument  # refused by the kernel
    assert ix.remove_token(t, 3, idx) == ix.Status.InvalidArgument


def test_stale_and_corrupt_indexes_are_refused_like_the_oracle():
    ties = cell_table([0, 0], [0, 0])
    t, idx = device(ties)
    assert ix.build(t, idx) == ix.Status.Ok
    good = idx.to_host()
    cases = {}
    stale = good.copy()
    stale.cells[0] = 7
    cases["stale"] = stale
    corrupt = good.copy()
    corrupt.offsets[1] = 99
    cases["offsets"] = corrupt
    far = good.copy()
    far.cells[0] = 999
    cases["range"] = far
    order = good.copy()
    order.members[:] = [1, 0]
    cases["order"] = order
    count = good.copy()
    count.absent_count = 1
    cases["count"] = count
    for name, bad in cases.items():
        idx.load(bad)
        assert int(ix.validate(t, idx)) == oracle.index_validate(ties, R, bad), name
        assert int(ix.validate_structure(idx)) == oracle.index_validate_structure(bad), name
        st = int(ix.update(t, 0, idx))
        assert st == oracle.index_update(ties, R, 0, bad)[0], name
        assert idx.to_host().same(bad), name  # refused: nothing moved
        idx.load(bad)
        assert int(ix.remove_token(t, 0, idx)) == oracle.index_remove(2, 0, bad)[0], name
        # A probe with check=False still stays inside the table: out-of-range ranges are
        # reported, not followed.
        res = ix.probe(t, query_at(0)[None], 1, idx, check=False)
        assert res.status[0] in (ix.Status.Ok, ix.Status.CsrInvariant)
        res = ix.probe(t, query_at(0)[None], 1, idx)  # validates first, as the reference
        assert res.status[0] == ix.Status.CsrInvariant, name
    idx.load(corrupt)
    res = ix.probe(t, query_at(0)[None], 1, idx, check=False)
    assert res.status[0] == ix.Status.CsrInvariant


@pytest.mark.parametrize("v", [1, 64, 256, 4096])
@pytest.mark.parametrize("k", [1, 8, 16])
def test_probe_and_full_scan_seeded(v, k):
    table = table_of(v)
    t, idx = device(table)
    assert ix.build(t, idx) == ix.Status.Ok
    host = oracle_built(table)
    queries = np.stack([query_at(s) for s in range(37)])
    check_scan(ix.probe(t, queries, k, idx), table, queries, k, host)
    check_scan(ix.full_scan(t, queries, k), table, queries, k)


def test_probe_batches_on_random_tables():
    rng = np.random.default_rng(9)
    for count, width, cells in ((20_000, 32, 256), (3000, 64, 12), (50_000, 16, 256)):
        table = random_table(rng, count, width, absent_frac=0.1, cells=cells)
        t, idx = device(table)
        assert ix.build(t, idx, True) == ix.Status.Ok
        host = oracle_built(table, True)
        queries = rng.integers(-(1 << 31), 1 << 31, size=(301, width), dtype=np.int64)
        queries = queries.astype(np.int32)
        pick = rng.integers(0, 16, size=(301, 2))
        queries[:, :8], queries[:, -8:] = R[pick[:, 0]], R[pick[:, 1]]
        for k in (1, 5, 16):
            check_scan(ix.probe(t, queries, k, idx), table, queries, k, host)
        check_scan(ix.full_scan(t, queries[:40], 8), table, queries[:40], 8)


def test_refused_k_and_sizes():
    table = table_of(64)
    t, idx = device(table)
    assert ix.build(t, idx) == ix.Status.Ok
    for k in (0, 17):
        assert (ix.probe(t, query_at(0)[None], k, idx).status == ix.Status.InvalidArgument).all()
        assert (ix.full_scan(t, query_at(0)[None], k).status == ix.Status.InvalidArgument).all()
    other = ix.Index(65)
    assert ix.build(t, other) == ix.Status.InvalidArgument


def test_middle_blocks_and_extreme_distances():
    changes = predictions = 0
    for v in (64, 256):
        varied, zero = device(table_of(v))[0], device(zero_table_of(v))[0]
        qa = np.stack([query_at(s) for s in range(4)])
        qb = np.stack([zero_query_at(s) for s in range(4)])
        for k in (1, 8, 16):
            a, b = ix.full_scan(varied, qa, k), ix.full_scan(zero, qb, k)
            check_scan(a, table_of(v), qa, k)
            changes += int((a.top8 != b.top8).any(axis=1).sum())
            predictions += int((a.prediction != b.prediction).sum())
    assert changes >= 3 and predictions >= 1
    extreme = table_of(2)
    extreme[:, 8:24] = np.iinfo(np.int32).max
    q = query_at(0)
    q[8:24] = np.iinfo(np.int32).min
    t, idx = device(extreme)
    assert ix.build(t, idx) == ix.Status.Ok
    check_scan(ix.probe(t, q[None], 1, idx), extreme, q[None], 1, oracle_built(extreme))
