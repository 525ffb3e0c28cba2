"""Inputs and independent numpy checks for the CSR drawer index tests.

The seeded tables and queries follow the reference's own test inputs
(projects/uor-cuda-inverted-file/tests/inverted_file_test.cpp:39-75: token_at, table_of,
zero_table_of, query_at, zero_query_at), so the same cases run here; the roots are the
committed codebook fixture. The np_* functions restate cells, build and probe with numpy
(broadcast matches, a stable argsort, lexsorted ranking) as a check on the C oracle that does
not share its loops.
"""

from __future__ import annotations

import os

import numpy as np

ABSENT = 0xFFFFFFFF
HERE = os.path.dirname(os.path.abspath(__file__))


def roots() -> np.ndarray:
    rows = [line.split() for line in open(os.path.join(HERE, "golden", "index", "codebook.txt"))
            if line.strip() and not line.startswith("#")]
    r = np.array(rows, dtype=np.int32)
    assert r.shape == (16, 8)
    return r


R = roots()


def token_at(i: int) -> np.ndarray:
    t = np.zeros((4, 8), np.int32)
    t[0] = R[(i * 7 + 1) % 16]
    t[3] = R[(i * 11 + 3) % 16]
    d = np.arange(8)
    t[1] = (i * 29 + d * 7) % 37 - 18
    t[2] = (i * 13 + d * 5) % 41 - 20
    return t.reshape(32)


def table_of(count: int) -> np.ndarray:
    return np.stack([token_at(i) for i in range(count)]) if count else np.zeros((0, 32), np.int32)


def zero_table_of(count: int) -> np.ndarray:
    t = np.zeros((count, 4, 8), np.int32)
    i = np.arange(count)
    t[:, 0] = R[(i * 7 + 1) % 16]
    t[:, 3] = R[(i * 11 + 3) % 16]
    return t.reshape(count, 32)


def query_at(seed: int) -> np.ndarray:
    q = np.zeros((4, 8), np.int32)
    q[0] = R[seed % 16]
    q[3] = R[(seed * 5 + 1) % 16]
    d = np.arange(8)
    q[1] = (seed * 11 + d * 3) % 23 - 11
    q[2] = (seed * 17 + d * 2) % 19 - 9
    return q.reshape(32)


def zero_query_at(seed: int) -> np.ndarray:
    q = np.zeros((4, 8), np.int32)
    q[0] = R[seed % 16]
    q[3] = R[(seed * 5 + 1) % 16]
    return q.reshape(32)


def cell_table(cells_first, cells_last, width=32, fill=0) -> np.ndarray:
    """Rows whose first/last blocks are the given roots (ABSENT-able: -1 = a zero block)."""
    n = len(cells_first)
    t = np.full((n, width), fill, np.int32)
    for i, (a, b) in enumerate(zip(cells_first, cells_last)):
        t[i, :8] = R[a] if a >= 0 else 0
        t[i, width - 8:] = R[b] if b >= 0 else 0
    return t


def random_table(rng, count, width=32, absent_frac=0.0, cells=256) -> np.ndarray:
    """Random middle values; endpoints from the roots (a zero block for an absent token).
    `cells` < 256 draws from the first `cells` cells only (skewed occupancy)."""
    t = rng.integers(-(1 << 31), 1 << 31, size=(count, width), dtype=np.int64).astype(np.int32)
    c = rng.integers(0, cells, size=count)
    t[:, :8] = R[c // 16]
    t[:, width - 8:] = R[c % 16]
    gone = rng.random(count) < absent_frac
    t[gone, :8] = 0
    return t


# ---- independent numpy restatement

def np_root_ids(blocks: np.ndarray) -> np.ndarray:
    eq = (blocks[:, None, :] == R[None, :, :]).all(axis=2)
    return np.where(eq.any(axis=1), eq.argmax(axis=1), -1)


def np_cells(table: np.ndarray) -> np.ndarray:
    a, b = np_root_ids(table[:, :8]), np_root_ids(table[:, -8:])
    return np.where((a >= 0) & (b >= 0), a * 16 + b, ABSENT).astype(np.uint32)


def np_build(table: np.ndarray):
    """(offsets, members, cells, absent_count)."""
    cells = np_cells(table)
    present = np.nonzero(cells != ABSENT)[0]
    members = present[np.argsort(cells[present], kind="stable")].astype(np.uint32)
    counts = np.bincount(cells[present].astype(np.int64), minlength=256)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    return offsets, members, cells, int(len(cells) - len(present))


def np_probe(table, query, k, offsets, members):
    """(admitted [16], top8 [8]) of the reference's probe on a valid index."""
    q = query.astype(np.int64)
    da = np.abs(q[None, :8] - R.astype(np.int64)).sum(1)
    db = np.abs(q[None, -8:] - R.astype(np.int64)).sum(1)
    c = np.arange(256)
    cd = da[c // 16] + db[c % 16]
    occupied = np.nonzero(np.diff(offsets.astype(np.int64)) > 0)[0]
    order = occupied[np.lexsort((occupied, cd[occupied]))][:k]
    admitted = np.full(16, ABSENT, np.uint32)
    admitted[:len(order)] = order
    cand = np.concatenate([members[offsets[x]:offsets[x + 1]] for x in order]) if len(order) else \
        np.zeros(0, np.uint32)
    top8 = np.full(8, ABSENT, np.uint32)
    if len(cand):
        l1 = np.abs(table[cand].astype(np.int64) - q[None, :]).sum(1)
        best = cand[np.lexsort((cand, l1))][:8]
        top8[:len(best)] = best
    return admitted, top8
