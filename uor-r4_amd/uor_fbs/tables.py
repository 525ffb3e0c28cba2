"""Fixed integer tables of the SpiralCore/FBS step.

The route states, orbit roots and icosians are data of the reference model format; they are
kept here as data (not code) and checked by closed-form tests:

- ``AXES``: the 64-state Cl(0,6) signed-axis table, state ``a`` in ``AXES[8a:8a+8]``,
  ``code & 7`` the source lane and ``code & 8`` a negation
  (crates/uor-r4-integer/src/discrete_d11.rs:35-55, read by ``cl06_axes`` :899-904).
- ``ROOTS``: the 16 orbit roots of the Cl(0,6) anchor ``[2, 2, 0, ...]``
  (discrete_d11.rs:227-244); the writer scores them at Q12 (``<< 12``,
  stack/session.rs:728-730).
- ``icosian_coefficients()``: the 120 unit icosians as ``(a, b)`` pairs meaning
  ``(a + b phi) / 2`` per coordinate, in the order built by
  ``historical_root_coefficients`` (crates/uor-r4-integer/src/h4_classifier.rs:20-76):
  8 axis roots, 16 half roots, then 12 even permutations x 8 sign choices.
- ``BFS``: for orbit roots ``s`` and ``d``, the route state ``BFS[16 s + d]`` that carries root
  ``s`` to root ``d`` (discrete_d11.rs:246-258, read by ``cl06_bfs`` :916-918); of the several
  states that do, the table's own choice, so it is data.
- ``BRANCH``: the three successor roots of each root on the discrete route's later stages
  (discrete_d11.rs:259-276).
- ``compose_table()``: the 64 x 64 product of route states, ``compose(a, b)`` the state acting
  as ``a`` after ``b`` (the relation the reference's ``COMPOSE`` table holds,
  discrete_d11.rs:57-226), derived here from ``AXES``.
- ``keep_q31()``: ``isqrt(2^62 - 2^(60 - 2 i))``, the geometric drive weights
  (stack/session.rs:87-108).
"""

from __future__ import annotations

import math

import numpy as np

AXES = np.array([
    0, 1, 2, 3, 4, 5, 6, 7, 12, 10, 1, 14, 0, 7, 3, 13, 15, 11, 6, 1, 5, 12, 10, 0, 2, 12, 8, 13, 1, 3, 15, 6,
    14, 13, 15, 4, 11, 1, 0, 2, 5, 14, 11, 2, 7, 8, 1, 12, 13, 14, 11, 2, 15, 0, 1, 4, 9, 0, 12, 7, 2, 6, 13, 11,
    3, 7, 13, 8, 14, 2, 4, 9, 15, 3, 14, 9, 5, 12, 2, 0, 14, 5, 15, 12, 3, 9, 0, 2, 10, 12, 0, 13, 1, 3, 7, 14,
    4, 10, 1, 14, 8, 15, 3, 5, 15, 3, 6, 9, 13, 4, 10, 0, 11, 15, 13, 0, 14, 2, 4, 1, 9, 0, 4, 7, 10, 14, 5, 11,
    8, 9, 10, 11, 12, 13, 14, 15, 7, 3, 14, 9, 13, 4, 2, 8, 10, 4, 0, 5, 9, 11, 7, 14, 6, 5, 7, 12, 3, 9, 8, 10,
    13, 6, 3, 10, 15, 0, 9, 4, 11, 7, 5, 8, 14, 2, 12, 1, 9, 8, 12, 15, 10, 14, 13, 11, 0, 9, 10, 11, 4, 5, 14, 7,
    5, 14, 3, 2, 15, 0, 9, 12, 6, 5, 15, 12, 11, 1, 0, 10, 2, 12, 0, 13, 9, 11, 7, 6, 5, 6, 3, 10, 7, 8, 9, 12,
    3, 15, 13, 0, 6, 10, 4, 9, 1, 0, 4, 7, 2, 6, 5, 3, 8, 1, 2, 3, 12, 13, 6, 15, 8, 1, 10, 3, 4, 5, 14, 15,
    9, 8, 4, 15, 2, 6, 5, 11, 3, 15, 5, 0, 14, 2, 12, 9, 1, 8, 4, 15, 10, 14, 5, 3, 6, 13, 7, 4, 11, 1, 8, 10,
    13, 6, 11, 10, 7, 8, 1, 4, 14, 13, 7, 4, 3, 9, 8, 2, 0, 9, 2, 11, 12, 13, 6, 7, 1, 0, 12, 7, 10, 14, 13, 3,
    4, 2, 1, 6, 0, 7, 3, 5, 11, 15, 5, 0, 6, 10, 12, 1, 2, 4, 8, 5, 9, 11, 15, 6, 7, 11, 14, 1, 5, 12, 2, 8,
    10, 4, 8, 5, 1, 3, 15, 14, 11, 7, 13, 8, 6, 10, 4, 1, 12, 10, 9, 14, 8, 15, 11, 13, 7, 11, 6, 1, 13, 4, 10, 8,
    12, 2, 9, 6, 0, 7, 11, 13, 3, 7, 5, 8, 6, 10, 12, 9, 1, 8, 12, 15, 2, 6, 13, 3, 4, 2, 9, 6, 8, 15, 11, 5,
    12, 2, 1, 6, 8, 15, 3, 13, 10, 12, 8, 13, 9, 11, 15, 14, 6, 13, 15, 4, 3, 9, 0, 10, 4, 10, 9, 14, 0, 7, 11, 5,
    2, 4, 0, 5, 1, 3, 7, 6, 8, 9, 2, 11, 4, 5, 6, 15, 14, 5, 7, 12, 11, 1, 8, 2, 0, 1, 10, 3, 12, 13, 14, 7,
    13, 14, 3, 2, 7, 8, 9, 4, 5, 6, 11, 10, 15, 0, 1, 12, 15, 11, 14, 1, 13, 4, 2, 0, 7, 3, 6, 9, 5, 12, 10, 8,
], dtype=np.uint8)

ROOTS = np.array([
    (2, 2, 0, 0, 0, 0, 0, 0),
    (-2, -2, 0, 0, 0, 0, 0, 0),
    (-2, 2, 0, 0, 0, 0, 0, 0),
    (0, 0, -2, 0, -2, 0, 0, 0),
    (0, 0, -2, 0, 2, 0, 0, 0),
    (0, 0, 0, -2, 0, 0, 0, -2),
    (0, 0, 0, -2, 0, 0, 0, 2),
    (0, 0, 0, 0, 0, -2, -2, 0),
    (0, 0, 0, 0, 0, -2, 2, 0),
    (0, 0, 0, 0, 0, 2, -2, 0),
    (0, 0, 0, 0, 0, 2, 2, 0),
    (0, 0, 0, 2, 0, 0, 0, -2),
    (0, 0, 0, 2, 0, 0, 0, 2),
    (0, 0, 2, 0, -2, 0, 0, 0),
    (0, 0, 2, 0, 2, 0, 0, 0),
    (2, -2, 0, 0, 0, 0, 0, 0),
], dtype=np.int32)

BFS = np.array([
    0, 16, 7, 42, 3, 8, 9, 27, 5, 24, 4, 47, 2, 12, 1, 34, 16, 0, 34, 1, 12, 2, 47, 4, 24, 5, 27, 9, 8, 3, 42, 7,
    34, 7, 0, 26, 11, 9, 14, 10, 6, 4, 5, 2, 47, 1, 3, 16, 1, 42, 3, 0, 15, 4, 5, 8, 13, 9, 2, 10, 27, 7, 16, 48,
    12, 3, 1, 7, 0, 5, 6, 9, 2, 41, 13, 4, 35, 16, 15, 11, 2, 8, 47, 27, 24, 0, 7, 1, 3, 12, 42, 34, 16, 5, 4, 9,
    47, 9, 2, 10, 4, 34, 0, 3, 11, 1, 26, 16, 7, 6, 5, 14, 4, 27, 5, 2, 13, 42, 48, 0, 7, 15, 16, 3, 1, 9, 8, 10,
    35, 5, 4, 9, 41, 12, 1, 15, 0, 16, 7, 11, 3, 2, 13, 6, 5, 35, 6, 13, 2, 3, 11, 7, 16, 0, 15, 1, 12, 41, 9, 4,
    27, 4, 10, 8, 9, 1, 3, 16, 15, 7, 0, 48, 42, 13, 2, 5, 9, 47, 14, 5, 6, 7, 16, 26, 1, 11, 3, 0, 34, 4, 10, 2,
    8, 2, 9, 4, 5, 16, 34, 42, 12, 3, 1, 7, 0, 24, 27, 47, 3, 12, 11, 15, 16, 35, 4, 13, 41, 2, 9, 6, 5, 0, 7, 1,
    42, 1, 48, 16, 7, 27, 10, 2, 9, 13, 8, 5, 4, 15, 0, 3, 7, 34, 16, 3, 1, 47, 2, 5, 4, 6, 10, 14, 9, 11, 26, 0,
], dtype=np.uint8)

BRANCH = np.array([
    0, 14, 3, 1, 3, 14, 2, 13, 4, 3, 0, 1, 4, 2, 15, 5, 7, 10, 6, 9, 8, 7, 12, 5,
    8, 6, 11, 9, 11, 6, 10, 5, 12, 11, 8, 9, 12, 10, 7, 13, 15, 2, 14, 1, 0, 15, 4, 13,
], dtype=np.uint8).reshape(16, 3)

# Output axis -> base coordinate for the 12 even permutations of four axes
# (h4_classifier.rs:23-36); base coordinates 1, 2, 3 carry the signs s1, s2, s3.
EVEN_PERMUTATIONS = (
    (0, 1, 2, 3), (0, 2, 3, 1), (0, 3, 1, 2), (1, 0, 3, 2), (1, 2, 0, 3), (1, 3, 2, 0),
    (2, 0, 1, 3), (2, 1, 3, 0), (2, 3, 0, 1), (3, 0, 2, 1), (3, 1, 0, 2), (3, 2, 1, 0),
)


def icosian_coefficients() -> np.ndarray:
    """The 120 unit icosians, shape (120, 4, 2) int8: coordinate c is (a + b phi) / 2."""
    roots = np.zeros((120, 4, 2), dtype=np.int8)
    index = 0
    for axis in range(4):  # -1 and +1 on each axis: index 0 is -1, index 1 is +1
        roots[index, axis] = (-2, 0)
        roots[index + 1, axis] = (2, 0)
        index += 2
    for signs in range(16):  # (+-1/2, +-1/2, +-1/2, +-1/2), bit `axis` set = positive
        for axis in range(4):
            roots[index, axis] = (1 if signs >> axis & 1 else -1, 0)
        index += 1
    for perm in EVEN_PERMUTATIONS:  # even permutations of (0, 1/2, phi/2, (phi-1)/2)
        for signs in range(8):  # s3 changes fastest
            s1 = 1 if signs & 4 else -1
            s2 = 1 if signs & 2 else -1
            s3 = 1 if signs & 1 else -1
            base = ((0, 0), (s1, 0), (0, s2), (-s3, s3))
            for axis in range(4):
                roots[index, axis] = base[perm[axis]]
            index += 1
    assert index == 120
    return roots


def keep_q31() -> np.ndarray:
    """GEOMETRIC_KEEP_Q31[i] = isqrt(2^62 - 2^(60 - 2 i)), i = 0..15."""
    return np.array([math.isqrt((1 << 62) - (1 << (60 - 2 * i))) for i in range(16)], dtype=np.uint64)


def roots_q12() -> np.ndarray:
    """The orbit roots at Q12, shape (16, 8) int32."""
    return (ROOTS.astype(np.int32) << 12).astype(np.int32)


def axes_codes(state: int) -> np.ndarray:
    """The eight signed-axis codes of Cl(0,6) state ``state`` (< 64)."""
    return AXES[8 * state: 8 * state + 8]


def act(state: int, x) -> np.ndarray:
    """Route state ``state`` applied to an 8-vector: out[d] = +-x[code & 7] (code & 8 negates)."""
    state = int(state)
    codes = AXES[8 * state: 8 * state + 8]
    x = np.asarray(x)
    return np.where(codes & 8, -x[codes & 7], x[codes & 7])


def compose_table() -> np.ndarray:
    """(64, 64) uint8: entry (a, b) is the state c with act(c, x) == act(a, act(b, x))."""
    probe = np.arange(1, 9)
    index = {tuple(act(c, probe)): c for c in range(64)}
    out = np.zeros((64, 64), np.uint8)
    for a in range(64):
        for b in range(64):
            out[a, b] = index[tuple(act(a, act(b, probe)))]
    return out


def root_id(x) -> int:
    """The orbit root equal to ``x``, or -1."""
    hit = np.nonzero((ROOTS == np.asarray(x)).all(axis=1))[0]
    return int(hit[0]) if len(hit) else -1
