"""The reference's witness models for the discrete M1 evaluator, built with uor_fbs.d11's
container writer exactly as the reference's tests build them
(crates/uor-r4-integer/src/discrete_d11.rs:1996-2458), with their literal expectations.
Shared by the oracle tests (CPU) and the HIP scorer tests (GPU)."""

import numpy as np

from uor_fbs import d11

A = [2, 2, 0, 0, 0, 0, 0, 0]
NEG_A = [-2, -2, 0, 0, 0, 0, 0, 0]
C_ROOT = [-2, 2, 0, 0, 0, 0, 0, 0]
NEG_B = [0, 0, -2, 0, -2, 0, 0, 0]
B = [0, 0, 2, 0, 2, 0, 0, 0]
D_ROOT = [2, -2, 0, 0, 0, 0, 0, 0]


def shape(vocabulary, blocks, context, kept_cells, stages, read_mode="route", read_kept=0,
          read_sweeps=0, policy="nearest_address_margin_v1", init="zero_gates_v1", epoch=0):
    return d11.Shape(vocabulary, blocks, context, kept_cells, stages, read_mode, read_kept,
                     read_sweeps, policy, init, 7, epoch)


def model(shape_, tokens, routes, gates, trunk=None):
    """The parsed artifact of the container the reference's builder writes."""
    blob = d11.build_container(shape_, np.array(tokens, np.int32), np.array(routes, np.uint32),
                               np.array(gates, np.int32), trunk)
    return d11.parse_container(blob), blob


def flat(*blocks):
    return [v for b in blocks for v in b]


# 1. Two-token exact writer witness (:2088-2145).
SHAPE_2 = shape(2, 2, 1, 2, 1)
WRITER_2 = ([[A, A], [NEG_A, NEG_A]], [0, 0], [0, 0])
WRITER_2_EDITED = ([[A, NEG_A], [NEG_A, A]], [0, 0], [0, 0])
# (prefix, target) -> prediction, admitted cells, top8, token rivals, address rivals, loss
WRITER_2_EXPECT = {((0,), 0): (0, [0, 17], [0, 1], 1, 1, 0),
                   ((1,), 0): (1, [17, 0], [1, 0], 1, 1, 640)}

# 2. Three-token context transport witness (:2147-2171).
SHAPE_3 = shape(3, 2, 3, 3, 2)
TRANSPORT_3 = ([[A, A], [NEG_A, NEG_A], [B, B]], [0, 0, 0, 0], [0, 0, 0, 0])
TRANSPORT_3_EXPECT = {(0, 1, 2): flat(NEG_B, NEG_B), (0, 0, 2): flat(B, B)}

# 3. Flock and Relation copy successor (:2174-2249).
COPY_TOKENS = [[B, A], [A, D_ROOT], [NEG_A, NEG_B], [C_ROOT, A], [D_ROOT, A]]
COPY_PREFIX = [0, 1, 2, 3, 4, 1]
FLOCK_SHAPE = shape(5, 2, 6, 2, 2, "flock", 1, 0, init="active_leaf_v1")
FLOCK_GATES = [0, 0, 1, 0]
REL_SHAPE = shape(5, 2, 6, 2, 2, "relation", 1, 1, init="active_leaf_v1")
REL_BASE_GATES = [0] * 14
REL_BASE_GATES[2] = 1
REL_ACTIVE_GATES = list(REL_BASE_GATES)
REL_ACTIVE_GATES[6] = 1
COPY_BASE_READ = flat(A, D_ROOT)
COPY_ACTIVE_READ = flat(A, B)
# block 1's relation scores at nodes 0, 1, 2, 4, 5 under the active gates
REL_ACTIVE_B1 = [0, 0, 8, 0, 4]

# 4. Refusals (:2252-2303).
REFUSE_SHAPE = shape(2, 2, 2, 2, 1, policy="occupied_cell_rank_hinge_v1")
REFUSE_MODEL = ([[A, A], [NEG_A, NEG_A]], [0, 0], [0, 0])

# 5. The 19-table trunk's joint pointer (:2306-2458).
TRUNK_SHAPE = shape(3, 4, 4, 3, 2, epoch=1)
TRUNK_TOKENS = [[A, A, A, A], [NEG_A, NEG_A, NEG_A, NEG_A], [B, B, B, B]]


def trunk_witness():
    sparse = {name: np.zeros((0, 3), np.uint32) for name in d11.TRUNK_SPARSE}
    sparse["query_table"] = np.array([[0, 2, 5]], np.uint32)
    return d11.Trunk(np.ones(64, np.uint32), np.zeros(4, np.uint32),
                     np.array([0, 10, 5, 3], np.uint32), sparse)


TRUNK_EXPECT = {(0,): (flat(B, B, B, B), 2), (0, 1, 2, 0): (flat(NEG_A, NEG_A, NEG_A, NEG_A), 1)}


def rows_of(cases):
    """(prefixes, lengths, targets) of a list of (prefix, target)."""
    stride = max(len(p) for p, _ in cases)
    pre = np.zeros((len(cases), stride), np.uint32)
    for i, (p, _) in enumerate(cases):
        pre[i, :len(p)] = p
    return (pre, np.array([len(p) for p, _ in cases], np.int32),
            np.array([t for _, t in cases], np.uint32))
