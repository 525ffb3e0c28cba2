"""The discrete M1 oracle (oracle/d11_oracle.c) pinned to the reference's own witness tests
(crates/uor-r4-integer/src/discrete_d11.rs:2088-2458, literal read vectors, admitted cells,
rankings, rival counts, losses and relation scores), the container reader's refusals against
the reference's planted faults, the geometry tables against closed forms, and the row plan
against its closed-form node counts."""

import json

import numpy as np
import pytest

import d11_cases as W
import oracle
from uor_fbs import d11, tables


def score(art, cases):
    return oracle.d11_score_rows(art, *W.rows_of(cases), threads=1)


def test_route_writer_witness():
    art, _ = W.model(W.SHAPE_2, *W.WRITER_2)
    out = score(art, list(W.WRITER_2_EXPECT))
    for rec, want in zip(out, W.WRITER_2_EXPECT.values()):
        pred, admitted, top8, trivals, arivals, loss = want
        assert rec["status"] == 0
        assert rec["prediction"] == pred
        assert rec["admitted"][:rec["admitted_count"]].tolist() == admitted
        assert rec["top8"][:rec["top8_count"]].tolist() == top8
        assert (rec["token_rivals"], rec["address_rivals"], rec["selected_loss"]) == (trivals, arivals, loss)
    # The edited table changes the read vector and the admitted cells (:2124-2144).
    edited, _ = W.model(W.SHAPE_2, *W.WRITER_2_EDITED)
    e = score(edited, [((0,), 0)])[0]
    assert e["admitted"][:e["admitted_count"]].tolist() == [1, 16]
    assert e["read_vector"][:16].tolist() != out[0]["read_vector"][:16].tolist()


def test_context_transport_witness():
    art, _ = W.model(W.SHAPE_3, *W.TRANSPORT_3)
    out = score(art, [(p, 0) for p in W.TRANSPORT_3_EXPECT])
    for rec, want in zip(out, W.TRANSPORT_3_EXPECT.values()):
        assert rec["status"] == 0 and rec["read_vector"][:16].tolist() == want


def test_flock_and_relation_copy_successor_witness():
    flock, _ = W.model(W.FLOCK_SHAPE, W.COPY_TOKENS, [0, 0, 0, 0], W.FLOCK_GATES)
    f = score(flock, [(W.COPY_PREFIX, 2)])[0]
    assert f["read_vector"][:16].tolist() == W.COPY_BASE_READ and f["selected_loss"] == 640
    base, _ = W.model(W.REL_SHAPE, W.COPY_TOKENS, [0, 0, 0, 0], W.REL_BASE_GATES)
    b = score(base, [(W.COPY_PREFIX, 2)])[0]
    assert b["read_vector"][:16].tolist() == W.COPY_BASE_READ and b["selected_loss"] == 640
    active, _ = W.model(W.REL_SHAPE, W.COPY_TOKENS, [0, 0, 0, 0], W.REL_ACTIVE_GATES)
    rec, rel = oracle.d11_row_relation(active, W.COPY_PREFIX, 2)
    assert rec["read_vector"][:16].tolist() == W.COPY_ACTIVE_READ and rec["selected_loss"] == 448
    b1 = rel[1]
    assert [b1[0], b1[1], b1[2], b1[4], b1[5]] == W.REL_ACTIVE_B1


def test_trunk_joint_pointer_witness():
    art, blob = W.model(W.TRUNK_SHAPE, W.TRUNK_TOKENS, [0] * 8, [0] * 8, W.trunk_witness())
    assert art.trunk is not None
    out = score(art, [(p, 0) for p in W.TRUNK_EXPECT])
    for rec, (read, pred) in zip(out, W.TRUNK_EXPECT.values()):
        assert rec["status"] == 0
        assert rec["read_vector"][:32].tolist() == read and rec["prediction"] == pred
    # Planted faults (:2438-2457): a trailing byte, a tail token outside the vocabulary.
    with pytest.raises(d11.DiscreteError):
        d11.parse_container(blob + b"\0")
    hlen = int.from_bytes(blob[8:16], "little")
    start = 16 + hlen + (64 - (16 + hlen) % 64) % 64
    header = json.loads(blob[16:16 + hlen])
    off = start + header["tables"][14]["span"]["offset"] + 4
    bad = bytearray(blob)
    bad[off:off + 4] = (99).to_bytes(4, "little")
    with pytest.raises(d11.DiscreteError, match="invalid token"):
        d11.parse_container(bytes(bad))


def test_refusals_of_containers_and_prefixes():
    art, blob = W.model(W.REFUSE_SHAPE, *W.REFUSE_MODEL)
    out = score(art, [((), 0), ((0, 1, 0), 0), ((2,), 0), ((0,), 2)])
    assert out["status"].tolist() == [1, 1, 2, 8]
    bad = bytearray(blob)
    bad[0] ^= 1
    with pytest.raises(d11.DiscreteError, match="magic"):
        d11.parse_container(bytes(bad))
    hlen = int.from_bytes(blob[8:16], "little")
    unaligned = 16 + hlen
    start = unaligned + (64 - unaligned % 64) % 64
    if unaligned < start:
        bad = bytearray(blob)
        bad[unaligned] = 1
        with pytest.raises(d11.DiscreteError, match="padding"):
            d11.parse_container(bytes(bad))
    header = json.loads(blob[16:16 + hlen])
    bad = bytearray(blob)
    bad[start + header["tables"][1]["span"]["offset"]] ^= 1
    with pytest.raises(d11.DiscreteError, match="cells"):
        d11.parse_container(bytes(bad))
    sh = W.shape(2, 2, 2, 2, 2, policy="occupied_cell_rank_hinge_v1")
    with pytest.raises(d11.DiscreteError, match="shape"):
        W.model(sh, *W.REFUSE_MODEL)


def test_geometry_tables():
    # COMPOSE is the product of route states; BFS carries root s to root d; every state is a
    # signed permutation; the orbit of the anchor under the 64 states is the 16 roots.
    comp = tables.compose_table()
    x = np.arange(1, 9)
    for a in range(64):
        assert sorted(tables.AXES[8 * a:8 * a + 8] & 7) == list(range(8))
        for b in range(0, 64, 7):
            assert (tables.act(comp[a, b], x) == tables.act(a, tables.act(b, x))).all()
        assert comp[a, comp[a, comp[a, a]]] == 0          # a^4 = identity (cl06_inverse)
    for s in range(16):
        for d in range(16):
            assert tables.root_id(tables.act(tables.BFS[16 * s + d], tables.ROOTS[s])) == d
    orbit = {tables.root_id(tables.act(a, tables.ROOTS[0])) for a in range(64)}
    assert orbit == set(range(16))
    assert all(len(set(row)) == 3 for row in tables.BRANCH)
    # The C header holds the same arrays.
    text = open(oracle.ROOT + "/uor-r4_amd/csrc/d11_tables.h").read()
    for name, arr in d11.tables_header_arrays().items():
        body = text.split(name)[1].split("};")[0].split("=", 1)[1]
        vals = [int(v) for v in body.replace("{", " ").replace("}", " ").replace(",", " ").split()]
        assert vals == np.asarray(arr).reshape(-1).astype(int).tolist(), name


@pytest.mark.parametrize("n", [1, 2, 3, 4, 8, 9, 13, 26, 27, 100, 192, 242, 243])
def test_row_plan_counts(n):
    # Nodes: every atom plus one parent per completed triple at each level; the frontier holds
    # the base-3 digits of n (digit k = nodes of level k still waiting for a parent).
    nodes, frontier = oracle.d11_plan(n)
    inner, m = 0, n
    while m >= 3:
        inner += m // 3
        m //= 3
    digits, m = 0, n
    while m:
        digits += m % 3
        m //= 3
    assert (nodes, frontier) == (n + inner, digits)
    # Stages: one per base-3 digit of the context.
    assert d11.expected_stages(n) == len(np.base_repr(n, 3))


def brute_writer(art, read):
    """The writer's admission and ranking by sorting (no insertion loops)."""
    q = np.array(read, np.int64).reshape(art.shape.blocks, 8)
    R = tables.ROOTS.astype(np.int64)
    occ = sorted(set(art.cells.tolist()))
    ad = {c: int(np.abs(q[0] - R[c >> 4]).sum() + np.abs(q[-1] - R[c & 15]).sum()) for c in occ}
    admitted = sorted(occ, key=lambda c: (ad[c], c))[:art.shape.kept_cells]
    toks = [t for t in range(art.shape.vocabulary) if art.cells[t] in admitted]
    td = {t: int(np.abs(q - art.table[t]).sum()) for t in toks}
    return admitted, sorted(toks, key=lambda t: (td[t], t))[:8]


@pytest.mark.parametrize("mode,seed", [("route", 1), ("flock", 2), ("relation", 3)])
def test_writer_orderings_brute_force(mode, seed):
    art = d11.synthetic(vocabulary=300, blocks=3, context=20, kept_cells=5, read_mode=mode,
                        read_kept=3, read_sweeps=2, seed=seed, trunk=False)
    pre, lens, tg = d11.panel_rows(art, 40, seed)
    out = oracle.d11_score_rows(art, pre, lens, tg, threads=2)
    assert (out["status"] == 0).all()
    for rec in out:
        admitted, top8 = brute_writer(art, rec["read_vector"][:24])
        assert rec["admitted"][:rec["admitted_count"]].tolist() == admitted
        assert rec["top8"][:rec["top8_count"]].tolist() == top8


def test_synthetic_container_round_trip():
    art = d11.synthetic(vocabulary=500, context=30, seed=4, trunk_entries=300)
    blob = d11.build_container(art.shape, art.table, art.routes, art.gates, art.trunk)
    back = d11.parse_container(blob)
    assert back.shape == art.shape and (back.table == art.table).all()
    for name in d11.TRUNK_SPARSE:
        assert (back.trunk.sparse[name] == art.trunk.sparse[name]).all()
