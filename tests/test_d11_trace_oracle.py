"""The discrete oracle's traced evaluation (evaluate_prefix_traced, discrete_d11.rs:1768-1770;
trace words :293-297, :1337-1451, :1453-1741) and its state-transport knockout
(with_state_transport_knockout, :1283-1304; :1346-1361, :1810-1814), pinned by what the
already-pinned outputs and the geometry fix:

- tracing changes no record;
- route words: stage 0's goal is the frontier port nearest the transported query, later goals
  the nearest branch of the previous root, by (L1, Hamming) with the first port on ties (brute
  force over the ports); roots and composed states chain stage to stage through BFS and the
  composition table; the nodes follow the row plan from the frontier down to the header's atom;
  and the final state carries that atom's token block onto the block's read vector;
- active words: the query frame and payload roots, each level's eligible count from the row
  plan, found = min(kept, eligible), the kept nodes equal to a brute-force sort of the eligible
  nodes by (relation score desc, L1, Hamming, last position desc, node), their route states
  from BFS, level-0 carried roots in closed form, each level's snapped root recomputed from the
  carried roots, and the block's read recomputed from the gated snapped roots;
- relation words: the relation scores of d11_oracle_row_relation (pinned by the reference's
  witness), padded to a full context's node count;
- knockout: the last token's blocks read untransported, no trunk, gates and routes inert.
"""

import numpy as np
import pytest

import d11_cases as W
import oracle
from uor_fbs import d11, tables

NONE = 0xFFFFFFFF
ROOTS = tables.ROOTS.astype(np.int64)
COMPOSE = tables.compose_table()


def plan(length):
    """build_row_plan (discrete_d11.rs:813-884): nodes as (children, atom, level, first, last) and
    the frontier, each new atom merging the last three frontier nodes while they share a level."""
    nodes, frontier = [], []
    for atom in range(length):
        frontier.append(len(nodes))
        nodes.append((None, atom, 0, atom, atom))
        while len(frontier) >= 3 and len({nodes[i][2] for i in frontier[-3:]}) == 1:
            c = tuple(frontier[-3:])
            nodes.append((c, None, nodes[c[0]][2] + 1, nodes[c[0]][3], nodes[c[2]][4]))
            del frontier[-3:]
            frontier.append(len(nodes) - 1)
    return nodes, frontier


def root_id(x):
    return tables.root_id(np.asarray(x, np.int64))


def cost(x, r):
    d = np.asarray(x, np.int64) - ROOTS[r]
    return int(np.abs(d).sum()), int((d != 0).sum())


def snap(x, n):
    """The nearest n-fold root by (L1, Hamming), lowest root on ties: a brute force over 16."""
    x = np.asarray(x, np.int64)
    return min(range(16), key=lambda r: (int(np.abs(x - n * ROOTS[r]).sum()),
                                         int((x != n * ROOTS[r]).sum()), r))


def block(art, tok, b):
    return art.table.reshape(art.shape.vocabulary, art.shape.blocks, 8)[tok, b]


def traced(art, rows, knockout=False):
    pre, lens, tg = rows
    out, tr, rel = oracle.d11_score_rows_traced(art, pre, lens, tg, knockout=knockout, threads=2)
    return out, tr, rel


def random_rows(art, n, seed):
    pre, lens, tg = d11.panel_rows(art, n, seed)
    lens[:3] = [1, 2, art.shape.context]
    return pre, lens, tg


def check_route(art, prefix, rec, words):
    s = art.shape
    S = s.stages
    stride = 4 + 6 * S
    nodes, frontier = plan(len(prefix))
    routes = np.asarray(art.routes).reshape(s.blocks, S)
    last = int(prefix[-1])
    for b in range(s.blocks):
        w = words[b * stride:(b + 1) * stride]
        read = rec["read_vector"][8 * b:8 * b + 8]
        assert w[0] == len(frontier) and w[1] == root_id(read)
        taken = int(w[2])
        assert 1 <= taken <= S
        root, total, node = 0, 0, None
        for st in range(S):
            ws = w[4 + 6 * st:10 + 6 * st]
            if st >= taken:
                assert (ws == NONE).all()
                continue
            frame, r0, best, goal, tot, nxt = (int(v) for v in ws)
            assert frame == routes[b, st] and r0 == root
            q = tables.act(frame, block(art, last, b))
            ports = list(range(len(frontier))) if st == 0 else list(tables.BRANCH[root])
            want = min(range(len(ports)), key=lambda p: (*cost(q, ports[p]), p))
            assert best == want and goal == ports[best]
            total = int(COMPOSE[tables.BFS[(root << 4) + goal], total])
            assert tot == total
            root = goal
            node = frontier[best] if st == 0 else nodes[node][0][best]
            assert nxt == node
        assert nodes[node][1] == w[3]
        carried = tables.act(total, block(art, int(prefix[w[3]]), b))
        assert carried.tolist() == read.tolist()


def check_active(art, prefix, rec, words, rel):
    s = art.shape
    S, B = s.stages, s.blocks
    stride = 4 + 28 * S
    nodes, _ = plan(len(prefix))
    L = len(prefix)
    last = int(prefix[-1])
    gates = np.asarray(art.gates)[:B * S].reshape(B, S)
    for b in range(B):
        w = words[b * stride:(b + 1) * stride]
        f = B - 1 if b == 0 else 0
        fq = root_id(block(art, last, f))
        read = rec["read_vector"][8 * b:8 * b + 8]
        assert (w[0], w[1], w[3]) == (fq, root_id(read), root_id(block(art, last, b)))
        frame = [root_id(block(art, int(prefix[n[3]]), f)) for n in nodes]
        u = block(art, last, b).astype(np.int64)
        terms = 1
        for l in range(S):
            wl = w[4 + 28 * l:4 + 28 * (l + 1)]
            gate = int(gates[b, l])
            elig = [i for i, n in enumerate(nodes) if n[2] == l and n[4] + 1 < L]
            found = min(s.read_kept, len(elig))
            assert (wl[0], wl[1], wl[3]) == (gate + 1, found, len(elig))
            r = (lambda i: int(rel[b, i])) if rel is not None else (lambda i: 0)
            top = sorted(elig, key=lambda i: (-r(i), *cost(ROOTS[frame[i]], fq), -nodes[i][4], i))[:found]
            assert wl[4:4 + found].tolist() == top
            assert (wl[4 + found:12] == NONE).all() and (wl[12 + found:20] == NONE).all()
            assert (wl[20 + found:28] == NONE).all()
            if found == 0:
                assert wl[2] == NONE
                continue
            acts = [int(tables.BFS[(frame[i] << 4) + fq]) for i in top]
            assert wl[12:12 + found].tolist() == acts
            for k, i in enumerate(top):
                if nodes[i][1] is not None:  # an atom's payload is its token's block
                    assert wl[20 + k] == root_id(tables.act(acts[k], block(art, int(prefix[nodes[i][1]]), b)))
            m = snap(ROOTS[wl[20:20 + found]].sum(0), found)
            assert wl[2] == m
            if gate:
                u += gate * ROOTS[m]
                terms += 1
        assert w[2] == terms and snap(u, terms) == root_id(read)


MODELS = [
    ("route", 2, 300, 30, 4, 0, 0, False, 31),
    ("route", 4, 2000, 192, 8, 0, 0, True, 32),
    ("flock", 3, 700, 81, 6, 3, 0, False, 33),
    ("relation", 2, 200, 27, 3, 1, 1, False, 34),
    ("relation", 4, 1500, 100, 8, 8, 2, True, 35),
]


@pytest.mark.parametrize("case", MODELS, ids=[f"{c[0]}-b{c[1]}-ctx{c[3]}" for c in MODELS])
def test_traced_rows(case):
    mode, blocks, V, ctx, kc, kept, sweeps, trunk, seed = case
    art = d11.synthetic(vocabulary=V, blocks=blocks, context=ctx, kept_cells=kc, read_mode=mode,
                        read_kept=kept, read_sweeps=sweeps, seed=seed, trunk=trunk,
                        trunk_entries=5000)
    rows = random_rows(art, 24, seed + 1)
    plain = oracle.d11_score_rows(art, *rows, threads=2)
    out, tr, rel = traced(art, rows)
    assert (out["status"] == 0).all()
    assert out.tobytes() == plain.tobytes()
    words = (4 + (6 if mode == "route" else 28) * art.shape.stages) * blocks
    assert tr.shape == (24, words)
    full = len(plan(ctx)[0])
    assert (rel is None) == (mode != "relation")
    for r in range(24):
        prefix = rows[0][r, :rows[1][r]]
        if art.trunk is not None:
            continue  # the pointer gate moves the read after the trace; checked untrunked below
        if mode == "route":
            check_route(art, prefix, out[r], tr[r])
        else:
            rr = None
            if rel is not None:
                _, want = oracle.d11_row_relation(art, prefix, int(rows[2][r]))
                n = want.shape[1]
                assert rel.shape[2] == full
                assert (rel[r][:, :n].view(np.int32) == want).all() and (rel[r][:, n:] == NONE).all()
                rr = want
            check_active(art, prefix, out[r], tr[r], rr)


def test_trunk_models_trace_the_read_before_the_pointer_gate():
    """With the trunk the trace records the read; the same model without its trunk gives the
    same words and a record whose read the checks above hold to."""
    for mode in ("route", "relation"):
        art = d11.synthetic(vocabulary=1500, context=100, read_mode=mode, read_kept=8,
                            read_sweeps=2, seed=36, trunk_entries=5000)
        bare = d11.Artifact(art.shape, art.table, art.cells, art.routes, art.gates, None)
        rows = random_rows(art, 16, 37)
        _, tr, rel = traced(art, rows)
        out_b, tr_b, rel_b = traced(bare, rows)
        assert (tr == tr_b).all() and (rel is None or (rel == rel_b).all())
        for r in range(16):
            prefix = rows[0][r, :rows[1][r]]
            if mode == "route":
                check_route(bare, prefix, out_b[r], tr_b[r])
            else:
                _, want = oracle.d11_row_relation(bare, prefix, int(rows[2][r]))
                check_active(bare, prefix, out_b[r], tr_b[r], want)


def test_relation_witness_trace():
    """The reference's active relation witness (discrete_d11.rs:2368-2458): its block-1 relation
    scores appear in the relation words, and the active read's trace checks out."""
    art, _ = W.model(W.REL_SHAPE, W.COPY_TOKENS, [0, 0, 0, 0], W.REL_ACTIVE_GATES)
    out, tr, rel = traced(art, W.rows_of([(W.COPY_PREFIX, 2)]))
    assert out[0]["read_vector"][:16].tolist() == W.COPY_ACTIVE_READ
    b1 = rel[0][1].view(np.int32)
    assert [b1[0], b1[1], b1[2], b1[4], b1[5]] == W.REL_ACTIVE_B1
    _, want = oracle.d11_row_relation(art, np.asarray(W.COPY_PREFIX), 2)
    check_active(art, np.asarray(W.COPY_PREFIX), out[0], tr[0], want)


@pytest.mark.parametrize("mode", ["route", "flock", "relation"])
def test_knockout(mode):
    art = d11.synthetic(vocabulary=1500, context=100, read_mode=mode, read_kept=8, read_sweeps=2,
                        seed=38, trunk_entries=5000)
    rows = random_rows(art, 16, 39)
    out, tr, rel = traced(art, rows, knockout=True)
    plain = oracle.d11_score_rows(art, *rows, threads=2)
    assert (out["status"] == 0).all()
    S, B = art.shape.stages, art.shape.blocks
    for r in range(16):
        prefix = rows[0][r, :rows[1][r]]
        last = int(prefix[-1])
        want = np.concatenate([block(art, last, b) for b in range(B)])
        # Untransported and ungated: the last token's blocks, no pointer gate.
        assert out[r]["read_vector"][:8 * B].tolist() == want.tolist()
        if mode == "route":
            stride = 4 + 6 * S
            _, frontier = plan(len(prefix))
            for b in range(B):
                w = tr[r][b * stride:(b + 1) * stride]
                assert w[:3].tolist() == [len(frontier), root_id(block(art, last, b)), 0]
                assert (w[3:] == NONE).all()
        else:
            zero = d11.Artifact(art.shape, art.table, art.cells, np.zeros_like(art.routes),
                                np.zeros_like(art.gates), None)
            _, tr0, rel0 = traced(zero, rows)
            assert (tr[r] == tr0[r]).all()
            if rel is not None:
                assert (rel[r] == rel0[r]).all()
                n = len(plan(len(prefix))[0])
                assert (rel[r][:, :n] == 0).all()
    # The knockout is the flag's alone: the model's own evaluation is unchanged.
    assert oracle.d11_score_rows(art, *rows, threads=2).tobytes() == plain.tobytes()


def test_m1_shape_reads_hold_to_the_trace_checks():
    """At the M1 panel's shape (vocabulary 4,096, 4 blocks, context 192, relation read keeping 8
    with one sweep), the oracle's reads on rows of 186-192 tokens satisfy every check above: the
    kept nodes by brute-force sort, each level's snapped root and the block's read recomputed
    from the words. (The trunk's pointer gate comes after the read; the model is taken without it.)"""
    art = d11.synthetic(vocabulary=4096, blocks=4, context=192, kept_cells=8, read_mode="relation",
                        read_kept=8, read_sweeps=1, seed=44, trunk=False)
    pre, lens, tg = d11.panel_rows(art, 6, 45, min_len=186)
    out, tr, rel = traced(art, (pre, lens, tg))
    assert (out["status"] == 0).all()
    for r in range(6):
        prefix = pre[r, :lens[r]]
        _, want = oracle.d11_row_relation(art, prefix, int(tg[r]))
        check_active(art, prefix, out[r], tr[r], want)
