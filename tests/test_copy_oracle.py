"""The copy heads' Hamming read oracle (oracle/copy_oracle.c) pinned to the reference's own
copy-rule tests (hamming.rs:705-1058, literal positions and means), the margin weight against
its closed form, and the rules against brute force on random streams."""

import numpy as np
import pytest

import copy_cases as K
import oracle
from uor_fbs.copy import RULES, copy_weight_q31, pack_rows


class OracleRead:
    def __init__(self, heads):
        self.heads = heads

    def _run(self, tokens, opening):
        tok, lens = pack_rows([list(tokens)])
        return oracle.copy_mean_rows(self.heads, tok, lens, [int(opening)])

    def mean_at(self, tokens, opening=False):
        out, found, _ = self._run(tokens, opening)
        return out[0].tolist() if found[0] else None

    def mean(self, tokens):
        return self.mean_at(tokens, False)

    def choose_ruled(self, h, tokens, opening=False):
        _, _, chosen = self._run(tokens, opening)
        return [(int(v) & 0xffffff, int(v) >> 24) for v in chosen[0, h] if v >= 0]


def make_oracle(kept, rule, **kw):
    return OracleRead(K.heads(kept, rule, **kw))


def test_the_reference_copy_rule_tests():
    K.check_rust_tests(make_oracle)


def test_copy_weight_closed_form():
    # max(0, m - d) / max(m, 1) at Q31, floored; a 4-bit margin gives 1, 3/4, 1/2, 1/4, 0.
    assert [copy_weight_q31(4 << 16, d) for d in range(6)] == [1 << 31, 3 << 29, 1 << 30, 1 << 29, 0, 0]
    assert copy_weight_q31(0, 0) == 0 and copy_weight_q31(100, 0) == (100 << 31) // (1 << 16)


def tdiv(a, b):
    """Integer division truncating toward zero (Rust's and C's)."""
    q = abs(a) // b
    return q if a >= 0 else -q


def brute(heads, tokens, opening):
    """Each rule by its definition over explicit candidate lists (no insertion or scans)."""
    codes, width = heads.codes, heads.table.shape[1]
    out, found = np.zeros(width, dtype=object), 0
    n = len(tokens)
    for h in range(codes.shape[1]):
        first = 0 if heads.pair_first is None else int(heads.pair_first[h])
        code = lambda v: int(codes[v, h])                                        # noqa: E731
        join = lambda a, b: (code(a) & first) | (code(b) & ~first) if first else code(a)  # noqa: E731
        if n == 0:
            continue
        t = n - 1
        q = join(tokens[t], tokens[max(t - 1, 0)])
        keys = {s: join(tokens[s - 1], tokens[max(s - 2, 0)]) for s in range(1, t)}
        dist = {s: bin(q ^ k).count("1") for s, k in keys.items()}
        rule = heads.rule
        if rule == "longest-after-opening":
            opens = (n >= 2 and (tokens[t - 1], tokens[t]) == tuple(heads.marker)) if heads.marker else opening
            rule = "latest-exact" if opens else "longest-exact"
        if rule == "mean":
            picks = sorted(dist, key=lambda s: (dist[s], s))[:heads.kept]
        elif rule == "latest-exact":
            picks = [max(s for s in dist if dist[s] == 0)] if any(d == 0 for d in dist.values()) else []
        elif rule == "latest-nearest":
            picks = [max(s for s in dist if dist[s] == min(dist.values()))] if dist else []
        else:
            kd = 2 if first else 1
            ex = [s for s in dist if keys[s] == q]
            lg = [s for s in ex if s > kd and code(tokens[s - 1 - kd]) == code(tokens[t - kd])]
            picks = [max(lg)] if lg else ([max(ex)] if ex else [])
        acc, count = np.zeros(width, dtype=object), 0
        for s in picks:
            w = copy_weight_q31(int(heads.margins_q16[h]), dist[s])
            if w:
                count += 1
                acc += np.array(heads.table[tokens[s]], dtype=object) * w
        if count:
            found += 1
            out += np.array([tdiv(int(v), count) for v in acc], dtype=object)
    if not found:
        return None
    return [tdiv(int(v), found) for v in out]


@pytest.mark.parametrize("rule", sorted(RULES))
def test_rules_against_brute_force(rule):
    heads = K.random_heads(7 + RULES[rule], rule=rule)
    tok, lens, opening = K.random_streams(11 + RULES[rule], 300, 60, 40)
    out, found, _ = oracle.copy_mean_rows(heads, tok, lens, opening)
    for r in range(len(lens)):
        want = brute(heads, [int(x) for x in tok[r, :lens[r]]], bool(opening[r]))
        got = out[r].tolist() if found[r] else None
        assert got == want, r


def test_vocab_codes_restatement_closed_form():
    # The identity rotation (raw [1, 0, 0, 0]: unit 2^31) leaves each point, so a code's bits are
    # the signs of the table row (bit c set at or above 0); a half turn about the first axis
    # (raw [0, 1, 0, 0]) maps (a, b, c, d) to (-b, a, -d, c).
    rng = np.random.default_rng(3)
    table = rng.integers(-5, 6, (40, 32)).astype(np.int16)
    ident = np.tile(np.array([1, 0, 0, 0], np.int32), 8)
    codes = oracle.copy_vocab_codes(ident, table, 2, 2)
    for v in range(40):
        for h in range(2):
            want = sum(1 << c for c in range(16) if table[v, 16 * h + c] >= 0)
            assert int(codes[v, h]) == want
    turn = np.tile(np.array([0, 1, 0, 0], np.int32), 8)
    codes = oracle.copy_vocab_codes(turn, table, 2, 1)
    for v in range(40):
        q = table[v, :16].reshape(4, 4).astype(int)
        rot = np.stack([-q[:, 1], q[:, 0], -q[:, 3], q[:, 2]], 1).reshape(-1)
        assert int(codes[v, 0]) == sum(1 << c for c in range(16) if rot[c] >= 0)
