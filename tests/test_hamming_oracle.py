"""The oracle's Hamming reads (oracle/fbs_oracle.c, the lut-stack/6 reads inside the step) pinned
without retyping them:

- the hook sums against the reference's literal known answers (tests.rs:5679-5707);
- every vocabulary entry's key codes against an f64 sign code of the rotated table point and
  against the copy read's separate restatement (oracle/copy_oracle.c);
- the copy heads inside the step against oracle/copy_oracle.c (itself pinned by the reference's
  copy-rule tests), under every rule, mixed copy keys and the reply marker;
- the type heads against an f64 reference of the float read, as type_heads_match_the_f64_reference
  (tests.rs:5757-5856): payloads within half a step, the read's move within a step and a half;
- the ask heads and their carry against an f64 reference, as
  an_asking_read_brings_back_the_kept_tokens_points (tests.rs:8380-8470), within 0.6 of a step;
- zero weights reduce the model to the read-free one, and a decode split and resumed through the
  session stream equals the decode in one call;
- the type and ask heads' integers exactly, on cases whose answers the quaternion units' table
  and the definitions fix: payloads under the units 1, -1, i, j, k equal the point permuted and
  negated, and under the half unit each signed sum halved with odd negative sums rounded away
  from zero; one head keeping one position moves the stream by its weight times the payload; a
  head's halving by its count and the heads' halving by their number truncate toward zero (sums
  built to land half a step from a rounding boundary of the hook's output); an ask head brings
  back the kept position's own token's row, raised 4 bits. Each of these fails on the oracle
  with a planted mistake (payload rounding half up, either halving floored).
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import synth
from uor_fbs.copy import Heads

RULE_NAMES = ["mean", "latest-exact", "latest-nearest", "longest-exact", "longest-after-opening"]
BASE = synth.Spec(vocab=256, width=64, mlp=64, layers=2, context=64, kept=8)


def test_hook_sums_known_answers():
    # the_hooks_round_the_sum_not_the_product (tests.rs:5679-5690)
    assert oracle.stream_sum(3, -1, 1 << 50, 0, 0) == 3
    assert oracle.stream_sum(-3, 1, 1 << 50, 0, 0) == -3
    assert oracle.stream_sum(3, 1, 1 << 50, 0, 0) == 4
    assert oracle.readout_sum(3, 1, (3 << 19) - (1 << 42), 0, 0) == 3
    assert oracle.readout_sum(-3, 1, (-3 << 19) + (1 << 42), 0, 0) == -3
    assert oracle.readout_sum(-7, 1 << 24, 5 << 19, 0, 0) == 5
    # the_type_term_joins_the_single_rounding (tests.rs:5697-5707)
    assert oracle.stream_sum(3, 0, 0, -1, 1 << 54) == 3
    assert oracle.stream_sum(-3, 0, 0, 1, 1 << 54) == -3
    assert oracle.stream_sum(3, 1, 1 << 49, 1, 1 << 53) == 4
    assert oracle.readout_sum(3, 5, None, 1, 1 << 54) == 4
    assert oracle.readout_sum(3, 5, None, -1, 1 << 54) == 3
    assert oracle.readout_sum(3, 5, None, 0, 1 << 54) == 3
    # readout_ask_sum (hamming.rs:1946-1953) by its definition: no move without a match; at
    # w = 2^24 (1.0) a move lands on its mean exactly; two half moves meet in the middle, and a
    # move of half a step rounds away from zero.
    assert oracle.readout_ask_sum(-9, 1 << 24, None, 1 << 24, None) == -9
    assert oracle.readout_ask_sum(-7, 1 << 24, 5 << 19, 0, None) == 5
    assert oracle.readout_ask_sum(-7, 0, None, 1 << 24, 5 << 19) == 5
    assert oracle.readout_ask_sum(0, 1 << 23, 4 << 19, 1 << 23, 8 << 19) == 6
    assert oracle.readout_ask_sum(3, 1, (3 << 19) + (1 << 42), 0, None) == 4
    assert oracle.readout_ask_sum(-3, 0, None, 1, (-3 << 19) - (1 << 42)) == -4


# ---- f64 restatements of the float read (tests.rs:5710-5755) ---------------------------------

def f64_units(raw):
    g = np.asarray(raw, np.float64).reshape(-1, 4) * 2.0 ** -24
    r = np.sqrt((g * g).sum(1, keepdims=True))
    return np.where(r > 0, g / np.where(r > 0, r, 1.0), 0.0)


def f64_hamilton(a, b):
    a0, a1, a2, a3 = a.T
    b0, b1, b2, b3 = b.T
    return np.stack([a0 * b0 - a1 * b1 - a2 * b2 - a3 * b3,
                     a0 * b1 + a1 * b0 + a2 * b3 - a3 * b2,
                     a0 * b2 - a1 * b3 + a2 * b0 + a3 * b1,
                     a0 * b3 + a1 * b2 - a2 * b1 + a3 * b0], 1)


def f64_rotated(raw, point):
    return f64_hamilton(f64_units(raw), np.asarray(point, np.float64).reshape(-1, 4)).reshape(-1)


def f64_codes(raw, point, heads):
    rot = f64_rotated(raw, point)
    hw = rot.size // heads
    return [sum(1 << c for c in range(hw) if rot[h * hw + c] >= 0) for h in range(heads)]


def f64_weight(margin_q16, d):
    m = margin_q16 / 65536.0
    return max(m - d, 0.0) / max(m, 1.0)


def f64_nearest(query, keys, t, kept):
    """`nearest` (hamming.rs:690-701): positions 1 <= s < t by (distance, position)."""
    cand = sorted((bin(query ^ keys[s]).count("1"), s) for s in range(1, t))
    return [(s, d) for d, s in cand[:kept]]


def make(spec, seed, **ham):
    return synth.make_artifact(replace(spec, hamming=synth.HammingSpec(**ham)), seed)


def streams(seed, rows, vocab=12, n=3):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, rows).astype(np.uint32) for _ in range(n)]


def test_codes_match_f64_and_the_copy_read():
    art = make(BASE, 5, heads=4, depths=(1, 2), kept=8)
    table = art.writer_table.reshape(BASE.vocab, BASE.width)
    for r, read in enumerate(art.hamming_reads):
        codes = oracle.hamming_codes(art, r)
        for v in range(BASE.vocab):
            assert list(map(int, codes[v])) == f64_codes(read.key_rotation, table[v] / 4096.0, 4), (r, v)
        copy = oracle.copy_vocab_codes(read.key_rotation, table, 4, 2)
        assert np.array_equal(codes[:, :2], copy)


def copy_heads_of(art, read, rule_name):
    h = art.hamming
    codes = oracle.hamming_codes(art, art.hamming_reads.index(read))[:, : h.heads // 2]
    hw = art.spec.width // h.heads
    keys = h.copy_keys or (h.copy_key,) * (h.heads // 2)
    pair = np.array([(1 << (hw // 2)) - 1 if k == 2 else 0 for k in keys], np.uint64)
    table = art.writer_table.reshape(art.spec.vocab, art.spec.width)
    return Heads(codes, read.margin[: h.heads // 2], table, h.kept, rule_name, pair, h.copy_longest)


COPY_CASES = [
    ("mean", dict()),
    ("latest-exact", dict(copy_latest=True)),
    ("latest-nearest", dict(rule=2)),
    ("longest-exact", dict(rule=3, copy_keys=(1, 2))),
    ("longest-after-opening", dict(copy_latest=True, copy_longest=(3, 5))),
    ("longest-after-opening", dict(rule=4)),          # no marker: no row opens a reply
    ("mean", dict(copy_key=2, margin_bits=(6, 14))),
]


@pytest.mark.parametrize("case", range(len(COPY_CASES)))
def test_copy_heads_equal_the_copy_read(case):
    name, kw = COPY_CASES[case]
    art = make(BASE, 11 + case, heads=4, depths=(1, 2), kept=4, typed=False, **kw)
    d = BASE.width
    rng = np.random.default_rng(case)
    matched = 0
    for tokens in streams(case, 40, vocab=8):
        if name == "longest-after-opening":
            tokens[10:12] = (3, 5)
            tokens[25:27] = (3, 5)
        for read in art.hamming_reads:
            heads = copy_heads_of(art, read, name)
            rows = np.stack([np.where(np.arange(40) <= t, tokens, 0) for t in range(40)]).astype(np.uint32)
            c, found, _ = oracle.copy_mean_rows(heads, rows, np.arange(1, 41, dtype=np.int32))
            w_c = read.weight[:d]
            for t in range(40):
                window = tokens[: t + 1]
                if read.depth < BASE.layers:
                    x = rng.integers(-(1 << 19), 1 << 19, d).astype(np.int32)
                    got, _ = oracle.hamming_row(art, read.depth, window, x=x)
                    want = [oracle.stream_sum(int(x[k]), int(w_c[k]), int(c[t, k]), 0, 0) if found[t]
                            else int(x[k]) for k in range(d)]
                else:
                    n = rng.integers(-(1 << 39), 1 << 39, d).astype(np.int64)
                    got, _ = oracle.hamming_row(art, read.depth, window, n=n)
                    want = [oracle.readout_sum(int(n[k]), int(w_c[k]), int(c[t, k]) if found[t] else None, 0, 0)
                            for k in range(d)]
                assert list(map(int, got)) == want, (name, read.depth, t)
                matched += int(found[t])
    assert matched > 20, matched


@pytest.mark.parametrize("seed", range(7))
def test_type_heads_match_the_f64_reference(seed):
    """As tests.rs:5757-5856: seeds 0-1 narrow margins, 2-4 wide, 5-6 one type head wide."""
    art = make(BASE, 195 + seed, heads=4, depths=(1,), kept=16)
    d, rows, copy = BASE.width, 48, 2
    read = art.hamming_reads[0]
    if 2 <= seed <= 4:
        read.margin[:] = [((33 + 2 * k) << 16) + 12345 for k in range(4)]
    elif seed >= 5:
        read.margin[copy + seed - 5] = (37 << 16) + 12345
    read.weight[:d] = 0
    read.weight[d:] = 1 << 24
    table = art.writer_table.reshape(BASE.vocab, d)
    key = [f64_codes(read.key_rotation, table[v] / 4096.0, 4) for v in range(BASE.vocab)]
    rng = np.random.default_rng(seed + 7)
    tokens = rng.integers(0, 12, rows).astype(np.uint32)
    points = rng.integers(-(1 << 18), (1 << 18) + 1, (rows, d)).astype(np.int32)
    pay = None
    payload_ref = []
    found_rows = one_found = 0
    for t in range(rows):
        got, pay = oracle.hamming_row(art, 1, tokens[: t + 1], x=points[t], payloads=pay)
        real = points[t] / 65536.0
        payload_ref.append(f64_rotated(read.value_rotation, real))
        off = np.abs(pay[0, t] - payload_ref[t] * 65536.0)
        assert off.max() <= 0.5 + 2.0 ** -10, (seed, t, off.max())
        queries = f64_codes(read.query_rotation, real, 4)
        total, found = np.zeros(d), 0
        for j in range(2):
            kept = f64_nearest(queries[copy + j], [0] + [key[tokens[s - 1]][copy + j] for s in range(1, t)], t, 16)
            head, count = np.zeros(d), 0
            for s, dist in kept:
                w = f64_weight(int(read.margin[copy + j]), dist)
                if w > 0:
                    count += 1
                    head += w * payload_ref[s]
            if count:
                found += 1
                total += head / count
        if found == 0:
            assert np.array_equal(got, points[t]), (seed, t)
            continue
        found_rows += 1
        one_found += found == 1
        want = points[t] + 65536.0 * total / found
        assert np.abs(got - want).max() <= 1.5, (seed, t, np.abs(got - want).max())
    if seed >= 2:
        assert found_rows > 20, found_rows
    if seed >= 5:
        assert one_found >= 3, one_found


@pytest.mark.parametrize("zero", [False, True])
def test_asking_reads_match_the_f64_reference(zero):
    """As tests.rs:8380-8470, with the readout read's question carry (hamming.rs:1161-1181):
    the stream read at depth 1 and the readout at depth 2, within 0.6 of a step."""
    art = make(BASE, 353, heads=4, depths=(1, 2), kept=16, asks=(True, True), carry_rows=3,
               margin_bits=(20, 40))
    d, copy = BASE.width, 2
    table = art.writer_table.reshape(BASE.vocab, d).astype(np.int64)
    if zero:
        for read in art.hamming_reads:
            read.ask[:] = 0
    rng = np.random.default_rng(353)
    tokens = np.array([(t * 7) % 5 + (t // 11) % 3 for t in range(40)], np.uint32)
    found = [0, 0]
    for r, read in enumerate(art.hamming_reads):
        ask = table + read.ask.reshape(BASE.vocab, d)
        key = [f64_codes(read.key_rotation, table[v] / 4096.0, 4) for v in range(BASE.vocab)]
        heads = copy_heads_of(art, read, "mean")
        w_c = read.weight[:d] * 2.0 ** -24
        w_y = read.weight[d:] * 2.0 ** -24
        for t in range(1, len(tokens)):
            window = tokens[: t + 1]
            point = ask[window[t]] * 65536
            if read.carry is not None:
                for s in range(1, min(3, t) + 1):
                    point = point + int(read.carry[window[t - s]]) * ask[window[t - s]]
            queries = f64_codes(read.key_rotation, point.astype(np.float64), 4)
            total, finders = np.zeros(d), 0
            for j in range(2):
                kept = f64_nearest(queries[copy + j], [0] + [key[window[s - 1]][copy + j] for s in range(1, t)], t, 16)
                head, count = np.zeros(d), 0
                for s, dist in kept:
                    w = f64_weight(int(read.margin[copy + j]), dist)
                    if w > 0:
                        count += 1
                        head += w * table[window[s]] / 4096.0
                if count:
                    finders += 1
                    total += head / count
            y = total / finders if finders else None
            found[r] += y is not None
            c_int, c_found, _ = oracle.copy_mean_rows(heads, window[None, :], np.array([t + 1], np.int32))
            c = c_int[0] * 2.0 ** -43 if c_found[0] else None
            if read.depth == 1:
                x = rng.integers(-(1 << 19), 1 << 19, d).astype(np.int32)
                got, pay = oracle.hamming_row(art, 1, window, x=x)
                added = (w_c * c if c is not None else 0.0) + (w_y * y if y is not None else 0.0)
                want = x + 65536.0 * added
            else:
                unit = 2.0 ** -24
                n = rng.integers(-(1 << 39), 1 << 39, d).astype(np.int64)
                got, pay = oracle.hamming_row(art, 2, window, n=n)
                nf = n * unit
                moved = lambda w, m: 0.0 if m is None else w * (m - nf)  # noqa: E731
                want = (nf + moved(w_c, c) + moved(w_y, y)) / unit
            assert np.abs(got.astype(np.float64) - want).max() <= 0.6, (zero, read.depth, t)
            assert pay.size == 0, "an asking read keeps no payloads"
    assert found[0] > 0 and found[1] > 0, found


def test_zero_weights_reduce_to_the_read_free_model():
    spec = replace(BASE, layers=3)
    art = make(spec, 21, heads=4, depths=(1, 2, 3), kept=8, asks=(False, True, False))
    for read in art.hamming_reads:
        read.weight[:] = 0
    free = replace(art, hamming=None, hamming_reads=None)
    prompts = synth.uniform_prompts(spec.vocab, 3, 12, 4)
    a = oracle.decode(art, prompts, 20)
    b = oracle.decode(free, prompts, 20)
    for k in ("reply", "state", "history", "position"):
        assert np.array_equal(a[k], b[k]), k


STREAM_CASES = [
    dict(heads=4, depths=(1, 3), kept=8),
    dict(heads=8, depths=(2, 3), kept=4, asks=(False, True), carry_rows=2, copy_latest=True),
    dict(heads=4, depths=(1, 2, 3), kept=16, copy_keys=(2, 1), rule=2),
]


@pytest.mark.parametrize("case", range(len(STREAM_CASES)))
def test_the_reads_move_the_decode_and_a_resumed_stream_continues_it(case):
    spec = replace(BASE, layers=3, context=48)
    art = make(spec, 40 + case, **STREAM_CASES[case])
    free = replace(art, hamming=None, hamming_reads=None)
    prompts = synth.uniform_prompts(spec.vocab, 3, 10, 9 + case) % 16  # repeats for the heads
    whole = oracle.decode_stream(art, prompts, 30)
    assert whole["status"] == 0
    assert not np.array_equal(whole["reply"], oracle.decode(free, prompts, 30)["reply"])
    plain = oracle.decode(art, prompts, 30)
    assert np.array_equal(plain["reply"], whole["reply"])
    assert np.array_equal(whole["tokens"][:, :40], np.concatenate([prompts, whole["reply"][:, :30]], 1))
    first = oracle.decode_stream(art, prompts, 14)
    resumed = oracle.decode_stream(art, first["reply"][:, -1:], 15, resume=first)
    assert np.array_equal(resumed["reply"], whole["reply"][:, 15:])
    for k in ("state", "history", "position", "tokens", "payloads"):
        assert np.array_equal(resumed[k], whole[k]), k
    # Teacher-forced rows of the same tokens choose what the decode chose.
    rows = np.concatenate([prompts, whole["reply"][:, :30]], 1)
    st, tok, _, _ = oracle.sequences(art, rows)
    assert st == 0
    assert np.array_equal(tok[:, 9:], whole["reply"])


def test_the_context_slide_continues_as_an_unbounded_context():
    """set_context_slide (session.rs:2391-2402, :4143-4151): a full context continues; nothing
    else in the step reads the position past its ring slot, so the slid decode equals the decode
    of the same weights with a context that never fills. Without the slide the step refuses at
    the bound (status 2), and a model with Hamming reads refuses the slide (can_slide_tokens,
    :1146-1151)."""
    small = synth.make_artifact(replace(BASE, context=16, window=5), 61)
    big = replace(small, spec=replace(small.spec, context=200))
    prompts = synth.uniform_prompts(BASE.vocab, 3, 9, 62)
    slid = oracle.decode(small, prompts, 40, slide=True)
    assert slid["status"] == 0
    want = oracle.decode(big, prompts, 40)
    for k in ("reply", "state", "history", "position"):
        assert np.array_equal(slid[k], want[k]), k
    assert int(slid["position"][0]) == 9 + 40 > 16
    assert oracle.decode(small, prompts, 40)["status"] == 2
    ham = make(BASE, 63, heads=4, depths=(1,), kept=4)
    assert oracle.decode(ham, prompts, 4, slide=True)["status"] == 4


# ---- exact cases of the type and ask heads (hamming.rs:1204-1334) ---------------------------
#
# Rotations whose unit quaternions are exact at Q31 (stack_rotation of (c, 0, 0, 0) is the
# identity 2^31, of (0, c, 0, 0) the unit i, of (c, c, c, c) 2^30 on every coordinate), key and
# query rotations that leave a point's sign code as the signs of its coordinates, and table rows
# whose codes sit at chosen distances: every quantity below follows from the quaternion units'
# multiplication table and the definitions of the weight, the means and the rounding.

ONE = 1 << 24  # a raw rotation coordinate of 1.0 at 2^-24
HW = BASE.width // 4  # coordinates a head covers (4 heads)


def exact_read(seed, kept, margins, value_raw=(ONE, 0, 0, 0), asks=None):
    art = make(BASE, seed, heads=4, depths=(1,), kept=kept, asks=asks)
    read = art.hamming_reads[0]
    d = BASE.width
    ident = np.tile(np.array([ONE, 0, 0, 0], np.int32), d // 4)
    read.key_rotation[:] = ident
    read.query_rotation[:] = ident
    read.value_rotation[:] = np.tile(np.asarray(value_raw, np.int32), d // 4)
    read.weight[:d] = 0          # no copy term: the hook moves by the type (or ask) mean alone
    read.weight[d:] = ONE
    read.margin[:] = margins
    if read.ask is not None:
        read.ask[:] = 0
    return art, read


def weight_q31(margin, dist):
    """copy_weight_q31 (hamming.rs:243-251) by its definition."""
    over = margin - (dist << 16)
    return 0 if over <= 0 else (over << 31) // max(margin, 1 << 16)


def half_away(n, shift):
    """round_shift (hamming.rs:1354-1361): n / 2^shift rounded half away from zero."""
    q = (abs(n) + (1 << (shift - 1))) >> shift
    return q if n >= 0 else -q


def trunc_div(a, b):
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b > 0) else -q


def set_row(art, token, signs):
    """Table row of `token`: magnitude 1000 with the given signs (64 of them)."""
    table = art.writer_table.reshape(BASE.vocab, BASE.width)
    table[token] = np.where(np.asarray(signs) >= 0, 1000, -1000).astype(table.dtype)


def head_signs(pattern2, pattern3):
    """Signs for a row or point: copy heads' coordinates positive, type heads' as given."""
    s = np.ones(BASE.width, np.int64)
    s[2 * HW:3 * HW] = pattern2
    s[3 * HW:] = pattern3
    return s


PERMUTED = {
    # u (x) (a, b, c, d) for the units 1, -1, i, j, k (the Hamilton product's table)
    "identity": ((ONE, 0, 0, 0), lambda a, b, c, d: (a, b, c, d)),
    "minus": ((-ONE, 0, 0, 0), lambda a, b, c, d: (-a, -b, -c, -d)),
    "i": ((0, ONE, 0, 0), lambda a, b, c, d: (-b, a, -d, c)),
    "j": ((0, 0, ONE, 0), lambda a, b, c, d: (-c, d, a, -b)),
    "k": ((0, 0, 0, ONE), lambda a, b, c, d: (-d, -c, b, a)),
}


@pytest.mark.parametrize("name", sorted(PERMUTED) + ["half"])
def test_type_payloads_under_exact_rotations(name):
    # TypeHeads::payload (hamming.rs:1204-1218): round_shift(u (x) p, 31). Under 1, -1, i, j, k
    # the payload is the point permuted and negated exactly; under the half unit (2^30 on each
    # coordinate) it is each signed sum of the four coordinates halved, an odd one rounded away
    # from zero (a negative odd sum fixes the direction against rounding half up).
    raw = (ONE, ONE, ONE, ONE) if name == "half" else PERMUTED[name][0]
    art, read = exact_read(7, 4, [1 << 16] * 4, value_raw=raw)
    rng = np.random.default_rng(11)
    rows = 24
    tokens = rng.integers(0, 12, rows).astype(np.uint32)
    points = rng.integers(-(1 << 20), 1 << 20, (rows, BASE.width)).astype(np.int32)
    pay = None
    odd_negative = 0
    for t in range(rows):
        _, pay = oracle.hamming_row(art, 1, tokens[: t + 1], x=points[t], payloads=pay)
        p = points[t].astype(np.int64).reshape(-1, 4)
        if name == "half":
            a, b, c, d = p.T
            sums = [a - b - c - d, a + b - c + d, a + b + c - d, a - b + c + d]
            want = np.stack([[half_away(int(v) << 30, 31) for v in s] for s in sums], 1)
            odd_negative += sum(int(((s < 0) & (s % 2 != 0)).sum()) for s in sums)
        else:
            want = np.stack(PERMUTED[name][1](*p.T), 1)
        assert np.array_equal(pay[0, t].reshape(-1, 4), want), (name, t)
    if name == "half":
        assert odd_negative > 100


def run_exact(art, read, tokens, point):
    """The hook's output at the last row of `tokens` for the stream input `point`, with every
    earlier row's payload formed by the oracle at its own row (points: the rows' inputs)."""
    pay = None
    for t in range(len(tokens)):
        got, pay = oracle.hamming_row(art, 1, tokens[: t + 1], x=point[t], payloads=pay)
    return got


def test_one_type_head_keeping_one_position_moves_by_its_weighted_payload():
    # One type head finds one position (kept 1) at distance 1 inside a margin with a fraction,
    # the other finds none (distance 8 against a margin of 2 bits): the mean is w v exactly, and
    # the stream moves by it through stream_sum (pinned by the reference's literal answers).
    A, B = 3, 4
    m2 = (3 << 16) + 12345
    art, read = exact_read(8, 1, [1 << 16, 1 << 16, m2, 2 << 16])
    one_off = np.ones(HW, np.int64)
    one_off[5] = -1
    set_row(art, A, head_signs(one_off, np.ones(HW)))      # head 2 code: one bit off all-ones
    set_row(art, B, head_signs(-np.ones(HW), -np.ones(HW)))
    tokens = np.array([A, B, B, B, A, B], np.uint32)       # position 1's key is A's row
    rng = np.random.default_rng(12)
    pts = rng.integers(-(1 << 20), 1 << 20, (len(tokens), BASE.width)).astype(np.int64)
    mixed = np.array([1, -1] * (HW // 2))
    last = head_signs(np.ones(HW), mixed) * np.abs(pts[-1]) + head_signs(np.ones(HW), mixed)
    pts[-1] = last
    got = run_exact(art, read, tokens, pts.astype(np.int32))
    # positions 1..4: keys A, B, B, B -> distances 1, 16, 16, 16 for head 2; the query of head 3
    # (alternating signs) is 8 from both A's and B's codes.
    w = weight_q31(m2, 1)
    assert 0 < w < 1 << 31
    y = [w * int(v) for v in pts[1]]                        # payload of position 1 = its point
    want = [oracle.stream_sum(int(last[k]), 0, 0, ONE, y[k]) for k in range(BASE.width)]
    assert list(map(int, got)) == want


def half_step_pair(w2, k=3):
    """Payload values v1, v2 with 2^31 v1 + w2 v2 = -(2 k + 1) 2^31 + 1 (w2 odd): the sum is odd
    and negative, and half of it lies a half step inside -(k + 1/2) 2^31, so the two ways of
    rounding the halving (toward zero, or down) move the hook's Q16 output differently."""
    m = 1 << 31
    v2 = pow(w2, -1, m)                       # w2 v2 = 1 + j 2^31
    j = (w2 * v2 - 1) >> 31
    v1 = -(2 * k + 1) - j
    assert 2**31 * v1 + w2 * v2 == -(2 * k + 1) * 2**31 + 1 and abs(v1) < 2**31 and v2 < 2**31
    return v1, v2


def odd_weight_margin(dist):
    for m in range((4 << 16) + 1, (5 << 16)):
        if weight_q31(m, dist) % 2 == 1:
            return m
    raise AssertionError


@pytest.mark.parametrize("split", ["within_a_head", "across_heads"])
def test_type_means_truncate_toward_zero(split):
    # TypeHeads::mean_by (hamming.rs:1282-1334) halves twice: a head's sum by its count of kept
    # positions, and the heads' total by the heads that found one, both truncating toward zero.
    # Either the head with two kept positions (distances 0 and 1) or two heads each keeping one
    # carry the sum 2^31 v1 + w v2 = -(2 k + 1) 2^31 + 1 on coordinate 0, whose half rounds to
    # the hook's output one way if truncated and another if floored.
    A, C2, B = 3, 5, 4
    m = odd_weight_margin(1)
    w0, w1 = weight_q31(m, 0), weight_q31(m, 1)
    assert w0 == 1 << 31 and w1 % 2 == 1
    mixed = np.array([1, -1] * (HW // 2))
    off1 = np.ones(HW, np.int64)
    off1[2] = -1
    if split == "within_a_head":
        kept, margins = 2, [1 << 16, 1 << 16, m, 2 << 16]   # head 3 finds nothing
        row_a = head_signs(np.ones(HW), np.ones(HW))         # head 2: distance 0
        row_c = head_signs(off1, np.ones(HW))                # head 2: distance 1
        last = head_signs(np.ones(HW), mixed)
    else:
        kept, margins = 1, [1 << 16, 1 << 16, m, m]
        row_a = head_signs(np.ones(HW), -np.ones(HW))        # head 2: 0, head 3: 16 (far)
        row_c = head_signs(-np.ones(HW), off1)               # head 2: 16, head 3: 1
        last = head_signs(np.ones(HW), np.ones(HW))
    art, read = exact_read(9, kept, margins)
    set_row(art, A, row_a)
    set_row(art, C2, row_c)
    set_row(art, B, head_signs(-np.ones(HW), -np.ones(HW)))  # 8 or 16 from every query
    tokens = np.array([A, C2, B, B, B, B, A], np.uint32)   # keys of positions 1, 2: A, C2
    rng = np.random.default_rng(13)
    pts = rng.integers(-(1 << 20), 1 << 20, (len(tokens), BASE.width)).astype(np.int64)
    v1, v2 = half_step_pair(w1)
    pts[1][0], pts[2][0] = v1, v2
    pts[-1] = last * (np.abs(pts[-1]) + 1)
    pts[-1][0] = -5          # a negative sum: its rounding goes away from zero (down)
    got = run_exact(art, read, tokens, pts.astype(np.int32))
    total = [w0 * int(pts[1][k]) + w1 * int(pts[2][k]) for k in range(BASE.width)]
    # One head with two positions: total / 2, then / 1; two heads with one position each:
    # (v / 1 + v' / 1) / 2. Either way the halving of the total.
    y = [trunc_div(v, 2) for v in total]
    want = [oracle.stream_sum(int(pts[-1][k]), 0, 0, ONE, y[k]) for k in range(BASE.width)]
    floored = oracle.stream_sum(int(pts[-1][0]), 0, 0, ONE, total[0] // 2)
    assert floored != want[0]                               # the case tells the two apart
    assert list(map(int, got)) == want


def test_an_ask_head_brings_back_the_kept_token_point_exactly():
    # An asking read (hamming.rs:1149-1181, mean_by over Brought::Points): the question is the
    # code of (table + a)[x_t] (a = 0, no carry) through the key rotation; one ask head keeps
    # the position whose key (the row before it) is one bit off, and brings back the table row
    # of that position's own token times the weight; the stream raises it by 4 bits to the type
    # term's exponent (hamming.rs:1849-1855).
    A, B, P = 3, 4, 6
    m2 = (3 << 16) + 4321
    art, read = exact_read(10, 1, [1 << 16, 1 << 16, m2, 2 << 16], asks=(True,))
    assert read.ask is not None
    one_off = np.ones(HW, np.int64)
    one_off[7] = -1
    mixed = np.array([1, -1] * (HW // 2))
    set_row(art, A, head_signs(one_off, np.ones(HW)))
    set_row(art, B, head_signs(-np.ones(HW), -np.ones(HW)))
    set_row(art, P, head_signs(np.ones(HW), mixed))       # the asking token: head 2 all ones
    table = art.writer_table.reshape(BASE.vocab, BASE.width)
    rng = np.random.default_rng(14)
    table[B] = (table[B] * rng.integers(1, 30, BASE.width)).astype(table.dtype)  # varied values
    tokens = np.array([A, B, B, B, P], np.uint32)          # position 1 (key A) holds token B
    x = rng.integers(-(1 << 20), 1 << 20, BASE.width).astype(np.int32)
    got, pay = oracle.hamming_row(art, 1, tokens, x=x)
    assert pay.size == 0
    w = weight_q31(m2, 1)
    y = [(w * int(v)) << 4 for v in table[B]]
    want = [oracle.stream_sum(int(x[k]), 0, 0, ONE, y[k]) for k in range(BASE.width)]
    assert list(map(int, got)) == want
