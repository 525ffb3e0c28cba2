"""The reference's copy-rule tests (crates/uor-r4-integer/src/stack/hamming.rs:705-1058) with
their literal expectations, over any implementation of the read: `make(kept, rule, codes=...,
pair=..., marker=...)` returns an object with `mean(tokens)`, `mean_at(tokens, opening)` and
`choose_ruled(h, tokens, opening)`. Shared by the oracle tests (CPU) and the HIP tests (GPU)."""

import numpy as np

from uor_fbs.copy import Heads

FULL = 1 << 31
CODES = [0b0000, 0b1111, 0b0011, 0b0001]


def heads(kept, rule, codes=None, pair=None, marker=None):
    """One copy head on copy key 1 over a vocabulary of 4, 4-bit codes, a 4-bit margin, and the
    table whose row v is [10 v + 1; 4] (hamming.rs:719-733)."""
    return Heads(np.array(codes or CODES, np.uint64).reshape(4, 1), np.array([4 << 16], np.int32),
                 np.array([[10 * v + 1] * 4 for v in range(4)], np.int16), kept, rule,
                 None if pair is None else np.array([pair], np.uint64), marker)


def row(v, w):
    return [(10 * v + 1) * w] * 4


def check_rust_tests(make):
    # candidates_include_the_immediate_predecessor_and_exclude_the_current_row (:705-711)
    assert make(16, "mean", codes=[0, 0, 0, 0]).choose_ruled(0, [0, 0, 0, 0, 0]) == [(1, 0), (2, 0), (3, 0)]
    # two_exact_matches_blend_under_the_mean_and_the_latest_rules_take_the_last (:822-835)
    tokens = [1, 2, 0, 1, 3, 0, 1]
    assert make(16, "mean").mean(tokens) == [211 * (1 << 27)] * 4
    for rule in ("latest-exact", "latest-nearest"):
        assert make(16, rule).mean(tokens) == row(3, FULL), rule
    # without_an_exact_match_only_the_nearest_rule_reads (:837-848)
    tokens = [2, 0, 2, 3, 1]
    assert make(16, "mean").mean(tokens) == [16 * (1 << 30)] * 4
    assert make(16, "latest-exact").mean(tokens) is None
    assert make(16, "latest-nearest").mean(tokens) == row(3, 1 << 30)
    # the_latest_match_is_found_past_the_kept_count (:850-863)
    tokens = [1, 0, 1, 2, 1, 3, 1]
    mean2 = make(2, "mean")
    assert mean2.choose_ruled(0, tokens) == [(1, 0), (3, 0)]
    assert mean2.mean(tokens) == row(1, FULL)
    for rule in ("latest-exact", "latest-nearest"):
        assert make(2, rule).mean(tokens) == row(3, FULL), rule
    # the_longest_rule_takes_the_match_of_two_tokens_before_a_later_match_of_one (:865-875)
    tokens = [2, 1, 3, 0, 1, 2, 2, 1]
    latest, longest = make(16, "latest-exact"), make(16, "longest-exact")
    assert latest.mean(tokens) == row(2, FULL)
    assert longest.choose_ruled(0, tokens) == [(2, 0)]
    assert longest.mean(tokens) == row(3, FULL)
    # the_longest_rule_takes_the_latest_of_its_longer_matches (:877-887)
    tokens = [2, 1, 3, 2, 1, 0, 0, 1, 2, 2, 1]
    assert latest.mean(tokens) == row(2, FULL)
    assert longest.choose_ruled(0, tokens) == [(5, 0)]
    assert longest.mean(tokens) == row(0, FULL)
    # the_longest_rule_falls_back_to_the_latest_exact_match (:889-904)
    one = [0, 1, 3, 0, 1, 2, 2, 1]
    assert longest.choose_ruled(0, one) == [(5, 0)]
    assert longest.mean(one) == latest.mean(one)
    assert longest.mean([2, 0, 2, 3, 1]) is None
    first = [1, 3, 0, 1]
    assert longest.choose_ruled(0, first) == [(1, 0)]
    assert longest.mean(first) == row(3, FULL)
    # under_copy_key_two_the_longer_match_is_of_three_tokens (:906-923)
    tokens = [0, 1, 3, 2, 2, 1, 3, 0, 0, 1, 3]
    assert make(16, "latest-exact", pair=0b0011).choose_ruled(0, tokens) == [(7, 0)]
    lp = make(16, "longest-exact", pair=0b0011)
    assert lp.choose_ruled(0, tokens) == [(3, 0)]
    assert lp.mean(tokens) == row(2, FULL)
    assert lp.choose_ruled(0, [1, 3, 0, 1, 3]) == [(2, 0)]
    # the_longer_match_is_by_the_heads_code (:925-937)
    tokens = [3, 1, 0, 0, 1, 3, 2, 1]
    assert longest.choose_ruled(0, tokens) == [(5, 0)]
    edited = make(16, "longest-exact", codes=[CODES[0], CODES[1], CODES[2], CODES[2]])
    assert edited.choose_ruled(0, tokens) == [(2, 0)]
    assert edited.mean(tokens) == row(0, FULL)
    # the_marker_names_the_opening_row_in_place_of_the_caller (:939-960)
    tokens = [2, 1, 3, 0, 1, 2, 2, 1]
    m21 = make(16, "longest-after-opening", marker=(2, 1))
    m31 = make(16, "longest-after-opening", marker=(3, 1))
    for caller in (False, True):
        assert m21.choose_ruled(0, tokens, caller) == [(5, 0)]
        assert m21.mean_at(tokens, caller) == row(2, FULL)
        assert m31.choose_ruled(0, tokens, caller) == [(2, 0)]
        assert m31.mean_at(tokens, caller) == row(3, FULL)
    assert m21.mean(tokens) == row(2, FULL)
    # the_longest_after_opening_rule_is_latest_at_the_opening_and_longest_elsewhere (:962-977)
    spared = make(16, "longest-after-opening")
    assert spared.choose_ruled(0, tokens, True) == [(5, 0)] == latest.choose_ruled(0, tokens)
    assert spared.mean_at(tokens, True) == row(2, FULL)
    assert spared.choose_ruled(0, tokens, False) == [(2, 0)] == longest.choose_ruled(0, tokens)
    assert spared.mean_at(tokens, False) == row(3, FULL) == spared.mean(tokens)
    # the_opening_moves_no_other_rule (:979-989)
    for rule in ("mean", "latest-exact", "latest-nearest", "longest-exact"):
        h = make(16, rule)
        assert h.choose_ruled(0, tokens, True) == h.choose_ruled(0, tokens, False), rule
        assert h.mean_at(tokens, True) == h.mean(tokens), rule
    # a_row_with_no_earlier_position_reads_nothing (:1029-1045)
    for rule in ("latest-exact", "latest-nearest", "longest-exact", "longest-after-opening"):
        h = make(16, rule)
        assert h.mean_at([1, 1], True) is None
        assert h.mean([1]) is None and h.mean([1, 1]) is None and h.mean([]) is None


def random_heads(seed, vocab=300, width=96, copy=4, kept=8, rule="mean", bits=12):
    """Heads with few distinct codes (so that exact and near matches are common), margins of
    2-12 bits, copy key 2 on odd heads, and a marker on the longest-after-opening rule."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, (vocab, copy)).astype(np.uint64)
    codes |= rng.integers(0, 2, (vocab, copy)).astype(np.uint64) << np.uint64(63)
    margins = (rng.integers(2, 13, copy) << 16).astype(np.int32)
    margins[0] = 3 << 16 | 12345            # a margin off the bit grid
    pair = np.array([0 if h % 2 == 0 else (1 << (bits // 2)) - 1 for h in range(copy)], np.uint64)
    table = rng.integers(-32768, 32768, (vocab, width)).astype(np.int16)
    marker = (int(rng.integers(0, vocab)), int(rng.integers(0, vocab))) if rule == "longest-after-opening" and seed % 2 else None
    return Heads(codes, margins, table, kept, rule, pair, marker)


def random_streams(seed, vocab, rows, stride, small_vocab=24):
    """Streams of lengths 0..stride over a small part of the vocabulary (repeats are common)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, stride + 1, rows).astype(np.int32)
    lens[:4] = [0, 1, 2, stride]
    tok = rng.integers(0, min(vocab, small_vocab), (rows, stride)).astype(np.uint32)
    tok = np.where(np.arange(stride)[None, :] < lens[:, None], tok, 0).astype(np.uint32)
    return tok, lens, rng.integers(0, 2, rows).astype(np.uint8)
