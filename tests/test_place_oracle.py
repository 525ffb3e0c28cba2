"""The place read in the oracle (oracle/fbs_oracle.c's place register, place_find and place_pick,
and the readout's offer), pinned by the reference's own tests of it: every case of
fbs_snapshot.rs's place_tests (:3136-3370) run through the same register with the same injected
finds, the marks check, the pick's ties and margins, the container's round trip and refusals
(stack/tests.rs:8800-8880), and a session that serves the place read (stack/tests.rs:8882-8930)
on a seeded artifact built as the reference's place trunk is: the readout's question table moves
the asking token's point onto the stated token's, so the question finds the place after it.
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from test_uorlut import _build, _split, fixture, MANIFEST
from uor_fbs import synth, uorlut
from uor_fbs.synth import PLACE_ARM, PLACE_OPEN, PLACE_STOP, PlaceMarks

# The place_tests' image (fbs_snapshot.rs:3142-3158).
BOS, EOS, SEP, USER, MODEL = 0, 1, 2, 4, 5
IS, DOT, ASK = 10, 13, 15
MARKS = PlaceMarks(bos=BOS, eos=EOS, sep=(SEP,), system=(3,), user=(USER,), assistant=(MODEL,))
CLASS = np.zeros(20, np.int16)
CLASS[DOT] = PLACE_STOP
CLASS[14] = PLACE_STOP
CLASS[ASK] = PLACE_ARM
CLASS[IS] = PLACE_STOP | PLACE_OPEN
# "<u> name is V1 V2 . </s> <sep> <m> ok </s> <sep> <u> what ? <sep> <m> is V1 V2 ."
TALK = [BOS, USER, 9, IS, 11, 12, DOT, EOS, SEP, MODEL, 16, EOS, SEP, USER, 14, ASK, SEP, MODEL,
        IS, 11, 12, DOT]
DEFAULT = (None, None, False, None)


def rows(tokens, at, pos, more=()):
    """Each row as (held, offer, stepped, asked): asked is (content range, finds) or None (with
    `more` finds, the asked finds' count and the last of them)."""
    out = []
    for held, offer, stepped, a, b, n, fa, fp in oracle.place_rows(MARKS, CLASS, tokens,
                                                                  [(at, pos), *more]):
        assert n <= 1 or more
        asked = None if a < 0 else (range(a, b), [(int(fa), int(fp))] * int(n) if n <= 1 else (int(n), int(fa), int(fp)))
        out.append((None if held < 0 else int(held), None if offer < 0 else int(offer),
                    bool(stepped), asked))
    return out


def test_the_turns_are_cut_before_the_separator_and_the_end_mark():
    r = rows(TALK, -1, 0)
    # The first user turn loses its end mark and its separator; the second has no end mark.
    assert r[9][3] == (range(2, 7), [])
    assert r[17][3] == (range(14, 16), [])
    assert sum(x[3] is not None for x in r) == 2
    # The start mark forgets the document: a reply after it has no user turn to answer.
    again = rows(TALK + [BOS, MODEL, 16], -1, 0)
    assert all(x[3] is None for x in again[22:])


def test_a_marker_inside_a_turn_is_not_a_turn():
    tokens = [BOS, USER, 9, USER, 9, SEP, MODEL]
    r = rows(tokens, -1, 0)
    assert r[6][3] == (range(2, 5), [])
    assert all(x[3] is None for x in r[:6])


def test_the_register_is_armed_opened_stepped_and_stopped():
    r = rows(TALK, 15, 4)
    assert r[17][3] == (range(14, 16), [(15, 4)])
    assert (r[17][0], r[17][1]) == (4, None)
    assert r[18][:3] == (4, 4, False)
    assert r[19][:3] == (5, 5, True)
    assert r[20][:3] == (None, None, False)
    assert r[21] == DEFAULT
    assert all(x[0] is None and x[1] is None for x in r[:17])
    assert r[9][3] == (range(2, 7), [])
    assert sum(x[3] is not None for x in r) == 2


def test_a_miss_closes_its_row_only_and_the_end_mark_ends_the_reply():
    tokens = TALK[:18] + [IS, 16, IS, 11, EOS, SEP]
    r = rows(tokens, 15, 4)
    assert (r[18][1], r[19][1], r[19][0]) == (4, None, 4)
    assert not r[19][2]
    assert (r[20][1], r[21][1], r[21][2]) == (4, 5, True)
    assert r[22] == DEFAULT
    assert r[23] == DEFAULT


def test_a_row_arms_only_by_its_token_and_only_inside_the_question():
    for at in (14, 16):
        r = rows(TALK, at, 4)
        assert r[17][3] == (range(14, 16), [(14, 4)] if at == 14 else [])
        assert all(x[0] is None and x[1] is None for x in r)
    # A find outside every finished user turn sets nothing.
    assert all(x[0] is None for x in rows(TALK, 15, 10))


def test_a_step_onto_the_end_of_the_places_turn_stops_the_read():
    tokens = [BOS, USER, 9, IS, 11, 12, EOS, SEP, MODEL, 16, EOS, SEP, USER, 14, ASK, SEP, MODEL,
              IS, 11, 12, 16]
    r = rows(tokens, 14, 4)
    assert r[16][3] == (range(13, 15), [(14, 4)])
    assert (r[17][1], r[18][1], r[18][2]) == (4, 5, True)
    assert r[19][:3] == (None, None, False)
    assert r[20] == DEFAULT


def test_a_reply_answers_the_latest_user_turn_once():
    twice = rows(TALK + [EOS, SEP, MODEL, IS, 11], 15, 4)
    assert twice[17][3] == (range(14, 16), [(15, 4)])
    assert all(x == DEFAULT for x in twice[22:])
    # A system turn between the question and its reply changes nothing: the reply asks.
    lined = rows(TALK[:16] + [SEP, 3, 9, SEP, MODEL, IS, 11], 15, 4)
    assert lined[20][3] == (range(14, 16), [(15, 4)])
    assert (lined[20][0], lined[21][1], lined[22][1]) == (4, 4, 5)


def test_the_last_arming_row_of_the_question_sets_the_register():
    # "A row of a user turn's content records the place its question finds ... the last recorded
    # row whose token has PLACE_ARM sets the register to its find" (PlaceState, :2885-2891): two
    # arming rows, the later finding place 5; then a later non-arming find changes nothing.
    tokens = TALK[:16] + [ASK, 16, SEP, MODEL, IS, 12, DOT]
    r = rows(tokens, 15, 4, more=[(16, 5), (17, 3)])
    assert r[19][3] == (range(14, 18), (3, 17, 3))
    assert (r[19][0], r[20][1], r[21][1]) == (5, 5, None)
    assert r[21][2] is False


def test_a_user_turn_clears_the_register():
    r = rows(TALK[:18] + [16, SEP, USER, 14, SEP, MODEL, IS], 15, 4)
    assert (r[18][0], r[19][0]) == (4, 4)
    assert all(x[0] is None and x[1] is None for x in r[20:])


def test_marks_the_turn_reader_cannot_tell_apart_are_refused():
    good = MARKS
    assert good.check(20) is None
    assert good.check(5) is not None  # the assistant marker is outside a vocabulary of 5
    for bad in (replace(good, sep=()), replace(good, user=()), replace(good, assistant=()),
                replace(good, eos=good.bos), replace(good, assistant=good.user),
                replace(good, assistant=(7, USER)), replace(good, system=(7, MODEL))):
        assert bad.check(20) is not None, bad
    # Markers that share only their last token are told apart; the system marker may be empty.
    assert replace(good, user=(7, 8), assistant=(6, 8)).check(20) is None
    assert replace(good, system=()).check(20) is None


def test_the_pick_is_the_nearest_key_the_later_on_ties_inside_the_margin():
    keys = [0b1111, 0b0001, 0b0011, 0b0001, 0b0111]
    one = 1 << 16
    assert oracle.place_pick([0b0001], [one], [(1, 5)], keys) == 3
    assert oracle.place_pick([0b0001], [one], [(0, 2)], keys) is None
    assert oracle.place_pick([0b0011], [2 * one], [(2, 3), (4, 5)], keys) == 2
    assert oracle.place_pick([0b0110], [one], [(1, 5)], keys) is None
    assert oracle.place_pick([0b0110], [2 * one], [(1, 5)], keys) == 4
    assert oracle.place_pick([0b0101], [2 * one], [(3, 5)], keys) == 4
    assert oracle.place_pick([0b0001, 0b0011], [one, one], [(0, 5)], keys) == 3
    assert oracle.place_pick([0b0011, 0b1111], [one, one], [(0, 5)], keys) == 2
    assert oracle.place_pick([0b0001], [one], [], keys) is None


# ---- A session that serves the place read (stack/tests.rs:8750-8930) ----------------------

P_BOS, P_EOS, P_SEP, P_USER, P_MODEL = 500, 501, 502, 504, 505
P_BEFORE, P_ASK, P_OPENS, P_DOT = 21, 50, 60, 32
P_TALK = [P_BOS, P_USER, 20, P_BEFORE, 30, 31, P_DOT, P_EOS, P_SEP, P_MODEL, 40, P_EOS, P_SEP,
          P_USER, 20, P_ASK, P_SEP, P_MODEL, P_OPENS, 30, 31, P_DOT]
P_MARKS = PlaceMarks(bos=P_BOS, eos=P_EOS, sep=(P_SEP,), system=(503,), user=(P_USER,),
                     assistant=(P_MODEL,))


def place_trunk(spec=None, seed=41, heads=4, margin_bits=(2, 12)):
    """(asked, placed): a seeded trunk with reads after layer 1 and on the readout, its type
    weights 0, whose readout read asks with a question table that moves P_ASK's point onto
    P_BEFORE's; and the same with the place read (P_DOT stops, P_ASK arms, P_OPENS opens)."""
    spec = spec or synth.Spec(vocab=512, width=64, mlp=64, layers=3, context=32, kept=8)
    h = synth.HammingSpec(heads=heads, depths=(1, spec.layers), kept=8, asks=(False, True),
                          typed=False, margin_bits=margin_bits)
    asked = synth.make_artifact(replace(spec, hamming=h), seed)
    d = spec.width
    for r in asked.hamming_reads:
        r.weight[:d] = 1 << 24  # copy weights at one
    t = asked.writer_table.reshape(spec.vocab, d)
    t[P_ASK] = t[P_BEFORE] // 2  # so the question table's entry fits i16
    ask = np.zeros((spec.vocab, d), np.int16)
    ask[P_ASK] = t[P_BEFORE] - t[P_ASK]
    asked.hamming_reads[-1].ask = ask.reshape(-1)
    placed = synth.make_artifact(replace(spec, hamming=replace(h, place=P_MARKS)), seed)
    placed.writer_table = asked.writer_table.copy()
    placed.hamming_reads = asked.hamming_reads
    cls = np.zeros(spec.vocab, np.int16)
    cls[P_DOT], cls[P_ASK], cls[P_OPENS] = PLACE_STOP, PLACE_ARM, PLACE_OPEN
    placed.hamming_place = cls
    return asked, placed


def served(art, tokens):
    st, tok, query, place = oracle.place_sequences(art, np.asarray([tokens], np.uint32))
    assert st == 0
    return tok[0], query[0], [tuple(None if v < 0 else int(v) for v in p) for p in place[0]]


def test_a_session_serves_the_place_read():
    asked, placed = place_trunk()
    _, free, plain = served(asked, P_TALK)
    _, query, read = served(placed, P_TALK)
    assert all(p == (None, None) for p in plain)
    for t, (place, q, f) in enumerate(zip(read, query, free)):
        want = {17: (4, None), 18: (4, 4), 19: (5, 5)}.get(t, (None, None))
        assert place == want, t
        # The readout moves at an open row only.
        assert (not np.array_equal(q, f)) == (want[1] is not None), t
    # A reply that says another token after P_OPENS is offered nothing at that row, and the
    # register stays where it is.
    miss = P_TALK[:19] + [40, P_OPENS, 30]
    _, _, read = served(placed, miss)
    assert read[18:] == [(4, 4), (4, None), (4, 4), (5, 5)]
    # A fresh session from the reply on arms nothing (a reset forgets the conversation).
    _, _, read = served(placed, P_TALK[13:19])
    assert read[-1] == (None, None)


def test_the_offer_is_the_token_at_the_place_in_place_of_the_copy_mean():
    # With every copy weight at one (2^24 at 2^-24, as the reference's trunk), the readout move
    # n + w_c (c - n) is c itself, exactly (readout_sum, hamming.rs:1933-1940, no type term):
    # at an open row the query is the table's point of the token at the place, whatever n was.
    _, placed = place_trunk()
    d = placed.spec.width
    table = placed.writer_table.reshape(-1, d)
    _, query, read = served(placed, P_TALK)
    for row in (18, 19):
        np.testing.assert_array_equal(query[row], table[P_TALK[read[row][1]]])


# ---- The container (stack/tests.rs:8800-8880) ----------------------------------------------

def asked_container():
    _, data, _ = fixture(sorted(MANIFEST)[0])
    spec = uorlut.load(data).spec
    h = synth.HammingSpec(heads=8, depths=(2, spec.layers), kept=16, asks=(False, True))
    reads = synth.hamming_reads(spec, h, 7)
    return spec, uorlut.add_hamming(data, h, reads)


def test_the_place_read_round_trips_and_is_refused_by_name():
    spec, asked = asked_container()
    assert uorlut.load(asked).hamming.place is None
    cls = np.zeros(spec.vocab, np.int16)
    cls[5], cls[6], cls[7] = PLACE_STOP, PLACE_ARM, PLACE_OPEN | PLACE_STOP
    marks = PlaceMarks(bos=1, eos=2, sep=(3,), system=(), user=(4, 9), assistant=(4, 10))
    placed = uorlut.add_hamming_place(asked, marks, cls)
    art = uorlut.load(placed)
    assert art.hamming.place == marks and np.array_equal(art.hamming_place, cls)
    # Every earlier section keeps its bytes, and a place read is added once.
    hdr_a, body_a = _split(asked)
    hdr_p, body_p = _split(placed)
    assert body_p[:len(body_a)] == body_a
    with pytest.raises(uorlut.UorlutError):
        uorlut.add_hamming_place(placed, marks, cls)
    # A class table without its record, and a record without its table, are refused by name.
    orphan = dict(hdr_p, hamming={k: v for k, v in hdr_p["hamming"].items() if k != "place"})
    with pytest.raises(uorlut.UorlutError, match="names no place read"):
        uorlut.load(_build(orphan, body_p))
    bare = dict(hdr_a, hamming=dict(hdr_a["hamming"], place=marks.to_json()))
    with pytest.raises(uorlut.UorlutError, match="missing section"):
        uorlut.load(_build(bare, body_a))
    outside = dict(hdr_p, hamming=dict(hdr_p["hamming"], place=dict(marks.to_json(), bos=spec.vocab)))
    with pytest.raises(uorlut.UorlutError, match="outside the vocabulary"):
        uorlut.load(_build(outside, body_p))
    for why, bad in (("a separator", replace(marks, sep=())),
                     ("ends with another", replace(marks, assistant=marks.user)),
                     ("one token", replace(marks, eos=marks.bos))):
        with pytest.raises(uorlut.UorlutError, match=why):
            uorlut.add_hamming_place(asked, bad, cls)
    with pytest.raises(uorlut.UorlutError, match="one class|entries"):
        uorlut.add_hamming_place(asked, marks, cls[1:])
    wide = cls.copy()
    wide[0] = 8
    with pytest.raises(uorlut.UorlutError, match="stop, arm and open"):
        uorlut.add_hamming_place(asked, marks, wide)
    # The readout read must ask.
    _, data, _ = fixture(sorted(MANIFEST)[0])
    h = synth.HammingSpec(heads=8, depths=(2, spec.layers), kept=16, asks=(True, False))
    inner = uorlut.add_hamming(data, h, synth.hamming_reads(spec, h, 7))
    with pytest.raises(uorlut.UorlutError, match="a readout read that asks"):
        uorlut.add_hamming_place(inner, marks, cls)
