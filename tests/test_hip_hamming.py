"""The Hamming reads inside the served step on the GPU (fbs_hamming.h through the C ABI) against
the oracle, bit for bit: greedy decode replies, exported state and window, teacher-forced
choices, kept drawers and queries, and a decode split and resumed through the session stream
(tokens and payload caches, uor_fbs_decode_stream). Cases cover every kernel width (Q = 1, 2, 4
quaternions a lane), copy, type and ask heads with the question carry, every copy rule with mixed
copy keys and the reply marker, and a trained artifact with seeded reads added; then the
refusals of what this build does not serve. Sessions of these models served from pool slots
(uor_fbs_serve_slots_stream_async: serve_step and snapshots, stack/session.rs:2777-3440) equal
the oracle's stream decode.
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from test_uorlut import HAM, MANIFEST, fixture
from uor_fbs import session_codec, synth, uorlut
from uor_fbs.hip import FbsError, Model
from uor_fbs.session import Session, SessionError, SessionPool, serve_steps

pytestmark = pytest.mark.gpu

H = synth.HammingSpec
CASES = {
    # Copy and type heads at a stream read and at the readout.
    "w64_copy_type": (synth.Spec(vocab=256, width=64, mlp=64, layers=3, context=64, kept=8),
                      H(heads=4, depths=(1, 3), kept=8), 3, 24, 30),
    # Ask heads on the readout with the question carry; latest-exact copy heads; 8-wide heads.
    "w64_ask_carry": (synth.Spec(vocab=256, width=64, mlp=96, layers=3, context=64, kept=8),
                      H(heads=8, depths=(2, 3), kept=8, asks=(False, True), carry_rows=3,
                        copy_latest=True), 3, 20, 36),
    # Width 128, window 8, keyed drawers; mixed copy keys under latest-nearest; three reads.
    "w128_rules": (replace(synth.CONFIGS["c2"], layers=3, context=64),
                   H(heads=8, depths=(1, 2, 3), kept=16, copy_keys=(1, 2, 1, 2), rule=2), 4, 24, 32),
    # Width 256 (C3's shape, Zipf drawers): the longest rule after the reply marker.
    "w256_marker": (replace(synth.CONFIGS["c3"], layers=2, context=64),
                    H(heads=8, depths=(1, 2), kept=16, copy_latest=True, copy_longest=(3, 5)),
                    3, 24, 30),
    # Width 512 (two quaternions a lane), int8 table, asking stream read and typed readout.
    "w512": (replace(synth.CONFIGS["c5"], layers=2, context=48, vocab=4096),
             H(heads=16, depths=(1, 2), kept=8, asks=(True, False)), 2, 16, 24),
    # Width 1024 (four quaternions a lane), 64-coordinate heads, longest-exact.
    "w1024": (synth.Spec(vocab=512, width=1024, mlp=256, layers=2, context=40, kept=8),
              H(heads=16, depths=(1, 2), kept=12, rule=3), 2, 12, 20),
}


def build(name):
    spec, ham, n, plen, gen = CASES[name]
    art = synth.make_artifact(replace(spec, hamming=ham), 500 + list(CASES).index(name))
    prompts = synth.uniform_prompts(spec.vocab, n, plen, 77) % 16  # repeats for the heads
    if name == "w256_marker":
        prompts[:, 6:8] = (3, 5)
    return art, prompts.astype(np.uint32), gen


@pytest.mark.parametrize("name", sorted(CASES))
def test_decode_matches_the_oracle(name):
    art, prompts, gen = build(name)
    print(f"case {name} prompts {prompts.shape} gen {gen}", flush=True)
    model = Model(art)
    # Paired at one quaternion a lane (widths up to 256), one wavefront wider.
    assert model.block_waves(len(prompts)) == (2 if art.spec.width <= 256 else 1)
    got = model.decode(prompts, gen)
    want = oracle.decode(art, prompts, gen, threads=4)
    assert want["status"] == 0
    for k in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{name} {k}")


@pytest.mark.parametrize("name", sorted(CASES))
def test_sequences_match_the_oracle(name):
    art, prompts, gen = build(name)
    rows = np.concatenate([prompts, prompts[:, ::-1]], 1)[:, : art.spec.context]
    print(f"case {name} rows {rows.shape}", flush=True)
    tok, kept, query = Model(art).sequences(rows)
    st, t2, k2, q2 = oracle.sequences(art, rows, threads=4)
    assert st == 0
    np.testing.assert_array_equal(tok, t2)
    np.testing.assert_array_equal(kept, k2)
    np.testing.assert_array_equal(query, q2)


@pytest.mark.parametrize("name", sorted(CASES))
def test_a_resumed_stream_matches_the_oracle(name):
    art, prompts, gen = build(name)
    print(f"case {name} stream", flush=True)
    model = Model(art)
    first = model.decode_stream(prompts, gen // 2)
    want = oracle.decode_stream(art, prompts, gen // 2, threads=4)
    pos = int(want["position"][0])
    np.testing.assert_array_equal(first["reply"], want["reply"])
    np.testing.assert_array_equal(first["tokens"][:, :pos], want["tokens"][:, :pos])
    np.testing.assert_array_equal(first["payloads"][:, :, :pos], want["payloads"][:, :, :pos])
    again = model.decode_stream(first["reply"][:, -1:], gen - gen // 2 - 1, resume=first)
    want2 = oracle.decode_stream(art, want["reply"][:, -1:], gen - gen // 2 - 1, threads=4,
                                 resume=want)
    whole = oracle.decode(art, prompts, gen, threads=4)
    np.testing.assert_array_equal(again["reply"], want2["reply"])
    np.testing.assert_array_equal(again["reply"], whole["reply"][:, gen // 2 + 1:])
    for k in ("state", "history", "position"):
        np.testing.assert_array_equal(again[k], whole[k], err_msg=k)
    pos = int(whole["position"][0])
    np.testing.assert_array_equal(again["tokens"][:, :pos], want2["tokens"][:, :pos])
    np.testing.assert_array_equal(again["payloads"][:, :, :pos], want2["payloads"][:, :, :pos])


def test_a_trained_artifact_with_reads_matches_the_oracle():
    _, data, _ = fixture(sorted(MANIFEST)[0])
    reads = synth.hamming_reads(uorlut.load(data).spec, HAM, 7)
    art = uorlut.load(uorlut.add_hamming(data, HAM, reads))
    prompts = ((np.arange(2 * 40, dtype=np.uint32).reshape(2, 40) * 37) % 60).astype(np.uint32)
    print("case trained+hamming", flush=True)
    got = Model(art).decode(prompts, 40)
    want = oracle.decode(art, prompts, 40, threads=4)
    for k in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)


def test_refusals():
    art, prompts, gen = build("w64_copy_type")
    model = Model(art)
    first = model.decode(prompts, 2)
    with pytest.raises(FbsError) as e:  # resuming without the stream
        model.decode(prompts[:, :1], 2, in_state=first["state"], in_history=first["history"],
                     in_position=first["position"])
    assert e.value.code == 6
    bad = synth.make_artifact(replace(CASES["w64_copy_type"][0], hamming=H(heads=4, depths=(1, 3), kept=65)), 1)
    with pytest.raises(FbsError) as e:
        Model(bad)
    assert e.value.code == 6
    bad.hamming_reads[0].margin[1] = 0
    bad.hamming = replace(bad.hamming, kept=8)
    with pytest.raises(FbsError) as e:
        Model(bad)
    assert e.value.code == 4


def test_a_resumed_token_outside_the_vocabulary_is_refused():
    art, prompts, _ = build("w64_copy_type")
    model = Model(art)
    first = model.decode_stream(prompts, 3)
    bad = dict(first, tokens=first["tokens"].copy())
    bad["tokens"][1, 2] = art.spec.vocab
    with pytest.raises(FbsError) as e:
        model.decode_stream(first["reply"][:, -1:], 2, resume=bad)
    assert e.value.code == 1


def served_payloads(snap, art):
    """A snapshot's payload caches as [typed, context, width] (the reads that keep one)."""
    d, n = art.spec.width, art.spec.context
    return np.array([np.reshape(p, (n, d)) for p in snap.hamming_payloads if p],
                    np.int64).reshape(-1, n, d)


@pytest.mark.parametrize("name", ["w64_copy_type", "w64_ask_carry", "w256_marker", "w512"])
def test_a_serving_loop_of_sessions_matches_the_oracle(name):
    # Sessions in scrambled slots join the loop at different steps; each launch steps whichever
    # sessions have a token, in a shuffled order. Replies, state, window, token stream and
    # payload caches must equal the oracle's stream decode of the same prompts.
    art, prompts, gen = build(name)
    n = len(prompts)
    print(f"case {name} serving loop: {n} sessions, gen {gen}", flush=True)
    model = Model(art)
    want = oracle.decode_stream(art, prompts, gen, threads=4)
    assert want["status"] == 0
    pool = SessionPool(model, capacity=2 * n + 3)
    pool.acquire(1), pool.acquire(4)
    sessions = [Session(pool) for _ in range(n)]
    start = [0, 2, 1, 3][:n]
    nxt, got = [None] * n, [[] for _ in range(n)]
    rng = np.random.default_rng(11)
    for step in range(max(start) + gen + 1):
        batch, toks = [], []
        for i in rng.permutation(n):
            k = step - start[i]
            if k == 0:
                half = prompts.shape[1] // 2  # the prompt in two launches
                sessions[i].feed(prompts[i, :half])
                nxt[i] = sessions[i].feed(prompts[i, half:]).token
                got[i].append(nxt[i])
            elif 0 < k <= gen:
                batch.append(sessions[i])
                toks.append(nxt[i])
        if batch:
            for s, (tok, _) in zip(batch, serve_steps(batch, toks)):
                i = sessions.index(s)
                nxt[i] = tok
                got[i].append(tok)
    for i, s in enumerate(sessions):
        np.testing.assert_array_equal(np.array(got[i], np.uint32), want["reply"][i], err_msg=str(i))
        snap = s.save_state()
        pos = int(want["position"][i])
        assert snap.position == pos
        np.testing.assert_array_equal(np.concatenate([l.state for l in snap.layers]), want["state"][i])
        np.testing.assert_array_equal(np.concatenate([l.history for l in snap.layers]),
                                      want["history"][i])
        assert snap.tokens == want["tokens"][i, :pos].tolist()
        pay = served_payloads(snap, art)
        assert pay.shape[0] == want["payloads"].shape[1]
        np.testing.assert_array_equal(pay[:, :pos], want["payloads"][i, :, :pos])


@pytest.mark.parametrize("name", ["w64_copy_type", "w512"])
def test_a_restored_session_continues_bit_for_bit(name, tmp_path):
    # A Hamming session saved mid-stream (tokens and payloads in the snapshot) and restored into
    # another slot, through the codec, JSON and in place, continues as the original did and as
    # the oracle's resumed stream decode does.
    art, prompts, gen = build(name)
    print(f"case {name} save/restore", flush=True)
    pool = SessionPool(Model(art), capacity=5)
    a = Session(pool, 2)
    tok = a.feed(prompts[0]).token
    for _ in range(4):
        tok, _ = a.serve_step(tok)
    snap = a.save_state()
    wire = session_codec.encode(snap)
    path = tmp_path / "h.json"
    a.save_session_to_file(path)
    cont, t = [], tok
    for _ in range(gen - 5):
        t, _ = a.serve_step(t)
        cont.append(t)
    want = oracle.decode_stream(art, prompts[:1], gen, threads=4)
    np.testing.assert_array_equal(np.array(cont, np.uint32), want["reply"][0, 5:gen])
    for how in ("codec", "json", "same-slot"):
        b = a if how == "same-slot" else Session(pool)
        if how == "codec":
            b.restore_state(session_codec.decode(wire))
        elif how == "json":
            b.restore_session_from_file(path)
        else:
            b.restore_state(snap)
        t, again = tok, []
        for _ in range(gen - 5):
            t, _ = b.serve_step(t)
            again.append(t)
        assert again == cont, how
        if b is not a:
            b.close()
    # A snapshot without its payloads is refused where the model keeps them.
    if served_payloads(snap, art).shape[0]:
        bare = session_codec.decode(wire)
        bare.hamming_payloads = []
        with pytest.raises(SessionError):
            Session(pool).restore_state(bare)


# ---- The place read (hamming.rs:1510-1533, 1625-1634, 1883-1913; fbs_snapshot.rs:2716-3135) ----
# The oracle's register is pinned by the reference's own place tests (test_place_oracle.py); here
# the GPU path is held to it, bit for bit, on the reference's talk and on seeded conversations
# whose words stop, arm and open at random, at every kernel width.

from test_place_oracle import P_ASK, P_BOS, P_EOS, P_MODEL, P_SEP, P_TALK, P_USER, place_trunk

PLACE_CASES = {  # shape, heads, the teacher-forced conversations' seed
    "w64": (synth.Spec(vocab=512, width=64, mlp=64, layers=3, context=64, kept=8), 4, 7),
    "w512": (synth.Spec(vocab=1024, width=512, mlp=128, layers=2, context=48, kept=8), 16, 7),
    "w1024": (synth.Spec(vocab=768, width=1024, mlp=128, layers=2, context=40, kept=8), 16, 14),
}


def place_case(name, seed=91):
    spec, heads, _ = PLACE_CASES[name]
    _, placed = place_trunk(spec, seed, heads=heads, margin_bits=(6, 24))
    rng = np.random.default_rng(seed)
    cls = placed.hamming_place.copy()
    words = np.arange(20, 40)
    cls[words] = (np.where(rng.random(20) < 0.15, 1, 0) | np.where(rng.random(20) < 0.35, 2, 0)
                  | np.where(rng.random(20) < 0.35, 4, 0))
    placed.hamming_place = cls
    return placed


def conversations(n, length, seed, end_in_reply=False):
    """Seeded conversations over the marks and a small alphabet (words repeat, so finds land)."""
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(n):
        toks = [P_BOS]
        while len(toks) < length:
            role = rng.choice([P_USER, P_MODEL, 503], p=[0.45, 0.45, 0.1])
            toks += [role] if len(toks) == 1 else [P_SEP, role]
            toks += [int(w) for w in rng.integers(20, 40, size=int(rng.integers(2, 9)))]
            if rng.random() < 0.3:
                toks.append(P_ASK)
            if rng.random() < 0.5:
                toks.append(P_EOS)
        toks = toks[:length]
        if end_in_reply:
            toks[-2:] = [P_SEP, P_MODEL]
        rows.append(toks)
    return np.asarray(rows, np.uint32)


@pytest.mark.parametrize("name", sorted(PLACE_CASES))
def test_the_place_read_matches_the_oracle_teacher_forced(name):
    art = place_case(name)
    rows = conversations(8, art.spec.context, PLACE_CASES[name][2])
    print(f"place {name} rows {rows.shape}", flush=True)
    st, tok, query, place = oracle.place_sequences(art, rows, threads=4)
    assert st == 0
    assert (place[..., 1] >= 0).sum() >= 3, "the register opens rows in these conversations"
    got_t, got_k, got_q = Model(art).sequences(rows)
    np.testing.assert_array_equal(got_t, tok)
    np.testing.assert_array_equal(got_q, query)
    _, _, k2, _ = oracle.sequences(art, rows, threads=4)
    np.testing.assert_array_equal(got_k, k2)


@pytest.mark.parametrize("name", sorted(PLACE_CASES))
def test_the_place_read_decodes_and_resumes_as_the_oracle(name):
    art = place_case(name)
    ctx = art.spec.context
    prompts = conversations(4, ctx // 2, 8, end_in_reply=True)
    gen = ctx - prompts.shape[1] - 1
    print(f"place {name} decode prompts {prompts.shape} gen {gen}", flush=True)
    model = Model(art)
    want = oracle.decode(art, prompts, gen, threads=4)
    assert want["status"] == 0
    got = model.decode(prompts, gen)
    for k in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{name} {k}")
    # Split and resumed through the session stream: the register is rebuilt from the tokens.
    half = gen // 2
    first = model.decode_stream(prompts, half)
    again = model.decode_stream(first["reply"][:, -1:], gen - half - 1, resume=first)
    np.testing.assert_array_equal(again["reply"], want["reply"][:, half + 1:])
    for k in ("state", "history", "position"):
        np.testing.assert_array_equal(again[k], want[k], err_msg=f"{name} resumed {k}")


def test_the_reference_talk_is_offered_its_place_on_the_gpu():
    # The reference's own session case (stack/tests.rs:8882-8930) through the GPU: with the copy
    # weights at one, an open row's query is the table point of the token at the place.
    asked, placed = place_trunk()
    d = placed.spec.width
    table = placed.writer_table.reshape(-1, d)
    rows = np.asarray([P_TALK], np.uint32)
    tok, _, query = Model(placed).sequences(rows)
    st, t2, q2, place = oracle.place_sequences(placed, rows)
    assert st == 0
    np.testing.assert_array_equal(tok, t2)
    np.testing.assert_array_equal(query, q2)
    np.testing.assert_array_equal(query[0, 18], table[P_TALK[4]])
    np.testing.assert_array_equal(query[0, 19], table[P_TALK[5]])
    _, _, free = Model(asked).sequences(rows)
    moved = [t for t in range(len(P_TALK)) if not np.array_equal(query[0, t], free[0, t])]
    assert moved == [18, 19]


def test_place_sessions_served_from_slots_match_the_oracle():
    art = place_case("w64")
    prompts = conversations(3, 20, 9, end_in_reply=True)
    gen = 24
    print("place sessions from slots", flush=True)
    want = oracle.decode_stream(art, prompts, gen, threads=4)
    pool = SessionPool(Model(art), capacity=5)
    sessions = [Session(pool, s) for s in (3, 0, 4)]
    nxt = [s.feed(p[:7]).token for s, p in zip(sessions, prompts)]
    nxt = [s.feed(p[7:]).token for s, p in zip(sessions, prompts)]
    got = [[t] for t in nxt]
    for _ in range(gen):
        for i, (tok, _) in enumerate(serve_steps(sessions, nxt)):
            got[i].append(tok)
            nxt[i] = tok
    np.testing.assert_array_equal(np.asarray(got, np.uint32), want["reply"])


@pytest.mark.parametrize("name", ["w64_copy_type", "w64_ask_carry", "w128_rules", "w256_marker"])
@pytest.mark.parametrize("waves", ["1", "2"])
def test_paired_and_one_wavefront_reads_are_the_oracles(name, waves, monkeypatch):
    # The paired kernels share each read's heads between the waves (wave 0 the even heads of each
    # kind, wave 1 the odd, partial sums added before the divisions); one wavefront takes them
    # all. Both bit for bit the oracle's: decode through the stream, resumed, and teacher-forced.
    monkeypatch.setenv("UOR_FBS_BLOCK_WAVES", waves)
    art, prompts, gen = build(name)
    print(f"case {name} on {waves} wavefront(s)", flush=True)
    model = Model(art)
    assert model.block_waves(len(prompts)) == int(waves)
    want = oracle.decode_stream(art, prompts, gen // 2, threads=4)
    first = model.decode_stream(prompts, gen // 2)
    for k in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(first[k], want[k], err_msg=f"{name} {k}")
    pos = int(want["position"][0])
    np.testing.assert_array_equal(first["tokens"][:, :pos], want["tokens"][:, :pos])
    np.testing.assert_array_equal(first["payloads"][:, :, :pos], want["payloads"][:, :, :pos])
    again = model.decode_stream(first["reply"][:, -1:], gen - gen // 2 - 1, resume=first)
    whole = oracle.decode(art, prompts, gen, threads=4)
    np.testing.assert_array_equal(again["reply"], whole["reply"][:, gen // 2 + 1:])
    for k in ("state", "history", "position"):
        np.testing.assert_array_equal(again[k], whole[k], err_msg=f"{name} resumed {k}")
    rows = np.concatenate([prompts, prompts[:, ::-1]], 1)[:, : art.spec.context]
    tok, kept, query = model.sequences(rows)
    st, t2, k2, q2 = oracle.sequences(art, rows, threads=4)
    np.testing.assert_array_equal(tok, t2)
    np.testing.assert_array_equal(kept, k2)
    np.testing.assert_array_equal(query, q2)
