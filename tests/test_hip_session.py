"""Serving sessions on the GPU (uor_fbs/session.py over uor_fbs_serve_slots_async) against the
batched decode and the oracle: IntegerStackSession's serving calls (stack/session.rs:2703-3440),
a serving loop that steps whichever sessions have a token, and snapshots that restore into any
slot and continue bit for bit (session.rs:2777-3290, session_codec.rs)."""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import hip, session_codec, synth
from uor_fbs.hipmem import DeviceArray
from uor_fbs.session import NO_CHOICE, Session, SessionError, SessionPool, serve_steps

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("block_waves")]

SPEC = replace(synth.CONFIGS["c2"], context=48, layers=3)
SEED = 71


@pytest.fixture(scope="module")
def art():
    return synth.make_artifact(SPEC, SEED)


def test_serving_loop_equals_batched_decode(art):
    S, P, G = 6, 10, 24
    prompts = synth.uniform_prompts(SPEC.vocab, S, P, 73)
    print(f"serving loop: {S} sessions, prompt {P}, gen {G}", flush=True)
    model = hip.Model(art)
    want = model.decode(prompts, gen=G)
    pool = SessionPool(model, capacity=11)
    # Slots taken out of order; sessions join the loop at different steps.
    pool.acquire(), pool.acquire()
    sessions = [Session(pool) for _ in range(S)]
    start = [0, 3, 1, 7, 2, 5]
    nxt = [None] * S
    got = [[] for _ in range(S)]
    rng = np.random.default_rng(5)
    for step in range(max(start) + G + 1):
        batch, toks = [], []
        for i in rng.permutation(S):
            k = step - start[i]
            if k == 0:
                nxt[i] = sessions[i].feed(prompts[i]).token     # the prompt in one launch
                got[i].append(nxt[i])
            elif 0 < k < G + 1:
                batch.append(sessions[i])
                toks.append(nxt[i])
        if batch:
            for s, (tok, margin) in zip(batch, serve_steps(batch, toks)):
                i = sessions.index(s)
                assert margin == 0
                nxt[i] = tok
                got[i].append(tok)
    # Each session has stepped its prompt and G fed-back choices, as the decode did.
    for i, s in enumerate(sessions):
        np.testing.assert_array_equal(np.array(got[i], np.uint32), want["reply"][i])
        st = s.save_state()
        np.testing.assert_array_equal(np.concatenate([l.state for l in st.layers]), want["state"][i])
        np.testing.assert_array_equal(np.concatenate([l.history for l in st.layers]), want["history"][i])
        assert st.position == want["position"][i] == P + G
        assert st.tokens == [int(t) for t in prompts[i]] + [int(t) for t in want["reply"][i, :G]]


def test_pool_larger_than_the_grid(art):
    # More live sessions than resident blocks (1,024 paired blocks on MI355X): one launch steps
    # 2,600 sessions held in scrambled slots of a 3,000-slot pool, blocks looping over them.
    # Each session's prompt feed and following steps must equal the batched decode's.
    S, P, G = 2600, 6, 4
    prompts = synth.uniform_prompts(SPEC.vocab, S, P, 83)
    model = hip.Model(art)
    want = model.decode(prompts, gen=G)
    pool = SessionPool(model, capacity=3000)
    slots = np.random.default_rng(9).permutation(3000)[:S].astype(np.uint32)
    print(f"pool of {pool.capacity}: {S} sessions", flush=True)
    out = pool.run(slots, prompts, gen=G)
    assert (out["status"] == 0).all()
    np.testing.assert_array_equal(out["reply"], want["reply"])
    for i in (0, 1023, 1024, 2047, 2048, S - 1):
        state, history, position = pool.read(int(slots[i]))
        np.testing.assert_array_equal(state, want["state"][i])
        np.testing.assert_array_equal(history, want["history"][i])
        assert position == P + G


def test_step_native_matches_the_oracle(art):
    tokens = synth.uniform_prompts(SPEC.vocab, 2, 14, 79)
    st, want_tok, want_kept, want_query = oracle.sequences(art, tokens, threads=2)
    assert st == 0
    print("step_native against the oracle", flush=True)
    pool = SessionPool(hip.Model(art), capacity=3)
    for r in range(2):
        s = Session(pool)
        for t in range(tokens.shape[1]):
            nat = s.step_native(int(tokens[r, t]))
            assert nat.token == want_tok[r, t] == s.last_native_token()
            np.testing.assert_array_equal(nat.kept_cells, want_kept[r, t])
            np.testing.assert_array_equal(nat.query_q12, want_query[r, t])
        # A feed of the same row in one launch ends in the same state and choice.
        s2 = Session(pool)
        assert s2.feed(tokens[r]).token == want_tok[r, -1]
        a, b = s.save_state(), s2.save_state()
        assert a.layers == b.layers and a.tokens == b.tokens and a.position == b.position
        s.close(), s2.close()


def test_save_restore_continues_bit_for_bit(art, tmp_path):
    prompts = synth.uniform_prompts(SPEC.vocab, 1, 9, 83)[0]
    print("save/restore", flush=True)
    model = hip.Model(art)
    pool = SessionPool(model, capacity=4)
    a = Session(pool)
    tok = a.feed(prompts).token
    for _ in range(5):
        tok, _ = a.serve_step(tok)
    snap = a.save_state()
    assert snap.position == len(prompts) + 5 and snap.cache_at == snap.position * SPEC.width
    assert len(snap.logits) == SPEC.vocab and not any(snap.logits)
    wire = session_codec.encode(snap)
    assert wire[:8] == b"UR4SESS1"
    path = tmp_path / "sess" / "a.json"
    a.save_session_to_file(path)
    cont = []
    t = tok
    for _ in range(12):
        t, _ = a.serve_step(t)
        cont.append(t)
    for how in ("codec", "json", "same-slot"):
        b = a if how == "same-slot" else Session(pool)
        if how == "codec":
            b.restore_state(session_codec.decode(wire))
        elif how == "json":
            b.restore_session_from_file(path)
        else:
            b.restore_state(snap)
        assert b.position == snap.position
        t, again = tok, []
        for _ in range(12):
            t, _ = b.serve_step(t)
            again.append(t)
        assert again == cont, how
        if b is not a:
            b.close()


def test_reset_and_refusals_leave_state(art):
    print("reset and refusals", flush=True)
    pool = SessionPool(hip.Model(art), capacity=2)
    s = Session(pool)
    first = s.feed([1, 2, 3]).token
    before = s.save_state()
    with pytest.raises(SessionError) as e:
        s.step_native(SPEC.vocab)
    assert e.value.kind == "Token" and s.save_state() == before
    # A feed stops at the refused token, the tokens before it stepped.
    with pytest.raises(SessionError):
        s.feed([4, 5, SPEC.vocab + 7, 6])
    assert s.position == 5 and s.tokens == [1, 2, 3, 4, 5]
    s.reset()
    assert s.position == 0 and s.last_native_token() is None
    assert s.feed([1, 2, 3]).token == first
    # The context: exactly `context` tokens step, the next is refused.
    s.reset()
    s.feed(list(range(1, SPEC.context)))
    s.serve_step(1)
    with pytest.raises(SessionError) as e:
        s.serve_step(1)
    assert e.value.kind == "ContextFull" and s.position == SPEC.context
    # Restores check the serving identity.
    other = SessionPool(hip.Model(synth.make_artifact(SPEC, SEED + 1)), capacity=1)
    with pytest.raises(SessionError) as e:
        Session(other).restore_state(before)
    assert e.value.kind == "Numerics"


def test_nearest_head_read_step_chooses_nothing():
    spec = replace(synth.NON_SQUARE, head=1, context=12)
    art = synth.make_artifact(spec, 89)
    print("nearest head read_step", flush=True)
    pool = SessionPool(hip.Model(art), capacity=2)
    a, b = Session(pool), Session(pool)
    a.read_step(3)
    assert a.last_native_token() is None and a._native.token == NO_CHOICE
    b.step_native(3)
    assert b.last_native_token() is not None
    assert a.save_state().layers == b.save_state().layers


def test_slot_bounds_are_checked_by_the_kernel(art):
    """A slot at or past the capacity gets status 3 and touches nothing; the others step."""
    print("slot bounds", flush=True)
    model = hip.Model(art)
    pool = SessionPool(model, capacity=2)
    arr = lambda a: DeviceArray(len(a), np.uint32)  # noqa: E731
    slots, toks = arr([1, 2, 0]), arr([5, 5, 5])
    slots.upload(np.array([1, 2, 0], np.uint32))
    toks.upload(np.array([5, 5, 5], np.uint32))
    reply, status = DeviceArray(3, np.uint32), DeviceArray(3, np.int32)
    hip._check(hip.lib().uor_fbs_decode_slots_async(
        model.handle, slots.ptr, 3, 2, toks.ptr, 1, 0, reply.ptr, pool.state.ptr, pool.history.ptr,
        pool.position.ptr, None, None, status.ptr, None))
    assert status.download().tolist() == [0, 3, 0]
    assert pool.position.download().tolist() == [1, 1]
    r = reply.download()
    assert r[0] == r[2]


def test_session_slots_are_checked_on_the_host(art):
    """A caller-chosen slot must lie in the pool and be free; it is then held like an acquired
    one. Device rows are bounds-checked before any copy."""
    print("session slot checks", flush=True)
    pool = SessionPool(hip.Model(art), capacity=3)
    with pytest.raises(ValueError):
        Session(pool, slot=3)
    a = Session(pool, slot=1)
    with pytest.raises(ValueError):
        Session(pool, slot=1)
    b, c = Session(pool), Session(pool)
    assert sorted([a.slot, b.slot, c.slot]) == [0, 1, 2]
    with pytest.raises(SessionError):
        Session(pool)
    a.close()
    assert Session(pool, slot=1).slot == 1
    with pytest.raises(IndexError):
        pool.position.zero([3])
    with pytest.raises(IndexError):
        pool.position.download(row=3)


def test_a_slid_session_equals_the_oracle(art):
    """set_context_slide (session.rs:2391-2402): a session at its context continues; its tokens,
    state, window and position equal the oracle's sliding decode, one token per launch through
    the pool's serving cache."""
    small = replace(art, spec=replace(art.spec, context=16))
    prompts = synth.uniform_prompts(SPEC.vocab, 2, 10, 91)
    G = 30
    want = oracle.decode(small, prompts, G, slide=True)
    assert want["status"] == 0
    model = hip.Model(small)
    pool = SessionPool(model, capacity=4)
    plain = Session(pool)
    plain.feed(prompts[0])
    with pytest.raises(SessionError) as e:
        for _ in range(G):
            plain.serve_step(int(prompts[0, 0]))
    assert e.value.kind == "ContextFull" and plain.position == 16
    for i in range(2):
        s = Session(pool)
        s.set_context_slide(True)
        got = [s.feed(prompts[i]).token]
        for _ in range(G):
            got.append(s.serve_step(got[-1])[0])
        np.testing.assert_array_equal(np.array(got, np.uint32), want["reply"][i])
        st = s.save_state()
        np.testing.assert_array_equal(np.concatenate([l.state for l in st.layers]), want["state"][i])
        np.testing.assert_array_equal(np.concatenate([l.history for l in st.layers]), want["history"][i])
        assert st.position == want["position"][i] == 10 + G
        assert len(st.tokens) == 16
        s.reset()
        assert s.slide  # reset keeps the caller's setting
        s.close()


def test_the_slide_is_refused_where_the_reference_refuses_it(art):
    ham = synth.make_artifact(replace(SPEC, hamming=synth.HammingSpec(heads=4, depths=(1,), kept=4)), 3)
    s = Session(SessionPool(hip.Model(ham), capacity=1))
    with pytest.raises(SessionError):
        s.set_context_slide(True)
    mem = replace(art, turn_memory=True)
    s = Session(SessionPool(hip.Model(mem), capacity=1))
    with pytest.raises(SessionError):
        s.set_context_slide(True)


def test_the_serving_cache_equals_launches_without_it(art):
    """uor_fbs_serve_slots_async with each slot's cache (window sums for the next step, writer
    memory) against the same entry without one, one token a launch for 12 launches over
    scrambled slots, and both against the batched decode. (Slots rewritten by the caller, whose
    cache entries SessionPool.write zeroes, continue bit for bit in the snapshot tests above.)"""
    n, cap, P, K = 5, 9, 8, 12
    model = hip.Model(art)
    L = hip.lib()
    prompts = synth.uniform_prompts(SPEC.vocab, n, P, 95)
    want = model.decode(prompts, gen=K)
    slots = np.array([7, 2, 5, 0, 8], np.uint32)
    pools = []
    for cached in (True, False):
        st = DeviceArray((cap, model.state_words), np.int64)
        hi = DeviceArray((cap, model.history_words), np.int32)
        po = DeviceArray(cap, np.uint32)
        ca = DeviceArray((cap, int(L.uor_fbs_slot_cache_bytes(model.handle))), np.uint8)
        for a in (st, hi, po, ca):
            a.zero()
        pools.append((st, hi, po, ca if cached else None))
    d_slots = DeviceArray(n, np.uint32)
    d_slots.upload(slots)
    status = DeviceArray(n, np.int32)
    outs = []
    for st, hi, po, ca in pools:
        toks = prompts
        got = []
        for k in range(K + 1):
            d_tok = DeviceArray(toks.size, np.uint32)
            d_tok.upload(np.ascontiguousarray(toks, np.uint32).reshape(-1))
            reply = DeviceArray((n, 1), np.uint32)
            hip._check(L.uor_fbs_serve_slots_async(
                model.handle, d_slots.ptr, n, cap, d_tok.ptr, toks.shape[1], 0, reply.ptr, st.ptr,
                hi.ptr, po.ptr, None if ca is None else ca.ptr, None, None, None, None, status.ptr,
                None))
            assert (status.download() == 0).all()
            r = reply.download()
            got.append(r[:, 0])
            toks = r
        outs.append(np.stack(got, 1))
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], want["reply"])


def test_snap_trace_follows_the_oracle():
    """enable_snap_trace on the device path: each step's transition roots (stack_lanes,
    session.rs:5117-5124) from the traced slot launch equal the oracle's teacher-forced trace;
    a traced snapshot continues its trace in another slot; the served tokens are unchanged."""
    from uor_fbs.session import transition_roots
    spec = replace(SPEC, raw_transition=False, raw_gates=False)
    art = synth.make_artifact(spec, 89)
    tokens = synth.uniform_prompts(spec.vocab, 1, 24, 97)[0]
    st, want_tok, _, _, tr = oracle.trace_sequences(art, tokens[None], threads=2)
    assert st == 0
    lanes = spec.width // 4
    per = spec.layers * lanes
    want = transition_roots(tr[0], spec.layers, lanes)
    print(f"snap trace: width {spec.width}, {spec.layers} layers, {len(tokens)} tokens", flush=True)
    pool = SessionPool(hip.Model(art), capacity=5)
    a, b, c = Session(pool), Session(pool), Session(pool)
    a.feed(tokens[:3])
    a.enable_snap_trace()
    assert a.feed(tokens[3:9]).token == want_tok[0, 8]
    for k in range(9, 14):
        assert a.serve_step(int(tokens[k]))[0] == want_tok[0, k]
    got = a.snap_trace()
    assert [e.root for e in got] == want[3 * per:14 * per].tolist()
    assert (got[0].position, got[-1].position) == (3, 13)
    assert a.save_state().snap_trace is None
    b.enable_snap_trace()
    b.feed(tokens[:10])
    snap = b.save_state()
    assert snap.snap_trace == want[:10 * per].tolist()
    c.restore_state(session_codec.decode(session_codec.encode(snap)))
    replies = serve_steps([c, a], [int(tokens[10]), int(tokens[14])])
    assert (replies[0][0], replies[1][0]) == (want_tok[0, 10], want_tok[0, 14])
    for t in tokens[11:]:
        c.serve_step(int(t))
    assert c.save_state().snap_trace == want.tolist()
    assert [e.root for e in a.snap_trace()] == want[3 * per:15 * per].tolist()
    b.reset()
    b.feed(tokens[:5])
    assert b.save_state().snap_trace == want[:5 * per].tolist()


def test_a_slot_rewritten_in_place_sums_its_window_afresh(art):
    """A caller that writes another session's state, history and position into a slot at the
    position the slot's cache entry was formed for, without clearing the entry (the C ABI does
    not require it to): the entry's sums were formed beside the slot's old state, whose
    fingerprint no longer matches, so the launch sums the window afresh and the slot continues as
    the session it now holds."""
    cap, P, K = 4, 10, 6
    A, B = 1, 2
    model = hip.Model(art)
    L = hip.lib()
    pa, pb = (synth.uniform_prompts(SPEC.vocab, 1, P, s) for s in (301, 302))
    st = DeviceArray((cap, model.state_words), np.int64)
    hi = DeviceArray((cap, model.history_words), np.int32)
    po = DeviceArray(cap, np.uint32)
    ca = DeviceArray((cap, int(L.uor_fbs_slot_cache_bytes(model.handle))), np.uint8)
    for a in (st, hi, po, ca):
        a.zero()
    status = DeviceArray(2, np.int32)

    def serve(slots, toks):
        d_slots = DeviceArray(len(slots), np.uint32)
        d_slots.upload(np.asarray(slots, np.uint32))
        toks = np.ascontiguousarray(toks, np.uint32)
        d_tok = DeviceArray(toks.size, np.uint32)
        d_tok.upload(toks.reshape(-1))
        reply = DeviceArray((len(slots), 1), np.uint32)
        hip._check(L.uor_fbs_serve_slots_async(
            model.handle, d_slots.ptr, len(slots), cap, d_tok.ptr, toks.shape[1], 0, reply.ptr,
            st.ptr, hi.ptr, po.ptr, ca.ptr, None, None, None, None, status.ptr, None))
        assert (status.download()[: len(slots)] == 0).all()
        return reply.download()[:, 0]

    first = serve([A, B], np.concatenate([pa, pb]))   # both slots at position P, entries cached
    rows = [a.download() for a in (st, hi, po)]
    assert not np.array_equal(rows[1][A], rows[1][B])
    for a, r in zip((st, hi, po), rows):
        r[A] = r[B]
        a.upload(r)
    want = model.decode(pb, gen=K)["reply"][0]
    tok_a = tok_b = first[1]
    got_a, got_b = [first[1]], [first[1]]
    for _ in range(K):
        tok_a, tok_b = serve([A, B], np.array([[tok_a], [tok_b]], np.uint32))
        got_a.append(tok_a)
        got_b.append(tok_b)
    np.testing.assert_array_equal(got_b, want)
    np.testing.assert_array_equal(got_a, want)
    end = [a.download() for a in (st, hi, po)]
    for r in end:                                     # the whole session, not only its tokens
        np.testing.assert_array_equal(r[A], r[B])
