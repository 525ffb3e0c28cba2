"""One-token serving launches with the drawer-major scan (fbs_serve.hip: the step stops at the
writer's drawer selection, a scan laid out by drawer scores every kept drawer's members against
the queries of every session that kept it, and each session takes the lowest (L1, token),
session.rs:4100-4121) against the writer inside the step (a model created with
UOR_FBS_SERVE_SCAN=fused; the drawer-major models are created with =drawer, which takes the scan
whatever the drawers' sizes) and the batched decode: tokens, kept drawers, queries, states, window
rings, positions and statuses equal, at Zipf drawer sizes (several 64-member chunks a drawer,
several 16-session slices), at more sessions than resident blocks, with permuted slots, with and
without the slot cache, with int8 tables, and with a refused session in a launch."""

import os
from dataclasses import replace

import numpy as np
import pytest

from uor_fbs import hip, synth
from uor_fbs.hipmem import DeviceArray

pytestmark = pytest.mark.gpu

SHAPES = {
    # C3's writer (256 Zipf drawers of 31..512 members, 8 kept) at a short context.
    "c3": replace(synth.CONFIGS["c3"], context=64),
    # C2's (64 drawers of 128, 4 kept): about 44 sessions a drawer at 700 sessions.
    "c2": replace(synth.CONFIGS["c2"], context=64, layers=3),
    # Width 64 (the 32-word rows) over the reference's 256 cells (t mod 256).
    "w64": synth.Spec(vocab=4096, width=64, mlp=96, layers=2, context=64, kept=8, window=3),
    # Width 32 (16-word rows, the smallest segment) over Zipf drawers.
    "w32": synth.Spec(vocab=2048, width=32, mlp=64, layers=2, context=64, kept=6, window=4,
                      drawers=200, probes=6, zipf_drawers=1.3, max_drawer=150),
    # C5's int8 codes (two quaternions a lane, 1,024 Zipf drawers of up to 1,024 probing 16).
    "c5": replace(synth.CONFIGS["c5"], context=64, layers=2),
    # An int8 table at one quaternion a lane.
    "w128i8": synth.Spec(vocab=8192, width=128, mlp=192, layers=2, context=64, kept=8, window=8,
                         drawers=128, probes=8, zipf_drawers=1.1, max_drawer=400, table="i8"),
}


def make_model(art, fused: bool):
    """A model whose one-token launches take the drawer-major scan (whatever its drawers' sizes)
    or keep the writer in the step."""
    os.environ["UOR_FBS_SERVE_SCAN"] = "fused" if fused else "drawer"
    try:
        return hip.Model(art)
    finally:
        os.environ.pop("UOR_FBS_SERVE_SCAN", None)


def serve(model, prompts, slots, cap, K, cached, refuse=None):
    """The prompt in one launch, then K one-token launches feeding each choice back. `refuse`:
    (launch, session) whose token is replaced by one outside the vocabulary."""
    L = hip.lib()
    n = len(slots)
    st = DeviceArray((cap, model.state_words), np.int64)
    hi = DeviceArray((cap, model.history_words), np.int32)
    po = DeviceArray(cap, np.uint32)
    ca = DeviceArray((cap, int(L.uor_fbs_slot_cache_bytes(model.handle))), np.uint8)
    for a in (st, hi, po, ca):
        a.zero()
    d_slots = DeviceArray(n, np.uint32)
    d_slots.upload(np.asarray(slots, np.uint32))
    status = DeviceArray(n, np.int32)
    kept = DeviceArray((n, model.probes), np.uint32)
    query = DeviceArray((n, model.width), np.int32)
    toks = np.ascontiguousarray(prompts, np.uint32)
    replies, kepts, queries, statuses = [], [], [], []
    for k in range(K + 1):
        if refuse is not None and k == refuse[0]:
            toks = toks.copy()
            toks[refuse[1], 0] = model.art.spec.vocab
        d_tok = DeviceArray(toks.size, np.uint32)
        d_tok.upload(toks.reshape(-1))
        reply = DeviceArray((n, 1), np.uint32)
        hip._check(L.uor_fbs_serve_slots_async(
            model.handle, d_slots.ptr, n, cap, d_tok.ptr, toks.shape[1], 0, reply.ptr, st.ptr,
            hi.ptr, po.ptr, ca.ptr if cached else None, None, kept.ptr, query.ptr, None,
            status.ptr, None))
        s = status.download()
        r = reply.download()
        statuses.append(s)
        replies.append(r[:, 0])
        if k:
            kepts.append(kept.download())
            queries.append(query.download())
        toks = r
    return dict(reply=np.stack(replies, 1), kept=np.stack(kepts), query=np.stack(queries),
                status=np.stack(statuses), state=st.download(), history=hi.download(),
                position=po.download())


@pytest.mark.parametrize("name,n,cached", [("c3", 1100, True), ("c3", 300, False),
                                           ("c2", 700, True), ("w64", 90, True),
                                           ("w32", 257, True), ("c5", 400, True),
                                           ("w128i8", 500, False)])
def test_drawer_major_serving_equals_the_fused_writer(name, n, cached):
    spec = SHAPES[name]
    art = synth.make_artifact(spec, 4242)
    P, K = 12, 6
    prompts = (synth.zipf_prompts(spec.vocab, n, P, 77) if spec.zipf_drawers
               else synth.uniform_prompts(spec.vocab, n, P, 77))
    cap = n + 7
    slots = np.random.default_rng(9).permutation(cap)[:n].astype(np.uint32)
    print(f"serve scan: {name}, {n} sessions, prompt {P}, {K} one-token launches, "
          f"cache {cached}", flush=True)
    deferred, fused = make_model(art, False), make_model(art, True)
    assert deferred.block_waves(n) == 2
    got = serve(deferred, prompts, slots, cap, K, cached)
    ref = serve(fused, prompts, slots, cap, K, cached)
    assert (got["status"] == 0).all() and (ref["status"] == 0).all()
    for key in ("reply", "kept", "query", "state", "history", "position"):
        np.testing.assert_array_equal(got[key], ref[key], err_msg=key)
    want = deferred.decode(prompts, gen=K, want_state=False)["reply"]
    np.testing.assert_array_equal(got["reply"], want)


def test_a_refused_session_leaves_the_others_served():
    """A session whose token lies outside the vocabulary is refused (status 1) and publishes no
    job; every other session of the launch takes the same token as the fused writer's."""
    spec = SHAPES["c3"]
    art = synth.make_artifact(spec, 4243)
    n, P, K = 200, 8, 3
    prompts = synth.zipf_prompts(spec.vocab, n, P, 78)
    slots = np.arange(n, dtype=np.uint32)
    print(f"serve scan: a refused session among {n}", flush=True)
    got = serve(make_model(art, False), prompts, slots, n, K, True, refuse=(K, 17))
    ref = serve(make_model(art, True), prompts, slots, n, K, True, refuse=(K, 17))
    assert got["status"][K, 17] == 1 and ref["status"][K, 17] == 1
    ok = np.ones(n, bool)
    ok[17] = False
    np.testing.assert_array_equal(got["status"], ref["status"])
    np.testing.assert_array_equal(got["reply"][ok], ref["reply"][ok])
    np.testing.assert_array_equal(got["state"], ref["state"])


def test_job_buffers_grow_and_the_memory_off_equals_the_fused_writer():
    """One model serving 40 sessions, then 600 (the job buffers grow between launches), then 40
    again; and a model created with the writer's memory off (every step a job). Each against the
    fused writer's launches from the same state."""
    spec = SHAPES["c2"]
    art = synth.make_artifact(spec, 4244)
    P, K = 10, 4
    print("serve scan: job buffers grow; writer memory off", flush=True)
    deferred, fused = make_model(art, False), make_model(art, True)
    for n in (40, 600, 40):
        prompts = synth.uniform_prompts(spec.vocab, n, P, 90 + n)
        slots = np.arange(n, dtype=np.uint32)[::-1].copy()
        got = serve(deferred, prompts, slots, n, K, True)
        ref = serve(fused, prompts, slots, n, K, True)
        for key in ("reply", "kept", "query", "state", "status"):
            np.testing.assert_array_equal(got[key], ref[key], err_msg=f"{n} {key}")
    os.environ["UOR_FBS_WRITER_MEMORY"] = "0"
    try:
        no_memory = make_model(art, False)
    finally:
        del os.environ["UOR_FBS_WRITER_MEMORY"]
    prompts = synth.uniform_prompts(spec.vocab, 64, P, 95)
    slots = np.arange(64, dtype=np.uint32)
    got = serve(no_memory, prompts, slots, 64, K, True)
    ref = serve(fused, prompts, slots, 64, K, True)
    for key in ("reply", "kept", "query", "state", "status"):
        np.testing.assert_array_equal(got[key], ref[key], err_msg=key)


def test_the_default_takes_the_scan_where_drawer_sizes_are_skewed():
    """Without the environment switch the drawers' sizes choose: C3's Zipf drawers (largest 512
    against a mean of 128) take the drawer-major scan, C2's uniform ones keep the writer in the
    step; either way a serving launch equals the batched decode."""
    for name in ("c3", "c2"):
        spec = SHAPES[name]
        art = synth.make_artifact(spec, 4245)
        n, P, K = 64, 8, 3
        prompts = (synth.zipf_prompts(spec.vocab, n, P, 79) if spec.zipf_drawers
                   else synth.uniform_prompts(spec.vocab, n, P, 79))
        model = hip.Model(art)
        got = serve(model, prompts, np.arange(n, dtype=np.uint32), n, K, True)
        want = model.decode(prompts, gen=K, want_state=False)["reply"]
        np.testing.assert_array_equal(got["reply"], want, err_msg=name)
