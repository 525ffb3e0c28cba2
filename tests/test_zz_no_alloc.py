"""The allocation-free decode (uor_fbs_decode_noalloc_async, include/uor_fbs.h) against
uor_fbs_decode_async: same replies, exported state, window rows, positions and statuses, bit for
bit, through the C ABI on device buffers. Two calls in a row on each model, the second smaller
and resumed from the first's state, so the shared scratch array carries the first call's
contents into the second. The width-512 model needs more window ring than the scratch holds for
its batch, so its launches run on fewer blocks than the allocating entry point's."""

from dataclasses import replace

import numpy as np
import pytest

from uor_fbs import hip, synth
from uor_fbs.hipmem import DeviceArray

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("block_waves")]


def _decode(model, entry, prompts, gen, resume=None):
    """One call of `entry` on device buffers; resume = (state, history, position) host arrays."""
    S, plen = prompts.shape
    dev = model.device

    def upload(a, dtype):
        d = DeviceArray(a.shape, dtype, dev)
        d.upload(a)
        return d

    d_prompts = upload(prompts, np.uint32)
    reply = DeviceArray((S, gen + 1), np.uint32, dev)
    state = DeviceArray((S, model.state_words), np.int64, dev)
    hist = DeviceArray((S, model.history_words), np.int32, dev)
    pos = DeviceArray(S, np.uint32, dev)
    status = DeviceArray(S, np.int32, dev)
    ins = [None, None, None]
    keep = []
    if resume is not None:
        keep = [upload(resume[0], np.int64), upload(resume[1], np.int32), upload(resume[2], np.uint32)]
        ins = [k.ptr for k in keep]
    # The null stream: the blocking downloads below wait for the launch.
    hip._check(getattr(hip.lib(), entry)(model.handle, d_prompts.ptr, S, plen, gen, reply.ptr,
                                         *ins, state.ptr, hist.ptr, pos.ptr, status.ptr, None))
    return dict(reply=reply.download(), state=state.download(), history=hist.download(),
                position=pos.download(), status=status.download())


def _check_pair(model, prompts, gen, resume=None):
    want = _decode(model, "uor_fbs_decode_async", prompts, gen, resume)
    got = _decode(model, "uor_fbs_decode_noalloc_async", prompts, gen, resume)
    assert (want["status"] == 0).all()
    for key in ("reply", "state", "history", "position", "status"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    return want


@pytest.mark.parametrize("name,spec,seed,first,second", [
    ("c2-like", replace(synth.CONFIGS["c2"], context=64), 301, (300, 7, 9), (37, 3, 5)),
    # 500 sequences of width 512 and window 32: the scratch holds 321 (paired) or 341 blocks.
    ("c5-like", replace(synth.CONFIGS["c5"], context=32), 305, (500, 4, 5), (200, 2, 3)),
])
def test_noalloc_decode_equals_the_allocating_decode(name, spec, seed, first, second):
    art = synth.make_artifact(spec, seed)
    model = hip.Model(art)
    S1, P1, G1 = first
    S2, P2, G2 = second
    print(f"noalloc {name}: {S1} x ({P1} + {G1}), then {S2} x ({P2} + {G2}) resumed", flush=True)
    p1 = synth.uniform_prompts(spec.vocab, S1, P1, seed + 1)
    a = _check_pair(model, p1, G1)
    p2 = synth.uniform_prompts(spec.vocab, S2, P2, seed + 2)
    _check_pair(model, p2, G2, resume=(a["state"][:S2], a["history"][:S2], a["position"][:S2]))
    model.close()
