"""The part clocks (uor_fbs_decode_parts_async, after the reference's measure_fbs_step_parts,
session.rs:4721-4779): the instrumented paired kernel decodes exactly as the served one (replies,
exported state, window and position), counts every step, and times every phase each wave runs.
"""

from dataclasses import replace

import numpy as np
import pytest

from uor_fbs import hip, synth
from uor_fbs.hip import FbsError, Model

pytestmark = pytest.mark.gpu

SHAPES = {
    "c2": (replace(synth.CONFIGS["c2"], context=40), 61, lambda s: synth.uniform_prompts(s.vocab, 5, 12, 62)),
    "c3": (replace(synth.CONFIGS["c3"], context=40), 63, lambda s: synth.zipf_prompts(s.vocab, 4, 12, 64)),
    "c5": (replace(synth.CONFIGS["c5"], context=24, layers=2), 65,
           lambda s: synth.uniform_prompts(s.vocab, 2, 8, 66)),
    "snapped": (replace(synth.CONFIGS["c2"], context=24, layers=2, raw_gates=False,
                        raw_transition=False), 67, lambda s: synth.uniform_prompts(s.vocab, 3, 8, 68)),
}

# Phases that every generating step runs on each wave (wave 0: the recurrence chain; wave 1:
# the window ring).
WAVE0 = ["embed", "norm_rec", "transition", "transport", "requant_rec", "residual_rec",
         "norm_mlp", "mlp", "requant_mlp", "residual_mlp", "final", "select", "step"]
WAVE1 = ["loads", "transition", "transport", "mlp", "requant_mlp"]


@pytest.fixture
def paired(monkeypatch):
    monkeypatch.setenv("UOR_FBS_BLOCK_WAVES", "2")


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_parts_decode_equals_the_decode(name, paired):
    spec, seed, make = SHAPES[name]
    art = synth.make_artifact(spec, seed)
    prompts = make(spec)
    gen = spec.context - prompts.shape[1] - 1
    print(f"parts {name}: prompts {prompts.shape} gen {gen}", flush=True)
    model = Model(art)
    assert model.block_waves(len(prompts)) == 2
    want = model.decode(prompts, gen)
    got = model.decode_parts(prompts, gen)
    for k in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    # Resumed from the exported session: the same again.
    half = model.decode(prompts, 2)
    more = model.decode_parts(half["reply"][:, -1:], gen - 3, half["state"], half["history"],
                              half["position"])
    np.testing.assert_array_equal(more["reply"], want["reply"][:, 3:])
    np.testing.assert_array_equal(more["state"], want["state"])

    names = hip.part_names()
    parts = got["parts"]
    assert parts.shape == (len(prompts), 2, len(names))
    np.testing.assert_array_equal(got["steps"], prompts.shape[1] + gen)
    assert (got["ticks"] > 0).all()
    for w, need in ((0, WAVE0), (1, WAVE1)):
        for n in need:
            assert (parts[:, w, names.index(n)] > 0).all(), (w, n)
    # Wave 0's laps tile its run: their sum is its time between the first and last clock read,
    # which the 100 MHz ticks bound from above at any shader clock below 10 GHz.
    assert (parts[:, 0].sum(-1) < got["ticks"].astype(np.float64) * 100).all()


def test_parts_refuse_a_one_wave_model(monkeypatch):
    monkeypatch.setenv("UOR_FBS_BLOCK_WAVES", "1")
    spec, seed, make = SHAPES["c2"]
    model = Model(synth.make_artifact(spec, seed))
    with pytest.raises(FbsError):
        model.decode_parts(make(spec), 4)
