"""The HIP path at BASELINE's full shapes, through properties that hold at any size, plus the
oracle on whole sequences drawn from the same batch.

- C3 and C2 decode at batch 1,024 with their full prompt and reply lengths (1,024 + 1,024 and
  512 + 512): the one-launch decode equals prefill + resumed decode through the exported
  session (save_state/restore_state, session.rs:2777-3290), equals a teacher-forced replay of
  its own reply through the rows kernel (decode = step_native fed its choices,
  fbs-toks.rs:1513-1533), and equals the oracle's decode (reply, state, window, position) on
  sampled sequences.
- C4 teacher-forced scoring rows (128 tokens, Zipf prompts): the match count is additive over
  any split of the rows, equals the count recomputed from the per-position choices, and the
  choices equal the oracle's on sampled rows.
- C5 (width 512, int8 codes, window 32, 1,024 drawers probing 16) decode at a reduced batch
  and length, with the same properties.
Every comparison is exact equality.
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import synth
from uor_fbs.hip import Model

pytestmark = pytest.mark.gpu


def _decode_properties(name, spec, seed, batch, prompt, gen, zipf, sample, replay):
    spec = replace(spec, context=prompt + gen + 1)
    art = synth.make_artifact(spec, seed)
    make = synth.zipf_prompts if zipf else synth.uniform_prompts
    prompts = make(spec.vocab, batch, prompt, seed + 1)
    print(f"{name}: batch {batch} prompt {prompt} gen {gen}", flush=True)
    model = Model(art)
    full = model.decode(prompts, gen=gen)
    assert len(np.unique(full["reply"])) > 16  # not degenerate
    np.testing.assert_array_equal(full["position"], np.full(batch, prompt + gen, np.uint32))

    # Prefill, then resume for the rest: the same replies and the same end session.
    pre = model.decode(prompts, gen=0)
    np.testing.assert_array_equal(pre["reply"][:, 0], full["reply"][:, 0])
    rest = model.decode(pre["reply"][:, -1:], gen=gen - 1, in_state=pre["state"],
                        in_history=pre["history"], in_position=pre["position"])
    np.testing.assert_array_equal(rest["reply"], full["reply"][:, 1:])
    for key in ("state", "history", "position"):
        np.testing.assert_array_equal(rest[key], full[key])

    # Teacher-forced replay of the reply: the choice at every fed position is the next token.
    rows = np.concatenate([prompts[:replay], full["reply"][:replay, :-1]], axis=1)
    tok, _, _ = model.sequences(rows, want_kept=False, want_query=False)
    np.testing.assert_array_equal(tok[:, prompt - 1:], full["reply"][:replay])

    # The oracle on whole sequences spread over the batch.
    pick = np.linspace(0, batch - 1, sample).astype(np.int64)
    want = oracle.decode(art, prompts[pick], gen, threads=min(16, sample))
    assert want["status"] == 0
    for key in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(full[key][pick], want[key], err_msg=key)


def test_c3_decode_full_size():
    _decode_properties("c3", synth.CONFIGS["c3"], 2026120203, batch=1024, prompt=1024, gen=1024,
                       zipf=True, sample=8, replay=64)


def test_c2_decode_full_size():
    _decode_properties("c2", synth.CONFIGS["c2"], 2026120202, batch=1024, prompt=512, gen=512,
                       zipf=False, sample=8, replay=64)


def test_c5_decode_reduced_batch():
    _decode_properties("c5", synth.CONFIGS["c5"], 2026120205, batch=256, prompt=256, gen=256,
                       zipf=False, sample=2, replay=8)


def test_c4_scoring_rows():
    spec = synth.CONFIGS["c4"]
    art = synth.make_artifact(spec, 2026120204)
    n = 131072
    rows = synth.zipf_prompts(spec.vocab, n, 128, 2026120205)
    print(f"c4: {n} rows x 128", flush=True)
    model = Model(art)
    total, argmin = model.score(rows)
    # The count is the number of positions whose choice is the row's next token.
    assert total == int((argmin[:, :-1] == rows[:, 1:]).sum())
    assert total > 0
    # Additive over a split of the rows, and the choices do not depend on the batch.
    a, arg_a = model.score(rows[: n // 3])
    b, _ = model.score(rows[n // 3:], want_argmin=False)
    assert a + b == total
    np.testing.assert_array_equal(arg_a, argmin[: n // 3])
    # The oracle on sampled rows.
    pick = np.linspace(0, n - 1, 512).astype(np.int64)
    st, want_matches, want_argmin = oracle.score(art, rows[pick], threads=16)
    assert st == 0
    np.testing.assert_array_equal(argmin[pick], want_argmin)
    assert want_matches == int((argmin[pick, :-1] == rows[pick, 1:]).sum())
