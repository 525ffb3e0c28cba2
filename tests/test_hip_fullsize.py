"""The HIP path at BASELINE's full shapes, through properties that hold at any size, plus the
oracle on whole sequences drawn from the same batch.

- C1 decode at its full shape (batch 1, the 6-layer width-128 artifact, 256 + 256): the whole
  sequence against the oracle (reply, state, window, position).
- C3 decode at BASELINE's batch of 4,096 and C2 at 1,024, with their full prompt and reply
  lengths (1,024 + 1,024 and 512 + 512): the one-launch decode equals prefill + resumed decode through the exported
  session (save_state/restore_state, session.rs:2777-3290), equals a teacher-forced replay of
  its own reply through the rows kernel (decode = step_native fed its choices,
  fbs-toks.rs:1513-1533), and equals the oracle's decode (reply, state, window, position) on
  sampled sequences.
- C4 teacher-forced scoring at BASELINE's 1,048,576 rows of 128 tokens (Zipf prompts): the
  match count is additive over
  any split of the rows, equals the count recomputed from the per-position choices, and the
  choices equal the oracle's on sampled rows.
- C5 (width 512, int8 codes, window 32, 1,024 drawers probing 16) decode at its per-sequence
  length (4,096 + 4,096) over 2,048 sequences (more than the 1,024 resident blocks, so blocks
  take a second sequence), with the same properties and two whole sequences against the oracle;
  and at BASELINE's batch of 16,384 (16 sequences a block), five whole replies against the
  oracle.
- C3 and C5 oracle samples sit on both sides of every block boundary a launch has.
Every comparison is exact equality.
"""

from dataclasses import replace

import numpy as np
import pytest

import oracle
from uor_fbs import synth
from uor_fbs.hip import Model

pytestmark = pytest.mark.gpu


def _decode_properties(name, spec, seed, batch, prompt, gen, zipf, replay, picks, min_unique=16):
    spec = replace(spec, context=prompt + gen + 1)
    art = synth.make_artifact(spec, seed)
    make = synth.zipf_prompts if zipf else synth.uniform_prompts
    prompts = make(spec.vocab, batch, prompt, seed + 1)
    print(f"{name}: batch {batch} prompt {prompt} gen {gen}", flush=True)
    model = Model(art)
    full = model.decode(prompts, gen=gen)
    assert len(np.unique(full["reply"])) > min_unique  # not degenerate
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

    # The oracle on whole sequences of the batch.
    pick = np.asarray(picks, np.int64)
    print(f"{name}: oracle on sequences {list(pick)}", flush=True)
    want = oracle.decode(art, prompts[pick], gen, threads=min(16, len(pick)))
    assert want["status"] == 0
    for key in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(full[key][pick], want[key], err_msg=key)


def test_c1_decode_full_size():
    # One sequence: its reply may settle on a repeated token, so no spread is asked of it.
    _decode_properties("c1", synth.CONFIGS["c1"], 2026120201, batch=1, prompt=256, gen=256,
                       zipf=False, replay=1, picks=[0], min_unique=0)


def test_c3_decode_full_size():
    _decode_properties("c3", synth.CONFIGS["c3"], 2026120203, batch=4096, prompt=1024, gen=1024,
                       zipf=True, replay=64, picks=[0, 1023, 1024, 2047, 2048, 4095])


def test_c2_decode_full_size():
    _decode_properties("c2", synth.CONFIGS["c2"], 2026120202, batch=1024, prompt=512, gen=512,
                       zipf=False, replay=64, picks=np.linspace(0, 1023, 8).astype(np.int64))


@pytest.mark.timeout(400)
def test_c5_decode_full_length():
    _decode_properties("c5", synth.CONFIGS["c5"], 2026120205, batch=2048, prompt=4096, gen=4096,
                       zipf=False, replay=8, picks=[0, 2047])


@pytest.mark.timeout(900)
def test_c5_decode_full_batch():
    # BASELINE's C5 batch: 16,384 sequences of 4,096 + 4,096 (16 a resident block), replies only;
    # the oracle on sequences at both ends and on both sides of the first block boundary.
    spec = replace(synth.CONFIGS["c5"], context=4096 + 4096 + 1)
    art = synth.make_artifact(spec, 2026120205)
    batch = 16384
    prompts = synth.uniform_prompts(spec.vocab, batch, 4096, 2026120206)
    print(f"c5: batch {batch} prompt 4096 gen 4096", flush=True)
    full = Model(art).decode(prompts, gen=4096, want_state=False)
    assert len(np.unique(full["reply"])) > 16
    pick = np.array([0, 1023, 1024, 8191, 16383], np.int64)
    print(f"c5: oracle on sequences {list(pick)}", flush=True)
    want = oracle.decode(art, prompts[pick], 4096, threads=len(pick), want_state=False)
    assert want["status"] == 0
    np.testing.assert_array_equal(full["reply"][pick], want["reply"])


def test_c4_scoring_rows():
    # BASELINE's C4 shape: 1,048,576 Zipf rows of 128 tokens (about 13 s a pass on MI355X).
    spec = synth.CONFIGS["c4"]
    art = synth.make_artifact(spec, 2026120204)
    n = 1 << 20
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
    pick = np.concatenate([np.linspace(0, n - 1, 510).astype(np.int64), [131071, 131072]])
    st, want_matches, want_argmin = oracle.score(art, rows[pick], threads=16)
    assert st == 0
    np.testing.assert_array_equal(argmin[pick], want_argmin)
    assert want_matches == int((argmin[pick, :-1] == rows[pick, 1:]).sum())
