"""The HIP path on trained FBS artifacts the reference holds (tests/golden/trained/, read by the
UORLUT01 reader): every position's token, kept drawers and Q12 query against the reference
twin's golden vectors, and greedy decode with the exported session against the oracle."""

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from uor_fbs import synth, uorlut
from uor_fbs.hip import Model

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("block_waves")]

TRAINED = os.path.join(GOLDEN, "trained")
MANIFEST = json.load(open(os.path.join(TRAINED, "manifest.json")))


def load(name):
    entry = MANIFEST[name]
    art = uorlut.load(os.path.join(TRAINED, entry["artifact"]))
    return entry, art, np.load(os.path.join(TRAINED, f"{name}.npz"))


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_trained_artifact_matches_twin(name):
    entry, art, g = load(name)
    print(f"trained {name} tokens {g['tokens'].shape}", flush=True)
    tok, kept, query = Model(art).sequences(g["tokens"])
    np.testing.assert_array_equal(tok, g["out_tokens"])
    np.testing.assert_array_equal(kept, g["out_kept"])
    assert [hashlib.sha256(q.tobytes()).hexdigest() for q in query] == entry["query_sha256"]


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_trained_artifact_decode_matches_oracle(name):
    _, art, _ = load(name)
    prompts = synth.uniform_prompts(art.spec.vocab, 64, 32, 401)
    print(f"trained decode {name} prompts {prompts.shape}", flush=True)
    got = Model(art).decode(prompts, gen=art.spec.context - 32)
    want = oracle.decode(art, prompts[:8], art.spec.context - 32, threads=8)
    for key in ("reply", "state", "history", "position"):
        np.testing.assert_array_equal(got[key][:8], want[key], err_msg=key)
    assert len(np.unique(got["reply"])) > 16
