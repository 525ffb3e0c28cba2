"""Write golden vectors of the reference's own C++ twin of the FBS step.

Run in a container that has the reference checkout (the twin is compiled from its sources by
`make -C oracle ref` into oracle/_ref/, never committed):

    python tests/golden/make_golden.py

Each case is a seeded artifact of this repository's generator (rebuilt from its spec and seed
by the tests, whose table digest is recorded to catch generator drift), a block of input
tokens, and the twin's outputs at every position (`fbs_host_sequences`,
docs/labs/d11-exporter-float-trunk/instrument/src/host_kernel.cpp:16-29): chosen tokens, kept
cells and the Q12 query (kept whole for narrow shapes, as a SHA-256 per sequence for wide
ones). The fixtures are data: inputs and expected outputs.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
from dataclasses import asdict, replace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "uor-r4_amd"))

import oracle  # noqa: E402
sys.path.insert(0, os.path.join(ROOT, "tests"))
from make_golden_digest import artifact_digest  # noqa: E402
from uor_fbs import synth  # noqa: E402

SNAPS = [(True, True), (False, False), (True, False), (False, True)]


def cases():
    out = []
    for name, spec, seed in (("small", synth.SMALL, 20261025), ("non_square", synth.NON_SQUARE, 20261026),
                             ("tiny_gain", synth.TINY, 20261026)):
        for rg, rt in SNAPS:
            sp = replace(spec, raw_gates=rg, raw_transition=rt)
            # single tokens across the whole vocabulary, then 16 sequences of full context
            out.append((f"{name}_g{int(rg)}t{int(rt)}_single", sp, seed,
                        np.arange(sp.vocab, dtype=np.uint32).reshape(-1, 1)))
            out.append((f"{name}_g{int(rg)}t{int(rt)}_seq", sp, seed,
                        synth.uniform_prompts(sp.vocab, 16, sp.context, 7)))
    long = replace(synth.NON_SQUARE, context=64)
    out.append(("non_square_64", long, 20261027, synth.uniform_prompts(long.vocab, 8, 64, 11)))
    # Reference-exact twins of BASELINE's configs (256 cells, t mod 256, window 3, i16).
    c12 = synth.reference_twin(synth.CONFIGS["c2"])
    c12 = replace(c12, context=64)
    out.append(("c2_twin", c12, 2026120201, synth.uniform_prompts(c12.vocab, 6, 64, 12)))
    c3 = replace(synth.reference_twin(synth.CONFIGS["c3"]), context=48)
    out.append(("c3_twin", c3, 2026120203, synth.zipf_prompts(c3.vocab, 4, 48, 13)))
    c3s = replace(c3, raw_gates=False, raw_transition=False)
    out.append(("c3_twin_snapped", c3s, 2026120203, synth.zipf_prompts(c3s.vocab, 4, 48, 14)))
    c5 = replace(synth.reference_twin(synth.CONFIGS["c5"]), context=24, layers=2)
    out.append(("c5_twin", c5, 2026120205, synth.uniform_prompts(c5.vocab, 2, 24, 15)))
    # The twin reads any vocabulary: 32768 rows, 128 per cell.
    big = replace(c3, vocab=32768, context=16)
    out.append(("vocab32768_twin", big, 2026120206, synth.zipf_prompts(big.vocab, 3, 16, 16)))
    return out


def main():
    if not oracle.twin_available():
        raise SystemExit("oracle/_ref/libfbs_twin.so is missing: run `make -C oracle ref`")
    manifest = {}
    for name, spec, seed, tokens in cases():
        art = synth.make_artifact(spec, seed)
        st, tok, kept, query = oracle.twin_sequences(art, tokens)
        assert st == 0, (name, st)
        entry = dict(spec=asdict(spec), seed=seed, artifact_sha256=artifact_digest(art))
        arrays = dict(tokens=tokens, out_tokens=tok, out_kept=kept)
        if spec.width <= 64:
            arrays["out_query"] = query
        else:
            entry["query_sha256"] = [hashlib.sha256(q.tobytes()).hexdigest() for q in query]
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        manifest[name] = entry
        print(name, tokens.shape, "distinct tokens", len(np.unique(tok)))
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
