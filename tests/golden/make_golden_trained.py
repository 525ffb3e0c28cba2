"""Golden vectors of the reference's own C++ twin on trained FBS artifacts the reference holds.

Run where the reference checkout is present (the twin is compiled from its sources by
`make -C oracle ref` into oracle/_ref/, never committed):

    python tests/golden/make_golden_trained.py

Two trained `UORLUT01` containers (one turn-memory `lut-stack/7`, one point-key `lut-stack/8`;
V 4,096, d 256, m 384, six layers, raw gates and transition, eight kept cells) are copied as data
fixtures into tests/golden/trained/ with their SHA-256 and source path. For each, the twin's
`fbs_host_sequences` (docs/labs/d11-exporter-float-trunk/instrument/src/host_kernel.cpp:16-29)
gives every position's token, kept cells and Q12 query on: seeded uniform token rows of full
context, and greedy chains (a prompt followed by the oracle's own decode, which the twin run
teacher-forced must reproduce). Queries are kept as a SHA-256 per row.
"""

from __future__ import annotations

import hashlib
import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "uor-r4_amd"))

import oracle  # noqa: E402
from uor_fbs import synth, uorlut  # noqa: E402

REFERENCE = os.environ.get("UOR_REFERENCE", "/root/reference")
SOURCES = {
    "content_seed1_s7": "docs/labs/cpu-training-pilot-content-serving-2026-11-04/evidence-attempt-1/"
                        "seed-1/serving.uorlut",
    "pilot130_medoid_s8": "docs/loop/tasks/cpu-training-pilot/deepseek-130/evidence/"
                          "seed-1-repeat.point-medoid.uorlut",
}


def main():
    if not oracle.twin_available():
        raise SystemExit("oracle/_ref/libfbs_twin.so is missing: run `make -C oracle ref`")
    out_dir = os.path.join(HERE, "trained")
    os.makedirs(out_dir, exist_ok=True)
    manifest = {}
    for i, (name, rel) in enumerate(sorted(SOURCES.items())):
        src = os.path.join(REFERENCE, rel)
        dst = os.path.join(out_dir, f"{name}.uorlut")
        shutil.copyfile(src, dst)
        data = open(dst, "rb").read()
        art = uorlut.load(data)
        s = art.spec
        rows = synth.uniform_prompts(s.vocab, 4, s.context, 300 + i)
        prompts = synth.uniform_prompts(s.vocab, 2, 16, 310 + i)
        dec = oracle.decode(art, prompts, s.context - 16, threads=2, want_state=False)
        assert dec["status"] == 0
        chains = np.concatenate([prompts, dec["reply"][:, :-1]], axis=1)
        tokens = np.concatenate([rows, chains], axis=0).astype(np.uint32)
        st, tok, kept, query = oracle.twin_sequences(art, tokens)
        assert st == 0, (name, st)
        # The chains are the oracle's greedy decode, so the twin chooses the same replies.
        assert np.array_equal(tok[4:, 15:], dec["reply"]), name
        np.savez_compressed(os.path.join(out_dir, f"{name}.npz"), tokens=tokens, out_tokens=tok,
                            out_kept=kept)
        manifest[name] = dict(
            artifact=f"{name}.uorlut", artifact_sha256=hashlib.sha256(data).hexdigest(),
            source=rel, schema=json.loads(data[16:16 + int.from_bytes(data[8:16], "little")])["schema"],
            query_sha256=[hashlib.sha256(q.tobytes()).hexdigest() for q in query])
        print(name, tokens.shape, "distinct tokens", len(np.unique(tok)))
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
