"""Write golden snap traces of the reference's own C++ twin of the FBS step.

Run in a container that has the reference checkout (the twin is compiled from its sources by
`make -C oracle ref` into oracle/_ref/, never committed):

    python tests/golden/make_golden_trace.py

For the golden cases whose artifacts snap a gate or the transition (and their unsnapped
siblings, whose traces are all 255), the twin's `fbs_host_trace_sequences`
(docs/labs/d11-exporter-float-trunk/instrument/src/host_kernel.cpp:31-49) gives every position's
snap trace: per layer the transition's root per lane, the output gate's root per lane, then the
feed-forward gate's root per 4 MLP channels (fbs_core.h:488-501). Kept whole for narrow
shapes, as a SHA-256 per sequence for wide ones, in tests/golden/trace/. Data only: the inputs
are the golden cases' own tokens (tests/golden/*.npz).
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "uor-r4_amd"))

import oracle  # noqa: E402
from uor_fbs import synth  # noqa: E402

CASES = [f"{b}_g{g}t{t}_seq" for b in ("small", "non_square", "tiny_gain") for g in (0, 1)
         for t in (0, 1)] + ["c3_twin_snapped"]


def main():
    if not oracle.twin_available():
        raise SystemExit("oracle/_ref/libfbs_twin.so is missing: run `make -C oracle ref`")
    manifest = json.load(open(os.path.join(HERE, "manifest.json")))
    out = {}
    for name in CASES:
        entry = manifest[name]
        spec = synth.Spec(**{k: tuple(v) if isinstance(v, list) else v for k, v in entry["spec"].items()})
        art = synth.make_artifact(spec, entry["seed"])
        tokens = np.load(os.path.join(HERE, f"{name}.npz"))["tokens"]
        st, _, _, _, trace = oracle.twin_trace_sequences(art, tokens)
        assert st == 0, (name, st)
        rec = {"stride": int(trace.shape[-1])}
        if spec.width <= 64:
            np.savez_compressed(os.path.join(HERE, "trace", f"{name}.npz"), trace=trace)
        else:
            rec["trace_sha256"] = [hashlib.sha256(t.tobytes()).hexdigest() for t in trace]
        rec["roots_seen"] = int(len(np.unique(trace)))
        out[name] = rec
        print(name, trace.shape, "distinct bytes", rec["roots_seen"])
    with open(os.path.join(HERE, "trace", "manifest.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
