"""The artifact digest the golden manifest records (shared with tests/golden/make_golden.py)."""

import hashlib

import numpy as np


def artifact_digest(art) -> str:
    h = hashlib.sha256()
    for ly in art.layers:
        for a in (ly.rec_gain, ly.mlp_gain, ly.taps, ly.conv_bias, ly.gate_bias, ly.decay_offset):
            h.update(np.ascontiguousarray(a).tobytes())
        for name in sorted(ly.maps):
            for a in ly.maps[name]:
                h.update(np.ascontiguousarray(a).tobytes())
    h.update(art.final_gain.tobytes())
    h.update(art.writer_table.tobytes())
    return h.hexdigest()
