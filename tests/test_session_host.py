"""Host logic of the serving sessions (uor_fbs/session.py) that needs no GPU: restore_state's
refusals (stack/session.rs:2876-3090) and the JSON size bound (session.rs:2281-2345), checked
against snapshots built by hand."""

import dataclasses
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN
from uor_fbs import synth, uorlut
from uor_fbs.session import (TRACE_UNSET, ModelInfo, SessionError, SnapTrace,
                             max_serialized_session_bytes, model_identity, transition_roots,
                             validate_restore)
from uor_fbs.session_codec import (STACK_SESSION_SCHEMA, ReadLayer, RecurrenceLayer,
                                   SerializedStackSession)

INFO = ModelInfo(sha256="ab" * 32, vocab=100, width=32, layers=2, window=3, context=16)


def saved(pos=3, **kw) -> SerializedStackSession:
    d, w = INFO.width, INFO.window
    s = SerializedStackSession(
        schema=STACK_SESSION_SCHEMA, version=1, artifact_sha256=INFO.sha256, position=pos,
        cache_at=pos * d, lift_at=pos, logits=[0] * INFO.vocab if pos else [],
        tokens=list(range(1, pos + 1)),
        layers=[RecurrenceLayer([l] * d, [l] * (w * d)) for l in range(INFO.layers)])
    return dataclasses.replace(s, **kw)


def refused(kind, s):
    with pytest.raises(SessionError) as e:
        validate_restore(INFO, s)
    assert e.value.kind == kind, e.value


def test_a_valid_snapshot_passes():
    validate_restore(INFO, saved())
    validate_restore(INFO, saved(pos=0))
    validate_restore(INFO, saved(pos=INFO.context, tokens=[1] * INFO.context))
    validate_restore(INFO, saved(snap_trace=[]))  # an empty trace on an unsnapped model


def test_each_refusal():
    refused("Schema", saved(schema="uor-r4.stack-session/2"))
    refused("Schema", saved(version=2))
    refused("Numerics", saved(artifact_sha256="cd" * 32))
    refused("ContentReadout", saved(content_readout_sha256="cd" * 32))
    refused("ContextFull", saved(pos=INFO.context + 1, tokens=[1] * (INFO.context + 1)))
    refused("SessionState", saved(cache_at=1))
    refused("SessionState", saved(lift_at=4))
    refused("SessionState", saved(layers=saved().layers[:1]))
    refused("SessionState", saved(logits=[0] * 3))
    refused("SessionState", saved(pos=0, logits=[0]))
    refused("SessionState", saved(tokens=[1, 2]))
    refused("SessionState", saved(pointer_keys=[1]))
    refused("SessionState", saved(mixture=[1]))
    refused("Token", saved(tokens=[1, 2, INFO.vocab]))
    refused("SessionState", saved(snap_trace=[0, 1]))
    refused("SessionState", saved(layers=[RecurrenceLayer([0] * 32, [0] * 96), ReadLayer([], [], [])]))
    refused("SessionState", saved(layers=[RecurrenceLayer([0] * 31, [0] * 96)] * 2))
    refused("SessionState", saved(layers=[RecurrenceLayer([0] * 32, [0] * 64)] * 2))


def test_snapped_traces():
    info = dataclasses.replace(INFO, snapped=True)
    lanes = info.width // 4
    ok = saved(snap_trace=[])
    with pytest.raises(SessionError) as e:  # the wrong length
        validate_restore(info, ok)
    assert e.value.kind == "SessionState"
    validate_restore(info, saved(snap_trace=[7] * (3 * lanes * info.layers)))
    with pytest.raises(SessionError) as e:
        validate_restore(info, saved(snap_trace=[120] * (3 * lanes * info.layers)))
    assert e.value.kind == "SessionState"
    validate_restore(info, saved(pos=0, tokens=[], logits=[], snap_trace=[]))


def test_size_bound():
    # Layers (W+1)·d·24 each, vocab·24 of logits, context·24 of tokens, 128 KiB of margin.
    assert max_serialized_session_bytes(INFO) == 2 * 4 * 32 * 24 + 100 * 24 + 16 * 24 + 131072
    snapped = dataclasses.replace(INFO, snapped=True)
    assert max_serialized_session_bytes(snapped) - max_serialized_session_bytes(INFO) == 16 * 8 * 2 * 24


def test_hamming_payload_caches():
    # One cache per read with payload-bringing type heads (an asking read and a read without
    # type weights keep none, hamming.rs:1678-1685); a type-head snapshot without them, or with
    # caches of other lengths, is refused (session.rs:2894-2910); the size bound counts them.
    spec = dataclasses.replace(synth.SMALL, context=16,
                               hamming=synth.HammingSpec(heads=2, depths=(1, 2), kept=4,
                                                         asks=(False, True)))
    art = synth.make_artifact(spec, 3)
    info = ModelInfo.of(art)
    d = spec.width
    assert info.hamming and info.payload_reads == (True, False) and info.payload_slots == 1
    assert [len(p) for p in info.payload_caches()] == [16 * d, 0]
    art.hamming_reads[0].weight[d:] = 0  # no type weights: no cache
    assert ModelInfo.of(art).payload_reads == (False, False)
    ok = dataclasses.replace(saved(), artifact_sha256=info.sha256)
    ok = dataclasses.replace(ok, layers=[RecurrenceLayer([0] * d, [0] * (info.window * d))] * info.layers,
                             logits=[0] * info.vocab, tokens=[1, 2, 3])
    validate_restore(info, dataclasses.replace(ok, hamming_payloads=info.payload_caches()))
    for bad in ([], [[0] * (16 * d)], [[0] * (16 * d - 1), []]):
        with pytest.raises(SessionError) as e:
            validate_restore(info, dataclasses.replace(ok, hamming_payloads=bad))
        assert e.value.kind == "Shape"
    plain = dataclasses.replace(info, payload_reads=(False, False))
    assert max_serialized_session_bytes(info) - max_serialized_session_bytes(plain) == 16 * d * 24


def test_a_place_read_session_is_not_restored():
    # The reference saves neither the place register nor the turns, and refuses the restore by
    # name (session.rs:2911-2919).
    info = dataclasses.replace(INFO, hamming=True, place=True)
    with pytest.raises(SessionError, match="place read") as e:
        validate_restore(info, saved())
    assert e.value.kind == "Shape"


def test_serving_identity():
    path = os.path.join(GOLDEN, "trained", "content_seed1_s7.uorlut")
    art = uorlut.load(path)
    assert model_identity(art) == hashlib.sha256(open(path, "rb").read()).hexdigest()
    info = ModelInfo.of(art)
    assert (info.width, info.layers, info.window, info.heads) == (256, 6, 3, 1)
    a = synth.make_artifact(synth.SMALL, 1)
    b = synth.make_artifact(synth.SMALL, 2)
    assert model_identity(a) == model_identity(synth.make_artifact(synth.SMALL, 1))
    assert model_identity(a) != model_identity(b) and len(model_identity(a)) == 64


def test_snap_trace_buffer():
    """SnapTrace::record (session.rs:2050-2058): stores in order while room is left, and keeps
    counting past the end; clear (session.rs:2728-2737) starts over with every entry unset."""
    t = SnapTrace(5, 2)
    t.record([3, 4])
    t.record([5, 6, 7, 8])
    assert t.selected.tolist() == [3, 4, 5, 6, 7] and t.written == 6 and t.origin_position == 2
    t.clear(7)
    assert t.selected.tolist() == [TRACE_UNSET] * 7 and t.written == 0 and t.origin_position == 0


def test_transition_roots_from_trace_bytes():
    """Per step, per layer, the first width/4 bytes (the transition's roots) of the layer's
    2 width/4 + mlp/4; the zero-quaternion byte reads as root 0."""
    layers, lanes, mlp4 = 2, 3, 2
    per_layer = 2 * lanes + mlp4
    tr = np.arange(3 * layers * per_layer, dtype=np.uint8).reshape(3, layers * per_layer) % 119
    tr[1, per_layer + 2] = 255
    got = transition_roots(tr, layers, lanes)
    want = [int(tr[s, l * per_layer + k]) for s in range(3) for l in range(layers) for k in range(lanes)]
    want[(1 * layers + 1) * lanes + 2] = 0
    assert got.tolist() == want
