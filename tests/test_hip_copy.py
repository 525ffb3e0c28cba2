"""The HIP copy heads' Hamming read (uor_copy_mean_rows) against the reference's copy-rule
tests (hamming.rs:705-1058, literal positions and means) and against the oracle, stream for
stream and bit for bit: every rule, copy key 1 and 2 heads, reply markers and the caller's
opening flags, streams from empty to the 4,096-token stride."""

import numpy as np
import pytest

import copy_cases as K
import oracle
from uor_fbs.copy import RULES, CopyHeads

pytestmark = pytest.mark.gpu


def test_the_reference_copy_rule_tests_on_the_gpu():
    print("copy rule tests", flush=True)
    made = []

    def make(kept, rule, **kw):
        h = CopyHeads(K.heads(kept, rule, **kw))
        made.append(h)
        return h
    try:
        K.check_rust_tests(make)
    finally:
        for h in made:
            h.close()


@pytest.mark.parametrize("rule", sorted(RULES))
@pytest.mark.parametrize("shape", [(300, 96, 4, 8, 40, 200), (5000, 512, 8, 32, 4096, 64),
                                   (64, 1024, 16, 1, 300, 40)])
def test_random_streams_match_the_oracle(rule, shape):
    vocab, width, copy, kept, stride, rows = shape
    heads = K.random_heads(RULES[rule] * 7 + width, vocab=vocab, width=width, copy=copy,
                           kept=kept, rule=rule)
    tok, lens, opening = K.random_streams(RULES[rule] + width, vocab, rows, stride)
    print(f"copy {rule} {shape}", flush=True)
    gpu = CopyHeads(heads)
    try:
        out, found, chosen = gpu.mean_rows(tok, lens, opening)
    finally:
        gpu.close()
    w_out, w_found, w_chosen = oracle.copy_mean_rows(heads, tok, lens, opening)
    np.testing.assert_array_equal(chosen, w_chosen)
    np.testing.assert_array_equal(found, w_found)
    np.testing.assert_array_equal(out, w_out)
    assert found.sum() > rows // 4


def test_vocab_codes_match_the_restatement():
    from uor_fbs.copy import vocab_codes
    rng = np.random.default_rng(8)
    table = rng.integers(-32768, 32768, (500, 256)).astype(np.int16)
    table[:5] = 0                                   # points on the sign boundary
    rot = rng.integers(-(1 << 31), 1 << 31, 256, dtype=np.int64).astype(np.int32)
    rot[:4] = 0                                     # a zero quaternion: the unit of nothing
    print("copy vocab codes", flush=True)
    got = vocab_codes(rot, table, 8, 4)
    want = oracle.copy_vocab_codes(rot, table, 8, 4)
    np.testing.assert_array_equal(got, want)
    got2 = vocab_codes(rot[:128], table[:, :128], 2, 1)
    np.testing.assert_array_equal(got2, oracle.copy_vocab_codes(rot[:128], table[:, :128], 2, 1))


def test_device_buffers_and_a_stream_outside_the_vocabulary_reads_nothing():
    # uor_copy_mean_rows_async over device arrays on the default stream: a stream holding a
    # token outside the vocabulary (the host call refuses it) reads nothing; the others equal
    # the oracle. The same for lengths outside 0..stride.
    from uor_fbs import copy as cp
    from uor_fbs.hipmem import DeviceArray
    heads = K.random_heads(5, vocab=100, width=64, copy=2, kept=4)
    tok, lens, _ = K.random_streams(6, 100, 12, 30)
    tok[3, 2] = 100
    lens[3] = max(lens[3], 5)
    lens[4] = 31                                    # longer than the stride
    print("copy device buffers", flush=True)
    gpu = CopyHeads(heads)
    try:
        dt, dl = DeviceArray(tok.shape, np.uint32), DeviceArray(lens.shape, np.int32)
        do, df = DeviceArray((12, 64), np.int64), DeviceArray(12, np.uint8)
        dt.upload(tok)
        dl.upload(lens)
        assert cp.lib().uor_copy_mean_rows_async(gpu.handle, dt.ptr, dl.ptr, None, 12, 30,
                                                 do.ptr, df.ptr, None, None) == 0
        out, found = do.download(), df.download().astype(bool)
    finally:
        gpu.close()
    assert not found[3] and not found[4] and not out[3].any() and not out[4].any()
    keep = [r for r in range(12) if r not in (3, 4)]
    w_out, w_found, _ = oracle.copy_mean_rows(heads, tok[keep], lens[keep])
    np.testing.assert_array_equal(out[keep], w_out)
    np.testing.assert_array_equal(found[keep], w_found)
