"""CPU checks of the product library: it loads, exports every entry point include/uor_fbs.h
declares, and its structs have the reference's layout; and the kernels' exact integer arithmetic
(uor-r4_amd/csrc/fbs_int.h, compiled for the host into libuor_fbs_hostprims.so) equals the
oracle's and Python's exact integers over many inputs."""

import ctypes as C
import math
import os
import random
import re

import numpy as np
import pytest

import oracle
from conftest import ROOT
from uor_fbs import hip, tables
from uor_fbs.cabi import ExtS, LayerS, ModelS

# UOR_HOSTPRIMS_LIB selects another build of the host arithmetic (the sanitizer build,
# tests/test_sanitized_cpu.py).
HP_PATH = os.environ.get("UOR_HOSTPRIMS_LIB") or os.path.join(ROOT, "uor-r4_amd", "lib",
                                                              "libuor_fbs_hostprims.so")
P = C.c_void_p
U64 = (1 << 64) - 1


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "uor_fbs.h")).read()
    return set(re.findall(r"\b(uor_fbs_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_entry_point():
    L = hip.lib()
    names = declared_symbols()
    assert names == set(hip.SYMBOLS)
    for name in names:
        assert hasattr(L, name), name
    assert L.uor_fbs_abi_version() == 3


def test_struct_layout_matches_the_reference_image():
    L = hip.lib()
    assert L.uor_fbs_sizeof_model() == C.sizeof(ModelS)
    assert L.uor_fbs_sizeof_layer() == C.sizeof(LayerS)
    assert L.uor_fbs_sizeof_ext() == C.sizeof(ExtS)
    if oracle.twin_available():  # the reference's own fbs_host_sizeof_* (host_kernel.cpp:8-9)
        T = oracle.twin()
        assert T.fbs_host_sizeof_model() == C.sizeof(ModelS)
        assert T.fbs_host_sizeof_layer() == C.sizeof(LayerS)


def test_model_create_refuses_bad_images_without_a_device():
    """Validation runs before any device call: a bad image fails with a shape error."""
    from dataclasses import replace
    from uor_fbs import synth
    from uor_fbs.cabi import Image
    art = synth.make_artifact(synth.SMALL, 3)
    img = Image(art)
    img.model.width = 40
    h = P()
    assert hip.lib().uor_fbs_model_create(C.byref(img.model), None, 0, C.byref(h)) == 4
    assert b"width" in hip.lib().uor_fbs_last_error()
    img = Image(art)
    art.layers[0].rec_gain[3] = -32768  # not a grid code (kernels.rs:116-120)
    img = Image(art)
    assert hip.lib().uor_fbs_model_create(C.byref(img.model), None, 0, C.byref(h)) == 4
    assert b"grid code" in hip.lib().uor_fbs_last_error()
    art = synth.make_artifact(synth.SMALL, 3)
    art.layers[1].maps["mlp_up"][0][2] = 4  # atom outside 4 input blocks
    img = Image(art)
    assert hip.lib().uor_fbs_model_create(C.byref(img.model), None, 0, C.byref(h)) == 4
    assert b"atom" in hip.lib().uor_fbs_last_error()
    art = synth.make_artifact(replace(synth.SMALL, window=5), 3)
    img = Image(art)
    img.ext.wide_taps = None
    assert hip.lib().uor_fbs_model_create(C.byref(img.model), C.byref(img.ext), 0, C.byref(h)) == 4


def test_index_entry_points_refuse_bad_arguments_before_any_launch():
    """The CSR index's entry points check pointers, sizes, widths, alignment and k on the host
    and return UOR_FBS_ERR_ARGUMENT (3) without a launch; the workspace size is 16 header words
    plus 257 words per build tile and 257 totals; a tile is 512 tokens times the largest
    power of two up to 16 that leaves about 256 tiles."""
    L = hip.lib()
    fake = P(4096)  # never dereferenced: every call below is refused first
    odd = P(4100)   # a table pointer that is not 16-byte aligned
    mx = 1 << 30
    for count, tiles in ((1, 1), (512, 1), (513, 2), (65536, 128), (262144, 256),
                         (1 << 20, 256), (1 << 24, 2048), ((1 << 24) + 1, 2049)):
        assert L.uor_fbs_index_workspace_bytes(count) == 4 * (16 + 257 * (tiles + 1)), count
    build = L.uor_fbs_index_build_async
    assert build(None, 10, 32, fake, 0, fake, fake, fake, fake, fake, fake, None) == 3
    assert build(fake, 0, 32, fake, 0, fake, fake, fake, fake, fake, fake, None) == 3
    assert build(fake, mx + 1, 32, fake, 0, fake, fake, fake, fake, fake, fake, None) == 3
    for width in (8, 12, 30, 260):
        assert build(fake, 10, width, fake, 0, fake, fake, fake, fake, fake, fake, None) == 3
    assert build(odd, 10, 32, fake, 0, fake, fake, fake, fake, fake, fake, None) == 3
    assert build(fake, 10, 32, fake, 0, fake, fake, fake, fake, None, fake, None) == 3
    assert L.uor_fbs_index_update_async(fake, 10, 32, None, 0, fake, fake, fake, fake, fake, fake,
                                        None) == 3
    assert L.uor_fbs_index_remove_async(0, 0, fake, fake, fake, fake, fake, fake, None) == 3
    assert L.uor_fbs_index_remove_async(10, 0, fake, None, fake, fake, fake, fake, None) == 3
    assert L.uor_fbs_index_validate_async(fake, 10, 18, fake, fake, fake, fake, fake, fake, fake,
                                          None) == 3
    probe = L.uor_fbs_index_probe_async
    for k in (0, 17):
        assert probe(fake, 10, 32, fake, fake, 1, k, fake, fake, fake, fake, fake, fake, None) == 3
    assert probe(fake, 10, 32, fake, fake, 0, 8, fake, fake, fake, fake, fake, fake, None) == 3
    assert probe(fake, 10, 32, fake, fake, 1, 8, fake, None, fake, fake, fake, fake, None) == 3
    scan = L.uor_fbs_index_full_scan_async
    assert scan(fake, 10, 32, fake, fake, 1, 17, fake, fake, fake, fake, fake, None) == 3
    assert scan(fake, 10, 32, fake, None, 1, 8, fake, fake, fake, fake, fake, None) == 3


@pytest.fixture(scope="module")
def hp():
    if not os.path.exists(HP_PATH):
        pytest.skip("libuor_fbs_hostprims.so is not built")
    L = C.CDLL(HP_PATH)
    L.fbs_hp_isqrt128_many.argtypes = [P, P, P, C.c_uint64]
    L.fbs_hp_div_many.argtypes = [P, P, P, P, C.c_uint64]
    L.fbs_hp_rotation_many.argtypes = [P, C.c_uint64, C.c_uint64, P, C.c_uint64]
    L.fbs_hp_snap_rotation_many.argtypes = [P, P, C.c_uint64, P, C.c_uint64]
    L.fbs_hp_hamilton_check.argtypes = [P, P, C.c_uint64]
    L.fbs_hp_hamilton_check.restype = C.c_uint64
    L.fbs_hp_shift.argtypes = [C.c_int64, C.c_int32]
    L.fbs_hp_shift.restype = C.c_int64
    L.fbs_hp_grid_apply.argtypes = [C.c_int64, C.c_int16]
    L.fbs_hp_grid_apply.restype = C.c_int64
    L.fbs_hp_rms_norm_fine.argtypes = [P, C.c_uint32, C.c_int64, C.c_int32, P]
    return L


def _u64(vals):
    return np.array([v & U64 for v in vals], dtype=np.uint64)


def test_isqrt128_is_floor_sqrt(hp):
    rng = random.Random(1)
    vals = [0, 1, 2, 3, 4, (1 << 128) - 1, 1 << 127, 1 << 126, (1 << 126) - 1]
    for k in (1, 2, 3, (1 << 32) - 1, 1 << 32, 1 << 63, (1 << 64) - 1, (1 << 48) + 7):
        vals += [k * k - 1, k * k, min(k * k + 2 * k, (1 << 128) - 1)]
    vals += [rng.getrandbits(rng.randint(1, 128)) for _ in range(60000)]
    for _ in range(30000):  # perfect squares and their neighbours at every size
        k = rng.getrandbits(rng.randint(1, 64))
        vals += [k * k, max(k * k - 1, 0), min(k * k + 2 * k, (1 << 128) - 1)]
    hi, lo = _u64([v >> 64 for v in vals]), _u64(vals)
    out = np.zeros(len(vals), np.uint64)
    hp.fbs_hp_isqrt128_many(hi.ctypes.data_as(P), lo.ctypes.data_as(P), out.ctypes.data_as(P), len(vals))
    assert [int(x) for x in out] == [math.isqrt(v) for v in vals]


def test_div128_is_floor_division(hp):
    rng = random.Random(2)
    ns, ds = [], []
    for _ in range(60000):
        d = rng.getrandbits(rng.randint(1, 64)) or 1
        q = rng.getrandbits(rng.randint(0, 64))
        ns.append(q * d + rng.randint(0, d - 1))
        ds.append(d)
    for d in (1, 2, 3, 1 << 63, (1 << 63) + 1, U64, (1 << 32) - 1, 1 << 32):
        for q in (0, 1, U64, 1 << 63, 1 << 32):
            for r in (0, d - 1):
                ns.append(q * d + r)
                ds.append(d)
    ns.append(5), ds.append(0)  # zero divisor -> 0, as the reference's checked_div
    out = np.zeros(len(ns), np.uint64)
    hp.fbs_hp_div_many(_u64([n >> 64 for n in ns]).ctypes.data_as(P), _u64(ns).ctypes.data_as(P),
                       _u64(ds).ctypes.data_as(P), out.ctypes.data_as(P), len(ns))
    assert [int(x) for x in out] == [n // d if d else 0 for n, d in zip(ns, ds)]


def _raw_quaternions(rng, n):
    raw = []
    for i in range(n):
        sh = rng.randint(0, 31)
        q = [rng.randint(-(1 << 31), (1 << 31) - 1) >> sh for _ in range(4)]
        if i % 7 == 0:  # one nonzero axis, extremes, zero
            q = [0, 0, 0, 0]
            q[rng.randint(0, 3)] = rng.choice([1, -1, (1 << 31) - 1, -(1 << 31), rng.randint(-9, 9)])
        if i % 11 == 0:
            q = [rng.choice([-(1 << 31), (1 << 31) - 1]) for _ in range(4)]
        raw.append(q)
    return np.array(raw, np.int32)


@pytest.mark.parametrize("eps", [0, 4295])
@pytest.mark.parametrize("lam_exp", [31, 30, 27, 15])
def test_unit_rotation_equals_oracle(hp, eps, lam_exp):
    rng = random.Random(eps + lam_exp)
    raw = _raw_quaternions(rng, 20000)
    out = np.zeros((len(raw), 4), np.int64)
    hp.fbs_hp_rotation_many(raw.ctypes.data_as(P), 1 << lam_exp, eps, out.ctypes.data_as(P), len(raw))
    want = np.zeros(4, np.int64)
    ico = np.ascontiguousarray(tables.icosian_coefficients())
    for i in range(0, len(raw), 7):  # the oracle routine, one at a time
        oracle.lib().fbs_oracle_serve_rotation(ico.ctypes.data_as(P), 1, raw[i].ctypes.data_as(P),
                                               1 << lam_exp, eps, want.ctypes.data_as(P))
        assert list(out[i]) == list(want), raw[i]
    # and all of them against the closed form
    for i in range(len(raw)):
        v = [int(x) for x in raw[i]]
        norm = math.isqrt((sum(x * x for x in v) + eps) << 32)
        exp = [((1 << lam_exp) * ((-1 if x < 0 else 1) * ((abs(x) << 46) // norm if norm else 0))) >> 30 for x in v]
        assert list(out[i]) == exp


def test_snap_rotation_equals_oracle(hp):
    rng = random.Random(7)
    raw = _raw_quaternions(rng, 3000)
    ico = np.ascontiguousarray(tables.icosian_coefficients())
    out = np.zeros((len(raw), 4), np.int64)
    hp.fbs_hp_snap_rotation_many(ico.ctypes.data_as(P), raw.ctypes.data_as(P), 1 << 30,
                                 out.ctypes.data_as(P), len(raw))
    want = np.zeros(4, np.int64)
    for i in range(len(raw)):
        oracle.lib().fbs_oracle_serve_rotation(ico.ctypes.data_as(P), 0, raw[i].ctypes.data_as(P),
                                               1 << 30, 0, want.ctypes.data_as(P))
        assert list(out[i]) == list(want)


def test_hamilton32_equals_the_wide_product(hp):
    """The 32 x 32 partial-product form equals the i64 x i64 -> i128 Hamilton product for left
    operands of L1 norm <= 2^31 (unit quaternions times lambda), right operands anywhere."""
    rng = np.random.default_rng(3)
    n = 40000
    a = np.zeros((n, 4), np.int64)
    for i in range(n):
        v = rng.integers(-(1 << 30), 1 << 30, 4)
        s = np.abs(v).sum()
        if s > (1 << 31):
            v = v * (1 << 31) // s
        a[i] = v
    a[::5] = [[1 << 29, -(1 << 29), 1 << 29, -(1 << 29)]]
    a[1::5] = [[1 << 30, 0, 0, 0]]
    a = a.astype(np.int32)
    b = rng.integers(-(1 << 63), (1 << 63) - 1, (n, 4), dtype=np.int64)
    b[::3] = np.iinfo(np.int64).max
    b[1::3] = np.iinfo(np.int64).min
    b[2::7] = rng.integers(-(1 << 31), 1 << 31, (len(b[2::7]), 4))
    assert hp.fbs_hp_hamilton_check(a.ctypes.data_as(P), b.ctypes.data_as(P), n) == 0


def test_shift_and_grid_apply_equal_oracle(hp):
    rng = random.Random(4)
    for _ in range(20000):
        v = rng.randint(-(1 << 63), (1 << 63) - 1) >> rng.randint(0, 63)
        s = rng.randint(-70, 70)
        assert hp.fbs_hp_shift(v, s) == oracle.lib().fbs_oracle_shift(v, s)
        code = rng.choice([0, 1, -1]) * ((rng.randint(1, 127) << 4) | rng.randint(0, 15))
        assert hp.fbs_hp_grid_apply(v, code) == oracle.lib().fbs_oracle_grid_apply(v, code)


def test_rms_norm_fine_equals_oracle(hp):
    rng = random.Random(11)
    for trial in range(400):
        n = rng.choice([32, 64, 96, 256, 512])
        top = rng.randint(0, 31)
        x = np.array([rng.randint(-(1 << top), (1 << top)) for _ in range(n)], np.int32)
        if trial % 9 == 0:
            x[:] = 0
        if trial % 13 == 0:
            x[rng.randint(0, n - 1)] = -(1 << 31)
        eps_m, eps_e = rng.choice([(2814749767, -48), (0, 0), (1, 40), ((1 << 62), -2), (7, -70)])
        got = np.zeros(n, np.int64)
        want = np.zeros(n, np.int64)
        hp.fbs_hp_rms_norm_fine(x.ctypes.data_as(P), n, eps_m, eps_e, got.ctypes.data_as(P))
        oracle.lib().fbs_oracle_rms_norm_fine(x.ctypes.data_as(P), n, eps_m, eps_e, want.ctypes.data_as(P))
        np.testing.assert_array_equal(got, want)


def _near_square_quaternions(rng, n):
    """Quaternions whose sum of squares puts X 2^32 next to a perfect square m^2 (from either
    side), split greedily into four squares: the root and quotient corrections of unit_q30 run
    on exactly these inputs."""
    raw = []
    while len(raw) < n:
        m = (rng.getrandbits(64) >> rng.randint(0, 47)) | 1
        if rng.random() < 0.5:
            m = (m << 17) ^ rng.getrandbits(17)
        t = (m * m >> 32) + rng.randint(0, 2)
        if t >> 65:
            continue
        q, left = [], t
        for _ in range(4):
            v = min(math.isqrt(left), 1 << 31)
            left -= v * v
            q.append(-(1 << 31) if v == 1 << 31 else (v if rng.random() < 0.5 else -v))
        raw.append(q)
    return np.array(raw, np.int32)


@pytest.mark.parametrize("eps", [0, 4295])
def test_unit_q30_equals_the_128bit_form(hp, eps):
    # The kernels' branch-free unit quaternion against the 128-bit restoring form (both from
    # fbs_int.h, compiled for the host): random widths, near-perfect squares, equal components.
    hp.fbs_hp_unit_check.argtypes = [P, C.c_uint64, C.c_uint64]
    hp.fbs_hp_unit_check.restype = C.c_uint64
    rng = random.Random(91 + eps)
    nprng = np.random.default_rng(92 + eps)
    wide = (nprng.integers(-(1 << 31), 1 << 31, size=(400000, 4), dtype=np.int64)
            >> nprng.integers(0, 32, size=(400000, 1))).astype(np.int32)
    v = (nprng.integers(-(1 << 31), 1 << 31, size=100000, dtype=np.int64)
         >> nprng.integers(0, 32, size=100000)).astype(np.int32)
    ties = np.stack([v, v, np.zeros_like(v), np.where(v % 2 == 0, v, 0)], 1)
    for raw in (wide, ties, _near_square_quaternions(rng, 60000), _raw_quaternions(rng, 20000)):
        raw = np.ascontiguousarray(raw, np.int32)
        assert hp.fbs_hp_unit_check(raw.ctypes.data_as(P), eps, len(raw)) == 0


def test_div_2p96_is_the_exact_floor(hp):
    # floor(2^96 / s) for s in [2^34, 2^64): random widths, powers of two and their neighbours,
    # divisors of 2^96 - k for small k (quotients landing on and next to integers).
    hp.fbs_hp_div_2p96_many.argtypes = [P, P, C.c_uint64]
    rng = random.Random(97)
    ss = [rng.getrandbits(64) >> rng.randint(0, 30) for _ in range(200000)]
    ss += [(1 << e) + dlt for e in range(34, 64) for dlt in (-1, 0, 1) if (1 << e) + dlt >= 1 << 34]
    ss += [(1 << 64) - 1 - k for k in range(64)]
    for _ in range(20000):
        q = rng.randint(1 << 32, (1 << 62)) >> rng.randint(0, 28)
        s = (1 << 96) // q
        ss += [x for x in (s - 1, s, s + 1) if (1 << 34) <= x < (1 << 64)]
    ss = [x for x in ss if (1 << 34) <= x < (1 << 64)]
    arr = np.array(ss, dtype=np.uint64)
    out = np.zeros(len(arr), np.uint64)
    hp.fbs_hp_div_2p96_many(arr.ctypes.data_as(P), out.ctypes.data_as(P), len(arr))
    assert [int(o) for o in out] == [(1 << 96) // s for s in ss]


def test_norm_factor_pow2_equals_the_general_form(hp):
    # The kernels' RMSNorm factor for power-of-two widths against the general 128-bit form,
    # including sums whose root extension f sits at its limit and epsilons that wrap.
    hp.fbs_hp_norm_factor_check.argtypes = [P, P, C.c_uint64, C.c_uint32]
    hp.fbs_hp_norm_factor_check.restype = C.c_uint64
    rng = np.random.default_rng(98)
    n = 300000
    sums = (rng.integers(0, 2**63, n, dtype=np.uint64)
            >> rng.integers(0, 64, n).astype(np.uint64)).astype(np.uint64)
    r = rng.integers(1, 2**32, n // 2, dtype=np.uint64)
    sums[: n // 2] = (r * r + rng.integers(0, 3, n // 2, dtype=np.uint64)) << rng.integers(0, 8, n // 2).astype(np.uint64)
    eps = rng.choice(np.array([0, 1, 42950, 2**20, 2**40, 2**59, 2**60, 2**62, 2**63 - 1, -5],
                              dtype=np.int64), n)
    for log2n in (5, 8, 10):
        assert hp.fbs_hp_norm_factor_check(sums.ctypes.data_as(P), eps.ctypes.data_as(P), n, log2n) == 0


def test_grid_descriptor_forms_equal_grid_apply(hp):
    # Every valid grid code: the gains' grid_desc forms (32- and 64-bit inputs) and the window
    # taps' tap_desc form (both halves of a word) against grid_apply, on extremes and random
    # values of every width.
    hp.fbs_hp_grid_check.argtypes = [P, C.c_uint64]
    hp.fbs_hp_grid_check.restype = C.c_uint64
    rng = np.random.default_rng(99)
    v = np.concatenate([
        rng.integers(-2**63, 2**63 - 1, 600, dtype=np.int64) >> rng.integers(0, 63, 600),
        np.array([0, 1, -1, 2**31 - 1, -2**31, 2**31, -2**31 - 1, 2**57 - 1, -(2**57 - 1), 2**57,
                  -2**57, 2**63 - 1, -2**63, 127, 128, -128, -129, 255, 256], dtype=np.int64)])
    assert hp.fbs_hp_grid_check(v.ctypes.data_as(P), len(v)) == 0


def test_d11_library_exports_and_layout():
    """include/uor_d11.h: every declared entry point is exported; the model image and the row
    record have the layout the Python face writes and reads."""
    from uor_fbs import d11
    text = open(os.path.join(ROOT, "include", "uor_d11.h")).read()
    names = set(re.findall(r"\b(uor_d11_[a-z0-9_]+)\s*\(", text))
    assert names == set(d11.SYMBOLS)
    L = d11.lib()
    for name in names:
        assert hasattr(L, name), name
    assert L.uor_d11_abi_version() == 2
    assert L.uor_d11_sizeof_row_out() == d11.ROW_DTYPE.itemsize == 656


@pytest.mark.parametrize("edit,msg", [
    (lambda a: setattr(a.shape, "stages", a.shape.stages + 1), b"shape"),
    (lambda a: a.routes.__setitem__(0, 64), b"routes"),
    (lambda a: a.gates.__setitem__(1, 2), b"gates"),
    (lambda a: a.cells.__setitem__(3, a.cells[3] ^ 1), b"cells"),
    (lambda a: a.table.__setitem__((2, 1, 0), 1), b"orbit"),
    (lambda a: a.trunk.step_candidates.__setitem__(5, 16), b"step_candidates"),
    (lambda a: a.trunk.sparse["query_table"].__setitem__((0, 2), 0), b"zero count"),
])
def test_d11_model_create_refuses_without_a_device(edit, msg):
    """The library repeats the loader's checks before any device call."""
    from uor_fbs import d11
    art = d11.synthetic(vocabulary=64, context=12, seed=5, trunk_entries=50)
    art.table, art.cells, art.routes, art.gates = (art.table.copy(), art.cells.copy(),
                                                   art.routes.copy(), art.gates.copy())
    edit(art)
    m, keep = d11.c_model(art)
    h = P()
    assert d11.lib().uor_d11_model_create(C.byref(m), 0, C.byref(h)) == -1
    assert msg in d11.lib().uor_d11_last_error()


def test_copy_library_exports_and_refusals():
    """include/uor_copy.h: every declared entry point is exported; create refuses shapes
    outside its limits before any device call."""
    from uor_fbs import copy as cp
    text = open(os.path.join(ROOT, "include", "uor_copy.h")).read()
    names = set(re.findall(r"\b(uor_copy_[a-z0-9_]+)\s*\(", text))
    assert names == set(cp.SYMBOLS)
    L = cp.lib()
    for name in names:
        assert hasattr(L, name), name
    assert L.uor_copy_abi_version() == 1
    import copy_cases as K
    for kw in ({"kept": 33}, {"kept": 0}):
        heads = K.heads(kw["kept"], "mean")
        s, keep = heads.c_struct()
        h = P()
        assert L.uor_copy_create(C.byref(s), 0, C.byref(h)) == -1
    heads = K.heads(4, "longest-after-opening", marker=(9, 1))
    s, keep = heads.c_struct()
    assert L.uor_copy_create(C.byref(s), 0, C.byref(P())) == -1
    assert b"marker" in L.uor_copy_last_error()


def test_norm_factor_wave_equals_the_general_form(hp):
    # The lane-parallel factor (three windows of 64 candidates, each the last that passes its
    # exact test; the host runs the 64 tests in turn) against the general 128-bit form: random
    # and near-square sums, wrapping epsilons, every mean square below 2^20 (quotients up to
    # 2^62), the edges of the ranges, and the kernels' usual range. None is sent to the fallback.
    f = hp.fbs_hp_norm_factor_wave_check
    f.argtypes = [P, P, C.c_uint64, C.c_uint32, P]
    f.restype = C.c_uint64

    def check(sums, eps, log2n):
        refused = np.zeros(1, np.uint64)
        bad = f(sums.ctypes.data_as(P), eps.ctypes.data_as(P), len(eps), log2n,
                refused.ctypes.data_as(P))
        assert (bad, int(refused[0])) == (0, 0)

    rng = np.random.default_rng(99)
    n = 200000
    sums = (rng.integers(0, 2**63, n, dtype=np.uint64)
            >> rng.integers(0, 64, n).astype(np.uint64)).astype(np.uint64)
    r = rng.integers(1, 2**32, n // 2, dtype=np.uint64)
    sums[: n // 2] = (r * r + rng.integers(0, 3, n // 2, dtype=np.uint64)) << rng.integers(0, 8, n // 2).astype(np.uint64)
    eps = rng.choice(np.array([0, 1, 42950, 2**20, 2**40, 2**59, 2**60, 2**62, 2**63 - 1, -5],
                              dtype=np.int64), n)
    for log2n in (5, 8, 10):
        check(sums, eps, log2n)
    small = np.arange(1, 2**20, dtype=np.int64)
    check(np.zeros(len(small), np.uint64), small, 5)
    vals = [1, 2, 3, 15, 16, 17, 2**60 - 1, 2**60 - 2, 2**60 - 17, 2**59, 2**59 - 1, 2**59 + 1]
    for k in range(1, 31):
        for v in (k * k, (2**k) ** 2, (2**k - 1) ** 2, 3**k):
            vals += [v - 1, v, v + 1]
    for k in range(1, 61):
        vals += [2**k - 1, 2**k, 2**k + 1]
    edge = np.array([v for v in vals if 0 < v < 2**63], dtype=np.int64)
    check(np.zeros(len(edge), np.uint64), edge, 5)
    usual = rng.integers(2**30, 2**50, 500000, dtype=np.uint64) << np.uint64(8)
    check(usual, np.full(len(usual), 42950, np.int64), 8)


def test_norm_factor_pow2_at_its_edges(hp):
    # The factor's double estimates at the ends of their ranges: mean squares of 1 (s = 2^34,
    # r = 2^62), at the 60-bit mask's top, on and one off perfect squares and powers of two,
    # each entered as epsilon over a zero sum.
    hp.fbs_hp_norm_factor_check.argtypes = [P, P, C.c_uint64, C.c_uint32]
    hp.fbs_hp_norm_factor_check.restype = C.c_uint64
    vals = [1, 2, 3, 15, 16, 17, 2**60 - 1, 2**60 - 2, 2**60 - 17, 2**59, 2**59 - 1, 2**59 + 1]
    for k in range(1, 31):
        for v in (k * k, (2**k) ** 2, (2**k - 1) ** 2, 3**k):
            vals += [v - 1, v, v + 1]
    for k in range(1, 61):
        vals += [2**k - 1, 2**k, 2**k + 1]
    eps = np.array([v for v in vals if 0 < v < 2**63], dtype=np.int64)
    sums = np.zeros(len(eps), np.uint64)
    assert hp.fbs_hp_norm_factor_check(sums.ctypes.data_as(P), eps.ctypes.data_as(P), len(eps), 5) == 0
