"""ctypes binding of the test oracle (oracle/lib/libfbs_oracle.so) and of the reference's own
twin (oracle/_ref/libfbs_twin.so, built only where /root/reference exists).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker or the timed CPU baseline, never as the product.
"""

from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "uor-r4_amd"))

from uor_fbs.cabi import Image, ptr  # noqa: E402

ORACLE_SO = os.path.join(HERE, "lib", "libfbs_oracle.so")
TWIN_SO = os.path.join(HERE, "_ref", "libfbs_twin.so")

_lib = None
_twin = None

P = C.c_void_p


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} is not built (make -C oracle)")
        L = C.CDLL(ORACLE_SO)
        L.fbs_oracle_sequences.argtypes = [P, P, P, C.c_uint32, C.c_uint32, P, P, P, C.c_int]
        L.fbs_oracle_decode.argtypes = [P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, P, P, P, P,
                                        P, P, P, P, C.c_int]
        L.fbs_oracle_score.argtypes = [P, P, P, C.c_uint64, C.c_uint32, P, P, C.c_int]
        L.fbs_oracle_shift.argtypes = [C.c_int64, C.c_int32]
        L.fbs_oracle_shift.restype = C.c_int64
        L.fbs_oracle_shift_wide.argtypes = [C.c_int64, C.c_uint64, C.c_uint32]
        L.fbs_oracle_shift_wide.restype = C.c_int64
        L.fbs_oracle_grid_apply.argtypes = [C.c_int64, C.c_int16]
        L.fbs_oracle_grid_apply.restype = C.c_int64
        L.fbs_oracle_isqrt.argtypes = [C.c_uint64, C.c_uint64, P]
        L.fbs_oracle_div_u128.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, P]
        L.fbs_oracle_snap_select.argtypes = [P, P]
        L.fbs_oracle_snap_select.restype = C.c_uint32
        L.fbs_oracle_diff_positive.argtypes = [C.c_int64, C.c_int64]
        L.fbs_oracle_serve_rotation.argtypes = [P, C.c_uint32, P, C.c_uint64, C.c_uint64, P]
        L.fbs_oracle_quantize16.argtypes = [P, C.c_uint32, C.c_int32, P]
        L.fbs_oracle_quantize16.restype = C.c_int32
        L.fbs_oracle_rms_norm_fine.argtypes = [P, C.c_uint32, C.c_int64, C.c_int32, P]
        L.fbs_oracle_writer.argtypes = [P, P, P, P, P]
        L.fbs_oracle_writer.restype = C.c_uint32
        _lib = L
    return _lib


def twin_available() -> bool:
    return os.path.exists(TWIN_SO)


def twin():
    global _twin
    if _twin is None:
        T = C.CDLL(TWIN_SO)
        T.fbs_host_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P]
        T.fbs_host_sizeof_model.restype = C.c_int64
        T.fbs_host_sizeof_layer.restype = C.c_int64
        _twin = T
    return _twin


def _vp(a):
    return None if a is None else a.ctypes.data_as(P)


def sequences(art, tokens: np.ndarray, threads: int = 1, image: Image | None = None):
    """Oracle teacher-forced outputs: (tokens [S,len], kept [S,len,P], query [S,len,d])."""
    img = image or Image(art)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    P_ = art.probes
    out_t = np.zeros((S, n), np.uint32)
    out_k = np.zeros((S, n, P_), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    st = lib().fbs_oracle_sequences(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                    _vp(tokens), S, n, _vp(out_t), _vp(out_k), _vp(out_q), threads)
    return st, out_t, out_k, out_q


def decode(art, prompts: np.ndarray, gen: int, threads: int = 1, image: Image | None = None,
           in_state=None, in_history=None, in_position=None, want_state: bool = True):
    """Oracle greedy decode: dict(status, reply [S, gen+1], state, history, position, candidates)."""
    img = image or Image(art)
    prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
    S, plen = prompts.shape
    s = art.spec
    reply = np.zeros((S, gen + 1), np.uint32)
    state = np.zeros((S, s.layers * s.width), np.int64) if want_state else None
    hist = np.zeros((S, s.layers * s.window * s.width), np.int32) if want_state else None
    pos = np.zeros(S, np.uint32) if want_state else None
    cand = np.zeros(S, np.uint64)
    st = lib().fbs_oracle_decode(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                 _vp(prompts), S, plen, gen, _vp(reply), _vp(in_state),
                                 _vp(in_history), _vp(in_position), _vp(state), _vp(hist),
                                 _vp(pos), _vp(cand), threads)
    return dict(status=st, reply=reply, state=state, history=hist, position=pos, candidates=cand)


def score(art, rows: np.ndarray, threads: int = 1, image: Image | None = None, want_argmin=True):
    img = image or Image(art)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    n, length = rows.shape
    argmin = np.zeros((n, length), np.uint32) if want_argmin else None
    matches = np.zeros(1, np.uint64)
    st = lib().fbs_oracle_score(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                _vp(rows), n, length, _vp(argmin), _vp(matches), threads)
    return st, int(matches[0]), argmin


def twin_sequences(art, tokens: np.ndarray):
    """The reference twin's fbs_host_sequences on the artifact (reference shapes only)."""
    assert art.spec.reference_shape and art.spec.head == 0
    img = Image(art, with_ext=False)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    out_t = np.zeros((S, n), np.uint32)
    out_k = np.zeros((S, n, art.spec.kept), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    st = twin().fbs_host_sequences(C.addressof(img.model), _vp(tokens), S, n, _vp(out_t),
                                   _vp(out_k), _vp(out_q))
    return st, out_t, out_k, out_q
