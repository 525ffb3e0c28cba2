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

# UOR_ORACLE_LIB_DIR=oracle/lib_san selects the AddressSanitizer + UBSan build of the oracle
# libraries (make -C oracle sanitize; tests/test_sanitized_cpu.py).
LIB_DIR = os.environ.get("UOR_ORACLE_LIB_DIR") or os.path.join(HERE, "lib")
ORACLE_SO = os.path.join(LIB_DIR, "libfbs_oracle.so")
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
        u32, i32, i64, u64 = C.c_uint32, C.c_int32, C.c_int64, C.c_uint64
        L.fbs_oracle_trace_stride.argtypes = [P]
        L.fbs_oracle_trace_stride.restype = u64
        L.fbs_oracle_trace_sequences.argtypes = [P, P, P, u32, u32, P, P, P, P, C.c_int]
        L.fbs_oracle_decode_slide.argtypes = [P, P, P, u32, u32, u32, P, P, P, P, P, P, P, C.c_int]
        L.fbs_oracle_decode_stream.argtypes = [P, P, P, u32, u32, u32, P, P, P, P, P, P, P, P, P,
                                               P, P, C.c_int]
        L.fbs_oracle_hamming_typed.argtypes = [P, P]
        L.fbs_oracle_hamming_typed.restype = u32
        L.fbs_oracle_hamming_row.argtypes = [P, P, u32, P, u32, P, P, P]
        L.fbs_oracle_hamming_codes.argtypes = [P, P, u32, P]
        L.fbs_oracle_stream_sum.argtypes = [i32, i32, i64, u64, i32, i64, u64]
        L.fbs_oracle_stream_sum.restype = i32
        L.fbs_oracle_readout_sum.argtypes = [i64, i32, C.c_int, i64, u64, i32, i64, u64]
        L.fbs_oracle_readout_sum.restype = i64
        L.fbs_oracle_readout_ask_sum.argtypes = [i64, i32, C.c_int, i64, u64, i32, C.c_int, i64,
                                                 u64]
        L.fbs_oracle_readout_ask_sum.restype = i64
        L.fbs_oracle_place_sequences.argtypes = [P, P, P, u32, u32, P, P, P, C.c_int]
        L.fbs_oracle_place_rows.argtypes = [P, u32, P, u64, P, u32, P]
        L.fbs_oracle_place_pick.argtypes = [P, P, u32, P, u32, P]
        L.fbs_oracle_place_pick.restype = i64
        L.fbs_oracle_decision_stride.argtypes = [P, P, C.c_int]
        L.fbs_oracle_decision_stride.restype = u64
        L.fbs_oracle_decision_sequences.argtypes = [P, P, P, u32, u32, C.c_int, P, P, P, P, P, P,
                                                    C.c_int]
        _lib = L
    return _lib


def twin_available() -> bool:
    return os.path.exists(TWIN_SO)


def twin():
    global _twin
    if _twin is None:
        T = C.CDLL(TWIN_SO)
        T.fbs_host_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P]
        T.fbs_host_trace_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P, P]
        T.fbs_host_trace_stride.argtypes = [P]
        T.fbs_host_trace_stride.restype = C.c_uint64
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


def place_sequences(art, tokens: np.ndarray, threads: int = 1, image: Image | None = None):
    """Teacher-forced outputs with the place register after every step: (status, tokens [S,len],
    query [S,len,d], place [S,len,2] as (held, offered), -1 for none)."""
    img = image or Image(art)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    out_t = np.zeros((S, n), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    out_p = np.zeros((S, n, 2), np.int64)
    st = lib().fbs_oracle_place_sequences(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                          _vp(tokens), S, n, _vp(out_t), _vp(out_q), _vp(out_p), threads)
    return st, out_t, out_q, out_p


def decision_sequences(art, tokens: np.ndarray, decisions: bool = True, force=None,
                       threads: int = 1, image: Image | None = None):
    """The oracle's traced teacher-forced windows: (status, tokens, query, raw records
    [S, len, stride]), the records laid out as uor_fbs_decision_sequences writes them; `force` as
    hip.Model.decision_trace's."""
    from uor_fbs import trace as tr
    img = image or Image(art)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    layout = tr.TraceLayout.of(art, decisions)
    if not isinstance(force, (list, tuple)):
        force = [force] * S
    fb, fc, fm = layout.force_arrays(force, S, n)
    ext = img.ext_ptr() and C.addressof(img.ext)
    stride = int(lib().fbs_oracle_decision_stride(C.addressof(img.model), ext, int(decisions)))
    assert stride == layout.stride, (stride, layout.stride)
    out_t = np.zeros((S, n), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    raw = np.zeros((S, n, max(stride, 1)), np.uint8)
    st = lib().fbs_oracle_decision_sequences(C.addressof(img.model), ext, _vp(tokens), S, n,
                                             int(decisions), _vp(fb), _vp(fc), _vp(fm),
                                             _vp(out_t), _vp(out_q), _vp(raw), threads)
    return st, out_t, out_q, raw


def place_rows(marks, classes, tokens, finds) -> np.ndarray:
    """The place register over `tokens` from a fresh state, the question at each row `at` of
    `finds` [(at, pos), ...] finding `pos` (every other row nothing): per row (held, offer,
    stepped, asked start, asked end, finds in the asked turn, the last find's row and place), -1
    for none."""
    from uor_fbs.cabi import PlaceS
    keep = []

    def ids(v):
        a = np.ascontiguousarray(v, np.uint32)
        keep.append(a)
        return ptr(a, C.c_uint32) if len(a) else ptr(None, C.c_uint32)

    pm = PlaceS()
    pm.bos, pm.eos = marks.bos, marks.eos
    for name in ("sep", "system", "user", "assistant"):
        setattr(pm, name + "_len", len(getattr(marks, name)))
        setattr(pm, name, ids(getattr(marks, name)))
    cls = np.ascontiguousarray(classes, np.int16)
    pm.class_table = ptr(cls, C.c_int16)
    tok = np.ascontiguousarray(tokens, np.uint32)
    out = np.zeros((len(tok), 8), np.int64)
    f = np.ascontiguousarray(np.asarray(finds, np.int64).reshape(-1), np.int64)
    lib().fbs_oracle_place_rows(C.addressof(pm), len(cls), _vp(tok), len(tok),
                                _vp(f) if f.size else None, f.size // 2, _vp(out))
    return out


def place_pick(queries, margins, ranges, keys) -> int | None:
    """place_pick with every head's key at position s keys[s]; None when nothing is found."""
    q = np.ascontiguousarray(queries, np.uint64)
    m = np.ascontiguousarray(margins, np.int32)
    r = np.ascontiguousarray(np.asarray(ranges, np.uint64).reshape(-1), np.uint64)
    k = np.ascontiguousarray(keys, np.uint64)
    got = lib().fbs_oracle_place_pick(_vp(q), _vp(m), len(q), _vp(r) if r.size else None,
                                      r.size // 2, _vp(k))
    return None if got < 0 else int(got)


def decode(art, prompts: np.ndarray, gen: int, threads: int = 1, image: Image | None = None,
           in_state=None, in_history=None, in_position=None, want_state: bool = True,
           slide: bool = False):
    """Oracle greedy decode: dict(status, reply [S, gen+1], state, history, position, candidates);
    `slide`: every session's context slide on (a full context continues)."""
    img = image or Image(art)
    prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
    S, plen = prompts.shape
    s = art.spec
    reply = np.zeros((S, gen + 1), np.uint32)
    state = np.zeros((S, s.layers * s.width), np.int64) if want_state else None
    hist = np.zeros((S, s.layers * s.window * s.width), np.int32) if want_state else None
    pos = np.zeros(S, np.uint32) if want_state else None
    cand = np.zeros(S, np.uint64)
    conv = lambda a, t: None if a is None else np.ascontiguousarray(a, t)  # noqa: E731
    in_state, in_history = conv(in_state, np.int64), conv(in_history, np.int32)
    in_position = conv(in_position, np.uint32)
    if slide:
        st = lib().fbs_oracle_decode_slide(
            C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext), _vp(prompts), S, plen,
            gen, _vp(reply), _vp(in_state), _vp(in_history), _vp(in_position), _vp(state),
            _vp(hist), _vp(pos), threads)
        return dict(status=st, reply=reply, state=state, history=hist, position=pos, candidates=None)
    st = lib().fbs_oracle_decode(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                 _vp(prompts), S, plen, gen, _vp(reply), _vp(in_state),
                                 _vp(in_history), _vp(in_position), _vp(state), _vp(hist),
                                 _vp(pos), _vp(cand), threads)
    return dict(status=st, reply=reply, state=state, history=hist, position=pos, candidates=cand)


def _ext(img):
    return img.ext_ptr() and C.addressof(img.ext)


def hamming_typed(art, image: Image | None = None) -> int:
    """Typed reads whose payloads a session keeps (ServedHamming::payload_caches)."""
    img = image or Image(art)
    return int(lib().fbs_oracle_hamming_typed(C.addressof(img.model), _ext(img)))


def decode_stream(art, prompts: np.ndarray, gen: int, threads: int = 1, image: Image | None = None,
                  resume: dict | None = None):
    """Oracle greedy decode with the Hamming reads' session stream: dict(status, reply, state,
    history, position, tokens [S, context], payloads [S, typed, context, width]); `resume` is
    a dict of the same arrays to continue from."""
    img = image or Image(art)
    prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
    S, plen = prompts.shape
    s = art.spec
    typed = hamming_typed(art, img)
    out = dict(reply=np.zeros((S, gen + 1), np.uint32),
               state=np.zeros((S, s.layers * s.width), np.int64),
               history=np.zeros((S, s.layers * s.window * s.width), np.int32),
               position=np.zeros(S, np.uint32), tokens=np.zeros((S, s.context), np.uint32),
               payloads=np.zeros((S, typed, s.context, s.width), np.int64))
    r = resume or {}
    conv = lambda k, t: None if k not in r else np.ascontiguousarray(r[k], t)  # noqa: E731
    ins = [conv("state", np.int64), conv("history", np.int32), conv("position", np.uint32),
           conv("tokens", np.uint32), conv("payloads", np.int64)]
    st = lib().fbs_oracle_decode_stream(
        C.addressof(img.model), _ext(img), _vp(prompts), S, plen, gen, _vp(out["reply"]),
        *[_vp(a) for a in ins], _vp(out["state"]), _vp(out["history"]), _vp(out["position"]),
        _vp(out["tokens"]), _vp(out["payloads"]), threads)
    out["status"] = st
    return out


def hamming_row(art, depth: int, tokens, x=None, n=None, payloads=None, image: Image | None = None):
    """One Hamming read at the last row of `tokens` (the stream read on x at depth < layers, the
    readout read on n at the layer count), in place; returns (x or n, payloads)."""
    img = image or Image(art)
    tok = np.ascontiguousarray(tokens, dtype=np.uint32)
    s = art.spec
    typed = hamming_typed(art, img)
    pay = (np.zeros((typed, s.context, s.width), np.int64) if payloads is None
           else np.ascontiguousarray(payloads, np.int64))
    xa = None if x is None else np.ascontiguousarray(x, np.int32).copy()
    na = None if n is None else np.ascontiguousarray(n, np.int64).copy()
    st = lib().fbs_oracle_hamming_row(C.addressof(img.model), _ext(img), depth, _vp(tok),
                                      len(tok) - 1, _vp(xa), _vp(na), _vp(pay))
    assert st == 0
    return (xa if x is not None else na), pay


def hamming_codes(art, read: int, image: Image | None = None) -> np.ndarray:
    """Every vocabulary entry's code per head through read `read`'s key rotation."""
    img = image or Image(art)
    out = np.zeros((art.spec.vocab, art.hamming.heads), np.uint64)
    assert lib().fbs_oracle_hamming_codes(C.addressof(img.model), _ext(img), read, _vp(out)) == 0
    return out


def _split128(v: int):
    v &= (1 << 128) - 1
    hi = v >> 64
    return (hi - (1 << 64) if hi >= 1 << 63 else hi), v & ((1 << 64) - 1)


def stream_sum(x, w_c, c, w_y, y) -> int:
    return int(lib().fbs_oracle_stream_sum(x, w_c, *_split128(c), w_y, *_split128(y)))


def readout_sum(n, w_c, c, w_y, y) -> int:
    return int(lib().fbs_oracle_readout_sum(n, w_c, int(c is not None), *_split128(c or 0), w_y,
                                            *_split128(y)))


def readout_ask_sum(n, w_c, c, w_y, y) -> int:
    return int(lib().fbs_oracle_readout_ask_sum(n, w_c, int(c is not None), *_split128(c or 0),
                                                w_y, int(y is not None), *_split128(y or 0)))


def score(art, rows: np.ndarray, threads: int = 1, image: Image | None = None, want_argmin=True):
    img = image or Image(art)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    n, length = rows.shape
    argmin = np.zeros((n, length), np.uint32) if want_argmin else None
    matches = np.zeros(1, np.uint64)
    st = lib().fbs_oracle_score(C.addressof(img.model), img.ext_ptr() and C.addressof(img.ext),
                                _vp(rows), n, length, _vp(argmin), _vp(matches), threads)
    return st, int(matches[0]), argmin


def trace_sequences(art, tokens: np.ndarray, threads: int = 1, image: Image | None = None):
    """Oracle teacher-forced outputs with every position's snap trace:
    (status, tokens, kept, query, trace [S, len, stride] u8)."""
    img = image or Image(art)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    stride = int(lib().fbs_oracle_trace_stride(C.addressof(img.model)))
    out_t = np.zeros((S, n), np.uint32)
    out_k = np.zeros((S, n, art.probes), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    out_tr = np.full((S, n, stride), 0xEE, np.uint8)
    st = lib().fbs_oracle_trace_sequences(C.addressof(img.model), _ext(img), _vp(tokens), S, n,
                                          _vp(out_t), _vp(out_k), _vp(out_q), _vp(out_tr), threads)
    return st, out_t, out_k, out_q, out_tr


def twin_trace_sequences(art, tokens: np.ndarray):
    """The reference twin's fbs_host_trace_sequences (reference shapes only)."""
    assert art.spec.reference_shape and art.spec.head == 0
    img = Image(art, with_ext=False)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    S, n = tokens.shape
    stride = int(twin().fbs_host_trace_stride(C.addressof(img.model)))
    out_t = np.zeros((S, n), np.uint32)
    out_k = np.zeros((S, n, art.spec.kept), np.uint32)
    out_q = np.zeros((S, n, art.spec.width), np.int32)
    out_tr = np.full((S, n, stride), 0xEE, np.uint8)
    st = twin().fbs_host_trace_sequences(C.addressof(img.model), _vp(tokens), S, n, _vp(out_t),
                                         _vp(out_k), _vp(out_q), _vp(out_tr))
    return st, out_t, out_k, out_q, out_tr


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


# ---- the CSR drawer index (fbs_index_oracle.c) and the reference's own inverted file
# (oracle/_ref/libif_ref.so over projects/uor-cuda-inverted-file/src/inverted_file.cpp)

IF_REF_SO = os.path.join(HERE, "_ref", "libif_ref.so")
_if_ref = None


def _index_lib():
    L = lib()
    if not hasattr(L, "_index_bound"):
        u32 = C.c_uint32
        L.fbs_oracle_index_cell.argtypes = [P, u32, P]
        L.fbs_oracle_index_cell.restype = u32
        L.fbs_oracle_index_build.argtypes = [P, u32, u32, P, C.c_int, P, P, P, P]
        L.fbs_oracle_index_update.argtypes = [P, u32, u32, P, u32, P, P, P, P]
        L.fbs_oracle_index_remove.argtypes = [u32, u32, P, P, P, P]
        L.fbs_oracle_index_validate_structure.argtypes = [P, P, P, u32, u32]
        L.fbs_oracle_index_validate.argtypes = [P, u32, u32, P, P, P, P, u32]
        L.fbs_oracle_index_probe.argtypes = [P, u32, u32, P, P, u32, P, P, P, u32, P, P, P]
        L.fbs_oracle_index_full_scan.argtypes = [P, u32, u32, P, P, u32, P, P, P]
        L._index_bound = True
    return L


def if_ref_available() -> bool:
    return os.path.exists(IF_REF_SO)


def if_ref():
    global _if_ref
    if _if_ref is None:
        R = C.CDLL(IF_REF_SO)
        u32 = C.c_uint32
        R.if_ref_codebook.argtypes = [P]
        R.if_ref_build.argtypes = [P, u32, C.c_int, P, P, P, P]
        R.if_ref_update.argtypes = [P, u32, u32, P, P, P, P]
        R.if_ref_remove.argtypes = [P, u32, u32, P, P, P, P]
        R.if_ref_validate.argtypes = [P, u32, P, P, P, u32]
        R.if_ref_validate_structure.argtypes = [P, P, P, u32, u32]
        R.if_ref_probe.argtypes = [P, u32, P, u32, P, P, P, u32, P, P, P]
        R.if_ref_full_scan.argtypes = [P, u32, P, u32, P, P, P]
        _if_ref = R
    return _if_ref


def _flat(idx, count):
    """A HostIndex as the flat buffers both libraries take (members with room for count)."""
    off = np.ascontiguousarray(idx.offsets, dtype=np.uint32).copy()
    mem = np.zeros(max(count, 1), np.uint32)
    n = min(len(idx.members), count)
    mem[:n] = idx.members[:n]
    cells = np.ascontiguousarray(idx.cells, dtype=np.uint32).copy()
    return off, mem, cells, C.c_uint32(int(idx.absent_count))


def _host(off, mem, cells, absent, count):
    from uor_fbs.index import HostIndex
    return HostIndex(off, mem[:min(int(off[256]), count)].copy(), cells, int(absent.value))


def _table(table):
    t = np.ascontiguousarray(table, dtype=np.int32)
    return t, t.shape[0], t.shape[1]


def index_cell(row, roots) -> int:
    row = np.ascontiguousarray(row, dtype=np.int32)
    return int(_index_lib().fbs_oracle_index_cell(_vp(row), row.size,
                                                  _vp(np.ascontiguousarray(roots, np.int32))))


def index_build(table, roots, allow_absent=False):
    """(status, HostIndex) of build (inverted_file.cpp:112-138)."""
    t, count, width = _table(table)
    roots = np.ascontiguousarray(roots, np.int32)
    off, mem, cells = np.zeros(257, np.uint32), np.zeros(max(count, 1), np.uint32), np.zeros(max(count, 1), np.uint32)
    absent = C.c_uint32()
    st = _index_lib().fbs_oracle_index_build(_vp(t), count, width, _vp(roots), int(allow_absent),
                                             _vp(off), _vp(mem), _vp(cells), C.byref(absent))
    return st, _host(off, mem, cells[:count], absent, count)


def index_update(table, roots, moved, idx):
    """(status, HostIndex after) of update (inverted_file.cpp:182-236)."""
    t, count, width = _table(table)
    off, mem, cells, absent = _flat(idx, count)
    st = _index_lib().fbs_oracle_index_update(_vp(t), count, width,
                                              _vp(np.ascontiguousarray(roots, np.int32)), moved,
                                              _vp(off), _vp(mem), _vp(cells), C.byref(absent))
    return st, _host(off, mem, cells, absent, count)


def index_remove(count, moved, idx):
    """(status, HostIndex after) of remove_token (inverted_file.cpp:238-249)."""
    off, mem, cells, absent = _flat(idx, count)
    st = _index_lib().fbs_oracle_index_remove(count, moved, _vp(off), _vp(mem), _vp(cells),
                                              C.byref(absent))
    return st, _host(off, mem, cells, absent, count)


def index_validate(table, roots, idx) -> int:
    t, count, width = _table(table)
    off, mem, cells, absent = _flat(idx, count)
    return _index_lib().fbs_oracle_index_validate(
        _vp(t), count, width, _vp(np.ascontiguousarray(roots, np.int32)), _vp(off), _vp(mem),
        _vp(cells), absent.value)


def index_validate_structure(idx) -> int:
    count = len(idx.cells)
    off, mem, cells, absent = _flat(idx, count)
    return _index_lib().fbs_oracle_index_validate_structure(_vp(off), _vp(mem), _vp(cells), count,
                                                            absent.value)


def _scan_out():
    return np.zeros(16, np.uint32), np.zeros(8, np.uint32), C.c_uint32()


def index_probe(table, roots, query, k, idx):
    """(status, admitted [16], top8 [8], prediction) of probe (inverted_file.cpp:250-258)."""
    t, count, width = _table(table)
    q = np.ascontiguousarray(query, np.int32).reshape(width)
    off, mem, cells, absent = _flat(idx, count)
    adm, top, pred = _scan_out()
    st = _index_lib().fbs_oracle_index_probe(
        _vp(t), count, width, _vp(np.ascontiguousarray(roots, np.int32)), _vp(q), k, _vp(off),
        _vp(mem), _vp(cells), absent.value, _vp(adm), _vp(top), C.byref(pred))
    return st, adm, top, pred.value


def index_full_scan(table, roots, query, k):
    """(status, admitted, top8, prediction) of full_scan (inverted_file.cpp:260-270)."""
    t, count, width = _table(table)
    q = np.ascontiguousarray(query, np.int32).reshape(width)
    adm, top, pred = _scan_out()
    st = _index_lib().fbs_oracle_index_full_scan(
        _vp(t), count, width, _vp(np.ascontiguousarray(roots, np.int32)), _vp(q), k, _vp(adm),
        _vp(top), C.byref(pred))
    return st, adm, top, pred.value


# The reference library's calls (width-32 tables, its own codebook).

def ref_codebook() -> np.ndarray:
    roots = np.zeros((16, 8), np.int32)
    if_ref().if_ref_codebook(_vp(roots))
    return roots


def ref_build(table, allow_absent=False):
    t, count, width = _table(table)
    assert width == 32
    off, mem, cells = np.zeros(257, np.uint32), np.zeros(max(count, 1), np.uint32), np.zeros(max(count, 1), np.uint32)
    absent = C.c_uint32()
    st = if_ref().if_ref_build(_vp(t), count, int(allow_absent), _vp(off), _vp(mem), _vp(cells),
                               C.byref(absent))
    return st, _host(off, mem, cells[:count], absent, count)


def ref_update(table, moved, idx):
    t, count, _ = _table(table)
    off, mem, cells, absent = _flat(idx, count)
    st = if_ref().if_ref_update(_vp(t), count, moved, _vp(off), _vp(mem), _vp(cells),
                                C.byref(absent))
    return st, _host(off, mem, cells, absent, count)


def ref_remove(table, moved, idx):
    t, count, _ = _table(table)
    off, mem, cells, absent = _flat(idx, count)
    st = if_ref().if_ref_remove(_vp(t), count, moved, _vp(off), _vp(mem), _vp(cells),
                                C.byref(absent))
    return st, _host(off, mem, cells, absent, count)


def ref_validate(table, idx) -> int:
    t, count, _ = _table(table)
    off, mem, cells, absent = _flat(idx, count)
    return if_ref().if_ref_validate(_vp(t), count, _vp(off), _vp(mem), _vp(cells), absent.value)


def ref_probe(table, query, k, idx):
    t, count, _ = _table(table)
    q = np.ascontiguousarray(query, np.int32).reshape(32)
    off, mem, cells, absent = _flat(idx, count)
    adm, top, pred = _scan_out()
    st = if_ref().if_ref_probe(_vp(t), count, _vp(q), k, _vp(off), _vp(mem), _vp(cells),
                               absent.value, _vp(adm), _vp(top), C.byref(pred))
    return st, adm, top, pred.value


def ref_full_scan(table, query, k):
    t, count, _ = _table(table)
    q = np.ascontiguousarray(query, np.int32).reshape(32)
    adm, top, pred = _scan_out()
    st = if_ref().if_ref_full_scan(_vp(t), count, _vp(q), k, _vp(adm), _vp(top), C.byref(pred))
    return st, adm, top, pred.value


# ---------------------------------------------------------------------------------------------
# The discrete M1 evaluator (oracle/lib/libd11_oracle.so, d11_oracle.c).

D11_SO = os.path.join(LIB_DIR, "libd11_oracle.so")
_d11 = None


def d11_lib():
    global _d11
    if _d11 is None:
        if not os.path.exists(D11_SO):
            raise FileNotFoundError(f"{D11_SO} is not built (make -C oracle)")
        L = C.CDLL(D11_SO)
        L.d11_oracle_score_rows.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, C.c_int]
        L.d11_oracle_row_relation.argtypes = [P, P, C.c_int32, C.c_uint32, P, P]
        L.d11_oracle_plan.argtypes = [C.c_int32, P, P]
        L.d11_oracle_open.argtypes = [P]
        L.d11_oracle_open.restype = P
        L.d11_oracle_close.argtypes = [P]
        L.d11_oracle_close.restype = None
        L.d11_oracle_score_open.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, C.c_int]
        L.d11_oracle_trace_words.argtypes = [P, P]
        L.d11_oracle_trace_words.restype = C.c_uint32
        L.d11_oracle_score_rows_traced.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P,
                                                   C.c_int]
        _d11 = L
    return _d11


def d11_score_rows(art, prefixes, lengths, targets, threads=8):
    """One uor_d11_row_out record per row (uor_fbs.d11.ROW_DTYPE), as the HIP scorer writes."""
    from uor_fbs import d11
    m, keep = d11.c_model(art)
    prefixes = np.ascontiguousarray(prefixes, np.uint32)
    rows, stride = prefixes.shape
    lengths = np.ascontiguousarray(lengths, np.int32)
    targets = np.ascontiguousarray(targets, np.uint32)
    out = np.zeros(rows, d11.ROW_DTYPE)
    d11_lib().d11_oracle_score_rows(C.byref(m), prefixes.ctypes.data, lengths.ctypes.data,
                                    targets.ctypes.data, rows, stride, out.ctypes.data, threads)
    return out


def d11_score_rows_traced(art, prefixes, lengths, targets, knockout=False, threads=8):
    """evaluate_prefix_traced for every row: (records, trace words [rows, words], relation
    trace words [rows, blocks, a full context's node count] or None), of the model or of its
    state-transport knockout."""
    from uor_fbs import d11
    m, keep = d11.c_model(art, knockout=knockout)
    prefixes = np.ascontiguousarray(prefixes, np.uint32)
    rows, stride = prefixes.shape
    lengths = np.ascontiguousarray(lengths, np.int32)
    targets = np.ascontiguousarray(targets, np.uint32)
    rw = C.c_uint32()
    words = d11_lib().d11_oracle_trace_words(C.byref(m), C.byref(rw))
    out = np.zeros(rows, d11.ROW_DTYPE)
    trace = np.zeros((rows, words), np.uint32)
    rel = np.zeros((rows, rw.value), np.uint32) if rw.value else None
    d11_lib().d11_oracle_score_rows_traced(C.byref(m), prefixes.ctypes.data, lengths.ctypes.data,
                                           targets.ctypes.data, rows, stride, out.ctypes.data,
                                           trace.ctypes.data, None if rel is None else rel.ctypes.data,
                                           threads)
    if rel is not None:
        rel = rel.reshape(rows, art.shape.blocks, -1)
    return out, trace, rel


def d11_row_relation(art, prefix, target=0):
    """(record, relation scores (blocks, nodes)) of one row."""
    from uor_fbs import d11
    m, keep = d11.c_model(art)
    prefix = np.ascontiguousarray(prefix, np.uint32)
    out = np.zeros(1, d11.ROW_DTYPE)
    rel = np.zeros(art.shape.blocks * 512, np.int32)
    n = d11_lib().d11_oracle_row_relation(C.byref(m), prefix.ctypes.data, len(prefix), target,
                                          out.ctypes.data, rel.ctypes.data)
    return out[0], rel[:art.shape.blocks * n].reshape(art.shape.blocks, n)


def d11_plan(length):
    nodes, frontier = C.c_int32(), C.c_int32()
    st = d11_lib().d11_oracle_plan(length, C.byref(nodes), C.byref(frontier))
    return None if st else (nodes.value, frontier.value)


class D11Oracle:
    """The oracle with its model loaded once (timing covers the rows alone)."""

    def __init__(self, art):
        from uor_fbs import d11
        self.m, self.keep = d11.c_model(art)
        self.h = d11_lib().d11_oracle_open(C.byref(self.m))

    def score_rows(self, prefixes, lengths, targets, threads=8):
        from uor_fbs import d11
        prefixes = np.ascontiguousarray(prefixes, np.uint32)
        rows, stride = prefixes.shape
        lengths = np.ascontiguousarray(lengths, np.int32)
        targets = np.ascontiguousarray(targets, np.uint32)
        out = np.zeros(rows, d11.ROW_DTYPE)
        d11_lib().d11_oracle_score_open(self.h, prefixes.ctypes.data, lengths.ctypes.data,
                                        targets.ctypes.data, rows, stride, out.ctypes.data, threads)
        return out

    def close(self):
        if self.h:
            d11_lib().d11_oracle_close(self.h)
            self.h = None


# ---------------------------------------------------------------------------------------------
# The copy heads' Hamming read (oracle/lib/libcopy_oracle.so, copy_oracle.c).

COPY_SO = os.path.join(LIB_DIR, "libcopy_oracle.so")
_copy = None


def copy_mean_rows(heads, tokens, lengths, opening=None):
    """(out, found, chosen) as uor_copy_mean_rows writes them."""
    global _copy
    if _copy is None:
        _copy = C.CDLL(COPY_SO)
        _copy.copy_oracle_mean_rows.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P]
    s, keep = heads.c_struct()
    tokens = np.ascontiguousarray(tokens, np.uint32)
    rows, stride = tokens.shape
    lengths = np.ascontiguousarray(lengths, np.int32)
    op = None if opening is None else np.ascontiguousarray(opening, np.uint8)
    width, copy = heads.table.shape[1], heads.codes.shape[1]
    out = np.zeros((rows, width), np.int64)
    found = np.zeros(rows, np.uint8)
    chosen = np.zeros((rows, copy, heads.kept), np.int32)
    _copy.copy_oracle_mean_rows(C.byref(s), tokens.ctypes.data, lengths.ctypes.data,
                                None if op is None else op.ctypes.data, rows, stride,
                                out.ctypes.data, found.ctypes.data, chosen.ctypes.data)
    return out, found.astype(bool), chosen


def copy_vocab_codes(key_rotation, table, heads_total, copy):
    """vocab_codes (hamming.rs:541-582) restated: units from the oracle's stack_rotation (raw
    form, lambda 2^31, epsilon 0), then each head's sign word of stack_hamilton(unit, point)."""
    rot = np.ascontiguousarray(key_rotation, np.int32)
    table = np.asarray(table, np.int64)
    vocab, width = table.shape
    units = []
    for q in range(width // 4):
        out = np.zeros(4, np.int64)
        lib().fbs_oracle_serve_rotation(None, 1, rot[4 * q:4 * q + 4].ctypes.data, 1 << 31, 0,
                                        out.ctypes.data)
        units.append([int(x) for x in out])
    hw = width // heads_total
    codes = np.zeros((vocab, copy), np.uint64)
    for v in range(vocab):
        p = [int(x) for x in table[v]]
        for h in range(copy):
            word = 0
            for c in range(0, hw, 4):
                at = h * hw + c
                a, b = units[at // 4], p[at:at + 4]
                r = [a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3],
                     a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2],
                     a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1],
                     a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0]]
                for i, x in enumerate(r):
                    if x >= 0:
                        word |= 1 << (c + i)
            codes[v, h] = word
    return codes
