"""ctypes binding of the product library, uor-r4_amd/lib/libuor_fbs_hip.so (include/uor_fbs.h).

The Python face of the boundary the reference's Rust host binds through `extern "C"`
(docs/labs/d11-exporter-float-trunk/instrument/src/lib.rs:14-95, device.rs:93-302): a model
handle created from the `fbs_model` image, then teacher-forced `sequences`, greedy `decode`
with state export/import, and `score`. Errors raise `FbsError` carrying the library's status
code (1 token outside the vocabulary, 2 context exceeded, as fbs_core.h:625-628) and message.
There is no fallback: a missing library or device raises.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .cabi import Image

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "lib", "libuor_fbs_hip.so")

P = C.c_void_p
_lib = None

# Every entry point include/uor_fbs.h declares (checked by the CPU tests).
SYMBOLS = (
    "uor_fbs_abi_version", "uor_fbs_sizeof_model", "uor_fbs_sizeof_layer", "uor_fbs_sizeof_ext",
    "uor_fbs_last_error", "uor_fbs_model_create", "uor_fbs_model_destroy", "uor_fbs_state_words",
    "uor_fbs_history_words", "uor_fbs_sequences", "uor_fbs_sequences_async", "uor_fbs_decode",
    "uor_fbs_decode_async", "uor_fbs_decode_noalloc_async", "uor_fbs_score",
    "uor_fbs_score_async", "uor_fbs_block_waves",
    "uor_fbs_decode_slots_async", "uor_fbs_index_workspace_bytes", "uor_fbs_index_build_async",
    "uor_fbs_index_update_async", "uor_fbs_index_remove_async", "uor_fbs_index_validate_async",
    "uor_fbs_index_probe_async", "uor_fbs_index_full_scan_async", "uor_fbs_stream_words",
    "uor_fbs_payload_words", "uor_fbs_decode_stream", "uor_fbs_decode_stream_async",
    "uor_fbs_slot_cache_bytes", "uor_fbs_serve_slots_async", "uor_fbs_trace_stride",
    "uor_fbs_trace_sequences", "uor_fbs_trace_sequences_async", "uor_fbs_part_count",
    "uor_fbs_part_name", "uor_fbs_decode_parts_async", "uor_fbs_serve_slots_stream_async",
    "uor_fbs_decision_stride", "uor_fbs_decision_sequences",
)


class FbsError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"uor_fbs status {code}: {message}")
        self.code = code


def lib():
    """The loaded library (raises if it is not built: there is no other implementation)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        L = C.CDLL(LIB_PATH)
        L.uor_fbs_abi_version.restype = C.c_uint32
        L.uor_fbs_sizeof_model.restype = C.c_int64
        L.uor_fbs_sizeof_layer.restype = C.c_int64
        L.uor_fbs_sizeof_ext.restype = C.c_int64
        L.uor_fbs_last_error.restype = C.c_char_p
        L.uor_fbs_model_create.argtypes = [P, P, C.c_int32, C.POINTER(P)]
        L.uor_fbs_model_destroy.argtypes = [P]
        L.uor_fbs_model_destroy.restype = None
        L.uor_fbs_state_words.argtypes = [P]
        L.uor_fbs_state_words.restype = C.c_uint64
        L.uor_fbs_history_words.argtypes = [P]
        L.uor_fbs_history_words.restype = C.c_uint64
        L.uor_fbs_block_waves.argtypes = [P, C.c_uint32]
        L.uor_fbs_block_waves.restype = C.c_uint32
        L.uor_fbs_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P]
        L.uor_fbs_sequences_async.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P, P, P]
        L.uor_fbs_decode.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, P, P, P, P, P, P, P]
        L.uor_fbs_decode_async.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, P, P, P, P, P,
                                           P, P, P, P]
        L.uor_fbs_decode_noalloc_async.argtypes = L.uor_fbs_decode_async.argtypes
        L.uor_fbs_serve_slots_stream_async.argtypes = [P, P, C.c_uint32, C.c_uint32, P, C.c_uint32,
                                                       C.c_uint32] + [P] * 11
        L.uor_fbs_decision_stride.argtypes = [P, C.c_uint32]
        L.uor_fbs_decision_stride.restype = C.c_uint64
        L.uor_fbs_decision_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, P, P, P,
                                                 P, P, P]
        L.uor_fbs_part_count.restype = C.c_uint32
        L.uor_fbs_part_name.argtypes = [C.c_uint32]
        L.uor_fbs_part_name.restype = C.c_char_p
        L.uor_fbs_decode_parts_async.argtypes = L.uor_fbs_decode_async.argtypes[:-1] + [P, P]
        L.uor_fbs_stream_words.argtypes = [P]
        L.uor_fbs_stream_words.restype = C.c_uint64
        L.uor_fbs_payload_words.argtypes = [P]
        L.uor_fbs_payload_words.restype = C.c_uint64
        L.uor_fbs_decode_stream.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32] + [P] * 11
        L.uor_fbs_decode_stream_async.argtypes = ([P, P, C.c_uint32, C.c_uint32, C.c_uint32]
                                                  + [P] * 13)
        L.uor_fbs_decode_slots_async.argtypes = [P, P, C.c_uint32, C.c_uint32, P, C.c_uint32,
                                                 C.c_uint32, P, P, P, P, P, P, P, P]
        L.uor_fbs_trace_stride.argtypes = [P]
        L.uor_fbs_trace_stride.restype = C.c_uint64
        L.uor_fbs_trace_sequences.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P, P]
        L.uor_fbs_trace_sequences_async.argtypes = [P, P, C.c_uint32, C.c_uint32, P, P, P, P, P, P]
        L.uor_fbs_slot_cache_bytes.argtypes = [P]
        L.uor_fbs_slot_cache_bytes.restype = C.c_uint64
        L.uor_fbs_serve_slots_async.argtypes = [P, P, C.c_uint32, C.c_uint32, P, C.c_uint32,
                                                C.c_uint32, P, P, P, P, P, P, P, P, P, P, P]
        L.uor_fbs_score.argtypes = [P, P, C.c_uint64, C.c_uint32, P, P]
        L.uor_fbs_score_async.argtypes = [P, P, C.c_uint64, C.c_uint32, P, P, P, P]
        u32 = C.c_uint32
        L.uor_fbs_index_workspace_bytes.argtypes = [u32]
        L.uor_fbs_index_workspace_bytes.restype = C.c_uint64
        L.uor_fbs_index_build_async.argtypes = [P, u32, u32, P, u32, P, P, P, P, P, P, P]
        L.uor_fbs_index_update_async.argtypes = [P, u32, u32, P, u32, P, P, P, P, P, P, P]
        L.uor_fbs_index_remove_async.argtypes = [u32, u32, P, P, P, P, P, P, P]
        L.uor_fbs_index_validate_async.argtypes = [P, u32, u32, P, P, P, P, P, P, P, P]
        L.uor_fbs_index_probe_async.argtypes = [P, u32, u32, P, P, u32, u32, P, P, P, P, P, P, P]
        L.uor_fbs_index_full_scan_async.argtypes = [P, u32, u32, P, P, u32, u32, P, P, P, P, P,
                                                    P]
        _lib = L
    return _lib


def _vp(a):
    return None if a is None else a.ctypes.data_as(P)


def _check(code: int):
    if code:
        raise FbsError(code, lib().uor_fbs_last_error().decode())


def part_names() -> list[str]:
    """The part clocks' phases in their order (uor_fbs_part_name)."""
    L = lib()
    return [L.uor_fbs_part_name(i).decode() for i in range(int(L.uor_fbs_part_count()))]


class Model:
    """A model on one HIP device (IntegerStackModel + DeviceEvaluator in one handle)."""

    def __init__(self, art, device: int = 0, image: Image | None = None):
        self.art = art
        self.image = image or Image(art)
        h = P()
        ext = C.byref(self.image.ext) if self.image.ext is not None else None
        _check(lib().uor_fbs_model_create(C.byref(self.image.model), ext, device, C.byref(h)))
        self.handle = h
        self.device = device
        s = art.spec
        self.width, self.layers, self.window = s.width, s.layers, s.window
        self.probes = art.probes

    def close(self):
        if self.handle:
            lib().uor_fbs_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def state_words(self) -> int:
        return int(lib().uor_fbs_state_words(self.handle))

    @property
    def history_words(self) -> int:
        return int(lib().uor_fbs_history_words(self.handle))

    def block_waves(self, n: int) -> int:
        """Wavefronts per sequence of the kernels a run of n sequences launches (1 or 2)."""
        return int(lib().uor_fbs_block_waves(self.handle, n))

    def sequences(self, tokens, want_kept=True, want_query=True):
        """Teacher-forced runs from fresh sessions: (tokens [S,len], kept [S,len,P], query [S,len,d])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        S, n = tokens.shape
        out_t = np.zeros((S, n), np.uint32)
        out_k = np.zeros((S, n, self.probes), np.uint32) if want_kept else None
        out_q = np.zeros((S, n, self.width), np.int32) if want_query else None
        _check(lib().uor_fbs_sequences(self.handle, _vp(tokens), S, n, _vp(out_t), _vp(out_k), _vp(out_q)))
        return out_t, out_k, out_q

    def decode(self, prompts, gen: int, in_state=None, in_history=None, in_position=None,
               want_state: bool = True):
        """Greedy decode: dict(reply [S, gen+1], state, history, position)."""
        prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
        S, plen = prompts.shape
        reply = np.zeros((S, gen + 1), np.uint32)
        state = np.zeros((S, self.state_words), np.int64) if want_state else None
        hist = np.zeros((S, self.history_words), np.int32) if want_state else None
        pos = np.zeros(S, np.uint32) if want_state else None
        conv = lambda a, t: None if a is None else np.ascontiguousarray(a, dtype=t)  # noqa: E731
        in_state, in_history, in_position = conv(in_state, np.int64), conv(in_history, np.int32), conv(in_position, np.uint32)
        _check(lib().uor_fbs_decode(self.handle, _vp(prompts), S, plen, gen, _vp(reply),
                                    _vp(in_state), _vp(in_history), _vp(in_position), _vp(state),
                                    _vp(hist), _vp(pos)))
        return dict(reply=reply, state=state, history=hist, position=pos)

    def decode_parts(self, prompts, gen: int, in_state=None, in_history=None, in_position=None):
        """decode() on the part clocks' kernels (uor_fbs_decode_parts_async, device buffers):
        dict(reply, state, history, position, parts [S, 2, part_count()] cycles of each wave in
        each part over the sequence's steps, steps [S], ticks [S] of the 100 MHz clock)."""
        from .hipmem import DeviceArray, runtime
        prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
        S, plen = prompts.shape
        npart = int(lib().uor_fbs_part_count())

        def dev(a, t):
            if a is None:
                return None
            d = DeviceArray(np.shape(a), t, self.device)
            d.upload(np.ascontiguousarray(a, t))
            return d

        d_prompts = dev(prompts, np.uint32)
        d_in = [dev(in_state, np.int64), dev(in_history, np.int32), dev(in_position, np.uint32)]
        reply = DeviceArray((S, gen + 1), np.uint32, self.device)
        state = DeviceArray((S, self.state_words), np.int64, self.device)
        hist = DeviceArray((S, self.history_words), np.int32, self.device)
        pos = DeviceArray(S, np.uint32, self.device)
        status = DeviceArray(S, np.int32, self.device)
        parts = DeviceArray((S, 2 * npart + 2), np.uint64, self.device)
        ptr = lambda d: None if d is None else d.ptr  # noqa: E731
        _check(lib().uor_fbs_decode_parts_async(
            self.handle, d_prompts.ptr, S, plen, gen, reply.ptr, *[ptr(d) for d in d_in],
            state.ptr, hist.ptr, pos.ptr, status.ptr, parts.ptr, None))
        runtime().hipDeviceSynchronize()
        st = status.download()
        if st.any():
            raise FbsError(int(st[st != 0][0]), "a sequence failed in the part clocks' decode")
        raw = parts.download()
        return dict(reply=reply.download(), state=state.download(), history=hist.download(),
                    position=pos.download(), parts=raw[:, :2 * npart].reshape(S, 2, npart),
                    steps=raw[:, 2 * npart], ticks=raw[:, 2 * npart + 1])

    @property
    def stream_words(self) -> int:
        """Tokens a session of a Hamming model keeps (the context), else 0."""
        return int(lib().uor_fbs_stream_words(self.handle))

    @property
    def payload_words(self) -> int:
        """int64 payload values a session of a Hamming model keeps, [typed read][context][width]."""
        return int(lib().uor_fbs_payload_words(self.handle))

    def decode_stream(self, prompts, gen: int, resume: dict | None = None):
        """Greedy decode with the Hamming reads' session stream: dict(reply, state, history,
        position, tokens [S, context], payloads [S, typed, context, width]); `resume` holds the
        same arrays (state, history, position, tokens, payloads) to continue from."""
        prompts = np.ascontiguousarray(prompts, dtype=np.uint32)
        S, _ = prompts.shape
        tw, pw = self.stream_words, self.payload_words
        typed = pw // max(1, self.width * max(tw, 1))
        out = dict(reply=np.zeros((S, gen + 1), np.uint32),
                   state=np.zeros((S, self.state_words), np.int64),
                   history=np.zeros((S, self.history_words), np.int32),
                   position=np.zeros(S, np.uint32), tokens=np.zeros((S, tw), np.uint32),
                   payloads=np.zeros((S, typed, tw, self.width), np.int64))
        r = resume or {}
        conv = lambda k, t: None if k not in r else np.ascontiguousarray(r[k], t)  # noqa: E731
        ins = [conv("state", np.int64), conv("history", np.int32), conv("position", np.uint32),
               conv("tokens", np.uint32), conv("payloads", np.int64)]
        _check(lib().uor_fbs_decode_stream(
            self.handle, _vp(prompts), S, prompts.shape[1], gen, _vp(out["reply"]),
            *[_vp(a) for a in ins], _vp(out["state"]), _vp(out["history"]), _vp(out["position"]),
            _vp(out["tokens"]) if tw else None, _vp(out["payloads"]) if pw else None))
        return out

    def decision_trace(self, tokens, decisions: bool = True, force=None):
        """Teacher-forced windows from fresh sessions with every position's trace record
        (uor_fbs_decision_sequences): the decision trace (`decisions`, each step a
        trace.DecisionStep with the nearest added from its query) or the Hamming trace alone
        (each step a list of trace.HammingStepRead). `force`: a trace.DecisionForceWindow per
        row (or one for every row), None for none. Returns dict(tokens, query, steps)."""
        from . import trace as tr
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        S, n = tokens.shape
        layout = tr.TraceLayout.of(self.art, decisions)
        if not isinstance(force, (list, tuple)):
            force = [force] * S
        fb, fc, fm = layout.force_arrays(force, S, n)
        stride = int(lib().uor_fbs_decision_stride(self.handle, int(decisions)))
        assert stride == layout.stride, (stride, layout.stride)
        out_t = np.zeros((S, n), np.uint32)
        out_q = np.zeros((S, n, self.width), np.int32)
        raw = np.zeros((S, n, max(stride, 1)), np.uint8)
        _check(lib().uor_fbs_decision_sequences(
            self.handle, _vp(tokens), S, n, int(decisions), _vp(fb), _vp(fc), _vp(fm),
            _vp(out_t), _vp(out_q), _vp(raw)))
        table = self.art.writer_table.reshape(-1, self.width)
        steps = []
        for i in range(S):
            rows = []
            for t in range(n):
                rec = raw[i, t].tobytes()
                if decisions:
                    step = layout.step(rec)
                    step.nearest = tr.nearest(out_q[i, t], table)
                    rows.append(step)
                else:
                    rows.append(layout.reads(rec))
            steps.append(rows)
        return dict(tokens=out_t, query=out_q, steps=steps, raw=raw)

    def trace_sequences(self, tokens):
        """Teacher-forced runs with every position's snap trace: (tokens [S,len], kept
        [S,len,P], query [S,len,d], trace [S,len,stride] u8)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        S, n = tokens.shape
        stride = int(lib().uor_fbs_trace_stride(self.handle))
        out_t = np.zeros((S, n), np.uint32)
        out_k = np.zeros((S, n, self.probes), np.uint32)
        out_q = np.zeros((S, n, self.width), np.int32)
        out_tr = np.zeros((S, n, stride), np.uint8)
        _check(lib().uor_fbs_trace_sequences(self.handle, _vp(tokens), S, n, _vp(out_t), _vp(out_k),
                                             _vp(out_q), _vp(out_tr)))
        return out_t, out_k, out_q, out_tr

    def score(self, rows, want_argmin=True):
        """Teacher-forced scoring: (matches, argmin [n, len] or None)."""
        rows = np.ascontiguousarray(rows, dtype=np.uint32)
        n, length = rows.shape
        argmin = np.zeros((n, length), np.uint32) if want_argmin else None
        matches = np.zeros(1, np.uint64)
        _check(lib().uor_fbs_score(self.handle, _vp(rows), n, length, _vp(argmin), _vp(matches)))
        return int(matches[0]), argmin
