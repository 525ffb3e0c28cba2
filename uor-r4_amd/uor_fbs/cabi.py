"""ctypes mirror of include/uor_fbs.h and the image builder for an Artifact.

`uor_fbs_model` has the layout of the reference's `CModel` / `fbs_model`
(docs/labs/d11-exporter-float-trunk/instrument/src/lib.rs:14-63, fbs_core.h:42-73): the same
struct reaches the HIP library, the test oracle and the reference's own twin.
"""

from __future__ import annotations

import ctypes as C

import numpy as np


class Map(C.Structure):
    _fields_ = [("atoms", C.POINTER(C.c_uint16)), ("codes", C.POINTER(C.c_uint8)),
                ("blocks", C.c_uint32)]


class LayerS(C.Structure):
    _fields_ = [("rec_gain", C.POINTER(C.c_int16)), ("mlp_gain", C.POINTER(C.c_int16)),
                ("rec_in", Map), ("rec_gate", Map), ("rec_out", Map), ("mlp_gate", Map),
                ("mlp_up", Map), ("mlp_down", Map), ("taps", C.POINTER(C.c_int16)),
                ("conv_bias", C.POINTER(C.c_int32)), ("gate_bias", C.POINTER(C.c_int32)),
                ("decay_offset", C.POINTER(C.c_int32))]


class ModelS(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("width", C.c_uint32), ("mlp", C.c_uint32),
                ("context", C.c_uint32), ("kept", C.c_uint32), ("layer_count", C.c_uint32),
                ("eps_mantissa", C.c_int64), ("eps_exp", C.c_int32),
                ("layers", C.POINTER(LayerS)), ("final_gain", C.POINTER(C.c_int16)),
                ("writer_table", C.POINTER(C.c_int16)), ("roots_q12", C.POINTER(C.c_int32)),
                ("icosian", C.POINTER(C.c_int8)), ("keep_q31", C.POINTER(C.c_uint64)),
                ("raw_gates", C.c_uint32), ("raw_transition", C.c_uint32)]


class HammingReadS(C.Structure):
    _fields_ = [("depth", C.c_uint32), ("carry_rows", C.c_uint32),
                ("query_rotation", C.POINTER(C.c_int32)), ("key_rotation", C.POINTER(C.c_int32)),
                ("value_rotation", C.POINTER(C.c_int32)), ("margin", C.POINTER(C.c_int32)),
                ("weight", C.POINTER(C.c_int32)), ("ask", C.POINTER(C.c_int16)),
                ("carry", C.POINTER(C.c_int32))]


class PlaceS(C.Structure):
    _fields_ = [("bos", C.c_uint32), ("eos", C.c_uint32), ("sep_len", C.c_uint32),
                ("system_len", C.c_uint32), ("user_len", C.c_uint32), ("assistant_len", C.c_uint32),
                ("sep", C.POINTER(C.c_uint32)), ("system", C.POINTER(C.c_uint32)),
                ("user", C.POINTER(C.c_uint32)), ("assistant", C.POINTER(C.c_uint32)),
                ("class_table", C.POINTER(C.c_int16))]


class HammingS(C.Structure):
    _fields_ = [("heads", C.c_uint32), ("kept", C.c_uint32), ("copy_key", C.c_uint32),
                ("copy_latest", C.c_uint32), ("copy_keys", C.POINTER(C.c_uint32)),
                ("copy_longest", C.c_uint32), ("marker", C.c_uint32 * 2), ("rule", C.c_uint32),
                ("read_count", C.c_uint32), ("reads", C.POINTER(HammingReadS)),
                ("place", C.POINTER(PlaceS))]


class ExtS(C.Structure):
    _fields_ = [("window", C.c_uint32), ("drawers", C.c_uint32), ("probes", C.c_uint32),
                ("head", C.c_uint32), ("wide_taps", C.POINTER(C.POINTER(C.c_int16))),
                ("drawer_keys", C.POINTER(C.c_int32)), ("drawer_offsets", C.POINTER(C.c_uint32)),
                ("drawer_members", C.POINTER(C.c_uint32)), ("table_i8", C.POINTER(C.c_int8)),
                ("table_shift", C.c_uint32), ("reserved", C.c_uint32),
                ("hamming", C.POINTER(HammingS))]


_CT = {np.dtype(np.int8): C.c_int8, np.dtype(np.uint8): C.c_uint8, np.dtype(np.int16): C.c_int16,
       np.dtype(np.uint16): C.c_uint16, np.dtype(np.int32): C.c_int32,
       np.dtype(np.uint32): C.c_uint32, np.dtype(np.int64): C.c_int64,
       np.dtype(np.uint64): C.c_uint64}


def ptr(a: np.ndarray | None, ctype=None):
    """A typed pointer to a C-contiguous array (NULL for None)."""
    if a is None:
        return None if ctype is None else C.POINTER(ctype)()
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(C.POINTER(ctype or _CT[a.dtype]))


class Image:
    """The C image of an artifact; keeps every array it points into alive."""

    def __init__(self, art, *, with_ext: bool | None = None):
        s = art.spec
        keep = []

        def arr(a, dtype):
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return a

        layers = (LayerS * s.layers)()
        for l, ly in enumerate(art.layers):
            L = layers[l]
            L.rec_gain = ptr(arr(ly.rec_gain, np.int16))
            L.mlp_gain = ptr(arr(ly.mlp_gain, np.int16))
            for name in ("rec_in", "rec_gate", "rec_out", "mlp_gate", "mlp_up", "mlp_down"):
                atoms, codes = ly.maps[name]
                a, c = arr(atoms, np.uint16), arr(codes, np.uint8)
                setattr(L, name, Map(ptr(a), ptr(c), len(a)))
            L.taps = ptr(arr(ly.taps, np.int16))
            L.conv_bias = ptr(arr(ly.conv_bias, np.int32))
            L.gate_bias = ptr(arr(ly.gate_bias, np.int32))
            L.decay_offset = ptr(arr(ly.decay_offset, np.int32))
        keep.append(layers)
        m = ModelS()
        m.vocab, m.width, m.mlp = s.vocab, s.width, s.mlp
        m.context, m.kept, m.layer_count = s.context, s.kept, s.layers
        m.eps_mantissa, m.eps_exp = art.eps_mantissa, art.eps_exp
        m.layers = C.cast(layers, C.POINTER(LayerS))
        m.final_gain = ptr(arr(art.final_gain, np.int16))
        m.writer_table = ptr(arr(art.writer_table, np.int16))
        m.roots_q12 = ptr(arr(art.roots_q12, np.int32))
        m.icosian = ptr(arr(art.icosian, np.int8))
        m.keep_q31 = ptr(arr(art.keep_q31, np.uint64))
        m.raw_gates, m.raw_transition = int(s.raw_gates), int(s.raw_transition)
        self.model = m
        ham = getattr(art, "hamming", None)
        needs_ext = (not s.reference_shape or s.head != 0 or art.drawer_keys is not None
                     or ham is not None)
        if with_ext is None:
            with_ext = needs_ext
        self.ext = None
        if with_ext:
            e = ExtS()
            e.window = s.window
            e.drawers = art.drawers
            e.probes = art.probes
            e.head = s.head
            if any(ly.wide_taps is not None for ly in art.layers):
                tp = (C.POINTER(C.c_int16) * s.layers)()
                for l, ly in enumerate(art.layers):
                    wt = ly.wide_taps if ly.wide_taps is not None else ly.taps
                    tp[l] = ptr(arr(wt, np.int16))
                keep.append(tp)
                e.wide_taps = C.cast(tp, C.POINTER(C.POINTER(C.c_int16)))
            e.drawer_keys = ptr(None if art.drawer_keys is None else arr(art.drawer_keys, np.int32),
                                C.c_int32)
            e.drawer_offsets = ptr(None if art.drawer_offsets is None
                                   else arr(art.drawer_offsets, np.uint32), C.c_uint32)
            e.drawer_members = ptr(None if art.drawer_members is None
                                   else arr(art.drawer_members, np.uint32), C.c_uint32)
            e.table_i8 = ptr(None if art.table_i8 is None else arr(art.table_i8, np.int8), C.c_int8)
            e.table_shift = s.table_shift if art.table_i8 is not None else 0
            if ham is not None:
                reads = (HammingReadS * len(art.hamming_reads))()
                for i, r in enumerate(art.hamming_reads):
                    R = reads[i]
                    R.depth, R.carry_rows = r.depth, (ham.carry_rows if r.carry is not None else 0)
                    R.query_rotation = ptr(arr(r.query_rotation, np.int32))
                    R.key_rotation = ptr(arr(r.key_rotation, np.int32))
                    R.value_rotation = ptr(arr(r.value_rotation, np.int32))
                    R.margin = ptr(arr(r.margin, np.int32))
                    R.weight = ptr(arr(r.weight, np.int32))
                    R.ask = ptr(None if r.ask is None else arr(r.ask, np.int16), C.c_int16)
                    R.carry = ptr(None if r.carry is None else arr(r.carry, np.int32), C.c_int32)
                keep.append(reads)
                H = HammingS()
                H.heads, H.kept, H.copy_key = ham.heads, ham.kept, ham.copy_key
                H.copy_latest = int(ham.copy_latest)
                H.copy_keys = ptr(None if ham.copy_keys is None
                                  else arr(np.array(ham.copy_keys), np.uint32), C.c_uint32)
                H.copy_longest = int(ham.copy_longest is not None)
                if ham.copy_longest is not None:
                    H.marker[0], H.marker[1] = ham.copy_longest
                H.rule = ham.rule
                H.read_count = len(art.hamming_reads)
                H.reads = C.cast(reads, C.POINTER(HammingReadS))
                if ham.place is not None:
                    pm, P = ham.place, PlaceS()
                    P.bos, P.eos = pm.bos, pm.eos
                    for name in ("sep", "system", "user", "assistant"):
                        ids = np.asarray(getattr(pm, name), np.uint32)
                        setattr(P, name + "_len", len(ids))
                        setattr(P, name, ptr(arr(ids, np.uint32) if len(ids) else None, C.c_uint32))
                    P.class_table = ptr(arr(art.hamming_place, np.int16), C.c_int16)
                    keep.append(P)
                    H.place = C.pointer(P)
                keep.append(H)
                e.hamming = C.pointer(H)
            self.ext = e
        self._keep = keep

    def model_ptr(self):
        return C.byref(self.model)

    def ext_ptr(self):
        return C.byref(self.ext) if self.ext is not None else None
