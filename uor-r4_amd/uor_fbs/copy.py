"""The copy heads' Hamming read on the GPU (include/uor_copy.h).

Mirrors ``CopyHeads`` (crates/uor-r4-integer/src/stack/hamming.rs:266-538): ``CopyRule`` and its
names (:180-228), ``copy_weight_q31`` (:243-252), and the read at a stream's last row --
``choose_ruled`` (:356-371) for each head's positions and ``mean`` / ``mean_at`` (:475-504) for
the heads' margin-weighted mean. Every read runs in the HIP library (``uor_copy_*``); there is
no host evaluation path. ``mean_rows`` reads many streams in one launch.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

RULES = {"mean": 0, "latest-exact": 1, "latest-nearest": 2, "longest-exact": 3,
         "longest-after-opening": 4}
SYMBOLS = ("uor_copy_abi_version", "uor_copy_last_error", "uor_copy_create", "uor_copy_destroy",
           "uor_copy_mean_rows", "uor_copy_mean_rows_async", "uor_copy_vocab_codes")
MAX_KEPT = 32


class CopyError(ValueError):
    pass


class CHeads(C.Structure):
    _fields_ = [("vocabulary", C.c_uint32), ("width", C.c_uint32), ("copy", C.c_uint32),
                ("kept", C.c_uint32), ("rule", C.c_uint32), ("has_marker", C.c_uint32),
                ("marker", C.c_uint32 * 2), ("codes", C.c_void_p), ("margins_q16", C.c_void_p),
                ("pair_first", C.c_void_p), ("table", C.c_void_p)]


def copy_weight_q31(margin_q16: int, distance: int) -> int:
    """max(0, m - d) / max(m, 1) at Q31, floored (hamming.rs:243-252)."""
    over = margin_q16 - (distance << 16)
    return 0 if over <= 0 else (over << 31) // max(margin_q16, 1 << 16)


@dataclass
class Heads:
    """A read's copy heads as ``CopyHeads`` holds them."""
    codes: np.ndarray                 # (vocab, copy) uint64
    margins_q16: np.ndarray           # (copy,) int32
    table: np.ndarray                 # (vocab, width) int16
    kept: int
    rule: str = "mean"
    pair_first: np.ndarray | None = None   # (copy,) uint64, 0 = copy key 1
    marker: tuple | None = None

    def c_struct(self):
        codes = np.ascontiguousarray(self.codes, np.uint64)
        vocab, copy = codes.shape
        margins = np.ascontiguousarray(self.margins_q16, np.int32)
        pair = np.ascontiguousarray(np.zeros(copy, np.uint64) if self.pair_first is None
                                    else self.pair_first, np.uint64)
        table = np.ascontiguousarray(self.table, np.int16)
        mk = (C.c_uint32 * 2)(*(self.marker or (0, 0)))
        s = CHeads(vocab, table.shape[1], copy, self.kept, RULES[self.rule],
                   int(self.marker is not None), mk, codes.ctypes.data, margins.ctypes.data,
                   pair.ctypes.data, table.ctypes.data)
        return s, (codes, margins, pair, table)


_lib = None


def lib():
    global _lib
    if _lib is None:
        from . import hip
        L = hip.lib()
        P = C.c_void_p
        L.uor_copy_abi_version.restype = C.c_uint32
        L.uor_copy_last_error.restype = C.c_char_p
        L.uor_copy_create.argtypes = [C.POINTER(CHeads), C.c_int32, C.POINTER(P)]
        L.uor_copy_destroy.argtypes = [P]
        L.uor_copy_destroy.restype = None
        L.uor_copy_mean_rows.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P]
        L.uor_copy_mean_rows_async.argtypes = [P, P, P, P, C.c_uint32, C.c_uint32, P, P, P, P]
        L.uor_copy_vocab_codes.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                           C.c_int32, P]
        _lib = L
    return _lib


def _check(code):
    if code:
        raise CopyError(f"uor_copy status {code}: {lib().uor_copy_last_error().decode()}")


def vocab_codes(key_rotation, table, heads_total, copy, device=0):
    """(vocab, copy) uint64: every entry's code per copy head (hamming.rs:566-582), on the GPU."""
    rot = np.ascontiguousarray(key_rotation, np.int32)
    table = np.ascontiguousarray(table, np.int16)
    vocab, width = table.shape
    codes = np.zeros((vocab, copy), np.uint64)
    _check(lib().uor_copy_vocab_codes(rot.ctypes.data, table.ctypes.data, vocab, width,
                                      heads_total, copy, device, codes.ctypes.data))
    return codes


def pack_rows(streams, stride=None):
    """(tokens (rows, stride) uint32 zero-padded, lengths int32) of a list of streams."""
    stride = stride or max(1, max((len(s) for s in streams), default=1))
    tok = np.zeros((len(streams), stride), np.uint32)
    for i, s in enumerate(streams):
        tok[i, :len(s)] = s
    return tok, np.array([len(s) for s in streams], np.int32)


class CopyHeads:
    """Copy heads resident on one GPU (the reference's method names)."""

    def __init__(self, heads: Heads, device: int = 0):
        self.heads = heads
        s, self._keep = heads.c_struct()
        h = C.c_void_p()
        _check(lib().uor_copy_create(C.byref(s), device, C.byref(h)))
        self.handle = h
        self.copy = heads.codes.shape[1]
        self.width = heads.table.shape[1]

    def close(self):
        if getattr(self, "handle", None):
            lib().uor_copy_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def mean_rows(self, tokens, lengths, opening=None):
        """(out (rows, width) int64, found (rows,) bool, chosen (rows, copy, kept) int32)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        rows, stride = tokens.shape
        lengths = np.ascontiguousarray(lengths, np.int32)
        op = None if opening is None else np.ascontiguousarray(opening, np.uint8)
        out = np.zeros((rows, self.width), np.int64)
        found = np.zeros(rows, np.uint8)
        chosen = np.zeros((rows, self.copy, self.heads.kept), np.int32)
        if rows:
            _check(lib().uor_copy_mean_rows(self.handle, tokens.ctypes.data, lengths.ctypes.data,
                                            None if op is None else op.ctypes.data, rows, stride,
                                            out.ctypes.data, found.ctypes.data,
                                            chosen.ctypes.data))
        return out, found.astype(bool), chosen

    def mean_at(self, tokens, opening=False):
        """The copy mean at the last row (None when no head kept a position in its margin)."""
        tok, lens = pack_rows([list(tokens)])
        out, found, _ = self.mean_rows(tok, lens, [int(opening)])
        return out[0].tolist() if found[0] else None

    def mean(self, tokens):
        return self.mean_at(tokens, False)

    def choose_ruled(self, h, tokens, opening=False):
        """Head h's (position, distance) pairs at the last row, in the order read."""
        tok, lens = pack_rows([list(tokens)])
        _, _, chosen = self.mean_rows(tok, lens, [int(opening)])
        return [(int(v) & 0xffffff, int(v) >> 24) for v in chosen[0, h] if v >= 0]


def synthetic(vocab=32768, width=256, copy=4, kept=16, rule="mean", seed=1, margin_bits=28):
    """Random heads: 64-bit codes per token and head, margins of `margin_bits` bits, copy key 2
    on odd heads (first half the low 32 bits), a Q12-range table."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << 63, (vocab, copy), dtype=np.int64).astype(np.uint64)
    codes ^= rng.integers(0, 2, (vocab, copy)).astype(np.uint64) << np.uint64(63)
    pair = np.array([0 if h % 2 == 0 else (1 << 32) - 1 for h in range(copy)], np.uint64)
    table = rng.integers(-4096, 4097, (vocab, width)).astype(np.int16)
    return Heads(codes, np.full(copy, margin_bits << 16, np.int32), table, kept, rule, pair)
