"""Serving sessions on the GPU: IntegerStackSession's serving surface for FBS models
(stack/session.rs:2703-3440: reset, step, step_native, read_step, serve_step, save_state,
restore_state, save_session_to_file, restore_session_from_file) over a pool of session slots
held in device memory.

A `SessionPool` owns, per slot, one session's recurrence state, window history and position
in HBM, a serving cache (the window sums formed for the slot's next step and the writer's
memory of its last query) and a context-slide flag; `uor_fbs_serve_slots_async` steps any set
of slots in one launch and updates them in place, so a serving loop batches whichever sessions
have a token ready (`serve_steps`) without moving state through the host. `Session` is one sequence in a slot with the
reference's per-call semantics; its snapshots are the reference's `SerializedStackSession`,
encodable as `UR4SESS1` bytes or the JSON of `save_session_to_file` (`session_codec`).

A model with Hamming reads also keeps each slot's token stream and the typed reads' payloads
of every position in HBM (`uor_fbs_serve_slots_stream_async`); its snapshots carry them as the
reference's `tokens` and `hamming_payloads`.

A session's opt-in snap trace (`enable_snap_trace`) records each step's transition roots from
the launch's trace output. What the GPU path does not keep (and so refuses to restore, rather
than continuing differently): read-layer caches (the FBS trunk has none).
"""

from __future__ import annotations

import hashlib
import os
from dataclasses import dataclass

import numpy as np

from . import hip
from .hipmem import DeviceArray
from .session_codec import (STACK_SESSION_SCHEMA, CodecError, RecurrenceLayer, SerializedStackSession,
                            from_json, to_json)

NO_CHOICE = 0xFFFFFFFF  # session.rs:4406: a nearest-head read step chose no token
TRACE_UNSET = 0xFFFFFFFF  # a snap trace entry no step has written (session.rs:2580-2584)
TRACE_ZERO = 255  # the launch's trace byte for a zero raw quaternion, whose selection is root 0


class SessionError(ValueError):
    """A refusal of the reference's session API; `kind` names its `StackError` variant
    (Schema, Numerics, ContentReadout, ContextFull, SessionState, Token, Shape)."""

    def __init__(self, kind: str, message: str):
        super().__init__(f"{kind}: {message}")
        self.kind = kind


@dataclass
class NativeStep:
    """`NativeStep` (session.rs:484-493): the writer's token, kept drawers and Q12 query."""
    token: int
    kept_cells: np.ndarray
    query_q12: np.ndarray


def model_identity(art) -> str:
    """The session's serving identity: the artifact container's SHA-256 (format.rs:1493,
    session.rs:1049); a generated artifact has no container, so its identity is the SHA-256 of
    this build's tag, its spec and its seed."""
    if art.sha256:
        return art.sha256
    tag = f"uor-fbs-synthetic/1\0{art.spec!r}\0{art.seed}".encode()
    return hashlib.sha256(tag).hexdigest()


@dataclass(frozen=True)
class SnapTraceEntry:
    """`SnapTraceEntry` (session.rs:2021-2034): the root the snapped transition chose at one
    (layer, position, lane)."""
    layer: int
    position: int
    lane: int
    root: int


class SnapTrace:
    """The opt-in trace buffer (session.rs:2040-2058): one root index per (position, layer,
    lane) in step order, `context * layers * lanes` entries allocated once; `written` keeps
    counting past the end (a sliding session), where nothing more is stored."""

    def __init__(self, entries: int, origin_position: int):
        self.origin_position = origin_position
        self.selected = np.full(entries, TRACE_UNSET, np.uint32)
        self.written = 0

    def record(self, roots) -> None:
        """`SnapTrace::record` for each of `roots` in order."""
        roots = np.asarray(roots, np.uint32).reshape(-1)
        lo = min(self.written, len(self.selected))
        hi = min(self.written + len(roots), len(self.selected))
        self.selected[lo:hi] = roots[:hi - lo]
        self.written += len(roots)

    def clear(self, entries: int) -> None:
        """reset's handling (session.rs:2728-2737): origin 0, nothing written, every entry unset."""
        self.origin_position = 0
        self.written = 0
        if len(self.selected) < entries:
            self.selected = np.full(entries, TRACE_UNSET, np.uint32)
        self.selected.fill(TRACE_UNSET)


def transition_roots(trace: np.ndarray, layers: int, lanes: int) -> np.ndarray:
    """The roots a session's snap trace records from the launch's trace bytes of some steps
    ([steps, trace stride]): per step, per layer, the transition's root per lane (stack_lanes,
    session.rs:5117-5124); the byte for a zero raw quaternion reads as root 0, the index
    stack_snap_select (stack/kernels.rs:1474-1528) gives it (every root scores 0; the lowest
    index wins the tie)."""
    t = np.asarray(trace, np.uint8).reshape(len(trace), layers, -1)[:, :, :lanes]
    return np.where(t == TRACE_ZERO, 0, t).astype(np.uint32).reshape(-1)


@dataclass(frozen=True)
class ModelInfo:
    """What restore_state checks a snapshot against."""
    sha256: str
    vocab: int
    width: int
    layers: int
    window: int
    context: int
    heads: int = 1       # every served FBS shape has one head (format.rs:616-752)
    snapped: bool = False
    hamming: bool = False
    # Per Hamming read: whether it keeps a payload cache (type heads that bring a payload back,
    # payload_caches, hamming.rs:1678-1685).
    payload_reads: tuple = ()
    place: bool = False  # a place read, whose register and turns a snapshot does not carry

    @staticmethod
    def of(art) -> "ModelInfo":
        s = art.spec
        reads = getattr(art, "hamming_reads", None) or []
        d = s.width
        cached = tuple(bool(r.ask is None and np.any(np.asarray(r.weight)[d:] != 0)) for r in reads)
        ham = getattr(art, "hamming", None)
        return ModelInfo(model_identity(art), s.vocab, s.width, s.layers, s.window, s.context,
                         1, not s.raw_transition, ham is not None, cached,
                         ham is not None and ham.place is not None)

    @property
    def payload_slots(self) -> int:
        return sum(self.payload_reads)

    def payload_caches(self) -> list:
        """A fresh session's hamming_payloads: `context * width` zeros per read that keeps one,
        an empty list per other read, none without Hamming reads (hamming.rs:1678-1685)."""
        n = self.context * self.width
        return [[0] * n if c else [] for c in self.payload_reads]

    @property
    def state_words(self) -> int:
        return self.layers * self.width

    @property
    def history_words(self) -> int:
        return self.layers * self.window * self.width

    @property
    def lanes(self) -> int:
        return self.width // 4

    @property
    def trace_entries(self) -> int:
        """A full context's snap trace entries (session.rs:2578-2580): every layer recurs."""
        return self.context * self.layers * self.lanes


def max_serialized_session_bytes(info: ModelInfo) -> int:
    """The JSON size bound restore_session_from_file enforces (session.rs:2281-2345), for the FBS
    trunk: every layer a recurrence, no pointer; a Hamming read's payloads `context * width`
    numbers per read that keeps them; 24 bytes per number."""
    layer_bytes = info.layers * (info.window + 1) * info.width * 24
    logits_bytes = info.vocab * 24
    tokens_bytes = info.context * 24
    trace_bytes = info.context * (info.width // 4) * info.layers * 24 if info.snapped else 0
    payload_bytes = info.payload_slots * info.context * info.width * 24
    return layer_bytes + logits_bytes + tokens_bytes + trace_bytes + payload_bytes + 131072


def validate_restore(info: ModelInfo, saved: SerializedStackSession) -> None:
    """restore_state's checks (session.rs:2876-3090) for an FBS model, in the reference's order;
    raises SessionError and changes nothing."""
    # A type-head session's payloads travel with it (session.rs:2894-2910); a snapshot without
    # them, or with caches of other lengths, is refused.
    if info.payload_slots:
        want = [len(p) for p in info.payload_caches()]
        if [len(p) for p in saved.hamming_payloads] != want:
            raise SessionError("Shape", "a type-head session needs its per-position payloads, "
                                        "which this snapshot does not carry")
    if info.place:  # session.rs:2911-2919
        raise SessionError("Shape", "a session of a place read cannot be restored yet: its register "
                                    "and turns are not saved")
    if saved.schema != STACK_SESSION_SCHEMA:
        raise SessionError("Schema", f"expected {STACK_SESSION_SCHEMA}, found {saved.schema}")
    if saved.version != 1:
        raise SessionError("Schema", f"unsupported session version {saved.version}")
    if saved.artifact_sha256 != info.sha256:
        raise SessionError("Numerics", f"session serving identity mismatch: session has "
                                       f"'{saved.artifact_sha256}', model has '{info.sha256}'")
    if saved.content_readout_sha256 is not None:
        raise SessionError("ContentReadout", "session content-readout identity differs from the attached sidecar")
    pos = saved.position
    if pos > info.context:
        raise SessionError("ContextFull", f"context {info.context}")
    if saved.cache_at != pos * info.width or saved.lift_at != pos * info.heads:
        raise SessionError("SessionState", "cache_at/lift_at do not match the position")
    if len(saved.layers) != info.layers:
        raise SessionError("SessionState", f"{len(saved.layers)} layers, the model has {info.layers}")
    if (pos == 0 and saved.logits) or (pos > 0 and len(saved.logits) != info.vocab):
        raise SessionError("SessionState", "pending logits of the wrong length")
    if len(saved.tokens) != pos:
        raise SessionError("SessionState", "the ingested tokens do not match the position")
    if saved.pointer_keys or saved.pointer_lifts or saved.mixture:
        raise SessionError("SessionState", "pointer state for a model without a pointer head")
    for t in saved.tokens:
        if not 0 <= t < info.vocab:
            raise SessionError("Token", f"token {t} outside vocab {info.vocab}")
    if saved.snap_trace is not None:
        if not info.snapped:
            if saved.snap_trace:
                raise SessionError("SessionState", "a snap trace for a model without snapped transport")
        else:
            want = pos * (info.width // 4) * info.layers
            if len(saved.snap_trace) != want or any(not 0 <= r < 120 for r in saved.snap_trace):
                raise SessionError("SessionState", "a snap trace of the wrong length or roots")
    for layer in saved.layers:
        if not isinstance(layer, RecurrenceLayer):
            raise SessionError("SessionState", "a read layer's cache for a recurrence layer")
        if len(layer.state) != info.width or len(layer.history) != info.window * info.width:
            raise SessionError("SessionState", "a layer of the wrong width or window")


class SessionPool:
    """`capacity` session slots of one model in device memory, stepped together."""

    def __init__(self, model: "hip.Model", capacity: int):
        if capacity <= 0:
            raise ValueError("a pool needs at least one slot")
        self.model = model
        self.info = ModelInfo.of(model.art)
        self.capacity = capacity
        dev = model.device
        self.state = DeviceArray((capacity, model.state_words), np.int64, dev)
        self.history = DeviceArray((capacity, model.history_words), np.int32, dev)
        self.position = DeviceArray(capacity, np.uint32, dev)
        # Each slot's serving cache (zero: holds nothing) and context-slide flag.
        self.cache_bytes = int(hip.lib().uor_fbs_slot_cache_bytes(model.handle))
        self.cache = DeviceArray((capacity, self.cache_bytes), np.uint8, dev)
        self.cache.zero()
        self.slide = DeviceArray(capacity, np.uint8, dev)
        self.slide.zero()
        # A Hamming model's sessions also keep their token stream and the typed reads' payloads
        # of every position, which the reads look back over.
        tw, pw = model.stream_words, model.payload_words
        self.stream = DeviceArray((capacity, tw), np.uint32, dev) if self.info.hamming else None
        self.payloads = DeviceArray((capacity, pw), np.int64, dev) if pw else None
        for a in (self.stream, self.payloads):
            if a is not None:
                a.zero()
        self._free = list(range(capacity - 1, -1, -1))

    def acquire(self, slot: int | None = None) -> int:
        """A free slot holding a fresh session: the next free one, or `slot` if it is free."""
        if slot is None:
            if not self._free:
                raise SessionError("Shape", f"all {self.capacity} session slots are in use")
            slot = self._free.pop()
        else:
            slot = int(slot)
            if not 0 <= slot < self.capacity:
                raise ValueError(f"slot {slot} outside the pool's {self.capacity}")
            if slot not in self._free:
                raise ValueError(f"slot {slot} is held by another session")
            self._free.remove(slot)
        self.clear([slot])
        return slot

    def release(self, slot: int):
        if slot in self._free or not 0 <= slot < self.capacity:
            raise ValueError(f"slot {slot} is not held")
        self._free.append(slot)

    def clear(self, slots):
        """A fresh session in each slot (reset, session.rs:2703-2760); the slide setting stays,
        as reset keeps it."""
        slots = list(slots)
        for a in (self.state, self.history, self.position, self.cache, self.stream, self.payloads):
            if a is not None:
                a.zero(slots)

    def set_slide(self, slot: int, on: bool):
        flags = self.slide.download()
        flags[slot] = 1 if on else 0
        self.slide.upload(flags)

    def _ring_rows(self, position: int) -> np.ndarray:
        """Ring row holding history row r (the drive r + 1 positions back) at `position`."""
        w = self.info.window
        return (position - 1 - np.arange(w)) % w

    def read(self, slot: int):
        """(state [L*d] i64, history [L*W*d] i32 newest row first, position) of one slot; the
        device holds the history as the kernel's ring (row p mod W = the drive of position p)."""
        pos = int(self.position.download()[slot])
        i = self.info
        ring = self.history.download(slot).reshape(i.layers, i.window, i.width)
        return self.state.download(slot), ring[:, self._ring_rows(pos)].reshape(-1), pos

    def write(self, slot: int, state, history, position: int):
        i = self.info
        rows = np.asarray(history, np.int32).reshape(i.layers, i.window, i.width)
        ring = np.empty_like(rows)
        ring[:, self._ring_rows(position)] = rows
        self.state.upload(state, slot)
        self.history.upload(ring.reshape(-1), slot)
        p = self.position.download()
        p[slot] = position
        self.position.upload(p)
        self.cache.zero([slot])  # its window sums were formed for the state it held

    def read_stream(self, slot: int, position: int):
        """(tokens [position], payloads [payload reads, context, width]) of a Hamming slot."""
        i = self.info
        tokens = self.stream.download(slot)[:position]
        pay = (self.payloads.download(slot) if self.payloads is not None
               else np.zeros(0, np.int64)).reshape(i.payload_slots, i.context, i.width)
        return tokens, pay

    def write_stream(self, slot: int, tokens, payloads):
        """A Hamming slot's token stream (the first len(tokens) entries) and payload caches."""
        row = np.zeros(self.stream.shape[1], np.uint32)
        row[:len(tokens)] = np.asarray(tokens, np.uint32)
        self.stream.upload(row, slot)
        if self.payloads is not None:
            self.payloads.upload(np.asarray(payloads, np.int64).reshape(-1), slot)

    def run(self, slots, tokens, gen: int = 0, native: bool = False, trace: bool = False):
        """One launch: the sessions in `slots` take tokens [n, len] and `gen` greedy steps.
        Returns dict(reply [n, gen+1], status [n], kept [n, P], query [n, d], trace [n, len + gen,
        trace stride]) (kept and query when `native`, trace when `trace`)."""
        slots = np.asarray(slots, dtype=np.uint32).reshape(-1)
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = len(slots)
        if tokens.ndim != 2 or tokens.shape[0] != n or tokens.shape[1] == 0:
            raise ValueError("tokens must be [sessions, len >= 1]")
        if len(set(slots.tolist())) != n:
            raise ValueError("a slot appears twice in one step")
        if np.any(slots >= self.capacity):
            raise ValueError("a slot outside the pool")
        dev = self.model.device
        d_slots, d_tok = DeviceArray(n, np.uint32, dev), DeviceArray(tokens.size, np.uint32, dev)
        d_slots.upload(slots)
        d_tok.upload(tokens.reshape(-1))
        reply = DeviceArray((n, gen + 1), np.uint32, dev)
        status = DeviceArray(n, np.int32, dev)
        kept = DeviceArray((n, self.model.probes), np.uint32, dev) if native else None
        query = DeviceArray((n, self.model.width), np.int32, dev) if native else None
        steps = tokens.shape[1] + gen
        stride = int(hip.lib().uor_fbs_trace_stride(self.model.handle))
        snap = DeviceArray((n, steps, stride), np.uint8, dev) if trace else None
        ptr = lambda x: None if x is None else x.ptr  # noqa: E731
        # The null stream: the runtime's blocking copies below wait for the launch.
        if self.stream is not None:
            if trace:
                raise SessionError("Shape", "the snap trace is not served with Hamming reads")
            hip._check(hip.lib().uor_fbs_serve_slots_stream_async(
                self.model.handle, d_slots.ptr, n, self.capacity, d_tok.ptr, tokens.shape[1], gen,
                reply.ptr, self.state.ptr, self.history.ptr, self.position.ptr, self.stream.ptr,
                ptr(self.payloads), self.cache.ptr, ptr(kept), ptr(query), status.ptr, None))
        else:
            hip._check(hip.lib().uor_fbs_serve_slots_async(
                self.model.handle, d_slots.ptr, n, self.capacity, d_tok.ptr, tokens.shape[1], gen,
                reply.ptr, self.state.ptr, self.history.ptr, self.position.ptr, self.cache.ptr,
                self.slide.ptr, ptr(kept), ptr(query), ptr(snap), status.ptr, None))
        out = dict(reply=reply.download(), status=status.download())
        if native:
            out["kept"] = kept.download()
            out["query"] = query.download()
        if trace:
            out["trace"] = snap.download()
        return out


_STATUS = {1: ("Token", "a token lies outside the vocabulary"),
           2: ("ContextFull", "the session is at its context"),
           3: ("Shape", "a slot outside the pool")}


class Session:
    """One sequence in a pool slot, with IntegerStackSession's serving calls."""

    def __init__(self, pool: SessionPool, slot: int | None = None):
        self.pool = pool
        self.info = pool.info
        self.slot = pool.acquire(slot)
        self.slide = False
        pool.set_slide(self.slot, False)
        self.trace: SnapTrace | None = None  # off by default (session.rs:2570-2576)
        self.hamming_trace: list | None = None   # off by default (session.rs:2361-2370)
        self.decision: dict | None = None        # off by default (session.rs:2438-2515)
        self._reset_host()

    def _reset_host(self):
        self.slide = getattr(self, "slide", False)  # a caller's setting: reset keeps it
        self.position = 0
        self.tokens: list[int] = []
        self.logits: list[int] | None = None   # pending logits from a restore; zeros otherwise
        self.hamming_payloads: list = self.info.payload_caches()
        self._native: NativeStep | None = None

    def close(self):
        if self.slot is not None:
            self.pool.release(self.slot)
            self.slot = None

    def reset(self):
        """Start a new stream (session.rs:2703-2760); a snap trace stays enabled and starts over."""
        self.pool.clear([self.slot])
        self._reset_host()
        if self.trace is not None:
            self.trace.clear(self.info.trace_entries)

    def enable_snap_trace(self) -> None:
        """Record the root each step's snapped transition selects at every (layer, lane)
        (session.rs:2570-2585): the buffer is allocated here, once, for a full context; from the
        session's current position. A model without a snap records nothing."""
        self.trace = SnapTrace(self.info.trace_entries, self.position)

    def snap_trace(self) -> list[SnapTraceEntry] | None:
        """The recorded trace as (layer, position, lane, root) entries in step order, or None
        when tracing is off (session.rs:2587-2620)."""
        if self.trace is None:
            return None
        lanes, per = self.info.lanes, self.info.layers * self.info.lanes
        written = min(self.trace.written, len(self.trace.selected))
        return [SnapTraceEntry(rem // lanes, self.trace.origin_position + k // per, rem % lanes,
                               int(self.trace.selected[k]))
                for k in range(written) for rem in (k % per,)]

    def set_context_slide(self, on: bool) -> None:
        """Let a full context continue instead of refusing (session.rs:2391-2402): refused for a
        model whose reads name token positions (Hamming reads) or that has a turn memory
        (can_slide_tokens, :1146-1151)."""
        art = self.pool.model.art
        if on and (getattr(art, "hamming", None) is not None or getattr(art, "turn_memory", False)):
            raise SessionError("Shape", "a context slide needs a model whose reads do not use "
                                        "token positions")
        self.slide = bool(on)
        self.pool.set_slide(self.slot, self.slide)

    # ---- stepping ----
    def _admit(self, tokens) -> list[int]:
        """The prefix of `tokens` the reference would step before refusing one (a token outside
        the vocabulary, or the context full), and the refusal, if any."""
        ok = []
        for tok in tokens:
            if not 0 <= tok < self.info.vocab:
                return ok, SessionError("Token", f"token {tok} outside vocab {self.info.vocab}")
            if self.position + len(ok) >= self.info.context and not self.slide:
                return ok, SessionError("ContextFull", f"context {self.info.context}")
            ok.append(int(tok))
        return ok, None

    def _after(self, fed: list[int], reply, kept, query, trace=None):
        if self.trace is not None and trace is not None:
            self.trace.record(transition_roots(trace[:len(fed)], self.info.layers, self.info.lanes))
        self.position += len(fed)
        self.tokens.extend(fed)
        # A sliding session keeps its last `context` tokens (session.rs:4149-4151).
        del self.tokens[:max(0, len(self.tokens) - self.info.context)]
        self._native = NativeStep(int(reply[-1]), kept, query)
        self._record_traces(len(fed))

    # ---- the Hamming and decision traces (session.rs:2361-2370, 2438-2515) ----
    def _record_traces(self, fed: int) -> None:
        """The fed steps' records: the session's tokens run again from position 0 through the
        traced teacher-forced kernels. Neither trace changes a step, and a position's decisions
        are a function of the tokens up to it, so the records are the served steps' own."""
        if self.hamming_trace is None and self.decision is None:
            return
        decisions = self.decision is not None
        got = self.pool.model.decision_trace(np.asarray([self.tokens], np.uint32), decisions)
        new = got["steps"][0][len(self.tokens) - fed:]
        if decisions:
            for step in new:
                step.nearest = None  # the caller's to add, from the step's query
            self.decision["steps"].extend(new)
        else:
            for reads in new:
                self.hamming_trace.extend(reads)

    def set_hamming_trace(self, on: bool) -> None:
        """Record each Hamming read's choices from the next step on, or stop and drop them
        (session.rs:2361-2363)."""
        self.hamming_trace = [] if on else None

    def take_hamming_trace(self):
        """The reads recorded since the trace was turned on, in step order, each step's stream
        reads in depth order and then its readout read (trace.HammingStepRead); the trace stays
        on, empty. None while it is off (session.rs:2365-2370)."""
        if self.hamming_trace is None:
            return None
        out, self.hamming_trace = self.hamming_trace, []
        return out

    def set_decision_trace(self, force=None) -> None:
        """Record every step's decisions from the next step on (session.rs:2438-2510): each
        layer's rate buckets and the stream read after it, and the readout read; the nearest is
        the caller's to add from the step's query. It turns the Hamming trace off. Refused as the
        reference refuses it: a snapped artifact, a head other than the nearest, a session that
        has stepped. A forced set that forces something runs as teacher-forced windows
        (hip.Model.decision_trace): a live session's steps are the served ones."""
        art = self.pool.model.art
        if not art.spec.raw_gates or not art.spec.raw_transition:
            raise SessionError("Shape", "the decision trace reads an unsnapped artifact: the snap is "
                                        "not a decision it records")
        if art.spec.head != 1:
            raise SessionError("Shape", "the decision trace reads the Hamilton gate and the nearest "
                                        "head, with no point key")
        if self.position != 0:
            raise SessionError("Shape", "the decision trace starts in a fresh session")
        if force is not None and (force.buckets or force.codes):
            raise SessionError("Shape", "a forced replay runs as teacher-forced windows "
                                        "(Model.decision_trace), not on a served session")
        if self.slide:
            raise SessionError("Shape", "a sliding session's decisions are not replayed")
        self.hamming_trace = None
        self.decision = dict(force=force, steps=[])

    def take_decision_trace(self):
        """The decisions recorded since set_decision_trace (trace.DecisionStep), one a step, and
        the trace turned off; None while it is off (session.rs:2512-2515)."""
        if self.decision is None:
            return None
        steps, self.decision = self.decision["steps"], None
        return steps

    def feed(self, tokens) -> NativeStep:
        """The prompt tokens in one launch: read_step for all but the last, then step_native on
        the last. A refused token stops the feed there, with the tokens before it stepped."""
        ok, err = self._admit(list(tokens))
        if ok:
            traced = self.trace is not None and self.info.snapped  # unsnapped: nothing recorded
            out = self.pool.run([self.slot], np.asarray([ok], np.uint32), native=True, trace=traced)
            st = int(out["status"][0])
            if st:
                raise SessionError(*_STATUS.get(st, ("Shape", f"status {st}")))
            self._after(ok, out["reply"][0], out["kept"][0], out["query"][0],
                        out["trace"][0] if traced else None)
        if err:
            raise err
        return self._native

    def step_native(self, token: int) -> NativeStep:
        """Feed one token and return the native writer's choice (session.rs:3356-3371)."""
        return self.feed([token])

    def step(self, token: int) -> np.ndarray:
        """Feed one token; an FBS step returns no logits, an empty slice (session.rs:3320-3330)."""
        self.feed([token])
        return np.zeros(0, np.int32)

    def read_step(self, token: int) -> None:
        """A token whose successor the caller holds (session.rs:3392-3397): the state as step
        leaves it; under the nearest head no token is chosen."""
        self.feed([token])
        if self.pool.model.art.spec.head == 1:
            self._native = NativeStep(NO_CHOICE, self._native.kept_cells, self._native.query_q12)

    def serve_step(self, token: int) -> tuple[int, int]:
        """The served greedy next token and margin (session.rs:3405-3425): an FBS model's native
        token, margin 0."""
        return self.feed([token]).token, 0

    def last_native_token(self) -> int | None:
        """session.rs:3373-3380: None before any step and after a nearest-head read step."""
        if self._native is None or self._native.token == NO_CHOICE:
            return None
        return self._native.token

    def last_query_q12(self) -> np.ndarray | None:
        return None if self._native is None else self._native.query_q12

    # ---- snapshots ----
    def save_state(self) -> SerializedStackSession:
        """session.rs:2777-2870 for an FBS session: every layer a recurrence."""
        state, hist, pos = self.pool.read(self.slot)
        assert pos == self.position, (pos, self.position)
        i, d, w = self.info, self.info.width, self.info.window
        layers = [RecurrenceLayer(state[l * d:(l + 1) * d].tolist(),
                                  hist[l * w * d:(l + 1) * w * d].tolist()) for l in range(i.layers)]
        logits = [] if pos == 0 else (list(self.logits) if self.logits is not None else [0] * i.vocab)
        # The trace travels when it covers every step from position 0 (session.rs:2827-2845).
        snap = None
        if i.snapped and self.trace is not None:
            want = pos * i.lanes * i.layers
            t = self.trace
            if t.origin_position == 0 and t.written == want and want <= len(t.selected):
                snap = t.selected[:want].tolist()
        payloads = []
        if i.hamming:
            tokens, pay = self.pool.read_stream(self.slot, pos)
            assert tokens.tolist() == self.tokens, "the slot's stream and the session's tokens"
            it = iter(pay)
            payloads = [next(it).reshape(-1).tolist() if c else [] for c in i.payload_reads]
        return SerializedStackSession(STACK_SESSION_SCHEMA, 1, i.sha256, pos, pos * d, pos * i.heads,
                                      0, logits, list(self.tokens), payloads, snap, [], [], [],
                                      None, layers)

    def restore_state(self, saved: SerializedStackSession) -> None:
        """session.rs:2876-3190: validate everything, then replace the slot's state."""
        validate_restore(self.info, saved)
        state = np.concatenate([np.asarray(l.state, np.int64) for l in saved.layers])
        hist = np.concatenate([np.asarray(l.history, np.int64).astype(np.int32) for l in saved.layers])
        if self.info.hamming:
            caches = saved.hamming_payloads if self.info.payload_slots else []
            pay = [np.asarray(p, np.int64) for p, c in zip(caches, self.info.payload_reads) if c]
            self.pool.write_stream(self.slot, saved.tokens,
                                   np.concatenate(pay) if pay else np.zeros(0, np.int64))
        self.pool.write(self.slot, state, hist, saved.position)
        self.position = saved.position
        self.tokens = list(saved.tokens)
        self.logits = list(saved.logits) if saved.position > 0 else None
        self.hamming_payloads = ([list(p) for p in saved.hamming_payloads] if saved.hamming_payloads
                                 else self.info.payload_caches())
        self._native = None
        # The trace continues from a traced snapshot; an untraced one turns tracing off, so no
        # partial root history carries over (session.rs:3172-3190).
        self.trace = None
        if saved.snap_trace is not None and self.info.snapped:
            self.trace = SnapTrace(self.info.trace_entries, 0)
            self.trace.record(saved.snap_trace)

    def save_session_to_file(self, path) -> None:
        """JSON to `path`, atomically and durably (session.rs:3202-3262): an exclusive temporary
        sibling, flushed and synced, renamed over `path`, then the directory synced."""
        data = to_json(self.save_state())
        path = os.fspath(path)
        parent = os.path.dirname(path) or "."
        os.makedirs(parent, exist_ok=True)
        tmp = os.path.join(parent, f".{os.path.basename(path) or 'session'}.tmp-{os.getpid()}-{id(data)}")
        fd = os.open(tmp, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
        try:
            with os.fdopen(fd, "wb") as f:
                f.write(data)
                f.flush()
                os.fsync(f.fileno())
            os.replace(tmp, path)
        except BaseException:
            if os.path.exists(tmp):
                os.remove(tmp)
            raise
        dfd = os.open(parent, os.O_RDONLY)
        try:
            os.fsync(dfd)
        finally:
            os.close(dfd)

    def restore_session_from_file(self, path) -> None:
        """session.rs:3264-3290: bounded by max_serialized_session_bytes before reading."""
        bound = max_serialized_session_bytes(self.info)
        if os.path.getsize(path) > bound:
            raise SessionError("Numerics", f"session file size {os.path.getsize(path)} exceeds "
                                           f"maximum expected bound {bound}")
        with open(path, "rb") as f:
            data = f.read(bound + 1)
        if len(data) > bound:
            raise SessionError("Numerics", f"session file size exceeds maximum expected bound {bound}")
        try:
            saved = from_json(data)
        except CodecError as e:
            raise SessionError("Numerics", str(e)) from None
        self.restore_state(saved)


def serve_steps(sessions: list[Session], tokens: list[int]) -> list[tuple[int, int]]:
    """serve_step for many sessions of one pool in one launch: the serving loop's batch. A
    session whose token is refused raises after the others have stepped."""
    if not sessions:
        return []
    pool = sessions[0].pool
    if any(s.pool is not pool for s in sessions):
        raise ValueError("sessions of one pool")
    go, errs = [], []
    for s, tok in zip(sessions, tokens):
        ok, err = s._admit([tok])
        (go.append((s, ok)) if ok else errs.append(err))
    if go:
        traced = any(s.trace is not None for s, _ in go) and pool.info.snapped
        out = pool.run([s.slot for s, _ in go], np.asarray([ok for _, ok in go], np.uint32),
                       native=True, trace=traced)
        for i, (s, ok) in enumerate(go):
            st = int(out["status"][i])
            if st:
                errs.append(SessionError(*_STATUS.get(st, ("Shape", f"status {st}"))))
                continue
            s._after(ok, out["reply"][i], out["kept"][i], out["query"][i],
                     out["trace"][i] if traced else None)
    if errs:
        raise errs[0]
    return [(s._native.token, 0) for s in sessions]
