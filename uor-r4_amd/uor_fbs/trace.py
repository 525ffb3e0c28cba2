"""The Hamming trace and the decision trace with the forced replay: the reference's record types
(HammingStepRead / HammingStepHead, stack/hamming.rs:1378-1395; DecisionStep, DecisionLayer,
DecisionRead, DecisionHead, DecisionNearest, DecisionForceWindow, ForcedBucket, ForcedCode,
fbs_snapshot.rs:643-797), the byte layout of a traced position's record as
uor_fbs_decision_sequences writes it, and the forced set's arrays.

A record holds, with the decisions, each layer's rate scores (i32 [layer][lane]) and the entries
used (u8 [layer][lane]), padded to 8 bytes; then each Hamming read in depth order, each head it
serves (the copy heads, then the type heads where the read serves them): the query (u64), the key
at the row (u64), the kept count (u32) and the kept positions (u32, `kept` of them), padded to 8
bytes.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

HEAD_FIXED = 20


@dataclass
class HammingStepHead:
    query: int
    key: int
    kept: list


@dataclass
class HammingStepRead:
    depth: int
    heads: list


@dataclass
class DecisionLayer:
    score_q16: list
    entry: list
    read: HammingStepRead | None = None


@dataclass
class DecisionNearest:
    """The whole table's top two by -L1 at Q12, ties to the smaller id, and the query."""
    pick: int
    score_q12: int
    runner_up: int
    runner_score_q12: int
    query_q12: list


@dataclass
class DecisionStep:
    layers: list
    readout: HammingStepRead | None = None
    memory: None = None       # this path serves no turn memory
    nearest: DecisionNearest | None = None


@dataclass
class ForcedBucket:
    step: int
    layer: int
    lane: int
    entry: int


@dataclass
class ForcedCode:
    step: int
    depth: int
    head: int
    role: str      # "query" or "key"
    code: int


@dataclass
class DecisionForceWindow:
    position: int = 0
    buckets: list = field(default_factory=list)
    codes: list = field(default_factory=list)


class TraceError(ValueError):
    pass


def head_bytes(kept: int) -> int:
    return (HEAD_FIXED + 4 * kept + 7) & ~7


@dataclass(frozen=True)
class TraceLayout:
    """Where a record's parts sit, for a model's shape and reads."""
    layers: int
    lanes: int
    decisions: bool
    depths: tuple         # each read's depth, in order
    served: tuple         # each read's served heads
    heads: int            # heads a read has (copy + type)
    kept: int

    @staticmethod
    def of(art, decisions: bool) -> "TraceLayout":
        s = art.spec
        ham = getattr(art, "hamming", None)
        reads = getattr(art, "hamming_reads", None) or []
        depths, served = [], []
        for r in reads:
            place_read = ham.place is not None and r.depth == s.layers
            typed = bool(np.any(np.asarray(r.weight)[s.width:] != 0)) and not place_read
            depths.append(int(r.depth))
            served.append(ham.heads // 2 + (ham.heads - ham.heads // 2 if typed else 0))
        return TraceLayout(s.layers, s.width // 4, bool(decisions), tuple(depths), tuple(served),
                           ham.heads if ham else 0, ham.kept if ham else 0)

    @property
    def bucket_bytes(self) -> int:
        return (5 * self.layers * self.lanes + 7) & ~7 if self.decisions else 0

    @property
    def stride(self) -> int:
        return self.bucket_bytes + sum(self.served) * head_bytes(self.kept)

    def reads(self, rec: bytes) -> list:
        """The record's reads, in depth order."""
        out, at, hb = [], self.bucket_bytes, head_bytes(self.kept)
        for depth, n in zip(self.depths, self.served):
            heads = []
            for _ in range(n):
                q, k, c = np.frombuffer(rec, np.uint64, 2, at), None, None
                c = int(np.frombuffer(rec, np.uint32, 1, at + 16)[0])
                kept = np.frombuffer(rec, np.uint32, c, at + HEAD_FIXED).tolist() if c else []
                heads.append(HammingStepHead(int(q[0]), int(q[1]), kept))
                at += hb
            out.append(HammingStepRead(depth, heads))
        return out

    def step(self, rec: bytes) -> DecisionStep:
        """A record as the decision trace's step (the nearest is the caller's to add)."""
        L, n = self.layers, self.layers * self.lanes
        score = np.frombuffer(rec, np.int32, n, 0).reshape(L, self.lanes)
        entry = np.frombuffer(rec, np.uint8, n, 4 * n).reshape(L, self.lanes)
        reads = {r.depth: r for r in self.reads(rec)}
        layers = [DecisionLayer(score[l].tolist(), entry[l].tolist(),
                                reads.get(l + 1) if l + 1 < L else None) for l in range(L)]
        return DecisionStep(layers, reads.get(L))

    def force_arrays(self, windows: list, sequences: int, length: int):
        """The forced sets of each sequence's window as the launch's arrays (buckets, codes,
        mask), None where nothing is forced; refused as `forcing` and set_decision_trace refuse
        (hamming.rs:1686-1740, session.rs:2471-2498)."""
        R, H = len(self.depths), self.heads
        fb = np.full((sequences, length, self.layers, self.lanes), 255, np.uint8)
        codes = np.zeros((sequences, length, max(R, 1), max(H, 1), 2), np.uint64)
        mask = np.zeros((sequences, length, max(R, 1), max(H, 1)), np.uint8)
        any_b = any_c = False
        for i, w in enumerate(windows or []):
            if w is None:
                continue
            for b in w.buckets:
                if (b.step >= length or b.layer >= self.layers or b.lane >= self.lanes
                        or not 0 <= b.entry <= 15):
                    raise TraceError("a forced bucket names a step, layer, lane or entry outside the model")
                if fb[i, b.step, b.layer, b.lane] != 255:
                    raise TraceError("a bucket is forced twice")
                fb[i, b.step, b.layer, b.lane] = b.entry
                any_b = True
            for c in w.codes:
                if c.depth not in self.depths:
                    raise TraceError("a forced code names a depth no read runs at")
                r = self.depths.index(c.depth)
                if not 0 <= c.head < self.served[r]:
                    raise TraceError("a forced code names a head its read does not serve")
                if c.step >= length:
                    raise TraceError("a forced code names a step past the context")
                role = {"query": 0, "key": 1}[c.role]
                if role == 1 and c.step == 0:
                    raise TraceError("a forced key at step 0 names no candidate")
                if mask[i, c.step, r, c.head] & (1 << role):
                    raise TraceError("a code is forced twice")
                mask[i, c.step, r, c.head] |= 1 << role
                codes[i, c.step, r, c.head, role] = c.code
                any_c = True
        if any_b and not self.decisions:
            raise TraceError("forced buckets need the decision trace")
        return (fb if any_b else None, codes if any_c else None, mask if any_c else None)


def nearest(query_q12, table) -> DecisionNearest:
    """The whole table's top two by -sum |q - T_u| at Q12, ties to the smaller id."""
    q = np.asarray(query_q12, np.int64)
    t = np.asarray(table, np.int64).reshape(-1, len(q))
    l1 = np.abs(t - q).sum(1)
    order = np.lexsort((np.arange(len(l1)), l1))
    a, b = int(order[0]), int(order[1])
    return DecisionNearest(a, -int(l1[a]), b, -int(l1[b]), q.astype(int).tolist())
