"""The 256-cell CSR drawer index on the GPU, with the API of the reference's inverted file
(projects/uor-cuda-inverted-file/include/uor_inverted_file.hpp:10-50): `build`, `update`,
`remove_token`, `validate`, `validate_structure`, `probe` and `full_scan` over the C ABI's
uor_fbs_index_* entry points (include/uor_fbs.h), with the reference's Status values
(hpp:29-37) and refusal order.

A table is `count` token rows of `width` int32 (the reference's Token is width 32: four blocks
of 8) and 16 roots of 8 values (the reference's codebook, src/codebook.cpp:5-14). A token's
cell is first_root * 16 + last_root when its first and last 8 values are roots, else ABSENT.
The index keeps offsets [257], members (each cell's tokens ascending), every token's cell and
the absent count, all in device memory (hipmem.DeviceArray, on the HIP runtime the library
links); `Index.to_host()` copies them out as a HostIndex, the reference's Index.

Where this differs from the host library: `probe` validates the index first only when
`check` is true (the default, as the reference's probe does on every call); a serving loop
validates once per change and probes with check=False. There is no other implementation: a
missing library or device raises.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass

import numpy as np

from . import hip
from .hipmem import DeviceArray

ABSENT = 0xFFFFFFFF
MAX_WIDTH = 256
MAX_TOKENS = 1 << 30


# The reference's 16 roots (src/codebook.cpp:5-14), the table its inverted file and tests use.
CODEBOOK = np.array([
    [2, 2, 0, 0, 0, 0, 0, 0], [-2, -2, 0, 0, 0, 0, 0, 0], [-2, 2, 0, 0, 0, 0, 0, 0],
    [0, 0, -2, 0, -2, 0, 0, 0], [0, 0, -2, 0, 2, 0, 0, 0], [0, 0, 0, -2, 0, 0, 0, -2],
    [0, 0, 0, -2, 0, 0, 0, 2], [0, 0, 0, 0, 0, -2, -2, 0], [0, 0, 0, 0, 0, -2, 2, 0],
    [0, 0, 0, 0, 0, 2, -2, 0], [0, 0, 0, 0, 0, 2, 2, 0], [0, 0, 0, 2, 0, 0, 0, -2],
    [0, 0, 0, 2, 0, 0, 0, 2], [0, 0, 2, 0, -2, 0, 0, 0], [0, 0, 2, 0, 2, 0, 0, 0],
    [2, -2, 0, 0, 0, 0, 0, 0]], dtype=np.int32)


def seeded_table(count: int) -> np.ndarray:
    """The reference tests' seeded width-32 table (tests/inverted_file_test.cpp:39-53,
    token_at / table_of): token i's endpoints are roots (7i+1) mod 16 and (11i+3) mod 16, its
    middle blocks (29i+7d) mod 37 - 18 and (13i+5d) mod 41 - 20."""
    i = np.arange(count, dtype=np.int64)[:, None]
    d = np.arange(8, dtype=np.int64)[None, :]
    t = np.empty((count, 4, 8), np.int32)
    t[:, 0] = CODEBOOK[(i[:, 0] * 7 + 1) % 16]
    t[:, 1] = (i * 29 + d * 7) % 37 - 18
    t[:, 2] = (i * 13 + d * 5) % 41 - 20
    t[:, 3] = CODEBOOK[(i[:, 0] * 11 + 3) % 16]
    return t.reshape(count, 32)


def seeded_query(seed: int) -> np.ndarray:
    """The reference tests' query (tests/inverted_file_test.cpp:63-71, query_at)."""
    d = np.arange(8, dtype=np.int64)
    q = np.empty((4, 8), np.int32)
    q[0] = CODEBOOK[seed % 16]
    q[1] = (seed * 11 + d * 3) % 23 - 11
    q[2] = (seed * 17 + d * 2) % 19 - 9
    q[3] = CODEBOOK[(seed * 5 + 1) % 16]
    return q.reshape(32)


class Status(enum.IntEnum):
    """uor_inverted_file::Status (hpp:29-37); the CUDA and telemetry values have no use here."""
    Ok = 0
    InvalidArgument = 1
    NonRootBlock = 2
    CsrInvariant = 3


@dataclass
class HostIndex:
    """uor_inverted_file::Index (hpp:19-24) in host memory."""
    offsets: np.ndarray  # uint32 [257]
    members: np.ndarray  # uint32 [offsets[256]]
    cells: np.ndarray    # uint32 [count]
    absent_count: int

    def copy(self) -> "HostIndex":
        return HostIndex(self.offsets.copy(), self.members.copy(), self.cells.copy(),
                         int(self.absent_count))

    def same(self, other: "HostIndex") -> bool:
        return (np.array_equal(self.offsets, other.offsets)
                and np.array_equal(self.members, other.members)
                and np.array_equal(self.cells, other.cells)
                and int(self.absent_count) == int(other.absent_count))


@dataclass
class ScanResult:
    """Per query row: uor_inverted_file::ScanResult (hpp:26-30) and the call's status."""
    status: np.ndarray      # int32 [rows]
    prediction: np.ndarray  # uint32 [rows]
    admitted: np.ndarray    # uint32 [rows, 16]
    top8: np.ndarray        # uint32 [rows, 8]


def _rows(a, width=None, name="rows") -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int32)
    if a.ndim != 2 or (width is not None and a.shape[1] != width):
        raise ValueError(f"{name} must be [n, {width or 'width'}] int32")
    return a


class Table:
    """Token rows [count, width] and roots [16, 8] resident on a HIP device."""

    def __init__(self, rows, roots, device: int = 0):
        rows = _rows(rows)
        roots = np.ascontiguousarray(roots, dtype=np.int32)
        self.count, self.width = rows.shape
        if roots.shape != (16, 8):
            raise ValueError("roots must be [16, 8] int32")
        if not (16 <= self.width <= MAX_WIDTH and self.width % 4 == 0):
            raise ValueError(f"width {self.width}: a multiple of 4 in 16..{MAX_WIDTH}")
        if not 0 < self.count <= MAX_TOKENS:
            raise ValueError(f"{self.count} tokens (1..{MAX_TOKENS})")
        self.device = device
        self.rows = DeviceArray((self.count, self.width), np.int32, device)
        self.rows.upload(rows)
        self.roots = DeviceArray((16, 8), np.int32, device)
        self.roots.upload(roots)

    def set_row(self, token: int, row):
        """A codebook change: token `token`'s row becomes `row` (then `update` the index)."""
        if not 0 <= token < self.count:
            raise IndexError(token)
        self.rows.upload(np.asarray(row, dtype=np.int32).reshape(self.width), row=token)


class Index:
    """An index's device buffers for a table of `count` tokens, with its own workspace."""

    def __init__(self, count: int, device: int = 0):
        if not 0 < count <= MAX_TOKENS:
            raise ValueError(f"{count} tokens (1..{MAX_TOKENS})")
        self.count, self.device = count, device
        self.offsets = DeviceArray(257, np.uint32, device)
        self.members = DeviceArray(count, np.uint32, device)
        self.cells = DeviceArray(count, np.uint32, device)
        self.absent = DeviceArray(1, np.uint32, device)
        ws = int(hip.lib().uor_fbs_index_workspace_bytes(count))
        self.workspace = DeviceArray(ws // 4, np.uint32, device)
        self.status = DeviceArray(1, np.int32, device)

    def to_host(self) -> HostIndex:
        offsets = self.offsets.download()
        used = min(int(offsets[256]), self.count)
        return HostIndex(offsets, self.members.download()[:used], self.cells.download(),
                         int(self.absent.download()[0]))

    def load(self, host: HostIndex):
        """Copies a host index in (members beyond the host's are left as they are)."""
        if len(host.cells) != self.count or len(host.members) > self.count:
            raise ValueError("index sizes do not match the table")
        self.offsets.upload(np.asarray(host.offsets, dtype=np.uint32))
        members = self.members.download()
        members[:len(host.members)] = host.members
        self.members.upload(members)
        self.cells.upload(np.asarray(host.cells, dtype=np.uint32))
        self.absent.upload(np.array([host.absent_count], np.uint32))

    def _status(self) -> Status:
        return Status(int(self.status.download()[0]))


def _launched(code: int):
    if code:
        hip._check(code)


def build(table: Table, index: Index, allow_absent: bool = False) -> Status:
    """build (inverted_file.cpp:112-138, 173-175)."""
    if index.count != table.count:
        return Status.InvalidArgument
    _launched(hip.lib().uor_fbs_index_build_async(
        table.rows.ptr, table.count, table.width, table.roots.ptr, int(allow_absent),
        index.offsets.ptr, index.members.ptr, index.cells.ptr, index.absent.ptr,
        index.workspace.ptr, index.status.ptr, None))
    return index._status()


def update(table: Table, moved: int, index: Index) -> Status:
    """update (inverted_file.cpp:182-236): token `moved`'s row changed."""
    if index.count != table.count or moved < 0:
        return Status.InvalidArgument
    _launched(hip.lib().uor_fbs_index_update_async(
        table.rows.ptr, table.count, table.width, table.roots.ptr, moved, index.offsets.ptr,
        index.members.ptr, index.cells.ptr, index.absent.ptr, index.workspace.ptr,
        index.status.ptr, None))
    return index._status()


def remove_token(table: Table, moved: int, index: Index) -> Status:
    """remove_token (inverted_file.cpp:238-249): token `moved` becomes ABSENT."""
    if index.count != table.count or moved < 0:
        return Status.InvalidArgument
    _launched(hip.lib().uor_fbs_index_remove_async(
        table.count, moved, index.offsets.ptr, index.members.ptr, index.cells.ptr,
        index.absent.ptr, index.workspace.ptr, index.status.ptr, None))
    return index._status()


def validate(table: Table, index: Index) -> Status:
    """validate (inverted_file.cpp:164-176)."""
    if index.count != table.count:
        return Status.CsrInvariant
    _launched(hip.lib().uor_fbs_index_validate_async(
        table.rows.ptr, table.count, table.width, table.roots.ptr, index.offsets.ptr,
        index.members.ptr, index.cells.ptr, index.absent.ptr, index.workspace.ptr,
        index.status.ptr, None))
    return index._status()


def validate_structure(index: Index) -> Status:
    """validate_structure (inverted_file.cpp:141-162)."""
    _launched(hip.lib().uor_fbs_index_validate_async(
        None, index.count, 16, None, index.offsets.ptr, index.members.ptr, index.cells.ptr,
        index.absent.ptr, index.workspace.ptr, index.status.ptr, None))
    return index._status()


def _every(rows: int, status: Status) -> ScanResult:
    return ScanResult(np.full(rows, int(status), np.int32), np.full(rows, ABSENT, np.uint32),
                      np.full((rows, 16), ABSENT, np.uint32), np.full((rows, 8), ABSENT, np.uint32))


def _scan(entry, table: Table, queries, k: int, offsets, members) -> ScanResult:
    q = _rows(queries, table.width, "queries")
    n = q.shape[0]
    if not 1 <= k <= 16 or n == 0:
        return _every(n, Status.InvalidArgument)
    dev = table.device
    d_q = DeviceArray(q.shape, np.int32, dev)
    d_q.upload(q)
    pred = DeviceArray(n, np.uint32, dev)
    adm = DeviceArray((n, 16), np.uint32, dev)
    top = DeviceArray((n, 8), np.uint32, dev)
    st = DeviceArray(n, np.int32, dev)
    args = [table.rows.ptr, table.count, table.width, table.roots.ptr, d_q.ptr, n, k, offsets.ptr]
    if members is not None:
        args.append(members.ptr)
    _launched(entry(*args, pred.ptr, adm.ptr, top.ptr, st.ptr, None))
    return ScanResult(st.download(), pred.download(), adm.download(), top.download())


def probe(table: Table, queries, k: int, index: Index, check: bool = True) -> ScanResult:
    """probe (inverted_file.cpp:250-258) for every row of `queries` [rows, width]. The status
    of a row: Ok, InvalidArgument (k outside 1..16, or nothing admitted), CsrInvariant (the
    index fails validation when `check`, or points outside the table)."""
    rows = _rows(queries, table.width, "queries").shape[0]
    if not 1 <= k <= 16:
        return _every(rows, Status.InvalidArgument)
    if check and validate(table, index) != Status.Ok:
        return _every(rows, Status.CsrInvariant)
    return _scan(hip.lib().uor_fbs_index_probe_async, table, queries, k, index.offsets,
                 index.members)


def full_scan(table: Table, queries, k: int, index: Index | None = None) -> ScanResult:
    """full_scan (inverted_file.cpp:260-270): cells admitted from an index of the table built
    with absent tokens allowed (built here, in `index` when given), then every token of the
    table in an admitted cell ranked."""
    rows = _rows(queries, table.width, "queries").shape[0]
    if not 1 <= k <= 16:
        return _every(rows, Status.InvalidArgument)
    index = index or Index(table.count, table.device)
    st = build(table, index, allow_absent=True)
    if st != Status.Ok:
        return _every(rows, st)
    return _scan(hip.lib().uor_fbs_index_full_scan_async, table, queries, k, index.offsets, None)


__all__ = ["ABSENT", "CODEBOOK", "seeded_table", "seeded_query", "Status", "HostIndex", "ScanResult", "Table", "Index", "build", "update",
           "remove_token", "validate", "validate_structure", "probe", "full_scan"]
