"""Execution feature order on the host side of the engine: the popularity order of a
quantized CSR's genes, the packed dense operand (W rows in execution order), and the
quantized CSR relabelled into execution order -- thin ctypes mirrors of the C-ABI entries
(include/cellerator_amd.h, exec_order.hip / exec_csr.cpp). The reference's counterparts are
pack_dense_operand_{host,cuda} (include/Cellerator/compute/math/packed_dense_operand.hh:16-70)
and execution_csr_view (include/Cellerator/compute/math/physical_csr.hh:40-215).
"""
from __future__ import annotations

import contextlib
import ctypes as C
import dataclasses
from typing import Optional

import numpy as np
import torch

from . import _native as N
from .engine import QcsrMatrix, _require_cuda, _stream, _torch_stream


def _on(stream, device):
    """Context in which torch allocations belong to the launch stream: buffers written by
    kernels on a caller's stream are then not handed out again before that stream is past
    them (torch's caching allocator keys reuse on the allocating stream)."""
    if stream is None:
        return contextlib.nullcontext()
    return torch.cuda.stream(_torch_stream(stream, device))


def _record(t: torch.Tensor, stream) -> None:
    """Marks a cached buffer as used by `stream` (see _on)."""
    if stream is not None:
        t.record_stream(_torch_stream(stream, t.device))


@dataclasses.dataclass
class ExecutionOrder:
    """feature_permutation[e] = canonical gene at execution position e; inverse the other
    way round. Both int32-stored u32 device tensors of length genes."""
    feature_permutation: torch.Tensor
    inverse_permutation: torch.Tensor

    @property
    def genes(self) -> int:
        return int(self.feature_permutation.numel())


def column_counts(m: QcsrMatrix, stream=None) -> torch.Tensor:
    """Stored entries per gene (device u32 as int32)."""
    _require_cuda(m.col_idx)
    counts = torch.empty(max(m.cols, 1), dtype=torch.int32, device=m.col_idx.device)
    d = m.descriptor()
    N.check("cx_qcsr_column_counts", N.engine().cx_qcsr_column_counts(C.byref(d), counts.data_ptr(),
                                                                      _stream(stream)))
    return counts[: m.cols]


def popularity_order(m: QcsrMatrix, stream=None) -> ExecutionOrder:
    """Genes by descending stored-entry count (ties by gene index): the order whose leading
    genes are dense enough for matrix-core tiles."""
    counts = column_counts(m, stream).cpu().numpy().view(np.uint32)
    perm = np.empty(m.cols, np.uint32)
    inv = np.empty(m.cols, np.uint32)
    lib = N.engine()
    st = lib.cx_popularity_order(counts.ctypes.data, m.cols, perm.ctypes.data, inv.ctypes.data)
    if st != 0:
        raise N.EngineError("cx_popularity_order", st, lib.cx_exec_last_error().decode())
    dev = m.col_idx.device
    return ExecutionOrder(torch.from_numpy(perm.view(np.int32)).to(dev),
                          torch.from_numpy(inv.view(np.int32)).to(dev))


def head_order(m: QcsrMatrix, head_cols: int, stream=None) -> tuple[ExecutionOrder, int]:
    """The execution order a prepared projection uses (cx_qcsr_head_order): the popularity
    order with every gene the matrix-core head cannot carry exactly moved after the head, and
    the head width it supports (head_cols capped at cols rounded down to 1,024, or fewer when
    fewer genes qualify)."""
    counts = column_counts(m, stream).cpu().numpy().view(np.uint32)

    def host(t: Optional[torch.Tensor]) -> Optional[np.ndarray]:
        return None if t is None else np.ascontiguousarray(t.detach().cpu().numpy().astype(np.float32, copy=False))

    scales, offsets, row_offsets = host(m.column_scales), host(m.column_offsets), host(m.row_offsets)
    perm = np.empty(m.cols, np.uint32)
    inv = np.empty(m.cols, np.uint32)
    head = C.c_uint32()
    lib = N.engine()

    def ptr(a):
        return None if a is None else a.ctypes.data

    st = lib.cx_qcsr_head_order(counts.ctypes.data, m.cols, m.bits, m.decode_policy, ptr(scales),
                                ptr(offsets) if m.decode_policy == N.DECODE_PER_GENE_AFFINE else None,
                                ptr(row_offsets) if m.decode_policy == N.DECODE_COLUMN_SCALE_ROW_OFFSET else None,
                                m.rows, head_cols,
                                perm.ctypes.data, inv.ctypes.data, C.byref(head))
    N.check("cx_qcsr_head_order", st)
    dev = m.col_idx.device
    return (ExecutionOrder(torch.from_numpy(perm.view(np.int32)).to(dev),
                           torch.from_numpy(inv.view(np.int32)).to(dev)), int(head.value))


def pack_rows(order: ExecutionOrder, canonical: torch.Tensor, stream=None) -> torch.Tensor:
    """Rows of a feature-major device tensor [genes, ...] gathered into execution order
    (cx_pack_dense_operand): the packed dense operand for a row-major W, or the per-gene
    metadata for a 1-D tensor (8-byte rows for interleaved pairs given as [genes, 2])."""
    _require_cuda(canonical)
    if canonical.shape[0] != order.genes or not canonical.is_contiguous():
        raise ValueError("canonical must be a contiguous [genes, ...] tensor")
    flat = canonical.reshape(order.genes, -1)
    row_bytes = flat.shape[1] * flat.element_size()
    if row_bytes in (1, 2, 4, 8):
        cols, ld, vsize = 1, 1, row_bytes
    else:
        cols, ld, vsize = flat.shape[1], flat.shape[1], flat.element_size()
    out = torch.empty_like(canonical)
    N.check("cx_pack_dense_operand", N.engine().cx_pack_dense_operand(
        order.feature_permutation.data_ptr(), order.genes, canonical.data_ptr(), cols, ld, 0, vsize,
        out.data_ptr(), out.numel() * out.element_size(), _stream(stream)))
    return out


def to_execution_order(m: QcsrMatrix, order: ExecutionOrder, stream=None) -> QcsrMatrix:
    """The matrix with genes relabelled by `order` and every row re-sorted (codes carried),
    per-gene metadata permuted alongside; row offsets are shared with `m`. Raises if a row
    repeats a gene or holds a column outside [0, cols)."""
    _require_cuda(m.row_ptr, m.col_idx)
    if order.genes != m.cols:
        raise ValueError("order must cover every gene of the matrix")
    dev = m.col_idx.device
    col_out = torch.empty_like(m.col_idx)
    packed_out = torch.zeros_like(m.packed_values) if m.packed_values is not None else None
    values_out = torch.empty_like(m.values) if m.values is not None else None
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    d = m.descriptor()
    s = _stream(stream)
    N.check("cx_qcsr_to_execution_order", N.engine().cx_qcsr_to_execution_order(
        C.byref(d), order.inverse_permutation.data_ptr(), col_out.data_ptr(),
        packed_out.data_ptr() if packed_out is not None else None,
        values_out.data_ptr() if values_out is not None else None, err.data_ptr(), s))
    ts = torch.cuda.ExternalStream(s, device=dev) if stream is not None else torch.cuda.current_stream(dev)
    with torch.cuda.stream(ts):
        bad = int(err.item())
    if bad:
        raise ValueError("to_execution_order: a row repeats a gene or holds a column outside [0, cols)")

    def meta(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if t is None:
            return None
        if m.decode_policy == N.DECODE_PER_GENE_AFFINE_PAIRS and t is m.column_scales:
            return pack_rows(order, t.view(m.cols, 2), stream).view(-1)
        return pack_rows(order, t, stream)

    return QcsrMatrix(m.rows, m.cols, m.bits, m.row_ptr, col_out, packed_row_ptr=m.packed_row_ptr,
                      packed_values=packed_out, column_scales=meta(m.column_scales),
                      column_offsets=meta(m.column_offsets), row_offsets=m.row_offsets,
                      values=values_out, decode_policy=m.decode_policy,
                      meta={**m.meta, "execution_order": order}, flags=N.QCSR_COLUMNS_SORTED)


@dataclasses.dataclass
class HybridProjection:
    """A quantized CSR in execution order prepared for cx_qcsr_spmm_fwd_hybrid: the dense
    copy of its first head_cols genes (codes and presence bits; head_cols a multiple of
    1,024), each row's first tail entry, and the pre-scaled head metadata. Built once per
    matrix by hybrid_prepare; independent of the weights."""
    matrix: QcsrMatrix
    head_cols: int
    layout: N.CxQcsrHybridLayout
    storage: Optional[torch.Tensor]
    workspaces: dict = dataclasses.field(default_factory=dict)
    tail: Optional[N.CxQcsrTailStream] = None        # prepared tail stream (hybrid_prepare(..., stream_tail=True))
    tail_storage: tuple = ()                         # (plan storage, entries) tensors behind `tail`

    @property
    def scale_exp(self) -> int:
        return int(self.layout.scale_exp)

    def workspace(self, out_cols: int, device) -> torch.Tensor:
        ws = self.workspaces.get(out_cols)
        if ws is None:
            nbytes = C.c_uint64()
            d = self.matrix.descriptor()
            N.check("cx_qcsr_hybrid_workspace", N.engine().cx_qcsr_hybrid_workspace(
                C.byref(d), self.head_cols, out_cols, C.byref(nbytes)))
            ws = torch.empty(max(nbytes.value, 256), dtype=torch.uint8, device=device)
            self.workspaces[out_cols] = ws
        return ws


def hybrid_prepare(m: QcsrMatrix, head_cols: int, stream=None, stream_tail: bool = False) -> HybridProjection:
    """m in execution order (sorted rows, flags QCSR_COLUMNS_SORTED). Raises if a row's genes
    are not strictly increasing or the head metadata is not finite. With stream_tail the
    tail's entries are also rearranged into the prepared tail stream (cx_qcsr_tail_plan /
    cx_qcsr_tail_fill), which the tail kernel then reads instead of the CSR."""
    _require_cuda(m.row_ptr)
    lib = N.engine()
    d = m.descriptor()
    nbytes = C.c_uint64()
    N.check("cx_qcsr_hybrid_layout_bytes", lib.cx_qcsr_hybrid_layout_bytes(C.byref(d), head_cols, C.byref(nbytes)))
    with _on(stream, m.row_ptr.device):
        storage = torch.empty(max(nbytes.value, 256), dtype=torch.uint8, device=m.row_ptr.device)
    layout = N.CxQcsrHybridLayout()
    N.check("cx_qcsr_hybrid_prepare", lib.cx_qcsr_hybrid_prepare(
        C.byref(d), head_cols, storage.data_ptr(), storage.numel(), C.byref(layout), _stream(stream)))
    p = HybridProjection(m, head_cols, layout, storage)
    if stream_tail:
        tail_prepare(p, stream)
    return p


def tail_prepare(p: HybridProjection, stream=None) -> N.CxQcsrTailStream:
    """Plans and fills the prepared tail stream of p and attaches it (p.layout.tail)."""
    lib = N.engine()
    d = p.matrix.descriptor()
    dev = p.matrix.row_ptr.device
    nbytes = C.c_uint64()
    N.check("cx_qcsr_tail_plan_bytes", lib.cx_qcsr_tail_plan_bytes(C.byref(d), C.byref(p.layout), C.byref(nbytes)))
    with _on(stream, dev):
        plan = torch.empty(max(nbytes.value, 256), dtype=torch.uint8, device=dev)
    ts = N.CxQcsrTailStream()
    entry_bytes = C.c_uint64()
    N.check("cx_qcsr_tail_plan", lib.cx_qcsr_tail_plan(C.byref(d), C.byref(p.layout), plan.data_ptr(), plan.numel(),
                                                        C.byref(ts), C.byref(entry_bytes), _stream(stream)))
    with _on(stream, dev):
        entries = torch.empty(max(entry_bytes.value, 256), dtype=torch.uint8, device=dev)
    N.check("cx_qcsr_tail_fill", lib.cx_qcsr_tail_fill(C.byref(d), C.byref(p.layout), C.byref(ts),
                                                        entries.data_ptr(), entries.numel(), _stream(stream)))
    p.tail, p.tail_storage = ts, (plan, entries)
    p.layout.tail = C.addressof(ts)
    return ts


def tail_arrays(p: HybridProjection):
    """(slot_rows [blocks, block_rows] int32 (u32 bits), fill_index [blocks * parts *
    block_rows / 8 + 1] int32 in (block, wave, part, layer) order, entries [fills, 128] int16
    or int32) of the prepared tail stream, as device views."""
    ts = p.tail
    plan, entries = p.tail_storage

    def view(t, ptr, count, dtype):
        off = ptr - t.data_ptr()
        size = torch.tensor([], dtype=dtype).element_size()
        return t[off:off + count * size].view(dtype)

    br = int(ts.block_rows)
    n = int(ts.blocks) * int(ts.parts) * (br // 8) + 1
    slot_rows = view(plan, ts.slot_rows, int(ts.blocks) * br, torch.int32).view(int(ts.blocks), br)
    index = view(plan, ts.fill_index, n, torch.int32)
    et = torch.int32 if ts.entry_bytes == 4 else torch.int16
    ents = view(entries, ts.entries, int(ts.fills) * 128, et).view(int(ts.fills), 128)
    return slot_rows, index, ents


def hybrid_head_arrays(p: HybridProjection):
    """The prepared head as device tensor views: (codes, masks, head_end, meta) in the words
    form -- codes [H * bits / 32, rows_ld] and masks [H / 32, rows_ld] int32 (u32 bits) --
    or (code_bytes, lut, head_end, meta) in the table form -- code_bytes [H / 32, rows_ld, 32]
    uint8 and lut [H, 17, 4] int16 (fp16 bits); head_end [rows] int32, meta [H, 2] float32
    (times 2^scale_exp)."""
    L, base = p.layout, p.storage.data_ptr()

    def view(ptr, count, dtype, shape):
        off = ptr - base
        size = torch.tensor([], dtype=dtype).element_size()
        return p.storage[off:off + count * size].view(dtype).view(shape)

    h, ld = p.head_cols, int(L.rows_ld)
    head_end = view(L.head_end, int(L.rows), torch.int32, (int(L.rows),))
    meta = view(L.meta, 2 * h, torch.float32, (h, 2))
    if L.head_form == N.HEAD_FORM_TABLE:
        code_bytes = view(L.code_bytes, h * ld, torch.uint8, (h // 32, ld, 32))
        lut = view(L.lut, h * 17 * 4, torch.int16, (h, 17, 4))
        return code_bytes, lut, head_end, meta
    codes = view(L.codes, h * L.bits // 32 * ld, torch.int32, (h * L.bits // 32, ld))
    masks = view(L.masks, h // 32 * ld, torch.int32, (h // 32, ld))
    return codes, masks, head_end, meta


def hybrid_spmm(p: HybridProjection, w: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None,
                epilogue=None) -> torch.Tensor:
    """Y = X . W (+ epilogue) on the prepared execution-order projection; w = the
    execution-order weights (F16 [genes, N], N in 64..256 by 64). Y rows are the matrix's
    rows (cells keep their order), columns the weights' columns."""
    m = p.matrix
    _require_cuda(w)
    if w.dim() != 2 or w.shape[0] != m.cols or w.dtype != torch.float16 or w.stride(1) != 1:
        raise ValueError("w must be a row-major F16 [genes, N] tensor")
    n = int(w.shape[1])
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=w.device)
    d = m.descriptor()
    e = epilogue.descriptor(out) if epilogue is not None else None
    ws = p.workspace(n, w.device) if p.head_cols else None
    if ws is not None:
        _record(ws, stream)
    N.check("cx_qcsr_spmm_fwd_hybrid", N.engine().cx_qcsr_spmm_fwd_hybrid(
        C.byref(d), C.byref(p.layout), w.data_ptr(), w.stride(0), n, out.data_ptr(), out.stride(0),
        C.byref(e) if e is not None else None, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream(stream)))
    return out


class ExecProjection:
    """The prepared execution-order projection of a quantized CSR (cx_qcsr_exec_prepare): the
    engine object that owns the popularity order, the execution-order metadata, the dense head
    and the tail stream. Launches (spmm) take canonical W and return Y in the matrix's row
    order. The device memory is held until close() (or garbage collection)."""

    def __init__(self, m: QcsrMatrix, head_cols: int = 2048, stream=None):
        _require_cuda(m.row_ptr)
        self._lib = N.engine()
        self._handle = C.c_void_p()
        d = m.descriptor()
        N.check("cx_qcsr_exec_prepare", self._lib.cx_qcsr_exec_prepare(C.byref(d), head_cols, C.byref(self._handle),
                                                                        _stream(stream)))
        self.device = m.row_ptr.device
        self.rows, self.cols = m.rows, m.cols
        self._workspaces: dict = {}

    @property
    def handle(self) -> int:
        return int(self._handle.value or 0)

    def info(self) -> N.CxQcsrExecInfo:
        i = N.CxQcsrExecInfo()
        N.check("cx_qcsr_exec_query", self._lib.cx_qcsr_exec_query(self._handle, C.byref(i)))
        return i

    def workspace(self, out_cols: int) -> torch.Tensor:
        ws = self._workspaces.get(out_cols)
        if ws is None:
            nbytes = C.c_uint64()
            N.check("cx_qcsr_exec_workspace_bytes",
                    self._lib.cx_qcsr_exec_workspace_bytes(self._handle, out_cols, C.byref(nbytes)))
            ws = torch.empty(max(nbytes.value, 256), dtype=torch.uint8, device=self.device)
            self._workspaces[out_cols] = ws
        return ws

    def spmm(self, w: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None, epilogue=None) -> torch.Tensor:
        """Y = X . W (+ epilogue) for canonical F16 W [genes, N], N in 64..256 by 64."""
        _require_cuda(w)
        if w.dim() != 2 or w.shape[0] != self.cols or w.dtype != torch.float16 or w.stride(1) != 1:
            raise ValueError("w must be a row-major F16 [genes, N] tensor in canonical gene order")
        n = int(w.shape[1])
        if out is None:
            out = torch.empty((self.rows, n), dtype=torch.float32, device=w.device)
        e = epilogue.descriptor(out) if epilogue is not None else None
        ws = self.workspace(n)
        _record(ws, stream)
        N.check("cx_qcsr_exec_spmm", self._lib.cx_qcsr_exec_spmm(
            self._handle, w.data_ptr(), w.stride(0), n, out.data_ptr(), out.stride(0),
            C.byref(e) if e is not None else None, ws.data_ptr(), ws.numel(), _stream(stream)))
        return out

    def close(self) -> None:
        if self._handle:
            self._lib.cx_qcsr_exec_destroy(self._handle)
            self._handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
