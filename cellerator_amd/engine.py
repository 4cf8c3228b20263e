"""Python host mirror of the engine's launch layer: device-resident matrix containers
and one function per C-ABI entry point. PyTorch only provides device memory and
streams; every operation runs the HIP kernels of libcellerator_amd.so.

Containers mirror the reference's types:
  QcsrMatrix -- cellerator::quantized::csr_matrix (include/Cellerator/quantized/layout.cuh:12-39)
  BellMatrix -- cellerator::quantized::blocked_ell::matrix (quantized/blocked_ell.cuh:18-35)
                and the plain Blocked-ELL of blocked_ell_spmm_fwd_f16_f32
  CpbpTiles  -- cellpack::warp_tile_view + feature_weighted_row_reduction_plan_view
                (components/CellPack/include/CellPack/warp_tiles.hh:41-79,
                 feature_weighted_row_reduction.hh:16-26)
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _native as N


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _torch_stream(stream, device) -> torch.cuda.Stream:
    """`stream` (None = the current stream, a torch stream, or a raw hipStream_t handle) as
    a torch stream object that can be made current."""
    if stream is None:
        return torch.cuda.current_stream(device)
    if isinstance(stream, torch.cuda.Stream):
        return stream
    return torch.cuda.ExternalStream(int(stream), device=device)


def _require_cuda(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("engine operands must be device tensors")


_DTYPE_CODE = {torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16}


@dataclass
class QcsrMatrix:
    rows: int
    cols: int
    bits: int  # 1, 2, 4, 8; 0 = unquantized `values`
    row_ptr: torch.Tensor  # int32 [rows + 1]
    col_idx: torch.Tensor  # int32 [nnz]
    packed_row_ptr: Optional[torch.Tensor] = None  # int32 [rows + 1]
    packed_values: Optional[torch.Tensor] = None  # uint8
    column_scales: Optional[torch.Tensor] = None  # float32 [cols]
    column_offsets: Optional[torch.Tensor] = None  # float32 [cols]
    row_offsets: Optional[torch.Tensor] = None  # float32 [rows]
    values: Optional[torch.Tensor] = None  # f16/f32 [nnz] when bits == 0
    decode_policy: int = N.DECODE_PER_GENE_AFFINE
    meta: dict = field(default_factory=dict)
    flags: int = 0  # cx_qcsr_matrix.flags: N.QCSR_COLUMNS_SORTED once qcsr_check_columns confirms it

    @property
    def nnz(self) -> int:
        return int(self.col_idx.numel())

    def descriptor(self) -> N.CxQcsrMatrix:
        d = N.CxQcsrMatrix()
        d.rows, d.cols, d.nnz = self.rows, self.cols, self.nnz
        d.bits, d.decode_policy = self.bits, self.decode_policy
        d.row_ptr, d.col_idx = _ptr(self.row_ptr), _ptr(self.col_idx)
        d.packed_row_ptr, d.packed_values = _ptr(self.packed_row_ptr), _ptr(self.packed_values)
        d.column_scales, d.column_offsets = _ptr(self.column_scales), _ptr(self.column_offsets)
        d.row_offsets, d.values = _ptr(self.row_offsets), _ptr(self.values)
        d.value_dtype = _DTYPE_CODE[self.values.dtype] if self.values is not None else 0
        d.flags = self.flags
        return d

    def nbytes_algorithmic(self, rhs_cols: int, rhs_bytes: int = 2) -> int:
        """Bytes the SpMM must move once: row_ptr (+ packed_row_ptr), col_idx, codes or
        values, per-gene metadata, the weight panel and the fp32 output."""
        b = self.row_ptr.numel() * 4 + self.col_idx.numel() * 4
        if self.bits:
            b += self.packed_row_ptr.numel() * 4 + self.packed_values.numel()
            b += sum(t.numel() * 4 for t in (self.column_scales, self.column_offsets,
                                             self.row_offsets) if t is not None)
        else:
            b += self.values.numel() * self.values.element_size()
        return b + self.cols * rhs_cols * rhs_bytes + self.rows * rhs_cols * 4


@dataclass
class Epilogue:
    """Fused SpMM epilogue: Y = act(alpha * (A . W) + beta * C + bias), kind = one of the
    reference's epilogue_kind values (N.EPILOGUE_*). `initial` (C, f32 [rows, N]) is read only
    when beta != 0 and may be the output itself (in-place update); `bias` is f32 [N] for the
    bias kinds."""
    kind: int = N.EPILOGUE_NONE
    alpha: float = 1.0
    beta: float = 0.0
    bias: Optional[torch.Tensor] = None
    initial: Optional[torch.Tensor] = None

    def descriptor(self, out: torch.Tensor) -> N.CxSpmmEpilogue:
        for t in (self.bias, self.initial):
            if t is not None and (t.dtype != torch.float32 or t.device != out.device):
                raise ValueError("epilogue tensors must be f32 on the output's device")
        if self.bias is not None and not self.bias.is_contiguous():
            raise ValueError("bias must be contiguous")
        if self.initial is not None and (self.initial.dim() != 2 or self.initial.stride(1) != 1):
            raise ValueError("initial must be a row-major [rows, N] tensor")
        return N.CxSpmmEpilogue(self.kind, 0, self.alpha, self.beta, _ptr(self.bias),
                                _ptr(self.initial),
                                self.initial.stride(0) if self.initial is not None else 0)


def qcsr_spmm(m: QcsrMatrix, rhs: torch.Tensor, out: Optional[torch.Tensor] = None,
              stream=None, epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """Y = decode(X) . rhs (fp32), optionally through a fused epilogue.
    rhs: [cols, N] f16/f32, row-major (leading dim = stride)."""
    _require_cuda(m.row_ptr, m.col_idx, rhs)
    if rhs.dim() != 2 or rhs.shape[0] != m.cols or rhs.stride(1) != 1:
        raise ValueError("rhs must be [cols, N] with unit column stride")
    n = rhs.shape[1]
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=rhs.device)
    d = m.descriptor()
    if epilogue is None:
        N.check("cx_qcsr_spmm_fwd", N.engine().cx_qcsr_spmm_fwd(
            C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
            out.stride(0), _stream(stream)))
    else:
        e = epilogue.descriptor(out)
        N.check("cx_qcsr_spmm_fwd_epilogue", N.engine().cx_qcsr_spmm_fwd_epilogue(
            C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
            out.stride(0), C.byref(e), _stream(stream)))
    return out


def qcsr_pack_gene_affine(m: QcsrMatrix, stream=None) -> QcsrMatrix:
    """The same matrix with its per-gene (scale, offset) interleaved into one array
    (decode policy CX_DECODE_PER_GENE_AFFINE_PAIRS): decodes bit-identically with one
    8-byte metadata gather per code. Built once per metadata generation."""
    if m.bits == 0 or m.decode_policy != N.DECODE_PER_GENE_AFFINE:
        raise ValueError("interleaved metadata applies to quantized per-gene-affine matrices")
    _require_cuda(m.row_ptr)
    pairs = torch.empty(2 * m.cols, dtype=torch.float32, device=m.row_ptr.device)
    N.check("cx_qcsr_pack_gene_affine", N.engine().cx_qcsr_pack_gene_affine(
        _ptr(m.column_scales), _ptr(m.column_offsets), m.cols, pairs.data_ptr(), _stream(stream)))
    return QcsrMatrix(m.rows, m.cols, m.bits, m.row_ptr, m.col_idx, packed_row_ptr=m.packed_row_ptr,
                      packed_values=m.packed_values, column_scales=pairs, column_offsets=None,
                      decode_policy=N.DECODE_PER_GENE_AFFINE_PAIRS, meta=dict(m.meta), flags=m.flags)


def qcsr_check_columns(m: QcsrMatrix, stream=None) -> QcsrMatrix:
    """The same matrix with flags = QCSR_COLUMNS_SORTED when every row's columns are
    non-decreasing and in [0, cols) (checked on the device, one pass over the structure),
    else flags = 0. Run once per structure: the gene-part kernels then skip their per-entry
    out-of-order check."""
    _require_cuda(m.row_ptr)
    dev = m.row_ptr.device
    # Allocation, launch and read all run on the check's stream: the flag's read-back then
    # waits for the check, and the buffer is released on the stream that wrote it.
    s = _torch_stream(stream, dev)
    with torch.cuda.stream(s):
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        d = m.descriptor()
        N.check("cx_qcsr_check_columns", N.engine().cx_qcsr_check_columns(
            C.byref(d), flag.data_ptr(), s.cuda_stream))
        value = int(flag.item())
    return dataclasses.replace(m, flags=value & N.QCSR_COLUMNS_SORTED)


def qcsr_transpose(m: QcsrMatrix, stream=None) -> QcsrMatrix:
    """A^T (genes x cells) as a plain f32 CSR, values decoded exactly as the forward decodes
    them; feeds qcsr_spmm (A^T . B) and qcsr_spmm_bwd_rhs. Built once per structure and
    value generation (device radix sort, deterministic)."""
    _require_cuda(m.row_ptr)
    d = m.descriptor()
    lib = N.engine()
    ws_bytes = C.c_uint64()
    N.check("cx_qcsr_transpose_workspace", lib.cx_qcsr_transpose_workspace(C.byref(d), C.byref(ws_bytes)))
    dev = m.row_ptr.device
    nnz = m.nnz
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=dev)
    t_row_ptr = torch.empty(m.cols + 1, dtype=torch.int32, device=dev)
    t_col_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    t_values = torch.empty(max(nnz, 1), dtype=torch.float32, device=dev)
    N.check("cx_qcsr_transpose", lib.cx_qcsr_transpose(
        C.byref(d), t_row_ptr.data_ptr(), t_col_idx.data_ptr(), t_values.data_ptr(),
        ws.data_ptr(), ws_bytes.value, _stream(stream)))
    # The workspace may be released once the build is ordered before later work: on the
    # current stream torch's allocator guarantees that; on another stream keep it alive.
    meta = {} if stream is None else {"transpose_workspace": ws}
    return QcsrMatrix(m.cols, m.rows, 0, t_row_ptr, t_col_idx[:nnz], values=t_values[:nnz],
                      meta=meta)


def qcsr_transpose_panelled(m: QcsrMatrix, panel_rows: int = 8192, stream=None) -> QcsrMatrix:
    """A^T with rows ordered by (cell panel, gene): rows = ceil(rows / panel_rows) * cols.
    meta["panels"] holds the panel count for qcsr_spmm_bwd_rhs."""
    _require_cuda(m.row_ptr)
    d = m.descriptor()
    lib = N.engine()
    ws_bytes = C.c_uint64()
    N.check("cx_qcsr_transpose_panelled_workspace",
            lib.cx_qcsr_transpose_panelled_workspace(C.byref(d), panel_rows, C.byref(ws_bytes)))
    dev = m.row_ptr.device
    panels = (m.rows + panel_rows - 1) // panel_rows
    nnz = m.nnz
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=dev)
    t_row_ptr = torch.empty(panels * m.cols + 1, dtype=torch.int32, device=dev)
    t_col_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    t_values = torch.empty(max(nnz, 1), dtype=torch.float32, device=dev)
    N.check("cx_qcsr_transpose_panelled", lib.cx_qcsr_transpose_panelled(
        C.byref(d), panel_rows, t_row_ptr.data_ptr(), t_col_idx.data_ptr(), t_values.data_ptr(),
        ws.data_ptr(), ws_bytes.value, _stream(stream)))
    meta = {"panels": panels, "panel_rows": panel_rows}
    if stream is not None:
        meta["transpose_workspace"] = ws
    return QcsrMatrix(panels * m.cols, m.rows, 0, t_row_ptr, t_col_idx[:nnz], values=t_values[:nnz],
                      meta=meta)


def qcsr_spmm_bwd_values(m: QcsrMatrix, grad_out: torch.Tensor, rhs: torch.Tensor,
                         out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """grad_values[i] = <grad_out[row_i, :], rhs[col_i, :]> for every stored entry (f32)."""
    _require_cuda(m.row_ptr, grad_out, rhs)
    if grad_out.dtype != torch.float32 or grad_out.stride(1) != 1 or rhs.stride(1) != 1:
        raise ValueError("grad_out must be row-major f32 and rhs row-major")
    n = rhs.shape[1]
    if grad_out.shape != (m.rows, n) or rhs.shape[0] != m.cols:
        raise ValueError("grad_out must be [rows, N] and rhs [cols, N]")
    if out is None:
        out = torch.empty(max(m.nnz, 1), dtype=torch.float32, device=rhs.device)[: m.nnz]
    d = m.descriptor()
    N.check("cx_qcsr_spmm_bwd_values", N.engine().cx_qcsr_spmm_bwd_values(
        C.byref(d), grad_out.data_ptr(), grad_out.stride(0), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype],
        rhs.stride(0), n, out.data_ptr(), _stream(stream)))
    return out


def qcsr_spmm_bwd_rhs(transposed: QcsrMatrix, grad_out: torch.Tensor,
                      out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """grad_rhs = A^T . grad_out with `transposed` from qcsr_transpose(A) or
    qcsr_transpose_panelled(A) (f32 [cols, N])."""
    _require_cuda(transposed.row_ptr, grad_out)
    if grad_out.dtype != torch.float32 or grad_out.stride(1) != 1 or grad_out.shape[0] != transposed.cols:
        raise ValueError("grad_out must be row-major f32 [rows of A, N]")
    n = grad_out.shape[1]
    panels = transposed.meta.get("panels", 1)
    d = transposed.descriptor()
    if panels > 1:
        genes = transposed.rows // panels
        if out is None:
            out = torch.empty((genes, n), dtype=torch.float32, device=grad_out.device)
        nbytes = C.c_uint64()
        N.check("cx_qcsr_spmm_bwd_rhs_panelled_workspace",
                N.engine().cx_qcsr_spmm_bwd_rhs_panelled_workspace(C.byref(d), panels, n, C.byref(nbytes)))
        ws = torch.empty(max(nbytes.value, 16), dtype=torch.uint8, device=grad_out.device)
        N.check("cx_qcsr_spmm_bwd_rhs_panelled", N.engine().cx_qcsr_spmm_bwd_rhs_panelled(
            C.byref(d), panels, grad_out.data_ptr(), grad_out.stride(0), n, out.data_ptr(),
            out.stride(0), ws.data_ptr(), ws.numel(), _stream(stream)))
        return out
    if out is None:
        out = torch.empty((transposed.rows, n), dtype=torch.float32, device=grad_out.device)
    ws = _balanced_workspace(d, n, grad_out.device)
    N.check("cx_qcsr_spmm_bwd_rhs", N.engine().cx_qcsr_spmm_bwd_rhs(
        C.byref(d), grad_out.data_ptr(), grad_out.stride(0), n, out.data_ptr(), out.stride(0),
        ws.data_ptr(), ws.numel(), _stream(stream)))
    return out


def _balanced_workspace(d, n: int, device) -> torch.Tensor:
    nbytes = C.c_uint64()
    N.check("cx_qcsr_spmm_balanced_workspace",
            N.engine().cx_qcsr_spmm_balanced_workspace(C.byref(d), n, C.byref(nbytes)))
    return torch.empty(max(nbytes.value, 16), dtype=torch.uint8, device=device)


def qcsr_spmm_balanced(m: QcsrMatrix, rhs: torch.Tensor, out: Optional[torch.Tensor] = None,
                       stream=None, epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """qcsr_spmm in the load-balanced (equal nnz chunks) form, for skewed row lengths."""
    _require_cuda(m.row_ptr, m.col_idx, rhs)
    if rhs.dim() != 2 or rhs.shape[0] != m.cols or rhs.stride(1) != 1:
        raise ValueError("rhs must be [cols, N] with unit column stride")
    n = rhs.shape[1]
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=rhs.device)
    d = m.descriptor()
    ws = _balanced_workspace(d, n, rhs.device)
    e = epilogue.descriptor(out) if epilogue is not None else None
    N.check("cx_qcsr_spmm_fwd_balanced", N.engine().cx_qcsr_spmm_fwd_balanced(
        C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
        out.stride(0), C.byref(e) if e is not None else None, ws.data_ptr(), ws.numel(),
        _stream(stream)))
    return out


def sort_pairs(keys: torch.Tensor, values: Optional[torch.Tensor] = None, key_bits: int = 32,
               stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable device radix sort of int32-stored u32 keys (low key_bits bits) with u32 values
    (None: the identity permutation). Returns (sorted keys, permuted values)."""
    _require_cuda(keys)
    count = keys.numel()
    lib = N.engine()
    ws_bytes = C.c_uint64()
    N.check("cx_sort_pairs_workspace", lib.cx_sort_pairs_workspace(count, key_bits, C.byref(ws_bytes)))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=keys.device)
    ko = torch.empty(max(count, 1), dtype=torch.int32, device=keys.device)
    vo = torch.empty(max(count, 1), dtype=torch.int32, device=keys.device)
    N.check("cx_sort_pairs", lib.cx_sort_pairs(
        keys.data_ptr(), _ptr(values), ko.data_ptr(), vo.data_ptr(), count, key_bits, ws.data_ptr(),
        ws_bytes.value, _stream(stream)))
    return ko[:count], vo[:count]


def exclusive_scan_u32(x: torch.Tensor, stream=None) -> torch.Tensor:
    """Exclusive prefix sum of int32-stored u32 values (modulo 2^32)."""
    _require_cuda(x)
    lib = N.engine()
    ws_bytes = C.c_uint64()
    N.check("cx_exclusive_scan_u32_workspace", lib.cx_exclusive_scan_u32_workspace(x.numel(), C.byref(ws_bytes)))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty_like(x)
    N.check("cx_exclusive_scan_u32", lib.cx_exclusive_scan_u32(
        x.data_ptr(), out.data_ptr(), x.numel(), ws.data_ptr(), ws_bytes.value, _stream(stream)))
    return out


@dataclass
class BellMatrix:
    rows: int
    cols: int
    block_size: int
    ell_cols: int
    block_col_idx: torch.Tensor  # uint32 as int32 storage [rows/bs, ell_cols/bs]
    # [rows, ell_cols] bf16/f16/f32, or block-major [rows/bs, ell_cols/bs, bs, bs] when
    # block_major is set (cx_bell_block_major_values)
    values: Optional[torch.Tensor] = None
    bits: int = 0
    decode_policy: int = N.DECODE_PER_GENE_AFFINE
    row_stride_bytes: int = 0
    packed_values: Optional[torch.Tensor] = None
    column_scales: Optional[torch.Tensor] = None
    column_offsets: Optional[torch.Tensor] = None
    row_offsets: Optional[torch.Tensor] = None
    meta: dict = field(default_factory=dict)
    block_major: bool = False

    def descriptor(self) -> N.CxBellMatrix:
        d = N.CxBellMatrix()
        d.rows, d.cols, d.block_size, d.ell_cols = self.rows, self.cols, self.block_size, self.ell_cols
        d.block_col_idx = _ptr(self.block_col_idx)
        d.values = _ptr(self.values)
        d.value_dtype = _DTYPE_CODE[self.values.dtype] if self.values is not None else 0
        d.bits, d.decode_policy, d.row_stride_bytes = self.bits, self.decode_policy, self.row_stride_bytes
        d.packed_values = _ptr(self.packed_values)
        d.column_scales, d.column_offsets = _ptr(self.column_scales), _ptr(self.column_offsets)
        d.row_offsets = _ptr(self.row_offsets)
        d.value_layout_flags = N.BELL_BLOCK_MAJOR_VALUES if self.block_major else 0
        return d


def bell_block_major(m: BellMatrix, stream=None) -> BellMatrix:
    """The same matrix with its values copied into block-major order
    (cx_bell_block_major_values): every block_size x block_size value block contiguous."""
    _require_cuda(m.block_col_idx)
    if m.values is None or m.bits != 0 or m.block_major:
        raise ValueError("bell_block_major takes a matrix with row-major unquantized values")
    bs, rb = m.block_size, (m.rows + m.block_size - 1) // m.block_size
    out = torch.empty((rb, m.ell_cols // bs, bs, bs), dtype=m.values.dtype, device=m.values.device)
    d = m.descriptor()
    N.check("cx_bell_block_major_values", N.engine().cx_bell_block_major_values(
        C.byref(d), out.data_ptr(), out.numel() * out.element_size(), _stream(stream)))
    return BellMatrix(m.rows, m.cols, bs, m.ell_cols, m.block_col_idx, values=out,
                      meta=dict(m.meta), block_major=True)


def bell_spmm(m: BellMatrix, rhs: torch.Tensor, out: Optional[torch.Tensor] = None,
              stream=None, epilogue: Optional[Epilogue] = None,
              row_block_order: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Reference-semantics Blocked-ELL SpMM with a row-major rhs [cols, N]. `row_block_order`
    (int32 storage of a u32 permutation of the row blocks, e.g. BellGroups.order): the
    quantized matrix-core forms take row blocks in that order (cx_bell_spmm_fwd_ordered);
    same results."""
    _require_cuda(m.block_col_idx, rhs)
    n = rhs.shape[1]
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=rhs.device)
    d = m.descriptor()
    if row_block_order is not None:
        if epilogue is not None:
            raise ValueError("a row-block order takes no epilogue")
        _require_cuda(row_block_order)
        if row_block_order.dtype != torch.int32 or row_block_order.numel() != (m.rows + m.block_size - 1) // m.block_size:
            raise ValueError("row_block_order must hold one int32 entry per row block")
        N.check("cx_bell_spmm_fwd_ordered", N.engine().cx_bell_spmm_fwd_ordered(
            C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
            out.stride(0), row_block_order.data_ptr(), _stream(stream)))
    elif epilogue is None:
        N.check("cx_bell_spmm_fwd", N.engine().cx_bell_spmm_fwd(
            C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
            out.stride(0), _stream(stream)))
    else:
        e = epilogue.descriptor(out)
        N.check("cx_bell_spmm_fwd_epilogue", N.engine().cx_bell_spmm_fwd_epilogue(
            C.byref(d), rhs.data_ptr(), _DTYPE_CODE[rhs.dtype], rhs.stride(0), n, out.data_ptr(),
            out.stride(0), C.byref(e), _stream(stream)))
    return out


def bell_pack_rhs(rhs: torch.Tensor, stream=None) -> torch.Tensor:
    """Packs a bf16 [K, N] row-major weight panel into the MFMA operand layout."""
    _require_cuda(rhs)
    if rhs.dtype != torch.bfloat16 or rhs.dim() != 2 or rhs.stride(1) != 1:
        raise ValueError("rhs must be a row-major bf16 [K, N] tensor")
    k, n = rhs.shape
    packed = torch.empty(((k + 31) // 32) * n * 32, dtype=torch.bfloat16, device=rhs.device)
    N.check("cx_bell_pack_rhs", N.engine().cx_bell_pack_rhs(
        rhs.data_ptr(), rhs.stride(0), k, n, packed.data_ptr(), _stream(stream)))
    return packed


def bell_spmm_packed(m: BellMatrix, packed_rhs: torch.Tensor, n: int,
                     out: Optional[torch.Tensor] = None, stream=None,
                     epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """MFMA Blocked-ELL SpMM against a packed bf16 panel (bell_pack_rhs)."""
    _require_cuda(m.block_col_idx, packed_rhs)
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=packed_rhs.device)
    d = m.descriptor()
    if epilogue is None:
        N.check("cx_bell_spmm_fwd_packed", N.engine().cx_bell_spmm_fwd_packed(
            C.byref(d), packed_rhs.data_ptr(), n, out.data_ptr(), out.stride(0), _stream(stream)))
    else:
        e = epilogue.descriptor(out)
        N.check("cx_bell_spmm_fwd_packed_epilogue", N.engine().cx_bell_spmm_fwd_packed_epilogue(
            C.byref(d), packed_rhs.data_ptr(), n, out.data_ptr(), out.stride(0), C.byref(e),
            _stream(stream)))
    return out


@dataclass
class BellGroups:
    """Row-block groups of a Blocked-ELL matrix for the grouped MFMA path (host-planned once
    per projection; see cx_bell_plan_groups and cx_bell_schedule_groups)."""
    group_count: int
    grouped_row_blocks: int
    single_count: int
    order: torch.Tensor          # int32 [row_blocks] (uint32 ids)
    group_offsets: torch.Tensor  # int32 [group_count + 1]
    planned_groups: int = 0      # groups of 2..4 the planner formed (before a schedule)
    planned_singles: int = 0     # row blocks it left single

    def descriptor(self) -> N.CxBellGroups:
        return N.CxBellGroups(self.group_count, self.grouped_row_blocks, self.single_count, 0,
                              _ptr(self.order), _ptr(self.group_offsets))


def bell_plan_groups(m: BellMatrix, max_group: int = 4, schedule: bool = True) -> BellGroups:
    """Groups row blocks whose valid block-column lists are prefixes of one another (host
    planner on a host copy of block_col_idx; the result is uploaded to m's device). With
    `schedule` (the default) the plan is laid out for the launch by cx_bell_schedule_groups:
    single row blocks become one-member groups and every XCD's range of groups carries about
    the same number of value blocks."""
    import numpy as np

    rb = (m.rows + m.block_size - 1) // m.block_size
    slots = m.ell_cols // m.block_size
    idx = np.ascontiguousarray(m.block_col_idx.cpu().numpy().view(np.uint32).reshape(rb, slots))
    order = np.zeros(rb, np.uint32)
    offs = np.zeros(rb + 1, np.uint32)
    gc, sc = C.c_uint32(), C.c_uint32()
    lib = N.engine()
    st = lib.cx_bell_plan_groups(idx.ctypes.data if idx.size else None, rb, slots, max_group,
                                 order.ctypes.data if order.size else None, offs.ctypes.data,
                                 C.byref(gc), C.byref(sc))
    if st != 0:
        raise N.EngineError("cx_bell_plan_groups", st, lib.cx_bell_plan_last_error().decode())
    planned = (gc.value, sc.value)
    grouped = int(offs[gc.value]) if gc.value else 0
    n_groups, singles = gc.value, sc.value
    if schedule:
        s_order = np.zeros(rb, np.uint32)
        s_offs = np.zeros(rb + 1, np.uint32)
        units = C.c_uint32()
        st = lib.cx_bell_schedule_groups(idx.ctypes.data if idx.size else None, rb, slots,
                                         order.ctypes.data if order.size else None, offs.ctypes.data,
                                         gc.value, sc.value, s_order.ctypes.data if s_order.size else None,
                                         s_offs.ctypes.data, C.byref(units))
        if st != 0:
            raise N.EngineError("cx_bell_schedule_groups", st, lib.cx_bell_plan_last_error().decode())
        order, offs, n_groups, grouped, singles = s_order, s_offs, units.value, rb, 0
    dev = m.block_col_idx.device
    return BellGroups(n_groups, grouped, singles,
                      torch.from_numpy(order.view(np.int32)).to(dev),
                      torch.from_numpy(offs[: n_groups + 1].view(np.int32).copy()).to(dev),
                      planned[0], planned[1])


def bell_spmm_grouped(m: BellMatrix, packed_rhs: torch.Tensor, groups: BellGroups, n: int,
                      out: Optional[torch.Tensor] = None, stream=None,
                      epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """MFMA Blocked-ELL with a planned row-block grouping; same contract as bell_spmm_packed."""
    _require_cuda(m.block_col_idx, packed_rhs)
    if out is None:
        out = torch.empty((m.rows, n), dtype=torch.float32, device=packed_rhs.device)
    d, g = m.descriptor(), groups.descriptor()
    if epilogue is None:
        N.check("cx_bell_spmm_fwd_grouped", N.engine().cx_bell_spmm_fwd_grouped(
            C.byref(d), packed_rhs.data_ptr(), C.byref(g), n, out.data_ptr(), out.stride(0),
            _stream(stream)))
    else:
        e = epilogue.descriptor(out)
        N.check("cx_bell_spmm_fwd_grouped_epilogue", N.engine().cx_bell_spmm_fwd_grouped_epilogue(
            C.byref(d), packed_rhs.data_ptr(), C.byref(g), n, out.data_ptr(), out.stride(0),
            C.byref(e), _stream(stream)))
    return out


@dataclass
class CpbpTiles:
    row_count: int
    feature_count: int
    tile_row_width: int
    feature_block_offsets: torch.Tensor  # u32 (int32 storage)
    feature_permutation: torch.Tensor
    tile_block_offsets: torch.Tensor
    tile_block_ids: torch.Tensor
    tile_block_cell_masks: torch.Tensor  # u32 (int32) or u64 (int64) storage
    block_row_entry_offsets: torch.Tensor
    row_block_gene_masks: torch.Tensor
    row_block_value_offsets: torch.Tensor
    values: torch.Tensor  # f16 / f32
    row_permutation: torch.Tensor
    meta: dict = field(default_factory=dict)

    @property
    def tile_count(self) -> int:
        return int(self.tile_block_offsets.numel()) - 1

    def descriptor(self) -> N.CxCpbpTiles:
        d = N.CxCpbpTiles()
        d.row_count, d.feature_count = self.row_count, self.feature_count
        d.feature_block_count = int(self.feature_block_offsets.numel()) - 1
        d.tile_row_width, d.tile_count = self.tile_row_width, self.tile_count
        d.tile_block_count = int(self.tile_block_ids.numel())
        d.row_block_entry_count = int(self.row_block_gene_masks.numel())
        d.nnz_count = int(self.values.numel())
        d.value_dtype = _DTYPE_CODE[self.values.dtype]
        for name in ("feature_block_offsets", "feature_permutation", "tile_block_offsets",
                     "tile_block_ids", "tile_block_cell_masks", "block_row_entry_offsets",
                     "row_block_gene_masks", "row_block_value_offsets", "values",
                     "row_permutation"):
            setattr(d, name, _ptr(getattr(self, name)))
        return d

    def nbytes_algorithmic(self) -> int:
        """Bytes of every tile array, the plan subset, the weights and the output once
        (the reference bench's accounting, feature_weighted_row_reduction_bench.cu:356-368)."""
        arrays = (self.feature_block_offsets, self.feature_permutation, self.tile_block_offsets,
                  self.tile_block_ids, self.tile_block_cell_masks, self.block_row_entry_offsets,
                  self.row_block_gene_masks, self.row_block_value_offsets, self.values,
                  self.row_permutation)
        b = sum(t.numel() * t.element_size() for t in arrays)
        return b + self.feature_count * 4 + self.row_count * 4


def cpbp_reduce(t: CpbpTiles, weights: torch.Tensor, out: Optional[torch.Tensor] = None,
                stream=None) -> torch.Tensor:
    _require_cuda(weights, t.values)
    if out is None:
        out = torch.empty(t.row_count, dtype=torch.float32, device=weights.device)
    d = t.descriptor()
    N.check("cx_cpbp_reduce", N.engine().cx_cpbp_reduce(
        C.byref(d), weights.data_ptr(), weights.numel(), out.data_ptr(), out.numel(),
        _stream(stream)))
    return out


def cpbp_entry_rows(t: CpbpTiles, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Every entry's tile row and block start (block start << 6 | row, int32 storage of u32),
    computed once per tile structure on the device (cx_cpbp_entry_rows): the per-entry
    array cpbp_reduce_rows reads instead of looking the entry's descriptor up."""
    d = t.descriptor()
    n = int(d.row_block_entry_count)
    if out is None:
        out = torch.empty(max(n, 1), dtype=torch.int32, device="cuda")
    _require_cuda(out)
    N.check("cx_cpbp_entry_rows", N.engine().cx_cpbp_entry_rows(
        C.byref(d), out.data_ptr(), out.numel(), _stream(stream)))
    return out


def cpbp_reduce_rows(t: CpbpTiles, entry_rows: torch.Tensor, weights: torch.Tensor,
                     out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """cpbp_reduce with the entries' rows and block starts read from `entry_rows`
    (cpbp_entry_rows of the same tiles) instead of the descriptors: same contract."""
    _require_cuda(weights, t.values, entry_rows)
    d = t.descriptor()
    if entry_rows.dtype != torch.int32 or entry_rows.numel() < int(d.row_block_entry_count):
        raise ValueError("entry_rows must be the int32 array cpbp_entry_rows made for these tiles")
    if out is None:
        out = torch.empty(t.row_count, dtype=torch.float32, device=weights.device)
    N.check("cx_cpbp_reduce_rows", N.engine().cx_cpbp_reduce_rows(
        C.byref(d), entry_rows.data_ptr(), weights.data_ptr(), weights.numel(), out.data_ptr(), out.numel(),
        _stream(stream)))
    return out


def csr_spmv(row_ptr: torch.Tensor, col_idx: torch.Tensor, values: torch.Tensor,
             x: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    _require_cuda(row_ptr, col_idx, values, x)
    rows = row_ptr.numel() - 1
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=x.device)
    N.check("cx_csr_spmv_fwd", N.engine().cx_csr_spmv_fwd(
        rows, row_ptr.data_ptr(), col_idx.data_ptr(), values.data_ptr(), _DTYPE_CODE[values.dtype],
        x.data_ptr(), out.data_ptr(), _stream(stream)))
    return out
