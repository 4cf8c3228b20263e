"""Host construction of the CP-BP warp-tile projection (canonical CSR -> cell-block records
-> local cell order -> warp tiles) through the engine's C-ABI builder, and its upload to the
device as a CpbpTiles the reduction kernel consumes.

Mirrors the reference's CellPack producers (components/CellPack/include/CellPack/
packing_plan.hh, apply_plan.hh, cell_block_records.hh, local_cell_ordering.hh,
warp_tiles.hh) for one row partition; the tile width may be up to 64 rows.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import _native as N

ORDER_INFERRED_MINHASH = 1
ORDER_ORIGINAL = 2
ORDER_DETERMINISTIC_RANDOM = 3
ORDER_ROW_NNZ_DESCENDING = 4
DEFAULT_ORDER_SEED = 0x6A09E667F3BCC909  # local_cell_order_config default (local_cell_ordering.hh:26)


@dataclass
class Plan:
    """Frozen packing plan subset: feature_permutation[execution] = canonical feature."""
    feature_permutation: np.ndarray  # uint32 [F]
    feature_block_offsets: np.ndarray  # uint32 [B + 1]

    @property
    def feature_count(self) -> int:
        return int(self.feature_permutation.size)

    @property
    def feature_block_count(self) -> int:
        return int(self.feature_block_offsets.size) - 1


def contiguous_plan(feature_count: int, block_width: int) -> Plan:
    """Identity execution order cut into consecutive blocks of `block_width` features."""
    offs = list(range(0, feature_count, block_width)) + [feature_count]
    return Plan(np.arange(feature_count, dtype=np.uint32), np.asarray(offs, dtype=np.uint32))


@dataclass
class HostTiles:
    """Host-resident warp tiles (the warp_tile_view arrays) plus the row permutation."""
    req: dict
    tile_block_offsets: np.ndarray
    tile_block_ids: np.ndarray
    tile_block_cell_masks: np.ndarray  # uint32 or uint64
    block_row_entry_offsets: np.ndarray
    row_block_gene_masks: np.ndarray
    row_block_value_offsets: np.ndarray
    values: np.ndarray  # float16 or float32
    row_permutation: np.ndarray
    primary_keys: np.ndarray


def _p(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


def build_tiles(plan: Plan, row_offsets: np.ndarray, canonical_features: np.ndarray,
                values: np.ndarray, *, kind: int = ORDER_INFERRED_MINHASH, window_size: int = 1024,
                group_width: int = 64, seed: int = DEFAULT_ORDER_SEED, global_row_begin: int = 0,
                threads: int | None = None) -> HostTiles:
    lib = N.engine()
    perm = np.ascontiguousarray(plan.feature_permutation, dtype=np.uint32)
    boffs = np.ascontiguousarray(plan.feature_block_offsets, dtype=np.uint32)
    ro = np.ascontiguousarray(row_offsets, dtype=np.uint32)
    cf = np.ascontiguousarray(canonical_features, dtype=np.uint32)
    if values.dtype not in (np.float16, np.float32):
        raise ValueError("CP-BP values must be float16 or float32")
    vals = np.ascontiguousarray(values)
    cplan = N.CxCpbpPlan(plan.feature_count, plan.feature_block_count, _p(perm), _p(boffs))
    csr = N.CxCpbpCsr(int(ro.size) - 1, vals.itemsize, _p(ro), _p(cf), _p(vals))
    cfg = N.CxCpbpOrderConfig(kind, window_size, group_width, 0, seed, global_row_begin)
    handle = C.c_void_p()
    nthreads = threads if threads is not None else min(16, os.cpu_count() or 1)
    st = lib.cx_cpbp_builder_create(C.byref(cplan), C.byref(csr), C.byref(cfg), nthreads,
                                    C.byref(handle))
    if st != 0:
        raise N.EngineError("cx_cpbp_builder_create", st, lib.cx_cpbp_build_last_error().decode())
    try:
        req = N.CxCpbpTileRequirements()
        N.check("cx_cpbp_builder_requirements", lib.cx_cpbp_builder_requirements(handle, C.byref(req)))
        mask_t = np.uint64 if req.cell_mask_bytes == 8 else np.uint32
        out = HostTiles(
            req={f: getattr(req, f) for f, _ in req._fields_},
            tile_block_offsets=np.zeros(req.tile_count + 1, np.uint32),
            tile_block_ids=np.zeros(req.tile_block_count, np.uint32),
            tile_block_cell_masks=np.zeros(req.tile_block_count, mask_t),
            block_row_entry_offsets=np.zeros(req.tile_block_count + 1, np.uint32),
            row_block_gene_masks=np.zeros(req.row_block_entry_count, np.uint32),
            row_block_value_offsets=np.zeros(req.row_block_entry_count + 1, np.uint32),
            values=np.zeros(req.nnz_count, vals.dtype),
            row_permutation=np.zeros(req.row_count, np.uint32),
            primary_keys=np.zeros(req.row_count, np.uint64))
        bufs = N.CxCpbpTileBuffers(
            _p(out.tile_block_offsets), _p(out.tile_block_ids), _p(out.tile_block_cell_masks),
            _p(out.block_row_entry_offsets), _p(out.row_block_gene_masks),
            _p(out.row_block_value_offsets), _p(out.values), _p(out.row_permutation),
            _p(out.primary_keys))
        st = lib.cx_cpbp_builder_export(handle, C.byref(bufs))
        if st != 0:
            raise N.EngineError("cx_cpbp_builder_export", st, lib.cx_cpbp_build_last_error().decode())
        return out
    finally:
        lib.cx_cpbp_builder_destroy(handle)


def build_tiles_device(plan: Plan, row_offsets, canonical_features, values, *,
                       kind: int = ORDER_INFERRED_MINHASH, window_size: int = 1024,
                       group_width: int = 64, seed: int = DEFAULT_ORDER_SEED,
                       global_row_begin: int = 0, stream=None):
    """Device construction of the tiles (cx_cpbp_device_builder_*): inputs are torch device
    tensors (int32 storage of u32 row offsets / canonical features, f16 or f32 values) or
    numpy arrays (uploaded first). Returns (CpbpTiles on the device, primary keys). The
    result is bit-identical to build_tiles + to_device."""
    import torch

    from .engine import CpbpTiles, _stream

    def dev_u32(a):
        if isinstance(a, torch.Tensor):
            return a.contiguous()
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()

    ro, cf = dev_u32(row_offsets), dev_u32(canonical_features)
    vals = values if isinstance(values, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(values)).cuda()
    if vals.dtype not in (torch.float16, torch.float32):
        raise ValueError("CP-BP values must be float16 or float32")
    perm = dev_u32(plan.feature_permutation)
    boffs = dev_u32(plan.feature_block_offsets)
    lib = N.engine()
    cplan = N.CxCpbpPlan(plan.feature_count, plan.feature_block_count, perm.data_ptr(), boffs.data_ptr())
    csr = N.CxCpbpCsr(ro.numel() - 1, vals.element_size(), ro.data_ptr(), cf.data_ptr(), vals.data_ptr())
    cfg = N.CxCpbpOrderConfig(kind, window_size, group_width, 0, seed, global_row_begin)
    handle = C.c_void_p()
    s = _stream(stream)
    st = lib.cx_cpbp_device_builder_create(C.byref(cplan), C.byref(csr), C.byref(cfg), s, C.byref(handle))
    if st != 0:
        raise N.EngineError("cx_cpbp_device_builder_create", st,
                            lib.cx_cpbp_device_build_last_error().decode())
    try:
        req = N.CxCpbpTileRequirements()
        N.check("cx_cpbp_device_builder_requirements",
                lib.cx_cpbp_device_builder_requirements(handle, C.byref(req)))

        def buf(n, dtype):
            return torch.empty(max(n, 1), dtype=dtype, device=vals.device)[:n]

        mask_dtype = torch.int64 if req.cell_mask_bytes == 8 else torch.int32
        t = CpbpTiles(
            row_count=req.row_count, feature_count=req.feature_count,
            tile_row_width=req.tile_row_width, feature_block_offsets=boffs,
            feature_permutation=perm,
            tile_block_offsets=buf(req.tile_count + 1, torch.int32),
            tile_block_ids=buf(req.tile_block_count, torch.int32),
            tile_block_cell_masks=buf(req.tile_block_count, mask_dtype),
            block_row_entry_offsets=buf(req.tile_block_count + 1, torch.int32),
            row_block_gene_masks=buf(req.row_block_entry_count, torch.int32),
            row_block_value_offsets=buf(req.row_block_entry_count + 1, torch.int32),
            values=buf(req.nnz_count, vals.dtype), row_permutation=buf(req.row_count, torch.int32),
            meta={"tile_requirements": {f: getattr(req, f) for f, _ in req._fields_}})
        primary = buf(req.row_count, torch.int64)
        ptr = lambda x: x.data_ptr() if x.numel() else None  # noqa: E731
        bufs = N.CxCpbpTileBuffers(
            ptr(t.tile_block_offsets), ptr(t.tile_block_ids), ptr(t.tile_block_cell_masks),
            ptr(t.block_row_entry_offsets), ptr(t.row_block_gene_masks),
            ptr(t.row_block_value_offsets), ptr(t.values), ptr(t.row_permutation), ptr(primary))
        st = lib.cx_cpbp_device_builder_export(handle, C.byref(bufs), s)
        if st != 0:
            raise N.EngineError("cx_cpbp_device_builder_export", st,
                                lib.cx_cpbp_device_build_last_error().decode())
        torch.cuda.current_stream().synchronize() if stream is None else None
        return t, primary
    finally:
        lib.cx_cpbp_device_builder_destroy(handle)


def to_device(plan: Plan, tiles: HostTiles, device="cuda"):
    """Uploads the tiles and the plan subset the kernel reads as a CpbpTiles."""
    import torch

    from .engine import CpbpTiles

    def up(a: np.ndarray, dtype):
        return torch.from_numpy(np.ascontiguousarray(a).view(dtype)).to(device)

    mask_dtype = torch.int64 if tiles.tile_block_cell_masks.dtype == np.uint64 else torch.int32
    val_dtype = torch.float16 if tiles.values.dtype == np.float16 else torch.float32
    vals = torch.from_numpy(tiles.values).to(device)
    assert vals.dtype == val_dtype
    return CpbpTiles(
        row_count=tiles.req["row_count"], feature_count=tiles.req["feature_count"],
        tile_row_width=tiles.req["tile_row_width"],
        feature_block_offsets=up(plan.feature_block_offsets.astype(np.uint32), np.int32),
        feature_permutation=up(plan.feature_permutation.astype(np.uint32), np.int32),
        tile_block_offsets=up(tiles.tile_block_offsets, np.int32),
        tile_block_ids=up(tiles.tile_block_ids, np.int32),
        tile_block_cell_masks=up(tiles.tile_block_cell_masks,
                                 np.int64 if mask_dtype == torch.int64 else np.int32),
        block_row_entry_offsets=up(tiles.block_row_entry_offsets, np.int32),
        row_block_gene_masks=up(tiles.row_block_gene_masks, np.int32),
        row_block_value_offsets=up(tiles.row_block_value_offsets, np.int32),
        values=vals, row_permutation=up(tiles.row_permutation, np.int32),
        meta={"tile_requirements": tiles.req})


def decode_tiles(plan: Plan, tiles: HostTiles) -> list[dict]:
    """Host decode of tiles back to canonical rows ({canonical feature: value} per row):
    the inverse of build_tiles, used to check the projection round-trips exactly
    (decode_warp_tiles_host, components/CellPack/src/warp_tiles.cc:515)."""
    rows = tiles.req["row_count"]
    w = tiles.req["tile_row_width"]
    out = [dict() for _ in range(rows)]
    for t in range(tiles.req["tile_count"]):
        for d in range(tiles.tile_block_offsets[t], tiles.tile_block_offsets[t + 1]):
            mask = int(tiles.tile_block_cell_masks[d])
            block = int(tiles.tile_block_ids[d])
            base = int(plan.feature_block_offsets[block])
            e = int(tiles.block_row_entry_offsets[d])
            for lane in range(w):
                if not (mask >> lane) & 1:
                    continue
                canon_row = int(tiles.row_permutation[t * w + lane])
                gm = int(tiles.row_block_gene_masks[e])
                v = int(tiles.row_block_value_offsets[e])
                for local in range(32):
                    if (gm >> local) & 1:
                        out[canon_row][int(plan.feature_permutation[base + local])] = tiles.values[v]
                        v += 1
                e += 1
    return out
