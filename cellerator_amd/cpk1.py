"""CPK1 persistent packing payload (the reference's pointer-free partition image,
components/CellPack/include/CellPack/persistent_packing_payload.hh): write an image of
host-built warp tiles, validate it, upload it to the device in one copy and rebind the
view there, so cx_cpbp_reduce runs directly on the uploaded image.

CPK1 v1 carries u32 cell masks (tile widths up to 32) and f16 values.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .cpbp import HostTiles, Plan

OBJECTIVE_TOTAL_BYTES, OBJECTIVE_ROW_ACTIVE_BLOCK_REFERENCES, OBJECTIVE_WEIGHTED = 1, 2, 3
ROW_DOMAIN_FULL, ROW_DOMAIN_SAMPLED = 1, 2


def _p(a: np.ndarray):
    return a.ctypes.data if a is not None and a.size else None


def _check(name: str, status: int) -> None:
    if status != 0:
        raise N.EngineError(name, status, N.engine().cx_cpk1_last_error().decode())


@dataclass
class Metadata:
    """The plan identity, row domain and local-order settings an image records."""
    feature_axis_fingerprint: int
    row_domain_identity: int
    full_row_count: int
    global_row_begin: int = 0
    feature_axis_fingerprint_version: int = 1
    row_domain_kind: int = ROW_DOMAIN_FULL
    evaluation_source_identity: int = 0
    sampling_provenance_identity: int = 0
    cost_policy_identity: int = 1
    objective_kind: int = OBJECTIVE_ROW_ACTIVE_BLOCK_REFERENCES
    row_group_width: int = 32
    row_group_offsets: np.ndarray | None = None
    maximum_feature_block_width: int = 0
    order_kind: int = 1
    window_size: int = 1024
    group_width: int = 32
    seed: int = 0x6A09E667F3BCC909

    def native(self) -> N.CxCpk1Metadata:
        groups = None if self.row_group_offsets is None else np.ascontiguousarray(
            self.row_group_offsets, dtype=np.uint32)
        m = N.CxCpk1Metadata(
            self.feature_axis_fingerprint, self.feature_axis_fingerprint_version,
            self.row_domain_kind, self.row_domain_identity, self.evaluation_source_identity,
            self.sampling_provenance_identity, self.cost_policy_identity, self.objective_kind,
            self.full_row_count, self.maximum_feature_block_width, self.row_group_width,
            0 if groups is None else groups.size - 1, 0, _p(groups), self.global_row_begin,
            N.CxCpbpOrderConfig(self.order_kind, self.window_size, self.group_width, 0, self.seed,
                                self.global_row_begin))
        m._keep = groups
        return m


def expected_of(view: N.CxCpk1View) -> N.CxCpk1Expected:
    """The compatibility identity a loader checks (persistent_packing_payload_compatibility)."""
    return N.CxCpk1Expected(view.global_row_begin, view.tiles.row_count, view.tiles.feature_count,
                            0, view.feature_axis_fingerprint,
                            view.feature_axis_fingerprint_version, 0, view.row_domain_identity,
                            view.payload_identity)


def write_image(plan: Plan, tiles: HostTiles, meta: Metadata) -> tuple[np.ndarray, N.CxCpk1View]:
    """The CPK1 image (uint8, 64-byte aligned) of host-built tiles, and its validated view."""
    lib = N.engine()
    req = N.CxCpbpTileRequirements(*[tiles.req[f] for f, _ in N.CxCpbpTileRequirements._fields_])
    groups = meta.row_group_offsets
    group_count = (len(groups) - 1) if groups is not None else \
        (meta.full_row_count + meta.row_group_width - 1) // meta.row_group_width
    nbytes = C.c_uint64()
    _check("cx_cpk1_image_bytes", lib.cx_cpk1_image_bytes(C.byref(req), group_count, C.byref(nbytes)))
    raw = np.zeros(nbytes.value + 64, np.uint8)
    off = (-raw.ctypes.data) % 64
    image = raw[off:off + nbytes.value]
    perm = np.ascontiguousarray(plan.feature_permutation, dtype=np.uint32)
    boffs = np.ascontiguousarray(plan.feature_block_offsets, dtype=np.uint32)
    cplan = N.CxCpbpPlan(plan.feature_count, plan.feature_block_count, _p(perm), _p(boffs))
    bufs = N.CxCpbpTileBuffers(
        _p(tiles.tile_block_offsets), _p(tiles.tile_block_ids), _p(tiles.tile_block_cell_masks),
        _p(tiles.block_row_entry_offsets), _p(tiles.row_block_gene_masks),
        _p(tiles.row_block_value_offsets), _p(tiles.values), _p(tiles.row_permutation), None)
    m = meta.native()
    view = N.CxCpk1View()
    _check("cx_cpk1_write", lib.cx_cpk1_write(C.byref(cplan), C.byref(m), C.byref(req), C.byref(bufs),
                                              image.ctypes.data, image.size, C.byref(view)))
    return image, view


def validate(image: np.ndarray, expected: N.CxCpk1Expected) -> N.CxCpk1View:
    """Host validation of an image (validate_persistent_packing_payload_host)."""
    image = np.ascontiguousarray(image, dtype=np.uint8)
    view = N.CxCpk1View()
    _check("cx_cpk1_validate", N.engine().cx_cpk1_validate(image.ctypes.data, image.size,
                                                            C.byref(expected), C.byref(view)))
    view._keep = image
    return view


@dataclass
class DeviceImage:
    """An image uploaded to the device in one copy and its rebound view: usable wherever a
    CpbpTiles is (cpbp_reduce reads row_count, values and descriptor())."""
    image: object            # torch uint8 device tensor holding the whole image
    view: N.CxCpk1View        # pointers rebound into `image`
    meta: dict = field(default_factory=dict)

    @property
    def row_count(self) -> int:
        return int(self.view.tiles.row_count)

    @property
    def values(self):
        return self.image

    def descriptor(self) -> N.CxCpbpTiles:
        return N.CxCpbpTiles.from_buffer_copy(self.view.tiles)


def upload(host_view: N.CxCpk1View, image: np.ndarray, device="cuda") -> DeviceImage:
    """One opaque upload of the validated image, then rebind_persistent_packing_payload."""
    import torch

    dev = torch.from_numpy(np.ascontiguousarray(image)).to(device)
    out = N.CxCpk1View()
    _check("cx_cpk1_rebind", N.engine().cx_cpk1_rebind(C.byref(host_view), dev.data_ptr(),
                                                        dev.numel(), C.byref(out)))
    return DeviceImage(dev, out)
