"""CPE2 execution image (cpe2.cpp) against the reference's own test
(components/CellPack/tests/persistence/execution_image_v2_test.cc): the 10-section,
2-projection image builds and validates, byte accounting adds up, prebinding gives each
projection its sections (and nothing for a lazy one), prebinding for an opaque destination
base keeps the validated offsets, a relocated copy validates and prebinds to the same bytes,
rebinding moves only the directories, and corruption, truncation, stale identities, bad
alignments and unknown required projections are rejected. Also the format constants the
reference asserts (256-byte header, 64-byte entries) and the CPK1 compatibility loader."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cellerator_amd import cpe2 as X


def reference_sections():
    """execution_image_v2_test.cc:113-148."""
    domains = np.array([11, 12], np.uint64)
    order = np.array([2, 0, 3, 1], np.uint32)
    relation = np.array([21, 22, 23], np.uint64)
    geometry = np.array([0, 2, 4, 8], np.uint32)
    values = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    payload = np.array([3, 1, 4, 1, 5], np.uint32)
    forward = np.array([0, 2, 1, 3], np.uint32)
    transpose = np.array([0, 2, 1, 3], np.uint32)
    summary = np.array([100, 200], np.uint64)
    extension = np.array([0x55, 0xAA], np.uint32)
    secs = [X.section(X.DOMAIN, 1, domains, element_count=2, element_bytes=8),
            X.section(X.ORDER, 2, order, element_count=4, element_bytes=4),
            X.section(X.RELATION, 3, relation), X.section(X.GEOMETRY, 4, geometry),
            X.section(X.INITIAL_VALUES, 5, values, element_count=4, element_bytes=4),
            X.section(X.PAYLOAD, 6, payload), X.section(X.FORWARD_MAP, 7, forward),
            X.section(X.TRANSPOSE_MAP, 8, transpose), X.section(X.SUMMARY, 9, summary),
            X.section(0x90000001, 10, extension, flags=X.OPTIONAL)]
    for s in secs:
        s.alignment = 64
    projs = [X.projection(101, X.NATIVE_ROW_MASKED, X.FORWARD_CAPABLE | X.TRANSPOSE_CAPABLE, 5, 6, 7, 8, 9),
             X.projection(102, 0x90000002, X.OPTIONAL | X.LAZY, X.INVALID)]
    return secs, projs, payload


def test_layout_constants():
    assert C.sizeof(X.Header) == 256 and C.sizeof(X.SectionEntry) == 64 and C.sizeof(X.ProjectionEntry) == 64
    assert X.Header.image_identity.offset == 32 and C.sizeof(X.AxisIdentity) == 72


def test_reference_image_round_trip():
    secs, projs, payload = reference_sections()
    req = X.request(secs, projs, 17)
    need = X.requirements(req)
    assert need.image_bytes > need.directory_bytes + need.section_bytes and need.alignment_padding_bytes != 0
    image, built = X.build(req)
    h = built.header
    assert bytes(h.magic) == b"CELLEX02" and h.schema_version == 2 and h.endian == 0x01020304
    assert h.image_identity != 0 and h.section_count == 10 and h.projection_count == 2
    assert need.image_bytes % 64 == 0 and h.section_directory_offset == 256 and h.projection_directory_offset % 64 == 0
    pre = X.prebind(built, 0)
    assert (pre.payload_bytes, pre.forward_map_bytes, pre.transpose_map_bytes, pre.scheduling_summary_bytes) == \
        (payload.nbytes, 16, 16, 16)
    dest = (C.c_ubyte * 8)()
    far = X.prebind(built, 0, C.addressof(dest), image.size)
    assert far.payload == C.addressof(dest) + built.sections[5].offset and far.payload_bytes == payload.nbytes
    with pytest.raises(X.Cpe2Error, match="destination size differs"):
        X.prebind(built, 0, C.addressof(dest), image.size - 1)
    lazy = X.prebind(built, 1)
    assert lazy.payload is None and lazy.payload_bytes == 0
    relocated = image.copy()
    rview = X.validate(relocated, X.expected(h.image_identity))
    rpre = X.prebind(rview, 0)
    assert rpre.payload != pre.payload
    assert bytes((C.c_ubyte * payload.nbytes).from_address(rpre.payload)) == payload.tobytes()
    placeholder = (C.c_ubyte * 8)()
    rebound = X.rebind(built, C.addressof(placeholder), image.size)
    assert rebound.image_base == C.addressof(placeholder)
    assert C.addressof(rebound.sections.contents) != C.addressof(built.sections.contents)


@pytest.mark.parametrize("case", ["corrupted", "truncated", "structure", "epoch", "catalog", "image_identity"])
def test_rejections(case):
    secs, projs, _ = reference_sections()
    image, built = X.build(X.request(secs, projs, 17))
    exp = X.expected()
    data = image.copy()
    if case == "corrupted":
        data[-1] ^= 0x80
    elif case == "truncated":
        data = data[:-1]
    elif case == "structure":
        exp.structure_identity.low ^= 1
    elif case == "epoch":
        exp.structure_epoch = 10
    elif case == "catalog":
        exp.projection_catalog_identity.high ^= 1
    elif case == "image_identity":
        exp.image_identity = built.header.image_identity ^ 1
    with pytest.raises(X.Cpe2Error):
        X.validate(data, exp)


def test_request_rejections():
    secs, projs, _ = reference_sections()
    bad = list(secs)
    bad[5] = X.section(X.PAYLOAD, 6, np.arange(5, dtype=np.uint32), alignment=3)
    with pytest.raises(X.Cpe2Error, match="section source is invalid"):
        X.requirements(X.request(bad, projs, 17))
    bad_projs = [projs[0], X.projection(102, 0x90000002, X.LAZY, X.INVALID)]
    with pytest.raises(X.Cpe2Error, match="projection descriptor is invalid"):
        X.requirements(X.request(secs, bad_projs, 17))
    # structure-only images (no initial values, generation 0) are allowed
    only = [secs[0], secs[1], secs[2], secs[3], secs[5]]
    p = X.projection(101, X.NATIVE_ROW_MASKED, X.FORWARD_CAPABLE, 4)
    X.requirements(X.request(only, [p], 0))
    with pytest.raises(X.Cpe2Error, match="present together"):
        X.requirements(X.request(only, [p], 5))
    dup = [secs[0], secs[1], secs[2], secs[3], secs[5], X.section(X.DOMAIN, 77, np.zeros(2, np.uint64))]
    with pytest.raises(X.Cpe2Error, match="incomplete or duplicated"):
        X.requirements(X.request(dup, [p], 0))
    no_lazy = X.projection(103, X.CSR, 0, X.INVALID)
    with pytest.raises(X.Cpe2Error, match="lazy-constructible"):
        X.requirements(X.request(only, [p, no_lazy], 0))
    wrong_map = X.projection(104, X.CSR, 0, 4, forward=2)
    with pytest.raises(X.Cpe2Error, match="forward map"):
        X.requirements(X.request(only, [p, wrong_map], 0))


def test_cpk1_compatibility_section():
    """load_cpk1_v1_compatibility_host: a native row-masked projection whose payload is a CPK1
    image validates through the CPK1 reader unchanged; other projections are refused."""
    from cellerator_amd import cpk1
    from tests.test_cpk1 import build_reference_image
    _, _, cimage, cview = build_reference_image()
    secs = [X.section(X.DOMAIN, 1, np.array([1, 2], np.uint64)), X.section(X.ORDER, 2, np.array([1, 0], np.uint32)),
            X.section(X.RELATION, 3, np.array([3, 4], np.uint64)), X.section(X.GEOMETRY, 4, np.array([0, 2], np.uint32)),
            X.section(X.CPK1_COMPAT, 5, cimage, alignment=256), X.section(X.PAYLOAD, 6, np.arange(4, dtype=np.uint32))]
    projs = [X.projection(10, X.NATIVE_ROW_MASKED, X.FORWARD_CAPABLE, 4),
             X.projection(11, X.CSR, X.FORWARD_CAPABLE, 5)]
    image, view = X.build(X.request(secs, projs, 0))
    loaded = X.load_cpk1(view, 0, cpk1.expected_of(cview))
    assert loaded.payload_identity == cview.payload_identity
    assert loaded.image_base == view.image_base + view.sections[4].offset
    with pytest.raises(X.Cpe2Error, match="does not contain a CPK1"):
        X.load_cpk1(view, 1, cpk1.expected_of(cview))


@pytest.mark.gpu
def test_cpk1_projection_runs_from_one_device_upload(oracle):
    """The whole execution image goes to the device in one copy; prebind_for_base against the
    device base gives the CPK1 compatibility payload's device address, the CPK1 view loaded on
    the host is rebound there, and the checked CP-BP reduction over it equals the reduction on
    separately uploaded tiles bit for bit (and the canonical oracle within f32 rounding)."""
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import cpbp, cpbp_reduce, cpk1
    from tests.test_cpk1 import build_reference_image, reference_source
    plan, tiles, cimage, cview = build_reference_image()
    secs = [X.section(X.DOMAIN, 1, np.array([1, 2], np.uint64)), X.section(X.ORDER, 2, np.array([1, 0], np.uint32)),
            X.section(X.RELATION, 3, np.array([3, 4], np.uint64)), X.section(X.GEOMETRY, 4, np.array([0, 2], np.uint32)),
            X.section(X.CPK1_COMPAT, 5, cimage, alignment=256)]
    image, view = X.build(X.request(secs, [X.projection(10, X.NATIVE_ROW_MASKED, X.FORWARD_CAPABLE, 4)], 0))
    dev = torch.from_numpy(image).cuda()
    pre = X.prebind(view, 0, dev.data_ptr(), dev.numel())
    assert pre.payload == dev.data_ptr() + view.sections[4].offset and pre.payload_bytes == cimage.size
    host = X.load_cpk1(view, 0, cpk1.expected_of(cview))
    moved = N.CxCpk1View()
    assert N.engine().cx_cpk1_rebind(C.byref(host), pre.payload, pre.payload_bytes, C.byref(moved)) == 0
    rv = N.CxCpbpReductionView()
    assert N.engine().cx_cpbp_reduction_view_from_cpk1(C.byref(moved), 0x5EED, C.byref(rv)) == 0
    w = torch.from_numpy((0.5 + 0.125 * np.arange(6)).astype(np.float32)).cuda()
    out = torch.full((int(moved.tiles.row_count),), -7.0, device="cuda")
    assert N.engine().cx_cpbp_reduce_checked(C.byref(rv), w.data_ptr(), w.numel(), out.data_ptr(), out.numel(),
                                             None) == 0
    direct = cpbp_reduce(cpbp.to_device(plan, tiles), w)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), direct.view(torch.int32))
    offs, feats, vals = reference_source()
    ref, _ = oracle.cpbp_canonical_f64(offs, feats, vals, w.cpu().numpy(), oracle.F16)
    assert np.allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
