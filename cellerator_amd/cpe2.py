"""CPE2 execution image (cpe2.cpp): ctypes mirrors of the C-ABI structs and a small host
front-end -- build, validate, rebind, prebind, and the CPK1 compatibility loader
(components/CellPack/include/CellPack/persistence/execution_image_v2.hh)."""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from . import _native as N

u16, u32, u64, p_void = C.c_uint16, C.c_uint32, C.c_uint64, C.c_void_p
INVALID = 0xFFFFFFFF
DOMAIN, ORDER, RELATION, GEOMETRY, INITIAL_VALUES, PAYLOAD = 1, 2, 3, 4, 5, 6
FORWARD_MAP, TRANSPOSE_MAP, HIERARCHY, SUMMARY, CPK1_COMPAT = 7, 8, 9, 10, 11
NATIVE_ROW_MASKED, CSR, BLOCKED_ELL = 1, 5, 8
OPTIONAL, DEVICE_READABLE, LAZY, FORWARD_CAPABLE, TRANSPOSE_CAPABLE = 1, 2, 4, 8, 16


class Id(C.Structure):
    _fields_ = [("low", u64), ("high", u64)]


class AxisRecord(C.Structure):
    _fields_ = [(n, u64) for n in ("domain_low", "domain_high", "order_low", "order_high", "geometry_low",
                                   "geometry_high", "partition_low", "partition_high")]


class AxisIdentity(C.Structure):
    _fields_ = [("schema_version", u16), ("record_kind", u16), ("byte_count", u32), ("domain", Id),
                ("order", Id), ("geometry", Id), ("partition", Id)]


class Header(C.Structure):
    _fields_ = [("magic", C.c_ubyte * 8), ("schema_version", u32), ("header_bytes", u32), ("endian", u32),
                ("alignment", u32), ("image_bytes", u64), ("image_identity", u64),
                ("structure_identity_low", u64), ("structure_identity_high", u64), ("structure_epoch", u64),
                ("semantic_geometry_identity_low", u64), ("semantic_geometry_identity_high", u64),
                ("projection_catalog_identity_low", u64), ("projection_catalog_identity_high", u64),
                ("initial_value_generation", u64), ("source_axis", AxisRecord), ("destination_axis", AxisRecord),
                ("section_count", u32), ("projection_count", u32), ("section_directory_offset", u64),
                ("projection_directory_offset", u64)]


class SectionEntry(C.Structure):
    _fields_ = [("kind", u32), ("schema_version", u32), ("flags", u32), ("alignment", u32),
                ("identity_low", u64), ("identity_high", u64), ("offset", u64), ("bytes", u64),
                ("checksum", u64), ("element_count", u32), ("element_bytes", u32)]


class ProjectionEntry(C.Structure):
    _fields_ = [("identity_low", u64), ("identity_high", u64), ("kind", u32), ("schema_version", u32),
                ("flags", u32), ("operation_family", u32), ("storage_type", u16), ("compute_type", u16),
                ("accumulation_type", u16), ("orientation", u16), ("architecture_class", u32),
                ("payload_section", u32), ("forward_map_section", u32), ("transpose_map_section", u32),
                ("scheduling_summary_section", u32), ("capability_section", u32)]


class SectionSource(C.Structure):
    _fields_ = [("kind", u32), ("schema_version", u32), ("flags", u32), ("alignment", u32),
                ("identity_low", u64), ("identity_high", u64), ("data", p_void), ("bytes", u64),
                ("element_count", u32), ("element_bytes", u32)]


class BuildRequest(C.Structure):
    _fields_ = [("structure_identity", Id), ("structure_epoch", u64), ("semantic_geometry_identity", Id),
                ("projection_catalog_identity", Id), ("initial_value_generation", u64),
                ("source_axis", AxisIdentity), ("destination_axis", AxisIdentity),
                ("sections", C.POINTER(SectionSource)), ("section_count", u32), ("reserved", u32),
                ("projections", C.POINTER(ProjectionEntry)), ("projection_count", u32), ("reserved2", u32)]


class Requirements(C.Structure):
    _fields_ = [("image_bytes", u64), ("directory_bytes", u64), ("section_bytes", u64),
                ("alignment_padding_bytes", u64)]


class Expected(C.Structure):
    _fields_ = [("structure_identity", Id), ("structure_epoch", u64), ("semantic_geometry_identity", Id),
                ("projection_catalog_identity", Id), ("image_identity", u64)]


class View(C.Structure):
    _fields_ = [("header", Header), ("image_base", p_void), ("image_bytes", u64),
                ("sections", C.POINTER(SectionEntry)), ("projections", C.POINTER(ProjectionEntry))]


class Prebound(C.Structure):
    _fields_ = [("descriptor", ProjectionEntry), ("payload", p_void), ("payload_bytes", u64),
                ("forward_map", p_void), ("forward_map_bytes", u64), ("transpose_map", p_void),
                ("transpose_map_bytes", u64), ("scheduling_summary", p_void), ("scheduling_summary_bytes", u64)]


_SIGS = {
    "cx_cpe2_query_requirements": (C.c_int, [C.POINTER(BuildRequest), C.POINTER(Requirements)]),
    "cx_cpe2_build": (C.c_int, [C.POINTER(BuildRequest), p_void, u64, C.POINTER(View)]),
    "cx_cpe2_validate": (C.c_int, [p_void, u64, C.POINTER(Expected), C.POINTER(View)]),
    "cx_cpe2_rebind": (C.c_int, [C.POINTER(View), p_void, u64, C.POINTER(View)]),
    "cx_cpe2_prebind": (C.c_int, [C.POINTER(View), u32, C.POINTER(Prebound)]),
    "cx_cpe2_prebind_for_base": (C.c_int, [C.POINTER(View), u32, p_void, u64, C.POINTER(Prebound)]),
    "cx_cpe2_load_cpk1": (C.c_int, [C.POINTER(View), u32, C.POINTER(N.CxCpk1Expected), C.POINTER(N.CxCpk1View)]),
    "cx_cpe2_last_error": (C.c_char_p, []),
}


def lib():
    e = N.engine()
    if not getattr(e, "_cpe2_sigs", False):
        for name, (res, args) in _SIGS.items():
            f = getattr(e, name)
            f.restype, f.argtypes = res, args
        e._cpe2_sigs = True
    return e


class Cpe2Error(RuntimeError):
    pass


def _check(name: str, rc: int) -> None:
    if rc != 0:
        raise Cpe2Error(f"{name}: {lib().cx_cpe2_last_error().decode()}")


def axis(seed: int) -> AxisIdentity:
    """A persistent axis identity record (identity.hh:94-100) with identities seed+1 .. seed+8."""
    a = AxisIdentity(1, 1, C.sizeof(AxisIdentity))
    a.domain, a.order = Id(seed + 1, seed + 2), Id(seed + 3, seed + 4)
    a.geometry, a.partition = Id(seed + 5, seed + 6), Id(seed + 7, seed + 8)
    return a


def section(kind: int, identity: int, data: np.ndarray, flags: int = DEVICE_READABLE, element_count: int = 0,
            element_bytes: int = 0, alignment: int = 64, identity_high: Optional[int] = None) -> SectionSource:
    data = np.ascontiguousarray(data)
    s = SectionSource(kind, 1, flags, alignment, identity,
                      identity ^ 0xA5A5A5A5 if identity_high is None else identity_high, data.ctypes.data,
                      data.nbytes, element_count, element_bytes)
    s._keep = data
    return s


def projection(identity: int, kind: int, flags: int, payload: int, forward: int = INVALID, transpose: int = INVALID,
               summary: int = INVALID, capability: int = INVALID) -> ProjectionEntry:
    return ProjectionEntry(identity, identity ^ 0x5A5A5A5A, kind, 1, flags, 7, 1, 2, 2, 1, 70, payload, forward,
                           transpose, summary, capability)


def request(sections: Sequence[SectionSource], projections: Sequence[ProjectionEntry], generation: int,
            structure=(0x101, 0x102), epoch=9, geometry=(0x201, 0x202), catalog=(0x301, 0x302)) -> BuildRequest:
    secs = (SectionSource * len(sections))(*sections)
    projs = (ProjectionEntry * len(projections))(*projections)
    r = BuildRequest(Id(*structure), epoch, Id(*geometry), Id(*catalog), generation, axis(0x1000), axis(0x2000),
                     C.cast(secs, C.POINTER(SectionSource)), len(sections), 0,
                     C.cast(projs, C.POINTER(ProjectionEntry)), len(projections), 0)
    r._keep = (secs, projs, sections)
    return r


def expected(image_identity: int = 0, structure=(0x101, 0x102), epoch=9, geometry=(0x201, 0x202),
             catalog=(0x301, 0x302)) -> Expected:
    return Expected(Id(*structure), epoch, Id(*geometry), Id(*catalog), image_identity)


def requirements(r: BuildRequest) -> Requirements:
    out = Requirements()
    _check("cx_cpe2_query_requirements", lib().cx_cpe2_query_requirements(C.byref(r), C.byref(out)))
    return out


def build(r: BuildRequest) -> tuple[np.ndarray, View]:
    req = requirements(r)
    image = np.zeros(req.image_bytes, np.uint8)
    view = View()
    _check("cx_cpe2_build", lib().cx_cpe2_build(C.byref(r), image.ctypes.data, image.size, C.byref(view)))
    view._keep = image
    return image, view


def validate(image: np.ndarray, exp: Expected) -> View:
    image = np.ascontiguousarray(image)
    view = View()
    _check("cx_cpe2_validate", lib().cx_cpe2_validate(image.ctypes.data, image.size, C.byref(exp), C.byref(view)))
    view._keep = image
    return view


def rebind(view: View, base: int, nbytes: int) -> View:
    out = View()
    _check("cx_cpe2_rebind", lib().cx_cpe2_rebind(C.byref(view), base, nbytes, C.byref(out)))
    return out


def prebind(view: View, index: int, base: Optional[int] = None, nbytes: Optional[int] = None) -> Prebound:
    out = Prebound()
    if base is None:
        _check("cx_cpe2_prebind", lib().cx_cpe2_prebind(C.byref(view), index, C.byref(out)))
    else:
        _check("cx_cpe2_prebind_for_base", lib().cx_cpe2_prebind_for_base(C.byref(view), index, base, nbytes,
                                                                          C.byref(out)))
    return out


def load_cpk1(view: View, index: int, exp: N.CxCpk1Expected) -> N.CxCpk1View:
    out = N.CxCpk1View()
    _check("cx_cpe2_load_cpk1", lib().cx_cpe2_load_cpk1(C.byref(view), index, C.byref(exp), C.byref(out)))
    return out
