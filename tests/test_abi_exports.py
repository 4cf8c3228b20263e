"""The C-ABI libraries load on a machine without a GPU and export every function the
public headers declare (include/cellerator_amd.h -> libcellerator_amd.so,
include/cellerator_amd_synth.h -> libcx_synth.so). No compute entry point is called."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from cellerator_amd import _native as N

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", re.M)


def declared_functions(header: Path) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
    names = []
    for m in DECL.finditer(text):
        line = text[m.start():text.find("\n", m.start())]
        if line.lstrip().startswith(("typedef", "return", "if", "for", "while")):
            continue
        names.append(m.group(1))
    return sorted(set(names))


@pytest.mark.parametrize("header,lib", [("cellerator_amd.h", N.ENGINE_PATH),
                                        ("cellerator_amd_synth.h", N.SYNTH_PATH)])
def test_library_exports_every_declared_function(header, lib):
    names = declared_functions(ROOT / "include" / header)
    assert len(names) >= 5, names
    handle = C.CDLL(str(lib))
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, f"{lib.name} lacks {missing}"


def test_header_parse_sees_the_main_entry_points():
    names = declared_functions(ROOT / "include" / "cellerator_amd.h")
    for n in ("cx_qcsr_spmm_fwd", "cx_bell_spmm_fwd_packed", "cx_cpbp_reduce",
              "cx_cpbp_builder_create", "cellerator_sparse_projection_forward"):
        assert n in names


def test_build_info_names_gfx950():
    lib = N.engine()
    info = lib.cx_build_info().decode()
    assert "gfx950" in info
