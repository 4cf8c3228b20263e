"""Seeded synthetic single-cell inputs for the BASELINE configs, generated on the GPU by
libcx_synth.so (see include/cellerator_amd_synth.h for the recipe and the choices it
makes where the configs are ambiguous). Bench and test support only."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _native as N
from .engine import BellMatrix, QcsrMatrix


@dataclass(frozen=True)
class QcsrConfig:
    name: str
    rows: int
    cols: int
    bits: int  # 0 = fp32 values
    nnz_mean: float
    nnz_sigma: float = 0.0
    row_dist: int = 0  # 0 lognormal, 1 poisson
    nnz_min: int = 1
    nnz_max: int = 1 << 30
    zipf_s: float = 1.1
    nb_mean: float = 2.0
    nb_size: float = 0.5
    n_out: int = 64
    seed: int = 0xCE11E7A70000000C

    def scaled(self, rows: int) -> "QcsrConfig":
        return QcsrConfig(**{**self.__dict__, "rows": rows, "name": f"{self.name}@{rows}"})


# BASELINE.json configs[0..2]
C1 = QcsrConfig("C1 fp32 CSR 10k x 2k", 10_000, 2_000, 0, 200.0, row_dist=1, nnz_min=1,
                nnz_max=2_000, zipf_s=0.0, nb_mean=2.0, nb_size=0.5, n_out=64,
                seed=0xCE11E7A700000001)
C2 = QcsrConfig("C2 8-bit qCSR 100k x 20k", 100_000, 20_000, 8, 2_000.0, 0.5, nnz_min=200,
                nnz_max=8_000, zipf_s=1.1, nb_mean=3.0, nb_size=0.4, n_out=64,
                seed=0xCE11E7A700000002)
C3 = QcsrConfig("C3 4-bit qCSR 1M x 33538", 1_000_000, 33_538, 4, 1_500.0, 0.6, nnz_min=1,
                nnz_max=33_538, zipf_s=1.1, nb_mean=2.0, nb_size=0.5, n_out=64,
                seed=0xCE11E7A700000003)


def dense_normal(shape, stddev: float, dtype: torch.dtype, seed: int, device="cuda",
                 stream=None) -> torch.Tensor:
    out = torch.empty(shape, dtype=dtype, device=device)
    code = {torch.float16: 1, torch.float32: 2, torch.bfloat16: 5}[dtype]
    s = (stream or torch.cuda.current_stream()).cuda_stream
    N.check_synth("cxs_dense_normal", N.synth().cxs_dense_normal(
        seed, out.numel(), stddev, code, out.data_ptr(), s))
    return out


def generate_qcsr(cfg: QcsrConfig, device="cuda") -> QcsrMatrix:
    """Builds the quantized (or fp32) CSR matrix of `cfg` directly in device memory."""
    lib = N.synth()
    p = N.CxsQcsrParams()
    p.seed, p.rows, p.cols, p.row_dist, p.bits = cfg.seed, cfg.rows, cfg.cols, cfg.row_dist, cfg.bits
    p.nnz_mean, p.nnz_sigma = cfg.nnz_mean, cfg.nnz_sigma
    p.nnz_min, p.nnz_max = cfg.nnz_min, min(cfg.nnz_max, cfg.cols)
    p.zipf_s, p.nb_mean, p.nb_size = cfg.zipf_s, cfg.nb_mean, cfg.nb_size
    gen = C.c_void_p()
    N.check_synth("cxs_qcsr_create", lib.cxs_qcsr_create(C.byref(p), C.byref(gen)))
    s = torch.cuda.current_stream().cuda_stream
    try:
        row_nnz = torch.empty(cfg.rows, dtype=torch.int32, device=device)
        N.check_synth("cxs_qcsr_count", lib.cxs_qcsr_count(gen, row_nnz.data_ptr(), s))
        counts = row_nnz.to(torch.int64)
        total = int(counts.sum().item())
        if total >= 2**31:
            raise ValueError(f"{cfg.name}: nnz {total} exceeds int32 row offsets")
        row_ptr = torch.zeros(cfg.rows + 1, dtype=torch.int32, device=device)
        row_ptr[1:] = torch.cumsum(counts, 0).to(torch.int32)
        col_idx = torch.empty(max(total, 1), dtype=torch.int32, device=device)[:total]
        gmin = torch.full((cfg.cols,), -1, dtype=torch.int32, device=device)  # 0xffffffff
        gmax = torch.zeros(cfg.cols, dtype=torch.int32, device=device)
        N.check_synth("cxs_qcsr_fill", lib.cxs_qcsr_fill(
            gen, row_ptr.data_ptr(), col_idx.data_ptr(), gmin.data_ptr(), gmax.data_ptr(), s))
        if cfg.bits == 0:
            values = torch.empty(max(total, 1), dtype=torch.float32, device=device)[:total]
            N.check_synth("cxs_qcsr_encode", lib.cxs_qcsr_encode(
                gen, row_ptr.data_ptr(), None, col_idx.data_ptr(), None, None, None,
                values.data_ptr(), s))
            torch.cuda.synchronize()
            return QcsrMatrix(cfg.rows, cfg.cols, 0, row_ptr, col_idx, values=values,
                              meta={"config": cfg.name})
        cpb = 8 // cfg.bits
        packed_counts = (counts + cpb - 1) // cpb
        packed_row_ptr = torch.zeros(cfg.rows + 1, dtype=torch.int32, device=device)
        packed_row_ptr[1:] = torch.cumsum(packed_counts, 0).to(torch.int32)
        packed_bytes = int(packed_counts.sum().item())
        # +16 so that vector loads of the last row's tail stay inside the allocation
        packed = torch.zeros(packed_bytes + 16, dtype=torch.uint8, device=device)
        scales = torch.empty(cfg.cols, dtype=torch.float32, device=device)
        offsets = torch.empty(cfg.cols, dtype=torch.float32, device=device)
        N.check_synth("cxs_qcsr_calibrate", lib.cxs_qcsr_calibrate(
            gen, gmin.data_ptr(), gmax.data_ptr(), scales.data_ptr(), offsets.data_ptr(), s))
        N.check_synth("cxs_qcsr_encode", lib.cxs_qcsr_encode(
            gen, row_ptr.data_ptr(), packed_row_ptr.data_ptr(), col_idx.data_ptr(),
            scales.data_ptr(), offsets.data_ptr(), packed.data_ptr(), None, s))
        torch.cuda.synchronize()
        return QcsrMatrix(cfg.rows, cfg.cols, cfg.bits, row_ptr, col_idx,
                          packed_row_ptr=packed_row_ptr, packed_values=packed,
                          column_scales=scales, column_offsets=offsets,
                          meta={"config": cfg.name})
    finally:
        lib.cxs_destroy(gen)


@dataclass(frozen=True)
class BellConfig:
    name: str
    rows: int
    cols: int
    block_size: int = 32
    ell_width: int = 64
    patterns: int = 40
    min_blocks: int = 24
    max_blocks: int = 64
    density: float = 0.35
    nb_mean: float = 2.0
    nb_size: float = 0.5
    n_out: int = 256
    seed: int = 0xCE11E7A700000004

    def scaled(self, rows: int) -> "BellConfig":
        return BellConfig(**{**self.__dict__, "rows": rows, "name": f"{self.name}@{rows}"})


# BASELINE.json configs[3]
C4 = BellConfig("C4 Blocked-ELL bf16 500k x 20k", 500_000, 20_000)


def generate_bell(cfg: BellConfig, device="cuda") -> BellMatrix:
    rb = cfg.rows // cfg.block_size
    idx = torch.empty((rb, cfg.ell_width), dtype=torch.int32, device=device)
    ell_cols = cfg.ell_width * cfg.block_size
    values = torch.empty((cfg.rows, ell_cols), dtype=torch.bfloat16, device=device)
    s = torch.cuda.current_stream().cuda_stream
    N.check_synth("cxs_bell_generate", N.synth().cxs_bell_generate(
        cfg.seed, cfg.rows, cfg.cols, cfg.block_size, cfg.ell_width, cfg.patterns,
        cfg.min_blocks, cfg.max_blocks, cfg.density, cfg.nb_mean, cfg.nb_size, idx.data_ptr(),
        values.data_ptr(), s))
    return BellMatrix(cfg.rows, cfg.cols, cfg.block_size, ell_cols, idx, values=values,
                      meta={"config": cfg.name})


@dataclass(frozen=True)
class CpbpConfig:
    name: str
    rows: int
    genes: int = 20_000
    modules: int = 200
    module_size: int = 100
    min_active: int = 3
    max_active: int = 8
    active_genes: int = 60  # 60% of a module's genes
    background: int = 50
    nb_mean: float = 2.0
    nb_size: float = 0.5
    block_width: int = 25  # module-aligned feature blocks (4 per module)
    tile_row_width: int = 64
    window_size: int = 1024
    seed: int = 0xCE11E7A700000005

    def scaled(self, rows: int) -> "CpbpConfig":
        return CpbpConfig(**{**self.__dict__, "rows": rows, "name": f"{self.name}@{rows}"})


# BASELINE.json configs[4]
C5 = CpbpConfig("C5 CP-BP 2M x 20k, 64-row tiles", 2_000_000)


def generate_cpbp_host(cfg: CpbpConfig, threads: int | None = None):
    """Canonical CSR (row_offsets uint32, features uint32, values float32) of config 5,
    generated on host threads (include/cellerator_amd_synth.h)."""
    import os

    import numpy as np

    lib = N.synth()
    p = N.CxsCpbpParams(cfg.seed, cfg.rows, cfg.genes, cfg.modules, cfg.module_size,
                        cfg.min_active, cfg.max_active, cfg.active_genes, cfg.background,
                        cfg.nb_mean, cfg.nb_size)
    nthreads = threads or min(16, os.cpu_count() or 1)
    counts = np.zeros(cfg.rows, np.uint32)
    N.check_synth("cxs_cpbp_count", lib.cxs_cpbp_count(C.byref(p), counts.ctypes.data, nthreads))
    offs = np.zeros(cfg.rows + 1, np.uint64)
    np.cumsum(counts, out=offs[1:])
    if offs[-1] >= 2**32:
        raise ValueError(f"{cfg.name}: nnz {int(offs[-1])} exceeds uint32 offsets")
    offs = offs.astype(np.uint32)
    feats = np.zeros(int(offs[-1]), np.uint32)
    vals = np.zeros(int(offs[-1]), np.float32)
    N.check_synth("cxs_cpbp_fill", lib.cxs_cpbp_fill(C.byref(p), offs.ctypes.data, feats.ctypes.data,
                                                      vals.ctypes.data, nthreads))
    return offs, feats, vals
