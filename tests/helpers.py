"""Shared helpers for the test suite: random CSR construction in numpy, upload to the
device, download of generated matrices, and tolerance checks against the oracle."""
from __future__ import annotations

import numpy as np

REL_TOL = 1e-4  # north_star: within 1e-4 relative (fp32 accumulation, reordered sums)
# Times sum |x||w| of the element: fp32 sums of n terms in any order stay within about
# n * 2^-24 * sum |x||w| (and typically sqrt(n) * 2^-24); 2^-20 covers the row lengths of the
# benchmark configurations (a few thousand terms) with room, and is the bound bench.py checks
# its timed outputs against. Losing one part of the matrix-core head's three-part split (an
# error of about 2^-12 of every head term) fails it at these row lengths.
ABS_TOL_SCALED = 2.0 ** -20


def random_csr(rng: np.random.Generator, rows: int, cols: int, mean_nnz: float,
               empty_every: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Row offsets and sorted unique columns; every `empty_every`-th row is empty."""
    counts = np.minimum(rng.poisson(mean_nnz, rows), cols).astype(np.int64)
    if empty_every:
        counts[::empty_every] = 0
    row_ptr = np.zeros(rows + 1, dtype=np.int64)
    row_ptr[1:] = np.cumsum(counts)
    cols_out = np.empty(int(row_ptr[-1]), dtype=np.int32)
    for r in range(rows):
        c = counts[r]
        if c:
            cols_out[row_ptr[r]:row_ptr[r + 1]] = np.sort(rng.choice(cols, size=c, replace=False))
    return row_ptr.astype(np.int32), cols_out


def quantized_fixture(oracle, rng, rows, cols, mean_nnz, bits, policy, empty_every=0):
    """A random quantized CSR in the reference container layout, packed by the oracle."""
    row_ptr, col_idx = random_csr(rng, rows, cols, mean_nnz, empty_every)
    qmax = (1 << bits) - 1
    scales = rng.uniform(0.05, 0.5, cols).astype(np.float32)
    offsets = rng.uniform(-0.5, 1.0, cols).astype(np.float32)
    row_offsets = rng.uniform(-1.0, 1.0, rows).astype(np.float32)
    codes = rng.integers(0, qmax + 1, len(col_idx))
    if policy == oracle.PER_GENE_AFFINE:
        values = (offsets[col_idx] + scales[col_idx] * codes).astype(np.float32)
    else:
        row_of = np.repeat(np.arange(rows), np.diff(row_ptr))
        values = (row_offsets[row_of] + scales[col_idx] * codes).astype(np.float32)
    packed_row_ptr = oracle.build_packed_row_ptr(bits, row_ptr)
    packed = oracle.pack_csr(bits, policy, row_ptr, packed_row_ptr, col_idx, values, scales,
                             offsets if policy == oracle.PER_GENE_AFFINE else None,
                             row_offsets if policy != oracle.PER_GENE_AFFINE else None)
    return dict(rows=rows, cols=cols, bits=bits, policy=policy, row_ptr=row_ptr,
                packed_row_ptr=packed_row_ptr, col_idx=col_idx, packed=packed, scales=scales,
                offsets=offsets if policy == oracle.PER_GENE_AFFINE else None,
                row_offsets=row_offsets if policy != oracle.PER_GENE_AFFINE else None)


def to_device_qcsr(fx: dict):
    import torch

    from cellerator_amd import QcsrMatrix

    def dev(a, dtype=None):
        if a is None:
            return None
        t = torch.from_numpy(np.ascontiguousarray(a))
        return t.to("cuda") if dtype is None else t.to(dtype).to("cuda")

    packed = np.concatenate([fx["packed"], np.zeros(16, np.uint8)])
    return QcsrMatrix(fx["rows"], fx["cols"], fx["bits"], dev(fx["row_ptr"]), dev(fx["col_idx"]),
                      packed_row_ptr=dev(fx["packed_row_ptr"]), packed_values=dev(packed),
                      column_scales=dev(fx["scales"]), column_offsets=dev(fx["offsets"]),
                      row_offsets=dev(fx["row_offsets"]), decode_policy=fx["policy"])


def qcsr_to_host(m) -> dict:
    """Downloads a device QcsrMatrix into the oracle's numpy form."""
    def host(t):
        return None if t is None else t.cpu().numpy()

    return dict(rows=m.rows, cols=m.cols, bits=m.bits, policy=m.decode_policy,
                row_ptr=host(m.row_ptr), packed_row_ptr=host(m.packed_row_ptr),
                col_idx=host(m.col_idx), packed=host(m.packed_values),
                scales=host(m.column_scales), offsets=host(m.column_offsets),
                row_offsets=host(m.row_offsets), values=host(m.values))


def check_against_referee(oracle, reference, magnitude, candidate, rel=REL_TOL,
                          abs_scaled=ABS_TOL_SCALED) -> dict:
    cmp = oracle.compare(reference, candidate, abs_scaled, rel, magnitude)
    assert cmp["status"] == 0, cmp
    assert cmp["within_tolerance"], cmp
    return cmp
