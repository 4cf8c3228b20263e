"""The device codec (qcsr_codec.hip) against the host restatement, as the reference's
quantized_matrix_test.cu:140-371 checks its own device pass: for every code width and
metadata policy, quantizing block by block on the device gives packed bytes identical to the
host pack (pack_row_values restated in the oracle), and dequantizing block by block gives the
host decode bit for bit and the input within half a quantization step. Odd row lengths leave
sub-byte tails; empty rows and the interleaved-pairs metadata are covered."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import random_csr
from tests.test_codec import uniform_blocks

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("policy", [1, 2, 3])
def test_device_codec_matches_host(oracle, bits, policy):
    import torch

    from cellerator_amd import QcsrMatrix
    from cellerator_amd.codec import dequantize, get_block, quantize
    rng = np.random.default_rng(100 * bits + policy)
    rows, cols = 333, 700
    row_ptr, col_idx = random_csr(rng, rows, cols, 37.3, empty_every=11)
    prp = oracle.build_packed_row_ptr(bits, row_ptr)
    qmax = (1 << bits) - 1
    scales = rng.uniform(0.05, 0.5, cols).astype(np.float32)
    scales[5] = 0.0  # a zero scale encodes every value as code 0
    offsets = rng.uniform(-0.5, 1.0, cols).astype(np.float32)
    row_offsets = rng.uniform(-1.0, 1.0, rows).astype(np.float32)
    row_of = np.repeat(np.arange(rows), np.diff(row_ptr))
    base = row_offsets[row_of] if policy == 2 else offsets[col_idx]
    # values around the representable range, including below 0 and above qmax codes
    values = (base + scales[col_idx] * rng.uniform(-1.0, qmax + 1.0, len(col_idx))).astype(np.float32)
    host_policy = 2 if policy == 2 else 1
    want_packed = oracle.pack_csr(bits, host_policy, row_ptr, prp, col_idx, values, scales,
                                  offsets if host_policy == 1 else None, row_offsets if host_policy == 2 else None)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    col_scales = dev(np.stack([scales, offsets], 1).reshape(-1)) if policy == 3 else dev(scales)
    packed = torch.zeros(int(prp[-1]) + 16, dtype=torch.uint8, device="cuda")
    m = QcsrMatrix(rows, cols, bits, dev(row_ptr), dev(col_idx), packed_row_ptr=dev(prp), packed_values=packed,
                   column_scales=col_scales, column_offsets=dev(offsets) if policy == 1 else None,
                   row_offsets=dev(row_offsets) if policy == 2 else None, decode_policy=policy)
    brp = uniform_blocks(rows, 29)
    vals_dev = dev(values)
    for k in range(len(brp) - 1):
        b = get_block(brp, row_ptr, prp, k)
        quantize(m, vals_dev[b.nnz_begin:].contiguous() if b.nnz_begin < len(values) else vals_dev, block=b)
    torch.cuda.synchronize()
    got = packed[:int(prp[-1])].cpu().numpy()
    assert np.array_equal(got, want_packed)
    assert not packed[int(prp[-1]):].any()  # nothing past the last row's bytes
    out = torch.full((len(values),), float("nan"), device="cuda")
    for k in range(len(brp) - 1):
        b = get_block(brp, row_ptr, prp, k)
        dequantize(m, out[b.nnz_begin:], block=b)
    torch.cuda.synchronize()
    decoded = out.cpu().numpy()
    want = oracle.decode_csr(bits, host_policy, row_ptr, prp, col_idx, want_packed, scales,
                             offsets if host_policy == 1 else None, row_offsets if host_policy == 2 else None)
    assert np.array_equal(decoded.view(np.uint32), want.view(np.uint32))
    # round trip: inside the code range the decoded value is within half a step
    q = (values - base) / np.where(scales[col_idx] == 0, 1, scales[col_idx])
    inside = (q >= 0) & (q <= qmax) & (scales[col_idx] != 0)
    step = scales[col_idx][inside]
    assert np.all(np.abs(decoded[inside] - values[inside])
                  <= 0.5 * step * (1 + 1e-5) + 2e-6 * np.abs(values[inside]) + 1e-6)


def test_whole_matrix_pass_and_rejections(oracle):
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd.codec import CxQcsrBlock, dequantize, quantize
    from tests.helpers import quantized_fixture, to_device_qcsr
    rng = np.random.default_rng(3)
    fx = quantized_fixture(oracle, rng, 500, 300, 25.0, 4, 1, empty_every=7)
    m = to_device_qcsr(fx)
    vals = dequantize(m)
    fresh = torch.zeros_like(m.packed_values)
    quantize(m, vals.contiguous(), packed_out=fresh)
    torch.cuda.synchronize()
    assert torch.equal(fresh[:len(fx["packed"])].cpu(), torch.from_numpy(fx["packed"]))
    bad = CxQcsrBlock(0, 10, 501, 0, 0, 0, 0, 0)
    with pytest.raises(N.EngineError, match="outside the matrix"):
        dequantize(m, block=bad)
