"""GPU parity of the execution-order quantized CSR SpMM with a matrix-core head
(cx_qcsr_spmm_fwd_hybrid, qcsr_hybrid.hip): the dense head layout is bit-exact against a
numpy restatement of its definition (codes, presence bits, tail starts, 2^k-scaled
metadata), the head's three-part fp16 split reproduces every decoded value exactly (an
identity weight panel), and the product over random and C3-generated matrices -- every
code width and decode policy, N = 64 and 128, fused epilogues, ragged workgroups, empty
rows and rows wholly inside or outside the head -- matches the float64 referee of the
canonical matrix. Repeats are bitwise equal."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee, qcsr_to_host, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _exec(m, head):
    """The matrix in the execution order a prepared projection with a `head`-gene head uses
    (cx_qcsr_head_order: popularity order, genes the head cannot carry exactly after it); the
    fixtures here have enough such genes for the full head."""
    from cellerator_amd.exec_order import head_order, to_execution_order
    order, h = head_order(m, head)
    assert h == min(head, m.cols // 1024 * 1024), (h, head)
    return to_execution_order(m, order), order


def _head_metadata(rng, fx, hostile):
    """Metadata the head carries exactly for most genes: decoded values from about 0.5 to 8.5
    whatever the code width (offsets 0.5..1, scales 0.05..0.5 times 15 / qmax), or under the
    row-offset policy scales and row offsets on a 2^-12 grid. A fraction `hostile` of the
    genes gets values the head cannot always carry (offsets -0.5..1 with values crossing
    zero at 0.05..0.5 steps; unrounded scales of 0.001..0.01 under row offsets)."""
    cols, rows, qmax = fx["cols"], fx["rows"], (1 << fx["bits"]) - 1
    scales = rng.uniform(0.05, 0.5, cols) * 15.0 / qmax
    bad = rng.random(cols) < hostile
    if fx["policy"] == 2:
        scales = np.maximum(np.round(scales * 4096.0), 1.0) / 4096.0
        scales[bad] = rng.uniform(0.001, 0.01, int(bad.sum()))
        row_offsets = np.round(rng.uniform(-1.0, 1.0, rows) * 4096.0) / 4096.0
        return dict(fx, scales=scales.astype(np.float32), row_offsets=row_offsets.astype(np.float32))
    offsets = rng.uniform(0.5, 1.0, cols)
    scales[bad] = rng.uniform(0.05, 0.5, int(bad.sum()))
    offsets[bad] = rng.uniform(-0.5, 1.0, int(bad.sum()))
    return dict(fx, scales=scales.astype(np.float32), offsets=offsets.astype(np.float32))


def _skewed(oracle, rng, rows, cols, bits, policy, hostile=0.05):
    """Row lengths from 0 to all genes, genes drawn with a Zipf-like popularity so the
    popularity order has a dense head; metadata from _head_metadata."""
    fx = _head_metadata(rng, quantized_fixture(oracle, rng, rows, cols, 10.0, bits, 1 if policy == 3 else policy),
                        hostile)
    weight = 1.0 / np.arange(1, cols + 1) ** 1.1
    weight = weight[rng.permutation(cols)]
    lengths = np.minimum(rng.lognormal(np.log(250.0), 0.8, rows).astype(np.int64), cols)
    lengths[::29] = 0
    lengths[5] = cols
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.empty(int(row_ptr[-1]), np.int32)
    p = weight / weight.sum()
    for r in range(rows):
        if lengths[r]:
            col_idx[row_ptr[r]:row_ptr[r + 1]] = np.sort(rng.choice(cols, lengths[r], replace=False, p=p))
    from tests.test_qcsr_parts_gpu import _rebuild
    return _rebuild(oracle, rng, fx, row_ptr.astype(np.int32), col_idx)


def _referee(oracle, fx, w):
    return oracle.qcsr_spmm_referee(fx["bits"], fx["policy"], fx["rows"], fx["cols"], fx["row_ptr"],
                                    fx["packed_row_ptr"], fx["col_idx"], fx["packed"], fx["scales"],
                                    fx["offsets"], fx["row_offsets"], w)


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 1), (2, 2), (1, 1), (4, 3), (8, 3)])
def test_hybrid_matches_referee(oracle, bits, policy):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(2000 + 10 * bits + policy)
    fx = _skewed(oracle, rng, 700, 3100, bits, policy)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    mx, order = _exec(m, 2048)
    w = (rng.standard_normal((3100, 64)) * 0.02).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    p = hybrid_prepare(mx, 2048)
    y = hybrid_spmm(p, wx)
    y2 = hybrid_spmm(p, wx)
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, dict(fx, policy=1 if policy == 3 else policy), w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 1), (2, 2)])
def test_identity_panel_gives_exact_decoded_values(oracle, bits, policy):
    """W = the identity on execution genes 0..31 (head) and 1024..1055 (tail): Y[r, c] is the
    decoded value of (r, gene), through the head's three-part split or the tail's fp32 sum --
    bitwise for every value, the head carrying only genes it decodes exactly."""
    import torch

    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm
    rng = np.random.default_rng(5 + bits)
    fx = _skewed(oracle, rng, 600, 2100, bits, policy, hostile=0.2)
    mx, order = _exec(to_device_qcsr(fx), 1024)
    genes = np.concatenate([np.arange(32), 1024 + np.arange(32)])
    w = torch.zeros((2100, 64), dtype=torch.float16, device="cuda")
    w[torch.from_numpy(genes).cuda(), torch.arange(64, device="cuda")] = 1.0
    p = hybrid_prepare(mx, 1024)
    y = hybrid_spmm(p, w)
    torch.cuda.synchronize()
    h = qcsr_to_host(mx)
    decoded = oracle.decode_csr(bits, policy, h["row_ptr"], h["packed_row_ptr"], h["col_idx"], h["packed"],
                                h["scales"], h["offsets"], h["row_offsets"])
    want = np.zeros((600, 64), np.float32)
    rows = np.repeat(np.arange(600), np.diff(h["row_ptr"]))
    column = np.full(2100, -1)
    column[genes] = np.arange(64)
    sel = column[h["col_idx"]] >= 0
    want[rows[sel], column[h["col_idx"][sel]]] = decoded[sel]
    got = y.cpu().numpy()
    assert sel.sum() > 1000
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _layout_reference(h, head, rows_ld):
    """The dense head layout by its definition, from the host CSR (sorted rows)."""
    bits, rows = h["bits"], len(h["row_ptr"]) - 1
    per_word = 32 // bits
    codes = np.zeros((head * bits // 32, rows_ld), np.uint32)
    masks = np.zeros((head // 32, rows_ld), np.uint32)
    head_end = np.zeros(rows, np.int32)
    packed = h["packed"]
    for r in range(rows):
        b, e = int(h["row_ptr"][r]), int(h["row_ptr"][r + 1])
        pbit = int(h["packed_row_ptr"][r]) * 8
        i = b
        while i < e and h["col_idx"][i] < head:
            g = int(h["col_idx"][i])
            bit = pbit + (i - b) * bits
            code = (int(packed[bit >> 3]) >> (bit & 7)) & ((1 << bits) - 1)
            codes[g // per_word, r] |= np.uint32(code << ((g % per_word) * bits))
            masks[g // 32, r] |= np.uint32(1 << (g % 32))
            i += 1
        head_end[r] = i
    return codes, masks, head_end


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 3), (2, 2), (1, 1)])
def test_dense_head_layout_is_bit_exact(oracle, bits, policy):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_head_arrays, hybrid_prepare
    rng = np.random.default_rng(700 + bits)
    fx = _skewed(oracle, rng, 300, 2500, bits, policy)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    mx, _ = _exec(m, 2048)
    p = hybrid_prepare(mx, 2048)
    first, second, head_end, meta = hybrid_head_arrays(p)
    torch.cuda.synchronize()
    h = qcsr_to_host(mx)
    want_codes, want_masks, want_end = _layout_reference(h, 2048, int(p.layout.rows_ld))
    table = bits <= 4 and policy != 2
    assert p.layout.head_form == (2 if table else 1)
    if table:
        # code bytes: code * 8 where stored, 128 elsewhere (the same codes and presence as the words)
        per_word = 32 // bits
        g = np.arange(2048)
        codes = (want_codes[g // per_word, :] >> ((g % per_word) * bits)[:, None]) & ((1 << bits) - 1)
        present = (want_masks[g // 32, :] >> (g % 32)[:, None]) & 1
        want_bytes = np.where(present == 1, codes * 8, 128).astype(np.uint8)  # [gene, rows_ld]
        got_bytes = first.cpu().numpy()  # [chunk, rows_ld, 32]
        assert np.array_equal(got_bytes.transpose(0, 2, 1).reshape(2048, -1), want_bytes)
    else:
        assert np.array_equal(first.cpu().numpy().view(np.uint32), want_codes)
        assert np.array_equal(second.cpu().numpy().view(np.uint32), want_masks)
    assert np.array_equal(head_end.cpu().numpy(), want_end)
    # scale exponent and metadata: k = 14 - floor(log2 B), B = largest |decoded value| of a head code
    if policy == 3:
        pairs = h["scales"].reshape(-1, 2)
        s, o = pairs[:2048, 0].astype(np.float64), pairs[:2048, 1].astype(np.float64)
    else:
        s = h["scales"][:2048].astype(np.float64)
        o = h["offsets"][:2048].astype(np.float64) if policy == 1 else np.zeros(2048)
    qmax = (1 << bits) - 1
    if policy == 2:
        bound = np.float32(np.max(np.abs(s) * qmax)) + np.float32(np.max(np.abs(h["row_offsets"])))
    else:
        bound = np.max(np.maximum(np.abs(o), np.abs(o + qmax * s)))
    k = 14 - int(np.floor(np.log2(bound)))
    assert p.scale_exp == k
    got_meta = meta.cpu().numpy()
    assert np.array_equal(got_meta[:, 0], (s * 2.0 ** k).astype(np.float32))
    if policy != 2:
        assert np.array_equal(got_meta[:, 1], (o * 2.0 ** k).astype(np.float32))
    if table:
        # the value table: three round-toward-zero fp16 parts of fma(code, 2^k s, 2^k o) in
        # float32, summing back to it exactly wherever the last part is normal; entry 16 zero
        lut = second.cpu().numpy().view(np.float16).astype(np.float32)  # [gene, 17, 4]
        sk, ok = got_meta[:, 0], got_meta[:, 1]
        x = np.arange(16, dtype=np.float64)[None, :] * sk[:, None].astype(np.float64) + ok[:, None].astype(np.float64)
        x32 = x.astype(np.float32)  # one rounding: the fp32 fma (the product is exact in fp64)
        # rtz to fp16 by truncating the float32 to 11 significant bits (values < 2^15 here)

        def rtz16(v):
            v = v.astype(np.float32)
            bits_ = v.view(np.uint32)
            e = ((bits_ >> 23) & 0xFF).astype(np.int64) - 127
            drop = np.clip(13 + np.maximum(0, -14 - e), 0, 23)  # fp16 subnormals keep fewer bits
            keep = np.where(e < -24, 0, ~((np.uint32(1) << drop.astype(np.uint32)) - np.uint32(1)))
            return (bits_ & keep.astype(np.uint32)).view(np.float32)

        hi = rtz16(x32)
        mid = rtz16(x32 - hi)
        lo = rtz16((x32 - hi) - mid)
        n = qmax + 1  # codes the width can hold; the other entries are zero
        assert np.array_equal(lut[:, :n, 0], hi[:, :n]) and np.array_equal(lut[:, :n, 1], mid[:, :n])
        assert np.array_equal(lut[:, :n, 2], lo[:, :n])
        assert np.all(lut[:, n:, :] == 0) and np.all(lut[:, :, 3] == 0)
        # the head holds only genes whose every value splits exactly
        assert np.array_equal((hi + mid + lo)[:, :n], x32[:, :n])


@pytest.mark.parametrize("n,kind,beta", [(128, 0, 0.0), (64, 6, 0.5), (128, 2, -1.0)])
def test_hybrid_epilogue_and_wide_outputs(oracle, n, kind, beta):
    import torch

    from cellerator_amd import Epilogue
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(3000 + n + kind)
    fx = _skewed(oracle, rng, 530, 2200, 4, 1)
    mx, order = _exec(to_device_qcsr(fx), 2048)
    w = (rng.standard_normal((2200, n)) * 0.05).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    bias = (rng.standard_normal(n) * 0.3).astype(np.float32)
    c0 = rng.standard_normal((530, n)).astype(np.float32)
    y = torch.from_numpy(c0.copy()).cuda()
    ep = Epilogue(kind, 1.5, beta, torch.from_numpy(bias).cuda() if kind in (1, 5, 6, 7) else None,
                  y if beta != 0.0 else None)
    hybrid_spmm(hybrid_prepare(mx, 2048), wx, out=y, epilogue=ep)
    torch.cuda.synchronize()
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    ref = oracle.spmm_referee(530, 2200, n, fx["row_ptr"], fx["col_idx"], decoded, w, alpha=1.5, beta=beta,
                              c0=c0 if beta else None, epilogue=kind,
                              bias=bias if kind in (1, 5, 6, 7) else None)
    mag = oracle.spmm_referee(530, 2200, n, fx["row_ptr"], fx["col_idx"], np.abs(decoded.astype(np.float64)),
                              np.abs(w.astype(np.float64)))
    check_against_referee(oracle, ref, 1.5 * mag + np.abs(beta * c0), y.cpu().numpy())


def test_hybrid_on_c3_rows(oracle):
    """C3-generated rows (4-bit, 33,538 genes, Zipf popularity) in popularity order with a
    4,096-gene head, several workgroups of 256 rows and a ragged last one."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(5 * 256 + 61))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=3)
    mx, order = _exec(qcsr_pack_gene_affine(m), 4096)
    wx = pack_rows(order, w)
    y = hybrid_spmm(hybrid_prepare(mx, 4096), wx)
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(4, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"], h["col_idx"],
                                        h["packed"], h["scales"], h["offsets"], None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


@pytest.mark.parametrize("head", [3072, 6144])
def test_hybrid_on_c2_rows(oracle, head):
    """C2-generated rows (8-bit codes, 20,000 genes, 2,000 nonzeros per cell) in popularity
    order with the 3,072-gene head bench.py runs at C2 (and 6,144; the words form), several
    workgroups of 256 rows and a ragged last one; repeats are bitwise equal."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    from cellerator_amd.synth import C2, dense_normal, generate_qcsr
    m = generate_qcsr(C2.scaled(3 * 256 + 37))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=5)
    mx, order = _exec(qcsr_pack_gene_affine(m), head)
    wx = pack_rows(order, w)
    p = hybrid_prepare(mx, head)
    y = hybrid_spmm(p, wx)
    y2 = hybrid_spmm(p, wx)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(8, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"], h["col_idx"],
                                        h["packed"], h["scales"], h["offsets"], None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


def test_hybrid_rejects_unsorted_rows_and_bad_metadata(oracle):
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm
    rng = np.random.default_rng(9)
    fx = _skewed(oracle, rng, 300, 2100, 4, 1, hostile=0.0)
    m = to_device_qcsr(fx)  # canonical order, flags 0
    with pytest.raises(N.EngineError, match="sorted"):
        hybrid_prepare(m, 1024)
    m.flags = N.QCSR_COLUMNS_SORTED
    with pytest.raises(N.EngineError, match="1,024"):
        hybrid_prepare(m, 1000)
    # a promise the rows break: two entries of row 7 swapped
    bad = dict(fx)
    col = fx["col_idx"].copy()
    b = int(fx["row_ptr"][7])
    assert fx["row_ptr"][8] - b >= 2
    col[b], col[b + 1] = col[b + 1], col[b]
    mb = to_device_qcsr(dict(bad, col_idx=col))
    mb.flags = N.QCSR_COLUMNS_SORTED
    with pytest.raises(N.EngineError, match="strictly increasing"):
        hybrid_prepare(mb, 1024)
    nan_meta = fx["scales"].copy()
    nan_meta[3] = np.nan
    mn = to_device_qcsr(dict(fx, scales=nan_meta))
    mn.flags = N.QCSR_COLUMNS_SORTED
    with pytest.raises(N.EngineError, match="finite"):
        hybrid_prepare(mn, 1024)
    # a layout used with another matrix
    p = hybrid_prepare(m, 1024)
    other = to_device_qcsr(_skewed(oracle, np.random.default_rng(10), 301, 2100, 4, 1, hostile=0.0))
    other.flags = N.QCSR_COLUMNS_SORTED
    w = torch.zeros((2100, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(N.EngineError, match="not prepared for this matrix"):
        hybrid_spmm(dataclasses_replace(p, matrix=other), w)


def dataclasses_replace(obj, **kw):
    import dataclasses
    return dataclasses.replace(obj, **kw)


def test_head_refuses_values_it_cannot_carry(oracle):
    """cx_qcsr_hybrid_prepare checks every value the head can decode: a head gene with a wide
    range (scale 1,000: the layout scale drops, and the other genes' values fall off the 2^-14
    grid) or with values near zero (offset and steps of 0.01) is refused, naming the
    gene; under the row-offset policy a row offset off the grid is refused, naming the row.
    The same genes placed after the head (cx_qcsr_head_order) are accepted."""
    from cellerator_amd import _native as N
    from cellerator_amd.exec_order import hybrid_prepare
    from tests.test_qcsr_parts_gpu import _rebuild
    rng = np.random.default_rng(19)
    fx = _skewed(oracle, rng, 300, 2100, 4, 1, hostile=0.0)

    def sorted_dev(f):
        m = to_device_qcsr(f)
        m.flags = N.QCSR_COLUMNS_SORTED
        return m

    assert hybrid_prepare(sorted_dev(fx), 1024).head_cols == 1024
    for gene, scale, offset in ((3, 1000.0, 0.5), (700, 0.01, 0.01)):
        s_, o_ = fx["scales"].copy(), fx["offsets"].copy()
        s_[gene], o_[gene] = scale, offset
        f = _rebuild(oracle, rng, dict(fx, scales=s_, offsets=o_), fx["row_ptr"], fx["col_idx"])
        with pytest.raises(N.EngineError, match="does not decode exactly") as err:
            hybrid_prepare(sorted_dev(f), 1024)
        assert err.value.status == 3  # CX_STATUS_UNSUPPORTED
        if gene == 700:
            assert "head gene 700 " in str(err.value)
        mx, _ = _exec(sorted_dev(f), 1024)  # the head order moves the gene behind the head
        assert hybrid_prepare(mx, 1024).head_cols == 1024
    fr = _skewed(oracle, rng, 300, 2100, 2, 2, hostile=0.0)
    assert hybrid_prepare(sorted_dev(fr), 1024).head_cols == 1024
    r_ = fr["row_offsets"].copy()
    r_[17] = np.float32(0.01)
    f = _rebuild(oracle, rng, dict(fr, row_offsets=r_), fr["row_ptr"], fr["col_idx"])
    with pytest.raises(N.EngineError, match="offset of row 17 "):
        hybrid_prepare(sorted_dev(f), 1024)


def test_words_head_gene_parts(oracle, monkeypatch):
    """A words-form head over fewer rows than four 64-row waves per SIMD splits its genes into
    up to three parts, one partial each (the workspace holds them all), summed in order by the
    tail; with the device counted as one CU (CX_BLOCKS_PER_ROUND=1) the same matrix runs in
    one part. Both agree with the referee; repeats are bitwise equal."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    from cellerator_amd.synth import C2, dense_normal, generate_qcsr
    m = generate_qcsr(C2.scaled(2 * 256 + 11))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=9)
    mx, order = _exec(qcsr_pack_gene_affine(m), 3072)
    wx = pack_rows(order, w)
    partial = (m.rows * 256 + 255) // 256 * 256
    panel = (3072 * 64 * 2 + 255) // 256 * 256
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(8, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"], h["col_idx"],
                                        h["packed"], h["scales"], h["offsets"], None, w.cpu().numpy())
    outs = []
    for units, parts in ((None, 3), ("1", 1)):
        if units is not None:
            monkeypatch.setenv("CX_BLOCKS_PER_ROUND", units)
        p = hybrid_prepare(mx, 3072)
        assert p.workspace(64, "cuda").numel() == parts * partial + panel
        y = hybrid_spmm(p, wx)
        y2 = hybrid_spmm(p, wx)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
        check_against_referee(oracle, ref, mag, y.cpu().numpy())
        outs.append(y)
    # the two split the head's sum differently: they differ by fp32 reordering only
    diff = np.abs(outs[0].cpu().numpy().astype(np.float64) - outs[1].cpu().numpy())
    assert np.all(diff <= 2.0 ** -20 * mag)
