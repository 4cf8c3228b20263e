"""GPU parity of the prepared tail stream (qcsr_stream.hip) and the walk that reads it
(qcsr_spmm_stream in qcsr_parts.hip): the slot rows, fill index and entries are bit-exact
against a numpy restatement of the stream's definition (rows sorted by tail length over the
whole matrix, sets of 8 adjacent rows dealt round-robin to the blocks, each block's sets
heaviest first to the least-loaded wave, per-part fills of 16 steps x 8 groups stored in
(block, wave, part, layer) order, parity order within each run,
pads of the parity opposite to the paired group's entry), and the product through the stream
-- every code width and decode policy, with and without a dense head, N = 64 and 128, fused
epilogues, empty rows, rows longer than a part, ragged last block -- matches the float64
referee of the canonical matrix; repeats are bitwise equal. Rows that break the
sorted-columns promise are rejected when the stream is planned."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee, qcsr_to_host, to_device_qcsr
from tests.test_hybrid_gpu import _exec, _head_metadata, _referee, _skewed

pytestmark = pytest.mark.gpu

WAVES, PART = 16, 1024


def _round_blocks(rows, units):
    """The planner's block count: the fewest blocks of at most 1,024 rows, or, when those would
    not fill one round of `units` (one block per compute unit), `units` blocks capped at one
    set of 8 rows per block."""
    need = -(-rows // 1024)
    return need if need >= units else min(units, -(-rows // 8))


def _units(monkeypatch, units):
    """Blocks per round for the next plan: the device's compute units (None) or an override."""
    import torch
    if units is None:
        monkeypatch.delenv("CX_BLOCKS_PER_ROUND", raising=False)
        return torch.cuda.get_device_properties(0).multi_processor_count
    monkeypatch.setenv("CX_BLOCKS_PER_ROUND", str(units))
    return units


def _stream_reference(h, head_end, head, bits, LAYERS, blocks):
    """slot_rows, fill_index and entries of the stream by its definition (16 waves of LAYERS
    layers of 8 rows per block, `blocks` blocks)."""
    ROWS_PER_BLOCK = WAVES * LAYERS * 8
    SLOTS = WAVES * LAYERS
    rows = len(h["row_ptr"]) - 1
    cols = int(h["cols"])
    first = head // PART
    parts = (cols + PART - 1) // PART - first
    wide = bits == 8
    slot_rows = np.full((blocks, ROWS_PER_BLOCK), 0xFFFFFFFF, np.uint32)
    runs = {}  # (block, part, slot) -> list of (local gene, code) in stored order
    counts = np.zeros(blocks * parts * SLOTS + 1, np.int64)
    lasts = np.zeros(blocks * parts * SLOTS, np.int64)

    def pos(b, p, ls):  # (block, wave, part, layer) order
        return ((b * WAVES + ls // LAYERS) * parts + p) * LAYERS + ls % LAYERS

    # rows by tail length over the whole matrix (descending; saturated at 2^24 - 1; ties by row);
    # sets of 8 adjacent rows dealt round-robin to the blocks
    tail_len = np.array([int(h["row_ptr"][r + 1]) - int(head_end[r]) for r in range(rows)], np.int64)
    by_length = np.argsort((1 << 24) - 1 - np.clip(tail_len, 0, (1 << 24) - 1), kind="stable")
    for b in range(blocks):
        lens = np.full(ROWS_PER_BLOCK, -1, np.int64)
        block_rows = np.full(ROWS_PER_BLOCK, rows, np.int64)
        for t in range(ROWS_PER_BLOCK):
            at = ((t // 8) * blocks + b) * 8 + t % 8
            if at < rows:
                block_rows[t] = by_length[at]
                lens[t] = tail_len[block_rows[t]]
        order = sorted(range(ROWS_PER_BLOCK), key=lambda t: (-lens[t], t))
        # sets (ranks 8s .. 8s + 7) heaviest first to the least-loaded wave with a layer left
        load, used, set_slot = [0] * WAVES, [0] * WAVES, []
        for st in range(SLOTS):
            sl = sum(max(int(lens[t]), 0) for t in order[st * 8:st * 8 + 8])
            w = min((wv for wv in range(WAVES) if used[wv] < LAYERS), key=lambda wv: (load[wv], wv))
            set_slot.append(w * LAYERS + used[w])
            used[w] += 1
            load[w] += sl
        for rank, t in enumerate(order):
            r = int(block_rows[t])
            slot_rows[b, set_slot[rank // 8] * 8 + rank % 8] = r if r < rows else 0xFFFFFFFF
        for slot in range(ROWS_PER_BLOCK):
            r = int(slot_rows[b, slot])
            if r == 0xFFFFFFFF:
                continue
            rb, re = int(h["row_ptr"][r]), int(h["row_ptr"][r + 1])
            pbit = int(h["packed_row_ptr"][r]) * 8
            for e in range(int(head_end[r]), re):
                gene = int(h["col_idx"][e])
                bit = pbit + (e - rb) * bits
                code = (int(h["packed"][bit >> 3]) >> (bit & 7)) & ((1 << bits) - 1)
                runs.setdefault((b, gene // PART - first, slot), []).append((gene % PART, code))
        for p in range(parts):
            for ls in range(SLOTS):
                m = 0
                for g in range(8):
                    run = runs.get((b, p, ls * 8 + g), [])
                    pref = g & 1
                    run.sort(key=lambda x: 0 if (x[0] & 1) == pref else 1)  # stable: gene order within a parity
                    m = max(m, len(run))
                k = pos(b, p, ls)
                counts[k] = (m + 15) // 16
                lasts[k] = 0 if m == 0 else m - 16 * (counts[k] - 1)
    starts = np.zeros_like(counts)
    starts[1:] = np.cumsum(counts)[:-1]
    index = starts.astype(np.uint64)
    index[:-1] |= np.where(lasts > 0, (lasts - 1) << 28, 0).astype(np.uint64)
    total = int(starts[-1])
    pad = 1024
    entries = np.full((total, 128), pad, np.uint32 if wide else np.uint16)
    for (b, p, slot), run in runs.items():
        ls, g = divmod(slot, 8)
        f0 = int(starts[pos(b, p, ls)])
        for k, (gene, code) in enumerate(run):
            entries[f0 + k // 16, g * 16 + k % 16] = gene | (code << (16 if wide else 11))
    # a pad beside a stored entry of the paired group (2i, 2i + 1) at the same step takes the
    # opposite parity: gene 1024 (even) or 1025 (odd)
    gene_mask = 0xFFFF if wide else 0x7FF
    e = entries.reshape(total, 4, 2, 16).astype(np.int64)  # [fill, pair, group of pair, step]
    pad = (e & gene_mask) >= 1024
    for side in (0, 1):
        other = e[:, :, 1 - side, :]
        fix = pad[:, :, side, :] & ~pad[:, :, 1 - side, :]
        e[:, :, side, :] = np.where(fix, np.where((other & 1) == 1, 1024, 1025), e[:, :, side, :])
    entries = e.reshape(total, 128).astype(entries.dtype)
    return slot_rows, index.astype(np.uint32), entries


@pytest.mark.parametrize("units", [None, 1])
@pytest.mark.parametrize("bits,head", [(4, 1024), (8, 0), (2, 2048)])
def test_stream_layout_is_bit_exact(oracle, monkeypatch, bits, head, units):
    """Bit-exact layout under both block geometries: one block per compute unit of the device
    (2,100 rows: blocks of ~8 rows) and, with one block per round, the fewest full blocks
    (two of 1,024 rows and a ragged one)."""
    import torch

    from cellerator_amd.exec_order import hybrid_prepare, tail_arrays
    rng = np.random.default_rng(40 + bits + head)
    fx = _skewed(oracle, rng, 2100, 3100, bits, 1)
    mx, _ = _exec(to_device_qcsr(fx), head)
    per_round = _units(monkeypatch, units)
    p = hybrid_prepare(mx, head, stream_tail=True)
    torch.cuda.synchronize()
    assert int(p.tail.blocks) == _round_blocks(2100, per_round)
    slot_rows, index, entries = tail_arrays(p)
    h = qcsr_to_host(mx)
    from cellerator_amd.exec_order import hybrid_head_arrays
    he = hybrid_head_arrays(p)[2].cpu().numpy()
    want_rows, want_index, want_entries = _stream_reference(h, he, head, bits, int(p.tail.layers), int(p.tail.blocks))
    assert int(p.tail.block_rows) == WAVES * int(p.tail.layers) * 8
    assert np.array_equal(slot_rows.cpu().numpy().view(np.uint32), want_rows)
    assert np.array_equal(index.cpu().numpy().view(np.uint32), want_index)
    got = entries.cpu().numpy().view(np.uint32 if bits == 8 else np.uint16)
    assert got.shape == want_entries.shape
    assert np.array_equal(got, want_entries)
    assert int(p.tail.fills) == want_entries.shape[0]


@pytest.mark.parametrize("bits,policy,head", [(4, 1, 2048), (4, 1, 0), (8, 1, 1024), (2, 2, 2048), (1, 1, 1024),
                                              (4, 3, 2048), (8, 3, 0)])
def test_stream_product_matches_referee(oracle, bits, policy, head):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(3000 + 10 * bits + policy + head)
    fx = _skewed(oracle, rng, 1300, 3100, bits, policy)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    mx, order = _exec(m, head)
    w = (rng.standard_normal((3100, 64)) * 0.02).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    p = hybrid_prepare(mx, head, stream_tail=True)
    y = hybrid_spmm(p, wx)
    y2 = hybrid_spmm(p, wx)
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, dict(fx, policy=1 if policy == 3 else policy), w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


def test_stream_epilogue_and_wide_outputs(oracle):
    import torch

    from cellerator_amd import Epilogue
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(77)
    fx = _skewed(oracle, rng, 900, 2500, 4, 1)
    mx, order = _exec(to_device_qcsr(fx), 1024)
    w = (rng.standard_normal((2500, 128)) * 0.02).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    bias = torch.from_numpy(rng.standard_normal(128).astype(np.float32)).cuda()
    c0 = torch.from_numpy(rng.standard_normal((900, 128)).astype(np.float32)).cuda()
    p = hybrid_prepare(mx, 1024, stream_tail=True)
    plain = hybrid_prepare(mx, 1024)
    y = c0.clone()
    hybrid_spmm(p, wx, out=y, epilogue=Epilogue(kind=5, alpha=0.5, beta=2.0, bias=bias, initial=y))
    base = hybrid_spmm(plain, wx)
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, fx, w)
    check_against_referee(oracle, ref, mag, base.cpu().numpy())
    want = np.maximum(0.5 * ref + 2.0 * c0.cpu().numpy() + bias.cpu().numpy(), 0.0)
    got = y.cpu().numpy()
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-4 * np.abs(want) + 1e-4 * mag)


def test_long_rows_and_unsorted_rows(oracle):
    """Rows longer than a part (several fills per layer) and a ragged last block; then a row
    that breaks the sorted promise in the tail is rejected by the planner."""
    import dataclasses

    import torch

    from cellerator_amd import _native as N
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm
    from tests.test_qcsr_parts_gpu import _rebuild
    from tests.helpers import quantized_fixture
    rng = np.random.default_rng(91)
    rows, cols = 530, 2048 + 700
    fx = _head_metadata(rng, quantized_fixture(oracle, rng, rows, cols, 5.0, 4, 1), 0.0)  # canonical order: a full head
    lengths = rng.integers(0, 40, rows)
    lengths[:20] = rng.integers(900, 1500, 20)  # dense rows: up to 1,500 entries, ~1,000 in one part
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.concatenate([np.sort(rng.choice(cols, n, replace=False)) for n in lengths]).astype(np.int32)
    fx = _rebuild(oracle, rng, fx, row_ptr.astype(np.int32), col_idx)
    m = dataclasses.replace(to_device_qcsr(fx), flags=N.QCSR_COLUMNS_SORTED)
    w = (rng.standard_normal((cols, 64)) * 0.02).astype(np.float16)
    p = hybrid_prepare(m, 1024, stream_tail=True)
    y = hybrid_spmm(p, torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, fx, w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    # swap two tail genes of a long row across a part boundary: still inside [head, cols),
    # but a gene of part 1 now follows one of part 2 (disorder inside a part leaves the
    # product unchanged and is not an error)
    bad = fx["col_idx"].copy()
    r = 3
    b, e = int(fx["row_ptr"][r]), int(fx["row_ptr"][r + 1])
    part1 = np.nonzero((bad[b:e] >= 1024) & (bad[b:e] < 2048))[0] + b
    part2 = np.nonzero(bad[b:e] >= 2048)[0] + b
    bad[part1[0]], bad[part2[0]] = bad[part2[0]], bad[part1[0]]
    mb = dataclasses.replace(m, col_idx=torch.from_numpy(bad).cuda())
    with pytest.raises(N.EngineError, match="not sorted"):
        hybrid_prepare(mb, 1024, stream_tail=True)


def test_prepare_and_launch_on_a_side_stream(oracle):
    """hybrid_prepare(..., stream=side) allocates the layouts on the side stream it fills them
    on, and launches on that stream give the default stream's product bitwise; the prepared
    projection object does the same."""
    import torch

    from cellerator_amd.exec_order import ExecProjection, hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(515)
    fx = _skewed(oracle, rng, 1400, 2600, 4, 1)
    m = to_device_qcsr(fx)
    mx, order = _exec(m, 1024)
    w = torch.from_numpy((rng.standard_normal((2600, 64)) * 0.02).astype(np.float16)).cuda()
    wx = pack_rows(order, w)
    base = hybrid_spmm(hybrid_prepare(mx, 1024, stream_tail=True), wx)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    p = hybrid_prepare(mx, 1024, stream=side, stream_tail=True)
    with torch.cuda.stream(side):
        y = torch.empty_like(base)
    hybrid_spmm(p, wx, out=y, stream=side)
    proj = ExecProjection(m, 1024, stream=side)
    with torch.cuda.stream(side):
        y2 = torch.empty_like(base)
    proj.spmm(w, out=y2, stream=side)
    side.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), base.view(torch.int32))
    assert torch.equal(y2.view(torch.int32), base.view(torch.int32))


@pytest.mark.parametrize("units", [None, 1])
def test_stream_layout_33_parts_head_0(oracle, monkeypatch, units):
    """34,000 genes with no head: 34 gene parts, so the plan kernel counts parts in two chunks
    (32 + 2) and every row's tail starts at its first entry; layout bit-exact under both block
    geometries, product within the referee's tolerance."""
    import torch

    from cellerator_amd.exec_order import hybrid_head_arrays, hybrid_prepare, hybrid_spmm, pack_rows, tail_arrays
    rng = np.random.default_rng(3333)
    fx = _skewed(oracle, rng, 1100, 34_000, 4, 1)
    mx, order = _exec(to_device_qcsr(fx), 0)
    per_round = _units(monkeypatch, units)
    p = hybrid_prepare(mx, 0, stream_tail=True)
    torch.cuda.synchronize()
    assert int(p.tail.parts) == 34
    assert int(p.tail.blocks) == _round_blocks(1100, per_round)
    slot_rows, index, entries = tail_arrays(p)
    h = qcsr_to_host(mx)
    he = hybrid_head_arrays(p)[2].cpu().numpy()
    want_rows, want_index, want_entries = _stream_reference(h, he, 0, 4, int(p.tail.layers), int(p.tail.blocks))
    assert np.array_equal(slot_rows.cpu().numpy().view(np.uint32), want_rows)
    assert np.array_equal(index.cpu().numpy().view(np.uint32), want_index)
    assert np.array_equal(entries.cpu().numpy().view(np.uint16), want_entries)
    w = (rng.standard_normal((34_000, 64)) * 0.02).astype(np.float16)
    y = hybrid_spmm(p, pack_rows(order, torch.from_numpy(w).cuda()))
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, fx, w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
