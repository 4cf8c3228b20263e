#!/usr/bin/env python3
"""Headline benchmark: quantized CSR SpMM on one MI355X.

Default workload = BASELINE.json configs[2] (the metric's "1M cells, N=64"): 4-bit packed
quantized CSR, 1,000,000 cells x 33,538 genes, row nnz ~ LogNormal(mean 1,500, sigma 0.6),
Zipf(1.1) gene popularity, per-gene scale/offset, fp16 W 33,538 x 64 ~ N(0, 0.02), fp32 Y.
Inputs are generated seeded on the GPU and are resident in HBM before timing starts.

One step = one launch of the prepared execution-order path over the whole matrix
(cx_qcsr_exec_spmm, what the CP-Math execution-order candidate runs: canonical W gathered into
execution order, the 2,048 most stored genes on the matrix cores (3,072 for c2), the rest through
the prepared tail stream; the projection is prepared once, untimed), with the canonical
cx_qcsr_spmm_fwd kernel timed beside it (--canonical makes it the headline).
Prints ONE JSON line: metric/value (nnz/s), ms_per_step, roofline of the kernels
(achieved algorithmic GB/s from HIP events on the launch stream vs 8 TB/s), and the CPU
baseline (the oracle's row-parallel fp32 restatement timed on this host).

Other configs: c2, c3n128 (the same path), c4 (Blocked-ELL on the matrix cores; block-major
values copied once before timing, the row-major values timed beside them; --row-major for
those alone), c4q (C4's block structure with 8-bit per-gene affine codes and f32 W, the
reference's quantized Blocked-ELL projection), c5 (CP-BP warp-tile reduction).

  python bench.py [--steps K] [--warmup W] [--config c3|c3n128|c2|c4|c4q|c5] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_FP32_PEAK_TFLOPS = 157.3  # fp32 dense matrix cores
# Matrix-core head width of the prepared qCSR path per configuration, from sweeps in steps of
# 1,024 genes: at C3 2,048 (3,072 and 4,096 slower); at C2 3,072 (2,048 and 4,096 within 4%,
# 6,144 13% slower), with C2's 100k rows spread over every compute unit in the tail walk.
HEAD_GENES = {"c3": 2048, "c3n128": 2048, "c2": 3072}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cores() -> int:
    """Threads for the CPU baselines: every core this process may run on, within the host's
    CPU share for one GPU when the environment states it (OMP_NUM_THREADS)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n)


def host_description() -> dict:
    """What the CPU baseline ran on: nproc, the affinity mask (as CPU ranges) and the model."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except AttributeError:
        cpus = list(range(os.cpu_count() or 1))
    ranges, start = [], None
    for i, c in enumerate(cpus):
        if start is None:
            start = c
        if i + 1 == len(cpus) or cpus[i + 1] != c + 1:
            ranges.append(f"{start}-{c}" if c != start else str(start))
            start = None
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": ",".join(ranges), "affinity_cpus": len(cpus),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "threads_used": host_cores(),
            "cpu_model": model}


def time_launches(torch, launch, steps: int, warmup: int, stream):
    """Runs `launch` warmup + steps times on `stream`; returns (wall ms/step, event ms list)."""
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        launch()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ev = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return wall_ms, ev


def cpu_baseline_qcsr(m, w, out, sample_rows: int, threads: int) -> tuple[dict, dict]:
    """Times the oracle's row-parallel fp32 restatement on the first `sample_rows` rows, then
    (untimed) checks the GPU's timed output on those rows against it: the CPU product and
    its magnitude Sigma |x||w| give |gpu - cpu| <= 1e-4 + 1e-4 |cpu| + 2^-20 Sigma |x||w|
    per element (both fp32, only the summation order differs)."""
    import numpy as np

    from oracle import pyoracle

    pyoracle.build()
    rows = min(sample_rows, m.rows)
    # download only the sampled rows' slices
    rp = m.row_ptr[: rows + 1].cpu().numpy()
    nnz = int(rp[-1])
    prp = m.packed_row_ptr[: rows + 1].cpu().numpy()
    cols = m.col_idx[:nnz].cpu().numpy()
    packed = m.packed_values[: int(prp[-1]) + 16].cpu().numpy()
    scales = m.column_scales.cpu().numpy()
    offsets = m.column_offsets.cpu().numpy()
    wn = w.cpu().numpy()
    args = (m.bits, m.decode_policy, rows, m.cols, rp, prp, cols, packed, scales, offsets, None, wn)
    cpu_out = pyoracle.qcsr_spmm_f32_mt(*args, threads=threads)  # warm caches / page-in
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cpu_out = pyoracle.qcsr_spmm_f32_mt(*args, threads=threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    base = {"value": nnz / t, "unit": "nnz/s", "cores": threads, "kind": "port",
            "sample": f"first {rows} of {m.rows} rows ({nnz} nnz), median of 3 after 1 warmup; "
                      f"oracle or_qcsr_spmm_f32_mt (decode + fp32 FMA, AVX2, row-parallel)",
            "seconds": t, "host": host_description()}
    mag = pyoracle.qcsr_spmm_f32_mt(*args, threads=threads, magnitude=True)
    return base, (rows, cpu_out, mag)


def full_output_check(out, cpu) -> dict:
    """The GPU's timed output against the CPU product on the CPU leg's rows: both fp32, only
    the summation order differs, so |gpu - cpu| <= 1e-4 + 1e-4 |cpu| + 2^-20 Sigma |x||w|."""
    import numpy as np

    rows, cpu_out, mag = cpu
    got = out[:rows].cpu().numpy()
    err = np.abs(got.astype(np.float64) - cpu_out)
    bound = 1e-4 + 1e-4 * np.abs(cpu_out) + 2.0 ** -20 * mag
    return {"rows": rows, "elements": int(got.size), "mismatches": int((err > bound).sum()),
            "max_abs_err": float(err.max()) if got.size else 0.0,
            "rule": "|gpu - cpu_fp32| <= 1e-4 + 1e-4 |cpu| + 2^-20 sum |x||w|"}


def bench_qcsr(args, torch, cfg, n_out: int) -> dict:
    """C2 / C3. The headline is the prepared execution-order path (cx_qcsr_spmm_fwd_hybrid
    with a dense head and the prepared tail stream), built once per structure (untimed,
    reported as prepare_ms); the canonical row-group kernel on the unprepared CSR is timed
    beside it (`canonical_kernel`), and --canonical makes it the headline."""
    from cellerator_amd import _native as N
    from cellerator_amd import qcsr_check_columns, qcsr_pack_gene_affine, qcsr_spmm
    from cellerator_amd.synth import dense_normal, generate_qcsr

    t0 = time.perf_counter()
    m = generate_qcsr(cfg)
    w = dense_normal((m.cols, n_out), 0.02, torch.float16, seed=cfg.seed + n_out)
    out = torch.empty((m.rows, n_out), dtype=torch.float32, device="cuda")
    # per-gene (scale, offset) interleaved once per metadata generation (untimed, like a
    # packed weight panel); decodes bit-identically to the separate arrays
    pairs = bool(m.bits) and m.decode_policy == N.DECODE_PER_GENE_AFFINE and not args.separate_meta
    mt = qcsr_pack_gene_affine(m) if pairs else m
    # the structure's column order checked once on the device (untimed prepare step): sorted
    # rows let the gene-part kernel skip its per-entry out-of-order check
    if not args.unchecked_columns:
        mt = qcsr_check_columns(mt)
    torch.cuda.synchronize()
    log(f"generated {cfg.name}: nnz={m.nnz} in {time.perf_counter() - t0:.1f}s")
    stream = torch.cuda.current_stream()
    alg_bytes = m.nbytes_algorithmic(n_out, 2)
    flops = 2.0 * m.nnz * n_out

    def roofline(kern_ms: float, kernel: str, traffic_key: str) -> dict:
        achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": load_traffic(traffic_key), "kernel": kernel,
                "kernel_ms_mean": kern_ms, "algorithmic_bytes": alg_bytes,
                "fp32_fma_tflops": flops / (kern_ms * 1e-3) / 1e12, "valu_fp32_peak_tflops_nonpacked": 78.6}

    def launch():
        qcsr_spmm(mt, w, out=out, stream=stream)

    wall_ms, ev = time_launches(torch, launch, args.steps, args.warmup, stream)
    kernel = (("qcsr_spmm_groups" if m.bits and n_out % 64 == 0 and n_out <= 256 else "qcsr_spmm_rowwave")
              + ("<gene-affine pairs>" if pairs else ""))
    canonical = {"ms_per_step": wall_ms, "value": m.nnz / (wall_ms * 1e-3), "unit": "nnz/s",
                 "kernel_ms_median": statistics.median(ev),
                 "roofline": roofline(statistics.mean(ev), kernel, cfg.name)}
    log(f"canonical {kernel}: {wall_ms:.3f} ms/step")
    prepared = None
    if not args.canonical and args.head >= 0 and m.bits and n_out % 64 == 0 and n_out <= 256:
        prepared, prep_out = bench_qcsr_prepared(args, torch, mt, w, n_out, stream)
        prepared["roofline"] = roofline(prepared.pop("kernel_ms_mean"), prepared["kernels"],
                                        cfg.name + " prepared")
    head = prepared if prepared is not None else canonical
    res = {
        "metric": "quantized CSR SpMM nnz/s + effective HBM GB/s (% roofline), 1M cells, N=64",
        "value": head["value"],
        "unit": "nnz/s",
        "ms_per_step": head["ms_per_step"],
        "dtype": f"u{m.bits}-codes/f16-W/f32-accumulate" if m.bits else "f32",
        "config": {"workload": cfg.name, "rows": m.rows, "genes": m.cols, "nnz": m.nnz,
                   "bits": m.bits, "n_out": n_out, "rhs": "fp16",
                   "nnz_per_row_mean": m.nnz / m.rows, "seed": hex(cfg.seed),
                   "columns_sorted": bool(mt.flags & N.QCSR_COLUMNS_SORTED),
                   "path": ("prepared execution order: dense head + tail stream" if prepared is not None
                            else "canonical row-group kernel")},
        "roofline": head["roofline"],
    }
    if prepared is not None:
        res["prepared_path"] = {k: v for k, v in prepared.items() if k not in ("value", "ms_per_step", "roofline")}
    res["canonical_kernel"] = canonical
    if not args.no_cpu:
        res["cpu_baseline"], cpu = cpu_baseline_qcsr(m, w, out, args.cpu_rows, host_cores())
        canonical["full_output_check"] = full_output_check(out, cpu)
        res["full_output_check"] = (full_output_check(prep_out, cpu) if prepared is not None
                                    else canonical["full_output_check"])
    canonical["parity_sample"] = parity_sample_qcsr(m, w, out, 2000, seed=cfg.seed)
    res["parity_sample"] = (parity_sample_qcsr(m, w, prep_out, 2000, seed=cfg.seed) if prepared is not None
                            else canonical["parity_sample"])
    return res


def bench_qcsr_prepared(args, torch, mt, w, n_out: int, stream):
    """The same product on the prepared execution-order projection (cx_qcsr_exec_prepare /
    cx_qcsr_exec_spmm, the object behind the CP-Math execution-order candidate): genes in
    popularity order, the first --head genes as a dense code plane on the matrix cores, the
    rest from the prepared tail stream. Built once per structure (untimed, reported as
    prepare_ms); each launch takes the canonical W, gathers it into execution order in its
    workspace and runs the head and the tail; output rows are the same cells in the same
    order."""
    from cellerator_amd.exec_order import ExecProjection

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    proj = ExecProjection(mt, args.head)
    torch.cuda.synchronize()
    prep_ms = (time.perf_counter() - t0) * 1e3
    info = proj.info()
    out = torch.empty((mt.rows, n_out), dtype=torch.float32, device="cuda")

    def launch():
        proj.spmm(w, out=out, stream=stream)

    wall_ms, ev = time_launches(torch, launch, args.steps, args.warmup, stream)
    log(f"prepared head={info.head_cols} + tail stream: {wall_ms:.3f} ms/step (prepare {prep_ms:.0f} ms)")
    head_kernel = {1: "qcsr_head_dense", 2: "qcsr_head_lut"}.get(int(info.head_form), "qcsr_head")
    kernels = (f"pack_dense_operand (W into execution order) + pack_rhs_kernel + {head_kernel} (matrix cores, "
               f"genes < {info.head_cols}) + qcsr_spmm_stream (tail) per 64 columns")
    res = {"ms_per_step": wall_ms, "value": mt.nnz / (wall_ms * 1e-3), "unit": "nnz/s",
           "head_genes": int(info.head_cols), "kernel_ms_mean": statistics.mean(ev),
           "kernel_ms_median": statistics.median(ev), "kernels": kernels, "prepare_ms": prep_ms,
           "prepare": "cx_qcsr_exec_prepare: popularity order, execution-order relabel (temporary), metadata in "
                      "execution order, dense head layout, tail stream (global sort by tail length, plan, fill)",
           "persistent_bytes": int(info.persistent_bytes), "tail_fills": int(info.tail_fills)}
    return res, out


def parity_sample_qcsr(m, w, out, count: int, seed: int) -> dict:
    """The timed output against the oracle's float64 referee on a seeded sample of rows
    spread over the whole matrix, plus the first 64 rows and the last 600 (the last
    workgroup of 512 rows, whose windows reach the array ends), at the tests' tolerance
    (1e-4 + 1e-4 relative + 1e-4 sum |x||w|)."""
    import numpy as np

    from oracle import pyoracle

    rng = np.random.default_rng(seed & 0xFFFFFFFF)
    tail = np.arange(max(0, m.rows - 600), m.rows)
    picks = np.unique(np.concatenate([np.arange(min(64, m.rows)), tail,
                                      rng.choice(m.rows, size=min(count, m.rows), replace=False)]))
    rp = m.row_ptr.cpu().numpy().astype(np.int64)
    prp = m.packed_row_ptr.cpu().numpy().astype(np.int64)
    lens, blens = rp[picks + 1] - rp[picks], prp[picks + 1] - prp[picks]
    # gather the sampled rows' entries and code bytes on the device into a compact matrix
    idx = np.concatenate([np.arange(a, b) for a, b in zip(rp[picks], rp[picks + 1])]) if lens.sum() else np.zeros(0, np.int64)
    bidx = np.concatenate([np.arange(a, b) for a, b in zip(prp[picks], prp[picks + 1])]) if blens.sum() else np.zeros(0, np.int64)
    import torch
    dev = m.col_idx.device
    cols = m.col_idx[torch.from_numpy(idx).to(dev)].cpu().numpy()
    packed = m.packed_values[torch.from_numpy(bidx).to(dev)].cpu().numpy()
    sub_rp = np.zeros(len(picks) + 1, np.int32)
    sub_rp[1:] = np.cumsum(lens)
    sub_prp = np.zeros(len(picks) + 1, np.int32)
    sub_prp[1:] = np.cumsum(blens)
    ref, mag = pyoracle.qcsr_spmm_referee(
        m.bits, m.decode_policy, len(picks), m.cols, sub_rp, sub_prp, cols,
        np.concatenate([packed, np.zeros(16, np.uint8)]), m.column_scales.cpu().numpy(),
        m.column_offsets.cpu().numpy(), None, w.cpu().numpy())
    got = out[torch.from_numpy(picks).to(dev)].cpu().numpy()
    cmp = pyoracle.compare(ref, got, 1e-4, 1e-4, mag)
    return {"rows": int(len(picks)), "sample": "seeded uniform over all rows + first 64 + last 600",
            "within_tolerance": bool(cmp["within_tolerance"]),
            "max_relative_error": float(cmp["max_relative_error"])}


def bench_bell_quantized(args, torch, cfg) -> dict:
    """Config 4 with 8-bit per-gene affine codes: the reference's quantized Blocked-ELL
    projection (quantized_blocked_ell_spmm_fwd_f32, f32 W) on C4's block structure, through
    cx_bell_spmm_fwd (fp32 matrix cores, each slot's W tile staged in LDS), N = 256."""
    import numpy as np

    from cellerator_amd import BellMatrix, bell_spmm
    from cellerator_amd.synth import dense_normal, generate_bell

    g = generate_bell(cfg)
    bs, n_out = g.block_size, cfg.n_out
    gen = torch.Generator(device="cuda").manual_seed(cfg.seed)
    codes = torch.randint(0, 256, (g.rows * g.ell_cols,), dtype=torch.uint8, device="cuda", generator=gen)
    scales = torch.rand(g.cols, device="cuda", generator=gen) * 0.02 + 0.001
    offsets = torch.rand(g.cols, device="cuda", generator=gen) * 0.5
    m = BellMatrix(g.rows, g.cols, bs, g.ell_cols, g.block_col_idx, bits=8, decode_policy=1,
                   row_stride_bytes=g.ell_cols, packed_values=codes, column_scales=scales, column_offsets=offsets)
    del g
    w = dense_normal((m.cols, n_out), 0.02, torch.float32, seed=cfg.seed + 7)
    out = torch.empty((m.rows, n_out), dtype=torch.float32, device="cuda")
    valid_blocks = int((m.block_col_idx != -1).sum().item())
    stream = torch.cuda.current_stream()
    # row blocks in the launch schedule's order (planned once per structure, untimed, as for C4)
    from cellerator_amd import bell_plan_groups
    order = bell_plan_groups(m).order
    wall_ms, ev = time_launches(torch, lambda: bell_spmm(m, w, out=out, stream=stream, row_block_order=order),
                                args.steps, args.warmup, stream)
    kern_ms = statistics.mean(ev)
    alg_bytes = (valid_blocks * bs * bs + m.block_col_idx.numel() * 4 + m.cols * 8 + m.cols * n_out * 4
                 + m.rows * n_out * 4)
    flops = 2.0 * valid_blocks * bs * bs * n_out
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
    tflops = flops / (kern_ms * 1e-3) / 1e12
    res = {
        "metric": "quantized Blocked-ELL SpMM (8-bit codes, f32 W): fp32 matrix-core TFLOP/s (% roofline), 500k x 20k, N=256",
        "value": valid_blocks * bs * bs / (wall_ms * 1e-3), "unit": "stored block elements/s",
        "ms_per_step": wall_ms, "dtype": "u8-codes/f32-W/f32-accumulate",
        "config": {"workload": cfg.name + " 8-bit codes", "rows": m.rows, "genes": m.cols, "block_size": bs,
                   "valid_blocks": valid_blocks, "n_out": n_out, "seed": hex(cfg.seed)},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_FP32_PEAK_TFLOPS, "traffic": load_traffic(cfg.name + " 8-bit codes"),
                     "kernel": "bell_spmm_quant_lds<8, per-gene affine, 1 buffer> (cx_bell_spmm_fwd_ordered: fp32 "
                               "matrix cores, W tiles and metadata through LDS, row blocks in the launch schedule's order)",
                     "kernel_ms_mean": kern_ms, "kernel_ms_median": statistics.median(ev),
                     "flops": flops, "algorithmic_bytes": alg_bytes, "hbm_gbs": achieved,
                     "hbm_frac": achieved / HBM_PEAK_GBS},
    }
    from oracle import pyoracle
    pyoracle.build()
    rb = min(4096 // bs, m.rows // bs)
    rows = rb * bs
    idx = m.block_col_idx[:rb].cpu().numpy().view(np.uint32)
    ref, mag = pyoracle.bell_spmm_referee(rows, m.cols, bs, m.ell_cols, idx, None, w.cpu().numpy(), bits=8,
                                          policy=1, row_stride_bytes=m.ell_cols,
                                          packed=codes[:rows * m.ell_cols].cpu().numpy(),
                                          scales=scales.cpu().numpy(), offsets=offsets.cpu().numpy())
    cmp = pyoracle.compare(ref, out[:rows].cpu().numpy(), 2.0 ** -20, 1e-4, mag)
    res["parity_sample"] = {"rows": rows, "within_tolerance": bool(cmp["within_tolerance"]),
                            "max_relative_error": float(cmp["max_relative_error"])}
    return res


def bench_bell(args, torch, cfg) -> dict:
    """Config 4: Blocked-ELL bf16 SpMM on MFMA (cx_bell_spmm_fwd_packed), N = 256."""
    import numpy as np

    from cellerator_amd import (bell_block_major, bell_pack_rhs, bell_plan_groups, bell_spmm_grouped,
                                bell_spmm_packed)
    from cellerator_amd.synth import dense_normal, generate_bell

    t0 = time.perf_counter()
    m = generate_bell(cfg)
    n_out = cfg.n_out
    w = dense_normal((m.cols, n_out), 0.02, torch.bfloat16, seed=cfg.seed + n_out)
    packed = bell_pack_rhs(w)
    out = torch.empty((m.rows, n_out), dtype=torch.float32, device="cuda")
    valid_blocks = int((m.block_col_idx != -1).sum().item())
    # row-block grouping planned once per projection (untimed, like the packed panel)
    groups = None if args.ungrouped else bell_plan_groups(m)
    torch.cuda.synchronize()
    log(f"generated {cfg.name}: {valid_blocks} valid 32x32 blocks in {time.perf_counter() - t0:.1f}s"
        + ("" if groups is None else f"; {groups.planned_groups} groups of 2..4 and {groups.planned_singles} "
                                     f"single row blocks, scheduled as {groups.group_count} units"))
    stream = torch.cuda.current_stream()
    # Headline: the values in block-major order (every 32x32 block's 2 KB contiguous, the
    # layout the CSR -> Blocked-ELL lowering emits), copied once like the packed panel; the
    # generator's row-major values are timed beside it.
    mb = None if args.row_major else bell_block_major(m)
    torch.cuda.synchronize()

    def launch_with(mat):
        def launch():
            if groups is None:
                bell_spmm_packed(mat, packed, n_out, out=out, stream=stream)
            else:
                bell_spmm_grouped(mat, packed, groups, n_out, out=out, stream=stream)
        return launch

    row_major = None
    if mb is not None:
        rm_wall, rm_ev = time_launches(torch, launch_with(m), args.steps, args.warmup, stream)
        row_major = {"ms_per_step": rm_wall, "kernel_ms_mean": statistics.mean(rm_ev),
                     "kernel_ms_median": statistics.median(rm_ev)}
    wall_ms, ev = time_launches(torch, launch_with(mb if mb is not None else m), args.steps, args.warmup,
                                stream)
    kern_ms = statistics.mean(ev)
    bs = m.block_size
    alg_bytes = (valid_blocks * bs * bs * 2 + m.block_col_idx.numel() * 4 + m.cols * n_out * 2
                 + m.rows * n_out * 4)
    flops = 2.0 * valid_blocks * bs * bs * n_out
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
    res = {
        "metric": "Blocked-ELL bf16 SpMM on MFMA: effective HBM GB/s (% roofline) and MFMA TFLOP/s, 500k x 20k, N=256",
        "value": valid_blocks * bs * bs / (wall_ms * 1e-3), "unit": "stored block elements/s",
        "ms_per_step": wall_ms, "dtype": "bf16-values/bf16-W/f32-accumulate",
        "config": {"workload": cfg.name, "rows": m.rows, "genes": m.cols, "block_size": bs,
                   "valid_blocks": valid_blocks, "ell_width": cfg.ell_width, "n_out": n_out,
                   "seed": hex(cfg.seed),
                   "value_layout": "row-major" if mb is None else "block-major (copied once, untimed)",
                   "row_block_groups": None if groups is None else {
                       "groups": groups.planned_groups, "single_row_blocks": groups.planned_singles,
                       "launch_units": groups.group_count,
                       "schedule": "XCD ranges balanced by value blocks (cx_bell_schedule_groups)"}},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic(cfg.name + ("" if mb is not None else " row-major")),
                     "kernel": ("bell_spmm_mfma<256>" if groups is None else "bell_spmm_mfma_slab<256> (grouped, scheduled)")
                               + (", row-major values" if mb is None else ", block-major values"),
                     "kernel_ms_mean": kern_ms,
                     "kernel_ms_median": statistics.median(ev), "algorithmic_bytes": alg_bytes,
                     "mfma_tflops": flops / (kern_ms * 1e-3) / 1e12,
                     "mfma_frac_of_bf16_dense_peak": flops / (kern_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS},
    }
    if row_major is not None:
        res["row_major_path"] = row_major
    if not args.no_cpu:
        from oracle import pyoracle
        pyoracle.build()
        rb = min(args.cpu_rows // bs, m.rows // bs)
        rows = rb * bs
        idx = m.block_col_idx[:rb].cpu().numpy()
        vals = m.values[:rows].view(torch.int16).cpu().numpy().view(np.uint16)
        wn = w.view(torch.int16).cpu().numpy().view(np.uint16)
        threads = host_cores()
        cpu_out = pyoracle.bell_spmm_bf16_mt(rows, m.cols, bs, m.ell_cols, idx, vals, wn,
                                             threads=threads)  # warm caches / page-in
        times = []
        for _ in range(3):
            t1 = time.perf_counter()
            cpu_out = pyoracle.bell_spmm_bf16_mt(rows, m.cols, bs, m.ell_cols, idx, vals, wn,
                                                 threads=threads)
            times.append(time.perf_counter() - t1)
        t = statistics.median(times)
        nvalid = int((idx != np.uint32(0xFFFFFFFF).astype(idx.dtype)).sum())
        got = out[:rows].cpu().numpy()
        err = np.abs(got.astype(np.float64) - cpu_out)
        res["full_output_check"] = {
            "rows": rows, "elements": int(got.size),
            "mismatches": int((err > 1e-4 + 1e-4 * np.abs(cpu_out)).sum()),
            "max_abs_err": float(err.max()) if got.size else 0.0,
            "rule": "|gpu - cpu_fp32| <= 1e-4 + 1e-4 |cpu|"}
        prb = min(rb, 4096 // bs)
        ref, mag = pyoracle.bell_spmm_referee(prb * bs, m.cols, bs, m.ell_cols, idx[:prb],
                                              vals[:prb * bs], wn, value_type=pyoracle.BF16,
                                              rhs_type=pyoracle.BF16)
        cmp = pyoracle.compare(ref, out[:prb * bs].cpu().numpy(), 1e-4, 1e-4, mag)
        res["parity_sample"] = {"rows": prb * bs, "within_tolerance": bool(cmp["within_tolerance"]),
                                "max_relative_error": float(cmp["max_relative_error"])}
        res["cpu_baseline"] = {"value": nvalid * bs * bs / t, "unit": "stored block elements/s",
                               "cores": threads, "kind": "port",
                               "sample": f"first {rows} of {m.rows} rows ({nvalid} blocks), median of 3 "
                                         f"after 1 warmup; oracle or_bell_spmm_bf16_mt (fp32 FMA in slot "
                                         f"order, AVX2, row-block-parallel, zero values skipped)",
                               "seconds": t, "host": host_description()}
    return res


def bench_cpbp(args, torch, cfg) -> dict:
    """Config 5: CP-BP feature-weighted row reduction on 64-row tiles (cx_cpbp_reduce_rows over
    per-entry rows made once; cx_cpbp_reduce timed beside it)."""
    import numpy as np

    from cellerator_amd import cpbp, cpbp_reduce
    from cellerator_amd.synth import dense_normal, generate_cpbp_host

    t0 = time.perf_counter()
    offs, feats, vals = generate_cpbp_host(cfg, threads=host_cores())
    plan = cpbp.contiguous_plan(cfg.genes, cfg.block_width)
    # tiles built on the device (cx_cpbp_device_builder, bitwise equal to the host builder)
    d_offs = torch.from_numpy(offs.view(np.int32)).cuda()
    d_feats = torch.from_numpy(feats.view(np.int32)).cuda()
    d_vals = torch.from_numpy(vals).cuda()
    torch.cuda.synchronize()
    tb = time.perf_counter()
    tiles, _ = cpbp.build_tiles_device(plan, d_offs, d_feats, d_vals, group_width=cfg.tile_row_width,
                                       window_size=cfg.window_size)
    torch.cuda.synchronize()
    build_ms = (time.perf_counter() - tb) * 1e3
    weights = dense_normal((cfg.genes,), 1.0, torch.float32, seed=cfg.seed + 1)
    out = torch.empty(cfg.rows, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    nnz = int(offs[-1])
    log(f"generated and tiled {cfg.name}: nnz={nnz}, "
        f"descriptors={tiles.meta['tile_requirements']['tile_block_count']} "
        f"in {time.perf_counter() - t0:.1f}s (device tile build {build_ms:.0f} ms)")
    stream = torch.cuda.current_stream()

    # Headline: the reduction with each entry's row and block start read from a per-entry
    # array made once per tile structure (cx_cpbp_entry_rows, untimed, like the Blocked-ELL
    # panel); the walk that looks every entry's descriptor up per launch is timed beside it
    # (bitwise the same output).
    from cellerator_amd import cpbp_entry_rows, cpbp_reduce_rows
    torch.cuda.synchronize()
    tr = time.perf_counter()
    entry_rows = cpbp_entry_rows(tiles, stream=stream)
    torch.cuda.synchronize()
    rows_ms = (time.perf_counter() - tr) * 1e3

    def launch():
        cpbp_reduce_rows(tiles, entry_rows, weights, out=out, stream=stream)

    wall_ms, ev = time_launches(torch, launch, args.steps, args.warmup, stream)
    kern_ms = statistics.mean(ev)
    desc_out = torch.empty_like(out)
    desc_wall, desc_ev = time_launches(torch, lambda: cpbp_reduce(tiles, weights, out=desc_out, stream=stream),
                                       args.steps, args.warmup, stream)
    torch.cuda.synchronize()
    desc_equal = bool(torch.equal(desc_out.view(torch.int32), out.view(torch.int32)))
    del desc_out
    alg_bytes = tiles.nbytes_algorithmic()
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
    # the N = 1 CSR comparator on the same canonical matrix, as the reference's reduction
    # bench times it (components/CellPack/bench/feature_weighted_row_reduction_bench.cu:339-344)
    from cellerator_amd import csr_spmv
    spmv_out = torch.empty(cfg.rows, dtype=torch.float32, device="cuda")
    _, spmv_ev = time_launches(torch, lambda: csr_spmv(d_offs, d_feats, d_vals, weights, out=spmv_out,
                                                         stream=stream),
                               args.steps, args.warmup, stream)
    spmv_ms = statistics.mean(spmv_ev)
    spmv_bytes = (cfg.rows + 1) * 4 + nnz * 8 + cfg.genes * 4 + cfg.rows * 4
    spmv_vs_tiles = float(torch.max(torch.abs(spmv_out - out)).item())
    del d_offs, d_feats, d_vals
    res = {
        "metric": "CP-BP feature-weighted row reduction: nnz/s + effective HBM GB/s (% roofline), 2M cells, 64-row tiles",
        "value": nnz / (wall_ms * 1e-3), "unit": "nnz/s", "ms_per_step": wall_ms,
        "dtype": "f32-values/f32-weights/f32-accumulate",
        "config": {"workload": cfg.name, "rows": cfg.rows, "genes": cfg.genes, "nnz": nnz,
                   "tile_row_width": cfg.tile_row_width, "block_width": cfg.block_width,
                   "tile_blocks": tiles.descriptor().tile_block_count,
                   "row_block_entries": tiles.descriptor().row_block_entry_count, "seed": hex(cfg.seed),
                   "tile_build": {"where": "device", "ms": build_ms},
                   "entry_rows": {"bytes": int(entry_rows.numel()) * 4, "ms": rows_ms,
                                  "note": "made once per tile structure (cx_cpbp_entry_rows), untimed"}},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": load_traffic(cfg.name + " entry rows"),
                     "kernel": "cpbp_reduce_kernel<u64,f32,lds-weights,with-entry-rows> (cx_cpbp_reduce_rows)",
                     "kernel_ms_mean": kern_ms,
                     "kernel_ms_median": statistics.median(ev), "algorithmic_bytes": alg_bytes},
        "descriptor_walk": {"kernel": "cpbp_reduce_kernel<u64,f32,lds-weights> (cx_cpbp_reduce)",
                            "ms_per_step": desc_wall, "kernel_ms_mean": statistics.mean(desc_ev),
                            "bitwise_equal_to_headline": desc_equal},
        "csr_spmv_comparator": {"kernel": "csr_spmv_kernel<f32>", "kernel_ms_mean": spmv_ms,
                                "algorithmic_bytes": spmv_bytes,
                                "achieved_gbs": spmv_bytes / (spmv_ms * 1e-3) / 1e9,
                                "max_abs_diff_vs_tiles": spmv_vs_tiles},
    }
    if not args.no_cpu:
        from oracle import pyoracle
        pyoracle.build()
        rows = min(args.cpu_rows, cfg.rows)
        sub_offs = offs[:rows + 1]
        n = int(sub_offs[-1])
        wn = weights.cpu().numpy()
        threads = host_cores()
        ref = pyoracle.cpbp_canonical_mt(sub_offs, feats[:n], vals[:n], wn, threads=threads)
        times = []
        for _ in range(3):
            t1 = time.perf_counter()
            ref = pyoracle.cpbp_canonical_mt(sub_offs, feats[:n], vals[:n], wn, threads=threads)
            times.append(time.perf_counter() - t1)
        t = statistics.median(times)
        res["cpu_baseline"] = {"value": n / t, "unit": "nnz/s", "cores": threads, "kind": "port",
                               "sample": f"first {rows} of {cfg.rows} rows ({n} nnz), median of 3 after "
                                         f"1 warmup; oracle or_cpbp_canonical_mt (the canonical referee, "
                                         f"fp32 accumulate, row-parallel)",
                               "seconds": t, "host": host_description()}
        # the timed output, checked on the same rows against the float64 referee (reference
        # tolerance 1e-5 abs + 1e-5 rel, widened for fp32 reordering)
        got = out[:rows].cpu().numpy()
        ref64, mag = pyoracle.cpbp_canonical_f64(sub_offs, feats[:n], vals[:n], wn)
        bad = np.abs(got.astype(np.float64) - ref64) > 1e-5 + 1e-5 * np.abs(ref64) + 2.0 ** -22 * mag
        res["parity_sample"] = {"rows": rows, "mismatches": int(bad.sum()),
                                "max_abs_err": float(np.max(np.abs(got - ref64))) if rows else 0.0}
        del ref
    return res


def load_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel calibration), or
    None when no summary exists for this workload."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        entry = json.loads(f.read_text()).get(workload)
    except (OSError, ValueError):
        return None
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def calibrate_copy(nbytes: int, reps: int) -> int:
    """Plain device-to-device copy of known size: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": src.numel() * 4, "reps": reps}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=["c3", "c3n128", "c2", "c4", "c4q", "c5"])
    ap.add_argument("--rows", type=int, default=0, help="override the row count (smaller runs)")
    ap.add_argument("--cpu-rows", type=int, default=0,
                    help="rows of the CPU-baseline sample (0: the whole matrix)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--row-major", action="store_true",
                    help="c4: time the generator's row-major values only (no block-major copy)")
    ap.add_argument("--ungrouped", action="store_true",
                    help="C4: time the per-row-block MFMA kernel without the row-block grouping")
    ap.add_argument("--unchecked-columns", action="store_true",
                    help="qCSR: skip the column-order check (kernel keeps its per-entry check)")
    ap.add_argument("--separate-meta", action="store_true",
                    help="C2/C3: time the separate scale/offset arrays instead of interleaved pairs")
    ap.add_argument("--head", type=int, default=None,
                    help="qCSR: matrix-core head genes of the prepared execution-order path (a multiple "
                         "of 1,024; 0: the whole matrix through the tail stream; -1 skips the path). "
                         "Default: the measured best per configuration, 2,048 for C3 (4-bit codes, "
                         "1M x 33,538) and 3,072 for C2 (8-bit codes, 100k x 20k, denser genes)")
    ap.add_argument("--canonical", action="store_true",
                    help="qCSR: headline the canonical row-group kernel on the unprepared CSR")
    ap.add_argument("--no-secondary", action="store_true",
                    help="c3: skip the secondary configurations timed after the headline")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="run only a plain copy of BYTES (rocprofv3 counter calibration)")
    args = ap.parse_args()
    if args.head is None:
        args.head = HEAD_GENES.get(args.config, 2048)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the projection shards by rows with no exchange "
              "between GPUs, so one GPU's throughput at its share's shape is the measurement; "
              "run with --gpus 1.",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy, max(args.steps, 1))
    if args.cpu_rows <= 0:
        args.cpu_rows = 1 << 31  # the whole matrix
    res = run_config(args, torch, args.config)
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": res.pop("dtype"), "data": "synthetic (seeded, generated on GPU)",
            **res}
    if args.config == "c3" and not args.no_secondary and not args.rows and not args.canonical:
        line["secondary"] = secondary_configs(args, torch)
    print(json.dumps(line), flush=True)
    return 0


def run_config(args, torch, name: str) -> dict:
    from cellerator_amd.synth import C2, C3
    if name in ("c4", "c4q", "c5"):
        from cellerator_amd.synth import C4, C5
        cfg = C5 if name == "c5" else C4
        if args.rows:
            cfg = cfg.scaled(args.rows)
        return {"c4": bench_bell, "c4q": bench_bell_quantized, "c5": bench_cpbp}[name](args, torch, cfg)
    cfg, n_out = {"c3": (C3, 64), "c3n128": (C3, 128), "c2": (C2, 64)}[name]
    if args.rows:
        cfg = cfg.scaled(args.rows)
    return bench_qcsr(args, torch, cfg, n_out)


def secondary_configs(args, torch) -> dict:
    """The other benchmark configurations, timed in the same run after the headline (10 steps
    after 3 warmup, no CPU leg): C3 at N = 128, C2, C4 (Blocked-ELL bf16), C4 with 8-bit codes
    (quantized Blocked-ELL, f32 W) and C5 (CP-BP). Each entry keeps the configuration's own
    metric, the kernel's roofline fraction and its parity sample against the referee."""
    import copy

    out = {}
    for name in ("c3n128", "c2", "c4", "c4q", "c5"):
        torch.cuda.empty_cache()
        a = copy.copy(args)
        a.config, a.steps, a.warmup, a.no_cpu = name, 10, 3, True
        a.head = HEAD_GENES.get(name, 2048)
        t0 = time.perf_counter()
        r = run_config(a, torch, name)
        roof = r.get("roofline", {})
        out[name] = {"workload": r.get("config", {}).get("workload"), "metric": r["metric"], "value": r["value"],
                     "unit": r["unit"], "ms_per_step": r["ms_per_step"], "dtype": r["dtype"],
                     "kernel": roof.get("kernel"), "kernel_ms_mean": roof.get("kernel_ms_mean"),
                     "roofline_frac": roof.get("frac"), "roofline_unit": roof.get("unit"),
                     "parity_sample": r.get("parity_sample"), "seconds": time.perf_counter() - t0}
        log(f"secondary {name}: {r['ms_per_step']:.3f} ms/step")
    torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
