"""The reference's end-to-end planner (src/planner/end_to_end_planner.cc, compiled from its
source into oracle/_ref/) over the engine's CP-Math candidates: it accepts, prices, ranks and
selects them, with the engine's analytical cost model (cpmath::planner_candidate_for) and the
host's policy -- kind mismatch, nondeterminism and memory limits reject candidates with the
reference's reasons; a measurement hook turns the choice empirical and fills the plan cache;
one-shot work skips tuning (tests/planner/end_to_end_planner_test.cc is the model)."""
from __future__ import annotations

import pytest

from tests.cpmath import planner as P

# C3: 1M cells x 33,538 genes, 1.5e9 4-bit entries, N = 64; as Blocked-ELL the scattered
# genes leave most of every 32 x 32 block empty (about 20,000 padded columns per row).
C3 = dict(rows=1_000_000, cols=33_538, nnz=1_498_000_000, n=64, ell_columns=20_000)
# C4: 500k x 20k with 64 dense-ish 32 x 32 blocks per row block (2,048 columns per row).
C4 = dict(rows=500_000, cols=20_000, nnz=358_000_000, n=256, ell_columns=2_048)


def test_analytical_ranking_follows_the_layout():
    r = P.plan(P.spmm_case(**C3))
    assert r.status == P.OK and r.source == P.ANALYTICAL and r.tuning_skipped
    assert r.legal == 2 and r.shortlist == 2
    assert r.winner == P.QCSR_ID
    assert r.diag(P.QCSR_ID).analytical_ns < r.diag(P.BELL_ID).analytical_ns
    r = P.plan(P.spmm_case(**C4))
    assert r.winner == P.BELL_ID
    assert r.diag(P.BELL_ID).analytical_ns < r.diag(P.QCSR_ID).analytical_ns


def test_operation_kind_mismatch_is_malformed():
    r = P.plan(P.spmm_case(**C4, mask=P.QCSR | P.BELL | P.CPBP))
    assert r.count == 3 and r.legal == 2
    assert r.diag(P.CPBP_ID).rejection == P.MALFORMED
    c = P.spmm_case(**C4, mask=P.QCSR | P.BELL | P.CPBP)
    c.problem_kind, c.tile_blocks, c.value_bytes = 2, 40_000_000, 2
    r = P.plan(c)
    assert r.winner == P.CPBP_ID and r.legal == 1
    assert r.diag(P.QCSR_ID).rejection == P.MALFORMED and r.diag(P.BELL_ID).rejection == P.MALFORMED


def test_memory_and_determinism_policy():
    base = P.plan(P.spmm_case(**C4))
    # a persistent limit between the two projections' bytes (quantized CSR about 1.6 GB,
    # Blocked-ELL about 2.1 GB) leaves the quantized CSR
    c = P.spmm_case(**C4, max_persistent=1_800_000_000)
    r = P.plan(c)
    assert r.diag(P.BELL_ID).rejection == P.PERSISTENT and r.winner == P.QCSR_ID
    c = P.spmm_case(**C4, max_transient=1_000_000)
    r = P.plan(c)
    assert r.diag(P.BELL_ID).rejection == P.TRANSIENT
    c = P.spmm_case(**C4, nondeterministic_mask=2)
    r = P.plan(c)
    assert r.diag(P.BELL_ID).rejection == P.NONDETERMINISTIC and r.winner == P.QCSR_ID
    c = P.spmm_case(**C4, nondeterministic_mask=3)
    r = P.plan(c)
    assert r.status == P.NO_LEGAL and r.legal == 0
    c = P.spmm_case(**C4, nondeterministic_mask=2, deterministic=0)
    assert P.plan(c).winner == base.winner


def test_unpriceable_shape_is_malformed():
    c = P.spmm_case(**C4)
    c.ell_columns = 0  # no Blocked-ELL geometry
    r = P.plan(c)
    assert r.diag(P.BELL_ID).rejection == P.MALFORMED and r.winner == P.QCSR_ID


def test_measurement_overrides_the_model_and_fills_the_cache():
    timings = {P.QCSR_ID: 900_000.0, P.BELL_ID: 2_500_000.0}

    def measure(identity):
        return dict(kernel_ns=timings[identity], samples=7, spread_percent=1.0)

    r = P.plan(P.spmm_case(**C4, use_cache=2), measure)
    assert r.status == P.OK and r.source == P.EMPIRICAL and r.measured == 2
    assert r.winner == P.QCSR_ID  # the analytical favourite lost on the clock
    assert r.diag(P.QCSR_ID).empirical_ns < r.diag(P.BELL_ID).empirical_ns
    assert r.confidence >= 0.8 and r.cache == P.MISS and r.stored
    again = P.plan(P.spmm_case(**C4, use_cache=1))
    assert again.source == P.CACHE and again.cache == P.HIT and again.winner == P.QCSR_ID
    stale = P.plan(P.spmm_case(**C4, use_cache=1, evidence_revision=45))
    assert stale.cache == P.STALE and stale.source == P.ANALYTICAL


def test_tuning_bounds_and_failures():
    calls = []

    def measure(identity):
        calls.append(identity)
        return dict(kernel_ns=1_000_000.0, samples=5, spread_percent=1.0)

    r = P.plan(P.spmm_case(**C4, structure_reuse=1, projection_reuse=1), measure)
    assert r.tuning_skipped and r.measured == 0 and not calls
    r = P.plan(P.spmm_case(**C4, max_measurements=1), measure)
    assert r.measured == 1 and len(calls) == 1
    r = P.plan(P.spmm_case(**C4), lambda identity: dict(kernel_ns=1.0, samples=5, spread_percent=50.0))
    assert r.source == P.ANALYTICAL and all(r.diags[k].rejection == P.CONTAMINATED for k in range(2))
    r = P.plan(P.spmm_case(**C4, allow_fallback=0), lambda identity: None)
    assert r.status == P.NO_CORRECT_MEASUREMENT
    r = P.plan(P.spmm_case(**C4), lambda identity: dict(kernel_ns=1.0, samples=5, spread_percent=1.0,
                                                        correct=identity != P.BELL_ID))
    assert r.diag(P.BELL_ID).rejection == P.INCORRECT and r.winner == P.QCSR_ID


def test_execution_order_candidate_is_chosen_for_reuse():
    """The execution-order candidate pays a one-time preparation (about 0.028 ns per stored
    entry: 41 ms at C3) and more persistent bytes for about half the launch time of the
    row-group candidate. The planner amortizes the preparation over the projection reuse
    (compute_total_cost, src/planner/end_to_end_planner.cc:184-213): a single run keeps the
    row-group candidate, a persistent projection takes the execution order, and a persistent
    limit below its layouts rejects it with the reference's reason."""
    both = P.QCSR | P.QCSR_EXEC
    single = P.plan(P.spmm_case(**C3, mask=both, structure_reuse=1, projection_reuse=1))
    assert single.status == P.OK and single.legal == 2
    assert single.winner == P.QCSR_ID
    ex, rg = single.diag(P.QCSR_EXEC_ID), single.diag(P.QCSR_ID)
    assert ex.analytical_ns > rg.analytical_ns > 0.0
    persistent = P.plan(P.spmm_case(**C3, mask=both, structure_reuse=1000, projection_reuse=1000))
    assert persistent.winner == P.QCSR_EXEC_ID
    ex, rg = persistent.diag(P.QCSR_EXEC_ID), persistent.diag(P.QCSR_ID)
    # measured launch times at C3: 3.31 ms against 6.99 ms
    assert 0.40 < ex.analytical_ns / rg.analytical_ns < 0.60
    # the prepared layouts add about 4 GB at C3 to the structure's 6.8 GB
    tight = P.plan(P.spmm_case(**C3, mask=both, structure_reuse=1000, projection_reuse=1000,
                               max_persistent=8_000_000_000))
    assert tight.diag(P.QCSR_EXEC_ID).rejection == P.PERSISTENT
    assert tight.winner == P.QCSR_ID
    # plain values have no execution-order form: the candidate's shape cannot be priced
    plain = P.plan(P.spmm_case(**C3, mask=both, bits=0, value_bytes=4, projection_reuse=1000))
    assert plain.diag(P.QCSR_EXEC_ID).rejection == P.MALFORMED and plain.winner == P.QCSR_ID
