"""CSR -> Blocked-ELL lowering (bell_lowering.cpp) on the host, against the reference's own
test vectors (tests/math_bell_lowering_test.cc: the 9 x 13 fixture at :28-114, candidate
geometry and safety-rule verdicts at :188-249, failure codes at :251-297), an independent
decode of every materialized candidate back to the canonical dense matrix (the reference
test's check, :136-186), and the oracle restatement (oracle/bell_lowering.py) on random
inputs: every candidate field and every materialized byte equal, in both value layouts."""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd.bell_lowering import (EMPTY_SOURCE, LEGAL, PERSISTENT_BYTES, STORAGE_EXPANSION,
                                          VALUE_EXPANSION, VALUES_BLOCK_MAJOR, VALUES_ROW_MAJOR,
                                          BellLoweringError, Lowering)
from oracle import bell_lowering as ob

ROWS, FEATURES = 9, 13
BLOCKS = [0, 3, 8, 13]
FPERM = [4, 0, 7, 2, 10, 1, 5, 8, 3, 6, 9, 11, 12]
RPERM = [2, 0, 4, 1, 6, 3, 7, 5, 8]
DESIRED = [(0, 3), (1, 4), (2, 5), (0, 6), (1, 7), (2, 3), (0, 4), (1, 5), (8, 12)]


def reference_fixture():
    """tests/math_bell_lowering_test.cc:28-114: execution row er holds execution features
    DESIRED[er]; canonical row RPERM[er] stores their canonical ids, sorted; value of
    (row, feature) = row * 100 + feature + 1 (float)."""
    canonical = [None] * ROWS
    for er in range(ROWS):
        canonical[RPERM[er]] = sorted(FPERM[d] for d in DESIRED[er])
    offsets, ids, values = [0], [], []
    for r in range(ROWS):
        for f in canonical[r]:
            ids.append(f)
            values.append(float(r * 100 + f + 1))
        offsets.append(len(ids))
    return offsets, ids, np.array(values, np.float32)


def make(offsets, ids, values, features=FEATURES, blocks=BLOCKS, fperm=FPERM, rperm=RPERM, **kw):
    return Lowering(offsets, ids, values, features, blocks, fperm, rperm, **kw)


def oracle_inputs(L: Lowering):
    src = dict(rows=L.source.row_count, features=L.source.feature_count, nnz=L.source.nnz_count,
               value_size=L.value_size, row_offsets=L.row_offsets, feature_ids=L.feature_ids, values=L.values)
    plan = dict(semantic_schema_version=1, full_row_count=L.plan.full_row_count, feature_count=L.plan.feature_count,
                feature_block_count=L.plan.feature_block_count, geometry_identity=L.plan.feature_block_geometry_identity,
                row_domain_identity=L.plan.row_domain_identity, block_offsets=L.block_offsets,
                feature_permutation=L.fperm, inverse_feature_permutation=L.finv)
    order = dict(order_schema_version=1, signature_algorithm_version=1, ordering_identity=L.order.ordering_identity,
                 window_size=L.order.window_size, group_width=L.order.group_width,
                 full_row_count=L.order.full_row_count, row_count=L.order.row_count,
                 feature_block_count=L.order.feature_block_count,
                 geometry_identity=L.order.feature_block_geometry_identity,
                 row_domain_identity=L.order.row_domain_identity, global_row_begin=L.order.global_row_begin,
                 row_permutation=L.rperm, inverse_row_permutation=L.rinv)
    return src, plan, order


def dense(L: Lowering) -> np.ndarray:
    d = np.zeros((L.source.row_count, L.source.feature_count), L.values.dtype)
    for r in range(L.source.row_count):
        for i in range(L.row_offsets[r], L.row_offsets[r + 1]):
            d[r, L.feature_ids[i]] = L.values[i]
    return d


def decode(L: Lowering, view, offsets, cols, vals, layout) -> np.ndarray:
    """Independent decode of a materialized candidate (the reference test's decode,
    math_bell_lowering_test.cc:136-186): every stored value lands on its canonical (row,
    feature); empty slots, padded rows and padded features hold zeros."""
    bs, ell = view.block_size, view.ell_columns // view.block_size
    v = vals.view(L.values.dtype)
    out = np.zeros((L.source.row_count, L.source.feature_count), L.values.dtype)
    blocks = L.block_offsets
    for br in range(view.padded_row_count // bs):
        for slot in range(ell):
            bi = br * ell + slot
            pb = int(cols[bi])
            for lane in range(bs):
                for local in range(bs):
                    idx = (bi * bs + lane) * bs + local if layout == VALUES_BLOCK_MAJOR else \
                        (br * bs + lane) * view.ell_columns + slot * bs + local
                    x = v[idx]
                    er = br * bs + lane
                    if pb < 0 or er >= view.row_count:
                        assert x == 0
                        continue
                    pf = pb * bs + local
                    s = int(np.searchsorted(offsets, pf, side="right")) - 1
                    assert s < len(blocks) - 1
                    within = pf - int(offsets[s])
                    if within >= blocks[s + 1] - blocks[s]:
                        assert x == 0
                        continue
                    out[L.rperm[er], L.fperm[blocks[s] + within]] = x
    return out


def test_reference_fixture_candidates_and_decode():
    L = make(*reference_fixture())
    relaxed = Lowering.policy(1000.0, 1000.0)
    cands = L.query(relaxed)
    # math_bell_lowering_test.cc:200-209
    assert [c.block_size for c in cands] == [8, 16, 32]
    assert [c.padded_feature_count for c in cands] == [24, 48, 96]
    assert [c.metrics.dense_value_slots for c in cands] == [256, 768, 3072]
    assert all(c.state == LEGAL for c in cands)
    want = dense(L)
    for c in cands:
        for layout in (VALUES_BLOCK_MAJOR, VALUES_ROW_MAJOR):
            view, offsets, cols, vals = L.materialize(c, relaxed, layout)
            assert view.candidate_identity == c.candidate_identity  # :225-226
            assert np.array_equal(decode(L, view, offsets, cols, vals, layout), want)
    # default policy (:230-244): only the absurd BELL32 expansion is rejected
    filtered = L.query()
    assert [c.state for c in filtered] == [LEGAL, LEGAL, VALUE_EXPANSION]
    assert abs(filtered[0].metrics.ell_slot_utilization - 0.75) < 1e-12


def test_reference_fixture_failures():
    """math_bell_lowering_test.cc:251-297: a stale ordering identity and a narrowed slot
    count are candidate mismatches; a repeated feature is an invalid source."""
    offsets, ids, values = reference_fixture()
    policy = Lowering.policy(1000.0, 1000.0)
    L = make(offsets, ids, values)
    cand = L.query(policy)[0]
    stale = make(offsets, ids, values, ordering_identity=0xFEDCBA98 ^ 1)
    with pytest.raises(BellLoweringError) as e:
        stale.materialize(cand, policy)
    assert e.value.code == ob.CANDIDATE_MISMATCH
    import copy
    narrow = copy.copy(cand)
    narrow.ell_blocks_per_row -= 1
    with pytest.raises(BellLoweringError) as e:
        L.materialize(narrow, policy)
    assert e.value.code == ob.CANDIDATE_MISMATCH
    dup = list(ids)
    dup[1] = dup[0]
    with pytest.raises(BellLoweringError) as e:
        make(offsets, dup, values).query(policy)
    assert e.value.code == ob.INVALID_SOURCE
    # a rejected candidate is not materialized; a bad policy is an invalid argument
    rejected = L.query()[2]
    with pytest.raises(BellLoweringError) as e:
        L.materialize(rejected)
    assert e.value.code == ob.CANDIDATE_REJECTED
    with pytest.raises(BellLoweringError) as e:
        L.query(Lowering.policy(float("nan"), 1.0))
    assert e.value.code == ob.INVALID_ARGUMENT


@pytest.mark.parametrize("case", ["row_maps", "feature_maps", "empty_block", "order_identity", "offsets"])
def test_inconsistent_inputs_are_rejected(case):
    offsets, ids, values = reference_fixture()
    kw = {}
    fperm, rperm, blocks = list(FPERM), list(RPERM), list(BLOCKS)
    want = {"row_maps": ob.INCOMPATIBLE_ORDER, "feature_maps": ob.INCOMPATIBLE_PLAN,
            "empty_block": ob.INCOMPATIBLE_PLAN, "order_identity": ob.INCOMPATIBLE_ORDER,
            "offsets": ob.INVALID_SOURCE}[case]
    L = make(offsets, ids, values, fperm=fperm, rperm=rperm, blocks=blocks, **kw)
    if case == "row_maps":
        L.rinv[0], L.rinv[1] = L.rinv[1], L.rinv[0]
    elif case == "feature_maps":
        L.finv[0], L.finv[1] = L.finv[1], L.finv[0]
    elif case == "empty_block":
        L.block_offsets[1] = 0
    elif case == "order_identity":
        L.order.feature_block_geometry_identity ^= 1
    elif case == "offsets":
        L.row_offsets[3], L.row_offsets[4] = L.row_offsets[4], L.row_offsets[3]
    with pytest.raises(BellLoweringError) as e:
        L.query()
    assert e.value.code == want


def random_case(rng, rows, features, nblocks, density, dtype=np.float32):
    cuts = np.sort(rng.choice(np.arange(1, features), nblocks - 1, replace=False))
    blocks = np.concatenate([[0], cuts, [features]])
    fperm = rng.permutation(features)
    rperm = rng.permutation(rows)
    offsets, ids = [0], []
    for r in range(rows):
        n = rng.binomial(features, density) if r % 7 != 3 else 0
        ids.extend(np.sort(rng.choice(features, n, replace=False)).tolist())
        offsets.append(len(ids))
    if dtype == np.uint8:
        values = rng.integers(1, 255, len(ids)).astype(np.uint8)
    else:
        values = (rng.standard_normal(len(ids)) + 3.0).astype(dtype)
    return offsets, ids, values, features, blocks, fperm, rperm


@pytest.mark.parametrize("seed,rows,features,nblocks,density,dtype", [
    (1, 37, 61, 5, 0.15, np.float32), (2, 70, 100, 9, 0.05, np.float16), (3, 16, 40, 1, 0.4, np.float64),
    (4, 33, 29, 29, 0.2, np.uint8), (5, 100, 257, 13, 0.02, np.float32)])
def test_engine_matches_oracle(seed, rows, features, nblocks, density, dtype):
    rng = np.random.default_rng(seed)
    offsets, ids, values, nf, blocks, fperm, rperm = random_case(rng, rows, features, nblocks, density, dtype)
    L = Lowering(offsets, ids, values, nf, blocks, fperm, rperm, row_domain_identity=77 + seed)
    relaxed = Lowering.policy(1e6, 1e6)
    src, plan, order = oracle_inputs(L)
    want = ob.query_candidates(src, plan, order, dict(maximum_value_slot_expansion=1e6,
                                                      maximum_storage_expansion=1e6,
                                                      maximum_persistent_bytes=(1 << 64) - 1))
    got = L.query(relaxed)
    full = dense(L)
    for c, w in zip(got, want):
        d = c.as_dict()
        for key in ("state", "block_size", "row_count", "feature_count", "padded_row_count", "padded_feature_count",
                    "block_row_count", "ell_blocks_per_row", "ell_columns", "feature_block_offset_count",
                    "column_index_count", "value_bytes", "candidate_identity"):
            assert d[key] == w[key], key
        for key, val in w["metrics"].items():
            assert d["metrics"][key] == val, key
        _, w_off, w_cols, w_vals = ob.materialize(src, plan, order, c.block_size,
                                                  dict(maximum_value_slot_expansion=1e6,
                                                       maximum_storage_expansion=1e6,
                                                       maximum_persistent_bytes=(1 << 64) - 1))
        view, offsets_out, cols, vals = L.materialize(c, relaxed, VALUES_BLOCK_MAJOR)
        assert np.array_equal(offsets_out, w_off)
        assert np.array_equal(cols, w_cols)
        assert np.array_equal(vals, w_vals)
        _, _, cols_r, vals_r = L.materialize(c, relaxed, VALUES_ROW_MAJOR)
        assert np.array_equal(cols_r, w_cols)
        assert np.array_equal(vals_r, ob.block_major_to_row_major(w_vals, c.block_row_count, c.ell_blocks_per_row,
                                                                  c.block_size, L.value_size))
        assert np.array_equal(decode(L, view, offsets_out, cols, vals, VALUES_BLOCK_MAJOR), full)
        # the gather map lays canonical weights out in physical feature order
        m = L.feature_map(view)
        assert len(m) == c.padded_feature_count
        assert sorted(m[m >= 0].tolist()) == list(range(nf))


def test_safety_rule_order_and_empty_source():
    rng = np.random.default_rng(11)
    offsets, ids, values, nf, blocks, fperm, rperm = random_case(rng, 40, 90, 6, 0.05)
    L = Lowering(offsets, ids, values, nf, blocks, fperm, rperm)
    c = L.query(Lowering.policy(1e9, 1e9))
    # storage expansion is tested after the value expansion; persistent bytes last
    s = L.query(Lowering.policy(1e9, c[1].metrics.storage_expansion * 0.999))
    assert s[1].state == STORAGE_EXPANSION
    p = L.query(Lowering.policy(1e9, 1e9, int(c[1].metrics.persistent_bytes) - 1))
    assert p[1].state == PERSISTENT_BYTES
    v = L.query(Lowering.policy(c[1].metrics.value_slot_expansion * 0.999, 1e-9))
    assert v[1].state == VALUE_EXPANSION
    empty = Lowering([0] * 41, [], np.zeros(0, np.float32), nf, blocks, fperm, rperm)
    assert [x.state for x in empty.query()] == [EMPTY_SOURCE] * 3
