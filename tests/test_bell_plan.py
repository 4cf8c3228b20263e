"""Host planner of the grouped Blocked-ELL path (cx_bell_plan_groups), on the CPU: the
order is a permutation of the row blocks, every group holds 2..max_group row blocks whose
valid block-column lists are prefixes of the group's last (longest) member, and the plan
is deterministic. Its launch schedule (cx_bell_schedule_groups) keeps the same units and
evens out the value blocks of the eight XCD ranges."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cellerator_amd import _native as N

INVALID = 0xFFFFFFFF


def plan(idx: np.ndarray, max_group: int = 4):
    rb, slots = idx.shape
    idx = np.ascontiguousarray(idx, np.uint32)
    order = np.zeros(max(rb, 1), np.uint32)
    offs = np.zeros(rb + 1, np.uint32)
    gc, sc = C.c_uint32(), C.c_uint32()
    st = N.engine().cx_bell_plan_groups(idx.ctypes.data, rb, slots, max_group, order.ctypes.data,
                                        offs.ctypes.data, C.byref(gc), C.byref(sc))
    if st != 0:
        raise N.EngineError("cx_bell_plan_groups", st, N.engine().cx_bell_plan_last_error().decode())
    return order[:rb], offs[: gc.value + 1], gc.value, sc.value


def valid_list(idx, r):
    return [int(c) for c in idx[r] if c != INVALID]


def patterned(rng, rb=400, slots=64, patterns=12, scatter_invalid=False):
    kb = 500
    pats = [np.sort(rng.choice(kb, slots, replace=False)) for _ in range(patterns)]
    idx = np.full((rb, slots), INVALID, np.uint32)
    for r in range(rb):
        c = int(rng.integers(0, slots + 1))
        lst = pats[int(rng.integers(0, patterns))][:c]
        if scatter_invalid and c < slots:
            pos = np.sort(rng.choice(slots, c, replace=False))
            idx[r, pos] = lst
        else:
            idx[r, :c] = lst
    return idx


def check_plan(idx, max_group):
    order, offs, gc, sc = plan(idx, max_group)
    rb = idx.shape[0]
    assert sorted(order.tolist()) == list(range(rb))
    grouped = int(offs[gc]) if gc else 0
    assert grouped + sc == rb
    for g in range(gc):
        members = order[offs[g]:offs[g + 1]].tolist()
        assert 2 <= len(members) <= max_group
        longest = valid_list(idx, members[-1])
        for r in members:
            lst = valid_list(idx, r)
            assert lst and lst == longest[:len(lst)]
    return order, offs, gc, sc


@pytest.mark.parametrize("max_group", [2, 3, 4])
@pytest.mark.parametrize("scatter", [False, True])
def test_groups_are_prefix_families(max_group, scatter):
    rng = np.random.default_rng(max_group * 10 + scatter)
    idx = patterned(rng, scatter_invalid=scatter)
    order, offs, gc, sc = check_plan(idx, max_group)
    # patterned rows share prefixes: nearly everything is grouped
    assert sc < idx.shape[0] // 4


def test_deterministic():
    idx = patterned(np.random.default_rng(7))
    a, b = plan(idx), plan(idx)
    assert all(np.array_equal(x, y) if isinstance(x, np.ndarray) else x == y for x, y in zip(a, b))


def test_unrelated_rows_stay_single_and_empty_rows_are_singles():
    rng = np.random.default_rng(9)
    idx = np.full((50, 16), INVALID, np.uint32)
    for r in range(50):
        idx[r, :8] = np.sort(rng.choice(100000, 8, replace=False))  # no shared prefixes
    idx[3] = INVALID
    order, offs, gc, sc = check_plan(idx, 4)
    assert gc == 0 and sc == 50


def test_max_group_is_validated():
    idx = patterned(np.random.default_rng(1), rb=10, slots=8)
    for bad in (0, 5):
        with pytest.raises(N.EngineError):
            plan(idx, bad)


def schedule(idx: np.ndarray, order, offs, gc, sc):
    rb, slots = idx.shape
    idx = np.ascontiguousarray(idx, np.uint32)
    s_order = np.zeros(max(rb, 1), np.uint32)
    s_offs = np.zeros(rb + 1, np.uint32)
    units = C.c_uint32()
    order = np.ascontiguousarray(order, np.uint32)
    offs = np.ascontiguousarray(offs, np.uint32)
    st = N.engine().cx_bell_schedule_groups(idx.ctypes.data, rb, slots, order.ctypes.data, offs.ctypes.data,
                                            gc, sc, s_order.ctypes.data, s_offs.ctypes.data, C.byref(units))
    if st != 0:
        raise N.EngineError("cx_bell_schedule_groups", st, N.engine().cx_bell_plan_last_error().decode())
    return s_order[:rb], s_offs[: units.value + 1], units.value


def xcd_units(units):
    """Units each XCD runs under the grouped kernels' workgroup mapping (workgroup i on XCD
    i % 8 runs unit (i % 8) * per + i / 8 below 8 * per, its own index above)."""
    per = units // 8
    ranges = [list(range(x * per, (x + 1) * per)) for x in range(8)]
    for i in range(8 * per, units):
        ranges[i % 8].append(i)
    return ranges


@pytest.mark.parametrize("rb", [5, 64, 400, 2003])
def test_schedule_keeps_the_units_and_balances_the_xcd_ranges(rb):
    rng = np.random.default_rng(rb)
    idx = patterned(rng, rb=rb, slots=64, patterns=12)
    order, offs, gc, sc = check_plan(idx, 4)
    s_order, s_offs, units = schedule(idx, order, offs, gc, sc)
    assert units == gc + sc
    assert sorted(s_order.tolist()) == list(range(rb)) and int(s_offs[units]) == rb
    planned = {tuple(order[offs[g]:offs[g + 1]].tolist()) for g in range(gc)}
    planned |= {(int(r),) for r in order[int(offs[gc]) if gc else 0:]}
    got = [tuple(s_order[s_offs[u]:s_offs[u + 1]].tolist()) for u in range(units)]
    assert sorted(got) == sorted(planned)  # the same units, members in the same order
    blocks = (idx != INVALID).sum(1)
    cost = [int(sum(blocks[r] for r in unit)) for unit in got]
    if units >= 8:
        per = units // 8
        work = [sum(cost[u] for u in range(x * per, (x + 1) * per)) for x in range(8)]
        # the ranges differ by less than one unit's blocks
        assert max(work) - min(work) <= max(cost)
        # the ragged tail holds the cheapest units
        tail = sorted(cost[8 * per:])
        assert tail == sorted(cost)[:len(tail)]
    assert np.array_equal(schedule(idx, order, offs, gc, sc)[0], s_order)  # deterministic


def test_schedule_balances_modules_of_unequal_length():
    # 40 modules of 24..64 block columns (the C4 shape): the planner's order cut into equal
    # counts leaves the XCD ranges unequal; the schedule evens them out
    rng = np.random.default_rng(40)
    slots, patterns, rb = 64, 40, 4000
    pats = [np.sort(rng.choice(625, int(rng.integers(24, 65)), replace=False)) for _ in range(patterns)]
    idx = np.full((rb, slots), INVALID, np.uint32)
    for r in range(rb):
        p = pats[int(rng.integers(0, patterns))]
        idx[r, :len(p)] = p
    order, offs, gc, sc = check_plan(idx, 4)
    blocks = (idx != INVALID).sum(1)

    def spread(o, f, units):
        per = units // 8
        w = [sum(int(blocks[o[f[u]:f[u + 1]]].sum()) for u in range(x * per, (x + 1) * per)) for x in range(8)]
        return max(w) - min(w), max(w)

    plain_offs = np.concatenate([offs[:gc + 1], offs[gc] + 1 + np.arange(sc, dtype=np.uint32)]) if gc else \
        np.arange(rb + 1, dtype=np.uint32)
    before, _ = spread(order, plain_offs, gc + sc)
    s_order, s_offs, units = schedule(idx, order, offs, gc, sc)
    after, heaviest = spread(s_order, s_offs, units)
    assert after < before and after <= 4 * 64
    # a module's units stay together: most units run in the range that holds most of
    # their module (the balancing swaps move a few)
    per = units // 8
    owner = {}
    for u in range(8 * per):
        first = int(idx[s_order[s_offs[u + 1] - 1], 0])
        owner.setdefault(first, []).append(u // per)
    together = sum(max(v.count(x) for x in set(v)) for v in owner.values())
    assert together >= 0.8 * 8 * per


def test_schedule_of_no_row_blocks():
    idx = np.zeros((0, 4), np.uint32)
    order, offs, gc, sc = plan(idx, 4)
    s_order, s_offs, units = schedule(idx, order, offs, gc, sc)
    assert units == 0 and s_offs[0] == 0


def test_schedule_rejects_a_bad_plan():
    idx = patterned(np.random.default_rng(3), rb=40, slots=16)
    order, offs, gc, sc = plan(idx, 4)
    bad = order.copy()
    bad[0] = bad[1]
    with pytest.raises(N.EngineError):
        schedule(idx, bad, offs, gc, sc)
    with pytest.raises(N.EngineError):
        schedule(idx, order, offs, gc, sc + 1)
