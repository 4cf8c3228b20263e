"""Host planner of the grouped Blocked-ELL path (cx_bell_plan_groups), on the CPU: the
order is a permutation of the row blocks, every group holds 2..max_group row blocks whose
valid block-column lists are prefixes of the group's last (longest) member, and the plan
is deterministic."""
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
