"""Pins the oracle's window plan (orc_make_windows, a restatement of
src/layers/seedvr2_dit_block.cpp:827-868) bit-exactly:
  * hand-derived known-answer plans of the reference rule at the benchmark
    grids (adaptive extents, the 2x16x30 shifted plan with its dropped empty
    windows, the explicit 2x8x10 and 2x9x16 plans and their sum of S^2);
  * an exact-integer brute force of the rule over every small grid;
  * partition invariants (every grid cell in exactly one window).
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

import winplan_exact as wx

L_TXT = 58


def test_adaptive_known_answers(orc):
    # seedvr2_dit_block.cpp:832-838 evaluated by hand
    assert orc.adaptive_window(2, 16, 30) == (1, 15, 28)
    assert orc.adaptive_window(6, 45, 80) == (2, 15, 27)
    assert orc.adaptive_window(2, 15, 20) == (1, 18, 23)
    assert orc.adaptive_window(1, 16, 30) == (1, 15, 28)
    assert orc.adaptive_window(21, 45, 80) == (6, 15, 27)
    assert orc.adaptive_window(40, 45, 80) == (8, 15, 27)  # frames capped at 30


def test_adaptive_2x16x30_shifted_drops_empty_windows(orc):
    # shift 0.5 on every axis (1 < 2, 15 < 16, 28 < 30); the loops run 3x3x3
    # but the intervals [0,0) / [2,2) etc. are empty and skipped
    expect = [(0, 1, 0, 7, 0, 14), (1, 2, 0, 7, 0, 14), (0, 1, 7, 16, 0, 14), (1, 2, 7, 16, 0, 14),
              (0, 1, 0, 7, 14, 30), (1, 2, 0, 7, 14, 30), (0, 1, 7, 16, 14, 30), (1, 2, 7, 16, 14, 30)]
    assert orc.make_windows(2, 16, 30, True) == expect


def test_adaptive_2x16x30_unshifted(orc):
    wins = orc.make_windows(2, 16, 30, False)
    assert len(wins) == 8
    sizes = sorted((w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) for w in wins)
    assert sizes == [2, 2, 28, 28, 30, 30, 420, 420]


def test_explicit_2x8x10_plans(orc):
    un = orc.make_windows(2, 16, 30, False, 2, 8, 10)
    assert len(un) == 6 and all((w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) == 160 for w in un)
    # w outer, h, t inner
    assert un[:3] == [(0, 2, 0, 8, 0, 10), (0, 2, 8, 16, 0, 10), (0, 2, 0, 8, 10, 20)]
    sh = orc.make_windows(2, 16, 30, True, 2, 8, 10)
    assert len(sh) == 12  # no t shift (window 2 == T), shift (4, 5) on h, w
    hs = sorted({(w[2], w[3]) for w in sh})
    ws = sorted({(w[4], w[5]) for w in sh})
    assert hs == [(0, 4), (4, 12), (12, 16)]
    assert ws == [(0, 5), (5, 15), (15, 25), (25, 30)]
    assert {w[:2] for w in sh} == {(0, 2)}


def test_explicit_720p_plans(orc):
    un = orc.make_windows(6, 45, 80, False, 2, 9, 16)
    assert len(un) == 75 and all((w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) == 288 for w in un)
    sh = orc.make_windows(6, 45, 80, True, 2, 9, 16)
    assert len(sh) == 144
    assert sorted({w[:2] for w in sh}) == [(0, 1), (1, 3), (3, 5), (5, 6)]
    assert sorted({w[2:4] for w in sh}) == [(0, 4), (4, 13), (13, 22), (22, 31), (31, 40), (40, 45)]
    assert sorted({w[4:] for w in sh}) == [(0, 8), (8, 24), (24, 40), (40, 56), (56, 72), (72, 80)]
    sizes = [(w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) for w in sh]
    assert min(sizes) == 32 and max(sizes) == 288


@pytest.mark.parametrize("args,expect", [
    ((2, 16, 30, False, 2, 8, 10), 285_144),
    ((2, 16, 30, True, 2, 8, 10), 247_728),
    ((6, 45, 80, False, 2, 9, 16), 8_978_700),
    ((6, 45, 80, True, 2, 9, 16), 7_194_816),
    ((6, 45, 80, False, 0, 0, 0), 19_881_828),
    ((6, 45, 80, True, 0, 0, 0), 12_832_376),
])
def test_sum_of_squared_sequence_lengths(orc, args, expect):
    # sum_w S_w^2 with S_w = window video tokens + 58 text tokens: the factor
    # of the attention flop count 4 * S^2 * 128 * heads
    wins = orc.make_windows(*args)
    assert sum(((w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) + L_TXT) ** 2 for w in wins) == expect


def test_adaptive_matches_exact_rule(orc):
    for T in (1, 2, 5, 21, 30, 31):
        for H in range(1, 65):
            for W in range(1, 65, 3):
                assert orc.adaptive_window(T, H, W) == wx.adaptive(T, H, W), (T, H, W)


def test_plan_matches_exact_rule_brute_force(orc):
    n = 0
    for T, H, W in itertools.product(range(1, 7), range(1, 13), range(1, 13)):
        for shifted in (False, True):
            assert orc.make_windows(T, H, W, shifted) == wx.plan(T, H, W, shifted), (T, H, W, shifted)
            for wt, wh, ww in ((1, 2, 3), (2, 3, 2), (3, 5, 4), (2, 9, 16)):
                got = orc.make_windows(T, H, W, shifted, wt, wh, ww)
                assert got == wx.plan(T, H, W, shifted, wt, wh, ww), (T, H, W, shifted, wt, wh, ww)
                n += 1
    assert n > 5000


@pytest.mark.parametrize("args", [
    (2, 16, 30, False, 2, 8, 10), (2, 16, 30, True, 2, 8, 10), (6, 45, 80, True, 2, 9, 16),
    (6, 45, 80, False, 0, 0, 0), (6, 45, 80, True, 0, 0, 0), (7, 13, 11, True, 3, 4, 5),
    (2, 15, 20, True, 0, 0, 0), (1, 1, 1, True, 0, 0, 0),
])
def test_plan_partitions_the_grid(orc, args):
    T, H, W = args[:3]
    wins = orc.make_windows(*args)
    cover = np.zeros((T, H, W), np.int32)
    for (t0, t1, h0, h1, w0, w1) in wins:
        assert 0 <= t0 < t1 <= T and 0 <= h0 < h1 <= H and 0 <= w0 < w1 <= W
        cover[t0:t1, h0:h1, w0:w1] += 1
    assert (cover == 1).all()
    idx = wx.index_map(T, H, W, wins)
    assert sorted(idx) == list(range(T * H * W))  # the gather map is a bijection
