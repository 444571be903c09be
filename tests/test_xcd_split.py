"""The packed GEMMs' per-XCD item ranges (cernels_amd/csrc/moe_split.h), evaluated on the CPU.

The route kernel computes them in integer and float arithmetic per expert; here the same header is
compiled for the host and its bounds are compared with the definition counted item by item: XCD x
starts at the first item whose cost prefix reaches ceil(x W / 8), an item of r rows costing
32 fw + r, where an equal split of the items gives each workgroup R >= 8 rounds; with fewer rounds
the split is the equal one. Where the cost split would give some XCD more than cap items (R rounds
plus R / 8) the bounds are clamped; every result covers the list once, in order, with at most cap
items per XCD.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def split_exe(tmp_path_factory):
    exe = tmp_path_factory.mktemp("split") / "xcd_split_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-DCMOE_HD=", "-I", str(ROOT / "cernels_amd" / "csrc"),
                    str(ROOT / "tests" / "xcd_split_check.cpp"), "-o", str(exe)], check=True)
    return exe


def _run(exe, cases):
    text = "".join(f"S {len(r)} {fw} {nt} {sl} " + " ".join(map(str, r)) + "\n" for r, fw, nt, sl in cases)
    out = subprocess.run([str(exe)], input=text, capture_output=True, text=True, check=True).stdout
    return [list(map(int, line.split())) for line in out.strip().splitlines()]


def _by_definition(runs, fw, n_tiles):
    """Unclamped bounds, counted over the item list (expert by expert, N-tile-major)."""
    costs = []
    for r in runs:
        nt = -(-r // 256)
        rows = np.minimum(256, r - 256 * np.arange(nt))
        costs.append(np.tile(32 * fw + rows, n_tiles))
    costs = np.concatenate(costs) if costs else np.zeros(0, np.int64)
    start = np.concatenate([[0], np.cumsum(costs)])[:-1]
    W = int(costs.sum())
    return [int(np.searchsorted(start, -(-k * W // 8), side="left")) for k in range(9)], len(costs)


def _rounds(total, slots):
    return -(-(-(-total // 8)) // slots)


def _cap(total, slots):
    rounds = _rounds(total, slots)
    return (rounds + rounds // 8) * slots


def _cases():
    rng = np.random.default_rng(7)
    cases = [([0] * 8, 8, 4, 32), ([1], 8, 1, 1), ([300], 1, 360, 32), ([256] * 64, 7, 8, 32),
             ([384] * 64, 8, 8, 32), ([512] * 32, 8, 23, 32), ([0, 0, 5, 0], 3, 2, 1)]
    for _ in range(300):
        E = int(rng.integers(1, 300))
        P = int(rng.integers(0, 60000))
        runs = rng.multinomial(P, rng.dirichlet(np.full(E, rng.uniform(0.05, 3.0)))).tolist()
        cases.append((runs, int(rng.integers(1, 9)), int(rng.integers(1, 48)), int(rng.integers(1, 33))))
    return cases


def _start_of(runs, fw, n_tiles, items):
    """Cost prefix before each given item index, from the per-expert closed form."""
    nt = -(-np.asarray(runs, np.int64) // 256)
    c = 32 * fw * nt + np.asarray(runs, np.int64)
    first = np.concatenate([[0], np.cumsum(nt * n_tiles)])
    S = np.concatenate([[0], np.cumsum(n_tiles * c)])
    items = np.asarray(items, np.int64)
    e = np.searchsorted(first, items, side="right") - 1
    e = np.minimum(e, len(runs) - 1)
    local = items - first[e]
    ntile = np.maximum(nt[e], 1)
    n, m = local // ntile, local % ntile
    return S[e] + n * c[e] + m * (32 * fw + 256), int(S[-1])


def test_split_matches_the_item_count_definition(split_exe):
    cases = _cases()
    got = _run(split_exe, cases)
    assert len(got) == len(cases)
    equal = split = clamped = 0
    for (runs, fw, n_tiles, slots), b in zip(cases, got):
        want, total = _by_definition(runs, fw, n_tiles)
        cap = _cap(total, slots)
        assert b[0] == 0 and b[8] == total and all(x <= y for x, y in zip(b, b[1:])), (runs[:8], b)
        assert max(y - x for x, y in zip(b, b[1:])) <= cap, (b, cap)
        if _rounds(total, slots) < 8:
            per = -(-total // 8)
            assert b == [min(k * per, total) for k in range(9)]
            equal += 1
        elif max(y - x for x, y in zip(want, want[1:])) <= cap:
            assert b == want, (fw, n_tiles, slots, b, want)
            split += 1
        else:
            clamped += 1
    assert min(equal, split, clamped) > 0  # every branch is exercised


def test_equal_items_split_evenly(split_exe):
    """Experts of equal size: the cost split is the equal item split (16 rounds of 8 workgroups)."""
    (b,) = _run(split_exe, [([256] * 64, 8, 16, 8)])
    assert b == [128 * x for x in range(9)]


def test_split_of_long_lists(split_exe):
    """2^29 pairs and over: cost prefixes beyond 2^32. Each bound is the first item whose cost prefix
    reaches ceil(x W / 8), checked at the bound and at the item before it (at this many rounds the
    clamp does not bind)."""
    rng = np.random.default_rng(11)
    cases = [(rng.integers(0, 1 << 20, size=1024).tolist(), 1, 360, 32),
             (rng.integers(0, 1 << 21, size=256).tolist(), 8, 23, 32)]
    big = 0
    for (runs, fw, n_tiles, slots), b in zip(cases, _run(split_exe, cases)):
        total = int((-(-np.asarray(runs) // 256)).sum()) * n_tiles
        cap = _cap(total, slots)
        assert b[0] == 0 and b[8] == total and all(x <= y for x, y in zip(b, b[1:]))
        assert max(y - x for x, y in zip(b, b[1:])) <= cap
        at, W = _start_of(runs, fw, n_tiles, b[1:8])
        before, _ = _start_of(runs, fw, n_tiles, [x - 1 for x in b[1:8]])
        big = max(big, W)
        for k in range(1, 8):
            t = -(-k * W // 8)
            assert before[k - 1] < t <= at[k - 1], (k, b)
    assert big > 1 << 32


def test_floordiv_at_integer_quotients(split_exe):
    """split_floordiv's float estimate is off by one just below and at exact quotients of large
    operands; the correction must give floor(a / b) there."""
    rng = np.random.default_rng(3)
    pairs = []
    for _ in range(400):
        b = int(rng.integers(1, 1 << 42))
        q = int(rng.integers(0, 1 << 20))
        for a in (q * b - 1, q * b, q * b + 1, q * b + b - 1):
            if a >= 0 and a // b < 1 << 20:
                pairs.append((a, b))
    text = "".join(f"D {a} {b}\n" for a, b in pairs)
    out = subprocess.run([str(split_exe)], input=text, capture_output=True, text=True, check=True).stdout.split()
    assert [int(v) for v in out] == [a // b for a, b in pairs]


def _tail_codes(exe, cases):
    text = "".join(f"T {len(rows)} {slots} {tail} {bm} " + " ".join(map(str, rows)) + "\n"
                   for rows, slots, tail, bm in cases)
    out = subprocess.run([str(exe)], input=text, capture_output=True, text=True, check=True).stdout
    got, cur = [], []
    for line in out.strip().splitlines():
        if line == "END":
            got.append(cur)
            cur = []
        else:
            cur.append(tuple(map(int, line.split())))
    return got


def test_tail_halves_cover_every_row_once(split_exe):
    """The gate_up GEMM's tail (moe_split.h tail_items / tail_splits / tail_part): the work codes of one XCD
    range give every row of every item to exactly one work unit; only ranges of three or more rounds have a
    tail, the whole items before it cover the first two offsets of every slot, only items of more than 3/4 bm
    rows are halved, and no half is empty."""
    rng = np.random.default_rng(5)
    cases = [([256] * 121, 32, 12, 256), ([256] * 95, 32, 12, 256), ([100] * 200, 32, 12, 256),
             ([193, 192, 256, 32] * 30, 32, 12, 256), ([256] * 5, 1, 12, 256), ([256] * 40, 8, 64, 256)]
    for _ in range(200):
        n = int(rng.integers(1, 400))
        rows = rng.integers(1, 257, size=n).tolist()
        cases.append((rows, int(rng.integers(1, 33)), int(rng.integers(0, 20)), 256))
    halved = 0
    for (rows, slots, tail, bm), codes in zip(cases, _tail_codes(split_exe, cases)):
        n = len(rows)
        n_tail = min(tail, 16, n - 2 * slots) if n >= 3 * slots else 0
        assert all(h == 0 for _, h, _, _ in codes[:n - n_tail])
        assert n - n_tail >= (2 * slots if n_tail else 0)
        covered = [np.zeros(r, np.int32) for r in rows]
        for item, h, rb, r in codes:
            assert r > 0 and 0 <= rb and rb + r <= rows[item], (item, h, rb, r)
            assert h == 0 or 4 * rows[item] > 3 * bm
            covered[item][rb:rb + r] += 1
        assert all((c == 1).all() for c in covered)
        assert [i for i, _, _, _ in codes] == sorted(i for i, _, _, _ in codes)
        halved += sum(h == 2 for _, h, _, _ in codes)
    assert halved > 0


def test_tile_rows_split_each_expert_evenly(split_exe):
    """An expert's M-tiles (moe_split.h tile_rows, used by both grouped GEMMs' item decode): ceil(rows / bm)
    tiles that cover the rows in order, exactly once, each starting on a 32-row block and holding 1 .. bm/32
    blocks, block counts that differ by at most one between tiles, and ceil(rows / 32) blocks in total (as many
    32-row MFMA blocks as bm, bm, ..., remainder tiles have)."""
    rng = np.random.default_rng(11)
    cases = [(r, bm) for bm in (128, 256) for r in range(1, 1100)]
    cases += [(int(r), bm) for bm in (128, 256) for r in rng.integers(1, 1 << 22, size=200)]
    cases += [(bm * bm + d, bm) for bm in (128, 256) for d in (-1, 0, 1)] + [((1 << 24) - 1, 256), (1 << 24, 128)]
    text = "".join(f"R {r} {bm}\n" for r, bm in cases)
    out = subprocess.run([str(split_exe)], input=text, capture_output=True, text=True, check=True).stdout
    tiles, cur = [], []
    for line in out.strip().splitlines():
        if line == "END":
            tiles.append(cur)
            cur = []
        else:
            cur.append(tuple(map(int, line.split())))
    assert len(tiles) == len(cases)
    for (rows, bm), ts in zip(cases, tiles):
        assert len(ts) == -(-rows // bm), (rows, bm)
        nxt = 0
        for rb, r in ts:
            assert rb == nxt and rb % 32 == 0 and 1 <= r <= bm, (rows, bm, rb, r)
            nxt = rb + r
        assert nxt == rows
        blocks = [-(-r // 32) for _, r in ts]
        assert sum(blocks) == -(-rows // 32) and max(blocks) - min(blocks) <= 1, (rows, bm, blocks)
