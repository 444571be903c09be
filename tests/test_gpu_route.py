"""GPU routing parity: bit-exact offsets, permutation and tile list against the C restatement and
the numpy closed form; the golden torch.where order; every BASELINE config's routing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN_NAMES, load_golden
from oracle import eager as O

pytestmark = pytest.mark.gpu


def _gpu_route(idx, E, device, tile_m=128):
    from cernels_amd import ops

    d = torch.as_tensor(np.asarray(idx), dtype=torch.int32).contiguous().to(device)
    offs, pairs, toff, texp, meta = ops.route(d, E, tile_m)
    torch.cuda.synchronize()
    meta = meta.cpu().numpy()
    nv, nt = int(meta[1]), int(meta[0])
    return dict(offsets=offs.cpu().numpy(), sorted_pairs=pairs.cpu().numpy()[:nv], tile_offsets=toff.cpu().numpy(),
                tile_expert=texp.cpu().numpy()[:nt], num_tiles=nt, num_valid=nv)


def _assert_same(a, b):
    for k in ("offsets", "sorted_pairs", "tile_offsets", "tile_expert"):
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert (a["num_tiles"], a["num_valid"]) == (b["num_tiles"], b["num_valid"])


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_route_golden(device, name):
    t, meta = load_golden(name)
    r = _gpu_route(t["top_k_index"].numpy(), meta["E"], device)
    np.testing.assert_array_equal(r["sorted_pairs"], t["where_pairs"].numpy())


@pytest.mark.parametrize(
    "T,K,E,invalid",
    [(1, 1, 1, False), (1, 8, 128, False), (7, 3, 5, True), (333, 6, 64, True), (2048, 8, 128, False),
     (4096, 10, 512, True), (5000, 4, 1024, False), (3, 2, 1024, True),
     # past the one-launch route's LDS limit ((tiles + 16) * E > 39 Ki cells): the count+scan and scatter
     # launches, and above tiles * E > 28 Ki cells the separate count launch
     (6000, 4, 1024, True), (8192, 8, 1024, False)],
)
def test_route_random(device, T, K, E, invalid):
    rng = np.random.default_rng(T * 31 + K * 7 + E)
    lo, hi = (-3, E + 3) if invalid else (0, E)
    idx = rng.integers(lo, hi, size=(T, K))
    for tile_m in (128, 64, 1):
        _assert_same(_gpu_route(idx, E, device, tile_m), O.route_reference(idx, E, tile_m))


@pytest.mark.parametrize("T,K,E,shift", [(333, 6, 64, 1), (2047, 3, 128, 3), (4095, 10, 512, 2)])
def test_route_unaligned_indices(device, T, K, E, shift):
    """indices starting 4*shift bytes into an allocation (a contiguous slice), T*K not a multiple of 4:
    the histogram pass reads idx in 16-byte chunks whatever the pointer's alignment and masks the tail."""
    from cernels_amd import ops

    rng = np.random.default_rng(T + 17 * shift)
    idx = rng.integers(-2, E + 2, size=(T, K))
    buf = torch.zeros(T * K + shift, dtype=torch.int32, device=device)
    d = buf[shift:].view(T, K)
    d.copy_(torch.as_tensor(idx, dtype=torch.int32))
    assert d.data_ptr() % 16 != 0 and d.is_contiguous()
    offs, pairs, toff, texp, meta = ops.route(d, E, 128)
    torch.cuda.synchronize()
    m = meta.cpu().numpy()
    got = dict(offsets=offs.cpu().numpy(), sorted_pairs=pairs.cpu().numpy()[: int(m[1])],
               tile_offsets=toff.cpu().numpy(), tile_expert=texp.cpu().numpy()[: int(m[0])],
               num_tiles=int(m[0]), num_valid=int(m[1]))
    _assert_same(got, O.route_reference(idx, E, 128))


def test_route_skewed_single_expert(device):
    idx = np.zeros((4096, 10), dtype=np.int64)  # every pair on expert 0
    idx[::7, 3] = 511
    _assert_same(_gpu_route(idx, 512, device), O.route_reference(idx, 512))


def test_route_empty(device):
    r = _gpu_route(np.zeros((0, 4), dtype=np.int64), 16, device)
    assert r["num_valid"] == 0 and r["num_tiles"] == 0
    assert (r["offsets"] == 0).all()


def test_route_baseline_configs(device):
    from cernels_amd.configs.registry import BASELINE_SHAPES
    from cernels_amd.configs.synth import make_inputs

    for name, s in BASELINE_SHAPES.items():
        inp = make_inputs(s)
        idx = inp.top_k_index.numpy()
        _assert_same(_gpu_route(idx, s.experts, device), O.route_reference(idx, s.experts))


def test_route_deterministic(device):
    rng = np.random.default_rng(5)
    idx = rng.integers(0, 64, size=(2048, 6))
    a, b = _gpu_route(idx, 64, device), _gpu_route(idx, 64, device)
    _assert_same(a, b)
