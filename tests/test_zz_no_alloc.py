"""The allocation-free decode entry (cernels_moe_experts_decode_noalloc), through the C ABI.

It runs the decode kernels on the library's static per-GPU scratch instead of a caller workspace.
Bar: bit-identical to cernels_moe_experts_decode (same kernels, same order of operations) on two
calls in a row, the second with a smaller input (the scratch keeps the first call's contents), plus
the fp64 oracle's tolerance on each; and the size check: a shape beyond the decode limits is
rejected before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import assert_within_tolerance, oracle_fp64, rand_case, to_device

pytestmark = pytest.mark.gpu


def _decode(L, d, noalloc, device):
    T, H = map(int, d["x"].shape)
    K = int(d["idx"].shape[1])
    E, F2, _ = map(int, d["W1"].shape)
    F = F2 // 2
    out = torch.empty(T, H, dtype=torch.bfloat16, device=device)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = torch.cuda.current_stream(device).cuda_stream
    args = (p(d["x"]), p(d["W1"]), p(d["b1"]), p(d["W2"]), p(d["b2"]), p(d["idx"]), p(d["w"]), T, H, F, E, K, 0, 0,
            p(out))
    if noalloc:
        st = L.cernels_moe_experts_decode_noalloc(*args, stream)
    else:
        nbytes = L.cernels_moe_experts_decode_workspace_bytes(T, H, F, E, K)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        st = L.cernels_moe_experts_decode(*args, p(ws), ctypes.c_size_t(nbytes), stream)
    assert st == 0, L.cernels_moe_status_string(st)
    torch.cuda.synchronize()
    return out.cpu()


def test_noalloc_decode_matches_decode_entry(device):
    from cernels_amd import _native

    L = _native.lib()
    first = rand_case(21, 8, 1280, 896, 64, 6)   # the decode T=8 shape: 48 pairs
    second = rand_case(22, 3, 1280, 896, 64, 4)  # smaller: 12 pairs, on the scratch the first call left
    for name, c in (("first", first), ("second", second)):
        print(f"[noalloc {name}]", flush=True)
        d = to_device(c, device)
        got = _decode(L, d, True, device)
        want = _decode(L, d, False, device)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{name}: differs from the decode entry"
        assert_within_tolerance(got, oracle_fp64(c), f"noalloc {name}")


def test_noalloc_decode_rejects_shapes_beyond_the_limits(device):
    from cernels_amd import _native

    L = _native.lib()
    T, H, F, E = 1, 256, 128, 8
    K = L.cernels_moe_decode_max_pairs() + 1  # T*K beyond the decode limit: rejected before any launch
    st = L.cernels_moe_experts_decode_noalloc(ctypes.c_void_p(16), ctypes.c_void_p(16), None, ctypes.c_void_p(16),
                                              None, ctypes.c_void_p(16), ctypes.c_void_p(16), T, H, F, E, K, 0, 0,
                                              ctypes.c_void_p(16), torch.cuda.current_stream(device).cuda_stream)
    assert st == 2, L.cernels_moe_status_string(st)  # CERNELS_MOE_UNSUPPORTED_SHAPE
