"""C ABI checks that need no GPU: the library loads, exports every function the header declares,
reports workspace sizes, and rejects bad arguments before touching the device."""

from __future__ import annotations

import ctypes

import pytest

from cernels_amd import _native


@pytest.fixture(scope="module")
def L():
    import torch  # noqa: F401  (the library binds to the HIP runtime torch loads)

    return _native.lib()


def test_every_declared_symbol_is_exported(L):
    names = _native.header_functions()
    assert len(names) >= 16
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(_native._SIGNATURES), "ctypes signature table out of sync with the header"


def test_no_undeclared_c_symbols_are_exported(L):
    """The library's unmangled (C-linkage) exports are exactly the header's functions: no internal helper
    leaks into the ABI a binding could come to depend on."""
    import shutil
    import subprocess

    if shutil.which("nm") is None:
        pytest.skip("nm not available")
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {parts[2] for parts in (line.split() for line in out.splitlines())
                if len(parts) == 3 and parts[1] == "T" and not parts[2].startswith("_Z")}
    assert exported == set(_native.header_functions()), sorted(exported ^ set(_native.header_functions()))


def test_version_and_status_strings(L):
    assert b"gfx950" in L.cernels_moe_version()
    for code, text in _native.STATUS.items():
        assert L.cernels_moe_status_string(code).decode() == text


def test_workspace_sizes(L):
    a = L.cernels_moe_experts_workspace_bytes(2048, 1280, 896, 64, 6)
    b = L.cernels_moe_experts_workspace_bytes(4096, 1280, 896, 64, 6)
    P = 2048 * 6
    assert a >= P * 896 * 4 + P * 1280 * 3  # glu as bf16 pairs + weighted down rows as 24-bit floats
    assert b > a
    assert L.cernels_moe_experts_workspace_bytes(-1, 1280, 896, 64, 6) == 0
    assert L.cernels_moe_experts_decode_workspace_bytes(1, 2048, 768, 128, 8) >= 8 * 768 * 2  # glu bf16
    assert L.cernels_moe_route_tile_capacity(2048, 6, 64, 128) == 96 + 64
    assert L.cernels_moe_route_tile_capacity(1, 8, 128, 128) == 1 + 8


def _fake(n=0x10000):
    return ctypes.c_void_p(n)


def _call(L, T=4, H=128, F=64, E=8, K=2, layout=0, act=0, ws_bytes=1 << 30, x=None, decode=False, E_over=False):
    p = _fake()
    fn = L.cernels_moe_experts_decode if decode else L.cernels_moe_experts
    return fn(x or p, p, None, p, None, p, p, T, H, F, E, K, layout, act, p, p, ctypes.c_size_t(ws_bytes), None)


def test_argument_checks_return_before_launch(L):
    assert _call(L, T=0) == 0  # no-op
    assert _call(L, T=-1) == 1
    assert _call(L, layout=7) == 1
    assert _call(L, act=9) == 1
    assert _call(L, H=96) == 2  # prefill needs H % 64 == 0
    assert _call(L, E=2000) == 2
    assert _call(L, x=_fake(0x10002)) == 3  # misaligned
    assert _call(L, ws_bytes=16) == 4
    assert _call(L, decode=True, layout=1) == 2  # decode is concat-only
    assert _call(L, decode=True, T=65) == 2
    assert _call(L, decode=True, T=64, K=5) == 2  # > 256 pairs
    assert _call(L, decode=True, H=4104) == 2


def test_null_pointers_rejected(L):
    p = _fake()
    st = L.cernels_moe_experts(None, p, None, p, None, p, p, 4, 128, 64, 8, 2, 0, 0, p, p, ctypes.c_size_t(1 << 30),
                               None)
    assert st == 1
    big = ctypes.c_size_t(1 << 20)
    st = L.cernels_moe_route(None, 4, 2, 8, 128, p, p, p, p, p, p, big, None)
    assert st == 1
    st = L.cernels_moe_route(p, 4, 2, 2048, 128, p, p, p, p, p, p, big, None)
    assert st == 1  # E > 1024
    st = L.cernels_moe_route(p, 4096, 10, 512, 128, p, p, p, p, p, p, ctypes.c_size_t(16), None)
    assert st == 4  # workspace too small
    assert L.cernels_moe_route_workspace_bytes(4096, 10, 512) == 40 * 512 * 4


def test_per_model_entries_check_arguments(L):
    p = _fake()
    ws = ctypes.c_size_t(16)
    for name in ("cernels_cohere2_moe_experts", "cernels_deepseek_ocr2_moe_experts", "cernels_qwen3_next_moe_experts"):
        assert getattr(L, name)(p, p, p, p, p, 4, 128, 64, 8, 2, p, p, ws, None) == 4
    for name in ("cernels_cohere2_moe_experts_decode", "cernels_deepseek_ocr2_moe_experts_decode"):
        assert getattr(L, name)(p, p, p, p, p, 4, 128, 64, 8, 2, p, p, ws, None) == 4
    assert L.cernels_gpt_oss_moe_experts(p, p, p, p, p, p, p, 4, 128, 64, 8, 2, p, p, ws, None) == 4


def test_noalloc_decode_refuses_what_the_decode_entry_refuses(L):
    """The allocation-free entry runs the decode entry's checks, in its order, before its scratch-size
    check: every refused call returns the decode entry's status, whatever F is."""
    p = _fake()
    cases = [dict(T=1, F=128, K=257), dict(T=1, F=4096, K=257), dict(T=65, F=4096, K=1), dict(T=4, F=4104, K=2),
             dict(T=4, F=64, K=2, layout=1), dict(T=-1, F=64, K=2), dict(T=4, F=64, K=2, act=9)]
    for c in cases:
        args = (p, p, None, p, None, p, p, c["T"], 256, c["F"], 8, c["K"], c.get("layout", 0), c.get("act", 0), p)
        want = L.cernels_moe_experts_decode(*args, p, ctypes.c_size_t(1 << 40), None)
        assert want != 0, c
        assert L.cernels_moe_experts_decode_noalloc(*args, None) == want, c
    mis = (_fake(0x10002), p, None, p, None, p, p, 1, 256, 128, 8, 2, 0, 0, p)
    assert L.cernels_moe_experts_decode_noalloc(*mis, None) == 3  # misaligned x, as the decode entry says
    assert L.cernels_moe_experts_decode_noalloc(p, p, None, p, None, p, p, 0, 256, 128, 8, 2, 0, 0, p, None) == 0
