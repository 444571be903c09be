"""ctypes binding of libcernels_moe.so (the C ABI declared in include/cernels_moe.h).

The library is built in-tree by ``python -m cernels_amd.build``. Nothing here falls back to
another implementation: if the library is missing or a call fails, a ``RuntimeError`` is raised.
Import torch before loading so the library binds to the HIP runtime torch already loaded
(both carry the soname libamdhip64.so.7, so the process keeps a single runtime).
"""

from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libcernels_moe.so")
HEADER = Path(__file__).resolve().parents[1] / "include" / "cernels_moe.h"

STATUS = {
    0: "ok",
    1: "invalid argument",
    2: "unsupported shape",
    3: "tensor pointer not 16-byte aligned",
    4: "workspace too small",
    5: "HIP kernel launch failed",
}
LAYOUT_CONCAT, LAYOUT_INTERLEAVED = 0, 1
ACT_SILU, ACT_GPTOSS = 0, 1
ACT_GELU_TANH, ACT_SILU_PLAIN, ACT_RELU = 2, 3, 4  # non-gated (megablocks)
GATE_UP, DOWN, UP = 0, 1, 2
ROUTER_SOFTMAX_TOPK, ROUTER_TOPK_SOFTMAX = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int32
_S = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "cernels_moe_version": (ctypes.c_char_p, []),
    "cernels_moe_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "cernels_moe_route_tile_capacity": (_S, [_I, _I, _I, _I]),
    "cernels_moe_route_workspace_bytes": (_S, [_I, _I, _I]),
    "cernels_moe_route": (ctypes.c_int, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _S, _P]),
    "cernels_moe_experts_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "cernels_moe_experts": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_moe_experts_staged": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P, _P],
    ),
    "cernels_moe_experts_decode_staged": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P, _P],
    ),
    "cernels_moe_packed_weight_bytes": (_S, [_I, _I, _I, _I]),
    "cernels_moe_pack_weights": (ctypes.c_int, [_P, _I, _I, _I, _I, _I, _P, _P]),
    "cernels_moe_experts_packed": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P],
    ),
    "cernels_moe_experts_packed_staged": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P, _P],
    ),
    "cernels_moe_router": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "cernels_megablocks_moe_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "cernels_megablocks_moe": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_moe_decode_max_tokens": (_I, []),
    "cernels_moe_decode_max_pairs": (_I, []),
    "cernels_moe_experts_decode_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "cernels_moe_experts_decode_noalloc": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    ),
    "cernels_moe_experts_decode": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _S, _P],
    ),
    "cernels_cohere2_moe_experts": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_cohere2_moe_experts_decode": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_deepseek_ocr2_moe_experts": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_deepseek_ocr2_moe_experts_decode": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P],
    ),
    "cernels_qwen3_next_moe_experts": (ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P]),
    "cernels_gpt_oss_moe_experts": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _S, _P],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def header_functions() -> list[str]:
    """Function names declared in include/cernels_moe.h."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(cernels_[A-Za-z0-9_]+)\s*\(", text, flags=re.M)


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH.name} is not built; run `python -m cernels_amd.build` (hipcc, gfx950)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {STATUS.get(status, f'status {status}')}")
