"""ctypes binding of the in-tree HIP library (``liblkamd.so``).

The library exposes the C ABI declared in ``include/lk_w4a16.h``. This module
declares each entry point's argument types once, and :func:`call` turns a
non-zero status into ``RuntimeError`` with the library's message. There is no
fallback: if the library is missing, every kernel call raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "liblkamd.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int

# name -> argument types (every entry point returns int status)
SIGNATURES: dict[str, list] = {
    "lk_w4a16_quantise": [_P, _P, _P, _I64, _I64, _I64, _P],
    "lk_w4a16_dequantise": [_P, _P, _P, _I64, _I64, _I64, _I, _P],
    "lk_w4a16_dense": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_dense_reference": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_grouped": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_grouped_reference": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_swiglu": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "lk_silu_mul": [_P, _P, _P, _I64, _P],
    "lk_route_combine": [_P, _P, _P, _I64, _I64, _I64, _P],
    "lk_w4a16_w2_combine": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "lk_moe_router": [_P, _P, _P, _P, _I64, _I64, _I64, _F, _I, _P],
    "lk_moe_router_grouped": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _P],
    "lk_router_logits": [_P, _P, _P, _I64, _I64, _I64, _I, _P],
    "lk_w4a16_moe_gateup": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            _I64, _I64, _I64, _I64, _I64, _F, _I, _I64, _P],
    "lk_w4a16_moe_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            _I64, _I64, _I64, _I64, _I64, _F, _I, _I64, _P],
    "lk_moe_schedule_sizes": [_I64, _I64, _I64, _P, _P],
    "lk_moe_schedule": [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P],
    "lk_w4a16_grouped_gemm": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                              _P, _I64, _P],
    "lk_w4a16_swiglu_gemm": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                             _P, _I64, _P],
    "lk_w4a16_dense_gemm": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_fused_qkv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "lk_w4a16_dense_gemm_ws": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "lk_w4a16_fused_qkv_ws": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                              _P, _I64, _P],
    "lk_w4a16_moe_forward": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                             _I64, _I64, _I64, _I64, _I64, _F, _I, _I64, _P],
    "lk_w4a16_moe_forward_static": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _I64, _I64, _I64, _I64, _I64, _F, _I, _I64, _P],
    "lk_mxfp4_quantise": [_P, _P, _P, _I64, _I64, _P],
    "lk_mxfp4_dequantise": [_P, _P, _P, _I64, _I64, _I, _P],
    "lk_mxfp4_gemm": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P],
    "lk_mxfp4_gemm_reference": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P],
    "lk_mxfp4_grouped_gemm": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "lk_mxfp4_swiglu_gemm": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                             _P, _I64, _P],
    "lk_mxfp4_moe_forward": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                             _I64, _I64, _I64, _I64, _I64, _F, _I, _P],
    "lk_mxfp4_expert_mlp": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _F, _P],
    "lk_mxfp4_split_activations": [_P, _P, _P, _P, _I64, _I64, _P],
    "lk_kda_decode_step": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _P],
    "lk_kda_short_conv_triple": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                 _I, _I, _P],
    "lk_kda_gates": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _I, _I,
                     _I, _P],
    "lk_kda_decode_layer": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            _I64, _I64, _I64, _F, _F, _I, _I, _I, _I, _P],
    "lk_kda_decode_layer_split": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                  _P, _P, _P, _I64, _I64, _I64, _F, _F, _I, _I, _I, _I, _P],
    "lk_rms_norm": [_P, _P, _P, _I64, _I64, _F, _I, _I, _P],
    "lk_add_rms_norm": [_P, _P, _P, _P, _P, _I64, _I64, _F, _I, _I, _P],
    "lk_rms_gated_norm": [_P, _P, _P, _P, _I64, _I64, _F, _I, _I, _I, _I, _P],
}

# name -> argument types of the size queries (they return int64, -1 on bad input)
QUERIES: dict[str, list] = {
    "lk_w4a16_moe_decode_workspace": [_I64, _I64, _I64, _I64, _I64],
    "lk_w4a16_moe_forward_static_capacity": [],
    "lk_w4a16_dense_gemm_workspace": [_I64, _I64, _I64],
    "lk_w4a16_grouped_gemm_workspace": [_I64, _I64, _I64],
    "lk_w4a16_moe_forward_workspace": [_I64, _I64, _I64, _I64, _I64],
    "lk_mxfp4_moe_forward_workspace": [_I64, _I64, _I64, _I64, _I64],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return LIB_PATH


def is_built() -> bool:
    return os.path.exists(LIB_PATH)


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"the HIP library {LIB_PATH} is not built; run "
                    "`python -m local_kimi_amd._build` (hipcc, gfx950) first"
                )
            lib = ctypes.CDLL(LIB_PATH)
            lib.lk_last_error.restype = ctypes.c_char_p
            lib.lk_last_error.argtypes = []
            lib.lk_abi_version.restype = ctypes.c_int
            lib.lk_abi_version.argtypes = []
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = ctypes.c_int
                fn.argtypes = argtypes
            lib.lk_set_path.restype = ctypes.c_int
            lib.lk_set_path.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
            lib.lk_get_path.restype = ctypes.c_int
            lib.lk_get_path.argtypes = [ctypes.c_char_p]
            for name, argtypes in QUERIES.items():
                fn = getattr(lib, name)
                fn.restype = ctypes.c_int64
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.lk_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {status}): {message}")


def query(name: str, *args) -> int:
    """Call a size query; raise ValueError when it rejects the dimensions."""
    value = int(getattr(load(), name)(*args))
    if value < 0:
        raise ValueError(f"{name}: invalid dimensions {args}")
    return value


def schedule_sizes(tokens: int, routes: int, experts: int) -> tuple[int, int]:
    """``(max_tiles, workspace_bytes)`` of :c:func:`lk_moe_schedule`."""
    max_tiles, ws = ctypes.c_int64(), ctypes.c_int64()
    call("lk_moe_schedule_sizes", tokens, routes, experts, ctypes.addressof(max_tiles),
         ctypes.addressof(ws))
    return max_tiles.value, ws.value


# kernel-form knobs of lk_set_path and their choices ("auto" first)
PATH_KNOBS: dict[str, tuple[str, ...]] = {
    "moe_gemm": ("auto", "lds", "stream16", "stream64"),
    "moe_persist": ("auto", "off"),
    "dense_gemm": ("auto", "lds"),
    "mxfp4_mfma": ("auto", "fp4", "bf16"),
    "moe_fused_schedule": ("auto", "off"),
    "moe_split_swiglu": ("auto", "off"),
}


def set_path(knob: str, choice: str) -> None:
    """Force one of the library's kernel forms for this process (see lk_set_path)."""
    lib = load()
    if lib.lk_set_path(knob.encode(), choice.encode()) != 0:
        raise ValueError(lib.lk_last_error().decode(errors="replace"))


def get_path(knob: str) -> str:
    index = load().lk_get_path(knob.encode())
    if index < 0:
        raise ValueError(f"unknown path knob {knob!r}")
    return PATH_KNOBS[knob][index]


@contextlib.contextmanager
def forced_path(knob: str, choice: str):
    """Run the body with one kernel form forced, then restore the previous choice."""
    previous = get_path(knob)
    set_path(knob, choice)
    try:
        yield
    finally:
        set_path(knob, previous)


def exported_symbols() -> list[str]:
    """Entry points this binding expects the library to export."""
    return ["lk_last_error", "lk_abi_version", "lk_set_path", "lk_get_path", *SIGNATURES,
            *QUERIES]
