"""The C-ABI library loads and exports every entry point include/lk_w4a16.h
declares (no compute calls: this runs without a GPU)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from local_kimi_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


PROBE_HEADER = "lk_probe.h"  # the benchmark's probe library, not the product library


def _declared(probe: bool = False) -> list[str]:
    names = []
    for header in os.listdir(os.path.join(ROOT, "include")):
        if header.endswith(".h") and (header == PROBE_HEADER) == probe:
            text = open(os.path.join(ROOT, "include", header)).read()
            names += re.findall(r"LK_API\s+[\w\s\*]+?\b(lk_\w+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not _lib.is_built():
        pytest.skip("library not built; run python -m local_kimi_amd._build")
    return _lib.load()


def test_header_declares_the_entry_points_the_binding_uses():
    declared = _declared()
    assert declared, "no LK_API declarations found"
    assert sorted(_lib.exported_symbols()) == declared


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_probe_library_is_separate_and_exports_its_symbols(lib):
    path = os.path.join(ROOT, "local_kimi_amd", "liblkprobe.so")
    if not os.path.exists(path):
        pytest.skip("probe library not built")
    probe = ctypes.CDLL(path)
    names = _declared(probe=True)
    assert names == ["lk_probe_empty", "lk_probe_last_error", "lk_probe_stream_read"]
    for name in names:
        assert isinstance(getattr(probe, name), ctypes._CFuncPtr), name
        with pytest.raises(AttributeError):
            getattr(lib, name)  # the product library does not carry the probes
    probe.lk_probe_stream_read.restype = ctypes.c_int
    probe.lk_probe_last_error.restype = ctypes.c_char_p
    # argument errors are reported on the host, before any launch
    assert probe.lk_probe_stream_read(None, None, 0, None, None) == 1
    assert b"null pointer" in probe.lk_probe_last_error()


def test_abi_version_and_error_string(lib):
    assert lib.lk_abi_version() == 2
    assert isinstance(lib.lk_last_error(), bytes)


def test_argument_errors_are_reported_without_touching_the_gpu(lib):
    # k=100 is not divisible by the group size: rejected on the host before any launch
    with pytest.raises(RuntimeError, match="divisible"):
        _lib.call("lk_w4a16_dense", 1, 1, 1, 1, 1, 8, 100, 32, None)
    with pytest.raises(RuntimeError, match="power of two"):
        _lib.call("lk_w4a16_dense", 1, 1, 1, 1, 1, 8, 192, 96, None)
    with pytest.raises(RuntimeError, match="top_k"):
        _lib.call("lk_moe_router", 1, None, 1, 1, 1, 4, 9, 1.0, 1, None)


def test_dense_workspace_sizes_and_refusals(lib):
    # paired rows (2 bytes per value) + group sums (4 bytes per 128 values), 256-byte aligned
    assert lib.lk_w4a16_dense_gemm_workspace(2048, 2304, 128) == 2048 * 2304 * 2 + 2048 * 18 * 4
    assert lib.lk_w4a16_dense_gemm_workspace(8, 2304, 128) == 0     # decode rows: the GEMV
    assert lib.lk_w4a16_dense_gemm_workspace(2048, 2304, 64) == 0   # other groups: staged rows
    assert lib.lk_w4a16_dense_gemm_workspace(-1, 2304, 128) == -1
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_w4a16_dense_gemm_ws", 1, 1, 1, 1, 64, 256, 512, 128, 1, 16, None)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_w4a16_fused_qkv_ws", 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 64, 256, 512, 128,
                  None, 0, None)


def test_grouped_router_argument_errors(lib):
    # (logits, bias, idx, w, tokens, experts, top_k, groups, topk_group, scale, renorm, stream)
    with pytest.raises(RuntimeError, match="divisible"):
        _lib.call("lk_moe_router_grouped", 1, None, 1, 1, 1, 10, 2, 4, 1, 1.0, 1, None)
    with pytest.raises(RuntimeError, match="topk_group"):
        _lib.call("lk_moe_router_grouped", 1, None, 1, 1, 1, 16, 2, 4, 5, 1.0, 1, None)
    with pytest.raises(RuntimeError, match="num_expert_group"):
        _lib.call("lk_moe_router_grouped", 1, None, 1, 1, 1, 256, 2, 128, 1, 1.0, 1, None)
    with pytest.raises(RuntimeError, match="experts"):
        _lib.call("lk_moe_router_grouped", 1, None, 1, 1, 1, 2048, 2, 8, 1, 1.0, 1, None)
    with pytest.raises(RuntimeError, match="top_k"):
        _lib.call("lk_moe_router_grouped", 1, None, 1, 1, 1, 16, 40, 4, 1, 1.0, 1, None)
    # no tokens: nothing to launch, no pointers needed
    assert lib.lk_moe_router_grouped(None, None, None, None, 0, 16, 2, 4, 2,
                                     ctypes.c_float(1.0), 1, None) == 0


def test_expert_major_sizes_and_argument_errors(lib):
    max_tiles, ws = _lib.schedule_sizes(2048, 9, 257)
    # prefill bound for the smaller (16-row) tiles: min(E + 1, n) + n / 16 + 1
    assert max_tiles == 258 + 18432 // 16 + 1
    assert ws >= 18432 * 4
    assert _lib.query("lk_w4a16_moe_forward_workspace", 64, 257, 2304, 1024, 8) > 0
    assert lib.lk_w4a16_moe_forward_workspace(64, 1000, 2304, 1024, 8) == -1
    assert lib.lk_w4a16_grouped_gemm_workspace(4, 0, 8) == -1
    with pytest.raises(RuntimeError, match="experts"):
        _lib.schedule_sizes(4, 8, 600)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_moe_schedule", 1, 4, 8, 16, -1, 64, 1, 1, 1, 1, 1, 8, None)
    with pytest.raises(RuntimeError, match="tile rows"):
        _lib.call("lk_moe_schedule", 1, 4, 8, 16, -1, 32, 1, 1, 1, 1, 1, 1 << 20, None)
    with pytest.raises(RuntimeError, match="divisible"):
        _lib.call("lk_w4a16_dense_gemm", 1, 1, 1, 1, 16, 8, 100, 32, None)


def test_workspace_sizes_are_checked_before_any_launch(lib):
    """Every entry point that writes a caller-owned workspace refuses one
    smaller than its size query, before touching device memory (the pointers
    here are never dereferenced)."""
    need = _lib.query("lk_w4a16_moe_forward_workspace", 64, 257, 2304, 1024, 8)
    # 13 device pointers, then workspace_bytes one short of the query
    args = [1] * 13 + [need - 1, 64, 257, 2304, 1024, 8, 1.0, 1, 128, None]
    with pytest.raises(RuntimeError, match="MoE workspace too small"):
        _lib.call("lk_w4a16_moe_forward", *args)
    gneed = _lib.query("lk_w4a16_grouped_gemm_workspace", 64, 9, 257)
    assert gneed > 0
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_w4a16_grouped_gemm", 1, 1, 1, 1, 1, 64, 9, 257, 2304, 1024, 128, 1,
                  gneed - 1, None)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_w4a16_swiglu_gemm", 1, 1, 1, 1, 1, 1, 1, 64, 9, 257, 1024, 2304, 128, 1,
                  gneed - 1, None)
    mxneed = _lib.query("lk_mxfp4_moe_forward_workspace", 64, 257, 2304, 1024, 8)
    margs = [1] * 13 + [mxneed - 1, 64, 257, 2304, 1024, 8, 1.0, 1, None]
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("lk_mxfp4_moe_forward", *margs)


def test_path_knobs_select_and_reject(lib):
    for knob, choices in _lib.PATH_KNOBS.items():
        assert _lib.get_path(knob) == "auto"
        for choice in choices:
            with _lib.forced_path(knob, choice):
                assert _lib.get_path(knob) == choice
        assert _lib.get_path(knob) == "auto"
    with pytest.raises(ValueError, match="unknown path knob"):
        _lib.set_path("no_such_knob", "auto")
    with pytest.raises(ValueError, match="unknown choice"):
        _lib.set_path("moe_gemm", "fastest")
    assert lib.lk_get_path(b"no_such_knob") == -1


def test_token_major_decode_route_limit_is_checked_before_any_launch(lib):
    # top_k = 32 -> 33 routes at intermediate 1024: the token-major W2 launch
    # cannot take it; the call is refused on the host (null device pointers are
    # never dereferenced) and the workspace query reports -1
    assert lib.lk_w4a16_moe_decode_workspace(1, 257, 2304, 1024, 32) == -1
    assert lib.lk_w4a16_moe_decode_workspace(4, 257, 2304, 1024, 8) == 4 * 9 * 1024 * 2
    assert lib.lk_w4a16_moe_decode_workspace(1, 257, 2304, 4096, 8) == -1  # I = 4096: LDS
    with pytest.raises(RuntimeError, match="token-major W2"):
        _lib.call("lk_w4a16_moe_decode", 1, 1, None, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                  1, 257, 2304, 1024, 32, 1.0, 1, 128, None)


def test_static_scratch_entry_point_refuses_oversized_calls_on_the_host(lib):
    # 161 Kimi-Linear tokens need more than the static scratch holds: refused
    # before the device is touched (null device pointers are never read)
    cap = lib.lk_w4a16_moe_forward_static_capacity()
    assert cap == 12 << 20
    assert lib.lk_w4a16_moe_forward_workspace(160, 257, 2304, 1024, 8) <= cap
    assert lib.lk_w4a16_moe_forward_workspace(161, 257, 2304, 1024, 8) > cap
    with pytest.raises(RuntimeError, match="static scratch holds"):
        _lib.call("lk_w4a16_moe_forward_static", 1, 1, None, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                  161, 257, 2304, 1024, 8, 1.0, 1, 128, None)
