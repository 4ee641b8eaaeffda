"""W4A16 checkpoints on disk and the bank builder (CPU).

The layout and its checks follow engine/klinear/weights.py:34-35, 130-143,
188-320 and 599-626; this build reads the group size from the index metadata
(32 when absent, as in the reference, or any power-of-two multiple of 32).
Round trips are bit-exact against the oracle's encoder; every index mistake
the reference rejects raises the same exception type here. The bank builder
follows engine/klinear/moe.py:224-276: routed experts in id order, then the
shared expert (gate_proj -> W1, up_proj -> W3, down_proj -> W2).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from local_kimi_amd.checkpoint import (INDEX_NAME, PACKED_SUFFIX, SCALES_SUFFIX, W4A16Index,
                                       build_moe_banks, expert_name, parse_index,
                                       save_w4a16_checkpoint, shared_expert_name)
from local_kimi_amd.quant.w4a16 import W4A16Tensor
from oracle import w4a16 as OW

from ._helpers import from_bits, random_bf16_bits, to_bits


def _encode(rng, n, k, g):
    p, s = OW.quantise(random_bf16_bits(rng, (n, k), 0.02), g)
    return W4A16Tensor(packed=torch.from_numpy(p), scales=from_bits(s), original_shape=(n, k),
                       group_size=g), p, s


@pytest.mark.parametrize("g", [32, 128])
def test_round_trip_is_bit_exact_with_shards(tmp_path, rng, g):
    a, pa, sa = _encode(rng, 96, 256, g)
    b, pb, sb = _encode(rng, 40, 512, g)
    router = torch.from_numpy(rng.normal(0, 1, (8, 256)).astype(np.float32))
    save_w4a16_checkpoint(tmp_path, {"layer.a.weight": a, "layer.b.weight": b, "router.weight": router},
                          shard_bytes=8 << 10)
    payload = json.loads((tmp_path / INDEX_NAME).read_text())
    assert payload["metadata"] == {"quantization": "W4A16", "group_size": g, "scale_dtype": "BF16"}
    assert len(set(payload["weight_map"].values())) > 1  # really sharded
    idx = W4A16Index(tmp_path)
    assert idx.quantized and idx.group_size == g
    got = idx.load_w4a16("layer.a.weight", (96, 256), device="cpu")
    assert got.group_size == g
    assert np.array_equal(got.packed.numpy(), pa) and np.array_equal(to_bits(got.scales), sa)
    got = idx.load_w4a16("layer.b.weight", (40, 512), device="cpu")
    assert np.array_equal(got.packed.numpy(), pb) and np.array_equal(to_bits(got.scales), sb)
    assert torch.equal(idx.load("router.weight"), router)
    assert idx.spec("layer.a.weight" + PACKED_SUFFIX) == ((96, 128), "U8")


def test_group_size_defaults_to_the_reference_group(tmp_path, rng):
    a, pa, _ = _encode(rng, 16, 64, 32)
    save_w4a16_checkpoint(tmp_path, {"w": a})
    payload = json.loads((tmp_path / INDEX_NAME).read_text())
    del payload["metadata"]["group_size"]
    (tmp_path / INDEX_NAME).write_text(json.dumps(payload))
    idx = W4A16Index(tmp_path)
    assert idx.group_size == 32
    assert np.array_equal(idx.load_w4a16("w", (16, 64), device="cpu").packed.numpy(), pa)


_PAIR = {"a.w4a16_packed": "s.safetensors", "a.w4a16_scales": "s.safetensors"}


@pytest.mark.parametrize("payload,match", [
    ({"weight_map": {}}, "no weight_map"),
    ({"weight_map": {"a": ""}}, "non-empty string pairs"),
    ({"weight_map": {"a": "s"}, "metadata": []}, "metadata must be an object"),
    ({"weight_map": {"a": "s"}, "metadata": {"quantization": "W8A8"}}, "unsupported checkpoint quantization"),
    ({"weight_map": {"a": "s"}, "metadata": {"quantization": "W4A16"}}, "declares quantization but has no packed"),
    ({"weight_map": {"a.w4a16_bogus": "s"}}, "unrecognized W4A16 tensor names"),
    ({"weight_map": {"a.w4a16_packed": "s"}}, "incomplete packed and scale pairs"),
    ({"weight_map": {**_PAIR, "a": "s.safetensors"}}, "packed and BF16 copies"),
    ({"weight_map": _PAIR, "metadata": {"group_size": 48}}, "power-of-two multiple of 32"),
    ({"weight_map": _PAIR, "metadata": {"group_size": True}}, "power-of-two multiple of 32"),
    ({"weight_map": _PAIR, "metadata": {"scale_dtype": "F16"}}, "scale dtype must be BF16"),
])
def test_index_mistakes_are_rejected(payload, match):
    with pytest.raises(ValueError, match=match):
        parse_index(payload)


def test_missing_files_and_tensors(tmp_path, rng):
    with pytest.raises(FileNotFoundError, match="index is missing"):
        W4A16Index(tmp_path)
    a, _, _ = _encode(rng, 16, 64, 32)
    save_w4a16_checkpoint(tmp_path, {"w": a})
    idx = W4A16Index(tmp_path)
    with pytest.raises(KeyError, match="absent"):
        idx.load("nope")
    with pytest.raises(ValueError, match="must be U8"):
        idx.load_w4a16("w", (16, 128), device="cpu")
    with pytest.raises(ValueError, match="divisible by 32"):
        idx.load_w4a16("w", (16, 48), device="cpu")
    payload = json.loads((tmp_path / INDEX_NAME).read_text())
    payload["weight_map"]["extra"] = "gone.safetensors"
    (tmp_path / INDEX_NAME).write_text(json.dumps(payload))
    with pytest.raises(FileNotFoundError, match="shard is missing"):
        W4A16Index(tmp_path)


def test_plain_checkpoint_is_not_w4a16(tmp_path):
    save_w4a16_checkpoint(tmp_path, {"x": torch.zeros(4, 4)})
    idx = W4A16Index(tmp_path)
    assert not idx.quantized
    with pytest.raises(ValueError, match="not W4A16"):
        idx.load_w4a16("x", (4, 4), device="cpu")


def test_one_checkpoint_holds_one_group_size(tmp_path, rng):
    a, _, _ = _encode(rng, 16, 128, 32)
    b, _, _ = _encode(rng, 16, 128, 128)
    with pytest.raises(ValueError, match="one group size"):
        save_w4a16_checkpoint(tmp_path, {"a": a, "b": b})


def test_bank_builder_order(tmp_path, rng):
    layer, experts, hidden, inter, g = 3, 4, 256, 128, 128
    tensors, want = {}, {"w1": [], "w3": [], "w2": []}
    shared = {"w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}
    for e in range(experts + 1):
        for bank, (n, k) in (("w1", (inter, hidden)), ("w3", (inter, hidden)), ("w2", (hidden, inter))):
            t, p, s = _encode(rng, n, k, g)
            name = expert_name(layer, e, bank) if e < experts else shared_expert_name(layer, shared[bank])
            tensors[name] = t
            want[bank].append((p, s))
    save_w4a16_checkpoint(tmp_path, tensors, shard_bytes=64 << 10)
    banks = build_moe_banks(W4A16Index(tmp_path), layer, num_experts=experts, hidden=hidden,
                            intermediate=inter, device="cpu")
    got = {"w1": (banks.w1_packed, banks.w1_scales), "w3": (banks.w3_packed, banks.w3_scales),
           "w2": (banks.w2_packed, banks.w2_scales)}
    for bank in ("w1", "w3", "w2"):
        packed, scales = got[bank]
        assert packed.shape[0] == experts + 1 and packed.is_contiguous()
        for e, (p, s) in enumerate(want[bank]):
            assert np.array_equal(packed[e].numpy(), p), (bank, e)
            assert np.array_equal(to_bits(scales[e]), s), (bank, e)
    with pytest.raises(KeyError, match="absent"):
        build_moe_banks(W4A16Index(tmp_path), layer + 1, num_experts=experts, hidden=hidden,
                        intermediate=inter, device="cpu")
