"""W4A16 checkpoints on disk and the expert banks built from them.

The on-disk layout is the reference's (engine/klinear/weights.py:34-35,
130-143, 188-320, 599-626): Hugging Face sharded safetensors with an index
``model.safetensors.index.json`` (``weight_map`` name -> shard, ``metadata``);
a quantized matrix ``name`` is the pair ``name.w4a16_packed`` (U8 ``[N, K/2]``,
byte j = k 2j in the low nibble and 2j + 1 in the high nibble) and
``name.w4a16_scales`` (BF16 ``[N, K/G]``). The index metadata carries
``quantization`` ("W4A16"), ``group_size`` and ``scale_dtype`` ("BF16").

The reference accepts only ``group_size == 32`` (weights.py:290-294); this
reader takes any power-of-two multiple of 32 from the metadata (G = 128 is the
size the HIP kernels are measured at) and defaults to 32 when the metadata
does not say, as the reference does. Index errors raise the reference's
exception types for the same mistakes (ValueError for a malformed or
inconsistent index, FileNotFoundError for a missing index or shard, KeyError
for absent tensors).

:func:`build_moe_banks` is the counterpart of ``prepare_grouped_w4a16``
(engine/klinear/moe.py:224-276): the routed experts 0..E-1 of a layer, then the
shared expert last (its gate_proj in the W1 bank, up_proj in W3, down_proj in
W2), each bank allocated once on the device and filled expert by expert from
the memory-mapped shards.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Mapping

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .quant.w4a16 import SCALE_DTYPE, W4A16Tensor

PACKED_SUFFIX = ".w4a16_packed"
SCALES_SUFFIX = ".w4a16_scales"
INDEX_NAME = "model.safetensors.index.json"
DEFAULT_GROUP_SIZE = 32  # the reference's GROUP_SIZE (engine/quant/w4a16.py)

def _valid_group(g: object) -> bool:
    return isinstance(g, int) and not isinstance(g, bool) and g > 0 and g % 32 == 0 and not (g & (g - 1))


def _weight_map(payload: Mapping) -> dict[str, str]:
    weight_map = payload.get("weight_map")
    if not isinstance(weight_map, Mapping) or not weight_map:
        raise ValueError("safetensors index has no weight_map")
    if not all(isinstance(n, str) and n and isinstance(s, str) and s for n, s in weight_map.items()):
        raise ValueError("safetensors weight_map must contain non-empty string pairs")
    return dict(weight_map)


def parse_index(payload: Mapping) -> tuple[dict[str, str], bool, int]:
    """``(weight_map, quantized, group_size)`` of an index, after the checks of
    engine/klinear/weights.py:188-320 restricted to BF16 and W4A16 payloads."""
    if not isinstance(payload, Mapping):
        raise ValueError("safetensors index must contain an object")
    names = _weight_map(payload)
    metadata = payload.get("metadata")
    if metadata is None:
        metadata = {}
    if not isinstance(metadata, Mapping):
        raise ValueError("safetensors index metadata must be an object")
    quantization = metadata.get("quantization")
    if quantization not in (None, "W4A16"):
        raise ValueError(f"unsupported checkpoint quantization: {quantization}")
    packed = {n[: -len(PACKED_SUFFIX)] for n in names if n.endswith(PACKED_SUFFIX)}
    scales = {n[: -len(SCALES_SUFFIX)] for n in names if n.endswith(SCALES_SUFFIX)}
    if not packed and not scales:
        if quantization == "W4A16":
            raise ValueError("W4A16 index declares quantization but has no packed tensors")
        if any(".w4a16_" in n for n in names):
            raise ValueError("checkpoint index contains unrecognized W4A16 tensor names")
        return names, False, DEFAULT_GROUP_SIZE
    missing_scales = sorted(packed - scales)
    missing_packed = sorted(scales - packed)
    if missing_scales or missing_packed:
        raise ValueError("W4A16 index has incomplete packed and scale pairs: "
                         f"missing_scales={missing_scales}, missing_packed={missing_packed}")
    duplicates = sorted(packed & set(names))
    if duplicates:
        raise ValueError(f"W4A16 index contains packed and BF16 copies of the same tensor: {duplicates}")
    group_size = metadata.get("group_size", DEFAULT_GROUP_SIZE)
    if not _valid_group(group_size):
        raise ValueError(f"W4A16 index group size must be a power-of-two multiple of 32, got {group_size}")
    scale_dtype = metadata.get("scale_dtype")
    if scale_dtype is not None and scale_dtype != "BF16":
        raise ValueError(f"W4A16 index scale dtype must be BF16, got {scale_dtype}")
    return names, True, int(group_size)


class W4A16Index:
    """Named tensors of a sharded safetensors checkpoint, read on demand."""

    def __init__(self, directory: str | Path, *, index_name: str = INDEX_NAME) -> None:
        self.directory = Path(directory)
        index_path = self.directory / index_name
        if not index_path.is_file():
            raise FileNotFoundError(f"safetensors index is missing: {index_path}")
        payload = json.loads(index_path.read_text(encoding="utf-8"))
        self._weight_map, self.quantized, self.group_size = parse_index(payload)
        self._shapes: dict[str, tuple[tuple[int, ...], str]] = {}
        self._handles: dict[str, object] = {}  # one open handle per shard (header parsed once)
        by_shard: dict[str, list[str]] = {}
        for name, shard in self._weight_map.items():
            by_shard.setdefault(shard, []).append(name)
        for shard in sorted(by_shard):
            if not (self.directory / shard).is_file():
                raise FileNotFoundError(f"safetensors shard is missing: {self.directory / shard}")
            f = self._handle(shard)
            present = set(f.keys())
            for name in by_shard[shard]:
                if name not in present:
                    raise ValueError(f"tensor {name} is not in its shard {shard}")
                sl = f.get_slice(name)
                self._shapes[name] = (tuple(sl.get_shape()), sl.get_dtype())

    def _handle(self, shard: str):
        f = self._handles.get(shard)
        if f is None:
            f = safe_open(str(self.directory / shard), framework="pt", device="cpu")
            self._handles[shard] = f
        return f

    def close(self) -> None:
        """Drop the open shard handles (their memory maps)."""
        self._handles.clear()

    @property
    def names(self) -> tuple[str, ...]:
        return tuple(sorted(self._weight_map))

    def spec(self, name: str) -> tuple[tuple[int, ...], str]:
        """``(shape, safetensors dtype)`` of one tensor."""
        try:
            return self._shapes[name]
        except KeyError:
            raise KeyError(f"checkpoint tensor is absent: {name}") from None

    def load(self, name: str, *, device: torch.device | str = "cpu",
             out: torch.Tensor | None = None) -> torch.Tensor:
        """One tensor, on ``device`` or copied into ``out`` (same shape and dtype)."""
        self.spec(name)
        t = self._handle(self._weight_map[name]).get_tensor(name)
        if out is not None:
            if tuple(out.shape) != tuple(t.shape) or out.dtype != t.dtype:
                raise ValueError(f"{name}: destination {tuple(out.shape)} {out.dtype} does not match "
                                 f"{tuple(t.shape)} {t.dtype}")
            out.copy_(t)
            return out
        return t.to(device)

    def _check_w4a16(self, name: str, original_shape: tuple[int, int]) -> None:
        if not self.quantized:
            raise ValueError("the checkpoint is not W4A16")
        n, k = original_shape
        g = self.group_size
        if k % g:
            raise ValueError(f"W4A16 reduction dimension must be divisible by {g}")
        for suffix, shape, dtype in ((PACKED_SUFFIX, (n, k // 2), "U8"), (SCALES_SUFFIX, (n, k // g), "BF16")):
            got = self.spec(name + suffix)
            if got != (shape, dtype):
                raise ValueError(f"{name + suffix} must be {dtype}{list(shape)}, got {got[1]}{list(got[0])}")

    def load_w4a16(self, name: str, original_shape: tuple[int, int], *,
                   device: torch.device | str) -> W4A16Tensor:
        """The quantized matrix ``name`` of logical shape ``[N, K]`` (weights.py:599-626)."""
        self._check_w4a16(name, original_shape)
        return W4A16Tensor(packed=self.load(name + PACKED_SUFFIX, device=device),
                           scales=self.load(name + SCALES_SUFFIX, device=device),
                           original_shape=tuple(original_shape), group_size=self.group_size)


def save_w4a16_checkpoint(directory: str | Path, tensors: Mapping[str, W4A16Tensor | torch.Tensor],
                          *, shard_bytes: int = 2 << 30) -> Path:
    """Write ``tensors`` (quantized pairs and plain tensors) as sharded
    safetensors plus the index, in the layout :class:`W4A16Index` reads."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    flat: dict[str, torch.Tensor] = {}
    groups = set()
    for name, value in tensors.items():
        if isinstance(value, W4A16Tensor):
            flat[name + PACKED_SUFFIX] = value.packed
            flat[name + SCALES_SUFFIX] = value.scales
            groups.add(value.group_size)
        else:
            flat[name] = value
    if len(groups) > 1:
        raise ValueError(f"one checkpoint holds one group size, got {sorted(groups)}")
    shards: list[dict[str, torch.Tensor]] = [{}]
    size = 0
    for name in sorted(flat):
        t = flat[name].detach().to("cpu").contiguous()
        nbytes = t.numel() * t.element_size()
        if shards[-1] and size + nbytes > shard_bytes:
            shards.append({})
            size = 0
        shards[-1][name] = t
        size += nbytes
    weight_map = {}
    for i, shard in enumerate(shards):
        fname = f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        save_file(shard, str(directory / fname))
        weight_map.update({n: fname for n in shard})
    metadata: dict[str, object] = {}
    if groups:
        metadata = {"quantization": "W4A16", "group_size": groups.pop(), "scale_dtype": "BF16"}
    index = directory / INDEX_NAME
    index.write_text(json.dumps({"metadata": metadata, "weight_map": weight_map}, indent=1),
                     encoding="utf-8")
    return index


def expert_name(layer: int, expert: int, projection: str) -> str:
    """Routed expert matrix name (engine/klinear/weights.py:758, 801)."""
    return f"model.layers.{layer}.block_sparse_moe.experts.{expert}.{projection}.weight"


def shared_expert_name(layer: int, projection: str) -> str:
    """Shared expert matrix name (engine/klinear/manifest.py:59-66)."""
    return f"model.layers.{layer}.block_sparse_moe.shared_experts.{projection}.weight"


@dataclass(frozen=True)
class MoeBanks:
    """One layer's expert banks, routed experts first and the shared expert
    last: W1 (gate) and W3 (up) ``[E+1, I, H/2]`` + ``[E+1, I, H/G]``, W2
    (down) ``[E+1, H, I/2]`` + ``[E+1, H, I/G]``; the argument order of the
    MoE block ops."""

    w1_packed: torch.Tensor
    w1_scales: torch.Tensor
    w3_packed: torch.Tensor
    w3_scales: torch.Tensor
    w2_packed: torch.Tensor
    w2_scales: torch.Tensor

    def as_tuple(self) -> tuple[torch.Tensor, ...]:
        return (self.w1_packed, self.w1_scales, self.w3_packed, self.w3_scales, self.w2_packed,
                self.w2_scales)


def build_moe_banks(index: W4A16Index, layer: int, *, num_experts: int, hidden: int,
                    intermediate: int, device: torch.device | str) -> MoeBanks:
    """Contiguous banks of one layer (engine/klinear/moe.py:224-276): each bank
    is allocated once on ``device`` and every expert is copied into its slot."""
    if not index.quantized:
        raise ValueError("the checkpoint is not W4A16")
    g = index.group_size
    e1 = num_experts + 1
    banks = {}
    for bank, (n, k) in (("w1", (intermediate, hidden)), ("w3", (intermediate, hidden)),
                         ("w2", (hidden, intermediate))):
        if k % g:
            raise ValueError(f"W4A16 reduction dimension must be divisible by {g}")
        banks[bank] = (torch.empty((e1, n, k // 2), dtype=torch.uint8, device=device),
                       torch.empty((e1, n, k // g), dtype=SCALE_DTYPE, device=device), (n, k))
    shared = {"w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}
    for e in range(e1):
        for bank, (packed, scales, shape) in banks.items():
            name = expert_name(layer, e, bank) if e < num_experts else shared_expert_name(layer, shared[bank])
            index._check_w4a16(name, shape)
            index.load(name + PACKED_SUFFIX, out=packed[e])
            index.load(name + SCALES_SUFFIX, out=scales[e])
    return MoeBanks(banks["w1"][0], banks["w1"][1], banks["w3"][0], banks["w3"][1], banks["w2"][0],
                    banks["w2"][1])
