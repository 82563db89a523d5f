# SPDX-License-Identifier: Apache-2.0
"""Checkpoint loaders and weight-format converters for the gfx950 library.

The reference reads quantized checkpoints with safetensors (``read_weight``,
rdna2-ops/bench_int4_v07.py:193-200: ``<name>`` int8 [N, K] and
``<name with .weight -> .weight_scale>`` reshaped to [N]) and decided against a
pre-transposed resident copy because a cache keyed by address and shape cannot
guarantee the latest weight after offload, LoRA application or
re-quantisation (production/README.md:83-101). On gfx950 the INT8 GEMM reads
the checkpoint's [N, K] storage in place (it is exactly the ``weight.T`` view
the MOSS node passes), so an INT8 checkpoint needs no converted copy at all;
converted layouts (packed W4, fp8 views) come from ``ResidentWeights``, whose
entries carry an explicit validity contract:

* an entry is the prepared copy of one source tensor together with a weak
  reference to the source's storage object and the source's signature —
  device, dtype, shape, strides, data pointer and in-place version counter
  (``Tensor._version``);
* ``get`` returns the entry only while the referenced storage is the
  source's and the signature is unchanged, and prepares it again otherwise
  (an in-place update such as a LoRA merge bumps the version; a reload or
  offload round trip is a new storage, even when the allocator places it at
  the old address with version 0);
* ``invalidate(key)`` / ``clear()`` drop entries explicitly — a caller that
  replaces a weight's contents by a route that keeps pointer and version (a
  raw device copy from outside PyTorch) must call it.

Tensors are loaded with safetensors only (nothing is unpickled).
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Dict, Optional
import weakref

import torch

_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def _digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def read_weight(path, name, *, scale_suffix=".weight_scale", device="cpu"):
    """(weight, scale or None, info) of tensor ``name`` in a safetensors file —
    bench_int4_v07.py:193-200: the scale is ``name`` with ``.weight`` replaced
    by ``scale_suffix``, reshaped to 1-D, absent if the file has none; info
    records the file, name, dtype, shape and sha256 digests."""
    from safetensors import safe_open
    path = Path(path)
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        if name not in keys:
            raise KeyError(f"{name} not in {path}")
        w = f.get_tensor(name)
        sname = name.replace(".weight", scale_suffix) if name.endswith(".weight") else None
        scale = f.get_tensor(sname).reshape(-1) if sname is not None and sname in keys else None
    info = {"file": str(path), "name": name, "dtype": str(w.dtype), "shape": list(w.shape),
            "tensor_sha256": _digest(w), "scale_sha256": None if scale is None else _digest(scale)}
    if device != "cpu":
        w = w.to(device)
        scale = None if scale is None else scale.to(device)
    return w, scale, info


@dataclass
class Int8Linear:
    """An INT8 linear layer of a checkpoint: weight int8 [N, K] (read in place
    by the INT8 GEMM), per-channel fp32 scale [N] (or one scalar), optional
    bias."""
    weight: torch.Tensor
    scale: torch.Tensor
    bias: Optional[torch.Tensor] = None

    def __call__(self, x, *, activation=None, out_dtype=None, rounding="half_even"):
        from .int8_gemm import w8a8_linear
        return w8a8_linear(x, self.weight, self.scale, self.bias, out_dtype=out_dtype, activation=activation,
                           rounding=rounding)


def _check_int8(name, w, scale):
    if w.dtype != torch.int8 or w.ndim != 2 or min(w.shape) <= 0:
        raise ValueError(f"{name}: int8 [N, K] weight required")
    if w.shape[1] > 131071:
        raise ValueError(f"{name}: K > 131071 could overflow the INT32 accumulator")
    if scale is None or not scale.is_floating_point() or scale.numel() not in (1, w.shape[0]):
        raise ValueError(f"{name}: floating weight_scale with 1 or N elements required")
    if not torch.isfinite(scale).all():
        raise ValueError(f"{name}: non-finite weight scale")


def load_int8_linears(path, *, device="cuda", prefix="", scale_suffix=".weight_scale",
                      bias_suffix=".bias") -> Dict[str, Int8Linear]:
    """Every ``<layer>.weight`` int8 tensor of the file (names starting with
    ``prefix``) with its ``<layer>.weight_scale`` (and ``<layer>.bias`` if
    present) as an ``Int8Linear`` on ``device``: weight contiguous int8
    [N, K], scale contiguous fp32 [N] or [1], bias in its stored dtype. Layers
    without a scale, or whose weight is not int8, are skipped."""
    from safetensors import safe_open
    out: Dict[str, Int8Linear] = {}
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for key in sorted(keys):
            if not key.startswith(prefix) or not key.endswith(".weight"):
                continue
            layer = key[: -len(".weight")]
            sname = layer + scale_suffix
            if sname not in keys:
                continue
            w = f.get_tensor(key)
            if w.dtype != torch.int8:
                continue
            scale = f.get_tensor(sname).reshape(-1)
            _check_int8(key, w, scale)
            bias = f.get_tensor(layer + bias_suffix) if layer + bias_suffix in keys else None
            if bias is not None and (bias.ndim != 1 or bias.numel() != w.shape[0] or not bias.is_floating_point()):
                raise ValueError(f"{layer}{bias_suffix}: floating bias [N] required")
            out[layer] = Int8Linear(w.contiguous().to(device), scale.to(torch.float32).contiguous().to(device),
                                    None if bias is None else bias.contiguous().to(device))
    return out


def load_fp8_weight(path, name, *, device="cuda", scale_suffix=".weight_scale"):
    """(weight fp8 [N, K] (e4m3fn / e5m2) on device, fp32 per-channel scale
    [N] or None) for fp8_weight_gemm (its ``w_scale``); a scalar scale is
    expanded to [N]."""
    w, scale, _ = read_weight(path, name, scale_suffix=scale_suffix)
    if w.dtype not in _FP8 or w.ndim != 2:
        raise ValueError(f"{name}: fp8 [N, K] weight required")
    if scale is not None:
        if not scale.is_floating_point() or scale.numel() not in (1, w.shape[0]):
            raise ValueError(f"{name}: floating weight_scale with 1 or N elements required")
        scale = scale.to(torch.float32).expand(w.shape[0]).contiguous().to(device)
    return w.contiguous().to(device), scale


def _signature(t: torch.Tensor):
    return (t.device, t.dtype, tuple(t.shape), tuple(t.stride()), t.data_ptr(), t._version)


class ResidentWeights:
    """Prepared copies of source weights with the validity contract in the
    module docstring. ``prepare(source) -> prepared`` makes the copy (e.g. a
    W4 packing); ``get(key, source)`` returns the cached copy only while the
    source is the same storage, unchanged, and prepares it again otherwise.

    "The same storage" is a weak reference to the source's storage object,
    not its address: a weight that is freed (offloaded) and reloaded is a new
    storage with in-place version 0, and the caching allocator often places it
    at the old address, so address, shape, strides and version alone would
    return the stale copy (the reference rejects address-keyed caches for this
    reason, production/README.md:96-101). A dead or different referent is a
    miss. The weak reference keeps nothing alive."""

    def __init__(self, prepare: Callable[[torch.Tensor], object]):
        self._prepare = prepare
        self._entries: Dict[str, tuple] = {}
        self.prepared = 0  # number of prepare calls (for tests and statistics)

    def get(self, key: str, source: torch.Tensor):
        storage = source.untyped_storage()
        entry = self._entries.get(key)
        if entry is not None and entry[1]() is storage and entry[0] == _signature(source):
            return entry[2]
        value = self._prepare(source)
        self.prepared += 1
        # the signature after preparing: a prepare that reads the source does
        # not change it; one that modified it in place is caught next time
        self._entries[key] = (_signature(source), weakref.ref(storage), value)
        return value

    def invalidate(self, key: Optional[str] = None) -> None:
        if key is None:
            self._entries.clear()
        else:
            self._entries.pop(key, None)

    def clear(self) -> None:
        self._entries.clear()

    def __contains__(self, key: str) -> bool:
        return key in self._entries

    def __len__(self) -> int:
        return len(self._entries)


def w4_converter(*, group_size=128, symmetric=False, uint4=False, layout="nk", order="low"):
    """A ``ResidentWeights`` that packs floating [N, K] weights to W4 on their
    device (pack_uint4 for the unsigned uint4 storage with packed zero points, pack_int4 otherwise)."""
    from . import int4_weight_gemm_v07 as w4

    def prepare(w):
        if uint4:
            return w4.pack_uint4(w, group_size=group_size)
        return w4.pack_int4(w, group_size=group_size, symmetric=symmetric, layout=layout, order=order)

    return ResidentWeights(prepare)


def dequantize_int8(weight: torch.Tensor, scale: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """fp32(weight) * scale[n], rounded once to ``dtype`` — the floating weight
    an INT8 checkpoint stands for (input to W4 conversion)."""
    if weight.dtype != torch.int8 or weight.ndim != 2:
        raise ValueError("int8 [N, K] weight required")
    s = scale.to(torch.float32).reshape(-1)
    if s.numel() not in (1, weight.shape[0]):
        raise ValueError("scale with 1 or N elements required")
    return (weight.to(torch.float32) * s.reshape(-1, 1)).to(dtype)
