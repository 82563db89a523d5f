"""Test double of the patientx Qwen INT8 bridge module (an external ComfyUI
node, not present here) that rdna2-ops/rdna2_ops/int8_gemm.py:274-330
patches. Only the interface is mirrored: the module's source path, its row
quantizer ``triton_quantize_rowwise`` and the two GEMM wrappers
``triton_int8_linear`` / ``triton_int8_linear_per_row`` with their
(x, weight, weight_scale, bias=None, compute_dtype=torch.float16) signature.
The wrappers' arithmetic here is a plain eager stand-in; the candidate
replaces them for fp32 calls and only calls them back for other precisions.
"""
import torch


def triton_quantize_rowwise(x):
    """Per-row absmax / 127, round half to even, clamp to +-127; fp32 steps [M, 1]."""
    x = x.float()
    step = torch.clamp(x.abs().amax(-1, keepdim=True) / 127.0, min=1e-20)
    return torch.round(x / step).clamp(-127, 127).to(torch.int8), step


def _eager(x, weight, scale, bias, compute_dtype):
    shape = x.shape
    q, step = triton_quantize_rowwise(x.reshape(-1, shape[-1]))
    acc = (q.cpu().to(torch.int64) @ weight.cpu().to(torch.int64).T).to(torch.int32).to(x.device)
    y = acc.float() * (step * scale)
    if bias is not None:
        y = y + bias.float().reshape(1, -1)
    return y.to(compute_dtype).reshape(*shape[:-1], weight.shape[0])


def triton_int8_linear(x, weight, weight_scale, bias=None, compute_dtype=torch.float16):
    scale = weight_scale if isinstance(weight_scale, torch.Tensor) else torch.tensor(weight_scale)
    return _eager(x, weight, scale.to(x.device, torch.float32).reshape(1, -1), bias, compute_dtype)


def triton_int8_linear_per_row(x, weight, weight_scale, bias=None, compute_dtype=torch.float16):
    return _eager(x, weight, weight_scale.to(x.device, torch.float32).reshape(1, -1), bias, compute_dtype)
