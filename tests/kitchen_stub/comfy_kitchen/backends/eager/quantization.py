"""Eager INT8 helpers of the Kitchen test double (see the package docstring)."""
import torch


def _int8_matmul_accumulate(a, b):
    """Exact INT8 x INT8 -> INT32 (int64 products on the CPU)."""
    return (a.cpu().to(torch.int64) @ b.cpu().to(torch.int64)).to(torch.int32).to(a.device)


def quantize_int8_rowwise(x):
    x = x.float()
    step = torch.clamp(x.abs().amax(-1, keepdim=True) / 127.0, min=1e-20)
    return torch.round(x / step).clamp(-127, 127).to(torch.int8), step


def _apply_input_act(x, input_act, input_act_weight, input_act_eps):
    if input_act is None:
        return x
    raise NotImplementedError("input activations are not modelled by the Kitchen test double")


def _build_hadamard(n, device=None, dtype=torch.float32):
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / n ** 0.5).to(device=device, dtype=dtype)


def _rotate_activation(x, h, groupsize):
    shape = x.shape
    return (x.reshape(*shape[:-1], shape[-1] // groupsize, groupsize) @ h).reshape(shape)


def _apply_residual(y, residual, residual_scale):
    if residual is None:
        return y
    return y + (residual if residual_scale is None else residual * residual_scale)


def int8_linear(x, weight, weight_scale, bias=None, out_dtype=torch.bfloat16, convrot=False,
                convrot_groupsize=256, input_act=None, input_act_weight=None, input_act_eps=0.0,
                residual=None, residual_scale=None):
    """Eager reference: quantize, INT32 GEMM through the hook, chunked fp32
    scaling, cast, bias in out_dtype, residual."""
    x = _apply_input_act(x, input_act, input_act_weight, input_act_eps)
    weight_scale = weight_scale.to(device=x.device, dtype=torch.float32).reshape(1, -1)
    if convrot:
        x = _rotate_activation(x, _build_hadamard(convrot_groupsize, x.device, x.dtype), convrot_groupsize)
    shape = x.shape
    x8, xs = quantize_int8_rowwise(x.reshape(-1, shape[-1]))
    acc = _int8_matmul_accumulate(x8, weight.T)
    y = (acc.float() * (xs.float() * weight_scale)).to(out_dtype)
    if bias is not None:
        y = y + bias.to(device=y.device, dtype=y.dtype).reshape(1, -1)
    return _apply_residual(y.reshape(*shape[:-1], weight.shape[0]), residual, residual_scale)
