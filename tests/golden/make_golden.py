"""Write the small golden fixtures of the INT8 path (tests/golden/int8_*.npz).

Inputs are drawn on the CPU from torch.Generator seeds in a fixed order.
Expected outputs come from the numpy oracle (oracle/int8.py) and are
cross-checked here, before anything is written, against an independent
implementation of the same reference formulas in torch CPU ops
(torch._int_mm / int64 matmul, torch fp32 arithmetic in the order of
rdna2-ops/rdna2_ops/int8_gemm.py:53-63 and comfy_int8.py:128-143,
torch.round for half-even). The fixtures shapes follow the reference's own
small checks: 37x53x79 with an offset, row-padded A view, both B layouts,
scalar and per-channel weight scales and an fp32 bias
(rdna2-ops/bench_int8_gemm.py:177-205), plus 37x64x256
(rdna2-ops/bench_int8_layout.py:33,47-49).

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import int8 as o  # noqa: E402


def _torch_epilogue_f(acc, sa, sb, bias):
    v = acc.to(torch.float32) * (sa.reshape(-1, 1) * sb.reshape(1, -1))
    return v + bias.reshape(1, -1) if bias is not None else v


def int8_small():
    g = torch.Generator().manual_seed(20261106)
    m, n, k = 37, 53, 79
    a_store = torch.randint(-128, 128, (m + 2, k + 3), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sa = torch.rand(m, generator=g) * 0.02 + 0.001
    sb = torch.rand(n, generator=g) * 0.02 + 0.001
    sb1 = torch.rand(1, generator=g) * 0.02 + 0.001
    bias = torch.randn(n, generator=g)
    a = a_store[1:1 + m, 1:1 + k]
    acc_t = (a.to(torch.int64) @ w.T.to(torch.int64)).to(torch.int32)
    acc = o.int8_matmul(a.numpy(), np.ascontiguousarray(w.numpy().T))
    assert np.array_equal(acc, acc_t.numpy())
    out = {"a_store": a_store.numpy(), "w": w.numpy(), "sa": sa.numpy(), "sb": sb.numpy(),
           "sb1": sb1.numpy(), "bias": bias.numpy(), "acc": acc}
    for label, scale in (("vec", sb), ("scalar", sb1)):
        f32 = o.epilogue_f(acc, sa.numpy(), scale.numpy(), bias.numpy(), out="f32")
        ref = _torch_epilogue_f(acc_t, sa, scale, bias).numpy()
        assert np.array_equal(f32.view(np.uint32), ref.view(np.uint32)), label
        out[f"f32_{label}"] = f32
        out[f"f16_{label}"] = o.encode(f32, "f16")
        assert np.array_equal(out[f"f16_{label}"], torch.from_numpy(ref).to(torch.float16).numpy())
        out[f"bf16_{label}"] = o.encode(f32, "bf16")
        assert np.array_equal(out[f"bf16_{label}"],
                              torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
        out[f"f32_nobias_{label}"] = o.epilogue_f(acc, sa.numpy(), scale.numpy(), None, out="f32")
        fused = o.epilogue_f(acc, sa.numpy(), scale.numpy(), bias.numpy(), out="f32", fused=True)
        out[f"f32_fused_{label}"] = fused
        eager16 = o.epilogue_e(acc, sa.numpy(), scale.numpy(), bias.numpy(), out="f16")
        t = (acc_t.float() * (sa.reshape(-1, 1) * scale.reshape(1, -1))).to(torch.float16)
        t = t + bias.to(torch.float16).reshape(1, -1)
        assert np.array_equal(o.encode(eager16, "f16"), t.numpy()), "eager order E"
        out[f"f16_eager_{label}"] = o.encode(eager16, "f16")
    gelu = o.epilogue_f(acc, sa.numpy(), sb.numpy(), bias.numpy(), out="f32", activation="gelu_tanh")
    ref = torch.nn.functional.gelu(_torch_epilogue_f(acc_t, sa, sb, bias), approximate="tanh").numpy()
    assert np.abs(gelu - ref).max() <= 1e-6
    out["f32_gelu_vec"] = gelu
    return out


def int8_layout():
    g = torch.Generator().manual_seed(20261105)
    m, n, k = 37, 64, 256
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    acc = o.int8_matmul(a.numpy(), np.ascontiguousarray(w.numpy().T))
    assert np.array_equal(acc, (a.to(torch.int32) @ w.to(torch.int32).T).numpy())
    assert np.array_equal(acc, torch._int_mm(a, w.T.contiguous()).numpy())
    return {"a": a.numpy(), "w": w.numpy(), "acc": acc}


def quant_small():
    g = torch.Generator().manual_seed(7)
    m, k = 19, 200
    x = torch.randn(m, k, generator=g)
    x[torch.rand(m, k, generator=g) < 0.01] *= 20
    x[3] = 0.0                                  # zero row -> step 1e-20, q = 0
    x[4, :8] = torch.tensor([127.0, -2.5, 2.5, 0.5, -0.5, 1.5, 126.5, -126.5])  # step == 1: exact ties
    x[5, 0] = 127.0
    x[5, 1] = 0.49999997                        # z + 0.5 rounds up to 1.0 in fp32
    x16 = x.to(torch.float16)
    out = {"x_f32": x.numpy(), "x_f16": x16.numpy()}
    for label, xv in (("f32", x.numpy()), ("f16", x16.float().numpy())):
        for rounding in ("half_even", "half_away"):
            q, step = o.quant_rows(xv, rounding)
            xt = torch.from_numpy(xv)
            st = torch.clamp(xt.abs().amax(1) / 127.0, min=1e-20)
            assert np.array_equal(step, st.numpy())
            z = xt / st[:, None]
            if rounding == "half_even":
                qt = torch.round(z)
            else:
                qt = torch.where(z >= 0, torch.floor(z + 0.5), torch.ceil(z - 0.5))
            assert np.array_equal(q, qt.clamp(-127, 127).to(torch.int8).numpy()), (label, rounding)
            out[f"q_{label}_{rounding}"] = q
            out[f"step_{label}_{rounding}"] = step
    assert out["q_f32_half_even"][4, :8].tolist() == [127, -2, 2, 0, 0, 2, 126, -126]
    assert out["q_f32_half_away"][4, :8].tolist() == [127, -3, 3, 1, -1, 2, 127, -127]
    assert out["q_f32_half_away"][5, 1] == 1 and out["q_f32_half_even"][5, 1] == 0
    return out


def main():
    manifest = {}
    for name, fn in (("int8_small", int8_small), ("int8_layout", int8_layout), ("quant_small", quant_small)):
        data = fn()
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **data)
        manifest[name] = {key: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()[:16]
                          for key, v in sorted(data.items())}
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print("wrote", ", ".join(manifest))


if __name__ == "__main__":
    main()
