"""numpy <-> device helpers for the GPU parity tests (inputs are produced on the
host by the oracle with YTensor's own RNG and rounding, then uploaded)."""
from __future__ import annotations

import numpy as np
import torch


def dev_bf16(bits: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def dev_f16(bits: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.float16).to(device)


def dev_f32(x: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def make_input(orc, x: np.ndarray, dtype: str, device="cuda"):
    """Round x with YTensor's conversion for `dtype`; return (device tensor,
    float32 host copy of exactly the values the device sees)."""
    if dtype == "f32":
        return dev_f32(x, device), np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "bf16":
        bits = orc.bf16_round(x)
        return dev_bf16(bits, device), orc.bf16_to_f32(bits)
    if dtype == "f16":
        bits = orc.f16_round(x)
        return dev_f16(bits, device), orc.f16_to_f32(bits)
    raise ValueError(dtype)


TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


REL_16 = 2e-2
MAE_16 = 1e-3


def floor16(orc, r: np.ndarray, dtype: str) -> float:
    """MAE that rounding the exact fp32 result to the 16-bit output type alone costs."""
    rb = orc.bf16_to_f32(orc.bf16_round(r)) if dtype == "bf16" else orc.f16_to_f32(orc.f16_round(r))
    return float(np.abs(rb.astype(np.float64) - r).mean())


def check16(orc, g: np.ndarray, r: np.ndarray, dtype: str, out16: bool, label: str = "") -> tuple[float, float]:
    """The 16-bit parity bar: max|g-r|/max|r| <= 2e-2 and MAE <= 1e-3, where for a
    16-bit OUTPUT the MAE bar is max(1e-3, 1.1 * rounding floor)."""
    g64, r64 = g.astype(np.float64), r.astype(np.float64)
    den = np.abs(r64).max()
    re = float(np.abs(g64 - r64).max() / (den if den > 0 else 1.0))
    me = float(np.abs(g64 - r64).mean())
    fl = floor16(orc, r, dtype) if out16 else 0.0
    bar = max(MAE_16, 1.1 * fl) if out16 else MAE_16
    print(f"{label}: rel={re:.3e} mae={me:.3e} floor={fl:.3e} bar={bar:.3e}", flush=True)
    assert re <= REL_16, f"{label}: rel err {re}"
    assert me <= bar, f"{label}: MAE {me} > {bar}"
    return re, me
