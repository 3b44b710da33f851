"""Seeded synthetic WKV7 operands with the value distributions the benchmark
configurations name.

The distributions follow how rwkv-nn's time mixer produces the operands
(crates/rwkv-nn/src/modules/time_mixer/weight_prepare.rs:282-317):

* r, k, v ~ N(0, 1)
* the ``weight_decay`` operand is a raw logit x ~ N(0, 1); the kernels form the
  decay exp(-e^{-1/2} * sigmoid(x)) themselves (wkv7_common/kernel.rs:63-65)
* kk ~ N(0, 1), L2-normalised per head over N; a = -kk and b = kk * sigmoid(g)
  with g ~ N(0, 1)
* the upstream gradient dy ~ N(0, 1); the initial state is zero or N(0, std)

bf16 configurations draw in fp32 and round to bf16 with round-to-nearest-even;
the returned float32 arrays then hold exactly the bf16 values.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as
    float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + bias) & np.uint32(0xFFFF0000)).view(np.float32)


def make_inputs(B: int, T: int, H: int, N: int = 64, seed: int = 0,
                s0_std: float | None = None, bf16: bool = False,
                with_grad: bool = True) -> dict:
    """Seeded operands as float32 numpy arrays, shapes [B, T, H, N] (state
    [B, H, N, N]). Keys: w, r, k, v, a, b, s0 (None when s0_std is None), dy,
    ds_T (zeros)."""
    rng = np.random.default_rng(seed)
    shape = (B, T, H, N)
    f = np.float32
    w = rng.standard_normal(shape, dtype=f)
    r = rng.standard_normal(shape, dtype=f)
    k = rng.standard_normal(shape, dtype=f)
    v = rng.standard_normal(shape, dtype=f)
    kk = rng.standard_normal(shape, dtype=f)
    kk = kk / np.maximum(np.linalg.norm(kk, axis=-1, keepdims=True), f(1e-12))
    g = rng.standard_normal(shape, dtype=f)
    a = -kk
    b = kk * (f(1.0) / (f(1.0) + np.exp(-g)))
    out = {"w": w, "r": r, "k": k, "v": v, "a": a.astype(f), "b": b.astype(f)}
    out["s0"] = (rng.standard_normal((B, H, N, N), dtype=f) * f(s0_std)
                 if s0_std is not None else None)
    if with_grad:
        out["dy"] = rng.standard_normal(shape, dtype=f)
        out["ds_T"] = np.zeros((B, H, N, N), f)
    if bf16:
        for key in ("w", "r", "k", "v", "a", "b", "dy"):
            if key in out and out[key] is not None:
                out[key] = bf16_round(out[key])
    return out


def make_inputs_torch(B: int, T: int, H: int, N: int = 64, seed: int = 0,
                      s0_std: float | None = None, dtype=None, device="cuda"):
    """Same distributions, generated on the device with torch (used by the
    benchmark, where numpy generation of the full-size tensors would dominate
    the run). Returns a dict of device tensors in ``dtype`` (operands) and
    float32 (state)."""
    import torch

    dtype = dtype or torch.bfloat16
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (B, T, H, N)

    def randn(*s):
        return torch.randn(*s, generator=gen, device=device, dtype=torch.float32)

    w, r, k, v = randn(*shape), randn(*shape), randn(*shape), randn(*shape)
    kk = torch.nn.functional.normalize(randn(*shape), dim=-1)
    g = randn(*shape)
    out = {"w": w, "r": r, "k": k, "v": v, "a": -kk, "b": kk * torch.sigmoid(g),
           "dy": randn(*shape)}
    out = {key: val.to(dtype).contiguous() for key, val in out.items()}
    out["s0"] = (randn(B, H, N, N) * s0_std) if s0_std is not None else None
    return out
