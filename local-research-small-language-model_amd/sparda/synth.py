"""Seeded synthetic workloads of the sparse attention path.

Inputs are drawn in fp32 on the CPU from ``torch.Generator().manual_seed``
in a fixed order (q, k, v, forecast), rotary embedding (base 10000) is
applied to q and k in fp32 at their absolute positions, and the result is
cast to the requested dtype — so every consumer sees identical bits.
"""

from __future__ import annotations

from typing import Dict

import torch


def _rope_fp32(x: torch.Tensor, pos: torch.Tensor, theta: float = 10000.0) -> torch.Tensor:
    """x [..., T, H, D] fp32 rotated at positions pos [T] (rotate-half pairs)."""
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = pos.to(torch.float32)[:, None] * inv[None, :]
    c = torch.cos(ang)[:, None, :]
    s = torch.sin(ang)[:, None, :]
    h = D // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


def prefill_inputs(B: int, T: int, Hq: int, Hkv: int, D: int, dtype=torch.bfloat16, seed: int = 1001,
                   device="cpu", Df: int = None) -> Dict[str, torch.Tensor]:
    """q [B,T,Hq,D], k/v [B,T,Hkv,D], forecast [B,T,Hkv,Df]; N(0,1), RoPE on q/k."""
    Df = Df or D
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=g)
    k = torch.randn(B, T, Hkv, D, generator=g)
    v = torch.randn(B, T, Hkv, D, generator=g)
    f = torch.randn(B, T, Hkv, Df, generator=g)
    pos = torch.arange(T)
    q = _rope_fp32(q, pos)
    k = _rope_fp32(k, pos)
    out = {"q": q, "k": k, "v": v, "forecast": f}
    return {n: t.to(dtype).to(device) for n, t in out.items()}


def decode_inputs(B: int, S: int, Hq: int, Hkv: int, D: int, dtype=torch.bfloat16, seed: int = 1002,
                  device="cpu", Df: int = None, capacity: int = None) -> Dict[str, torch.Tensor]:
    """One decode step at position S-1 over a cache holding tokens [0, S).

    k_cache/v_cache [B,capacity,Hkv,D] (RoPE on keys at 0..S-1, zeros past S),
    q [B,Hq,D] (RoPE at S-1), forecast [B,Hkv,Df]."""
    Df = Df or D
    capacity = capacity or S
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, 1, Hq, D, generator=g)
    k = torch.randn(B, S, Hkv, D, generator=g)
    v = torch.randn(B, S, Hkv, D, generator=g)
    f = torch.randn(B, Hkv, Df, generator=g)
    q = _rope_fp32(q, torch.tensor([S - 1]))[:, 0]
    k = _rope_fp32(k, torch.arange(S))
    kc = torch.zeros(B, capacity, Hkv, D)
    vc = torch.zeros(B, capacity, Hkv, D)
    kc[:, :S] = k
    vc[:, :S] = v
    out = {"q": q, "k_cache": kc, "v_cache": vc, "forecast": f}
    return {n: t.to(dtype).to(device) for n, t in out.items()}


def kv_chunks(B: int, S: int, Hkv: int, D: int, seed: int, chunk: int = 8192):
    """Keys (RoPE at their positions) and values ~N(0,1), fp32, in chunks of
    tokens: yields (pos0, k [B,n,Hkv,D], v [B,n,Hkv,D]) covering [0, S)."""
    g = torch.Generator().manual_seed(seed)
    for p0 in range(0, S, chunk):
        n = min(chunk, S - p0)
        k = torch.randn(B, n, Hkv, D, generator=g)
        v = torch.randn(B, n, Hkv, D, generator=g)
        yield p0, _rope_fp32(k, torch.arange(p0, p0 + n)), v
