"""Seeded synthetic inputs of the benchmark configs, generated on the GPU (no checkpoints or datasets exist here).

Trellis words are uniform 32-bit (every bitstream is a valid EXL3 tensor); suh / svh are a fair-coin sign times
U(0.5, 1.5) in fp16; activations are N(0, 1) in bf16; router logits N(0, 1) fp32. Zipf-skewed routing is produced as
logits that make the router pick a Zipf(s)-sampled set of distinct experts.
"""
from __future__ import annotations

import numpy as np
import torch

from gfr_moe import Exl3Experts, Fp8SharedWeights


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def trellis(shape, seed: int, device="cuda") -> torch.Tensor:
    return torch.randint(-(2 ** 31), 2 ** 31, shape, generator=_gen(seed, device), dtype=torch.int32, device=device)


def scales(shape, seed: int, device="cuda") -> torch.Tensor:
    g = _gen(seed, device)
    sign = torch.randint(0, 2, shape, generator=g, device=device, dtype=torch.int32) * 2 - 1
    mag = torch.rand(shape, generator=g, device=device) + 0.5
    return (sign * mag).to(torch.float16)


def experts(E: int, hidden: int, inter: int, bits: int, seed: int = 1234, device="cuda") -> Exl3Experts:
    D, N, W = hidden, inter, 8 * bits
    return Exl3Experts(
        gt=trellis((E, D // 16, N // 16, W), seed + 1, device),
        ut=trellis((E, D // 16, N // 16, W), seed + 2, device),
        dt=trellis((E, N // 16, D // 16, W), seed + 3, device),
        suh_g=scales((E, D), seed + 4, device), suh_u=scales((E, D), seed + 5, device),
        suh_d=scales((E, N), seed + 6, device), svh_g=scales((E, N), seed + 7, device),
        svh_u=scales((E, N), seed + 8, device), svh_d=scales((E, D), seed + 9, device), bits=bits)


def fp8_shared(hidden: int, inter: int, seed: int = 4321, device="cuda") -> Fp8SharedWeights:
    """An FP8 shared expert of the reference's layout (moe.shared.{gu,down}.{weight,scale}): weights N(0, 16^2)
    rounded to float8_e4m3fn (by torch, on the CPU), scales U(0.5, 1.5) / (16 sqrt(k)) in bf16, so that outputs of
    N(0, 1) inputs are of order one."""
    g = torch.Generator().manual_seed(seed)

    def mat(n, k):
        return (torch.randn((n, k), generator=g) * 16).to(torch.float8_e4m3fn).view(torch.uint8).to(device)

    def sc(n, k):
        return ((torch.rand(n, generator=g) + 0.5) / (16 * k ** 0.5)).to(torch.bfloat16).to(device)

    return Fp8SharedWeights(gu=mat(2 * inter, hidden), gu_scale=sc(2 * inter, hidden) * 2,
                            down=mat(hidden, inter), down_scale=sc(hidden, inter))


def activations(rows: int, hidden: int, seed: int, device="cuda") -> torch.Tensor:
    return torch.randn((rows, hidden), generator=_gen(seed, device), device=device).to(torch.bfloat16)


def logits(rows: int, E: int, seed: int, device="cuda") -> torch.Tensor:
    return torch.randn((rows, E), generator=_gen(seed, device), device=device)


def zipf_logits(rows: int, E: int, topk: int, s: float, seed: int, device="cuda") -> torch.Tensor:
    """Logits whose top-k is a set of distinct experts drawn with probability proportional to 1 / (rank + 1)^s
    (ranks over a seeded permutation of the experts); the picked logits decrease with the slot."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    base = rng.standard_normal((rows, E)).astype(np.float32)
    for r in range(rows):
        chosen = perm[rng.choice(E, size=topk, replace=False, p=p)]
        for j, e in enumerate(chosen):
            base[r, e] = 8.0 - 0.25 * j + 0.01 * rng.standard_normal()
    return torch.from_numpy(base).to(device)
