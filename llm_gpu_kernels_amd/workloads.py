"""Seeded synthetic MoE layers of the benchmark configurations.

* ``tiny``: T tokens, H=512, I=256, E=8, top-2 (CPU-reference sized).
* ``qwen``: Qwen3-30B-A3B MoE shape, H=2048, I=768, E=128, top-8.
* ``qwen-ep8``: one GPU's share of that layer under 8-way expert parallelism:
  its 16 experts, and one route per received row (the dispatch all-to-all
  delivers each (token, local expert) pair as a row; T rows here).
* ``qwen-tp8``: one GPU's share under 8-way tensor parallelism: all 128
  experts with I = 768 / 8 = 96 (gate/up rows and down columns sharded); the
  partial [T, H] outputs would then be summed across GPUs.
Weights ~ N(0, 0.02) bf16, hidden ~ N(0, 1) bf16, router logits ~ N(0, 1)
fp32.  ``routing="zipf"`` adds log(Zipf(s=1.2)) over a seeded expert
permutation to the logits, so a few experts receive hundreds of rows and many
receive none.  The generator lives on ``device`` (a CUDA generator for GPU
runs), so values depend on the device but are deterministic per seed.
"""
from __future__ import annotations

import torch

SHAPES = {
    "tiny": dict(E=8, H=512, I=256, K=2),
    "qwen": dict(E=128, H=2048, I=768, K=8),
    "qwen-ep8": dict(E=16, H=2048, I=768, K=1),
    "qwen-tp8": dict(E=128, H=2048, I=96, K=8),
}


def zipf_bias(experts: int, s: float, generator, device) -> torch.Tensor:
    perm = torch.randperm(experts, generator=generator, device=device)
    rank = torch.arange(1, experts + 1, dtype=torch.float32, device=device)
    p = rank.pow(-s)
    p = p / p.sum()
    bias = torch.empty(experts, dtype=torch.float32, device=device)
    bias[perm] = p.log()
    return bias


def make_layer(shape: str = "qwen", tokens: int = 17, *, routing: str = "uniform", seed: int = 0,
               device="cpu", weights: bool = True):
    """Return dict(x, gate_up, down, logits, E, H, I, K)."""
    dims = SHAPES[shape]
    e, h, inter, k = dims["E"], dims["H"], dims["I"], dims["K"]
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((tokens, h), generator=g, device=device).to(torch.bfloat16)
    gate_up = down = None
    if weights:
        gate_up = (torch.randn((e, 2 * inter, h), generator=g, device=device) * 0.02).to(torch.bfloat16)
        down = (torch.randn((e, h, inter), generator=g, device=device) * 0.02).to(torch.bfloat16)
    logits = torch.randn((tokens, e), generator=g, device=device)
    if routing == "zipf":
        logits = logits + zipf_bias(e, 1.2, g, device)[None, :]
    elif routing != "uniform":
        raise ValueError(f"unknown routing {routing}")
    return dict(x=x, gate_up=gate_up, down=down, logits=logits.contiguous(), E=e, H=h, I=inter, K=k)
