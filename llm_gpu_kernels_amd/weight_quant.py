"""Offline W4G128 gate/up preparation (never inside a forward).

``quantize_gate_up`` produces the reference's v1 format
(src/llm_gpu_kernels/moe_weight_quant.py:1-7, 55-105) for any [E, N, K] with
K % 128 == 0; ``tile_gate_up`` rearranges it into the gfx950 streaming
layout (role of repack_gate_up, moe_weight_layout.py:81-127), and
``dequantize_tiled`` expands tiled weights on the GPU with exactly the decode
the GEMM uses.  Quantisation and tiling run in the C library on the host.
"""
from __future__ import annotations

import ctypes
import hashlib
from dataclasses import dataclass, field

import torch

from . import _native as N

GROUP = 128


def _digest(t: torch.Tensor) -> str:
    t = t.detach().cpu().contiguous()
    h = hashlib.sha256(str((str(t.dtype), tuple(t.shape))).encode())
    h.update(t.view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


@dataclass(frozen=True)
class PackedGateUp:
    """v1 format: words int32 [E, N, K/8] (uint32 bit patterns), scales bf16 [E, N, K/128]."""
    words: torch.Tensor
    scales: torch.Tensor
    metadata: dict = field(default_factory=dict)

    @property
    def shape(self):
        e, n, kw = self.words.shape
        return (e, n, kw * 8)

    def to(self, device):
        return PackedGateUp(self.words.to(device), self.scales.to(device), self.metadata)


@dataclass(frozen=True)
class TiledGateUp:
    """gfx950 layout: words int32 [E, N/16, K/128, 64, 4], scales bf16 [E, N/16, K/128, 16]."""
    words: torch.Tensor
    scales: torch.Tensor
    logical_shape: tuple

    @property
    def shape(self):
        return self.logical_shape

    def to(self, device):
        return TiledGateUp(self.words.to(device).contiguous(), self.scales.to(device).contiguous(),
                           self.logical_shape)


def quantize_gate_up(weight: torch.Tensor) -> PackedGateUp:
    """Quantise a finite, contiguous CPU bf16 [E, N, K] weight (K % 128 == 0)."""
    if weight.device.type != "cpu" or weight.dtype != torch.bfloat16:
        raise ValueError("offline packing requires CPU BF16 weights")
    if weight.ndim != 3 or weight.shape[2] % GROUP or not weight.is_contiguous():
        raise ValueError("expected contiguous [E, N, K] with K % 128 == 0")
    e, n, k = weight.shape
    words = torch.empty((e, n, k // 8), dtype=torch.int32)
    scales = torch.empty((e, n, k // GROUP), dtype=torch.bfloat16)
    rc = N.lib().moe_w4_quantize(weight.data_ptr(), e, n, k, words.data_ptr(), scales.data_ptr())
    if rc != N.MOE_OK:
        raise ValueError("nonfinite source weights or unrepresentable scale")
    meta = dict(format_version=1, logical_shape=[e, n, k], group_size=GROUP,
                encoding="q+8, q in [-7,7], low nibble is earliest K",
                word_storage="int32 storage of uint32 bit pattern", scale_dtype="bfloat16",
                source_sha256=_digest(weight), words_sha256=_digest(words),
                scales_sha256=_digest(scales),
                packed_weight_bytes=words.numel() * 4, scale_bytes=scales.numel() * 2)
    return PackedGateUp(words, scales, meta)


def tile_gate_up(packed: PackedGateUp) -> TiledGateUp:
    """Rearrange v1 words/scales (any device) into the gfx950 layout on the host."""
    words = packed.words.detach().cpu().contiguous()
    scales = packed.scales.detach().cpu().contiguous()
    e, n, k = packed.shape
    if n % 16 or k % GROUP or words.dtype != torch.int32 or scales.dtype != torch.bfloat16:
        raise ValueError("tiling needs int32 words, bf16 scales, N % 16 == 0, K % 128 == 0")
    if tuple(scales.shape) != (e, n, k // GROUP):
        raise ValueError("scales must be [E, N, K/128]")
    wt = torch.empty((e, n // 16, k // GROUP, 64, 4), dtype=torch.int32)
    st = torch.empty((e, n // 16, k // GROUP, 16), dtype=torch.bfloat16)
    N.check(N.lib().moe_w4_tile(words.data_ptr(), scales.data_ptr(), e, n, k, wt.data_ptr(),
                                st.data_ptr()), "tile")
    return TiledGateUp(wt, st, (e, n, k))


def dequantize_tiled(tiled: TiledGateUp) -> torch.Tensor:
    """Expand GPU-resident tiled W4 into bf16 [E, N, K] with the GEMM's decode."""
    e, n, k = tiled.shape
    if tiled.words.device.type != "cuda":
        raise ValueError("dequantize_tiled runs on the GPU")
    out = torch.empty((e, n, k), dtype=torch.bfloat16, device=tiled.words.device)
    stream = torch.cuda.current_stream(out.device).cuda_stream
    with torch.cuda.device(out.device):
        N.check(N.lib().moe_w4_dequantize(tiled.words.data_ptr(), tiled.scales.data_ptr(), e, n, k,
                                          out.data_ptr(), ctypes.c_void_p(stream)), "dequantize")
    return out
