"""Offline W4G128 gate/up preparation (never inside a forward).

``quantize_gate_up`` produces the reference's v1 format
(src/llm_gpu_kernels/moe_weight_quant.py:1-7, 55-105) for any [E, N, K] with
K % 128 == 0; ``tile_gate_up`` rearranges it into the gfx950 streaming
layout (role of repack_gate_up, moe_weight_layout.py:81-127), and
``dequantize_tiled`` expands tiled weights on the GPU with exactly the decode
the GEMM uses.  Quantisation and tiling run in the C library on the host.

The reference's M24 physical layout (moe_weight_layout.py:14-19, the
``repack_gate_up`` output) is read and written bit-exactly by
``restore_v1_layout`` / ``repack_gate_up``; ``tile_gate_up`` accepts either
layout.
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


# M24 layout string and version of the reference (moe_weight_layout.py:14-17).
M24_LAYOUT = ("words[E,projection,Ntile,K32,word,Nlane];"
              "scales[E,projection,Ntile,K128,Nlane];Nlane-contiguous")
M24_LANES = 64


@dataclass(frozen=True)
class RepackedGateUp:
    """M24 physical layout: words int32 [E, 2, N/128, K/32, 4, 64] and scales
    bf16 [E, 2, N/128, K/128, 64] (projection = gate/up half of N, Ntile of 64
    rows, Nlane innermost), metadata format_version 2."""
    words: torch.Tensor
    scales: torch.Tensor
    metadata: dict = field(default_factory=dict)

    @property
    def shape(self):
        e, p, nt, k32, w, nl = self.words.shape
        return (e, p * nt * nl, k32 * w * 8)

    def to(self, device):
        return RepackedGateUp(self.words.to(device), self.scales.to(device), self.metadata)


def _check_v1(packed: PackedGateUp) -> tuple:
    """Digests of a v1 pack, verified against its metadata when recorded
    (moe_weight_layout.py:60-78): a pack whose bits differ from its recorded
    words_sha256 / scales_sha256 is rejected, not rearranged."""
    meta = packed.metadata or {}
    if meta:
        if meta.get("format_version", 1) != 1 or meta.get("group_size", GROUP) != GROUP:
            raise ValueError("v1 metadata must declare format_version=1 and group_size=128")
        if "logical_shape" in meta and tuple(meta["logical_shape"]) != tuple(packed.shape):
            raise ValueError("v1 metadata logical_shape does not match the buffers")
    words_sha, scales_sha = _digest(packed.words), _digest(packed.scales)
    for key, got in (("words_sha256", words_sha), ("scales_sha256", scales_sha)):
        if key in meta and meta[key] != got:
            raise ValueError(f"v1 packed buffers do not match their recorded {key}")
    return words_sha, scales_sha


def repack_gate_up(packed: PackedGateUp) -> RepackedGateUp:
    """v1 -> M24, a pure permutation of words and scales (moe_weight_layout.py:81-88):
    v1 word [e, p*(N/2) + t*64 + l, 4*k + w] -> [e, p, t, k, w, l]; v1 scale
    [e, p*(N/2) + t*64 + l, g] -> [e, p, t, g, l].  The metadata carries what the
    reference's restore_v1_layout checks (moe_weight_layout.py:130-175): the
    physical and canonical digests and a v1 metadata snapshot whose digests
    match the canonical ones, plus the byte ledger (moe_weight_layout.py:90-121)."""
    e, n, k = packed.shape
    if n % (2 * M24_LANES) or k % GROUP:
        raise ValueError("M24 layout needs N % 128 == 0 and K % 128 == 0")
    words_sha, scales_sha = _check_v1(packed)
    nt = n // (2 * M24_LANES)
    words = packed.words.reshape(e, 2, nt, M24_LANES, k // 32, 4).permute(0, 1, 2, 4, 5, 3)
    scales = packed.scales.reshape(e, 2, nt, M24_LANES, k // GROUP).permute(0, 1, 2, 4, 3)
    words, scales = words.contiguous(), scales.contiguous()
    v1_meta = dict(packed.metadata or {})
    v1_meta.setdefault("format_version", 1)
    v1_meta.setdefault("group_size", GROUP)
    v1_meta.setdefault("logical_shape", [e, n, k])
    v1_meta["words_sha256"], v1_meta["scales_sha256"] = words_sha, scales_sha
    wb, sb = packed.words.numel() * 4, packed.scales.numel() * 2
    meta = dict(format_version=2, layout=M24_LAYOUT, logical_shape=[e, n, k], group_size=GROUP,
                canonical_words_sha256=words_sha, canonical_scales_sha256=scales_sha,
                canonical_words_shape=list(packed.words.shape),
                canonical_scales_shape=list(packed.scales.shape),
                physical_words_shape=list(words.shape), physical_scales_shape=list(scales.shape),
                physical_words_sha256=_digest(words), physical_scales_sha256=_digest(scales),
                canonical_v1_metadata=v1_meta,
                byte_ledger=dict(canonical_words_bytes=wb, canonical_scales_bytes=sb,
                                 canonical_packed_total_bytes=wb + sb,
                                 physical_words_bytes=wb, physical_scales_bytes=sb,
                                 physical_packed_total_bytes=wb + sb,
                                 additional_repacked_tensor_bytes=wb + sb,
                                 canonical_plus_repacked_resident_bytes=2 * (wb + sb),
                                 physical_packed_total_mib=(wb + sb) / (1024 * 1024),
                                 interpretation="layout-only storage; quantization and total "
                                                "packed bytes are unchanged"))
    return RepackedGateUp(words, scales, meta)


def restore_v1_layout(repacked: RepackedGateUp) -> PackedGateUp:
    """M24 -> v1 with the original bit patterns (inverse permutation of
    moe_weight_layout.py:85-88).  Metadata, when present, must declare the M24
    layout (moe_weight_layout.py:134-141); every recorded digest is checked:
    the physical ones before the permutation, the canonical ones after it, and
    the v1 snapshot's digests against the canonical ones (:150-174)."""
    meta = repacked.metadata or {}
    if meta and (meta.get("format_version") != 2 or meta.get("layout") != M24_LAYOUT
                 or meta.get("group_size", GROUP) != GROUP):
        raise ValueError("unsupported M24 physical layout metadata")
    words, scales = repacked.words, repacked.scales
    if (words.ndim != 6 or scales.ndim != 5 or words.shape[4] != 4
            or words.shape[5] != M24_LANES or words.dtype != torch.int32
            or scales.dtype != torch.bfloat16 or tuple(scales.shape) != (
                words.shape[0], words.shape[1], words.shape[2], words.shape[3] // 4, M24_LANES)):
        raise ValueError("M24 words must be int32 [E,2,Nt,K/32,4,64], scales bf16 [E,2,Nt,K/128,64]")
    for key, t in (("physical_words_sha256", words), ("physical_scales_sha256", scales)):
        if key in meta and _digest(t) != meta[key]:
            raise ValueError(f"M24 buffer does not match its recorded {key}")
    e, p, nt, k32, _, nl = words.shape
    n, k = p * nt * nl, k32 * 32
    if "logical_shape" in meta and tuple(meta["logical_shape"]) != (e, n, k):
        raise ValueError("M24 metadata logical_shape does not match the buffers")
    v1_words = words.permute(0, 1, 2, 5, 3, 4).reshape(e, n, k // 8).contiguous()
    v1_scales = scales.permute(0, 1, 2, 4, 3).reshape(e, n, k // GROUP).contiguous()
    canon = {}
    for key, t in (("canonical_words_sha256", v1_words), ("canonical_scales_sha256", v1_scales)):
        if key in meta:
            canon[key] = _digest(t)
            if canon[key] != meta[key]:
                raise ValueError("restored v1 bit patterns do not match the canonical digests")
    v1_meta = dict(meta.get("canonical_v1_metadata", {}) or {})
    if v1_meta:
        if v1_meta.get("format_version", 1) != 1 or v1_meta.get("group_size", GROUP) != GROUP:
            raise ValueError("M24 metadata has no matching canonical v1 metadata snapshot")
        for v1_key, key in (("words_sha256", "canonical_words_sha256"),
                            ("scales_sha256", "canonical_scales_sha256")):
            if v1_key in v1_meta and key in meta and v1_meta[v1_key] != meta[key]:
                raise ValueError("M24 metadata has no matching canonical v1 metadata snapshot")
    return PackedGateUp(v1_words, v1_scales, v1_meta)


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


def tile_gate_up(packed) -> TiledGateUp:
    """Rearrange v1 (or M24) words/scales (any device) into the gfx950 layout on the host."""
    if isinstance(packed, RepackedGateUp):
        packed = restore_v1_layout(packed.to("cpu"))
    elif isinstance(packed, PackedGateUp) and packed.metadata:
        _check_v1(packed.to("cpu"))
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
