"""Segmented-KV GQA prefill attention on MI355X (secondary path).

Mirrors ``prepare_cuda_gqa_compact(q, segments, out=None, *, stages=1)``
(src/llm_gpu_kernels/attention_cuda_compact.py:135-186) and its input
validation (:97-121): Q [T, 32, 128] bf16 contiguous, segments = sequence of
(k, v) pairs [L, 8, 128] bf16 with inner strides (128, 1) and a token stride
>= heads*128 that is a multiple of 8, the last segment being the current
chunk (L == T, causal).  ``run()`` enqueues on the current stream with no
host sync and no allocation and returns the owned output.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _native as N

__all__ = ["PreparedSegmentedGQA", "prepare_segmented_gqa", "prepare_cuda_gqa_compact"]


def _validate(t, name, device, heads):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.ndim != 3 or tuple(t.shape[1:]) != (heads, 128):
        raise ValueError(f"{name} must have shape [L, {heads}, 128]")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must have dtype torch.bfloat16")
    if t.device != device:
        raise ValueError(f"{name} must be on q's device")
    if tuple(t.stride()[1:]) != (128, 1):
        raise ValueError(f"{name} must have inner strides (128, 1)")
    if t.shape[0] and (t.stride(0) < heads * 128 or t.stride(0) % 8):
        raise ValueError(f"{name} token stride must be at least {heads * 128} and divisible by 8")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} base address must be 16-byte aligned")


def check_out_storage(out, inputs):
    """Reject an output that shares storage with q or a K/V segment: the kernel
    writes out while other workgroups still read the inputs
    (attention_cuda_compact.py:175-177 rejects the same).  Empty tensors own no
    memory and cannot alias."""
    if out.numel() == 0:
        return
    storage = out.untyped_storage().data_ptr()
    if any(t.numel() and t.untyped_storage().data_ptr() == storage for t in inputs):
        raise ValueError("out must not share storage with any input")


class PreparedSegmentedGQA:
    """Owns the output and split-K workspace; binds q and the segments by address."""

    def __init__(self, q, segments, out=None, scale=None):
        if not isinstance(q, torch.Tensor) or q.ndim != 3 or q.shape[2] != 128:
            raise ValueError("q must be [T, Hq, 128]")
        if scale is not None and not (math.isfinite(float(scale)) and float(scale) > 0.0):
            # the C ABI reads a scale <= 0 or non-finite as "default"; an explicit
            # one must not be replaced silently
            raise ValueError(f"scale must be a positive finite number (got {scale!r})")
        if q.dtype != torch.bfloat16 or not q.is_contiguous() or q.device.type != "cuda":
            raise ValueError("q must be a contiguous bf16 GPU tensor")
        segments = [tuple(s) for s in segments]
        if not 1 <= len(segments) <= N.GQA_MAX_SEGMENTS:
            raise ValueError("1..4 KV segments required")
        t, hq, _ = q.shape
        hkv = segments[0][0].shape[1]
        for i, (k, v) in enumerate(segments):
            _validate(k, f"segments[{i}].k", q.device, hkv)
            _validate(v, f"segments[{i}].v", q.device, hkv)
            if k.shape[0] != v.shape[0]:
                raise ValueError(f"segments[{i}] k and v lengths differ")
        if segments[-1][0].shape[0] != t:
            raise ValueError("the current (last) segment must have T tokens")
        if out is None:
            out = torch.empty_like(q)
        if tuple(out.shape) != tuple(q.shape) or out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise ValueError("out must be a contiguous bf16 tensor shaped like q")
        check_out_storage(out, [q] + [t for pair in segments for t in pair])
        self.q, self.segments, self.output = q, segments, out
        d = N.GqaDesc()
        d.T, d.Hq, d.Hkv, d.D, d.num_segments = t, hq, hkv, 128, len(segments)
        for i, (k, v) in enumerate(segments):
            d.len[i] = k.shape[0]
            d.k[i] = k.data_ptr() if k.shape[0] else None
            d.v[i] = v.data_ptr() if v.shape[0] else None
            d.k_stride[i] = k.stride(0) if k.shape[0] else hkv * 128
            d.v_stride[i] = v.stride(0) if v.shape[0] else hkv * 128
        d.q, d.out = q.data_ptr(), out.data_ptr()
        d.scale = float(scale) if scale is not None else 1.0 / math.sqrt(128.0)
        nbytes = ctypes.c_size_t(0)
        with torch.cuda.device(q.device):
            N.check(N.lib().gqa_seg_workspace_bytes(ctypes.byref(d), ctypes.byref(nbytes)), "prepare")
            self.workspace = torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=q.device)
            d.workspace, d.workspace_bytes = self.workspace.data_ptr(), self.workspace.numel()
            handle = ctypes.c_void_p()
            N.check(N.lib().gqa_seg_plan_create(ctypes.byref(handle), ctypes.byref(d)), "prepare")
        self._desc, self._plan = d, handle
        self.splits_workspace_bytes = int(nbytes.value)

    def run(self):
        if self.q.shape[0] == 0:
            return self.output
        stream = torch.cuda.current_stream(self.q.device).cuda_stream
        N.check(N.lib().gqa_seg_plan_run(self._plan, ctypes.c_void_p(stream)), "run")
        return self.output

    def __del__(self):
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            try:
                N.lib().gqa_seg_plan_destroy(plan)
            except Exception:
                pass
            self._plan = None


def prepare_segmented_gqa(q, segments, out=None, *, scale=None):
    plan = PreparedSegmentedGQA(q, segments, out, scale)
    plan.run()
    return plan


def prepare_cuda_gqa_compact(q, segments, out=None, *, stages=1):
    """Reference entry point (attention_cuda_compact.py:135); ``stages`` is
    accepted for compatibility -- the gfx950 kernel's pipeline is fixed."""
    if stages not in (1, 2):
        raise ValueError("stages must be 1 or 2")
    return prepare_segmented_gqa(q, segments, out)
