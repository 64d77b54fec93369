"""CPU restatement of the reference MoE semantics (test infrastructure only).

This module is the checker for the HIP path in ``llm_gpu_kernels_amd``.  It
runs on the host with PyTorch CPU tensors and is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.
Every function names the reference file:line it restates (paths relative to
the reference repository root).

Pinning of each function (what a plausible mistake would fail):
  * make_ids / make_inputs / tensor_hash: the reference's recorded
    ``routing_sha256`` / ``input_sha256`` digests and expected counts/offsets
    for 21 cases (tests/golden/m4_reference_records.json).
  * moe_reference: brute-force pure-Python loops on tiny shapes, closed forms
    (E=1 identity, linearity in routing weights, duplicate IDs).
  * staged_bf16_oracle: tolerance against moe_reference (it is a
    rounding-staged variant of the same sum).
  * route_topk: brute-force sort of softmax probabilities.
  * canonical_dispatch: brute-force stable ranks and the reference's dispatch
    invariants plus the golden counts/offsets.
  * quantize_w4 / dequantize_w4: closed-form special cases (all-zero group,
    extremal values, half-way ties, nibble order) and round trip.
  * m24_repack: element positions computed by hand from the reference's
    LAYOUT string on distinct-valued inputs, the reference's physical shapes
    for the Qwen logical shape, and bijectivity.
  * gqa_segmented_reference: PyTorch SDPA math backend on concatenated KV.
"""
from __future__ import annotations

import hashlib
import math

import torch
import torch.nn.functional as F

# Tolerances of this build (stricter than the reference's 0.008/0.008 of
# src/llm_gpu_kernels/benchmark.py:20).
LIMITS = {"relative_rms": 5e-3, "normalized_max": 1e-2}

STATUS_BAD_ID = 1        # moe_ranked.py:26-31 bit 0
STATUS_BAD_WEIGHT = 2    # moe_ranked.py:26-31 bit 1
STATUS_BAD_LOGIT = 4     # build extension: non-finite router logit


# --------------------------------------------------------------------------
# Seeded synthetic inputs (src/llm_gpu_kernels/moe_benchmark.py:43-82)
# --------------------------------------------------------------------------
def make_ids(tokens, experts, topk, pattern, generator):
    """Fixed routes drawn on the CPU generator (moe_benchmark.py:43-64)."""
    if topk < 1 or topk > experts:
        raise ValueError("topk must be in [1, experts]")
    if tokens == 0:
        return torch.empty((0, topk), dtype=torch.int64)
    if pattern == "duplicate":
        base = torch.arange(tokens, dtype=torch.int64)[:, None] % experts
        slots = torch.arange(topk, dtype=torch.int64)[None, :]
        return (base + slots // 2) % experts
    if pattern == "all_hot":
        return torch.zeros((tokens, topk), dtype=torch.int64)
    if pattern == "hot":
        hot = min(experts, max(topk, experts // 8))
        hot_experts = torch.randperm(experts, generator=generator)[:hot]
        choice = torch.rand((tokens, hot), generator=generator)
        return hot_experts[choice.topk(topk, dim=1).indices]
    if pattern in ("random", "uniform_random"):
        scores = torch.rand((tokens, experts), generator=generator)
        return scores.topk(topk, dim=1).indices
    raise ValueError(f"unknown route pattern: {pattern}")


def make_inputs(*, tokens, experts, topk, hidden, intermediate, id_dtype, pattern, seed,
                signed_weights=False):
    """x, gate_up, down, ids, routing weights on the CPU (moe_benchmark.py:67-82).

    ``signed_weights`` applies the ``sub_(0.5)`` of moe_benchmark.py:405-406.
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((tokens, hidden), generator=g).to(torch.bfloat16)
    gate_up = torch.randn((experts, 2 * intermediate, hidden), generator=g).to(torch.bfloat16)
    down = torch.randn((experts, hidden, intermediate), generator=g).to(torch.bfloat16)
    ids = make_ids(tokens, experts, topk, pattern, g).to(id_dtype)
    rw = torch.rand((tokens, topk), generator=g, dtype=torch.float32)
    if signed_weights:
        rw.sub_(0.5)
    return x, gate_up, down, ids, rw


def tensor_hash(*tensors):
    """sha256 over (shape, dtype) text and raw bytes (benchmark.py:41-46)."""
    digest = hashlib.sha256()
    for t in tensors:
        digest.update(str((tuple(t.shape), str(t.dtype))).encode())
        digest.update(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes())
    return digest.hexdigest()


# --------------------------------------------------------------------------
# Error metric (src/llm_gpu_kernels/benchmark.py:28-38)
# --------------------------------------------------------------------------
def error(actual, oracle, limits=LIMITS):
    if actual.shape != oracle.shape:
        raise ValueError(f"shape mismatch {tuple(actual.shape)} != {tuple(oracle.shape)}")
    if actual.numel() == 0:
        return {"relative_rms": 0.0, "normalized_max": 0.0, "max_abs": 0.0,
                "finite": True, "passed": True}
    a, o = actual.detach().float().cpu(), oracle.detach().float().cpu()
    d = a - o
    rel = (d.square().mean().sqrt() / o.square().mean().sqrt().clamp_min(1e-12)).item()
    nmax = (d.abs().max() / o.abs().max().clamp_min(1e-12)).item()
    m = {"relative_rms": rel, "normalized_max": nmax, "max_abs": d.abs().max().item(),
         "finite": bool(torch.isfinite(a).all())}
    m["passed"] = m["finite"] and rel <= limits["relative_rms"] and nmax <= limits["normalized_max"]
    return m


# --------------------------------------------------------------------------
# FP32 semantic oracle (src/llm_gpu_kernels/reference.py:17-45)
# --------------------------------------------------------------------------
def moe_reference(x, gate_up, down, expert_ids, routing_weights):
    """Per-expert FP32 loop: sum_s w[t,s] * down(silu(gate x) * up x).

    Duplicate IDs in one token contribute separately (reference.py:20-22).
    """
    e, h, inter = down.shape
    if gate_up.shape != (e, 2 * inter, h) or x.shape[1] != h:
        raise ValueError("incompatible MoE shapes")
    if expert_ids.shape != routing_weights.shape or expert_ids.shape[0] != x.shape[0]:
        raise ValueError("incompatible route shapes")
    if torch.any((expert_ids < 0) | (expert_ids >= e)) or not torch.isfinite(routing_weights).all():
        raise ValueError("invalid expert IDs or nonfinite routing weights")
    out = torch.zeros((x.shape[0], h), dtype=torch.float32)
    xf = x.float()
    for expert in range(e):
        tokens, slots = torch.where(expert_ids == expert)
        if tokens.numel() == 0:
            continue
        proj = xf[tokens] @ gate_up[expert].float().T
        gate, up = proj[:, :inter], proj[:, inter:]
        value = (F.silu(gate) * up) @ down[expert].float().T
        out.index_add_(0, tokens, value * routing_weights[tokens, slots, None].float())
    return out


def staged_bf16_oracle(x, gate_up, down, expert_ids, routing_weights):
    """M4 rounding stages (moe_benchmark.py:85-111; moe_fused.py:64-73; moe.py:109-121).

    bf16(gate), bf16(up) -> FP32 SwiGLU -> bf16 act -> bf16 down -> FP32
    weighted sum in slot order -> bf16.  The projections are computed in FP32
    and rounded, which is what an FP32-accumulating kernel produces.
    """
    t, h = x.shape
    k = expert_ids.shape[1]
    inter = down.shape[2]
    if t == 0:
        return torch.empty((0, h), dtype=torch.bfloat16)
    route_values = torch.zeros((t, k, h), dtype=torch.float32)
    xf = x.float()
    for expert in range(gate_up.shape[0]):
        tok, slots = torch.where(expert_ids == expert)
        if tok.numel() == 0:
            continue
        proj = xf[tok] @ gate_up[expert].float().T
        gate = proj[:, :inter].to(torch.bfloat16).float()
        up = proj[:, inter:].to(torch.bfloat16).float()
        act = (gate / (1.0 + torch.exp(-gate)) * up).to(torch.bfloat16)
        route_values[tok, slots] = (act.float() @ down[expert].float().T).to(torch.bfloat16).float()
    acc = torch.zeros((t, h), dtype=torch.float32)
    for s in range(k):  # fixed slot order, unfused multiply then add (moe.py:114-121)
        acc = acc + route_values[:, s] * routing_weights[:, s, None].float()
    return acc.to(torch.bfloat16)


# --------------------------------------------------------------------------
# Router (scripts/capture_qwen3_moe_layer0.py:583-586)
# --------------------------------------------------------------------------
def route_topk(logits, topk, renormalize=True):
    """softmax(fp32) -> top-k (descending, ties to the lower expert) -> renormalise.

    Returns (ids int32 [T,K], weights fp32 [T,K]).  Softmax is monotone, so
    the selection equals the top-k of the logits themselves; the tie rule is
    this build's (torch leaves it unspecified).
    """
    probs = torch.softmax(logits.float(), dim=-1)
    t, e = probs.shape
    ids = torch.empty((t, topk), dtype=torch.int32)
    w = torch.empty((t, topk), dtype=torch.float32)
    for row in range(t):
        order = sorted(range(e), key=lambda j: (-float(logits[row, j]), j))[:topk]
        ids[row] = torch.tensor(order, dtype=torch.int32)
        w[row] = probs[row, order]
    if renormalize and t:
        w = w / w.sum(dim=-1, keepdim=True)
    return ids, w


# --------------------------------------------------------------------------
# Canonical permutation (build-defined; satisfies moe_benchmark.py:139-190 and
# ranked_moe_benchmark.py:120-167 invariants)
# --------------------------------------------------------------------------
def canonical_dispatch(ids, experts):
    """Stable grouping of routes q = t*K + s by expert.

    counts[e] = #routes of e; offsets = exclusive scan; rank[q] = #{q' < q :
    id[q'] == id[q]}; map[q] = offsets[id[q]] + rank[q]; row_route is the
    inverse of map.  Invalid IDs get rank = map = -1 and are not counted
    (moe_ranked.py:32-37, moe_ranked.py:52-59).
    """
    flat = ids.reshape(-1).to(torch.int64)
    r = flat.numel()
    counts = [0] * experts
    ranks = [-1] * r
    for q in range(r):
        e = int(flat[q])
        if 0 <= e < experts:
            ranks[q] = counts[e]
            counts[e] += 1
    offsets, run = [], 0
    for c in counts:
        offsets.append(run)
        run += c
    mapping = [offsets[int(flat[q])] + ranks[q] if ranks[q] >= 0 else -1 for q in range(r)]
    row_route = [-1] * r
    for q, p in enumerate(mapping):
        if p >= 0:
            row_route[p] = q
    as_t = lambda v: torch.tensor(v, dtype=torch.int32)
    return {"counts": as_t(counts), "offsets": as_t(offsets), "ranks": as_t(ranks),
            "map": as_t(mapping), "row_route": as_t(row_route)}


# --------------------------------------------------------------------------
# W4G128 format (src/llm_gpu_kernels/moe_weight_quant.py:35-105)
# --------------------------------------------------------------------------
W4_GROUP = 128


def quantize_w4(weight):
    """Symmetric int4 along K, group 128 (moe_weight_quant.py:55-105).

    weight: CPU bf16 [E, N, K] with K % 128 == 0.  scale = bf16(max|w|/7)
    (1 where max == 0); q = clamp(round_half_even(w / scale), -7, 7);
    nibble q + 8; word j holds K = 8j..8j+7 with the earliest K in the low
    nibble.  Returns (words int32 [E, N, K/8], scales bf16 [E, N, K/128]).
    """
    e, n, k = weight.shape
    if k % W4_GROUP:
        raise ValueError("K must be a multiple of 128")
    x = weight.float().reshape(e, n, k // W4_GROUP, W4_GROUP)
    max_abs = x.abs().amax(-1)
    scale = torch.where(max_abs == 0, torch.ones_like(max_abs), max_abs / 7).to(torch.bfloat16)
    q = torch.round(x / scale.float()[..., None]).clamp(-7, 7).to(torch.int64)
    shifts = torch.arange(8, dtype=torch.int64) * 4
    word = ((q.reshape(e, n, k // 8, 8) + 8) << shifts).sum(-1)
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)
    return word, scale


def dequantize_w4(words, scales):
    """bf16_rn(float(nibble - 8) * float(scale)) (moe_weight_quant.py:35-52)."""
    e, n, kw = words.shape
    shifts = torch.arange(8, dtype=torch.int64) * 4
    nib = (words.to(torch.int64)[..., None] >> shifts) & 15
    q = (nib.reshape(e, n, kw * 8 // W4_GROUP, W4_GROUP) - 8).float()
    return (q * scales.float()[..., None]).reshape(e, n, kw * 8).to(torch.bfloat16)


def dequantize_w4_unrounded(words, scales):
    """float(nibble - 8) * float(scale) in fp32, not rounded to bf16: the
    effective weights of the opt-in folded decode (no counterpart in the
    reference).  Exact: an int4 times an 8-bit-significand scale has at most
    12 significant bits; rounding it to bf16 gives dequantize_w4."""
    e, n, kw = words.shape
    shifts = torch.arange(8, dtype=torch.int64) * 4
    nib = (words.to(torch.int64)[..., None] >> shifts) & 15
    q = (nib.reshape(e, n, kw * 8 // W4_GROUP, W4_GROUP) - 8).float()
    return (q * scales.float()[..., None]).reshape(e, n, kw * 8)


def m24_repack(words, scales):
    """v1 -> M24 physical layout, the reference's permutation
    (src/llm_gpu_kernels/moe_weight_layout.py:85-88, LAYOUT at :14-17 with
    Ntile = 64 rows): words [E, N, K/8] viewed as [E, 2, N/128, 64, K/32, 4]
    and permuted to [E, 2, N/128, K/32, 4, 64]; scales [E, N, K/128] viewed as
    [E, 2, N/128, 64, K/128] and permuted to [E, 2, N/128, K/128, 64]."""
    e, n, kw = words.shape
    nt = n // 128
    w = words.reshape(e, 2, nt, 64, kw // 4, 4).permute(0, 1, 2, 4, 5, 3).contiguous()
    s = scales.reshape(e, 2, nt, 64, scales.shape[2]).permute(0, 1, 2, 4, 3).contiguous()
    return w, s


# --------------------------------------------------------------------------
# Segmented-KV GQA prefill (tests/e2e/test_compact_attention.py:49-78;
# docs/MOE_USAGE.md:128-134)
# --------------------------------------------------------------------------
def gqa_segmented_reference(q, segments):
    """FP32 SDPA math over the concatenation of the KV segments.

    q: [T, Hq, D]; segments: sequence of (k, v) with [L, Hkv, D]; the last
    segment is the current chunk (L == T) and is causal (key j visible to
    query i iff j <= i); the earlier segments are fully visible.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel
    t, hq, d = q.shape
    if t == 0:
        return torch.empty((0, hq, d), dtype=torch.float32)
    hkv = segments[0][0].shape[1]
    group = hq // hkv
    history = sum(k.shape[0] for k, _ in segments[:-1])
    keys = torch.cat([k.float().cpu() for k, _ in segments], 0)
    values = torch.cat([v.float().cpu() for _, v in segments], 0)
    keys = keys.repeat_interleave(group, dim=1).permute(1, 0, 2).unsqueeze(0)
    values = values.repeat_interleave(group, dim=1).permute(1, 0, 2).unsqueeze(0)
    query = q.float().cpu().permute(1, 0, 2).unsqueeze(0)
    pos = torch.arange(t)
    allowed = torch.ones((t, keys.shape[-2]), dtype=torch.bool)
    allowed[:, history:] = pos[None, :] <= pos[:, None]
    with sdpa_kernel(SDPBackend.MATH):
        out = F.scaled_dot_product_attention(query, keys, values, attn_mask=allowed,
                                             dropout_p=0.0, is_causal=False,
                                             scale=1.0 / math.sqrt(d))
    return out.squeeze(0).permute(1, 0, 2)
