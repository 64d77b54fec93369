"""Parity of the HIP MoE forward against the CPU oracle (MI355X only).

Bit-exact: router IDs, counts, offsets, canonical ranks, map, its inverse,
the task list and W4 dequantised values.  Tolerance (rel-RMS <= 5e-3,
normalised max <= 1e-2) for layer outputs against the FP32 oracle; the
reference's functional specs (N(0,1) weights) use the reference's own
0.008/0.008 limits against the FP32 oracle plus a tight check against the
rounding-staged oracle.
"""
import json
from pathlib import Path

import pytest
import torch

from llm_gpu_kernels_amd import (GemmConfig, dequantize_tiled, prepare_moe, prepare_routed_moe,
                                 prepare_w4_layout_moe, repack_gate_up,
                                 prepare_w4_moe, quantize_gate_up, tile_gate_up)
from llm_gpu_kernels_amd.workloads import make_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "m4_reference_records.json").read_text())
FUNCTIONAL = [c for c in GOLDEN["cases"] if c["family"] == "functional_cases"]
SMALL_PERF = [c for c in GOLDEN["cases"] if c["family"] == "performance_cases" and c["E"] == 16]
DT = {"torch.int32": torch.int32, "torch.int64": torch.int64}
REF_LIMITS = {"relative_rms": 0.008, "normalized_max": 0.008}
STAGED_LIMITS = {"relative_rms": 2e-3, "normalized_max": 8e-3}


def _to(dev, *ts):
    return [t.to(dev) for t in ts]


def _check_dispatch(plan, ids_cpu, experts):
    d = O.canonical_dispatch(ids_cpu, experts)
    torch.cuda.synchronize()
    assert torch.equal(plan.counts.cpu(), d["counts"])
    assert torch.equal(plan.offsets.cpu(), d["offsets"])
    assert torch.equal(plan.ranks.cpu(), d["ranks"])
    assert torch.equal(plan.mapping.cpu(), d["map"])
    assert torch.equal(plan.row_route.cpu(), d["row_route"])
    # Task list: expert-major blocks of token_block rows covering every row once.
    tb = plan.layout.token_block
    n = int(plan.num_tasks.item())
    tasks = plan.tasks[:n].cpu().tolist()
    expect = []
    for e in range(experts):
        c, off = int(d["counts"][e]), int(d["offsets"][e])
        expect += [[e, off + r0, min(tb, c - r0), 0] for r0 in range(0, c, tb)]
    assert tasks == expect


@pytest.mark.parametrize("case", FUNCTIONAL + SMALL_PERF, ids=lambda c: c["name"])
def test_reference_functional_specs(case, gpu_device):
    x, gu, dn, ids, rw = O.make_inputs(tokens=case["T"], experts=case["E"], topk=case["topk"],
                                       hidden=case["H"], intermediate=case["I"],
                                       id_dtype=DT[case["id_dtype"]], pattern=case["route_pattern"],
                                       seed=case["seed"], signed_weights=case.get("signed_weights", False))
    assert O.tensor_hash(ids) == case["routing_sha256"]
    dev = _to(gpu_device, x, gu, dn, ids, rw)
    plan = prepare_moe(*dev)
    out = plan.run()
    torch.cuda.synchronize()
    assert out.shape == (case["T"], case["H"]) and out.dtype == torch.bfloat16
    if case["T"] == 0:
        assert plan.launches == ()
        return
    plan.check_inputs()
    _check_dispatch(plan, ids, case["E"])
    m32 = O.error(out, O.moe_reference(x, gu, dn, ids, rw), REF_LIMITS)
    ms = O.error(out, O.staged_bf16_oracle(x, gu, dn, ids, rw), STAGED_LIMITS)
    assert m32["passed"], m32
    assert ms["passed"], ms


def test_token_block_invariance(gpu_device):
    """Streaming kernels: each grouped row's arithmetic is independent of the
    task size (16 or 32 rows), so the outputs are bitwise equal."""
    lay = make_layer("qwen", 193, seed=3, device=gpu_device)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    args = (lay["x"], lay["gate_up"], lay["down"], ids.to(gpu_device), w.to(gpu_device))
    pa = prepare_moe(*args, config=GemmConfig(block_m=16))
    pb = prepare_moe(*args, config=GemmConfig(block_m=32))
    assert pa.layout.fast_path == 1 and pb.layout.fast_path == 1
    a, b = pa.run().clone(), pb.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("tokens,w4", [(17, False), (193, False), (193, True)])
def test_tiled_path_forced(tokens, w4, gpu_device):
    """LDS-tiled kernels (64-row tasks) on small T: partial tiles and tail rows."""
    lay = make_layer("qwen", tokens, seed=4, device=gpu_device)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    gate_up, ref_gu = lay["gate_up"], lay["gate_up"].cpu()
    if w4:
        packed = quantize_gate_up(ref_gu)
        gate_up = tile_gate_up(packed).to(gpu_device)
        ref_gu = O.dequantize_w4(packed.words, packed.scales)
        plan = prepare_w4_moe(lay["x"], gate_up, lay["down"], ids.to(gpu_device), w.to(gpu_device),
                              down_config=GemmConfig(block_m=64))
    else:
        plan = prepare_moe(lay["x"], gate_up, lay["down"], ids.to(gpu_device), w.to(gpu_device),
                           config=GemmConfig(block_m=64))
    assert plan.layout.fast_path == 2
    out = plan.run()
    torch.cuda.synchronize()
    m = O.error(out, O.moe_reference(lay["x"].cpu(), ref_gu, lay["down"].cpu(), ids, w))
    assert m["passed"], m


def _ids_with_counts(counts, tokens, k):
    """[tokens, k] expert IDs whose per-expert counts are `counts` (each <= tokens):
    route q = k_slot * tokens + t takes the q-th entry of the expert-sorted list, so
    an expert's routes are consecutive q and land on distinct tokens."""
    flat = torch.repeat_interleave(torch.arange(len(counts)), torch.tensor(counts))
    assert flat.numel() == tokens * k and max(counts) <= tokens
    return flat.view(k, tokens).t().contiguous().to(torch.int32)


def test_w4_pair_passes_at_task_boundaries(gpu_device):
    """W4 gate/up with 64-row tasks (the pair kernel): experts with 1, 33, 64, 65, 96,
    97, 129 and 160 rows cover a single short task, a full task, two tasks run as one
    96-row pass, two tasks run separately and three tasks; every grouped row is
    checked against the FP32 oracle on the dequantised weights."""
    tokens, k, e = 160, 8, 128
    special = [96, 97, 65, 64, 129, 160, 1, 33]
    rest = tokens * k - sum(special)
    counts = special + [rest // (e - 8) + (1 if i < rest % (e - 8) else 0) for i in range(e - 8)]
    ids = _ids_with_counts(counts, tokens, k)
    lay = make_layer("qwen", tokens, seed=6, device=gpu_device)
    w = torch.softmax(torch.randn(tokens, k, generator=torch.Generator().manual_seed(6)), dim=-1)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    tiled = tile_gate_up(packed).to(gpu_device)
    ref_gu = O.dequantize_w4(packed.words, packed.scales)
    plan = prepare_w4_moe(lay["x"], tiled, lay["down"], ids.to(gpu_device), w.to(gpu_device),
                          down_config=GemmConfig(block_m=64))
    assert plan.layout.fast_path == 2
    out = plan.run()
    torch.cuda.synchronize()
    assert plan.base.counts.cpu().tolist() == counts
    m = O.error(out, O.moe_reference(lay["x"].cpu(), ref_gu, lay["down"].cpu(), ids.long(), w))
    assert m["passed"], m


CONFIGS = [("tiny", 17, "uniform"), ("qwen", 17, "uniform"), ("qwen", 193, "uniform"),
           ("qwen", 1024, "zipf"), ("qwen", 1024, "uniform")]


def _routed_parity(shape, tokens, routing, gpu_device, w4=False, expect_path=None):
    lay = make_layer(shape, tokens, routing=routing, seed=0, device=gpu_device)
    k = lay["K"]
    gate_up = lay["gate_up"]
    if w4:
        packed = quantize_gate_up(gate_up.cpu())
        tiled = tile_gate_up(packed).to(gpu_device)
        deq = dequantize_tiled(tiled)
        torch.cuda.synchronize()
        ref_deq = O.dequantize_w4(packed.words, packed.scales)
        assert torch.equal(deq.cpu().view(torch.int16), ref_deq.view(torch.int16))
        weights_for_oracle = ref_deq
        gate_up = tiled
    else:
        weights_for_oracle = gate_up.cpu()
    plan = prepare_routed_moe(lay["x"], lay["logits"], gate_up, lay["down"], k)
    if expect_path is None:
        expect_path = 2 if tokens * k >= 32 * lay["E"] else 1
    assert plan.layout.fast_path == expect_path
    out = plan.forward(lay["x"], lay["logits"])
    torch.cuda.synchronize()
    plan.check_inputs()
    logits = lay["logits"].cpu()
    ids, w = O.route_topk(logits, k)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, lay["E"])
    x, dn = lay["x"].cpu(), lay["down"].cpu()
    m = O.error(out, O.moe_reference(x, weights_for_oracle, dn, ids, w))
    assert m["passed"], m
    return plan


@pytest.mark.parametrize("shape,tokens,routing", CONFIGS, ids=lambda v: str(v))
def test_routed_bf16_layer(shape, tokens, routing, gpu_device):
    _routed_parity(shape, tokens, routing, gpu_device)


@pytest.mark.parametrize("tokens", [17, 193, 1024])
def test_routed_w4_layer(tokens, gpu_device):
    _routed_parity("qwen", tokens, "uniform", gpu_device, w4=True)


@pytest.mark.parametrize("tokens", [17, 193, 1024])
def test_routed_w4_fold_layer(tokens, gpu_device):
    """Opt-in folded W4 decode (group scale on the fp32 group sum): within
    tolerance of the FP32 oracle on the unrounded q * scale weights, router IDs
    bit-exact, bitwise repeatable; at T = 17 (the split-K streaming kernel that
    implements the fold) it differs from the exact decode's output."""
    lay = make_layer("qwen", tokens, seed=0, device=gpu_device)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    tiled = tile_gate_up(packed).to(gpu_device)
    plan = prepare_routed_moe(lay["x"], lay["logits"], tiled, lay["down"], lay["K"], w4_decode="fold")
    out = plan.forward(lay["x"], lay["logits"]).clone()
    again = plan.forward(lay["x"], lay["logits"]).clone()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    ids, w = O.route_topk(lay["logits"].cpu(), lay["K"])
    assert torch.equal(plan.ids.cpu(), ids)
    un = O.dequantize_w4_unrounded(packed.words, packed.scales)
    m = O.error(out, O.moe_reference(lay["x"].cpu(), un, lay["down"].cpu(), ids, w))
    assert m["passed"], m
    if tokens == 17:
        exact = prepare_routed_moe(lay["x"], lay["logits"], tiled, lay["down"], lay["K"])
        ex = exact.forward(lay["x"], lay["logits"])
        torch.cuda.synchronize()
        assert not torch.equal(ex.view(torch.int16), out.view(torch.int16))
    with pytest.raises(ValueError):
        prepare_routed_moe(lay["x"], lay["logits"], tiled, lay["down"], lay["K"], w4_decode="bf16")


@pytest.mark.parametrize("shift", ["x+3", "abs(x)+1", "x+16"])
def test_w4_fold_offset_heavy_inputs(shift, gpu_device):
    """The folded decode computes scale * (sum((136 + q) x) - 136 sum(x)) per
    128-K group in fp32, so its rounding error grows with the common offset of
    x (the two terms cancel).  With activations shifted away from zero it stays
    within the layer tolerance of the FP32 oracle on the unrounded weights;
    the printed errors are the bound recorded for the fold mode."""
    lay = make_layer("qwen", 17, seed=0, device=gpu_device)
    x = lay["x"].float()
    x = {"x+3": x + 3.0, "abs(x)+1": x.abs() + 1.0, "x+16": x + 16.0}[shift].to(torch.bfloat16)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    tiled = tile_gate_up(packed).to(gpu_device)
    plan = prepare_routed_moe(x, lay["logits"], tiled, lay["down"], lay["K"], w4_decode="fold")
    out = plan.forward(x, lay["logits"])
    torch.cuda.synchronize()
    ids, w = O.route_topk(lay["logits"].cpu(), lay["K"])
    un = O.dequantize_w4_unrounded(packed.words, packed.scales)
    m = O.error(out, O.moe_reference(x.cpu(), un, lay["down"].cpu(), ids, w))
    exact = prepare_routed_moe(x, lay["logits"], tiled, lay["down"], lay["K"])
    ex = exact.forward(x, lay["logits"])
    torch.cuda.synchronize()
    me = O.error(ex, O.moe_reference(x.cpu(), O.dequantize_w4(packed.words, packed.scales),
                                     lay["down"].cpu(), ids, w))
    print(f"fold {shift}: {m}  exact: {me}")
    assert m["passed"], m


# One GPU's share of the Qwen layer under 8-way expert parallelism (16 experts,
# one route per row: the streaming and the tiled kernels) and tensor parallelism
# (I = 96: the run-time-K kernels), as the bench measures them.
SHARD_CONFIGS = [("qwen-ep8", 17, "uniform", False, 1), ("qwen-ep8", 1024, "uniform", False, 2),
                 ("qwen-tp8", 17, "uniform", False, 0), ("qwen-tp8", 1024, "zipf", False, 0),
                 ("qwen-tp8", 17, "uniform", True, 0)]


@pytest.mark.parametrize("shape,tokens,routing,w4,path", SHARD_CONFIGS, ids=lambda v: str(v))
def test_parallel_shard_shapes(shape, tokens, routing, w4, path, gpu_device):
    _routed_parity(shape, tokens, routing, gpu_device, w4=w4, expect_path=path)


@pytest.mark.parametrize("tokens", [17, 193])
def test_w4_token_blocks(tokens, gpu_device):
    """W4 gate/up with 16-, 32- and 64-row tasks: at T=17 the split-K streaming kernel
    (16, 32 rows) and the one-unit-per-wave kernel (64 rows); at T=193 the wave kernel
    with 1, 2 and 4 token blocks per fragment.  Each within tolerance of the FP32
    oracle on the dequantised weights, and of the 16-row result."""
    lay = make_layer("qwen", tokens, seed=5, device=gpu_device)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    tiled = tile_gate_up(packed).to(gpu_device)
    ref = O.moe_reference(lay["x"].cpu(), O.dequantize_w4(packed.words, packed.scales),
                          lay["down"].cpu(), ids, w)
    outs = {}
    for bm in (16, 32, 64):
        plan = prepare_w4_moe(lay["x"], tiled, lay["down"], ids.to(gpu_device), w.to(gpu_device),
                              down_config=GemmConfig(block_m=bm))
        assert plan.layout.token_block == bm
        out = plan.run().clone()
        torch.cuda.synchronize()
        m = O.error(out, ref)
        assert m["passed"], (bm, m)
        outs[bm] = out
    for bm in (32, 64):
        m = O.error(outs[bm], outs[16].float().cpu())
        assert m["passed"], (bm, m)


# (tokens, experts, topk, H, I, W4): shapes outside the tuned kernels' compile-time K
# steps -- GPT-OSS-like H = 2880, DeepSeek-like H = 7168, H/I = 1056/608, W4 H = 1152 and
# 4096 -- through each run-time-K MFMA kernel (16/32/64-row tasks, bf16 and W4) and
# the W4 wave kernel taking a shape the split-K streaming kernel cannot.
FLEX_SHAPES = [
    (17, 8, 4, 2880, 1440, False),   # 16-row tasks
    (100, 8, 2, 2880, 1440, False),  # 32-row tasks
    (300, 8, 2, 1056, 608, False),   # 64-row tasks, I % 128 != 0
    (5, 4, 2, 7168, 512, False),
    (17, 8, 4, 4096, 512, True),     # W4: wave kernel gate/up, run-time-K down
    (9, 8, 2, 1152, 384, True),      # W4 run-time-K gate/up, 16-row tasks
    (100, 8, 2, 1152, 384, True),    # 32-row tasks
    (300, 8, 2, 1152, 384, True),    # 64-row tasks
    # K <= 256: the waves split the columns instead of K (gate/up at H = 256,
    # down at I = 96: one GPU's share of the Qwen layer under 8-way tensor parallelism)
    (100, 8, 2, 256, 96, False),     # 32-row tasks, both GEMMs column-split
    (300, 8, 2, 2048, 96, False),    # 64-row tasks, gate/up K-split, down column-split
    (17, 8, 4, 256, 96, True),       # W4 gate/up with two 128-wide groups, column-split
]


@pytest.mark.parametrize("tokens,experts,topk,hidden,inter,w4", FLEX_SHAPES,
                         ids=lambda v: str(v))
def test_run_time_k_shapes(tokens, experts, topk, hidden, inter, w4, gpu_device):
    """Shapes the compile-time-K kernels do not take run on the matrix cores
    (run-time-K MFMA kernels, or the W4 wave kernel) within tolerance of the
    FP32 oracle (dequantised weights for W4)."""
    x, gu, dn, ids, rw = O.make_inputs(tokens=tokens, experts=experts, topk=topk, hidden=hidden,
                                       intermediate=inter, id_dtype=torch.int32, pattern="random",
                                       seed=tokens + hidden + inter)
    xd, dnd, idd, rwd = _to(gpu_device, x, dn, ids, rw)
    if w4:
        packed = quantize_gate_up(gu)
        plan = prepare_w4_moe(xd, packed, dnd, idd, rwd)
        ref_gu = O.dequantize_w4(packed.words, packed.scales)
    else:
        plan = prepare_moe(xd, gu.to(gpu_device), dnd, idd, rwd)
        ref_gu = gu
    assert plan.layout.fast_path == 0
    out = plan.run().clone()
    torch.cuda.synchronize()
    assert plan.read_status() == 0
    m = O.error(out, O.moe_reference(x, ref_gu, dn, ids, rw))
    assert m["passed"], m


@pytest.mark.parametrize("tokens,experts,topk,hidden,inter,w4,block_m", [
    (200, 1, 1, 96, 32, False, 16),    # one expert: 13 tasks of 16 rows, K = 1
    (200, 1, 1, 96, 32, False, 64),    # 4 tasks of 64 rows, the last one ragged (8 rows)
    (1, 3, 2, 160, 64, False, 32),     # T = 1: one row per task
    (70, 2, 2, 128, 32, True, 64),     # W4: one 128-wide group per K-step
    (33, 5, 3, 384, 96, True, 16),
])
def test_run_time_k_edges(tokens, experts, topk, hidden, inter, w4, block_m, gpu_device):
    """Run-time-K kernels at their edges: minimal H and I, one expert with
    many tasks, K = 1, T = 1, ragged last tasks, int64 IDs; bitwise equal
    across two runs and within tolerance of the FP32 oracle."""
    x, gu, dn, ids, rw = O.make_inputs(tokens=tokens, experts=experts, topk=topk, hidden=hidden,
                                       intermediate=inter, id_dtype=torch.int64, pattern="random",
                                       seed=7 * tokens + hidden)
    xd, dnd, idd, rwd = _to(gpu_device, x, dn, ids, rw)
    cfg = GemmConfig(block_m=block_m)
    if w4:
        packed = quantize_gate_up(gu)
        plan = prepare_w4_moe(xd, packed, dnd, idd, rwd, down_config=cfg)
        ref_gu = O.dequantize_w4(packed.words, packed.scales)
    else:
        plan = prepare_moe(xd, gu.to(gpu_device), dnd, idd, rwd, config=cfg)
        ref_gu = gu
    assert plan.layout.fast_path == 0 and plan.layout.token_block == block_m
    a = plan.run().clone()
    b = plan.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert plan.read_status() == 0
    _check_dispatch(plan, ids, experts)
    m = O.error(a, O.moe_reference(x, ref_gu, dn, ids, rw))
    assert m["passed"], m


def test_w4_m24_layout_entry(gpu_device):
    """prepare_w4_layout_moe on the reference's M24 physical layout
    (moe_weight_layout.py:81-127) is bitwise the v1 entry's result."""
    lay = make_layer("qwen", 17, seed=11, device=gpu_device)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    ids, w = ids.to(gpu_device), w.to(gpu_device)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    a = prepare_w4_moe(lay["x"], packed, lay["down"], ids, w).run().clone()
    b = prepare_w4_layout_moe(lay["x"], repack_gate_up(packed), lay["down"], ids, w).run().clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("tokens", [1, 2, 5, 33])
@pytest.mark.parametrize("w4", [False, True])
def test_streaming_unit_blocks(tokens, w4, gpu_device):
    """Qwen shape at small T: fewer units than workgroups (T=1), a unit block
    per workgroup spanning several tasks (T=33), every expert receiving one
    route or many; the streaming kernels' unit blocks against the oracle."""
    lay = make_layer("qwen", tokens, seed=40 + tokens, device=gpu_device)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    ids, w = ids.to(gpu_device), w.to(gpu_device)
    if w4:
        packed = quantize_gate_up(lay["gate_up"].cpu())
        plan = prepare_w4_moe(lay["x"], packed, lay["down"], ids, w)
        ref_gu = O.dequantize_w4(packed.words, packed.scales)
    else:
        plan = prepare_moe(lay["x"], lay["gate_up"], lay["down"], ids, w)
        ref_gu = lay["gate_up"].cpu()
    assert plan.layout.fast_path == 1
    out = plan.run().clone()
    torch.cuda.synchronize()
    ref = O.moe_reference(lay["x"].cpu(), ref_gu, lay["down"].cpu(), ids.cpu(), w.cpu())
    m = O.error(out, ref)
    assert m["passed"], m


def test_streaming_one_hot_expert(gpu_device):
    """Every route of every token on expert 5 (one task of 16 rows per 16
    routes, all units of the launch on one expert), then a re-run with spread
    routes on the same prepared object."""
    lay = make_layer("qwen", 4, seed=77, device=gpu_device)
    ids = torch.full((4, 8), 5, dtype=torch.int32, device=gpu_device)
    w = torch.full((4, 8), 0.125, dtype=torch.float32, device=gpu_device)
    plan = prepare_moe(lay["x"], lay["gate_up"], lay["down"], ids, w)
    out = plan.run().clone()
    torch.cuda.synchronize()
    ref = O.moe_reference(lay["x"].cpu(), lay["gate_up"].cpu(), lay["down"].cpu(), ids.cpu(), w.cpu())
    assert O.error(out, ref)["passed"]
    ni, nw = O.route_topk(lay["logits"].cpu(), 8)
    ids.copy_(ni.to(gpu_device))
    w.copy_(nw.to(gpu_device))
    out = plan.run().clone()
    torch.cuda.synchronize()
    ref = O.moe_reference(lay["x"].cpu(), lay["gate_up"].cpu(), lay["down"].cpu(), ni, nw)
    assert O.error(out, ref)["passed"]


def test_status_bits(gpu_device):
    x, gu, dn, ids, rw = O.make_inputs(tokens=3, experts=4, topk=2, hidden=128, intermediate=128,
                                       id_dtype=torch.int32, pattern="random", seed=101)
    x, gu, dn, ids, rw = _to(gpu_device, x, gu, dn, ids, rw)
    plan = prepare_moe(x, gu, dn, ids, rw)
    plan.check_inputs()
    ids[0, 0] = 4
    plan.run()
    assert plan.read_status() == 1
    with pytest.raises(ValueError):
        plan.check_inputs()
    rw[1, 1] = float("nan")
    plan.run()
    assert plan.read_status() == 3
    ids[0, 0] = 1
    plan.run()
    assert plan.read_status() == 2
    rw[1, 1] = 0.5
    plan.run()
    assert plan.read_status() == 0
    # Router mode: a NaN logit sets bit 2 (and the weights it poisons bit 1).
    lay = make_layer("tiny", 5, device=gpu_device)
    p2 = prepare_routed_moe(lay["x"], lay["logits"], lay["gate_up"], lay["down"], 2)
    p2.check_inputs()
    lay["logits"][2, 3] = float("nan")
    p2.forward()
    assert p2.read_status() & 4


def test_empty_tokens(gpu_device):
    x, gu, dn, ids, rw = O.make_inputs(tokens=0, experts=8, topk=2, hidden=128, intermediate=128,
                                       id_dtype=torch.int32, pattern="random", seed=1)
    plan = prepare_moe(*_to(gpu_device, x, gu, dn, ids, rw))
    assert plan.launches == () and plan.run().shape == (0, 128)


def test_graph_capture_with_in_place_updates(gpu_device):
    """Graph replays follow in-place value updates (docs/MOE_USAGE.md:126-180)."""
    lay = make_layer("qwen", 17, seed=5, device=gpu_device)
    plan = prepare_routed_moe(lay["x"], lay["logits"], lay["gate_up"], lay["down"], 8)
    for _ in range(3):
        plan.run()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=gpu_device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(4):
            gout = plan.run()
    for step in range(3):
        nxt = make_layer("qwen", 17, seed=100 + step, device=gpu_device, weights=False)
        lay["x"].copy_(nxt["x"])
        lay["logits"].copy_(nxt["logits"])
        graph.replay()
        torch.cuda.synchronize()
        replay = gout.clone()
        eager = plan.run().clone()
        torch.cuda.synchronize()
        assert torch.equal(replay.view(torch.int16), eager.view(torch.int16))
        ids, _ = O.route_topk(nxt["logits"].cpu(), 8)
        assert torch.equal(plan.ids.cpu(), ids)
    plan.check_inputs()


def test_non_default_stream(gpu_device):
    lay = make_layer("tiny", 33, seed=9, device=gpu_device)
    plan = prepare_routed_moe(lay["x"], lay["logits"], lay["gate_up"], lay["down"], 2)
    base = plan.run().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = plan.run().clone()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(base.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("tokens,experts,k", [(17, 128, 8), (32, 128, 8), (31, 60, 1), (20, 8, 2),
                                              (25, 128, 32), (16, 100, 3), (18, 33, 5),
                                              (12, 256, 8), (16, 160, 16)])
def test_fused_router_two_tokens_per_wave(tokens, experts, k, gpu_device):
    """The planner routes 17..32 tokens two per wave when E <= 128 (and one per
    wave up to 16, e.g. E = 160 or 256): IDs bit-exact with the oracle's top-k
    on logits full of ties (ties go to the lower expert), weights to fp32
    rounding, the layer within tolerance, and a NaN logit raises status bit 2."""
    x, gu, dn, _, _ = O.make_inputs(tokens=tokens, experts=experts, topk=k, hidden=128,
                                    intermediate=128, id_dtype=torch.int32, pattern="random",
                                    seed=tokens + experts)
    g = torch.Generator().manual_seed(7 * tokens + k)
    logits = torch.randint(-6, 6, (tokens, experts), generator=g).float() * 0.75
    plan = prepare_routed_moe(*_to(gpu_device, x, logits, gu, dn), k)
    assert plan.launch_names[0] != "router"
    out = plan.forward()
    torch.cuda.synchronize()
    ids, w = O.route_topk(logits, k)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, experts)
    m = O.error(out, O.moe_reference(x, gu, dn, ids, w))
    assert m["passed"], m
    assert plan.read_status() == 0
    plan.logits[tokens - 1, experts // 2] = float("nan")
    plan.forward()
    assert plan.read_status() & 4


@pytest.mark.parametrize("tokens", [17, 193, 384])
def test_work_counters_return_to_zero(tokens, gpu_device):
    """Qwen shape, bf16: the LDS-streaming gate/up and down launches hand out
    units from device-wide counters that the last workgroup of each launch
    resets.  After every forward the counters read zero, and forwards over
    new tokens (T = 17: routed in the gate/up prologue; T = 193: planner
    launch; T = 384: 32-row tasks) each match the oracle -- a unit skipped or taken twice by a
    stale counter would leave the previous forward's rows in the output."""
    lay = make_layer("qwen", tokens, seed=50 + tokens, device=gpu_device)
    g = torch.Generator().manual_seed(tokens)
    logits = torch.randn(tokens, lay["E"], generator=g).to(gpu_device)
    plan = prepare_routed_moe(lay["x"], logits, lay["gate_up"], lay["down"], 8)
    gu, dn = lay["gate_up"].cpu(), lay["down"].cpu()
    for it in range(3 if tokens <= 32 else 2):
        lay["x"].copy_((torch.randn(lay["x"].shape, generator=g) * 0.5).to(torch.bfloat16))
        logits.copy_(torch.randn(tokens, lay["E"], generator=g))
        out = plan.forward().clone()
        torch.cuda.synchronize()
        assert plan.work_counters.cpu().tolist() == [0, 0, 0, 0], it
        m = O.error(out, O.moe_reference(lay["x"].cpu(), gu, dn, plan.ids.cpu(),
                                         plan.routing_weights.cpu()))
        assert m["passed"], (it, m)


@pytest.mark.parametrize("tokens", [1, 2, 16, 17, 31, 32])
def test_gate_up_with_planning_prologue(tokens, gpu_device):
    """bf16 Qwen shape, T <= 32: the gate/up launch routes and plans in its
    prologue (no planner launch).  IDs bit-exact on tie-heavy logits, weights to
    fp32 rounding, every global plan array equal to the canonical dispatch,
    the layer within tolerance and bitwise equal to the fixed-route path on the
    same routes; a NaN logit raises status bit 2."""
    lay = make_layer("qwen", tokens, seed=tokens, device=gpu_device)
    g = torch.Generator().manual_seed(tokens)
    logits = (torch.randint(-6, 6, (tokens, lay["E"]), generator=g).float() * 0.75).to(gpu_device)
    plan = prepare_routed_moe(lay["x"], logits, lay["gate_up"], lay["down"], 8)
    assert plan.launch_names == ("gate_up_swiglu", "down", "combine")
    out = plan.forward().clone()
    torch.cuda.synchronize()
    ids, w = O.route_topk(logits.cpu(), 8)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, lay["E"])
    assert plan.read_status() == 0
    x, gu, dn = lay["x"].cpu(), lay["gate_up"].cpu(), lay["down"].cpu()
    m = O.error(out, O.moe_reference(x, gu, dn, ids, w))
    assert m["passed"], m
    fixed = prepare_moe(lay["x"], lay["gate_up"], lay["down"], plan.ids.clone(),
                        plan.routing_weights.clone())
    assert torch.equal(fixed.run().view(torch.int16), out.view(torch.int16))
    logits[tokens - 1, 5] = float("nan")
    plan.forward()
    assert plan.read_status() & 4


@pytest.mark.parametrize("tokens,experts,k", [(17, 128, 8), (32, 128, 15), (16, 160, 8), (9, 256, 4),
                                              (20, 128, 20), (24, 128, 21)])
def test_w4_prologue_router_modes(tokens, experts, k, gpu_device):
    """The W4 register-streaming gate/up routes in its prologue with 16 lanes
    per token (E <= 128, K <= 16: up to 32 tokens in one pass), one full wave
    per token, two tokens per wave interleaved (E > 128, T <= 16), or two
    half-waves per wave (K > 16, T <= 32).  Each mode: IDs bit-exact with the
    oracle's top-k on tie-heavy logits, weights to fp32 rounding, and the layer
    within tolerance of the FP32 oracle on the dequantised weights."""
    x, gu, dn, _, _ = O.make_inputs(tokens=tokens, experts=experts, topk=k, hidden=2048,
                                    intermediate=256, id_dtype=torch.int32, pattern="random",
                                    seed=tokens * experts + k)
    packed = quantize_gate_up(gu)
    tiled = tile_gate_up(packed).to(gpu_device)
    g = torch.Generator().manual_seed(3 * tokens + k)
    logits = torch.randint(-6, 6, (tokens, experts), generator=g).float() * 0.75
    plan = prepare_routed_moe(*_to(gpu_device, x, logits), tiled, dn.to(gpu_device), k)
    assert plan.launch_names == ("gate_up_swiglu", "down", "combine")
    out = plan.forward()
    torch.cuda.synchronize()
    ids, w = O.route_topk(logits, k)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, experts)
    assert plan.read_status() == 0
    m = O.error(out, O.moe_reference(x, O.dequantize_w4(packed.words, packed.scales), dn, ids, w))
    assert m["passed"], m


@pytest.mark.parametrize("tokens,decode", [(1, "exact"), (16, "exact"), (17, "exact"), (32, "exact"),
                                           (16, "fold"), (17, "fold"), (31, "fold")])
def test_w4_gate_up_with_planning_prologue(tokens, decode, gpu_device):
    """W4 Qwen shape, T <= 32: the register-streaming W4 gate/up routes and
    plans in its prologue (one token per wave in two rounds up to T = 16, two
    per wave above), so the forward is three launches.  IDs bit-exact on
    tie-heavy logits, every global plan array equal to the canonical dispatch,
    the work counters zero, the layer within tolerance, and bitwise equal to
    the fixed-route W4 path (planner launch) on the same routes."""
    lay = make_layer("qwen", tokens, seed=40 + tokens, device=gpu_device)
    packed = quantize_gate_up(lay["gate_up"].cpu())
    tiled = tile_gate_up(packed).to(gpu_device)
    g = torch.Generator().manual_seed(tokens + 1)
    logits = (torch.randint(-6, 6, (tokens, lay["E"]), generator=g).float() * 0.75).to(gpu_device)
    plan = prepare_routed_moe(lay["x"], logits, tiled, lay["down"], 8, w4_decode=decode)
    assert plan.launch_names == ("gate_up_swiglu", "down", "combine")
    out = plan.forward().clone()
    torch.cuda.synchronize()
    ids, w = O.route_topk(logits.cpu(), 8)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, lay["E"])
    assert plan.read_status() == 0
    assert plan.work_counters.cpu().tolist() == [0, 0, 0, 0]
    deq = (O.dequantize_w4_unrounded if decode == "fold" else O.dequantize_w4)(packed.words, packed.scales)
    m = O.error(out, O.moe_reference(lay["x"].cpu(), deq, lay["down"].cpu(), ids, w))
    assert m["passed"], m
    fixed = prepare_w4_moe(lay["x"], tiled, lay["down"], plan.ids.clone(), plan.routing_weights.clone(),
                           w4_decode=decode)
    assert len(fixed.launches) == 4
    assert torch.equal(fixed.run().view(torch.int16), out.view(torch.int16))


QWEN_PERF = [c for c in GOLDEN["cases"] if c["family"] == "performance_cases" and c["E"] == 128]


@pytest.mark.parametrize("case", QWEN_PERF, ids=lambda c: c["name"])
def test_reference_qwen_shape_cases(case, gpu_device):
    """The reference's recorded Qwen3-30B-A3B-shape performance cases
    (moe_benchmark.py:380-400; routing digests in the golden records) through
    the MFMA kernels: dispatch bit-exact with the canonical one and the recorded
    counts/offsets, the output within the reference's limits of the FP32
    oracle and within 2e-3/8e-3 of the rounding-staged oracle; then the same
    routes through the W4 path against the FP32 oracle on the dequantised
    weights."""
    x, gu, dn, ids, rw = O.make_inputs(tokens=case["T"], experts=128, topk=8, hidden=2048,
                                       intermediate=768, id_dtype=torch.int32,
                                       pattern=case["route_pattern"], seed=case["seed"])
    assert O.tensor_hash(ids) == case["routing_sha256"]
    dev = _to(gpu_device, x, gu, dn, ids, rw)
    plan = prepare_moe(*dev)
    assert plan.layout.fast_path == 1
    out = plan.run().clone()
    torch.cuda.synchronize()
    plan.check_inputs()
    _check_dispatch(plan, ids, 128)
    assert plan.counts.cpu().tolist() == case["expected_counts"]
    assert plan.offsets.cpu().tolist() == case["expected_offsets"]
    m32 = O.error(out, O.moe_reference(x, gu, dn, ids, rw), REF_LIMITS)
    assert m32["passed"], m32
    ms = O.error(out, O.staged_bf16_oracle(x, gu, dn, ids, rw), STAGED_LIMITS)
    assert ms["passed"], ms
    packed = quantize_gate_up(gu)
    w4 = prepare_w4_moe(dev[0], packed, dev[2], dev[3], dev[4])
    out4 = w4.run().clone()
    torch.cuda.synchronize()
    w4.check_inputs()
    m4 = O.error(out4, O.moe_reference(x, O.dequantize_w4(packed.words, packed.scales), dn, ids, rw))
    assert m4["passed"], m4


def test_launch_objects_and_workspace_view(gpu_device):
    """``launches`` are launch objects whose ``run()`` enqueues one stage (the
    reference's _PreparedLaunch, moe_prepared.py:17-30): running them in order
    equals ``run()``.  ``base`` exposes the workspace arrays by the reference's
    names (moe.py:124-156)."""
    lay = make_layer("qwen", 193, seed=21, device=gpu_device)
    plan = prepare_routed_moe(lay["x"], lay["logits"], lay["gate_up"], lay["down"], 8)
    ref = plan.run().clone()
    plan.output.zero_()
    for launch in plan.launches:
        launch.run()
    torch.cuda.synchronize()
    assert [l.name for l in plan.launches] == list(plan.launch_names)
    assert torch.equal(plan.output.view(torch.int16), ref.view(torch.int16))
    base = plan.base
    assert base.output.data_ptr() == plan.output.data_ptr()
    assert torch.equal(base.counts.cpu(), torch.bincount(plan.ids.cpu().flatten().long(),
                                                         minlength=128).int())
    assert base.mapping.numel() == 193 * 8 and base.down_output.shape == (193 * 8, 2048)
    assert base.workspace_bytes == plan.workspace_bytes
    base.check_inputs()


@pytest.mark.parametrize("tokens,k,experts,id_dtype", [(1000, 4, 256, torch.int64),
                                                       (3000, 1, 7, torch.int32),
                                                       (2100, 8, 128, torch.int32)])
def test_multi_workgroup_planner_fixed_routes(tokens, k, experts, id_dtype, gpu_device):
    """Fixed routes over several planner workgroups (1024 // K tokens each):
    canonical ranks across chunk boundaries, a hot expert spanning chunks,
    invalid IDs and a non-finite weight in later chunks (status bits 1 and 2,
    the bad routes left out of every array), then the same routes made valid
    through the GEMMs against the FP32 oracle."""
    g = torch.Generator().manual_seed(tokens + k)
    ids = torch.randint(0, experts, (tokens, k), generator=g)
    ids[tokens // 3: tokens // 3 + 300, 0] = 3                    # hot expert across a chunk edge
    w = torch.rand((tokens, k), generator=g)
    x = torch.randn((tokens, 128), generator=g).to(torch.bfloat16)
    gu = (torch.randn((experts, 256, 128), generator=g) * 0.05).to(torch.bfloat16)
    dn = (torch.randn((experts, 128, 128), generator=g) * 0.05).to(torch.bfloat16)
    bad = ids.clone()
    bad[tokens - 5, k - 1] = experts                                # invalid, last chunk
    bad[tokens // 2, 0] = -1                                        # invalid, middle chunk
    wbad = w.clone()
    wbad[tokens - 700, 0] = float("nan")
    dev = _to(gpu_device, x, gu, dn, bad.to(id_dtype), wbad)
    plan = prepare_moe(*dev)
    assert plan.launch_names[0] == "route_plan"
    torch.cuda.synchronize()
    assert plan.read_status() == 3
    _check_dispatch(plan, bad, experts)
    # valid routes: dispatch and layer output
    plan.ids.copy_(ids.to(id_dtype).to(gpu_device))
    plan.routing_weights.copy_(w.to(gpu_device))
    out = plan.run().clone()
    torch.cuda.synchronize()
    assert plan.read_status() == 0
    _check_dispatch(plan, ids, experts)
    m = O.error(out, O.moe_reference(x, gu, dn, ids, w))
    assert m["passed"], m


def test_multi_workgroup_router(gpu_device):
    """Router mode above 32 tokens with E = 256 (no single-workgroup fusion):
    38 planner workgroups route 16 tokens each; IDs bit-exact on tie-heavy
    logits, the dispatch canonical, a NaN logit in the last chunk sets bit 4."""
    tokens, experts, k = 600, 256, 6
    g = torch.Generator().manual_seed(5)
    x = torch.randn((tokens, 128), generator=g).to(torch.bfloat16)
    gu = (torch.randn((experts, 256, 128), generator=g) * 0.05).to(torch.bfloat16)
    dn = (torch.randn((experts, 128, 128), generator=g) * 0.05).to(torch.bfloat16)
    logits = torch.randint(-5, 5, (tokens, experts), generator=g).float() * 0.5
    plan = prepare_routed_moe(*_to(gpu_device, x, logits, gu, dn), k)
    assert plan.launch_names[0] == "route_plan"
    out = plan.forward().clone()
    torch.cuda.synchronize()
    ids, w = O.route_topk(logits, k)
    assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
    assert torch.allclose(plan.routing_weights.cpu(), w, rtol=2e-6, atol=1e-7)
    _check_dispatch(plan, ids, experts)
    assert plan.read_status() == 0
    m = O.error(out, O.moe_reference(x, gu, dn, ids, w))
    assert m["passed"], m
    plan.logits[tokens - 3, 17] = float("nan")
    plan.forward()
    assert plan.read_status() & 4


def test_forward_rejects_mismatched_inputs(gpu_device):
    """forward(hidden, router_logits) copies only tensors of the bound shape,
    dtype and device (the prepare-time rules, moe.py:220-235): no broadcast of
    a [1, H] row, no silent fp32 cast, no host tensors."""
    lay = make_layer("tiny", 17, seed=3, device=gpu_device)
    plan = prepare_routed_moe(lay["x"], lay["logits"], lay["gate_up"], lay["down"], lay["K"])
    ref = plan.forward(lay["x"].clone(), lay["logits"].clone()).clone()
    bad = [
        (lay["x"][:1].clone(), None),                        # [1, H] would broadcast
        (lay["x"].float(), None),                            # fp32 hidden
        (lay["x"].cpu(), None),                              # host tensor
        (None, lay["logits"][:, :4].clone()),                # wrong E
        (None, lay["logits"].double()),                      # fp64 logits
    ]
    for hidden, logits in bad:
        with pytest.raises(ValueError):
            plan.forward(hidden, logits)
    assert torch.equal(plan.forward(lay["x"].clone(), lay["logits"].clone()), ref)
