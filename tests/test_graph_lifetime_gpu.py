"""Graph lifetime of every kernel family (MI355X only).

docs/MOE_USAGE.md:126-175 (reference): a prepared forward is captured once at
fixed addresses; callers then update input values in place on a producer
stream, order the replay after that update with an event, replay on another
stream and order their reads of the output after the replay.  The reference
checks this for the fixed-route path (moe_benchmark.py:290-321, the
``graph_updates`` functional spec at :368).

Each case below captures a graph of eight forwards of one prepared layer on
the Qwen3-30B-A3B shape and drives it through that protocol three times with
new inputs.  After every replay:
  * the replayed output is bitwise equal to an eager forward on the same inputs,
  * the streaming GEMMs' work counters read zero (they hand out units from
    device counters that must survive back-to-back forwards inside a graph),
  * the status word is clean;
and the last replay is within rel-RMS 5e-3 / normalised max 1e-2 of the FP32
oracle on the routes the GPU chose (whose IDs equal the oracle's top-k).
"""
import pytest
import torch

from llm_gpu_kernels_amd import (GemmConfig, prepare_moe, prepare_routed_moe, quantize_gate_up,
                                 tile_gate_up)
from llm_gpu_kernels_amd.workloads import make_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

# (id, T, routing, W4, launches expected, kernel family exercised)
FAMILIES = [
    ("bf16-t17-planning-gate-up", 17, "uniform", False, 3),   # dma gate/up with routing prologue
    ("bf16-t193-planner-dma", 193, "uniform", False, 4),      # multi-workgroup planner + counter-scheduled dma
    ("bf16-t384-32row-dma", 384, "uniform", False, 4),        # 32-row tasks, 32-row down units in fours
    ("bf16-t1024-zipf-tiled", 1024, "zipf", False, 4),        # LDS-tiled GEMMs, 64-row tasks
    ("w4-t17-stream", 17, "uniform", True, 3),                # W4 register-streaming gate/up, routing prologue
    ("w4-t193-wave", 193, "uniform", True, 4),                # W4 one-unit-per-wave gate/up
    ("w4-t1024-wave", 1024, "uniform", True, 4),              # W4 wave gate/up, 64-row tasks
    ("w4fold-t17-stream", 17, "uniform", "fold", 3),          # folded decode, split-K streaming, routing prologue
    ("w4fold-t193-stream", 193, "uniform", "fold", 4),        # folded decode, 16-row tasks
]

_WEIGHTS = {}


def _weights(w4, device):
    """Qwen-shape weights, built once per module (bf16 and their W4 tiling; with
    w4 == "fold" the oracle gets the unrounded q * scale weights)."""
    key = "w4fold" if w4 == "fold" else "w4" if w4 else "bf16"
    if key not in _WEIGHTS:
        lay = make_layer("qwen", 1, seed=0, device=device)
        if w4:
            packed = quantize_gate_up(lay["gate_up"].cpu())
            tiled = tile_gate_up(packed).to(device)
            ref = (O.dequantize_w4_unrounded if w4 == "fold" else O.dequantize_w4)(packed.words, packed.scales)
            _WEIGHTS[key] = (tiled, ref, lay["down"])
        else:
            _WEIGHTS[key] = (lay["gate_up"], lay["gate_up"].cpu(), lay["down"])
    return _WEIGHTS[key]


def _bits(t):
    return t.view(torch.int16).clone()


def _drive(plan, inputs, nexts, device, check_oracle):
    """Capture 8 forwards, then three update -> replay rounds through events."""
    for _ in range(3):
        plan.run()
    torch.cuda.synchronize(device)
    capture = torch.cuda.Stream(device=device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=capture):
        for _ in range(8):
            gout = plan.run()
    main = torch.cuda.current_stream(device)
    producer = torch.cuda.Stream(device=device)
    replay = torch.cuda.Stream(device=device)
    for step, nxt in enumerate(nexts):
        ready, done = torch.cuda.Event(), torch.cuda.Event()
        producer.wait_stream(main)
        with torch.cuda.stream(producer):
            for dst, src in zip(inputs, nxt):
                dst.copy_(src)
            ready.record()
        replay.wait_event(ready)
        with torch.cuda.stream(replay):
            graph.replay()
            done.record()
        main.wait_event(done)
        replayed = _bits(gout)
        torch.cuda.synchronize(device)
        assert plan.work_counters.cpu().tolist() == [0, 0, 0, 0], step
        assert plan.read_status() == 0, step
        eager = _bits(plan.run())
        torch.cuda.synchronize(device)
        assert torch.equal(replayed, eager), f"replay {step} differs from eager"
        if step == len(nexts) - 1:
            check_oracle(gout)


@pytest.mark.parametrize("name,tokens,routing,w4,launches", FAMILIES, ids=[f[0] for f in FAMILIES])
def test_routed_graph_replays(name, tokens, routing, w4, launches, gpu_device):
    gate_up, ref_gu, down = _weights(w4, gpu_device)
    lay = make_layer("qwen", tokens, routing=routing, seed=tokens, device=gpu_device,
                     weights=False)
    plan = prepare_routed_moe(lay["x"], lay["logits"], gate_up, down, 8,
                              w4_decode="fold" if w4 == "fold" else "exact")
    assert len(plan.launches) == launches, plan.launch_names
    nexts = []
    for step in range(3):
        n = make_layer("qwen", tokens, routing=routing, seed=1000 + 10 * tokens + step,
                       device=gpu_device, weights=False)
        nexts.append((n["x"], n["logits"]))

    def check(out):
        logits = nexts[-1][1].cpu()
        ids, w = O.route_topk(logits, 8)
        assert torch.equal(plan.ids.cpu(), ids), "router IDs differ"
        m = O.error(out, O.moe_reference(nexts[-1][0].cpu(), ref_gu, down.cpu(), ids, w))
        assert m["passed"], m

    _drive(plan, (lay["x"], lay["logits"]), nexts, gpu_device, check)


@pytest.mark.parametrize("tokens,block_m", [(17, 16), (193, 0), (1024, 0)])
def test_fixed_route_graph_updates(tokens, block_m, gpu_device):
    """Fixed routes (the reference's own graph-update case): x, ids and the
    routing weights change in place between replays, int64 IDs included."""
    gate_up, ref_gu, down = _weights(False, gpu_device)
    lay = make_layer("qwen", tokens, seed=tokens + 1, device=gpu_device, weights=False)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    ids_d = ids.to(torch.int64).to(gpu_device)
    w_d = w.to(gpu_device)
    cfg = GemmConfig(block_m=block_m) if block_m else None
    plan = prepare_moe(lay["x"], gate_up, down, ids_d, w_d, config=cfg)
    nexts = []
    for step in range(3):
        n = make_layer("qwen", tokens, routing="zipf" if step == 1 else "uniform",
                       seed=2000 + tokens + step, device=gpu_device, weights=False)
        ni, nw = O.route_topk(n["logits"].cpu(), 8)
        nexts.append((n["x"], ni.to(torch.int64).to(gpu_device), nw.to(gpu_device)))

    def check(out):
        x, ni, nw = (t.cpu() for t in nexts[-1])
        m = O.error(out, O.moe_reference(x, ref_gu, down.cpu(), ni, nw))
        assert m["passed"], m

    _drive(plan, (lay["x"], ids_d, w_d), nexts, gpu_device, check)


def test_dirty_counters_are_reported_and_healed(gpu_device):
    """A workspace whose work counters are left nonzero (an aborted launch, a
    reused arena): read_status flags it (bit 8), reset_counters clears it, and
    the planner launch clears them itself before the GEMMs start."""
    gate_up, _, down = _weights(False, gpu_device)
    lay = make_layer("qwen", 193, seed=7, device=gpu_device, weights=False)
    plan = prepare_routed_moe(lay["x"], lay["logits"], gate_up, down, 8)
    clean = _bits(plan.run())
    torch.cuda.synchronize(gpu_device)
    plan.work_counters.copy_(torch.tensor([5, 3, 7, 1], dtype=torch.int32))
    assert plan.read_status() & 8
    with pytest.raises(RuntimeError):
        plan.check_inputs()
    plan.reset_counters()
    assert plan.read_status() == 0
    # Planner path: dirty counters before a forward do not change its result.
    plan.work_counters.copy_(torch.tensor([9, 2, 4, 4], dtype=torch.int32))
    assert torch.equal(_bits(plan.run()), clean)
    torch.cuda.synchronize(gpu_device)
    assert plan.read_status() == 0
    # Routing in the gate/up prologue (no planner launch): the forward after
    # a dirty one is correct again, and the reset entry makes the first one so.
    small = make_layer("qwen", 17, seed=8, device=gpu_device, weights=False)
    p17 = prepare_routed_moe(small["x"], small["logits"], gate_up, down, 8)
    ref = _bits(p17.run())
    torch.cuda.synchronize(gpu_device)
    p17.work_counters.copy_(torch.tensor([3, 1, 3, 1], dtype=torch.int32))
    p17.run()
    torch.cuda.synchronize(gpu_device)
    # The dirty forward's units counter started at 3: the gate/up launch ran
    # fewer units than it has and latches bit 8 instead of a clean status.
    assert p17.read_status() & 8
    with pytest.raises(RuntimeError, match="work counters"):
        p17.check_inputs()
    assert torch.equal(_bits(p17.run()), ref)
    torch.cuda.synchronize(gpu_device)
    assert p17.read_status() == 0
    p17.work_counters.copy_(torch.tensor([3, 1, 3, 1], dtype=torch.int32))
    p17.reset_counters()
    assert torch.equal(_bits(p17.run()), ref)


def _planner_words(plan):
    """The multi-workgroup planner's exchange area: [W][E+1] tagged words and
    its arrival counter (int32 view of the workspace)."""
    lay = plan.layout
    return plan.workspace[lay.partials:lay.act].view(torch.int32)


@pytest.mark.parametrize("garbage", [False, True], ids=["withheld", "withheld-garbage"])
def test_stalled_planner_runs_no_tasks(garbage, gpu_device, monkeypatch):
    """A planner workgroup whose counts never arrive (forced from the host:
    the test hook makes the last workgroup withhold its words and every wait
    give up after a few rounds, so every kernel exits normally) leaves an
    incomplete view: the forward reports MOE_STATUS_STALLED, runs no GEMM
    task, advances the epoch and leaves the arrival counter at zero.  With
    garbage carrying the current epoch's tag in the withheld slot, every
    workgroup rejects the impossible counts the same way.  A plan created
    without the hook on the same shape is correct."""
    gate_up, ref_gu, down = _weights(False, gpu_device)
    lay = make_layer("qwen", 193, seed=11, device=gpu_device, weights=False)
    ids, w = O.route_topk(lay["logits"].cpu(), 8)
    ids_d, w_d = ids.to(gpu_device), w.to(gpu_device)
    monkeypatch.setenv("MOE_TEST_PLANNER_HOLD", "1")
    plan = prepare_moe(lay["x"], gate_up, down, ids_d, w_d)  # runs one forward
    monkeypatch.delenv("MOE_TEST_PLANNER_HOLD")
    torch.cuda.synchronize(gpu_device)
    assert plan.read_status() & 16
    with pytest.raises(RuntimeError, match="planner"):
        plan.check_inputs()
    words = _planner_words(plan)
    e = 128
    tpw = 1024 // 8  # fixed routes: 1024 / K tokens per planner workgroup
    W = (193 + tpw - 1) // tpw
    if garbage:
        st = plan.workspace[plan.layout.status:plan.layout.status + 16].view(torch.int32).cpu()
        tag = (int(st[2]) & 0x7FFF) | 0x8000
        junk = torch.full(((e + 1),), (tag << 16) | 0xFFFF, dtype=torch.int64)
        junk = torch.where(junk >= 2**31, junk - 2**32, junk).to(torch.int32)
        words[(W - 1) * (e + 1):W * (e + 1)].copy_(junk.to(gpu_device))
    st0 = int(plan.workspace[plan.layout.status:plan.layout.status + 16].view(torch.int32)[2])
    plan.run()
    torch.cuda.synchronize(gpu_device)
    st = plan.workspace[plan.layout.status:plan.layout.status + 16].view(torch.int32).cpu()
    assert int(st[0]) & 16
    assert int(st[2]) == st0 + 1, "the epoch advances on a stalled launch too"
    assert int(plan.num_tasks.item()) == 0
    assert int(words[W * (e + 1)].item()) == 0, "arrival counter back at zero"
    assert int(plan.work_counters.abs().sum().item()) == 0
    # Without the hook: a new plan on this shape is correct and clean.
    good = prepare_moe(lay["x"], gate_up, down, ids_d, w_d)
    out = good.run()
    torch.cuda.synchronize(gpu_device)
    assert good.read_status() == 0
    m = O.error(out, O.moe_reference(lay["x"].cpu(), ref_gu, down.cpu(), ids, w))
    assert m["passed"], m
