"""Segmented-KV GQA attention vs the FP32 SDPA-math oracle (MI355X only).

Cases follow tests/e2e/test_compact_attention.py of the reference (history
(2049, 0, 575): empty middle segment and a ragged tail; current-segment V
token stride 6144; graph replay after in-place updates; non-default stream)
and BASELINE config 5 (history 1024/512/256, T in {32, 96, 256}).
"""
import pytest
import torch

from llm_gpu_kernels_amd import prepare_segmented_gqa, prepare_cuda_gqa_compact
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
LIMITS = {"relative_rms": 5e-3, "normalized_max": 1e-2}


def _values(seed, tokens, history, device, v_stride=None, hq=32, hkv=8):
    g = torch.Generator().manual_seed(seed)

    def rnd(shape):
        return torch.randn(shape, generator=g).to(torch.bfloat16).to(device)

    q = rnd((tokens, hq, 128))
    segs = [(rnd((L, hkv, 128)), rnd((L, hkv, 128))) for L in (*history, tokens)]
    if v_stride:
        k, v = segs[-1]
        pv = torch.empty_strided(tuple(v.shape), (v_stride, 128, 1), dtype=v.dtype, device=device)
        pv.copy_(v)
        segs[-1] = (k, pv)
    return q, segs


def _check(out, q, segs):
    ref = O.gqa_segmented_reference(q.cpu(), [(k.cpu(), v.cpu()) for k, v in segs])
    m = O.error(out.cpu(), ref, LIMITS)
    assert m["passed"], m


@pytest.mark.parametrize("tokens", [32, 96, 256])
def test_baseline_config5(tokens, gpu_device):
    q, segs = _values(tokens, tokens, (1024, 512, 256), gpu_device)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    _check(plan.output, q, segs)


@pytest.mark.parametrize("tokens,hq,hkv", [(40, 32, 8), (100, 32, 8), (200, 32, 8), (512, 32, 8),
                                           (600, 8, 8)])
def test_launch_shapes(tokens, hq, hkv, gpu_device):
    """Every launch shape on 256 CUs (gqa_shape).  One 16-row block per wave:
    T = 40 four-wave workgroups with the keys split in two (merge launch),
    T = 100 eight-wave workgroups without a split.  Two row blocks per wave:
    T = 200 eight-wave workgroups without a split, T = 512 four-wave
    workgroups, two per CU; T = 600 with one query head per KV head (two
    token blocks per workgroup)."""
    q, segs = _values(tokens + 1, tokens, (300, 0, 129), gpu_device, hq=hq, hkv=hkv)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    _check(plan.output, q, segs)


@pytest.mark.parametrize("tokens,history", [(96, (2049, 0, 575)), (17, (0, 0, 0)), (1, (5, 0, 3)),
                                            (33, (64, 63, 1))])
def test_reference_shapes_and_tails(tokens, history, gpu_device):
    q, segs = _values(7, tokens, history, gpu_device, v_stride=6144 if tokens == 96 else None)
    plan = prepare_cuda_gqa_compact(q, segs, stages=2)
    torch.cuda.synchronize()
    _check(plan.output, q, segs)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (64, 8)])
def test_group_sizes(hq, hkv, gpu_device):
    q, segs = _values(3, 40, (100, 30, 7), gpu_device, hq=hq, hkv=hkv)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    _check(plan.output, q, segs)


def test_split_merge_partial_workgroup(gpu_device):
    """T * Hq = 66 (query) rows with the keys split: the merge launch's last
    workgroup holds fewer rows than the others."""
    q, segs = _values(5, 33, (200, 17, 0), gpu_device, hq=2, hkv=1)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    assert plan.splits_workspace_bytes > 0
    _check(plan.output, q, segs)


def test_empty_query(gpu_device):
    q, segs = _values(1, 0, (10, 0, 4), gpu_device)
    plan = prepare_segmented_gqa(q, segs)
    assert plan.run().shape == (0, 32, 128)


@pytest.mark.parametrize("tokens", [96, 32])
def test_graph_replay_and_stream(tokens, gpu_device):
    """T = 96 runs unsplit, T = 32 with a key split and the merge launch."""
    q, segs = _values(11, tokens, (1024, 512, 256), gpu_device)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=gpu_device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        gout = plan.run()
    for step in range(2):
        q2, segs2 = _values(100 + step, tokens, (1024, 512, 256), gpu_device)
        q.copy_(q2)
        for (k, v), (k2, v2) in zip(segs, segs2):
            k.copy_(k2)
            v.copy_(v2)
        graph.replay()
        torch.cuda.synchronize()
        replay = gout.clone()
        side = torch.cuda.Stream(device=gpu_device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager = plan.run().clone()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(replay.view(torch.int16), eager.view(torch.int16))
        _check(replay, q, segs)


@pytest.mark.parametrize("tokens", [32, 64])
def test_split_runs_repeat_bitwise(tokens, gpu_device):
    """Key-split shapes (T = 32: four splits, T = 64: two on 256 CUs):
    repeated runs of one plan merge the partial states in the same fixed order,
    so they give bitwise the same output."""
    q, segs = _values(21 + tokens, tokens, (1024, 512, 256), gpu_device)
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    assert plan.splits_workspace_bytes > 0
    first = plan.output.clone()
    _check(first, q, segs)
    for _ in range(4):
        plan.run()
    torch.cuda.synchronize()
    assert torch.equal(plan.output.view(torch.int16), first.view(torch.int16))


def test_rejects_bad_inputs(gpu_device):
    q, segs = _values(1, 8, (4, 0, 2), gpu_device)
    with pytest.raises(ValueError):
        prepare_segmented_gqa(q, segs[:-1] + [(segs[-1][0][:4], segs[-1][1][:4])])
    with pytest.raises(TypeError):
        prepare_segmented_gqa(q, [(k.float(), v) for k, v in segs])
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            prepare_segmented_gqa(q, segs, scale=bad)


def test_out_aliasing_rejected(gpu_device):
    """An output sharing storage with q or a K/V segment is rejected
    (attention_cuda_compact.py:175-177)."""
    from llm_gpu_kernels_amd import prepare_cuda_gqa_compact
    q = torch.randn(32, 32, 128, device=gpu_device).to(torch.bfloat16)
    kv = torch.randn(2, 64, 8, 128, device=gpu_device).to(torch.bfloat16)
    cur = torch.randn(2, 32, 8, 128, device=gpu_device).to(torch.bfloat16)
    segs = [(kv[0], kv[1]), (cur[0], cur[1])]
    with pytest.raises(ValueError, match="share storage"):
        prepare_cuda_gqa_compact(q, segs, out=q)
    big = torch.empty(2, 32, 32, 128, device=gpu_device, dtype=torch.bfloat16)
    segs_alias = [(kv[0], kv[1]), (big[1, :, :8], cur[1])]
    with pytest.raises(ValueError):
        prepare_cuda_gqa_compact(q, segs_alias, out=big[0])
    prepare_cuda_gqa_compact(q, segs)
