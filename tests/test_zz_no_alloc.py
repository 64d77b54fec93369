"""moe_forward_static: the forward that allocates nothing (MI355X only).

It runs the same kernels as a prepared plan, with the workspace in a static
device array instead of a caller allocation, so its outputs must be bitwise
equal to the plan's.  Two calls in a row, the second with fewer tokens (the
array keeps the first call's contents), then a W4 fixed-route call, each
against ``moe_plan_create``/``moe_plan_run`` on the same inputs; a shape whose
workspace exceeds the static array is rejected.
"""
import ctypes

import pytest
import torch

from llm_gpu_kernels_amd import _native as N
from llm_gpu_kernels_amd import prepare_routed_moe, prepare_w4_moe, quantize_gate_up, tile_gate_up
from llm_gpu_kernels_amd.workloads import make_layer

pytestmark = pytest.mark.gpu


def _desc(x, down, ids, w, out, *, gate_up=None, tiled=None, logits=None):
    d = N.MoeDesc()
    d.T, d.H = x.shape
    d.E, _, d.I = down.shape
    d.K = ids.shape[1]
    d.weight_format = N.WEIGHTS_W4G128 if tiled is not None else N.WEIGHTS_BF16
    d.id_dtype = N.IDS_INT64 if ids.dtype == torch.int64 else N.IDS_INT32
    d.route_mode = N.ROUTE_LOGITS if logits is not None else N.ROUTE_FIXED
    d.renormalize = 1
    d.x, d.ids, d.weights, d.down, d.out = (x.data_ptr(), ids.data_ptr(), w.data_ptr(),
                                            down.data_ptr(), out.data_ptr())
    d.logits = logits.data_ptr() if logits is not None else None
    d.gate_up = gate_up.data_ptr() if gate_up is not None else None
    d.w4_words = tiled.words.data_ptr() if tiled is not None else None
    d.w4_scales = tiled.scales.data_ptr() if tiled is not None else None
    d.workspace, d.workspace_bytes = None, 0
    return d


def _static(d):
    stream = torch.cuda.current_stream().cuda_stream
    return N.lib().moe_forward_static(ctypes.byref(d), ctypes.c_void_p(stream))


def _bits(t):
    return t.view(torch.int16).cpu()


def test_static_forward_matches_plan(gpu_device):
    lay = make_layer("qwen", 1, seed=0, device=gpu_device)
    gate_up, down = lay["gate_up"], lay["down"]
    for tokens in (193, 17):  # the second call is smaller than the first
        inp = make_layer("qwen", tokens, seed=300 + tokens, device=gpu_device, weights=False)
        plan = prepare_routed_moe(inp["x"], inp["logits"], gate_up, down, 8)
        ref = plan.run().clone()
        ids = torch.full((tokens, 8), -7, dtype=torch.int32, device=gpu_device)
        w = torch.zeros((tokens, 8), dtype=torch.float32, device=gpu_device)
        out = torch.zeros((tokens, 2048), dtype=torch.bfloat16, device=gpu_device)
        d = _desc(inp["x"], down, ids, w, out, gate_up=gate_up, logits=inp["logits"])
        assert _static(d) == 0, N.last_error()
        torch.cuda.synchronize()
        assert torch.equal(ids.cpu(), plan.ids.cpu())
        assert torch.equal(w.cpu(), plan.routing_weights.cpu())
        assert torch.equal(_bits(out), _bits(ref)), tokens
    # W4 gate/up, fixed int64 routes, 33 tokens.
    tiled = tile_gate_up(quantize_gate_up(gate_up.cpu())).to(gpu_device)
    inp = make_layer("qwen", 33, seed=333, device=gpu_device, weights=False)
    ids = torch.topk(inp["logits"], 8, dim=1).indices.contiguous()
    w = torch.softmax(inp["logits"], 1).gather(1, ids).contiguous()
    p4 = prepare_w4_moe(inp["x"], tiled, down, ids, w)
    expect = p4.run().clone()
    out = torch.zeros((33, 2048), dtype=torch.bfloat16, device=gpu_device)
    assert _static(_desc(inp["x"], down, ids, w, out, tiled=tiled)) == 0, N.last_error()
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(expect))


def _fits(tokens, route):
    d = N.MoeDesc()
    d.T, d.H, d.I, d.E, d.K, d.route_mode = tokens, 2048, 768, 128, 8, route
    lay = N.MoeLayout()
    assert N.lib().moe_workspace_layout(ctypes.byref(d), ctypes.byref(lay)) == 0
    return lay.total <= N.STATIC_WORKSPACE_BYTES


def test_static_forward_rejects_large_shapes(gpu_device):
    """The largest router-mode Qwen-shape forward that fits the static array
    runs; one token more is rejected with MOE_ESPACE and a message."""
    limit = max(t for t in range(1, 1024) if _fits(t, N.ROUTE_LOGITS))
    assert 256 <= limit < 1023
    lay = make_layer("qwen", 1, seed=0, device=gpu_device)
    inp = make_layer("qwen", limit + 1, seed=1, device=gpu_device, weights=False)
    ids = torch.zeros((limit + 1, 8), dtype=torch.int32, device=gpu_device)
    w = torch.zeros((limit + 1, 8), dtype=torch.float32, device=gpu_device)
    out = torch.zeros((limit + 1, 2048), dtype=torch.bfloat16, device=gpu_device)
    d = _desc(inp["x"], lay["down"], ids, w, out, gate_up=lay["gate_up"], logits=inp["logits"])
    assert _static(d) == N.MOE_ESPACE
    assert "static workspace" in N.last_error()
    d.T = limit
    assert _static(d) == 0, N.last_error()
    torch.cuda.synchronize()
