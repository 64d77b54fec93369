"""Prepared MoE forward on MI355X: the reference's operator API over the HIP library.

Mirrors the prepared-buffer interface of the reference
(``prepare_moe`` / ``PreparedMoE``: src/llm_gpu_kernels/moe.py:124-245;
``prepare_ranked_moe_launcher``: moe_ranked.py:99; ``prepare_configured_moe``:
moe_configured.py:17; ``prepare_cuda_moe``: moe_cuda.py:54; ``prepare_w4_moe``:
moe_w4_cuda.py:85; ``prepare_w4_layout_moe``: moe_w4_layout_cuda.py:152;
lifetime rules: docs/MOE_USAGE.md:93-146) and adds the router-inclusive
``prepare_routed_moe(...).forward(hidden, router_logits)``.

Every forward is three to five launches of hand-written gfx950 kernels on the
current stream: [router] -> planner -> gate/up+SwiGLU -> down -> combine, where
for few tokens the router runs inside the planner and, for bf16 weights, both
inside the gate/up launch (the header's launch count tells which).  No
host synchronisation, no allocation and no host readback happen in ``run()``;
the prepared object owns its output and workspace, binds the caller's tensors
by address, and may be captured in a HIP graph.  Values of the bound inputs
may change in place between runs (``copy_``); shapes and addresses may not.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass, field

import torch

from . import _native as N
from .weight_quant import PackedGateUp, RepackedGateUp, TiledGateUp, tile_gate_up

__all__ = [
    "GemmConfig", "FrozenMoEPolicy", "MoEWorkspace", "PreparedLaunch", "PreparedMoE", "PreparedRoutedMoE", "prepare_moe",
    "prepare_ranked_moe_launcher", "prepare_configured_moe", "prepare_cuda_moe",
    "prepare_w4_moe", "prepare_w4_layout_moe", "prepare_routed_moe",
]

_CREATE_LOCK = threading.Lock()


@dataclass(frozen=True)
class GemmConfig:
    """Tile choice (reference gemm.py:13-25).  Only ``block_m`` (grouped rows
    per task) is meaningful on gfx950: 16 or 32 select the weight-streaming
    kernels, 64 the LDS-tiled kernels; 0 lets the shape policy choose.  The
    column tiles and the K-pipeline depth are fixed by the kernels' wave
    layout."""
    block_m: int = 0
    block_n: int = 0
    block_k: int = 0
    warps: int = 8
    stages: int = 2


@dataclass(frozen=True)
class FrozenMoEPolicy:
    """Shape-only tile policy (role of moe_full_policy.py:49-194).

    Chooses ``block_m`` from mu = T*K/E alone -- never from route contents, so
    a captured graph stays valid when IDs change in place (docs/MOE_USAGE.md:78-83).
    """
    small_mu: float = 16.0

    def select(self, tokens, experts, topk, hidden, intermediate):
        mu = tokens * topk / max(experts, 1)
        if mu <= self.small_mu:
            return GemmConfig(block_m=16), "small"
        if mu < 2 * self.small_mu:
            return GemmConfig(block_m=32), "medium"
        return GemmConfig(block_m=64), "large"


@dataclass(frozen=True)
class PreparedLaunch:
    """One kernel launch of a prepared forward (role of ``_PreparedLaunch``,
    moe_prepared.py:17-30): ``run()`` enqueues that launch alone on the
    current stream; it reads what the launches before it wrote."""
    name: str
    stage: int
    plan: "PreparedMoE" = field(repr=False, compare=False)

    def run(self):
        self.plan.run_stage(self.stage)


@dataclass(frozen=True)
class MoEWorkspace:
    """The prepared workspace (role of the reference's ``base``: ``PreparedMoE``
    / ``W4Workspace``, moe.py:124-156, moe_w4_cuda.py:53-82): views of the
    bound inputs, the owned output and the device arrays of the last forward.
    ``down_output`` holds the down projections in route order (the reference's
    name for them); there is no ``grouped_input``, because the GEMMs gather
    the token rows of ``x`` directly."""
    x: torch.Tensor
    gate_up: object
    down: torch.Tensor
    ids: torch.Tensor
    routing_weights: torch.Tensor
    output: torch.Tensor
    counts: torch.Tensor
    offsets: torch.Tensor
    ranks: torch.Tensor
    mapping: torch.Tensor
    row_route: torch.Tensor
    tasks: torch.Tensor
    num_tasks: torch.Tensor
    activated: torch.Tensor
    down_output: torch.Tensor
    status: torch.Tensor
    work_counters: torch.Tensor
    config: GemmConfig
    workspace_bytes: int
    check_inputs: object = field(repr=False, compare=False)


def _device_check(tensors, device):
    for name, t in tensors.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.device != device:
            raise ValueError("all MoE tensors must be contiguous and on the same CUDA device")
        if not t.is_contiguous():
            raise ValueError("all MoE tensors must be contiguous and on the same CUDA device")


def _validate_common(x, down, ids, rw, gate_up_shape):
    if x.ndim != 2 or down.ndim != 3:
        raise ValueError("invalid ranks")
    e, h, inter = down.shape
    if not 0 < e <= 256 or h <= 0 or inter <= 0 or x.shape[1] != h:
        raise ValueError("invalid MoE shape; E in [1,256], H/I positive")
    if gate_up_shape is not None and tuple(gate_up_shape) != (e, 2 * inter, h):
        raise ValueError("gate_up must be [E, 2I, H]")
    if x.dtype != torch.bfloat16 or down.dtype != torch.bfloat16:
        raise ValueError("x and down must be bfloat16")
    if (ids.ndim != 2 or ids.dtype not in (torch.int32, torch.int64) or ids.shape[0] != x.shape[0]
            or not 0 < ids.shape[1] <= 32 or rw.shape != ids.shape or rw.dtype != torch.float32):
        raise ValueError("expected IDs[T, topk<=32] (int32/int64) and FP32 weights of identical shape")
    r = ids.numel()
    if r >= 2 ** 31 or r * max(h, 2 * inter) >= 2 ** 31:
        raise ValueError("routed/intermediate elements must be < 2**31")
    if x.device.type != "cuda":
        raise ValueError("MoE tensors must be on a GPU device")
    return e, h, inter


def _w4_decode_mode(mode, tiled):
    if mode not in ("exact", "fold"):
        raise ValueError(f"w4_decode must be 'exact' or 'fold' (got {mode!r})")
    if mode == "fold" and tiled is None:
        raise ValueError("w4_decode='fold' needs W4G128 gate/up weights")
    return mode


class PreparedMoE:
    """Fixed buffers and shapes; IDs and values may change in place.

    Attributes mirror the reference workspace (moe.py:124-156): ``output``,
    ``counts``, ``offsets``, ``ranks``, ``mapping``, ``row_route``, ``tasks``,
    ``status``; ``launches`` names the kernels of one forward.
    """

    def __init__(self, *, x, down, ids, routing_weights, gate_up=None, tiled=None, logits=None,
                 renormalize=True, config=None, w4_decode="exact"):
        device = x.device
        e, h, inter = down.shape
        t, k = ids.shape
        self.x, self.down, self.ids, self.routing_weights = x, down, ids, routing_weights
        self.gate_up, self.tiled, self.logits = gate_up, tiled, logits
        self.config = config or GemmConfig()
        self.output = torch.empty((t, h), dtype=torch.bfloat16, device=device)
        d = N.MoeDesc()
        d.T, d.H, d.I, d.E, d.K = t, h, inter, e, k
        self.w4_decode = _w4_decode_mode(w4_decode, tiled)
        d.weight_format = (N.WEIGHTS_BF16 if tiled is None else
                           N.WEIGHTS_W4G128_FOLD if self.w4_decode == "fold" else N.WEIGHTS_W4G128)
        d.id_dtype = N.IDS_INT64 if ids.dtype == torch.int64 else N.IDS_INT32
        d.route_mode = N.ROUTE_LOGITS if logits is not None else N.ROUTE_FIXED
        d.renormalize = 1 if renormalize else 0
        d.token_block = self.config.block_m if self.config.block_m in (16, 32, 64) else 0
        lay = N.MoeLayout()
        N.check(N.lib().moe_workspace_layout(ctypes.byref(d), ctypes.byref(lay)), "prepare")
        # Zero-initialised: the router flag word is self-clearing from then on.
        self.workspace = torch.zeros(max(int(lay.total), 256), dtype=torch.uint8, device=device)
        d.x = x.data_ptr()
        d.logits = logits.data_ptr() if logits is not None else None
        d.ids = ids.data_ptr()
        d.weights = routing_weights.data_ptr()
        d.gate_up = gate_up.data_ptr() if gate_up is not None else None
        d.w4_words = tiled.words.data_ptr() if tiled is not None else None
        d.w4_scales = tiled.scales.data_ptr() if tiled is not None else None
        d.down = down.data_ptr()
        d.out = self.output.data_ptr()
        d.workspace = self.workspace.data_ptr()
        d.workspace_bytes = self.workspace.numel()
        self._desc = d
        handle = ctypes.c_void_p()
        with _CREATE_LOCK, torch.cuda.device(device):
            N.check(N.lib().moe_plan_create(ctypes.byref(handle), ctypes.byref(d)), "prepare")
        self._plan = handle
        N.check(N.lib().moe_plan_layout(handle, ctypes.byref(lay)), "layout")
        self.layout = lay
        r = t * k
        ws = self.workspace

        def view(offset, count, dtype=torch.int32):
            nbytes = count * torch.empty((), dtype=dtype).element_size()
            return ws[offset:offset + nbytes].view(dtype)

        self.status = view(lay.status, 1)
        self.counts = view(lay.counts, e)
        self.offsets = view(lay.offsets, e)
        self.ranks = view(lay.ranks, r)
        self.mapping = view(lay.map, r)
        self.row_route = view(lay.row_route, r)
        self.tasks = view(lay.tasks, 4 * lay.task_capacity).view(-1, 4)
        self.num_tasks = view(lay.num_tasks, 1)
        # {units taken, workgroups finished} of the gate/up and down launches
        # that hand out work from a device counter; zero between launches.
        self.work_counters = view(lay.counters, 4)
        self.activated = view(lay.act, r * inter, torch.bfloat16).view(r, inter)
        self.routed_output = view(lay.routed, r * h, torch.bfloat16).view(r, h)
        if lay.launches == 3:  # gate/up routes and plans in its prologue
            names = ["gate_up_swiglu", "down", "combine"]
        else:
            names = (["router"] if (logits is not None and lay.launches == 5) else []) + \
                ["route_plan", "gate_up_swiglu", "down", "combine"]
        self.launch_names = tuple(names) if t else ()
        self.launches = tuple(PreparedLaunch(n, i, self) for i, n in enumerate(self.launch_names))
        self.fast_path = bool(lay.fast_path)
        self.base = MoEWorkspace(
            x=x, gate_up=gate_up if gate_up is not None else tiled, down=down, ids=ids,
            routing_weights=routing_weights, output=self.output, counts=self.counts,
            offsets=self.offsets, ranks=self.ranks, mapping=self.mapping,
            row_route=self.row_route, tasks=self.tasks, num_tasks=self.num_tasks,
            activated=self.activated, down_output=self.routed_output, status=self.status,
            work_counters=self.work_counters, config=self.config,
            workspace_bytes=int(lay.total), check_inputs=self.check_inputs)

    @property
    def workspace_bytes(self) -> int:
        return int(self.layout.total)

    def run(self):
        """Enqueue one forward on the current stream; returns the owned output."""
        if self.x.shape[0] == 0:
            return self.output
        stream = torch.cuda.current_stream(self.x.device).cuda_stream
        N.check(N.lib().moe_plan_run(self._plan, ctypes.c_void_p(stream)), "run")
        return self.output

    def run_stage(self, index: int):
        """Enqueue launch ``index`` of ``launches`` alone (per-kernel timing)."""
        stream = torch.cuda.current_stream(self.x.device).cuda_stream
        N.check(N.lib().moe_plan_run_stage(self._plan, int(index), ctypes.c_void_p(stream)),
                "run_stage")

    def read_status(self) -> int:
        flags = ctypes.c_uint32(0)
        stream = torch.cuda.current_stream(self.x.device).cuda_stream
        N.check(N.lib().moe_plan_read_status(self._plan, ctypes.c_void_p(stream),
                                             ctypes.byref(flags)), "status")
        return int(flags.value)

    def reset_counters(self):
        """Enqueue a kernel that zeroes the streaming GEMMs' work counters."""
        stream = torch.cuda.current_stream(self.x.device).cuda_stream
        N.check(N.lib().moe_plan_reset_counters(self._plan, ctypes.c_void_p(stream)),
                "reset_counters")

    def check_inputs(self):
        """Synchronising debug check of the last forward (moe.py:157-160)."""
        flags = self.read_status()
        if flags & N.STATUS_STALLED:
            raise RuntimeError(f"MoE planner did not complete (GPU status={flags}): its "
                               "workgroups were not resident together or its exchange area "
                               "was not zeroed; the forward ran no expert tasks")
        if flags & N.STATUS_DIRTY_COUNTERS:
            raise RuntimeError(f"MoE workspace work counters were not zero (GPU status={flags}): "
                               "a launch did not complete or the workspace was not zeroed; "
                               "the last output is invalid (call reset_counters())")
        if flags:
            raise ValueError(f"invalid runtime MoE inputs: GPU status={flags} "
                             "(1=IDs, 2=nonfinite weights, 4=nonfinite logits)")

    def __del__(self):
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            try:
                N.lib().moe_plan_destroy(plan)
            except Exception:
                pass
            self._plan = None


def prepare_moe(x, gate_up, down, ids, routing_weights, *, config=None):
    """Fixed-route BF16 MoE (moe.py:220-245).  Runs one preparation forward."""
    _validate_common(x, down, ids, routing_weights, tuple(gate_up.shape))
    if gate_up.dtype != torch.bfloat16:
        raise ValueError("gate_up must be bfloat16")
    _device_check({"gate_up": gate_up, "down": down, "ids": ids,
                   "routing_weights": routing_weights, "x": x}, x.device)
    plan = PreparedMoE(x=x, gate_up=gate_up, down=down, ids=ids, routing_weights=routing_weights,
                       config=config)
    plan.run()
    return plan


def prepare_ranked_moe_launcher(x, gate_up, down, ids, routing_weights):
    """Ranked dispatch entry (moe_ranked.py:99); ranks here are canonical."""
    return prepare_moe(x, gate_up, down, ids, routing_weights)


def prepare_configured_moe(x, gate_up, down, ids, routing_weights, config):
    """Explicit tile config (moe_configured.py:17)."""
    if not isinstance(config, GemmConfig):
        raise TypeError("config must be a GemmConfig")
    return prepare_moe(x, gate_up, down, ids, routing_weights, config=config)


# The reference's native gate/up variants (moe_cuda.py:17).  They differ only
# in SM86 copy pipelining; on gfx950 every name selects the same MFMA kernels.
CUDA_VARIANTS = ("sync", "async", "async_skip")


def prepare_cuda_moe(x, gate_up, down, ids, routing_weights, *, variant="sync", down_config=None):
    """Native BF16 gate/up entry (moe_cuda.py:54-73): the reference's variant
    names are accepted and anything else is rejected as there."""
    if variant not in CUDA_VARIANTS:
        raise ValueError("unsupported CUDA variant")
    return prepare_moe(x, gate_up, down, ids, routing_weights, config=down_config)


def _as_tiled(packed, device):
    if isinstance(packed, TiledGateUp):
        return packed.to(device)
    if isinstance(packed, (PackedGateUp, RepackedGateUp)):
        return tile_gate_up(packed).to(device)
    raise TypeError("PackedGateUp, RepackedGateUp or TiledGateUp required")


def prepare_w4_moe(x, packed, down, ids, routing_weights, *, down_config=None, w4_decode="exact"):
    """W4A16 MoE: int4 gate/up (W4G128), bf16 down (moe_w4_cuda.py:85).

    ``w4_decode="exact"`` (default) multiplies the reference's dequantised
    weights bf16_rn(q * scale); ``"fold"`` lets the about-one-row-per-expert
    gate/up kernel apply each group's scale to the fp32 sum of its MFMAs
    (effective weights q * scale exactly; no counterpart in the reference)."""
    e, h, inter = _validate_common(x, down, ids, routing_weights, None)
    tiled = _as_tiled(packed, x.device)
    if tuple(tiled.shape) != (e, 2 * inter, h):
        raise ValueError("packed gate_up must describe [E, 2I, H]")
    _device_check({"down": down, "ids": ids, "routing_weights": routing_weights, "x": x,
                   "words": tiled.words, "scales": tiled.scales}, x.device)
    plan = PreparedMoE(x=x, tiled=tiled, down=down, ids=ids, routing_weights=routing_weights,
                       config=down_config, w4_decode=w4_decode)
    plan.run()
    return plan


def prepare_w4_layout_moe(x, packed, down, ids, routing_weights, *, down_config=None):
    """Physical-layout W4 entry (moe_w4_layout_cuda.py:152): takes the reference's
    M24 ``RepackedGateUp`` (or v1 / tiled); the tiled layout is the only W4
    layout the gfx950 kernels read, and M24 words reach it bit-exactly."""
    return prepare_w4_moe(x, packed, down, ids, routing_weights, down_config=down_config)


class PreparedRoutedMoE(PreparedMoE):
    """Router-inclusive MoE: ``forward(hidden, router_logits) -> out``.

    softmax(fp32) -> top-k -> renormalise run on the GPU
    (scripts/capture_qwen3_moe_layer0.py:583-586); ``ids`` (int32) and
    ``routing_weights`` (fp32) are outputs of each forward.
    """

    def forward(self, hidden=None, router_logits=None):
        # Same rules as prepare_routed_moe: a bound buffer is only ever
        # overwritten by a tensor of its own shape, dtype and device (no
        # broadcast of a [1, H] row, no silent fp32 -> bf16 cast).
        for name, new, bound in (("hidden", hidden, self.x), ("router_logits", router_logits, self.logits)):
            if new is None:
                continue
            if not isinstance(new, torch.Tensor):
                raise ValueError(f"{name} must be a tensor")
            if tuple(new.shape) != tuple(bound.shape) or new.dtype != bound.dtype:
                raise ValueError(f"{name} must be {bound.dtype} {list(bound.shape)}, got "
                                 f"{new.dtype} {list(new.shape)}")
            if new.device != bound.device:
                raise ValueError(f"{name} must be on {bound.device}, got {new.device}")
        if hidden is not None and hidden.data_ptr() != self.x.data_ptr():
            self.x.copy_(hidden)
        if router_logits is not None and router_logits.data_ptr() != self.logits.data_ptr():
            self.logits.copy_(router_logits)
        return self.run()

    __call__ = forward


def prepare_routed_moe(hidden, router_logits, gate_up, down, top_k, *, renormalize=True,
                       config=None, w4_decode="exact"):
    """Prepare the full MoE forward.  ``gate_up`` is a bf16 [E,2I,H] tensor or
    a PackedGateUp / TiledGateUp (W4A16).  ``hidden`` and ``router_logits`` are
    bound by address; ``forward`` copies other tensors into them."""
    e, h, inter = down.shape
    t = hidden.shape[0]
    if router_logits.shape != (t, e) or router_logits.dtype != torch.float32:
        raise ValueError("router_logits must be fp32 [T, E]")
    if not 1 <= top_k <= min(e, 32):
        raise ValueError("top_k must be in [1, min(E, 32)]")
    device = hidden.device
    ids = torch.zeros((t, top_k), dtype=torch.int32, device=device)
    rw = torch.zeros((t, top_k), dtype=torch.float32, device=device)
    tiled = None
    if isinstance(gate_up, torch.Tensor):
        _validate_common(hidden, down, ids, rw, tuple(gate_up.shape))
        _device_check({"gate_up": gate_up, "down": down, "hidden": hidden,
                       "router_logits": router_logits}, device)
    else:
        _validate_common(hidden, down, ids, rw, None)
        tiled = _as_tiled(gate_up, device)
        gate_up = None
        _device_check({"down": down, "hidden": hidden, "router_logits": router_logits}, device)
    if config is None:
        config, _ = FrozenMoEPolicy().select(t, e, top_k, h, inter)
    plan = PreparedRoutedMoE(x=hidden, gate_up=gate_up, tiled=tiled, down=down, ids=ids,
                             routing_weights=rw, logits=router_logits, renormalize=renormalize,
                             config=config, w4_decode=w4_decode)
    plan.run()
    return plan
