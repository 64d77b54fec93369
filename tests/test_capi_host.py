"""C ABI checks that need no GPU: exports, validation, host-side W4 functions."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from llm_gpu_kernels_amd import _native as N
from llm_gpu_kernels_amd import quantize_gate_up, tile_gate_up
from oracle import moe_oracle as O

INCLUDE = Path(__file__).resolve().parents[1] / "include"


def _declared_functions():
    names = set()
    for header in INCLUDE.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M):
            if not m.group(0).lstrip().startswith(("typedef", "#")):
                names.add(m.group(1))
    return names


def test_library_exports_every_declared_function():
    lib = N.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert declared <= set(N.SIGNATURES), declared - set(N.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.moe_abi_version() == 2


def test_struct_sizes_match_header():
    # 10 int32 + 10 pointers + size_t; 14 size_t + 4 int32.
    assert ctypes.sizeof(N.MoeDesc) == 40 + 8 * 10 + 8
    assert ctypes.sizeof(N.MoeLayout) == 8 * 14 + 16
    # 9 int32 (+pad) + 2 + 8 pointers + 8 int64 + float (+pad) + pointer + size_t.
    assert ctypes.sizeof(N.GqaDesc) == 40 + 16 + 64 + 64 + 8 + 8 + 8


def _desc(**kw):
    d = N.MoeDesc()
    d.T, d.H, d.I, d.E, d.K = kw.get("T", 17), kw.get("H", 2048), kw.get("I", 768), \
        kw.get("E", 128), kw.get("K", 8)
    d.weight_format = kw.get("fmt", N.WEIGHTS_BF16)
    d.id_dtype = kw.get("ids", N.IDS_INT32)
    d.route_mode = kw.get("route", N.ROUTE_FIXED)
    d.token_block = kw.get("tb", 0)
    return d


def _layout(d):
    lay = N.MoeLayout()
    rc = N.lib().moe_workspace_layout(ctypes.byref(d), ctypes.byref(lay))
    return rc, lay


def test_layout_for_qwen_shape():
    rc, lay = _layout(_desc())
    assert rc == 0
    r = 17 * 8
    assert lay.token_block == 16 and lay.fast_path == 1 and lay.launches == 4
    assert lay.task_capacity == (r + 15) // 16 + 128
    assert lay.act % 256 == 0 and lay.routed % 256 == 0
    assert lay.total >= lay.routed + r * 2048 * 2
    rc, lay = _layout(_desc(T=1024))
    assert lay.token_block == 64 and lay.fast_path == 2
    rc, lay = _layout(_desc(T=300))
    assert lay.token_block == 32 and lay.fast_path == 1
    rc, lay = _layout(_desc(T=0))
    assert rc == 0 and lay.launches == 0
    # One multi-workgroup launch routes and plans (16 tokens per workgroup).
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=1024))
    assert lay.launches == 4
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=193))
    assert lay.launches == 4
    assert lay.partials % 256 == 0 and lay.act >= lay.partials + 13 * 129 * 4 + 4
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=16 * 256))
    assert lay.launches == 4
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=16 * 256 + 1))
    assert lay.launches == 5  # more workgroups than CUs: separate router launch
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=16))
    assert lay.launches == 3
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=17))
    assert lay.launches == 3  # bf16: routing and planning in the gate/up launch
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=32))
    assert lay.launches == 3
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=17, fmt=N.WEIGHTS_W4G128))
    assert lay.launches == 3  # W4: routing and planning in the gate/up launch too
    rc2, lay2 = _layout(_desc(route=N.ROUTE_LOGITS, T=17, fmt=N.WEIGHTS_W4G128_FOLD))
    assert rc2 == 0 and (lay2.total, lay2.launches, lay2.fast_path) == (lay.total, lay.launches, lay.fast_path)
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=17, H=4096))
    assert lay.launches == 4
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=33))
    assert lay.launches == 4
    rc, lay = _layout(_desc(route=N.ROUTE_LOGITS, T=17, E=256))
    assert lay.launches == 4
    rc, lay = _layout(_desc(H=33, I=19, E=8, K=2))
    assert rc == 0 and lay.fast_path == 0


@pytest.mark.parametrize("kw", [dict(E=0), dict(E=257), dict(K=0), dict(K=33), dict(H=0),
                                dict(I=-1), dict(T=-1), dict(fmt=7), dict(ids=9), dict(tb=8), dict(tb=48),
                                dict(route=N.ROUTE_LOGITS, ids=N.IDS_INT64),
                                dict(route=N.ROUTE_LOGITS, E=4, K=8),
                                dict(fmt=N.WEIGHTS_W4G128, H=192), dict(fmt=N.WEIGHTS_W4G128, H=512, I=48),
                                dict(fmt=N.WEIGHTS_W4G128_FOLD, H=192), dict(fmt=3),
                                dict(T=2 ** 27, K=16)])
def test_layout_rejects_invalid_descriptors(kw):
    rc, _ = _layout(_desc(**kw))
    assert rc == N.MOE_EINVAL
    assert N.last_error()


def test_plan_create_rejects_null_pointers():
    d = _desc()
    handle = ctypes.c_void_p()
    rc = N.lib().moe_plan_create(ctypes.byref(handle), ctypes.byref(d))
    assert rc == N.MOE_EINVAL and not handle.value
    with pytest.raises(ValueError):
        N.check(rc, "prepare")


@pytest.mark.parametrize("shape", [(2, 16, 128), (3, 32, 384), (1, 48, 1024)])
def test_quantize_matches_oracle_bit_exact(shape):
    g = torch.Generator().manual_seed(sum(shape))
    w = (torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16)
    w[0, 0, :128] = 0
    w[0, 1, :8] = torch.tensor([7.0, -7.0, 3.5, 4.5, -3.5, 0.5, 1.5, -0.5]).to(torch.bfloat16) * 1e-2
    p = quantize_gate_up(w.contiguous())
    ow, os_ = O.quantize_w4(w)
    assert torch.equal(p.words, ow)
    assert torch.equal(p.scales.view(torch.int16), os_.view(torch.int16))


def test_quantize_rejects_nonfinite():
    w = torch.zeros((1, 16, 128), dtype=torch.bfloat16)
    w[0, 3, 5] = float("nan")
    with pytest.raises(ValueError):
        quantize_gate_up(w)


def test_tile_layout_index_map():
    """words_t[e][rb][grp][lane][j] == v1 word 16*grp + 4*j + lane//16 of row 16*rb + lane%16."""
    e, n, k = 2, 32, 256
    words = torch.arange(e * n * k // 8, dtype=torch.int32).reshape(e, n, k // 8)
    scales = torch.arange(e * n * k // 128, dtype=torch.int16).view(torch.bfloat16).reshape(e, n, k // 128)
    t = tile_gate_up(O_packed(words, scales))
    for ei, rb, grp, lane, j in [(0, 0, 0, 0, 0), (1, 1, 1, 63, 3), (0, 1, 0, 17, 2), (1, 0, 1, 40, 1)]:
        r, g = lane % 16, lane // 16
        assert t.words[ei, rb, grp, lane, j] == words[ei, rb * 16 + r, 16 * grp + 4 * j + g]
        assert t.scales[ei, rb, grp, r].view(torch.int16) == scales[ei, rb * 16 + r, grp].view(torch.int16)
    assert sorted(t.words.reshape(-1).tolist()) == list(range(e * n * k // 8))


def O_packed(words, scales):
    from llm_gpu_kernels_amd.weight_quant import PackedGateUp
    return PackedGateUp(words, scales, {})


def _decode_word_like_kernel(word, s):
    """Host restatement of the kernel's w4_decode8 (llm_gpu_kernels_amd/csrc/common.h):
    nibble n at mantissa position p of 2^23 -> fma(2^23 + n*16^p, s*16^-p,
    -(2^(23-4p)+8)*s), evaluated exactly in float64, rounded once to fp32."""
    import struct
    def fl(b):
        return struct.unpack("<f", struct.pack("<I", b & 0xFFFFFFFF))[0]
    lo, hi = (word << 8) & 0xFFFFFFFF, word >> 12
    plan = [(lo, 2), (lo, 3), (word, 2), (word, 3), (word, 4), (hi, 2), (hi, 3), (hi, 4)]
    out = []
    for src, p in plan:
        v = fl(0x4B000000 | (src & (0xF << (4 * p))))
        sp = float(torch.tensor(s * 2.0 ** (-4 * p), dtype=torch.float32))
        cp = float(torch.tensor(-s * float(2 ** (23 - 4 * p) + 8), dtype=torch.float32))
        out.append(float(torch.tensor(v * sp + cp, dtype=torch.float32)))
    return out


def test_tile_emulated_decode_matches_oracle_dequant():
    """Host emulation of the kernel decode on the tiled layout == oracle dequant."""
    g = torch.Generator().manual_seed(11)
    w = (torch.randn((1, 32, 256), generator=g) * 0.03).to(torch.bfloat16)
    w[0, 5, :128] = 0  # scale 1 group
    p = quantize_gate_up(w)
    t = tile_gate_up(p)
    ref = O.dequantize_w4(p.words, p.scales)
    e, n, k = 1, 32, 256
    out = torch.empty((e, n, k), dtype=torch.bfloat16)
    wt = t.words.to(torch.int64) & 0xFFFFFFFF
    st = t.scales.float()
    for rb in range(n // 16):
        for grp in range(k // 128):
            for lane in range(64):
                r, gg = lane % 16, lane // 16
                s = float(st[0, rb, grp, r])
                for j in range(4):
                    vals = _decode_word_like_kernel(int(wt[0, rb, grp, lane, j]), s)
                    base = grp * 128 + 32 * j + 8 * gg
                    out[0, rb * 16 + r, base:base + 8] = torch.tensor(vals).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_cuda_variant_names_validated():
    """prepare_cuda_moe accepts the reference's variant names only
    (moe_cuda.py:17,57-58); the check precedes any device work."""
    from llm_gpu_kernels_amd import moe as M
    assert M.CUDA_VARIANTS == ("sync", "async", "async_skip")
    with pytest.raises(ValueError, match="unsupported CUDA variant"):
        M.prepare_cuda_moe(None, None, None, None, None, variant="mfma")


def test_attention_out_storage_check():
    """Output aliasing q or any K/V segment storage is rejected (views of one
    storage included); empty tensors never alias."""
    from llm_gpu_kernels_amd.attention import check_out_storage
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    kv = torch.zeros(2, 4, 8, 128, dtype=torch.bfloat16)
    out = torch.zeros_like(q)
    check_out_storage(out, [q, kv[0], kv[1]])
    with pytest.raises(ValueError, match="share storage"):
        check_out_storage(q, [q, kv[0], kv[1]])
    with pytest.raises(ValueError, match="share storage"):
        check_out_storage(kv[1], [q, kv[0]])
    check_out_storage(torch.empty(0, 32, 128), [torch.empty(0, 8, 128)])


def test_status_bit_values():
    """Status bits of the header, as the Python layer reads them."""
    text = (INCLUDE / "moe_mi355x.h").read_text()
    for name, value in (("BAD_ID", 1), ("BAD_WEIGHT", 2), ("BAD_LOGIT", 4), ("DIRTY_COUNTERS", 8), ("STALLED", 16)):
        assert re.search(rf"#define MOE_STATUS_{name} {value}u", text), name
        assert getattr(N, f"STATUS_{name}") == value


def test_static_workspace_size_matches_header():
    text = (INCLUDE / "moe_mi355x.h").read_text()
    assert re.search(r"#define MOE_STATIC_WORKSPACE_BYTES \(16u << 20\)", text)
    assert N.STATIC_WORKSPACE_BYTES == 16 << 20
