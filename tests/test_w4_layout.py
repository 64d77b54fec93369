"""M24 physical W4 layout (src/llm_gpu_kernels/moe_weight_layout.py:14-19, 81-127):
the oracle's restatement pinned by hand-computed positions, the library's
repack / restore bit-exact against it, and tiling from either layout identical."""
import pytest
import torch

from llm_gpu_kernels_amd import (PackedGateUp, RepackedGateUp, repack_gate_up,
                                 restore_v1_layout, tile_gate_up)
from llm_gpu_kernels_amd.weight_quant import M24_LAYOUT
from oracle import moe_oracle as O


def _distinct_pack(e, n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    words = torch.randperm(e * n * (k // 8), generator=g).to(torch.int32).reshape(e, n, k // 8)
    scales = torch.randn((e, n, k // 128), generator=g).to(torch.bfloat16)
    return words, scales


def test_oracle_positions_from_layout_string():
    # words[E,projection,Ntile,K32,word,Nlane]: v1 row n = p*(N/2) + t*64 + l,
    # v1 word j = 4*k32 + w (moe_weight_layout.py:14-17, 85-86).
    e, n, k = 2, 256, 512
    words, scales = _distinct_pack(e, n, k)
    pw, ps = O.m24_repack(words, scales)
    assert tuple(pw.shape) == (e, 2, n // 128, k // 32, 4, 64)
    assert tuple(ps.shape) == (e, 2, n // 128, k // 128, 64)
    half = n // 2
    g = torch.Generator().manual_seed(1)
    for _ in range(200):
        ei = int(torch.randint(e, (1,), generator=g))
        ni = int(torch.randint(n, (1,), generator=g))
        ji = int(torch.randint(k // 8, (1,), generator=g))
        gi = int(torch.randint(k // 128, (1,), generator=g))
        p, t, l = ni // half, (ni % half) // 64, ni % 64
        assert pw[ei, p, t, ji // 4, ji % 4, l] == words[ei, ni, ji]
        assert ps[ei, p, t, gi, l].view(torch.int16) == scales[ei, ni, gi].view(torch.int16)
    # A permutation: every word appears exactly once.
    assert torch.equal(pw.flatten().sort().values, words.flatten().sort().values)


def test_oracle_reference_physical_shapes():
    # PHYSICAL_WORDS_SHAPE / PHYSICAL_SCALES_SHAPE (moe_weight_layout.py:18-19)
    # for the audited logical shape [128, 1536, 2048], one expert here.
    words, scales = _distinct_pack(1, 1536, 2048)
    pw, ps = O.m24_repack(words, scales)
    assert tuple(pw.shape)[1:] == (2, 12, 64, 4, 64)
    assert tuple(ps.shape)[1:] == (2, 12, 16, 64)


def test_library_repack_restore_bit_exact():
    words, scales = _distinct_pack(3, 384, 1024, seed=3)
    packed = PackedGateUp(words, scales, {"format_version": 1})
    rep = repack_gate_up(packed)
    ow, os_ = O.m24_repack(words, scales)
    assert torch.equal(rep.words, ow)
    assert torch.equal(rep.scales.view(torch.int16), os_.view(torch.int16))
    assert rep.metadata["format_version"] == 2 and rep.metadata["layout"] == M24_LAYOUT
    back = restore_v1_layout(rep)
    assert torch.equal(back.words, words)
    assert torch.equal(back.scales.view(torch.int16), scales.view(torch.int16))
    assert back.shape == (3, 384, 1024) and rep.shape == (3, 384, 1024)


def test_restore_rejects_foreign_metadata_and_tampered_buffers():
    words, scales = _distinct_pack(1, 256, 256, seed=4)
    rep = repack_gate_up(PackedGateUp(words, scales, {}))
    with pytest.raises(ValueError):
        restore_v1_layout(RepackedGateUp(rep.words, rep.scales, dict(rep.metadata, layout="x")))
    tampered = rep.words.clone()
    tampered[0, 0, 0, 0, 0, 0] ^= 1
    with pytest.raises(ValueError):
        restore_v1_layout(RepackedGateUp(tampered, rep.scales, rep.metadata))
    with pytest.raises(ValueError):
        restore_v1_layout(RepackedGateUp(rep.words[..., :32], rep.scales, {}))
    # Without metadata the buffers are taken as given.
    assert torch.equal(restore_v1_layout(RepackedGateUp(rep.words, rep.scales)).words, words)


def test_tiling_from_m24_equals_tiling_from_v1():
    g = torch.Generator().manual_seed(5)
    w = (torch.randn((2, 256, 512), generator=g) * 0.02).to(torch.bfloat16)
    from llm_gpu_kernels_amd import quantize_gate_up
    packed = quantize_gate_up(w)
    a = tile_gate_up(packed)
    b = tile_gate_up(repack_gate_up(packed))
    assert torch.equal(a.words, b.words)
    assert torch.equal(a.scales.view(torch.int16), b.scales.view(torch.int16))


def _reference_restore_accepts(rep):
    """The metadata conditions of the reference's restore_v1_layout
    (moe_weight_layout.py:130-175), restated as checks on a pack this library
    wrote: layout declaration, physical digests of the buffers, canonical
    digests of the restored v1 bits, and a v1 snapshot carrying them."""
    from llm_gpu_kernels_amd.weight_quant import _digest
    meta = rep.metadata
    assert meta["format_version"] == 2 and meta["layout"] == M24_LAYOUT
    assert meta["group_size"] == 128 and tuple(meta["logical_shape"]) == rep.shape
    assert _digest(rep.words) == meta["physical_words_sha256"]
    assert _digest(rep.scales) == meta["physical_scales_sha256"]
    back = restore_v1_layout(rep)
    assert _digest(back.words) == meta["canonical_words_sha256"]
    assert _digest(back.scales) == meta["canonical_scales_sha256"]
    v1 = meta["canonical_v1_metadata"]
    assert v1["format_version"] == 1 and v1["group_size"] == 128
    assert tuple(v1["logical_shape"]) == rep.shape
    assert v1["words_sha256"] == meta["canonical_words_sha256"]
    assert v1["scales_sha256"] == meta["canonical_scales_sha256"]
    led = meta["byte_ledger"]
    assert led["physical_packed_total_bytes"] == led["canonical_packed_total_bytes"]
    return back


def test_m24_export_carries_what_reference_restore_checks():
    # The audited shape: 192 MiB of words + 6 MiB of scales = 198 MiB
    # (moe_weight_layout.py:119-120), v1 metadata as quantize_gate_up writes it.
    from llm_gpu_kernels_amd.weight_quant import _digest
    g = torch.Generator().manual_seed(9)
    words = torch.randint(-2**31, 2**31 - 1, (128, 1536, 256), generator=g, dtype=torch.int32)
    scales = torch.rand((128, 1536, 16), generator=g).to(torch.bfloat16)
    v1 = dict(format_version=1, logical_shape=[128, 1536, 2048], group_size=128,
              words_sha256=_digest(words), scales_sha256=_digest(scales))
    rep = repack_gate_up(PackedGateUp(words, scales, v1))
    assert tuple(rep.words.shape) == (128, 2, 12, 64, 4, 64)
    assert tuple(rep.scales.shape) == (128, 2, 12, 16, 64)
    assert rep.metadata["byte_ledger"]["physical_packed_total_mib"] == 198.0
    back = _reference_restore_accepts(rep)
    assert torch.equal(back.words, words)
    assert back.metadata["words_sha256"] == v1["words_sha256"]


def test_v1_digests_checked_on_import_and_restore():
    from llm_gpu_kernels_amd import quantize_gate_up
    g = torch.Generator().manual_seed(6)
    w = (torch.randn((2, 256, 256), generator=g) * 0.02).to(torch.bfloat16)
    packed = quantize_gate_up(w)
    _reference_restore_accepts(repack_gate_up(packed))
    bad = packed.words.clone()
    bad[0, 0, 0] ^= 0x10
    tampered = PackedGateUp(bad, packed.scales, packed.metadata)
    with pytest.raises(ValueError, match="words_sha256"):
        tile_gate_up(tampered)
    with pytest.raises(ValueError, match="words_sha256"):
        repack_gate_up(tampered)
    with pytest.raises(ValueError):
        tile_gate_up(PackedGateUp(packed.words, packed.scales, dict(packed.metadata, format_version=3)))
    rep = repack_gate_up(packed)
    # A physical pack consistent with its physical digests but not with the
    # canonical ones, or with a v1 snapshot of other bits, is refused.
    for key in ("canonical_words_sha256", "canonical_scales_sha256"):
        with pytest.raises(ValueError, match="canonical"):
            restore_v1_layout(RepackedGateUp(rep.words, rep.scales, dict(rep.metadata, **{key: "0" * 64})))
    snap = dict(rep.metadata["canonical_v1_metadata"], words_sha256="f" * 64)
    with pytest.raises(ValueError, match="snapshot"):
        restore_v1_layout(RepackedGateUp(rep.words, rep.scales, dict(rep.metadata, canonical_v1_metadata=snap)))
