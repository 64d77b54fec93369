"""Pin the CPU oracle: reference golden records, brute force and closed forms."""
import itertools
import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "m4_reference_records.json").read_text())
CASES = GOLDEN["cases"]
DT = {"torch.int32": torch.int32, "torch.int64": torch.int64}


def _inputs(c):
    return O.make_inputs(tokens=c["T"], experts=c["E"], topk=c["topk"], hidden=c["H"],
                         intermediate=c["I"], id_dtype=DT[c["id_dtype"]],
                         pattern=c["route_pattern"], seed=c["seed"],
                         signed_weights=c.get("signed_weights", False))


@pytest.mark.parametrize("case", [c for c in CASES if c["E"] <= 16], ids=lambda c: c["name"])
def test_generator_matches_reference_digests(case):
    """make_inputs/make_ids/tensor_hash reproduce the recorded sha256 digests."""
    x, gu, dn, ids, rw = _inputs(case)
    assert O.tensor_hash(ids) == case["routing_sha256"]
    assert O.tensor_hash(x, gu, dn, rw) == case["input_sha256"]


@pytest.mark.slow
def test_generator_matches_reference_digest_qwen_shape():
    case = next(c for c in CASES if c["name"] == "qwen3_30b_a3b_shape_T17_random")
    x, gu, dn, ids, rw = _inputs(case)
    assert O.tensor_hash(ids) == case["routing_sha256"]
    assert O.tensor_hash(x, gu, dn, rw) == case["input_sha256"]


@pytest.mark.parametrize("case", [c for c in CASES if "expected_counts" in c and c["E"] <= 16],
                         ids=lambda c: c["name"])
def test_dispatch_matches_recorded_counts_offsets(case):
    _, _, _, ids, _ = _inputs(case)
    d = O.canonical_dispatch(ids, case["E"])
    assert d["counts"].tolist() == case["expected_counts"]
    assert d["offsets"].tolist() == case["expected_offsets"]


def _check_dispatch_invariants(ids, experts, d):
    """The reference's validators (moe_benchmark.py:139-190, ranked_moe_benchmark.py:120-167)."""
    flat = ids.reshape(-1).long()
    counts = torch.bincount(flat, minlength=experts)
    assert d["counts"].tolist() == counts.tolist()
    assert d["offsets"].tolist() == (torch.cumsum(counts, 0) - counts).tolist()
    m = d["map"].long()
    assert sorted(m.tolist()) == list(range(flat.numel()))
    for q, p in enumerate(m.tolist()):
        e = int(flat[q])
        assert d["offsets"][e] <= p < d["offsets"][e] + counts[e]
        assert p == d["offsets"][e] + d["ranks"][q]
        assert d["row_route"][p] == q
    for e in range(experts):
        r = sorted(d["ranks"][flat == e].tolist())
        assert r == list(range(int(counts[e])))


@pytest.mark.parametrize("seed", range(6))
def test_canonical_dispatch_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    experts = [1, 3, 8, 16, 128, 256][seed]
    ids = torch.randint(0, experts, (37, 4), generator=g)
    d = O.canonical_dispatch(ids, experts)
    _check_dispatch_invariants(ids, experts, d)
    flat = ids.reshape(-1).tolist()
    for q in range(len(flat)):  # stable: rank = earlier routes with the same expert
        assert d["ranks"][q] == sum(1 for j in range(q) if flat[j] == flat[q])


def test_canonical_dispatch_invalid_ids():
    ids = torch.tensor([[0, 5], [-1, 1], [1, 0]])
    d = O.canonical_dispatch(ids, 2)
    assert d["counts"].tolist() == [2, 2]
    assert d["map"].tolist() == [0, -1, -1, 2, 3, 1]
    assert d["ranks"].tolist() == [0, -1, -1, 0, 1, 1]


def _brute_moe(x, gu, dn, ids, rw):
    t, h = x.shape
    e, _, inter = dn.shape
    out = [[0.0] * h for _ in range(t)]
    xf, guf, dnf = x.double().tolist(), gu.double().tolist(), dn.double().tolist()
    for ti, s in itertools.product(range(t), range(ids.shape[1])):
        ex = int(ids[ti, s])
        act = []
        for n in range(inter):
            g = sum(xf[ti][k] * guf[ex][n][k] for k in range(h))
            u = sum(xf[ti][k] * guf[ex][inter + n][k] for k in range(h))
            act.append(g / (1 + math.exp(-g)) * u)
        for o in range(h):
            out[ti][o] += float(rw[ti, s]) * sum(act[n] * dnf[ex][o][n] for n in range(inter))
    return torch.tensor(out)


@pytest.mark.parametrize("pattern", ["random", "duplicate", "all_hot"])
def test_moe_reference_brute_force(pattern):
    x, gu, dn, ids, rw = O.make_inputs(tokens=5, experts=4, topk=3, hidden=7, intermediate=5,
                                       id_dtype=torch.int64, pattern=pattern, seed=3,
                                       signed_weights=True)
    ref = O.moe_reference(x, gu, dn, ids, rw)
    brute = _brute_moe(x, gu, dn, ids, rw)
    assert torch.allclose(ref.double(), brute.double(), rtol=1e-4, atol=1e-4)


def test_moe_reference_closed_forms():
    # E=1, K=1, identity-like weights: out = w * silu(x) * x projected back.
    h = inter = 4
    x = torch.tensor([[0.5, -1.0, 2.0, 0.25]], dtype=torch.bfloat16)
    gu = torch.cat([torch.eye(4), torch.eye(4)]).to(torch.bfloat16)[None]
    dn = torch.eye(4, dtype=torch.bfloat16)[None]
    ids = torch.zeros((1, 1), dtype=torch.int64)
    rw = torch.tensor([[0.75]])
    ref = O.moe_reference(x, gu, dn, ids, rw)
    xf = x.float()
    assert torch.allclose(ref, 0.75 * F.silu(xf) * xf)
    # Linearity in routing weights and duplicate IDs add up.
    x, gu, dn, ids, rw = O.make_inputs(tokens=3, experts=2, topk=2, hidden=8, intermediate=4,
                                       id_dtype=torch.int64, pattern="random", seed=1)
    a = O.moe_reference(x, gu, dn, ids, rw)
    b = O.moe_reference(x, gu, dn, ids, 2 * rw)
    assert torch.allclose(2 * a, b, rtol=1e-6, atol=1e-6)
    dup = torch.zeros((3, 2), dtype=torch.int64)
    single = O.moe_reference(x, gu, dn, dup[:, :1], torch.ones((3, 1)))
    double = O.moe_reference(x, gu, dn, dup, torch.ones((3, 2)))
    assert torch.allclose(2 * single, double, rtol=1e-6, atol=1e-5)


def test_staged_oracle_within_tolerance_of_fp32():
    x, gu, dn, ids, rw = O.make_inputs(tokens=17, experts=8, topk=2, hidden=64, intermediate=32,
                                       id_dtype=torch.int64, pattern="random", seed=7)
    gu = (gu.float() * 0.05).to(torch.bfloat16)
    dn = (dn.float() * 0.05).to(torch.bfloat16)
    m = O.error(O.staged_bf16_oracle(x, gu, dn, ids, rw), O.moe_reference(x, gu, dn, ids, rw))
    assert m["passed"], m


def test_error_metric_known_values():
    o = torch.tensor([1.0, -2.0, 2.0])
    a = torch.tensor([1.0, -2.0, 2.02])
    m = O.error(a, o)
    assert math.isclose(m["normalized_max"], 0.01, rel_tol=1e-4)
    assert math.isclose(m["relative_rms"], math.sqrt(0.02 ** 2 / 3) / math.sqrt(3), rel_tol=1e-4)


@pytest.mark.parametrize("seed", range(4))
def test_route_topk_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn((9, 16), generator=g)
    ids, w = O.route_topk(logits, 4, renormalize=False)
    probs = torch.softmax(logits, -1)
    for t in range(9):
        order = sorted(range(16), key=lambda j: -float(probs[t, j]))[:4]
        assert ids[t].tolist() == order
        assert torch.allclose(w[t], probs[t, order])
    ids2, w2 = O.route_topk(logits, 4, renormalize=True)
    assert torch.equal(ids, ids2)
    assert torch.allclose(w2.sum(-1), torch.ones(9))
    tv, ti = torch.topk(probs, 4)
    assert torch.equal(ti.to(torch.int32), ids)


def test_route_topk_ties_choose_lower_index():
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.0, 3.0]])
    ids, _ = O.route_topk(logits, 3)
    assert ids.tolist() == [[1, 2, 4]]


def test_w4_quantize_closed_forms():
    w = torch.zeros((1, 2, 256), dtype=torch.float32)
    # group 0 of row 0 stays zero -> scale 1, q = 0 -> nibble 8.
    w[0, 0, 128:] = torch.linspace(-1, 1, 128)
    w[0, 1, :8] = torch.tensor([7.0, -7.0, 3.5, 4.5, -3.5, 0.5, 1.5, -0.5])
    wb = w.to(torch.bfloat16)
    words, scales = O.quantize_w4(wb)
    assert scales[0, 0, 0].item() == 1.0
    assert words[0, 0, :16].tolist() == [0x88888888 - 2 ** 32] * 16
    # max |w| = 7 -> scale 1; half-way values round to even: 3.5->4, 4.5->4, -3.5->-4,
    # 0.5->0, 1.5->2, -0.5->-0.
    assert scales[0, 1, 0].item() == 1.0
    expect_q = [7, -7, 4, 4, -4, 0, 2, 0]
    word = sum((q + 8) << (4 * i) for i, q in enumerate(expect_q))
    assert words[0, 1, 0].item() & 0xFFFFFFFF == word
    # extremal element maps to +-7 and the nibble order is earliest-K-lowest.
    deq = O.dequantize_w4(words, scales)
    assert deq[0, 1, :8].float().tolist() == [float(q) for q in expect_q]
    row = deq[0, 0, 128:].float()
    s = scales[0, 0, 1].float()
    assert s.item() == torch.tensor(1.0 / 7).to(torch.bfloat16).item()
    assert row.abs().max().item() == (7 * s).to(torch.bfloat16).item()


def test_w4_round_trip_error_bound():
    g = torch.Generator().manual_seed(5)
    w = (torch.randn((2, 16, 512), generator=g) * 0.02).to(torch.bfloat16)
    words, scales = O.quantize_w4(w)
    deq = O.dequantize_w4(words, scales).float()
    # |w - deq| <= scale/2 (+ bf16 rounding of the product).
    s = scales.float().repeat_interleave(128, -1)
    assert ((w.float() - deq).abs() <= 0.5 * s + s * 7 * 2 ** -8).all()
    # requantising the dequantised weights is idempotent.
    w2, s2 = O.quantize_w4(deq.to(torch.bfloat16))
    assert torch.equal(w2, words)


def test_w4_unrounded_dequantisation():
    """The folded decode's effective weights: q * scale exactly in fp32.  Closed
    forms (scale 3 * 2^-3 = 0.375: q * s needs up to 5 significant bits, so
    nothing rounds; scale 1 + 2^-7: 7 * s = 7 + 7/128 has 10 significant bits
    and rounds in bf16), and rounding to bf16 gives dequantize_w4 bitwise."""
    q = torch.tensor([-8, -7, -3, 0, 1, 3, 5, 7])
    word = int(sum((int(v) + 8) << (4 * i) for i, v in enumerate(q.tolist())))
    words = torch.tensor([[[word - 2 ** 32 if word >= 2 ** 31 else word] * 16]], dtype=torch.int32)
    for sc in (0.375, 1 + 2 ** -7):
        scales = torch.tensor([[[sc]]], dtype=torch.bfloat16)
        un = O.dequantize_w4_unrounded(words, scales)
        assert un[0, 0, :8].tolist() == [float(v) * sc for v in q.tolist()]
        assert torch.equal(un.to(torch.bfloat16), O.dequantize_w4(words, scales))
    assert O.dequantize_w4_unrounded(words, torch.tensor([[[1 + 2 ** -7]]], dtype=torch.bfloat16))[0, 0, 7] \
        != O.dequantize_w4(words, torch.tensor([[[1 + 2 ** -7]]], dtype=torch.bfloat16))[0, 0, 7].float()
    g = torch.Generator().manual_seed(9)
    w = (torch.randn((2, 16, 512), generator=g) * 0.02).to(torch.bfloat16)
    words, scales = O.quantize_w4(w)
    un, deq = O.dequantize_w4_unrounded(words, scales), O.dequantize_w4(words, scales)
    assert torch.equal(un.to(torch.bfloat16), deq)
    assert ((un - deq.float()).abs() <= un.abs() * 2 ** -8).all()  # bf16 unit roundoff


def test_gqa_reference_matches_manual_softmax():
    g = torch.Generator().manual_seed(0)
    t, hq, hkv, d = 3, 4, 2, 8
    q = torch.randn((t, hq, d), generator=g)
    segs = [(torch.randn((L, hkv, d), generator=g), torch.randn((L, hkv, d), generator=g))
            for L in (2, 0, 1, t)]
    out = O.gqa_segmented_reference(q, segs)
    keys = torch.cat([k for k, _ in segs])
    vals = torch.cat([v for _, v in segs])
    hist = keys.shape[0] - t
    for i in range(t):
        for h in range(hq):
            kv = h // (hq // hkv)
            n_vis = hist + i + 1
            sc = (keys[:n_vis, kv] @ q[i, h]) / math.sqrt(d)
            p = torch.softmax(sc, 0)
            assert torch.allclose(out[i, h], p @ vals[:n_vis, kv], atol=1e-5)


def test_gqa_reference_closed_forms():
    """Zero keys give uniform weights over the visible keys (history + causal prefix);
    query 0 of an empty history sees exactly one key; KV head j of constant value j
    shows the head mapping h // (Hq / Hkv)."""
    g = torch.Generator().manual_seed(1)
    t, hq, hkv, d = 5, 8, 2, 16
    q = torch.randn((t, hq, d), generator=g)
    lens = (3, 0, 2, t)
    segs = [(torch.zeros((L, hkv, d)), torch.randn((L, hkv, d), generator=g)) for L in lens]
    out = O.gqa_segmented_reference(q, segs)
    vals = torch.cat([v for _, v in segs])
    hist = sum(lens[:-1])
    for i in range(t):
        for h in range(hq):
            mean = vals[:hist + i + 1, h // (hq // hkv)].mean(0)
            assert torch.allclose(out[i, h], mean, atol=1e-6)
    # single visible key: the output is that key's value row exactly.
    one = [(torch.randn((t, hkv, d), generator=g), torch.randn((t, hkv, d), generator=g))]
    out1 = O.gqa_segmented_reference(q, one)
    for h in range(hq):
        assert torch.equal(out1[0, h], one[0][1][0, h // (hq // hkv)])
    # head mapping: KV head j holds the constant j in every value.
    const = [(torch.randn((L, hkv, d), generator=g),
              torch.arange(hkv, dtype=torch.float32).view(1, hkv, 1).expand(L, hkv, d).clone())
             for L in lens]
    out2 = O.gqa_segmented_reference(q, const)
    for h in range(hq):
        assert torch.allclose(out2[:, h], torch.full((t, d), float(h // (hq // hkv))), atol=1e-6)
