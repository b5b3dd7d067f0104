"""Pins the oracle's FFN-block functions (RMSNorm, fp64 → bf16 rounding, the block
composition) before the GPU block entry is checked against them."""
import json
import os
import random
from fractions import Fraction

import numpy as np
import pytest

from hydra_amd import formats as F
from oracle import oracle as O


def _golden(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


def _worst_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_rms_norm_matches_gpt_oss_fixture(golden_dir):
    """reference_ops.json["rms_norm"] (ReferenceOpsTests.swift:69-76): 1/√(mean+eps) form."""
    f = _golden(golden_dir, "reference_ops_moe.json")["rms_norm"]
    for row, exp in zip(f["input"], f["expected"]):
        assert _worst_rel(O.rms_norm(row, f["scale"], f["eps"]), exp) < 1e-12


def test_rms_norm_matches_gemma_fixtures(golden_dir):
    """gemma4_operators.json["rms_norm"] and ["rms_norm_unscaled"]: pow(mean+eps, -½) form,
    weight optional."""
    g = _golden(golden_dir, "gemma4_moe.json")
    f = g["rms_norm"]
    assert _worst_rel(O.rms_norm(f["input"], f["weight"], f["eps"], pow_form=True), f["expected"]) < 1e-12
    f = g["rms_norm_unscaled"]
    assert _worst_rel(O.rms_norm(f["input"], None, f["eps"], pow_form=True), f["expected"]) < 1e-12


def test_rms_norm_closed_forms():
    """A constant row c normalises to sign(c)·w/√(1+eps/c²); scaling a row leaves it (eps 0)."""
    w = np.linspace(0.5, 2.0, 16)
    out = O.rms_norm(np.full(16, -3.0), w, 1e-5)
    assert np.allclose(out, -w / np.sqrt(1 + 1e-5 / 9), rtol=1e-15, atol=0)
    x = np.random.default_rng(0).standard_normal(64)
    assert np.allclose(O.rms_norm(x, None, 0.0), O.rms_norm(1024 * x, None, 0.0), rtol=1e-14)
    assert np.isclose(np.mean(O.rms_norm(x, None, 0.0) ** 2), 1.0, rtol=1e-14)


def _exact_bf16(v: float) -> int:
    """bf16 bits of v by exact rational round-to-nearest-even (normal and subnormal range)."""
    if v == 0:
        return 0x8000 if np.signbit(v) else 0
    s = 0x8000 if v < 0 else 0
    q = Fraction(abs(v))
    e = q.numerator.bit_length() - q.denominator.bit_length()
    while Fraction(2) ** e > q:
        e -= 1
    while Fraction(2) ** (e + 1) <= q:
        e += 1
    e = max(e, -126)                               # subnormals share 2^-126's step
    step = Fraction(2) ** (e - 7)
    n = q / step
    k = int(n)
    r = n - k
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and k % 2):
        k += 1
    val = k * step
    if val >= Fraction(2) ** 128:
        return s | 0x7F80
    return s | int(np.float32(float(val)).view(np.uint32) >> 16)


def test_f64_to_bf16_rounds_once_to_nearest_even():
    """Against exact rational rounding: random values over the whole range, exact ties, and
    ties perturbed by less than an fp32 ulp (where rounding first to fp32 and then to bf16
    would land on the tie and pick the even neighbour)."""
    rng = random.Random(5)
    vals = []
    for _ in range(3000):
        vals.append(rng.uniform(-1, 1) * 2.0 ** rng.randint(-140, 127))
    for _ in range(500):
        b = rng.randint(0x0080, 0x7F7E)            # a normal bf16 value
        base = float(np.uint32(b << 16).view(np.float32))
        half = float(np.uint32((b << 16) | 0x8000).view(np.float32)) - base   # half a bf16 step
        tie = base + half
        vals += [tie, tie + half * 2.0 ** -30, tie - half * 2.0 ** -30, -tie]
    vals += [0.0, -0.0, 1.0, 2.0 ** -133, 2.0 ** -134, 3 * 2.0 ** -135, 3.4e38]
    got = O.f64_to_bf16(np.array(vals))
    for v, g in zip(vals, got):
        assert int(g) == _exact_bf16(v), (v, hex(int(g)), hex(_exact_bf16(v)))


def test_block_composition_matches_gemma_layer_fixture(golden_dir):
    """The reference's whole Gemma layer (gemma4_operators.json["layer"]): everything after the
    attention residual goes through O.block_forward (fp64, no bf16 rounding) with the oracle's
    fp64 expert path as moe(); the layer output must match the fixture."""
    f = _golden(golden_dir, "gemma4_moe.json")["layer"]
    w, eps = f["weights"], f["eps"]
    H, M, E, K = f["hiddenSize"], f["moeIntermediateSize"], f["expertCount"], f["topK"]
    mv = lambda m, v: np.asarray(m) @ np.asarray(v)
    hidden = np.array(f["input"])
    # attention with one cached position returns the value vector (as in test_oracle.py)
    normed = O.rms_norm(hidden, w["input_layernorm"], eps, pow_form=True)
    value = O.rms_norm(mv(w["v_proj"], normed), None, eps, pow_form=True)
    attn = np.concatenate([value] * (f["heads"] // f["keyValueHeads"]))
    hidden = hidden + O.rms_norm(mv(w["o_proj"], attn), w["post_attention_layernorm"], eps, pow_form=True)
    dense_in = O.rms_norm(hidden, w["pre_feedforward_layernorm"], eps, pow_form=True)
    g, u = mv(w["gate_proj"], dense_in), mv(w["up_proj"], dense_in)
    dense_out = mv(w["down_proj"], 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u)

    desc = F.MoEDesc(hidden=H, intermediate=M, experts=E, top_k=K, quant=O.QUANT_F64,
                     activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA, router_eps=eps)
    ex = f["experts"]
    blobs = O.pack_f64_experts(desc, [e["gate"] for e in ex], [e["up"] for e in ex],
                               [e["down"] for e in ex])

    def moe(x, xr):
        y, idx, wts, _ = O.moe_forward_f64(
            desc, blobs, x, np.array(w["router_proj"]), x_router=xr,
            router_scale=w["router_scale"], router_expert_scale=w["router_per_expert_scale"])
        return y, idx, wts

    norms = {"pre_norm": w["pre_feedforward_layernorm_2"],
             "post_expert_norm": w["post_feedforward_layernorm_2"],
             "post_dense_norm": w["post_feedforward_layernorm_1"],
             "post_norm": w["post_feedforward_layernorm"],
             "layer_scalar": w["layer_scalar"], "eps": eps}
    out, idx, wts, _ = O.block_forward(desc, norms, hidden, moe, dense_out=dense_out[None],
                                       bf16_input=False)
    assert idx[0].tolist() == f["expectedIndices"]
    assert np.max(np.abs(wts[0] - np.array(f["expectedWeights"]))) < 1e-12
    assert _worst_rel(out[0], f["expected"]) < 1e-12


def test_pre_norm_block_is_residual_plus_mixture():
    """Pre-norm structure (ReferenceLayer.swift:189-202): the block output minus its input is
    exactly the mixture of the normalised input, and the layer sees bf16(rmsnorm(hidden))."""
    from hydra_amd import synth
    desc = F.MoEDesc(hidden=128, intermediate=64, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                     activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1)
    layer = synth.make_layer(desc, seed=3)
    rng = np.random.default_rng(4)
    hidden = (rng.standard_normal((3, 128)) * 5).astype(np.float32)
    wn = synth.f32_to_bf16(rng.uniform(0.5, 1.5, 128).astype(np.float32))
    out, idx, w, x = O.block_forward_layer(layer, {"pre_norm": wn, "eps": 1e-5}, hidden)
    xn = O.rms_norm(hidden, O.bf16_to_f32(wn), 1e-5)
    assert np.array_equal(x, O.f64_to_bf16(xn))
    y, ridx, rw, _ = O.moe_forward(layer, x)
    assert np.array_equal(out, hidden.astype(np.float64) + y)
    assert np.array_equal(idx, ridx)
