"""Pins the fp64 oracle before anything is checked against it.

Each oracle function is checked against the reference's own golden vectors where they exist
(tests/golden/, copied from the reference's test fixtures) and otherwise against closed forms,
brute force, or the independent dense formulation in tests/dense_ref.py.
"""
import itertools
import json
import math
import os

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O

import dense_ref as D


def _golden(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


# ---- MXFP4 (MXFP4Tests.swift) ---------------------------------------------------------------

def test_mxfp4_matches_reference_golden_bit_for_bit(golden_dir):
    packed = np.fromfile(os.path.join(golden_dir, "mxfp4_packed.bin"), np.uint8)
    scales = np.fromfile(os.path.join(golden_dir, "mxfp4_scales.bin"), np.uint8)
    expected = np.fromfile(os.path.join(golden_dir, "mxfp4_expected.f32"), np.float32)
    got = O.mxfp4_decode(packed, scales)
    assert got.size == expected.size == 64 * 32
    # Stricter than the reference's `==`: the sign of zero must match as well.
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_mxfp4_low_nibble_is_even_index():
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x71
    out = O.mxfp4_decode(packed, np.array([127], np.uint8))
    assert out[0] == 0.5 and out[1] == 6.0


def test_mxfp4_full_e2m1_table():
    packed = np.zeros(16, np.uint8)
    for i in range(8):
        packed[i] = (2 * i) | ((2 * i + 1) << 4)
    out = O.mxfp4_decode(packed, np.array([127], np.uint8))
    exp = [0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6]
    assert out[:16].tolist() == exp
    assert np.signbit(out[8])


@pytest.mark.parametrize("exponent", [-127, -40, -8, -1, 0, 1, 8, 40, 127])
def test_mxfp4_scale_is_exact_power_of_two(exponent):
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x02
    out = O.mxfp4_decode(packed, np.array([127 + exponent], np.uint8))
    assert out[0] == np.float32(math.ldexp(1.0, exponent))


def test_mxfp4_scale_255_is_infinite_factor():
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x02
    out = O.mxfp4_decode(packed, np.array([255], np.uint8))
    assert np.isinf(out[0]) and np.isnan(out[2])   # 0 × inf


def test_blob_layout_matches_reference_byte_counts():
    off, by, payload, stride = O.blob_layout(F.GPT_OSS_20B)
    # MXFP4Tests.swift:106-119: gate_up [5760 × 2880] and down [2880 × 2880] of gpt-oss-20b.
    assert by[0] == 8_294_400 and by[1] == 518_400
    assert by[3] == 4_147_200 and by[4] == 259_200
    assert sum(by) == 13_236_480
    assert all(o % 256 == 0 for o in off) and stride % 16384 == 0 and stride >= payload
    assert sum(O.blob_layout(F.QWEN_35B_A3B_Q4)[1]) == 1_769_472
    assert sum(O.blob_layout(F.QWEN_35B_A3B_Q8)[1]) == 3_342_336
    assert sum(O.blob_layout(F.GEMMA_BF16)[1]) == 11_894_784
    for desc in F.CONFIGS.values():
        py = F.blob_layout(desc)
        assert [list(py.offsets), list(py.sizes)] == list(O.blob_layout(desc)[:2])
        assert (py.payload, py.stride) == O.blob_layout(desc)[2:]


# ---- BF16 (BF16.swift) ----------------------------------------------------------------------

def test_bf16_exhaustive_round_trip():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_to_f32(bits)
    assert np.array_equal(f.view(np.uint32), bits.astype(np.uint32) << 16)
    back = O.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.array_equal(back[nan], bits[nan] | 0x40)


def test_bf16_round_to_nearest_even():
    one = 1.0
    cases = {
        one: 0x3F80,
        one + 2.0 ** -8: 0x3F80,               # tie → even (down)
        one + 3 * 2.0 ** -8: 0x3F82,           # tie → even (up)
        one + 2.0 ** -8 + 2.0 ** -20: 0x3F81,  # above the tie → up
        -2.5: 0xC020,
        float("inf"): 0x7F80,
    }
    got = O.f32_to_bf16(np.array(list(cases), np.float32))
    assert got.tolist() == list(cases.values())
    assert np.array_equal(got, synth.f32_to_bf16(np.array(list(cases), np.float32)))


# ---- MLX affine (MLXAffineTests.swift) ------------------------------------------------------

def test_mlx_unpack_low_order_first():
    assert O.mlx_unpack(np.array([0x76543210], np.uint32), 4).tolist() == list(range(8))
    assert O.mlx_unpack(np.array([0x76543210], np.uint32), 8).tolist() == [0x10, 0x32, 0x54, 0x76]
    assert O.mlx_unpack(np.array([0xFFFFFFFF], np.uint32), 4).tolist() == [15] * 8


def test_mlx_dequant_is_affine():
    got = O.mlx_dequant(np.array([0x76543210], np.uint32), [0.5], [-4.0], 8, 4, 8)
    assert got.tolist() == [-4.0, -3.5, -3.0, -2.5, -2.0, -1.5, -1.0, -0.5]


def test_mlx_groups_run_along_the_row():
    got = O.mlx_dequant(np.array([0, 0x11111111], np.uint32), [1.0, 10.0], [0.0, 100.0], 16, 4, 8)
    assert got[:8].tolist() == [0.0] * 8 and got[8:].tolist() == [110.0] * 8


@pytest.mark.parametrize("bits", [4, 8])
def test_mlx_dequant_matches_fma_in_float32(bits):
    # The golden definition: fp32(fma(q, s, b)) equals the correctly rounded fp64 q·s+b.
    rng = np.random.default_rng(bits)
    cols, group = 256, 64
    words = rng.integers(0, 2 ** 32, cols * bits // 32, dtype=np.uint64).astype(np.uint32)
    s = D.bf16(synth.bf16_normal(1, "s", cols // group, 0.01, 0.002))
    b = D.bf16(synth.f32_to_bf16((-7.5 * s).astype(np.float32)))
    got = O.mlx_dequant(words, s, b, cols, bits, group)
    q = D.mlx_matrix(words, synth.f32_to_bf16(s.astype(np.float32)),
                     synth.f32_to_bf16(b.astype(np.float32)), 1, cols, bits, group)[0]
    assert np.array_equal(got, q)


# ---- activations ---------------------------------------------------------------------------

def test_swiglu_matches_reference_fixture(golden_dir):
    fx = _golden(golden_dir, "reference_ops_moe.json")["swiglu"]
    for row, exp in zip(fx["input"], fx["expected"]):
        got = O.swiglu(row, fx["alpha"], fx["limit"])
        assert np.max(np.abs(got - np.array(exp))) < 1e-12


def test_swiglu_clamps_gate_above_only_and_linear_both_sides():
    # gate -100 stays unclamped (σ → 0), gate 100 clamps to 7; linear ±100 clamps to ±7.
    got = O.swiglu([-100.0, 0.0, 100.0, 100.0, 100.0, -100.0])
    assert abs(got[0]) < 1e-60
    s7 = 7.0 / (1.0 + math.exp(-1.702 * 7.0))
    assert got[1] == pytest.approx(s7 * 8.0, rel=1e-15)
    assert got[2] == pytest.approx(s7 * -6.0, rel=1e-15)


def test_gelu_tanh_matches_reference_fixture(golden_dir):
    fx = _golden(golden_dir, "gemma4_moe.json")["gelu_tanh"]
    for x, exp in zip(fx["input"], fx["expected"]):
        assert abs(O.gelu_tanh(x) - exp) < 1e-12


def test_silu_and_sigmoid_closed_forms():
    for x in [-30.0, -1.5, 0.0, 0.25, 3.0, 40.0]:
        assert O.sigmoid(x) == pytest.approx(1.0 / (1.0 + math.exp(-x)), rel=1e-15)
        assert O.silu(x) == pytest.approx(x / (1.0 + math.exp(-x)), rel=1e-15, abs=1e-300)
    assert O.sigmoid(0.0) == 0.5 and O.silu(0.0) == 0.0


# ---- routers -------------------------------------------------------------------------------

def test_router_matches_reference_fixture(golden_dir):
    fx = _golden(golden_dir, "reference_ops_moe.json")["router"]
    for logits, idx, w in zip(fx["logits"], fx["indices"], fx["weights"]):
        gi, gw = O.router_topk_softmax(logits, fx["top_k"])
        assert gi.tolist() == idx
        assert np.max(np.abs(gw - np.array(w))) < 1e-12


def test_router_ties_pick_the_smaller_index():
    logits = [0.0, 2.0, 5.0, 2.0, 5.0, 1.0]
    idx, _ = O.router_topk_softmax(logits, 4)
    assert idx.tolist() == [2, 4, 1, 3]
    idx, _ = O.router_softmax_topk_renorm(logits, 4)
    assert idx.tolist() == [2, 4, 1, 3]


def test_qwen_router_equals_topk_then_softmax():
    # QwenMixtureTests.swift:34-65: softmax→top-k→renormalise ≡ top-k→softmax.
    rng = np.random.default_rng(3)
    for _ in range(200):
        E = int(rng.integers(8, 300))
        k = int(rng.integers(1, 9))
        logits = rng.normal(size=E) * 2
        a_idx, a_w = O.router_topk_softmax(logits, k)
        b_idx, b_w = O.router_softmax_topk_renorm(logits, k)
        assert a_idx.tolist() == b_idx.tolist()
        assert np.max(np.abs(a_w - b_w)) < 1e-12


def test_routers_brute_force_on_tiny_expert_counts():
    rng = np.random.default_rng(5)
    for _ in range(50):
        E, k = 5, 3
        logits = np.round(rng.normal(size=E), 1)   # rounding makes ties likely
        best = max(itertools.permutations(range(E), k),
                   key=lambda p: (tuple(logits[list(p)]), tuple(-np.array(p))))
        # best = the lexicographically largest logits tuple, smaller indices on ties
        idx, w = O.router_topk_softmax(logits, k)
        assert idx.tolist() == list(best)
        e = np.exp(logits[list(best)] - logits[list(best)].max())
        assert np.allclose(w, e / e.sum(), rtol=0, atol=1e-15)


def test_gemma_router_matches_reference_fixture(golden_dir):
    fx = _golden(golden_dir, "gemma4_moe.json")["router"]
    idx, w = O.router_gemma(fx["hidden"], fx["projection"], fx["scale"], fx["perExpertScale"],
                            fx["topK"], 1e-6)
    assert idx.tolist() == fx["expectedIndices"]
    assert np.max(np.abs(w - np.array(fx["expectedWeights"]))) < 1e-12


def _rms(x, w, eps):
    s = np.mean(np.asarray(x) ** 2) + eps
    out = np.asarray(x) * s ** -0.5
    return out if w is None else out * np.asarray(w)


def test_gemma_moe_branch_inside_the_reference_layer_fixture(golden_dir):
    """The reference's whole Gemma layer (gemma4_operators.json["layer"]) with its MoE branch
    computed by the oracle. With one cached position, attention returns the value vector, so
    the rest of the layer is a few numpy lines (Gemma4ReferenceLayer.swift:141-215)."""
    f = _golden(golden_dir, "gemma4_moe.json")["layer"]
    w, eps = f["weights"], f["eps"]
    H, M, E, K = f["hiddenSize"], f["moeIntermediateSize"], f["expertCount"], f["topK"]
    mv = lambda m, v: np.asarray(m) @ np.asarray(v)
    hidden = np.array(f["input"])
    normed = _rms(hidden, w["input_layernorm"], eps)
    value = _rms(mv(w["v_proj"], normed), None, eps)
    attn = np.concatenate([value] * (f["heads"] // f["keyValueHeads"]))
    hidden = hidden + _rms(mv(w["o_proj"], attn), w["post_attention_layernorm"], eps)
    residual = hidden
    dense_in = _rms(hidden, w["pre_feedforward_layernorm"], eps)
    g, u = mv(w["gate_proj"], dense_in), mv(w["up_proj"], dense_in)
    gelu = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
    branch1 = _rms(mv(w["down_proj"], gelu * u), w["post_feedforward_layernorm_1"], eps)

    desc = F.MoEDesc(hidden=H, intermediate=M, experts=E, top_k=K, quant=O.QUANT_F64,
                     activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA, router_eps=eps)
    ex = f["experts"]
    blobs = O.pack_f64_experts(desc, [e["gate"] for e in ex], [e["up"] for e in ex],
                               [e["down"] for e in ex])
    expert_in = _rms(residual, w["pre_feedforward_layernorm_2"], eps)
    mixed, idx, wts, _ = O.moe_forward_f64(
        desc, blobs, expert_in, np.array(w["router_proj"]), x_router=residual,
        router_scale=w["router_scale"], router_expert_scale=w["router_per_expert_scale"])
    assert idx[0].tolist() == f["expectedIndices"]
    assert np.max(np.abs(wts[0] - np.array(f["expectedWeights"]))) < 1e-12
    branch2 = _rms(mixed[0], w["post_feedforward_layernorm_2"], eps)
    out = (residual + _rms(branch1 + branch2, w["post_feedforward_layernorm"], eps)) * w["layer_scalar"]
    exp = np.array(f["expected"])
    assert np.max(np.abs(out - exp)) / np.max(np.abs(exp)) < 1e-12


# ---- expert products and the whole layer, every format --------------------------------------

TINY = {
    "mxfp4": F.MoEDesc(hidden=128, intermediate=64, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                       activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    "mlx4": F.MoEDesc(hidden=128, intermediate=64, experts=8, top_k=3, quant=F.QUANT_MLX4,
                      activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                      shared_intermediate=128, group_size=64),
    "mlx8": F.MoEDesc(hidden=128, intermediate=64, experts=8, top_k=3, quant=F.QUANT_MLX8,
                      activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                      shared_intermediate=64, group_size=64),
    "bf16": F.MoEDesc(hidden=128, intermediate=64, experts=5, top_k=2, quant=F.QUANT_BF16,
                      activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA),
}


@pytest.mark.parametrize("name", list(TINY))
def test_layer_matches_dense_formulation(name):
    desc = TINY[name]
    layer = synth.make_layer(desc, seed=11)
    x = synth.make_tokens(desc.hidden, 5, seed=12)
    y, idx, w, _ = O.moe_forward(layer, x)
    ry, ridx, rw = D.moe_forward(layer, x)
    assert np.array_equal(idx, ridx)
    assert np.max(np.abs(w - rw)) < 1e-13
    assert np.max(np.abs(y - ry)) / np.max(np.abs(ry)) < 1e-12


def test_gemma_router_input_is_separate_from_expert_input():
    desc = TINY["bf16"]
    layer = synth.make_layer(desc, seed=3)
    x = synth.make_tokens(desc.hidden, 3, seed=4)
    xr = synth.make_tokens(desc.hidden, 3, seed=5)
    y, idx, w, _ = O.moe_forward(layer, x, x_router=xr)
    ry, ridx, rw = D.moe_forward(layer, x, x_router=xr)
    assert np.array_equal(idx, ridx) and np.max(np.abs(y - ry)) / np.max(np.abs(ry)) < 1e-12


def test_expert_bias_and_shared_gate_matter():
    d = TINY["mxfp4"]
    layer = synth.make_layer(d, seed=1)
    x = synth.make_tokens(d.hidden, 2, seed=2)
    with_bias = O.moe_forward(layer, x)[0]
    without = O.moe_forward(dict(layer, desc=d.replace(expert_bias=0)), x)[0]
    assert np.max(np.abs(with_bias - without)) > 1e-3
    q = TINY["mlx4"]
    layer = synth.make_layer(q, seed=1)
    y_shared = O.moe_forward(layer, x[:, :q.hidden])[0]
    y_plain = O.moe_forward(dict(layer, desc=q.replace(shared_intermediate=0)), x[:, :q.hidden])[0]
    assert np.max(np.abs(y_shared - y_plain)) > 1e-3


def test_full_size_expert_matches_dense_formulation():
    """One GPT-OSS-20B-shaped expert at its real size through both formulations."""
    d = F.GPT_OSS_20B.replace(experts=1)
    layer = synth.make_layer(d, seed=7)
    x = D.bf16(synth.make_tokens(d.hidden, 1, seed=8))[0]
    got = O.expert_ffn(d, layer["experts"][0], x)
    ref = D.expert_ffn(d, layer["experts"][0], x)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-12


# ---- decode attention with sinks --------------------------------------------------------------

@pytest.mark.parametrize("key", ["sdpa_full", "sdpa_sliding"])
def test_attention_decode_matches_reference_sdpa_fixture(golden_dir, key):
    """reference_ops.json sdpa fixtures (gen_reference_fixtures.py:100-128): every query row t
    is one decode step over the keys its causal (and sliding) mask leaves visible."""
    f = _golden(golden_dir, "reference_ops_attention.json")[key]
    kv, m, d, W = f["kv_heads"], f["q_mult"], f["head_dim"], f["sliding_window"]
    Q, K, V = np.array(f["q"]), np.array(f["k"]), np.array(f["v"])
    for t in range(f["tokens"]):
        first = max(0, t - W + 1) if W > 0 else 0
        out = O.attention_decode(Q[t].reshape(kv * m, d), K, V, f["sinks"], kv, t - first + 1,
                                 first, 0, f["sm_scale"])
        np.testing.assert_allclose(out.reshape(-1), f["expected"][t], rtol=0, atol=1e-12)


def test_attention_decode_closed_forms():
    rng = np.random.default_rng(5)
    qh, kv, d, n = 6, 2, 16, 9
    q = rng.standard_normal((qh, d))
    k = rng.standard_normal((n, kv, d))
    v = rng.standard_normal((n, kv, d))
    # A sink of -inf is plain softmax attention.
    out = O.attention_decode(q, k, v, np.full(qh, -np.inf), kv, n)
    for h in range(qh):
        g = h // (qh // kv)
        lg = k[:, g, :] @ q[h] / np.sqrt(d)
        w = np.exp(lg - lg.max()); w /= w.sum()
        np.testing.assert_allclose(out[h], w @ v[:, g, :], rtol=1e-12, atol=1e-12)
    # One key and a sink far below it: the value row itself.
    out1 = O.attention_decode(q, k, v, np.full(qh, -1e3), kv, 1, start_position=4)
    for h in range(qh):
        np.testing.assert_allclose(out1[h], v[4, h // 3], rtol=1e-12)
    # A ring of R rows holding positions p at row p % R equals the linear history.
    R, start = 5, 7
    ring_k, ring_v = np.zeros((R, kv, d)), np.zeros((R, kv, d))
    lin_k, lin_v = rng.standard_normal((start + R, kv, d)), rng.standard_normal((start + R, kv, d))
    for p in range(start, start + R):
        ring_k[p % R], ring_v[p % R] = lin_k[p], lin_v[p]
    sinks = rng.standard_normal(qh)
    a = O.attention_decode(q, ring_k, ring_v, sinks, kv, R, start, R)
    b = O.attention_decode(q, lin_k, lin_v, sinks, kv, R, start, 0)
    np.testing.assert_allclose(a, b, rtol=0, atol=0)
