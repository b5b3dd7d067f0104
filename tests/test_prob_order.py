"""Selection by probability at fp64 exp underflow (SOFTMAX_TOPK_RENORM and GEMMA routers).

The reference ranks these routers' experts by fp64 probability exp(l − max) / Σ with ties to
the smaller index (QwenReferenceOps.swift:164-173, Gemma4ReferenceOps.swift:146-149). When
fewer than K experts lie within ≈ 745 of the largest logit, every other expert's probability
is exactly 0 (exp of anything below −745.14 is 0 in fp64, whatever the libm), so the reference
takes the remaining ranks by increasing index, not by logit. The layers below put 5 experts
(non-zero class) within 400 of the maximum and the rest more than 850 below it; K = 8.

Bars: top-k indices bit-exact with the oracle; weights within 1e-6; layer outputs within
rel-L2 1e-3; the T-token layer call equal to one-token calls bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O

STRONG = [5, 17, 40]      # largest logits
MIDDLE = [1, 33]          # within 400 of the maximum: non-zero probability
# zero class: everything else; the reference fills ranks 5..7 with experts 0, 2, 3


def _row_level(e, strong, middle, low):
    return strong if e in STRONG else middle if e in MIDDLE else low


def _tokens(H, T, seed):
    """x ≈ 1 + 0.05·N(0, 1) (bf16), so a row of constant level a has logit ≈ a·Σx."""
    n = synth.normal(seed, "po_x", T * H)
    return synth.f32_to_bf16((1.0 + 0.05 * n).astype(np.float32)).reshape(T, H)


def make_layer(desc, mlx_bits=0, seed=71):
    """A layer whose router puts STRONG and MIDDLE far above the rest (see module doc)."""
    H, E = desc.hidden, desc.experts
    layer = synth.make_layer(desc, seed=seed, router_bits=mlx_bits)
    noise = synth.normal(seed, "po_noise", E * H).reshape(E, H)
    if desc.router == F.ROUTER_GEMMA:
        # logit ≈ a·√H on unit-rms inputs (unit router scales): H = 512 → 22.6·a
        lv = np.array([_row_level(e, 20.0, 5.0, -20.0) for e in range(E)])
        W = lv[:, None] + 0.2 * noise
        layer["router_weight"] = synth.f32_to_bf16(W.astype(np.float32))
    elif mlx_bits:
        # dequantised row = q·1e-4 + a (group bias a): level a plus codes as small noise
        lv = np.array([_row_level(e, 0.5, -0.2, -1.5) for e in range(E)])
        ng = H // 64
        layer["router_scales"] = synth.f32_to_bf16(np.full((E, ng), 1e-4, np.float32))
        layer["router_biases"] = synth.f32_to_bf16(
            (lv[:, None] + 0.01 * noise[:, :ng]).astype(np.float32))
    else:
        lv = np.array([_row_level(e, 0.5, -0.2, -1.5) for e in range(E)])
        W = lv[:, None] + 0.01 * noise
        layer["router_weight"] = synth.f32_to_bf16(W.astype(np.float32))
    return layer


DESCS = {
    "qwen-e64": F.MoEDesc(hidden=512, intermediate=128, experts=64, top_k=8, quant=F.QUANT_MLX4,
                          activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                          shared_intermediate=128, group_size=64),
    "qwen-e256": F.MoEDesc(hidden=512, intermediate=128, experts=256, top_k=8, quant=F.QUANT_MLX4,
                           activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                           shared_intermediate=128, group_size=64),
    "mxfp4-renorm": F.MoEDesc(hidden=512, intermediate=256, experts=64, top_k=8,
                              quant=F.QUANT_MXFP4, activation=F.ACT_SWIGLU_OAI,
                              router=F.ROUTER_SOFTMAX_TOPK_RENORM, expert_bias=0),
    "gemma-e128": F.MoEDesc(hidden=512, intermediate=128, experts=128, top_k=8,
                            quant=F.QUANT_BF16, activation=F.ACT_GELU_TANH,
                            router=F.ROUTER_GEMMA, router_eps=1e-6),
}
CASES = [("qwen-e64", 0), ("qwen-e256", 0), ("qwen-e64", 8), ("qwen-e256", 8),
         ("mxfp4-renorm", 0), ("gemma-e128", 0)]


def _expected(E):
    zero = [e for e in range(E) if e not in STRONG + MIDDLE]
    return zero[:3]


# ---- the oracle, pinned by mathematics --------------------------------------------------------

def test_oracle_router_takes_zero_probabilities_by_index():
    """Logits built directly: 5 finite-probability experts, the rest 1000 below (exp = 0 in
    every libm). The oracle's Qwen router must rank the 5 by logit, then 0, 2, 3."""
    E = 64
    lg = -1000.0 - 3.0 * synth.uniform(3, "po_lg", E)          # zero class, distinct logits
    lg[STRONG] = [10.0, 9.5, 11.0]
    lg[MIDDLE] = [-300.0, -200.0]
    idx, w = O.router_softmax_topk_renorm(lg, 8)
    assert list(idx) == [40, 5, 17, 33, 1, 0, 2, 3]
    assert np.all(w[5:] == 0.0)
    assert abs(np.sum(w) - 1.0) < 1e-15
    # the logit order (GPT-OSS's convention) would take the largest zero-class logits instead
    idx2, _ = O.router_topk_softmax(lg, 8)
    assert list(idx2[:5]) == [40, 5, 17, 33, 1] and list(idx2[5:]) != [0, 2, 3]


def test_oracle_gemma_router_takes_zero_probabilities_by_index():
    H, E = 64, 16
    hidden = np.ones(H)
    proj = np.full((E, H), -80.0) + 0.01 * synth.normal(4, "po_proj", E * H).reshape(E, H)
    proj[3] = 80.0
    proj[9] = 30.0
    idx, w = O.router_gemma(hidden, proj, np.ones(H), np.ones(E), 4, 1e-6)
    assert list(idx) == [3, 9, 0, 1]
    assert np.all(w[2:] == 0.0)


@pytest.mark.parametrize("name,bits", CASES)
def test_oracle_layers_have_the_intended_logits(name, bits):
    desc = DESCS[name]
    layer = make_layer(desc, bits)
    x = _tokens(desc.hidden, 3, 72)
    lg = O.router_logits(desc, layer, x)
    for t in range(3):
        top = lg[t].max()
        nz = [e for e in range(desc.experts) if lg[t, e] - top > -745.2]
        assert sorted(nz) == sorted(STRONG + MIDDLE), (t, nz)
        assert np.all(lg[t, [e for e in range(desc.experts) if e not in nz]] - top < -850)
        assert np.all(lg[t, nz] - top > -400)
    _, idx, w, _ = O.moe_forward(layer, x)
    for t in range(3):
        assert list(idx[t, 5:]) == _expected(desc.experts)
        assert np.all(w[t, 5:] == 0.0)


# ---- the GPU against the oracle --------------------------------------------------------------

def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


@pytest.mark.gpu
@pytest.mark.parametrize("name,bits", CASES)
def test_gpu_router_topk_zero_probabilities(name, bits):
    import torch
    from hydra_amd._lib import check, desc_c, lib
    from hydra_amd.layer import Context, MoELayer, to_device
    desc = DESCS[name]
    print(f"[gpu] prob-order router {name} bits={bits}", flush=True)
    ctx = Context(0)
    try:
        layer = make_layer(desc, bits)
        L = MoELayer(layer, ctx)
        d = desc_c(desc)
        x_all = _tokens(desc.hidden, 48, 73)
        _, ridx, rw, _ = O.moe_forward(layer, x_all)
        # one-token, small-batch, screened (T > 16) and one-wave-per-token (T ≥ 1024; the 48
        # rows repeated) selection
        for T in (1, 8, 48, 1025):
            x = to_device(np.resize(x_all, (T, desc.hidden)), "cuda:0")
            idx = torch.full((T, 8), -1, dtype=torch.int32, device="cuda:0")
            w = torch.empty((T, 8), dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            check(lib().hh_router_topk(ctx.handle, C.byref(d), C.byref(L._weights_c), _p(x), T,
                                       None, _p(idx), _p(w), None))
            ctx.synchronize()
            got = idx.cpu().numpy()
            ri, rwt = np.resize(ridx, (T, 8)), np.resize(rw, (T, 8))
            assert np.array_equal(got, ri), (T, got[0], ri[0])
            assert np.max(np.abs(w.cpu().numpy() - rwt)) < 1e-6
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,bits", CASES)
def test_gpu_layer_zero_probabilities(name, bits):
    from hydra_amd.layer import Context, MoELayer
    desc = DESCS[name]
    print(f"[gpu] prob-order layer {name} bits={bits}", flush=True)
    ctx = Context(0)
    try:
        layer = make_layer(desc, bits)
        L = MoELayer(layer, ctx)
        x_all = _tokens(desc.hidden, 48, 74)
        ry, ridx, rw, _ = O.moe_forward(layer, x_all)
        for T in (1, 5, 48):      # decode selection inside the gate-up kernel; prefill routing
            y, idx, w = L.forward(x_all[:T])
            assert np.array_equal(idx.cpu().numpy(), ridx[:T]), T
            assert np.max(np.abs(w.cpu().numpy() - rw[:T])) < 1e-6
            yy = y.cpu().numpy().astype(np.float64)
            rel = np.linalg.norm(yy - ry[:T]) / np.linalg.norm(ry[:T])
            assert rel < 1e-3, (T, rel)
            if T == 5:
                for t in range(T):
                    y1 = L.forward(x_all[t:t + 1])[0].cpu().numpy()[0]
                    assert np.array_equal(y1.view(np.uint32), y.cpu().numpy()[t].view(np.uint32))
    finally:
        ctx.close()
