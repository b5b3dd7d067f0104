"""The MLX-affine router (Qwen's 8-bit mlp.gate and mlp.shared_expert_gate,
Qwen35MoeConfig.swift:340-342): the oracle pinned against an independent dense formulation,
then the GPU (hh_router_topk and the whole layer) against the oracle through the C ABI.

Bars: top-k indices bit-exact (ties to the smaller index); selected logits within 1e-12
relative of the fp64 oracle (both are fp64 sums of exact products); layer outputs within
rel-L2 1e-3; a T-token layer call equal to one-token calls bit for bit."""
import ctypes as C
import os

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O

QWEN_SMALL = F.MoEDesc(hidden=256, intermediate=128, experts=40, top_k=8, quant=F.QUANT_MLX4,
                       activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                       shared_intermediate=128, group_size=64)


def dense_router(words, scales, biases, bits):
    """Independent fp64 dequantisation: code j of a row sits at bit (j·bits) of the row's
    little-endian bit string (MLXAffine.unpack, low-order value first)."""
    rows = words.shape[0]
    raw = np.ascontiguousarray(words).view(np.uint8).reshape(rows, -1)
    if bits == 8:
        q = raw.astype(np.float64)
    else:
        q = np.stack([raw & 0xF, raw >> 4], axis=-1).reshape(rows, -1).astype(np.float64)
    s = np.repeat(synth.bf16_to_f32(scales).astype(np.float64), 64, axis=1)
    b = np.repeat(synth.bf16_to_f32(biases).astype(np.float64), 64, axis=1)
    return q * s + b


@pytest.mark.parametrize("bits", [4, 8])
def test_oracle_mlx_router_matches_dense_formulation(bits):
    layer = synth.make_layer(QWEN_SMALL, seed=7, router_bits=bits)
    x = synth.make_tokens(QWEN_SMALL.hidden, 6, seed=8)
    xd = synth.bf16_to_f32(x).astype(np.float64)
    Wd = dense_router(layer["router_words"], layer["router_scales"], layer["router_biases"], bits)
    lg = O.router_logits(QWEN_SMALL, layer, x)
    assert np.max(np.abs(lg - xd @ Wd.T)) <= 1e-12 * np.max(np.abs(lg))
    assert 0.5 < np.std(lg) < 2.0                 # logits ≈ N(0, 1) as generated
    _, idx, w, sw = O.moe_forward(layer, x)
    g = dense_router(layer["shared_gate_words"], layer["shared_gate_scales"],
                     layer["shared_gate_biases"], bits)[0]
    assert np.allclose(sw, 1 / (1 + np.exp(-(xd @ g))), rtol=1e-12, atol=0)
    for t in range(6):
        order = np.argsort(-lg[t], kind="stable")[:8]
        assert np.array_equal(idx[t], order)


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _tie_layer(bits):
    """Router rows duplicated exactly (ties → smaller index) and made strong enough to be
    selected."""
    layer = synth.make_layer(QWEN_SMALL, seed=9, router_bits=bits)
    for k in ("router_words", "router_scales", "router_biases"):
        a = layer[k].copy()
        for src, dst in [(3, 4), (10, 11), (20, 21)]:
            a[dst] = a[src]
        layer[k] = a
    sc = synth.bf16_to_f32(layer["router_scales"]).copy()
    bi = synth.bf16_to_f32(layer["router_biases"]).copy()
    for e in (3, 4, 10, 11, 20, 21):
        sc[e] *= 1.5
        bi[e] *= 1.5
    layer["router_scales"] = synth.f32_to_bf16(sc)
    layer["router_biases"] = synth.f32_to_bf16(bi)
    return layer


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_gpu_mlx_router_topk_exact(bits):
    import torch
    from hydra_amd._lib import check, desc_c, lib
    from hydra_amd.layer import Context, MoELayer, to_device
    print(f"[gpu] mlx router topk bits={bits}", flush=True)
    ctx = Context(0)
    try:
        layer = _tie_layer(bits)
        L = MoELayer(layer, ctx)
        d = desc_c(QWEN_SMALL)
        x_all = synth.make_tokens(QWEN_SMALL.hidden, 100, seed=10)
        ref = O.router_logits(QWEN_SMALL, layer, x_all)
        _, ridx_all, rw_all, rsw_all = O.moe_forward(layer, x_all)
        # the one-workgroup selection and the per-token selection (1029 tokens: the 100 rows
        # repeated; the multi-block dispatch)
        for T in (5, 100, 1029):
            x = to_device(np.resize(x_all, (T, QWEN_SMALL.hidden)), "cuda:0")
            ridx, rw, rsw = (np.resize(v, (T,) + v.shape[1:]) for v in (ridx_all, rw_all, rsw_all))
            rref = np.resize(ref, (T, ref.shape[1]))
            idx = torch.full((T, 8), -1, dtype=torch.int32, device="cuda:0")
            w = torch.empty((T, 8), dtype=torch.float32, device="cuda:0")
            lg = torch.empty((T, 8), dtype=torch.float64, device="cuda:0")
            sw = torch.empty((T,), dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            check(lib().hh_router_topk(ctx.handle, C.byref(d), C.byref(L._weights_c), _p(x), T,
                                       _p(lg), _p(idx), _p(w), _p(sw)))
            ctx.synchronize()
            got = idx.cpu().numpy()
            assert np.array_equal(got, ridx), T
            sel = np.take_along_axis(rref, got.astype(np.int64), axis=1)
            assert np.max(np.abs(lg.cpu().numpy() - sel)) <= 1e-12 * np.max(np.abs(sel))
            assert np.max(np.abs(w.cpu().numpy() - rw)) < 1e-6
            assert np.max(np.abs(sw.cpu().numpy() - rsw)) < 1e-6
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_gpu_qwen_layer_with_mlx_router(bits):
    """The Qwen-shaped layer (MLX-4 experts) with its router and shared
    gate in MLX-affine form, decode and prefill, against the oracle and token-by-token."""
    import torch
    from hydra_amd.layer import Context, MoELayer
    desc = F.QWEN_35B_A3B_Q4
    print(f"[gpu] qwen layer with mlx{bits} router", flush=True)
    ctx = Context(0)
    try:
        layer = synth.make_layer(desc, seed=0, router_bits=bits)
        L = MoELayer(layer, ctx)
        for T in (1, 7, 300):
            x = synth.make_tokens(desc.hidden, T, seed=1)
            y, idx, w = L.forward(x)
            y, idx = y.cpu().numpy(), idx.cpu().numpy()
            logits = O.router_logits(desc, layer, x)
            for t in range(T):
                ri, _ = O.router_softmax_topk_renorm(logits[t], desc.top_k)
                assert np.array_equal(idx[t], ri), (T, t)
            sample = sorted({0, T // 3, T - 1})
            ry, _, _, _ = O.moe_forward(layer, x[sample], nthreads=min(16, os.cpu_count() or 1))
            rel = np.linalg.norm(y[sample] - ry) / np.linalg.norm(ry)
            assert rel < 1e-3, (T, rel)
            for t in sample:
                y1 = L.forward(x[t:t + 1])[0].cpu().numpy()[0]
                assert np.array_equal(y1.view(np.uint32), y[t].view(np.uint32)), (T, t)
    finally:
        ctx.close()
