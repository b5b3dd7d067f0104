"""GPU parity: the HIP path against the fp64 oracle and against itself.

Bars: dequantisation and top-k indices bit-exact; layer output
within rel-L2 1e-3 of the oracle (fp32 accumulation); a T-token call bit-identical to T
one-token calls. Every test calls the library through its C ABI.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3          # layer output tolerance (north_star)


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    return torch


@pytest.fixture(scope="module")
def ctx(torch_dev):
    from hydra_amd.layer import Context
    c = Context(0)
    yield c
    c.close()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def dev(torch, a):
    """Host array → device tensor, with torch's copy finished before the library's stream
    (a different stream) reads it."""
    from hydra_amd.layer import to_device
    t = to_device(a, "cuda:0")
    torch.cuda.synchronize()
    return t


def _p(t):
    return C.c_void_p(t.data_ptr())


# ---- dequantisation -------------------------------------------------------------------------

def test_mxfp4_dequant_matches_reference_golden(torch_dev, ctx, golden_dir):
    from hydra_amd._lib import check, lib
    torch = torch_dev
    say("mxfp4 dequant golden")
    packed = np.fromfile(os.path.join(golden_dir, "mxfp4_packed.bin"), np.uint8)
    scales = np.fromfile(os.path.join(golden_dir, "mxfp4_scales.bin"), np.uint8)
    expected = np.fromfile(os.path.join(golden_dir, "mxfp4_expected.f32"), np.float32)
    b, s = dev(torch, packed), dev(torch, scales)
    out = torch.empty(expected.size, dtype=torch.float32, device="cuda:0")
    check(lib().hh_mxfp4_dequant(ctx.handle, _p(b), _p(s), scales.size, _p(out)))
    ctx.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_mxfp4_dequant_exhaustive_bytes_and_scales(torch_dev, ctx):
    """Every packed byte under every e8m0 scale byte, bit for bit against the oracle."""
    from hydra_amd._lib import check, lib
    torch = torch_dev
    say("mxfp4 dequant exhaustive")
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)          # 256 blocks of 16 → 16 per scale
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    exp = O.mxfp4_decode(packed, scales)
    b, s = dev(torch, packed), dev(torch, scales)
    out = torch.empty(exp.size, dtype=torch.float32, device="cuda:0")
    check(lib().hh_mxfp4_dequant(ctx.handle, _p(b), _p(s), scales.size, _p(out)))
    ctx.synchronize()
    got = out.cpu().numpy()
    both_nan = np.isnan(got) & np.isnan(exp)
    same = (got.view(np.uint32) == exp.view(np.uint32)) | both_nan
    bad = np.nonzero(~same)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first scale bytes {sorted(set(scales[bad // 32][:20].tolist()))}"


@pytest.mark.parametrize("bits", [4, 8])
def test_mlx_dequant_bit_exact(torch_dev, ctx, bits):
    from hydra_amd._lib import check, lib
    torch = torch_dev
    say(f"mlx{bits} dequant")
    rows, cols, group = 37, 512, 64
    words = synth.u64(5, "w", rows * cols * bits // 64).view(np.uint32)
    sc = synth.bf16_normal(5, "s", rows * cols // group, 0.01, 0.002)
    bi = synth.f32_to_bf16(-7.5 * synth.bf16_to_f32(sc))
    exp = np.stack([O.mlx_dequant(words.reshape(rows, -1)[r], synth.bf16_to_f32(sc.reshape(rows, -1)[r]),
                                  synth.bf16_to_f32(bi.reshape(rows, -1)[r]), cols, bits, group)
                    for r in range(rows)]).astype(np.float32)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda:0")
    dw, ds, db = dev(torch, words), dev(torch, sc), dev(torch, bi)   # kept alive for the call
    check(lib().hh_mlx_dequant(ctx.handle, _p(dw), _p(ds), _p(db), rows, cols, bits, group, _p(out)))
    ctx.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32))


# ---- activation -----------------------------------------------------------------------------

@pytest.mark.parametrize("act", [F.ACT_SWIGLU_OAI, F.ACT_SILU, F.ACT_GELU_TANH])
def test_activation_matches_oracle(torch_dev, ctx, act):
    from hydra_amd._lib import check, desc_c, lib
    torch = torch_dev
    say(f"activation {act}")
    rng = np.random.default_rng(act)
    g = np.concatenate([rng.normal(0, 3, 5000), [-20, -7.5, 0, 6.99, 7, 7.01, 30, 12, -12]]).astype(np.float32)
    u = np.concatenate([rng.normal(0, 3, 5000), [1, -8, 2, 7.5, -7.5, 0.5, 8, 3, 3]]).astype(np.float32)
    d = desc_c(F.GPT_OSS_20B.replace(activation=act))
    out = torch.empty(g.size, dtype=torch.float32, device="cuda:0")
    dg, du = dev(torch, g), dev(torch, u)   # kept alive for the call
    check(lib().hh_activation(ctx.handle, C.byref(d), _p(dg), _p(du), g.size, _p(out)))
    ctx.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    if act == F.ACT_SWIGLU_OAI:
        ref = np.array([O.swiglu([a, b])[0] for a, b in zip(g, u)])
    elif act == F.ACT_SILU:
        ref = np.array([O.silu(a) * b for a, b in zip(g, u)])
    else:
        ref = np.array([O.gelu_tanh(a) * b for a, b in zip(g, u)])
    # fp32 bound: 2e-6 relative, plus the absolute rounding of 1 + tanh(·) (or of the sigmoid)
    # near saturation, where the value is tiny and scales with |g|·|u|.
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    bound = 2e-6 * np.abs(ref) + 1e-7 * (np.abs(g64) + 1) * (np.abs(u64) + 1)
    assert np.all(np.abs(got - ref) <= bound)


# ---- router ---------------------------------------------------------------------------------

ROUTER_CASES = {
    "gpt-oss-20b": (F.GPT_OSS_20B, None),
    "gpt-oss-120b-zipf": (F.GPT_OSS_120B, 1.1),
    "qwen-q4": (F.QWEN_35B_A3B_Q4, None),
    "gemma": (F.GEMMA_BF16, None),
    # 19 expert tiles, the last one partial: at 1030 tokens four tiles per screening workgroup,
    # its last group ragged; H past a 512-column slice
    "e300": (F.MoEDesc(hidden=640, intermediate=64, experts=300, top_k=6, quant=F.QUANT_MXFP4,
                       activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                       expert_bias=1), None),
}


@pytest.mark.parametrize("name", list(ROUTER_CASES))
@pytest.mark.parametrize("T", [5, 96, 1030])   # 1030: the one-wave-per-token selection, a ragged last workgroup
def test_router_indices_bit_exact(torch_dev, ctx, name, T):
    from hydra_amd._lib import check, desc_c, lib
    from hydra_amd.layer import MoELayer
    torch = torch_dev
    desc, zipf = ROUTER_CASES[name]
    say(f"router {name} T={T}")
    small = desc.replace(intermediate=64, shared_intermediate=64 if desc.shared_intermediate else 0)
    layer = synth.make_layer(small, seed=21, zipf=zipf)
    x = synth.make_tokens(desc.hidden, T, seed=22)
    L = MoELayer(layer, ctx)
    d = desc_c(small)
    idx = torch.empty((T, desc.top_k), dtype=torch.int32, device="cuda:0")
    w = torch.empty((T, desc.top_k), dtype=torch.float32, device="cuda:0")
    lg = torch.empty((T, desc.top_k), dtype=torch.float64, device="cuda:0")
    xd = dev(torch, x)
    torch.cuda.synchronize()
    check(lib().hh_router_topk(ctx.handle, C.byref(d), C.byref(L._weights_c), _p(xd), T, _p(lg),
                               _p(idx), _p(w), None))
    ctx.synchronize()
    ref_logits = O.router_logits(small, layer, x)
    got_idx = idx.cpu().numpy()
    sel = np.take_along_axis(ref_logits, got_idx.astype(np.int64), axis=1)
    assert np.max(np.abs(lg.cpu().numpy() - sel)) < 1e-9
    ridx = np.empty((T, desc.top_k), np.int64)
    rw = np.empty((T, desc.top_k))
    for t in range(T):
        if small.router == F.ROUTER_TOPK_SOFTMAX:
            i, ww = O.router_topk_softmax(ref_logits[t], desc.top_k)
        else:
            i, ww = O.router_softmax_topk_renorm(ref_logits[t], desc.top_k)
            if small.router == F.ROUTER_GEMMA:
                ww = ww * synth.bf16_to_f32(layer["router_expert_scale"])[i]
        ridx[t], rw[t] = i, ww
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.max(np.abs(w.cpu().numpy() - rw)) < 1e-6


def test_permute_is_stable_grouping(torch_dev, ctx):
    from hydra_amd._lib import check, lib
    torch = torch_dev
    say("permute")
    rng = np.random.default_rng(9)
    # one workgroup below 1024 assignments; from 1024 on the multi-block dispatch (exactly 1024 and
    # one below it, 17 blocks with a partial last one, 64 blocks with empty trailing ones, 512
    # experts, a skewed load)
    for T, K, E, skew in [(1, 4, 32, 0), (7, 2, 5, 0), (300, 8, 256, 0), (2048, 4, 128, 0),
                          (1000, 8, 512, 0), (256, 4, 7, 0), (341, 3, 9, 0), (1031, 4, 7, 0),
                          (8193, 2, 64, 0), (4096, 2, 300, 1.1)]:
        p = None
        if skew:
            p = 1.0 / np.arange(1, E + 1) ** skew
            p /= p.sum()
        topk = np.stack([rng.choice(E, K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
        seg = torch.empty(E + 1, dtype=torch.int32, device="cuda:0")
        order = torch.empty(T * K, dtype=torch.int32, device="cuda:0")
        ti = dev(torch, topk)
        torch.cuda.synchronize()
        check(lib().hh_permute(ctx.handle, _p(ti), T, K, E, _p(seg), _p(order)))
        ctx.synchronize()
        flat = topk.ravel()
        exp_order = np.argsort(flat, kind="stable")
        exp_seg = np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))])
        assert np.array_equal(order.cpu().numpy(), exp_order), (T, K, E)
        assert np.array_equal(seg.cpu().numpy(), exp_seg), (T, K, E)


# ---- the layer ------------------------------------------------------------------------------

TINY = {
    "mxfp4": F.MoEDesc(hidden=256, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                       activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    "mxfp4-ragged": F.MoEDesc(hidden=2880, intermediate=320, experts=5, top_k=3,
                              quant=F.QUANT_MXFP4, activation=F.ACT_SWIGLU_OAI,
                              router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    "mxfp4-narrow": F.MoEDesc(hidden=192, intermediate=64, experts=4, top_k=2,
                              quant=F.QUANT_MXFP4, activation=F.ACT_SWIGLU_OAI,
                              router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    # Rows of ≥ 8 chunks in both products: the persistent LDS-ring prefill kernel.
    "mxfp4-wide": F.MoEDesc(hidden=1024, intermediate=1024, experts=8, top_k=4,
                            quant=F.QUANT_MXFP4, activation=F.ACT_SWIGLU_OAI,
                            router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    "mlx4": F.MoEDesc(hidden=256, intermediate=128, experts=8, top_k=3, quant=F.QUANT_MLX4,
                      activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                      shared_intermediate=192, group_size=64),
    "mlx8": F.MoEDesc(hidden=256, intermediate=192, experts=8, top_k=3, quant=F.QUANT_MLX8,
                      activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                      shared_intermediate=64, group_size=64),
    "bf16": F.MoEDesc(hidden=320, intermediate=192, experts=5, top_k=2, quant=F.QUANT_BF16,
                      activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA),
    # MLX decode stages each item's group scales and biases in LDS when the rows fit (gate-up
    # K ≤ 4096; down K ≤ 4096 with ≤ 4 slots, ≤ 2048 with more) and loads them per chunk
    # otherwise: a gate-up row of 65 chunks; down rows of 40 chunks with 3 slots (staged, 16-byte
    # vectors) and with 9 slots (per chunk).
    "mlx4-wide": F.MoEDesc(hidden=4160, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MLX4,
                           activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM, group_size=64),
    "mlx4-deep": F.MoEDesc(hidden=512, intermediate=2560, experts=6, top_k=3, quant=F.QUANT_MLX4,
                           activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM, group_size=64),
    "mlx8-long": F.MoEDesc(hidden=256, intermediate=2560, experts=10, top_k=8, quant=F.QUANT_MLX8,
                           activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                           shared_intermediate=128, group_size=64),
}


@pytest.mark.parametrize("name", list(TINY))
@pytest.mark.parametrize("T", [1, 2, 5, 70])   # T = 1 and 2: the decode selection split over waves
def test_layer_matches_oracle_small(torch_dev, ctx, name, T):
    from hydra_amd.layer import MoELayer
    desc = TINY[name]
    say(f"layer {name} T={T}")
    layer = synth.make_layer(desc, seed=31)
    x = synth.make_tokens(desc.hidden, T, seed=32)
    y, idx, w = MoELayer(layer, ctx).forward(x)
    ry, ridx, rw, _ = O.moe_forward(layer, x)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.max(np.abs(w.cpu().numpy() - rw)) < 1e-6
    assert rel_l2(y.cpu().numpy(), ry) < REL_L2


@pytest.mark.parametrize("name", list(TINY))
def test_prefill_equals_token_by_token_bit_for_bit(torch_dev, ctx, name):
    from hydra_amd.layer import MoELayer
    desc = TINY[name]
    say(f"prefill==decode {name}")
    layer = synth.make_layer(desc, seed=41)
    T = 80                                   # crosses the 64-token tile switch
    x = synth.make_tokens(desc.hidden, T, seed=42)
    L = MoELayer(layer, ctx)
    y_all, idx_all, w_all = L.forward(x)
    y_all = y_all.cpu().numpy()
    for t in range(T):
        y1, i1, w1 = L.forward(x[t:t + 1])
        assert np.array_equal(i1.cpu().numpy()[0], idx_all.cpu().numpy()[t])
        assert np.array_equal(y1.cpu().numpy()[0].view(np.uint32), y_all[t].view(np.uint32)), t
    # chunked prefill: uneven chunks give the same bits too
    parts = [L.forward(x[a:b])[0].cpu().numpy() for a, b in [(0, 3), (3, 67), (67, 80)]]
    assert np.array_equal(np.concatenate(parts).view(np.uint32), y_all.view(np.uint32))


@pytest.mark.parametrize("name", ["mxfp4", "mlx4", "bf16"])
def test_large_batch_equals_token_by_token_bit_for_bit(torch_dev, ctx, name):
    """From 1024 tokens the selection takes one wave per token and the grouping the multi-block
    dispatch: a 1100-token batch's outputs, top-k and weights equal single-token calls bit for bit
    (sampled tokens, the last workgroup's ragged ones included), and so do uneven chunks."""
    from hydra_amd.layer import MoELayer
    desc = TINY[name]
    say(f"large batch == decode {name}")
    layer = synth.make_layer(desc, seed=43)
    T = 1100
    x = synth.make_tokens(desc.hidden, T, seed=44)
    L = MoELayer(layer, ctx)
    y_all, idx_all, w_all = (v.cpu().numpy() for v in L.forward(x))
    for t in [0, 1, 511, 1023, 1024, 1097, 1098, 1099]:
        y1, i1, w1 = (v.cpu().numpy() for v in L.forward(x[t:t + 1]))
        assert np.array_equal(i1[0], idx_all[t]), t
        assert np.array_equal(w1[0].view(np.uint32), w_all[t].view(np.uint32)), t
        assert np.array_equal(y1[0].view(np.uint32), y_all[t].view(np.uint32)), t
    parts = [L.forward(x[a:b])[0].cpu().numpy() for a, b in [(0, 17), (17, 1041), (1041, 1100)]]
    assert np.array_equal(np.concatenate(parts).view(np.uint32), y_all.view(np.uint32))


WIDE = {
    "mxfp4-wide": TINY["mxfp4-wide"],
    # Gate-up rows of ≥ 12 chunks: the register-ring gate-up kernel (64-token items at T=300: the
    # experts average 150 tokens).
    "mxfp4-deep": F.MoEDesc(hidden=2048, intermediate=1024, experts=8, top_k=4, quant=F.QUANT_MXFP4,
                            activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    # Many experts (≈ 19 tokens each at T=300): 32-token items, the register-ring gate-up kernel's
    # 32-token tiles and the 128-row down tiles.
    "mxfp4-many": F.MoEDesc(hidden=2048, intermediate=1024, experts=64, top_k=4, quant=F.QUANT_MXFP4,
                            activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
}


@pytest.mark.parametrize("name", list(WIDE))
def test_wide_prefill_tiles_equal_token_by_token_bit_for_bit(torch_dev, ctx, name):
    """Large MXFP4 batches take the 256-row prefill tiles (32- or 64-token items): still the
    decode bits."""
    from hydra_amd.layer import MoELayer
    desc = WIDE[name]
    say(f"prefill==decode {name} T=300 (256-row tiles)")
    layer = synth.make_layer(desc, seed=43)
    T = 300                                  # 1200 assignments: ≥ 64 work items of 32 tokens
    x = synth.make_tokens(desc.hidden, T, seed=44)
    L = MoELayer(layer, ctx)
    y_all, idx_all, _ = L.forward(x)
    y_all = y_all.cpu().numpy()
    ry, ridx, _, _ = O.moe_forward(layer, x[:8])
    assert np.array_equal(idx_all.cpu().numpy()[:8], ridx)
    assert rel_l2(y_all[:8], ry) < REL_L2
    for t in range(0, T, 7):
        y1 = L.forward(x[t:t + 1])[0].cpu().numpy()[0]
        assert np.array_equal(y1.view(np.uint32), y_all[t].view(np.uint32)), t


def test_layer_is_deterministic_and_order_independent(torch_dev, ctx):
    from hydra_amd.layer import MoELayer
    desc = TINY["mxfp4"]
    say("determinism")
    layer = synth.make_layer(desc, seed=51)
    x = synth.make_tokens(desc.hidden, 100, seed=52)
    L = MoELayer(layer, ctx)
    a = L.forward(x)[0].cpu().numpy()
    b = L.forward(x)[0].cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    perm = np.random.default_rng(0).permutation(100)
    c = L.forward(x[perm])[0].cpu().numpy()
    assert np.array_equal(c.view(np.uint32), a[perm].view(np.uint32))


# ---- real shapes ----------------------------------------------------------------------------

FUSED_CASES = {
    "mxfp4": (TINY["mxfp4"], [5, 1, 8, 3, 16, 13, 5, 2]),
    "mxfp4-ragged": (TINY["mxfp4-ragged"], [3, 16, 1, 7]),
    "gpt-oss-20b": (F.GPT_OSS_20B, [1, 4, 16, 2, 8, 1]),
    "gpt-oss-120b": (F.GPT_OSS_120B, [1, 8, 3]),
    # the shared expert's gate row in the MXFP4 router workgroups; H past a 512-column slice
    "mxfp4-shared": (F.MoEDesc(hidden=640, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                               activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                               shared_intermediate=128, expert_bias=1), [1, 2, 5, 1]),
    # the BF16 / MLX decode gate-up kernel with its fused routers (bf16 GEMMA, 8-bit MLX)
    "gemma-bf16": (F.GEMMA_BF16, [1, 2, 5, 1]),
    "qwen-mlx4-router8": (F.QWEN_35B_A3B_Q4, [1, 2, 3, 1], 8),
    "qwen-mlx8-bf16router": (F.QWEN_35B_A3B_Q8, [2, 1]),
}


@pytest.mark.parametrize("name", list(FUSED_CASES))
def test_fused_decode_equals_three_launch_decode(torch_dev, ctx, name):
    """The two-launch decode (router workgroups inside the gate-up launch, hh_ctx_decode_fused
    2, the default) and the one-launch decode (1) against the three-launch decode (0), bit for
    bit (outputs, top-k indices and weights), over a sequence of batch sizes. The paths
    alternate on one context with new tokens at every step, so a fused call that read data left
    in the scratch or the flags by an earlier call (another batch size, other tokens) would
    show."""
    from hydra_amd.layer import MoELayer
    desc, Ts, *rb = FUSED_CASES[name]
    say(f"fused decode {name}")
    L = MoELayer(synth.make_layer(desc, seed=51, router_bits=rb[0] if rb else 0), ctx)
    try:
        for i, T in enumerate(Ts):
            x = synth.make_tokens(desc.hidden, T, seed=60 + i)
            ctx.decode_fused(0)
            ya, ia, wa = (v.cpu().numpy() for v in L.forward(x))
            for mode in (2, 1, -1):
                ctx.decode_fused(mode)
                yb, ib, wb = (v.cpu().numpy() for v in L.forward(x))
                assert np.array_equal(ia, ib), (name, T, mode)
                assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), (name, T, mode)
                assert not np.isnan(yb).any(), (name, T, mode)
                assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (name, T, mode)
    finally:
        ctx.decode_fused(-1)


FULL = {
    "gpt-oss-20b": (F.GPT_OSS_20B, None, [1, 2, 4, 8, 16]),
    "gpt-oss-120b-zipf": (F.GPT_OSS_120B, 1.1, [512, 2048]),
    "qwen-q4": (F.QWEN_35B_A3B_Q4, None, [1, 16, 1024]),
    "qwen-q8": (F.QWEN_35B_A3B_Q8, None, [1, 1024]),
    "gemma-bf16": (F.GEMMA_BF16, None, [1, 2048]),
}


def tile_edge_sample(idx, experts, T, seed=0):
    """At least 16 tokens (all of them when T < 16): the first and last token of the batch, a
    few random ones, and the tokens at the 32- and 64-token tile edges of the prefill work
    items (positions 0, 31, 32, 63, 64, 95, 96, 127, 128 and the last of an expert's segment in
    the stable (token, rank) order) of the busiest experts and of random ones."""
    if T <= 16:
        return list(range(T))
    rng = np.random.default_rng(T + seed)
    flat = idx.ravel()
    counts = np.bincount(flat, minlength=experts)
    picks = set([0, T - 1]) | set(rng.choice(T, 4, replace=False).tolist())
    busy = list(np.argsort(-counts, kind="stable")[:3])
    used = [e for e in range(experts) if counts[e] > 0]
    others = list(rng.choice(used, min(3, len(used)), replace=False))
    for e in busy + others:
        toks = np.nonzero(flat == e)[0] // idx.shape[1]     # stable (token, rank) order
        n = len(toks)
        for p in (0, 31, 32, 63, 64, 95, 96, 127, 128, n - 1):
            if 0 <= p < n:
                picks.add(int(toks[p]))
    while len(picks) < 16:
        picks.add(int(rng.integers(T)))
    return sorted(picks)


@pytest.mark.parametrize("name", list(FULL))
def test_full_size_layers_against_oracle_sample(torch_dev, ctx, name):
    """Each BASELINE configuration at its real shape: every token's top-k and a sample of
    tokens' outputs against the oracle; the whole batch against token-by-token decode."""
    from hydra_amd.layer import MoELayer
    torch = torch_dev
    desc, zipf, Ts = FULL[name]
    say(f"full {name}: building layer")
    layer = synth.make_layer(desc, seed=0, zipf=zipf)
    L = MoELayer(layer, ctx)
    for T in Ts:
        say(f"full {name} T={T}")
        x = synth.make_tokens(desc.hidden, T, seed=1)
        y, idx, w = L.forward(x)
        y = y.cpu().numpy()
        idx = idx.cpu().numpy()
        logits = O.router_logits(desc, layer, x)
        for t in range(T):
            if desc.router == F.ROUTER_TOPK_SOFTMAX:
                ri, _ = O.router_topk_softmax(logits[t], desc.top_k)
            else:
                ri, _ = O.router_softmax_topk_renorm(logits[t], desc.top_k)
            assert np.array_equal(idx[t], ri), t
        sample = tile_edge_sample(idx, desc.experts, T)
        ry, _, _, _ = O.moe_forward(layer, x[sample], nthreads=min(16, os.cpu_count() or 1))
        assert rel_l2(y[sample], ry) < REL_L2
        # the batch equals one-token calls, bit for bit, on a sample of tokens
        for t in sample:
            y1 = L.forward(x[t:t + 1])[0].cpu().numpy()[0]
            assert np.array_equal(y1.view(np.uint32), y[t].view(np.uint32)), (T, t)
        if zipf:
            counts = np.bincount(idx.ravel(), minlength=desc.experts)
            assert counts.max() > 8 * max(1, np.median(counts))   # the load really is skewed
    del L
    torch.cuda.empty_cache()


@pytest.mark.parametrize("router", [F.ROUTER_TOPK_SOFTMAX, F.ROUTER_SOFTMAX_TOPK_RENORM, F.ROUTER_GEMMA])
def test_router_near_ties_resolved_exactly(torch_dev, ctx, router):
    """Router rows that are exact duplicates (ties → smaller index) or differ by one ulp of a
    tiny element (logits that fp32 cannot separate but fp64 can)."""
    from hydra_amd._lib import check, desc_c, lib
    from hydra_amd.layer import MoELayer
    torch = torch_dev
    say(f"router near ties {router}")
    desc = F.MoEDesc(hidden=2880, intermediate=64, experts=32, top_k=4, quant=F.QUANT_MXFP4,
                     activation=F.ACT_SWIGLU_OAI, router=router, expert_bias=0)
    layer = synth.make_layer(desc, seed=61)
    W = layer["router_weight"].copy()
    W[:, 5] = synth.f32_to_bf16(np.float32(1e-7) * np.ones(32, np.float32))
    for a_, b_ in [(3, 4), (10, 11), (20, 21)]:
        W[b_] = W[a_]                         # exact duplicate
    for a_, b_ in [(7, 8), (14, 15), (25, 26)]:
        W[b_] = W[a_]
        W[b_, 5] = W[a_, 5] + 1               # one ulp of a 1e-7 weight
    # make the duplicated experts strong so they land in the top-k
    for e in [3, 4, 7, 8, 10, 11, 14, 15, 20, 21, 25, 26]:
        keep = W[e, 5]
        W[e] = synth.f32_to_bf16(synth.bf16_to_f32(W[e]) * np.float32(1.5))
        W[e, 5] = keep
    layer["router_weight"] = W
    x_all = synth.make_tokens(desc.hidden, 64, seed=62)
    L = MoELayer(layer, ctx)
    d = desc_c(desc)
    ref_all = O.router_logits(desc, layer, x_all)
    # the screened multi-workgroup path, the one-workgroup path and (1027 tokens: the rows
    # repeated) the one-wave-per-token selection
    for T in (64, 8, 1027):
        x = np.resize(x_all, (T, desc.hidden))
        idx = torch.empty((T, 4), dtype=torch.int32, device="cuda:0")
        w = torch.empty((T, 4), dtype=torch.float32, device="cuda:0")
        xd = dev(torch, x)
        check(lib().hh_router_topk(ctx.handle, C.byref(d), C.byref(L._weights_c), _p(xd), T,
                                   None, _p(idx), _p(w), None))
        ctx.synchronize()
        got = idx.cpu().numpy()
        for t in range(T):
            if router == F.ROUTER_TOPK_SOFTMAX:
                ri, _ = O.router_topk_softmax(ref_all[t % 64], 4)
            else:
                ri, _ = O.router_softmax_topk_renorm(ref_all[t % 64], 4)
            assert np.array_equal(got[t], ri), (T, t, got[t], ri)
