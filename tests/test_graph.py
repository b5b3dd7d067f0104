"""A layer stack recorded as one HIP graph (hh_ctx_capture_begin / _end, hh_graph_launch)
replays exactly what the eager calls compute.

Each replay follows eager work and host synchronisation on the same context and new inputs,
and is checked against eager results of the same inputs bit for bit.
"""
import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth

STACK = [
    F.MoEDesc(hidden=256, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
              activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    F.MoEDesc(hidden=256, intermediate=128, experts=8, top_k=3, quant=F.QUANT_MLX4,
              activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
              shared_intermediate=192, group_size=64),
    F.MoEDesc(hidden=320, intermediate=192, experts=5, top_k=2, quant=F.QUANT_BF16,
              activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA),
]


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 40])
def test_graph_replays_equal_eager_calls(T):
    import torch
    from hydra_amd.layer import Context, MoELayer, to_device
    print(f"[gpu] graph stack T={T}", flush=True)
    ctx = Context(0)
    try:
        layers = [MoELayer(synth.make_layer(d, seed=50 + i), ctx) for i, d in enumerate(STACK)]
        for d in STACK:
            ctx.reserve(d, T)
        dev = "cuda:0"
        xs = [torch.empty((T, d.hidden), dtype=torch.int16, device=dev) for d in STACK]
        ys = [torch.empty((T, d.hidden), dtype=torch.float32, device=dev) for d in STACK]
        ids = [torch.empty((T, d.top_k), dtype=torch.int32, device=dev) for d in STACK]
        ws = [torch.empty((T, d.top_k), dtype=torch.float32, device=dev) for d in STACK]
        torch.cuda.synchronize()
        before = ctx.dispatches
        graph = ctx.capture(lambda: [l.forward_into(x, y, i, w)
                                     for l, x, y, i, w in zip(layers, xs, ys, ids, ws)])
        assert ctx.dispatches == before            # recording runs nothing
        per_replay = None
        for rep in range(3):
            host = [synth.make_tokens(d.hidden, T, seed=700 + 10 * rep + j) for j, d in enumerate(STACK)]
            eager = [l.forward(h) for l, h in zip(layers, host)]   # eager work between replays
            for x, h in zip(xs, host):
                x.copy_(to_device(h, dev))
            for t in ys + ws:
                t.fill_(float("nan"))
            for t in ids:
                t.fill_(-1)
            torch.cuda.synchronize()
            d0 = ctx.dispatches
            graph.launch()
            ctx.synchronize()
            per_replay = ctx.dispatches - d0 if per_replay is None else per_replay
            assert ctx.dispatches - d0 == per_replay > 0
            for (ey, ei, ew), y, i, w in zip(eager, ys, ids, ws):
                assert torch.equal(i, ei) and torch.equal(w, ew) and torch.equal(y, ey), f"replay {rep}"
        graph.close()
    finally:
        ctx.close()


def test_capture_rules_are_enforced_without_a_gpu_call():
    """Entry points that would synchronise or allocate refuse a capturing context; these
    checks run on the host before any HIP call, so they need no device (a NULL context)."""
    import ctypes as C
    from hydra_amd._lib import lib
    L = lib()
    assert L.hh_ctx_capture_begin(None) != 0
    g = C.c_void_p()
    assert L.hh_ctx_capture_end(None, C.byref(g)) != 0
    assert L.hh_graph_launch(None) != 0
    assert L.hh_graph_destroy(None) == 0


@pytest.mark.gpu
def test_growing_scratch_is_refused_while_a_graph_lives():
    """A live graph holds the context's arena and attention-partial addresses: an eager call
    that would reallocate either fails with HH_EINVAL until the graph is destroyed; a call
    that fits still runs, and after destruction the growing call succeeds."""
    import torch
    from hydra_amd._lib import HydraHIPError
    from hydra_amd.layer import Context, MoELayer
    print("[gpu] graph blocks arena growth", flush=True)
    ctx = Context(0)
    try:
        d = STACK[0]
        layer = MoELayer(synth.make_layer(d, seed=55), ctx)
        ctx.reserve(d, 1)
        x = torch.zeros((1, d.hidden), dtype=torch.int16, device="cuda:0")
        y = torch.empty((1, d.hidden), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        graph = ctx.capture(lambda: layer.forward_into(x, y))
        layer.forward(synth.make_tokens(d.hidden, 1, seed=5))          # fits: runs
        with pytest.raises(HydraHIPError) as e:
            layer.forward(synth.make_tokens(d.hidden, 200, seed=6))    # would grow the arena
        assert e.value.code == -1 and "graph" in str(e.value)
        graph.launch()
        ctx.synchronize()
        graph.close()
        y2, _, _ = layer.forward(synth.make_tokens(d.hidden, 200, seed=6))
        assert torch.isfinite(y2).all()
    finally:
        ctx.close()


@pytest.mark.gpu
def test_attention_is_refused_inside_a_capture():
    """hh_attention_decode takes the key count and ring position as per-step arguments, which a
    graph would replay unchanged: it fails with HH_EINVAL while the context captures, the
    capture still ends cleanly, and the same call runs eagerly afterwards."""
    import torch
    from hydra_amd._lib import HydraHIPError
    from hydra_amd.attention import attention_decode_into
    from hydra_amd.layer import Context
    print("[gpu] attention refused under capture", flush=True)
    ctx = Context(0)
    try:
        dev = "cuda:0"
        q = torch.randn((8, 64), device=dev)
        k = torch.randn((512, 1, 64), device=dev).half()
        v = torch.randn((512, 1, 64), device=dev).half()
        sinks = torch.zeros(8, dtype=torch.int16, device=dev)
        out = torch.empty((8, 64), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        with pytest.raises(HydraHIPError) as e:
            ctx.capture(lambda: attention_decode_into(ctx, q, k, v, sinks, 300, out=out))
        assert e.value.code == -1 and "graph" in str(e.value)
        attention_decode_into(ctx, q, k, v, sinks, 300, out=out)
        ctx.synchronize()
        assert torch.isfinite(out).all()
    finally:
        ctx.close()
