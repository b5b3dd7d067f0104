"""hh_runner: a layer stack's MoE halves (FFN blocks) with the caller's per-layer hook in front
of each, eager and recorded as one HIP graph, against the same calls made one by one.

Three layers share one fp32 residual stream (H = 256): an MXFP4 GPT-OSS-style pre-norm block, a
Qwen-style MLX-4 block with a shared expert and an 8-bit MLX router, and a Gemma-style BF16
block with parallel branches whose dense output the hook writes. The hook enqueues a projection
of the current residual stream (hh_expert_gemm) before every layer, so the order of hooks and
blocks shows in its outputs. Bars: bit for bit."""
import ctypes as C

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth

pytestmark = pytest.mark.gpu

H = 256
DESCS = [
    (F.MoEDesc(hidden=H, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
               activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1), 0),
    (F.MoEDesc(hidden=H, intermediate=128, experts=8, top_k=3, quant=F.QUANT_MLX4,
               activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
               shared_intermediate=128, group_size=64), 8),
    (F.MoEDesc(hidden=H, intermediate=128, experts=5, top_k=2, quant=F.QUANT_BF16,
               activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA), 0),
]


def _norms(rng, gemma):
    nb = lambda: synth.f32_to_bf16(rng.uniform(0.5, 1.5, H).astype(np.float32))
    n = {"pre_norm": nb(), "eps": 1e-6 if gemma else 1e-5}
    if gemma:
        n.update(post_expert_norm=nb(), post_dense_norm=nb(), post_norm=nb(),
                 layer_scalar=synth.f32_to_bf16(np.array([0.5], np.float32)))
    return n


@pytest.mark.parametrize("T", [1, 24])
def test_runner_equals_calls_one_by_one(T):
    import torch
    from hydra_amd._lib import MatrixC, check, lib
    from hydra_amd.layer import Context, MoELayer, Runner, to_device
    print(f"[gpu] runner T={T}", flush=True)
    dev = "cuda:0"
    ctx = Context(0)
    try:
        rng = np.random.default_rng(71)
        layers, mats, probes = [], [], []
        dense = torch.zeros((T, H), dtype=torch.float32, device=dev)
        for i, (d, rb) in enumerate(DESCS):
            ml = MoELayer(synth.make_layer(d, seed=72 + i, router_bits=rb), ctx)
            gemma = d.router == F.ROUTER_GEMMA
            norms = {k: (v if k == "eps" else to_device(v, dev)) for k, v in _norms(rng, gemma).items()}
            layers.append((ml, norms, dense if gemma else None))
            rows = H if gemma else 64
            w = to_device(synth.bf16_normal(80 + i, "hook", rows * H, 0.0, 0.05), dev)
            mats.append((MatrixC(F.QUANT_BF16, rows, H, 64, C.c_void_p(w.data_ptr()), None, None, None), w))
            probes.append(dense if gemma else torch.empty((T, rows), dtype=torch.float32, device=dev))
        runner = Runner(ctx, layers)
        runner.reserve(T)

        def hook(l, hidden):
            out = probes[l]
            check(lib().hh_expert_gemm(ctx.handle, C.byref(mats[l][0]), C.c_void_p(hidden.data_ptr()),
                                       T, C.c_void_p(out.data_ptr())))

        def snapshot(hidden):
            return [hidden.cpu().numpy().copy()] + [p.cpu().numpy().copy() for p in probes]

        x0 = (rng.standard_normal((T, H)) * 2).astype(np.float32)
        # one by one
        hid = torch.from_numpy(x0.copy()).to(dev)
        torch.cuda.synchronize()
        for l, (ml, norms, dn) in enumerate(layers):
            hook(l, hid)
            ml.block_forward_into(norms, hid, dn)
        ctx.synchronize()
        ref = snapshot(hid)
        assert np.isfinite(ref[0]).all()
        # the runner, eager
        for p in probes:
            p.fill_(float("nan"))
        hid2 = torch.from_numpy(x0.copy()).to(dev)
        torch.cuda.synchronize()
        seen = []
        runner.forward(hid2, hook=lambda l: (seen.append(l), hook(l, hid2)))
        ctx.synchronize()
        assert seen == [0, 1, 2]
        for a, b in zip(snapshot(hid2), ref):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # one graph for the stack, replayed on new inputs
        buf = torch.empty((T, H), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        graph = runner.capture(buf, hook=lambda l: hook(l, buf))
        for rep in range(3):
            xr = (rng.standard_normal((T, H)) * 2).astype(np.float32)
            e = torch.from_numpy(xr.copy()).to(dev)
            torch.cuda.synchronize()
            runner.forward(e, hook=lambda l: hook(l, e))   # eager work between the replays
            ctx.synchronize()
            expect = snapshot(e)
            buf.copy_(torch.from_numpy(xr))
            for p in probes:
                p.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.launch()
            ctx.synchronize()
            for a, b in zip(snapshot(buf), expect):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), rep
        graph.close()
        runner.close()
    finally:
        ctx.close()


@pytest.mark.parametrize("T", [1, 64])
def test_runner_stack_against_chained_oracle(T):
    """The same 3-layer stack with hooks against the fp64 oracle chained layer by layer
    (ModelRunner.swift:110-230, 418-547: per layer the token mixer, then the MoE half on the
    residual stream): the hook is the oracle's matvec of the current residual, the block
    `block_forward_layer`. Bars: the final residual stream and every hook output within
    rel-L2 1e-3; every layer's top-k indices equal (read from the one-by-one calls, which the
    test above shows equal to the runner bit for bit)."""
    import torch
    from hydra_amd._lib import MatrixC, check, lib
    from hydra_amd.layer import Context, MoELayer, Runner, to_device
    from oracle import oracle as O
    print(f"[gpu] runner vs oracle T={T}", flush=True)
    dev = "cuda:0"
    ctx = Context(0)
    try:
        rng = np.random.default_rng(91)
        host_layers, layers, mats, probes, norms_host = [], [], [], [], []
        dense = torch.zeros((T, H), dtype=torch.float32, device=dev)
        for i, (d, rb) in enumerate(DESCS):
            hl = synth.make_layer(d, seed=92 + i, router_bits=rb)
            host_layers.append(hl)
            ml = MoELayer(hl, ctx)
            gemma = d.router == F.ROUTER_GEMMA
            nh = _norms(rng, gemma)
            norms_host.append(nh)
            norms = {k: (v if k == "eps" else to_device(v, dev)) for k, v in nh.items()}
            layers.append((ml, norms, dense if gemma else None))
            rows = H if gemma else 64
            wh = synth.bf16_normal(100 + i, "hook", rows * H, 0.0, 0.05)
            w = to_device(wh, dev)
            mats.append((MatrixC(F.QUANT_BF16, rows, H, 64, C.c_void_p(w.data_ptr()), None, None, None), w, wh, rows))
            probes.append(dense if gemma else torch.empty((T, rows), dtype=torch.float32, device=dev))
        x0 = (rng.standard_normal((T, H)) * 2).astype(np.float32)

        def hook(l, hidden):
            check(lib().hh_expert_gemm(ctx.handle, C.byref(mats[l][0]), C.c_void_p(hidden.data_ptr()),
                                       T, C.c_void_p(probes[l].data_ptr())))

        # the oracle chained in fp64
        hid_o = x0.astype(np.float64)
        ref_probes, ref_idx = [], []
        for l, hl in enumerate(host_layers):
            _, _, wh, rows = mats[l]
            p = O.matvec(F.QUANT_BF16, rows, H, wh, x=hid_o)
            ref_probes.append(p)
            gemma = hl["desc"].router == F.ROUTER_GEMMA
            lg = O.router_logits(hl["desc"], hl, O.f64_to_bf16(
                O.rms_norm(hid_o, O.bf16_to_f32(norms_host[l]["pre_norm"]), norms_host[l]["eps"],
                           pow_form=gemma)) if not gemma else O.f32_to_bf16(hid_o.astype(np.float32)))
            K = hl["desc"].top_k
            srt = np.sort(lg, axis=1)[:, ::-1]
            gap = (srt[:, K - 1] - srt[:, K]) / np.maximum(np.abs(srt[:, 0]), 1.0)
            assert np.all(gap > 1e-6), "near-tie in the test data: change the seed"
            hid_o, idx, _, _ = O.block_forward_layer(hl, norms_host[l], hid_o,
                                                     dense_out=p if gemma else None)
            ref_idx.append(idx)
        # the calls one by one, with per-layer top-k indices
        hid = torch.from_numpy(x0.copy()).to(dev)
        idxs = [torch.empty((T, d.top_k), dtype=torch.int32, device=dev) for d, _ in DESCS]
        torch.cuda.synchronize()
        for l, (ml, norms, dn) in enumerate(layers):
            hook(l, hid)
            ml.block_forward_into(norms, hid, dn, idx=idxs[l])
        ctx.synchronize()
        one = hid.cpu().numpy().copy()
        for l in range(3):
            assert np.array_equal(idxs[l].cpu().numpy(), ref_idx[l]), l
        # the runner
        hid2 = torch.from_numpy(x0.copy()).to(dev)
        for p in probes:
            p.fill_(float("nan"))
        torch.cuda.synchronize()
        runner = Runner(ctx, layers)
        runner.forward(hid2, hook=lambda l: hook(l, hid2))
        ctx.synchronize()
        got = hid2.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), one.view(np.uint32))
        rel = np.linalg.norm(got - hid_o) / np.linalg.norm(hid_o)
        assert rel < 1e-3, rel
        for l in range(3):
            pl = probes[l].cpu().numpy().astype(np.float64)
            r = np.linalg.norm(pl - ref_probes[l]) / np.linalg.norm(ref_probes[l])
            assert r < 1e-3, (l, r)
        print(f"[gpu] runner vs oracle T={T}: rel-L2 {rel:.2e}", flush=True)
        runner.close()
    finally:
        ctx.close()


def test_runner_hook_torch_work_and_errors():
    """A hook's torch work runs on the stream hh_runner hands it (ordered with the blocks: a
    copy of the residual stream taken by the hook of layer l equals the residual after layer
    l − 1 run one by one), and an exception raised by a hook comes back out of forward()."""
    import torch
    from hydra_amd.layer import Context, MoELayer, Runner, to_device
    print("[gpu] runner torch hook", flush=True)
    dev = "cuda:0"
    T = 8
    ctx = Context(0)
    try:
        rng = np.random.default_rng(93)
        layers = []
        for i, (d, rb) in enumerate(DESCS[:2]):
            ml = MoELayer(synth.make_layer(d, seed=94 + i, router_bits=rb), ctx)
            norms = {k: (v if k == "eps" else to_device(v, dev)) for k, v in _norms(rng, False).items()}
            layers.append((ml, norms, None))
        x0 = (rng.standard_normal((T, H)) * 2).astype(np.float32)
        hid = torch.from_numpy(x0.copy()).to(dev)
        torch.cuda.synchronize()
        after = []
        for ml, norms, _ in layers:
            ml.block_forward_into(norms, hid)
            ctx.synchronize()
            after.append(hid.cpu().numpy().copy())
        runner = Runner(ctx, layers)
        hid2 = torch.from_numpy(x0.copy()).to(dev)
        snaps = [torch.empty_like(hid2) for _ in layers]
        torch.cuda.synchronize()
        runner.forward(hid2, hook=lambda l: snaps[l].copy_(hid2 * 1.0))
        ctx.synchronize()
        assert np.array_equal(snaps[0].cpu().numpy(), x0)
        assert np.array_equal(snaps[1].cpu().numpy().view(np.uint32), after[0].view(np.uint32))
        assert np.array_equal(hid2.cpu().numpy().view(np.uint32), after[1].view(np.uint32))

        def bad(l):
            if l == 1:
                raise ValueError("hook failed on purpose")
        with pytest.raises(ValueError, match="on purpose"):
            runner.forward(hid2, hook=bad)
        ctx.synchronize()
        runner.close()
    finally:
        ctx.close()
