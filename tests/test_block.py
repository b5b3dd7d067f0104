"""GPU parity of the FFN block entry (hh_moe_block_forward): RMSNorm → MoE layer → residual add
(GPT-OSS, Qwen), and Gemma's parallel branches with their post-norms and layer scalar, against
the fp64 oracle (oracle.block_forward_layer), through the C ABI.

Bars: top-k indices bit-exact; the block's change to the residual stream within rel-L2 1e-3 of
the oracle's; the layer input bit-exact with the oracle's bf16 rounding (checked by running
hh_moe_forward on the oracle's bf16 input and requiring the block output to equal
fp32(hidden + y) bit for bit); a T-token block equal to T one-token blocks bit for bit."""
import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3

CASES = {
    "gpt-oss-20b": (F.GPT_OSS_20B, [1, 2, 8, 40]),
    # a shared expert (its gate row in the router) and H past a 512-column slice
    "mxfp4-shared": (F.MoEDesc(hidden=640, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                               activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                               shared_intermediate=128, expert_bias=1), [1, 2, 5]),
    "qwen-q4": (F.QWEN_35B_A3B_Q4, [1, 24]),
    "gemma-bf16": (F.GEMMA_BF16, [1, 40]),
}


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def make_norms(desc, seed):
    rng = np.random.default_rng(seed)
    H = desc.hidden
    nb = lambda: synth.f32_to_bf16(rng.uniform(0.5, 1.5, H).astype(np.float32))
    norms = {"pre_norm": nb(), "eps": 1e-6 if desc.router == F.ROUTER_GEMMA else 1e-5}
    if desc.router == F.ROUTER_GEMMA:
        norms.update(post_expert_norm=nb(), post_dense_norm=nb(), post_norm=nb(),
                     layer_scalar=synth.f32_to_bf16(np.array([0.75], np.float32)))
    return norms


@pytest.mark.parametrize("name", list(CASES))
def test_block_against_oracle(name):
    import torch
    from hydra_amd.layer import Context, MoELayer, to_device
    desc, Ts = CASES[name]
    print(f"[gpu] block {name} T={Ts}", flush=True)
    gemma = desc.router == F.ROUTER_GEMMA
    ctx = Context(0)
    try:
        layer = synth.make_layer(desc, seed=21)
        L = MoELayer(layer, ctx)
        norms = make_norms(desc, 22)
        dn = {k: (v if k == "eps" else to_device(v, "cuda:0")) for k, v in norms.items()}
        rng = np.random.default_rng(23)
        for T in Ts:
            print(f"[gpu] block {name} T={T}", flush=True)
            hidden = (rng.standard_normal((T, desc.hidden)) * 3).astype(np.float32)
            dense = (rng.standard_normal((T, desc.hidden))).astype(np.float32) if gemma else None
            h_dev = torch.from_numpy(hidden.copy()).to("cuda:0")
            d_dev = None if dense is None else torch.from_numpy(dense).to("cuda:0")
            idx = torch.full((T, desc.top_k), -1, dtype=torch.int32, device="cuda:0")
            w = torch.empty((T, desc.top_k), dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            L.block_forward_into(dn, h_dev, d_dev, idx, w)
            ctx.synchronize()
            out = h_dev.cpu().numpy()
            ref, ridx, rw, x = O.block_forward_layer(layer, norms, hidden, dense, nthreads=16)
            assert np.array_equal(idx.cpu().numpy(), ridx), (name, T)
            ls = 0.75 if gemma else 1.0
            assert rel_l2(out / ls - hidden, ref / ls - hidden) < REL_L2, (name, T)
            if not gemma:
                # the layer input equals the oracle's bf16 rounding: the same layer call on
                # the oracle's x reproduces the block output bit for bit
                y, _, _ = L.forward(x)
                expect = hidden + y.cpu().numpy()
                assert np.array_equal(out.view(np.uint32), expect.view(np.uint32)), (name, T)
            if T > 1:
                # T-token block == T one-token blocks, bit for bit
                for t in sorted({0, T // 2, T - 1}):
                    h1 = torch.from_numpy(hidden[t:t + 1].copy()).to("cuda:0")
                    d1 = None if dense is None else torch.from_numpy(dense[t:t + 1].copy()).to("cuda:0")
                    torch.cuda.synchronize()
                    L.block_forward_into(dn, h1, d1)
                    ctx.synchronize()
                    assert np.array_equal(h1.cpu().numpy()[0].view(np.uint32), out[t].view(np.uint32)), (name, T, t)
    finally:
        ctx.close()


def test_block_rejects_missing_gemma_norms():
    import torch
    from hydra_amd._lib import HydraHIPError
    from hydra_amd.layer import Context, MoELayer, to_device
    print("[gpu] block argument checks", flush=True)
    desc = F.GEMMA_BF16.replace(experts=8, intermediate=64)
    ctx = Context(0)
    try:
        L = MoELayer(synth.make_layer(desc, seed=24), ctx)
        norms = make_norms(desc, 25)
        dn = {k: (v if k == "eps" else to_device(v, "cuda:0")) for k, v in norms.items()}
        h = torch.zeros((2, desc.hidden), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        with pytest.raises(HydraHIPError) as e:
            L.block_forward_into(dn, h, None)             # Gemma branches need dense_out
        assert e.value.code == -1
        with pytest.raises(HydraHIPError):
            L.block_forward_into({"eps": 1e-6}, h, None)  # pre_norm is required
    finally:
        ctx.close()
