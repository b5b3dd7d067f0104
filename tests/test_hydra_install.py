"""Loading a layer from a .hydra installation (HydraLayout.swift:4-20): experts/layer_NN.bin as
the kernels' blobs, GPT-OSS routers from resident.bin at HydraLayout's placements, the manifest
checked first.

The resident tensor list is pinned by the reference's own declared install sizes
(GptOssConfigTests.swift:20-40: installedBytes = expert pool + resident tensors + embedding), and
placements by the rule its tests state (RepackPlanTests.swift:205-215: 256-byte aligned, in
order, disjoint)."""
import json
import os

import numpy as np
import pytest

from hydra_amd import checkpoint as CK
from hydra_amd import formats as F
from hydra_amd import synth

# GptOssConfigTests.swift:20-40 (b20, b120): installed, expert pool and embedding bytes.
INSTALLED = {"20b": (13_761_264_768, 10_165_616_640, 1_158_266_880, 24, 32),
             "120b": (65_248_815_744, 60_993_699_840, 1_158_266_880, 36, 128)}


@pytest.mark.parametrize("name", list(INSTALLED))
def test_resident_list_matches_reference_install_sizes(name):
    installed, pool, embed, layers, experts = INSTALLED[name]
    tensors = CK.gpt_oss_resident_tensors(2880, experts, layers)
    # residentTensors also ends with model.norm.weight and lm_head.weight (GptOssConfig.swift:190-199)
    total = sum(b for _, b in tensors) + 2 * 2880 + embed
    assert installed == pool + total + embed


def test_resident_placements_are_aligned_disjoint_and_ordered():
    tensors = CK.gpt_oss_resident_tensors(2880, 32, 24)
    place = CK.resident_placements(tensors)
    prev = 0
    for n, b in tensors:
        off, nb = place[n]
        assert off % 256 == 0 and off >= prev and nb == b
        assert off - prev < 256
        prev = off + nb
    assert place[tensors[0][0]][0] == 0


LAYER, LAYERS = 1, 3
GPT = F.MoEDesc(hidden=256, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1)


def write_install(root, desc, layer_dict, attention=(4, 64, 2)):
    """A minimal GPT-OSS .hydra: manifest, resident.bin (router tensors of layer LAYER at their
    placements, other bytes random), experts/layer_01.bin (the packed blobs)."""
    lay = F.blob_layout(desc)
    os.makedirs(os.path.join(root, "experts"), exist_ok=True)
    manifest = {"format": "hydra/1",
                "model": {"name": "synthetic", "layerCount": LAYERS, "expertCount": desc.experts,
                          "expertsPerToken": desc.top_k, "hiddenSize": desc.hidden,
                          "intermediateSize": desc.intermediate, "vocabSize": 16, "slidingWindow": 128,
                          "expertQuantization": "mxfp4", "architecture": "gptOss"},
                "layout": {"expertStrideBytes": lay.stride, "expertPayloadBytes": lay.payload,
                           "residentBytes": 0, "embeddingBytes": 0, "tensorAlignment": 256,
                           "pageAlignment": 16384},
                "files": {}, "sourceDescription": "synthetic", "sourceTotalBytes": 0, "tensors": [],
                "createdAt": 0}
    with open(os.path.join(root, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    heads, hd, kv = attention
    tensors = CK.gpt_oss_resident_tensors(desc.hidden, desc.experts, LAYERS, heads, hd, kv)
    place = CK.resident_placements(tensors)
    end = max(o + b for o, b in place.values())
    res = synth.random_bytes(5, "resident", end)
    for key, suffix in [("router_weight", "weight"), ("router_bias", "bias")]:
        off, nb = place[f"model.layers.{LAYER}.mlp.router.{suffix}"]
        res[off:off + nb] = np.asarray(layer_dict[key]).view(np.uint8).reshape(-1)
    res.tofile(os.path.join(root, "resident.bin"))
    layer_dict["experts"].tofile(os.path.join(root, "experts", f"layer_{LAYER:02d}.bin"))


def test_manifest_is_checked(tmp_path):
    layer = synth.make_layer(GPT, seed=9)
    write_install(str(tmp_path), GPT, layer)
    m = json.load(open(tmp_path / "manifest.json"))
    m["format"] = "hydra/0"
    json.dump(m, open(tmp_path / "manifest.json", "w"))
    with pytest.raises(CK.CheckpointError, match="format"):
        CK.load_hydra_layer(str(tmp_path), GPT, "gpt-oss", LAYER, attention=(4, 64, 2))
    m["format"] = "hydra/1"
    m["layout"]["expertStrideBytes"] += 16384
    json.dump(m, open(tmp_path / "manifest.json", "w"))
    with pytest.raises(CK.CheckpointError, match="stride"):
        CK.load_hydra_layer(str(tmp_path), GPT, "gpt-oss", LAYER, attention=(4, 64, 2))


@pytest.mark.gpu
def test_hydra_layer_equals_synthetic_layer(tmp_path):
    import torch
    from hydra_amd.layer import Context, MoELayer
    print("[gpu] .hydra layer", flush=True)
    layer = synth.make_layer(GPT, seed=9)
    write_install(str(tmp_path), GPT, layer)
    ctx = Context(0)
    try:
        loaded = CK.load_hydra_layer(str(tmp_path), GPT, "gpt-oss", LAYER, ctx=ctx, attention=(4, 64, 2))
        assert np.array_equal(loaded.experts.cpu().numpy(), layer["experts"])
        ref = MoELayer(layer, ctx)
        for T in (1, 40):
            x = synth.make_tokens(GPT.hidden, T, seed=10 + T)
            y0, i0, w0 = ref.forward(x)
            y1, i1, w1 = loaded.forward(x)
            assert torch.equal(i0, i1) and torch.equal(w0, w1) and torch.equal(y0, y1)
    finally:
        ctx.close()


@pytest.mark.gpu
def test_hydra_qwen_layer_with_router_from_checkpoint(tmp_path):
    """Qwen: routed experts from experts/layer_NN.bin, the 8-bit MLX router, shared gate and
    shared expert from the safetensors checkpoint."""
    import torch
    from hydra_amd.layer import Context, MoELayer
    import test_checkpoint as TC
    print("[gpu] .hydra qwen layer", flush=True)
    desc = TC.CASES["qwen3.5-moe"]
    tens, layer = TC.checkpoint_tensors(desc, "qwen3.5-moe", layer_idx=LAYER, router_bits=8)
    ckdir = tmp_path / "ck"
    os.makedirs(ckdir)
    TC.write_safetensors(ckdir / "model.safetensors", tens)
    root = tmp_path / "q.hydra"
    lay = F.blob_layout(desc)
    os.makedirs(root / "experts")
    json.dump({"format": "hydra/1",
               "model": {"name": "q", "layerCount": LAYERS, "expertCount": desc.experts,
                         "expertsPerToken": desc.top_k, "hiddenSize": desc.hidden, "vocabSize": 16,
                         "slidingWindow": 0, "expertQuantization": "mlx4", "architecture": "qwen35Moe"},
               "layout": {"expertStrideBytes": lay.stride, "expertPayloadBytes": lay.payload,
                          "residentBytes": 0, "embeddingBytes": 0, "tensorAlignment": 256,
                          "pageAlignment": 16384}}, open(root / "manifest.json", "w"))
    layer["experts"].tofile(str(root / "experts" / f"layer_{LAYER:02d}.bin"))
    ctx = Context(0)
    try:
        loaded = CK.load_hydra_layer(str(root), desc, "qwen3.5-moe", LAYER, ctx=ctx,
                                     router_checkpoint=str(ckdir))
        ref = MoELayer(layer, ctx)
        for T in (1, 40):
            x = synth.make_tokens(desc.hidden, T, seed=20 + T)
            y0, i0, w0 = ref.forward(x)
            y1, i1, w1 = loaded.forward(x)
            assert torch.equal(i0, i1) and torch.equal(w0, w1) and torch.equal(y0, y1)
    finally:
        ctx.close()
