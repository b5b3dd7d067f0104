"""Checkpoint loading: stacked expert tensors of a safetensors checkpoint scattered into the
expert blob layout (the reference installer's ScatterCopy, RepackPlan.swift:198-230,
GemmaRepackPlan.swift:137-155, QwenRepackPlan.swift:97-126).

The checkpoints are written here from the synthetic generator's per-slot tensors, so the blobs
the loader builds must equal `synth.make_layer`'s packed blobs byte for byte, and on the GPU
the loaded layer must give the synthetic layer's outputs bit for bit.
"""
import json
import os
import struct

import numpy as np
import pytest

from hydra_amd import checkpoint as CK
from hydra_amd import formats as F
from hydra_amd import synth

CASES = {
    "gpt-oss": F.MoEDesc(hidden=256, intermediate=128, experts=6, top_k=2, quant=F.QUANT_MXFP4,
                         activation=F.ACT_SWIGLU_OAI, router=F.ROUTER_TOPK_SOFTMAX, expert_bias=1),
    "gemma4": F.MoEDesc(hidden=320, intermediate=192, experts=5, top_k=2, quant=F.QUANT_BF16,
                        activation=F.ACT_GELU_TANH, router=F.ROUTER_GEMMA),
    "qwen3.5-moe": F.MoEDesc(hidden=256, intermediate=128, experts=8, top_k=3, quant=F.QUANT_MLX4,
                             activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM,
                             shared_intermediate=192, group_size=64),
}
# Qwen's published builds store the router and shared gate as 8-bit MLX (Qwen35MoeConfig.swift:340-342).
ROUTER_BITS = {"qwen3.5-moe": 8}
LAYER = 3
SEED = 41


def write_safetensors(path, tensors):
    """tensors: {name: (dtype, shape, uint8 bytes)} → one .safetensors file."""
    header, blobs, cursor = {}, [], 0
    for name, (dt, shape, data) in tensors.items():
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [cursor, cursor + data.size]}
        blobs.append(data)
        cursor += data.size
    raw = json.dumps(header).encode()
    raw += b" " * (-len(raw) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        for b in blobs:
            f.write(b.tobytes())


def checkpoint_tensors(desc, family, layer_idx=LAYER, seed=SEED, router_bits=None):
    """The synthetic layer as checkpoint tensors, and the layer dict itself."""
    rb = ROUTER_BITS.get(family, 0) if router_bits is None else router_bits
    layer = synth.make_layer(desc, seed=seed, router_bits=rb)
    _, routed = synth._expert_tensors(desc, seed, "experts", desc.experts, desc.intermediate)
    out = {}
    for slot, name, dt, shape in CK.expert_sources(desc, family, layer_idx):
        out[name] = (dt, shape, routed[slot])
    if desc.shared_intermediate:
        _, shared = synth._expert_tensors(desc, seed, "shared", 1, desc.shared_intermediate)
        for slot, name, dt, shape in CK.expert_sources(desc, family, layer_idx, shared=True):
            out[name] = (dt, shape, shared[slot])
    for key, (name, dt, shape, req) in CK.router_sources(desc, family, layer_idx, rb).items():
        if key in layer:
            out[name] = (dt, shape, layer[key])
    return out, layer


def write_checkpoint(tmp_path, family, shards=1):
    desc = CASES[family]
    tens, layer = checkpoint_tensors(desc, family)
    names = list(tens)
    if shards == 1:
        write_safetensors(tmp_path / "model.safetensors", tens)
    else:
        wm = {}
        for s in range(shards):
            fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = {n: tens[n] for n in names[s::shards]}
            write_safetensors(tmp_path / fn, part)
            wm.update({n: fn for n in part})
        with open(tmp_path / "model.safetensors.index.json", "w") as f:
            json.dump({"metadata": {}, "weight_map": wm}, f)
    return desc, layer


@pytest.mark.parametrize("family", list(CASES))
@pytest.mark.parametrize("shards", [1, 3])
def test_scatter_plan_rebuilds_the_packed_blobs(tmp_path, family, shards):
    """Host replay of the scatter each tensor gets (dst[e·stride + offset[slot]] = src[e]):
    the name → slot map and the shapes reproduce the blob layout byte for byte."""
    desc, layer = write_checkpoint(tmp_path, family, shards)
    ck = CK.Checkpoint(str(tmp_path))
    lay = F.blob_layout(desc)
    blobs = np.zeros((desc.experts, lay.stride), np.uint8)
    for slot, name, dt, shape in CK.expert_sources(desc, family, LAYER):
        data = np.asarray(ck.tensor(name, dt, shape)).reshape(desc.experts, -1)
        assert data.shape[1] == lay.sizes[slot]
        blobs[:, lay.offsets[slot]:lay.offsets[slot] + lay.sizes[slot]] = data
    assert np.array_equal(blobs, layer["experts"])
    if desc.shared_intermediate:
        slay = F.blob_layout(desc, desc.shared_intermediate)
        blob = np.zeros(slay.stride, np.uint8)
        for slot, name, dt, shape in CK.expert_sources(desc, family, LAYER, shared=True):
            blob[slay.offsets[slot]:slay.offsets[slot] + slay.sizes[slot]] = \
                np.asarray(ck.tensor(name, dt, shape)).reshape(-1)
        assert np.array_equal(blob, layer["shared_expert"])
    for key, (name, dt, shape, req) in CK.router_sources(desc, family, LAYER, ROUTER_BITS.get(family, 0)).items():
        if key in layer:
            got = np.asarray(ck.tensor(name, dt, shape)).reshape(-1)
            assert np.array_equal(got, np.asarray(layer[key]).view(np.uint8).reshape(-1))


def test_shape_and_dtype_mismatches_are_errors(tmp_path):
    desc = CASES["gpt-oss"]
    tens, _ = checkpoint_tensors(desc, "gpt-oss")
    name = f"model.layers.{LAYER}.mlp.experts.down_proj_scales"
    dt, shape, data = tens[name]
    tens[name] = (dt, (shape[0], shape[1] * shape[2]), data)          # flattened: wrong shape
    write_safetensors(tmp_path / "a.safetensors", tens)
    with pytest.raises(CK.CheckpointError, match="down_proj_scales"):
        CK.load_moe_layer(str(tmp_path / "a.safetensors"), desc, "gpt-oss", LAYER)
    tens[name] = ("I8", shape, data)                                   # wrong dtype
    write_safetensors(tmp_path / "b.safetensors", tens)
    with pytest.raises(CK.CheckpointError, match="expected U8"):
        CK.load_moe_layer(str(tmp_path / "b.safetensors"), desc, "gpt-oss", LAYER)
    del tens[name]                                                     # missing
    write_safetensors(tmp_path / "c.safetensors", tens)
    with pytest.raises(CK.CheckpointError, match="missing tensor"):
        CK.load_moe_layer(str(tmp_path / "c.safetensors"), desc, "gpt-oss", LAYER)
    with pytest.raises(CK.CheckpointError, match="missing tensor"):   # another layer index
        CK.load_moe_layer(str(tmp_path / "c.safetensors"), desc, "gpt-oss", LAYER + 1)
    with pytest.raises(CK.CheckpointError, match="BF16 routed"):      # family / format clash
        CK.load_moe_layer(str(tmp_path / "c.safetensors"), CASES["gemma4"].replace(quant=F.QUANT_MXFP4),
                          "gemma4", LAYER)


def test_router_format_is_read_from_the_checkpoint(tmp_path):
    """Qwen's router loads from MLX words (bit width from the word count) or from BF16; an
    MLX-quantised router of another family, or a word count of neither width, is an error."""
    desc = CASES["qwen3.5-moe"]
    stem = f"language_model.model.layers.{LAYER}.mlp.gate"
    ck8, _ = checkpoint_tensors(desc, "qwen3.5-moe", router_bits=8)
    write_safetensors(tmp_path / "q8.safetensors", ck8)
    assert CK._quantised_router_bits(CK.Checkpoint(str(tmp_path / "q8.safetensors")), desc,
                                     "qwen3.5-moe", LAYER) == 8
    ck4, _ = checkpoint_tensors(desc, "qwen3.5-moe", router_bits=4)
    write_safetensors(tmp_path / "q4.safetensors", ck4)
    assert CK._quantised_router_bits(CK.Checkpoint(str(tmp_path / "q4.safetensors")), desc,
                                     "qwen3.5-moe", LAYER) == 4
    bf, _ = checkpoint_tensors(desc, "qwen3.5-moe", router_bits=0)
    write_safetensors(tmp_path / "bf.safetensors", bf)
    assert CK._quantised_router_bits(CK.Checkpoint(str(tmp_path / "bf.safetensors")), desc,
                                     "qwen3.5-moe", LAYER) == 0
    E, H = desc.experts, desc.hidden
    bad = dict(ck8)
    bad[f"{stem}.weight"] = ("U32", (E, H // 16), np.zeros(E * H // 4, np.uint8))   # 2-bit
    write_safetensors(tmp_path / "bad.safetensors", bad)
    with pytest.raises(CK.CheckpointError, match="neither 4- nor 8-bit"):
        CK.load_moe_layer(str(tmp_path / "bad.safetensors"), desc, "qwen3.5-moe", LAYER)
    g = CASES["gpt-oss"]
    tens, _ = checkpoint_tensors(g, "gpt-oss")
    rs = f"model.layers.{LAYER}.mlp.router"
    tens[f"{rs}.weight"] = ("U32", (g.experts, g.hidden // 4), np.zeros(g.experts * g.hidden, np.uint8))
    tens[f"{rs}.scales"] = ("BF16", (g.experts, g.hidden // 64), np.zeros(g.experts * g.hidden // 32, np.uint8))
    write_safetensors(tmp_path / "g.safetensors", tens)
    with pytest.raises(CK.CheckpointError, match="only Qwen"):
        CK.load_moe_layer(str(tmp_path / "g.safetensors"), g, "gpt-oss", LAYER)


def test_truncated_byte_range_is_an_error(tmp_path):
    path = tmp_path / "t.safetensors"
    write_safetensors(path, {"w": ("BF16", (4, 4), np.zeros(30, np.uint8))})
    with pytest.raises(CK.CheckpointError, match="byte range"):
        CK.SafetensorsFile(str(path)).tensor("w")


@pytest.mark.gpu
@pytest.mark.parametrize("family", list(CASES))
def test_loaded_layer_equals_synthetic_layer_bit_for_bit(tmp_path, family):
    """Blobs scattered on the device equal the packed host blobs, and the layer computes the
    same outputs, indices and weights bit for bit (decode and prefill sizes)."""
    import torch
    from hydra_amd.layer import Context, MoELayer
    print(f"[gpu] checkpoint {family}", flush=True)
    desc, layer = write_checkpoint(tmp_path, family, shards=2)
    ctx = Context(0)
    try:
        loaded = CK.load_moe_layer(str(tmp_path), desc, family, LAYER, ctx=ctx)
        assert np.array_equal(loaded.experts.cpu().numpy(), layer["experts"])
        if desc.shared_intermediate:
            assert np.array_equal(loaded.tensors["shared_expert"].cpu().numpy(), layer["shared_expert"])
        ref = MoELayer(layer, ctx)
        for T in (1, 40):
            x = synth.make_tokens(desc.hidden, T, seed=SEED + T)
            y0, i0, w0 = ref.forward(x)
            y1, i1, w1 = loaded.forward(x)
            assert torch.equal(i0, i1) and torch.equal(w0, w1) and torch.equal(y0, y1)
    finally:
        ctx.close()


def test_reader_agrees_with_the_safetensors_library(tmp_path):
    """Files written by the safetensors package read back identically here, and ours read
    there (dtypes numpy can hold)."""
    st = pytest.importorskip("safetensors.numpy")
    a = np.arange(6 * 5 * 16, dtype=np.uint8).reshape(6, 5, 16)
    b = (np.arange(12, dtype=np.uint32) * 2654435761).astype(np.uint32).reshape(3, 4)
    st.save_file({"a": a, "b": b}, str(tmp_path / "lib.safetensors"))
    f = CK.SafetensorsFile(str(tmp_path / "lib.safetensors"))
    assert f.tensor("a")[:2] == ("U8", (6, 5, 16)) and np.array_equal(f.tensor("a")[2], a.reshape(-1))
    assert f.tensor("b")[:2] == ("U32", (3, 4))
    assert np.array_equal(np.asarray(f.tensor("b")[2]).view(np.uint32), b.reshape(-1))
    write_safetensors(tmp_path / "ours.safetensors", {"a": ("U8", a.shape, a), "b": ("U32", b.shape, b)})
    back = st.load_file(str(tmp_path / "ours.safetensors"))
    assert np.array_equal(back["a"], a) and np.array_equal(back["b"], b)
