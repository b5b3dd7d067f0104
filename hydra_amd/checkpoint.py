"""Checkpoint expert tensors straight into HBM.

The reference installs a checkpoint by repacking it into a `.hydra` file: every stacked expert
tensor of a layer (one safetensors entry holding all E experts' copies of one blob slot) is
scattered into E expert blobs at the slot's offset (`RepackPlan.swift:198-230` for GPT-OSS,
`GemmaRepackPlan.swift:137-155` for Gemma 4 BF16, `QwenRepackPlan.swift:97-126` for Qwen
MLX), and the runtime later reads those blobs through the SSD slot cache. Here every expert is
resident, so the same scatter goes from the safetensors bytes directly into the device blob
buffer the kernels read (`hh_scatter_expert_tensor`, one strided copy per tensor), and the
router tensors are copied as they are. The result is an `MoELayer` whose weights are
byte-for-byte the blobs the installer would have written.

Tensor names and shapes follow the reference's configs: `GptOssConfig.swift:164-165` and the
expert suffixes of `RepackPlan.swift:208-215`; `Gemma4Config.swift:183-208` (router
`router.proj.weight`, `router.scale`, `router.per_expert_scale`; experts `experts.gate_up_proj`
[E][2I][H], gate rows first, as `Gemma4Weights.swift:103-113` reads them, and
`experts.down_proj`); `Qwen35MoeConfig.swift:155-158, 341-368` (prefix
`language_model.model`, experts `mlp.switch_mlp.{gate,up,down}_proj.{weight,scales,biases}`,
shared expert `mlp.shared_expert.*`, router `mlp.gate`, shared gate `mlp.shared_expert_gate`).

Published Qwen MLX builds quantise `mlp.gate` and `mlp.shared_expert_gate` to 8 bits
(`Qwen35MoeConfig.swift:340-342`: `.weight` U32 words, `.scales` and `.biases` BF16, group 64);
they load as the layer's MLX-affine router (`hh_moe_weights.router_bits`, exact fp64 logits),
with the bit width read from the word count. A checkpoint that stores them as BF16 loads as a
bf16 router.
"""
from __future__ import annotations

import ctypes as C
import glob
import json
import os
import struct

import numpy as np
import torch

from . import formats as F
from ._lib import check, desc_c, lib
from .layer import Context, MoELayer

_ITEM = {"U8": 1, "I8": 1, "BF16": 2, "F16": 2, "U16": 2, "I16": 2, "F32": 4, "U32": 4,
         "I32": 4, "F64": 8, "I64": 8, "U64": 8, "BOOL": 1}


class CheckpointError(ValueError):
    """A tensor is missing, or its dtype or shape is not what the layer description implies."""


class SafetensorsFile:
    """One .safetensors file: the JSON header (8-byte little-endian length, then the header),
    and the data section mapped read-only."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            header = json.loads(f.read(n))
        self.meta = header.pop("__metadata__", None)
        self.entries = header
        self._base = 8 + n
        self._map = None

    def names(self):
        return list(self.entries)

    def tensor(self, name: str):
        """(dtype, shape, uint8 view of the tensor's bytes)."""
        e = self.entries[name]
        lo, hi = e["data_offsets"]
        shape = tuple(int(v) for v in e["shape"])
        if hi - lo != int(np.prod(shape, dtype=np.int64)) * _ITEM[e["dtype"]]:
            raise CheckpointError(f"{self.path}: {name}: byte range does not match its shape")
        if self._map is None:
            self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        return e["dtype"], shape, self._map[self._base + lo:self._base + hi]


class Checkpoint:
    """A checkpoint directory (or one file): tensor name → the file that holds it."""

    def __init__(self, path: str):
        if os.path.isdir(path):
            index = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index) as f:
                    wm = json.load(f)["weight_map"]
                files = sorted(set(wm.values()))
                self.files = {fn: SafetensorsFile(os.path.join(path, fn)) for fn in files}
                self.where = {k: self.files[v] for k, v in wm.items()}
            else:
                paths = sorted(glob.glob(os.path.join(path, "*.safetensors")))
                self.files = {os.path.basename(p): SafetensorsFile(p) for p in paths}
                self.where = {n: f for f in self.files.values() for n in f.names()}
        else:
            f = SafetensorsFile(path)
            self.files = {os.path.basename(path): f}
            self.where = {n: f for n in f.names()}

    def __contains__(self, name):
        return name in self.where

    def tensor(self, name: str, dtype: str, shape: tuple):
        """The bytes of `name`, checked against the expected dtype and shape."""
        if name not in self.where:
            raise CheckpointError(f"missing tensor {name}")
        dt, sh, data = self.where[name].tensor(name)
        if dt != dtype or sh != tuple(shape):
            raise CheckpointError(f"{name}: {dt}{list(sh)}, expected {dtype}{list(shape)}")
        return data


# ---- per-family tensor maps ------------------------------------------------------------------

def expert_sources(desc: F.MoEDesc, family: str, layer: int, shared: bool = False):
    """[(blob slot, tensor name, dtype, shape)] of the layer's stacked expert tensors, in blob
    slot order, or of the shared expert's tensors (Qwen, `shared=True`: no expert axis)."""
    H, E = desc.hidden, desc.experts
    I = desc.shared_intermediate if shared else desc.intermediate
    lead = () if shared else (E,)
    if family == "gpt-oss":
        if desc.quant != F.QUANT_MXFP4 or shared:
            raise CheckpointError("gpt-oss checkpoints hold MXFP4 routed experts")
        p = f"model.layers.{layer}.mlp.experts"
        spec = [("gate_up_proj_blocks", "U8", (2 * I, H // 32, 16)),
                ("gate_up_proj_scales", "U8", (2 * I, H // 32)),
                ("gate_up_proj_bias", "BF16", (2 * I,)),
                ("down_proj_blocks", "U8", (H, I // 32, 16)),
                ("down_proj_scales", "U8", (H, I // 32)),
                ("down_proj_bias", "BF16", (H,))]
    elif family == "gemma4":
        if desc.quant != F.QUANT_BF16 or shared:
            raise CheckpointError("gemma4 checkpoints hold BF16 routed experts")
        p = f"model.language_model.layers.{layer}.experts"
        spec = [("gate_up_proj", "BF16", (2 * I, H)), ("down_proj", "BF16", (H, I))]
    elif family == "qwen3.5-moe":
        if desc.quant not in (F.QUANT_MLX4, F.QUANT_MLX8):
            raise CheckpointError("qwen3.5-moe checkpoints hold MLX affine experts")
        vpw, g = 32 // desc.bits, desc.group_size
        p = f"language_model.model.layers.{layer}.mlp." + ("shared_expert" if shared else "switch_mlp")
        spec = []
        for proj, (rows, cols) in [("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))]:
            spec += [(f"{proj}.weight", "U32", (rows, cols // vpw)),
                     (f"{proj}.scales", "BF16", (rows, cols // g)),
                     (f"{proj}.biases", "BF16", (rows, cols // g))]
    else:
        raise CheckpointError(f"unknown family {family!r} (gpt-oss, gemma4, qwen3.5-moe)")
    return [(slot, f"{p}.{suffix}", dt, lead + shape) for slot, (suffix, dt, shape) in enumerate(spec)]


def router_sources(desc: F.MoEDesc, family: str, layer: int, router_bits: int = 0):
    """{MoELayer tensor key: (tensor name, dtype, shape, required)}; `router_bits` 4 or 8 names
    Qwen's MLX-affine router and shared-gate tensors instead of bf16 ones."""
    H, E = desc.hidden, desc.experts
    if family == "gpt-oss":
        p = f"model.layers.{layer}.mlp.router"
        return {"router_weight": (f"{p}.weight", "BF16", (E, H), True),
                "router_bias": (f"{p}.bias", "BF16", (E,), bool(desc.expert_bias))}
    if family == "gemma4":
        p = f"model.language_model.layers.{layer}.router"
        return {"router_weight": (f"{p}.proj.weight", "BF16", (E, H), True),
                "router_scale": (f"{p}.scale", "BF16", (H,), True),
                "router_expert_scale": (f"{p}.per_expert_scale", "BF16", (E,), True)}
    if family == "qwen3.5-moe":
        p = f"language_model.model.layers.{layer}.mlp"
        if router_bits:
            out = {}
            for key, stem, rows in [("router", f"{p}.gate", E), ("shared_gate", f"{p}.shared_expert_gate", 1)]:
                if key == "shared_gate" and not desc.shared_intermediate:
                    continue
                out[f"{key}_words"] = (f"{stem}.weight", "U32", (rows, H * router_bits // 32), True)
                out[f"{key}_scales"] = (f"{stem}.scales", "BF16", (rows, H // 64), True)
                out[f"{key}_biases"] = (f"{stem}.biases", "BF16", (rows, H // 64), True)
            return out
        out = {"router_weight": (f"{p}.gate.weight", "BF16", (E, H), True)}
        if desc.shared_intermediate:
            out["shared_gate"] = (f"{p}.shared_expert_gate.weight", "BF16", (1, H), True)
        return out
    raise CheckpointError(f"unknown family {family!r}")


def _quantised_router_bits(ck: Checkpoint, desc: F.MoEDesc, family: str, layer: int) -> int:
    """The MLX bit width of the layer's router tensor, 0 when it is stored as bf16."""
    name = router_sources(desc, family, layer)["router_weight"][0]
    stem = name[:-len(".weight")]
    if name not in ck or ck.where[name].entries[name]["dtype"] != "U32" or f"{stem}.scales" not in ck:
        return 0
    if family != "qwen3.5-moe":
        raise CheckpointError(f"{name} is MLX-quantised; only Qwen layers take an MLX router")
    words = ck.where[name].entries[name]["shape"][-1]
    bits = words * 32 // desc.hidden
    if bits not in (4, 8) or words * 32 != bits * desc.hidden:
        raise CheckpointError(f"{name}: {words} words per row of {desc.hidden} is neither 4- nor 8-bit")
    return bits


def load_moe_layer(path_or_ckpt, desc: F.MoEDesc, family: str, layer: int,
                   ctx: Context | None = None, device: int = 0) -> MoELayer:
    """The MoE half of decoder layer `layer` of a checkpoint, resident in HBM in the reference's
    expert blob layout. Checks every tensor's dtype and shape against `desc` first."""
    ck = path_or_ckpt if isinstance(path_or_ckpt, Checkpoint) else Checkpoint(path_or_ckpt)
    routed = expert_sources(desc, family, layer)
    shared = expert_sources(desc, family, layer, shared=True) if desc.shared_intermediate else []
    router_bits = _quantised_router_bits(ck, desc, family, layer)
    routers = router_sources(desc, family, layer, router_bits)
    # Every tensor is checked before any device memory is touched.
    routed_data = [(slot, ck.tensor(n, dt, sh)) for slot, n, dt, sh in routed]
    shared_data = [(slot, ck.tensor(n, dt, sh)) for slot, n, dt, sh in shared]
    router_data = {k: ck.tensor(n, dt, sh) for k, (n, dt, sh, req) in routers.items()
                   if req or n in ck}

    ctx = ctx or Context(device)
    dev = torch.device(f"cuda:{ctx.device}")
    d = desc_c(desc)
    lay = F.blob_layout(desc)
    torch.cuda.synchronize(dev)
    experts = torch.zeros((desc.experts, lay.stride), dtype=torch.uint8, device=dev)
    for slot, data in routed_data:
        check(lib().hh_scatter_expert_tensor(ctx.handle, C.byref(d), desc.intermediate, slot,
                                             desc.experts, C.c_void_p(data.ctypes.data),
                                             data.nbytes, C.c_void_p(experts.data_ptr()),
                                             lay.stride))
    tensors = {}
    if shared_data:
        slay = F.blob_layout(desc, desc.shared_intermediate)
        blob = torch.zeros((slay.stride,), dtype=torch.uint8, device=dev)
        for slot, data in shared_data:
            check(lib().hh_scatter_expert_tensor(ctx.handle, C.byref(d), desc.shared_intermediate,
                                                 slot, 1, C.c_void_p(data.ctypes.data),
                                                 data.nbytes, C.c_void_p(blob.data_ptr()),
                                                 slay.stride))
        tensors["shared_expert"] = blob
    for key, data in router_data.items():
        a = np.array(data)
        a = a.view(np.int32) if key.endswith("_words") else a.view(np.int16)
        tensors[key] = torch.from_numpy(a).to(dev)
    torch.cuda.synchronize(dev)
    return MoELayer.resident(desc, experts, lay.stride, tensors, ctx, router_bits=router_bits)


# ---- .hydra installations ----------------------------------------------------------------------
# A .hydra directory (HydraLayout.swift:4-20): manifest.json (format "hydra/1", the model's
# counts, the expert stride; Manifest.swift:9-80), resident.bin (the resident tensors in the
# model's declared order, each at a 256-byte aligned offset, HydraLayout.swift:52-70),
# experts/layer_NN.bin (E expert blobs at the blob stride, RepackPlan.swift:21, the exact bytes the
# kernels read).

HYDRA_FORMAT = "hydra/1"      # HydraManifest.currentFormat (Manifest.swift:13)


def hydra_manifest(path: str) -> dict:
    with open(os.path.join(path, "manifest.json")) as f:
        m = json.load(f)
    if m.get("format") != HYDRA_FORMAT:
        raise CheckpointError(f"{path}: manifest format {m.get('format')!r}, expected {HYDRA_FORMAT!r}")
    return m


def gpt_oss_resident_tensors(hidden: int, experts: int, layers: int, heads: int = 64,
                             head_dim: int = 64, kv_heads: int = 8):
    """GPT-OSS's resident tensor list in declaration order, (name, bytes), for layers
    0..layers-1 (GptOssConfig.residentTensorNames, GptOssConfig.swift:148-166; all BF16)."""
    q, kv = heads * head_dim, kv_heads * head_dim
    out = []
    for l in range(layers):
        p = f"model.layers.{l}"
        out += [(f"{p}.input_layernorm.weight", 2 * hidden),
                (f"{p}.self_attn.q_proj.weight", 2 * q * hidden), (f"{p}.self_attn.q_proj.bias", 2 * q),
                (f"{p}.self_attn.k_proj.weight", 2 * kv * hidden), (f"{p}.self_attn.k_proj.bias", 2 * kv),
                (f"{p}.self_attn.v_proj.weight", 2 * kv * hidden), (f"{p}.self_attn.v_proj.bias", 2 * kv),
                (f"{p}.self_attn.o_proj.weight", 2 * hidden * q), (f"{p}.self_attn.o_proj.bias", 2 * hidden),
                (f"{p}.self_attn.sinks", 2 * heads),
                (f"{p}.post_attention_layernorm.weight", 2 * hidden),
                (f"{p}.mlp.router.weight", 2 * experts * hidden), (f"{p}.mlp.router.bias", 2 * experts)]
    return out


def gemma4_resident_tensors(hidden: int = 2816, experts: int = 128, layers: int = 30,
                            intermediate: int = 2112, heads: int = 16, sliding_head_dim: int = 256,
                            sliding_kv_heads: int = 8, global_head_dim: int = 512,
                            global_kv_heads: int = 2, vocab: int = 262_144,
                            key_equals_value: bool = True):
    """Gemma 4's resident tensor list in placement order, (name, bytes), all BF16: per layer
    (Gemma4Config.residentTensors(atLayer:), Gemma4Config.swift:175-215) the attention with the
    geometry of its pattern (every sixth layer full: head_dim 512 and 2 kv heads, no v_proj when
    K equals V; the others sliding), the dense MLP, the expert branch's norms and router; then
    the final norm and the tied embedding (Gemma4Config.swift:218-225). Defaults: 26B-A4B."""
    out = []
    for l in range(layers):
        p = f"model.language_model.layers.{l}"
        full = (l + 1) % 6 == 0
        hd, kv = (global_head_dim, global_kv_heads) if full else (sliding_head_dim, sliding_kv_heads)
        q, kvd = heads * hd, kv * hd
        out += [(f"{p}.input_layernorm.weight", 2 * hidden),
                (f"{p}.self_attn.q_proj.weight", 2 * q * hidden),
                (f"{p}.self_attn.q_norm.weight", 2 * hd),
                (f"{p}.self_attn.k_proj.weight", 2 * kvd * hidden),
                (f"{p}.self_attn.k_norm.weight", 2 * hd)]
        if not (key_equals_value and full):
            out.append((f"{p}.self_attn.v_proj.weight", 2 * kvd * hidden))
        out += [(f"{p}.self_attn.o_proj.weight", 2 * hidden * q),
                (f"{p}.post_attention_layernorm.weight", 2 * hidden),
                (f"{p}.pre_feedforward_layernorm.weight", 2 * hidden),
                (f"{p}.mlp.gate_proj.weight", 2 * intermediate * hidden),
                (f"{p}.mlp.up_proj.weight", 2 * intermediate * hidden),
                (f"{p}.mlp.down_proj.weight", 2 * hidden * intermediate),
                (f"{p}.post_feedforward_layernorm_1.weight", 2 * hidden),
                (f"{p}.pre_feedforward_layernorm_2.weight", 2 * hidden),
                (f"{p}.router.proj.weight", 2 * experts * hidden),
                (f"{p}.router.scale", 2 * hidden),
                (f"{p}.router.per_expert_scale", 2 * experts),
                (f"{p}.post_feedforward_layernorm_2.weight", 2 * hidden),
                (f"{p}.post_feedforward_layernorm.weight", 2 * hidden),
                (f"{p}.layer_scalar", 2)]
    out.append(("model.language_model.norm.weight", 2 * hidden))
    out.append(("model.language_model.embed_tokens.weight", 2 * vocab * hidden))
    return out


def _mlx_parts(stem: str, rows: int, cols: int, bits: int, group: int):
    """The three tensors of an MLX-affine matrix (MLXAffineLayout.swift:45-54): codes, then bf16
    scales and biases per group."""
    words = cols // (32 // bits)
    return [(f"{stem}.weight", rows * words * 4), (f"{stem}.scales", rows * (cols // group) * 2),
            (f"{stem}.biases", rows * (cols // group) * 2)]


def qwen35_resident_tensors(hidden: int = 2048, experts: int = 256, layers: int = 40,
                            vocab: int = 248_320, full_interval: int = 4, heads: int = 16,
                            kv_heads: int = 2, head_dim: int = 256, output_gate: bool = True,
                            lin_key_heads: int = 16, lin_value_heads: int = 32,
                            lin_key_dim: int = 128, lin_value_dim: int = 128, conv_kernel: int = 4,
                            shared_intermediate: int = 512, quant_bits: int = 4,
                            gate_bits: int = 8, group: int = 64):
    """Qwen3.5/3.6-MoE's resident tensor list in placement order, (name, bytes)
    (Qwen35MoeConfig.residentTensors, Qwen35MoeConfig.swift:292-355): per layer the input norm,
    the attention (every `full_interval`-th layer) or the linear-attention block, the
    post-attention norm, the router and shared-expert gate (MLX `gate_bits`) and the shared
    expert (MLX `quant_bits`); then the final norm, the embedding and the untied head. Defaults:
    the published 35B-A3B 4-bit build."""
    out = []
    q, kvd = heads * head_dim, kv_heads * head_dim
    qrows = 2 * q if output_gate else q
    conv = 2 * lin_key_heads * lin_key_dim + lin_value_heads * lin_value_dim
    for l in range(layers):
        p = f"language_model.model.layers.{l}"
        out.append((f"{p}.input_layernorm.weight", 2 * hidden))
        if (l + 1) % full_interval == 0:
            out += _mlx_parts(f"{p}.self_attn.q_proj", qrows, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.self_attn.k_proj", kvd, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.self_attn.v_proj", kvd, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.self_attn.o_proj", hidden, q, quant_bits, group)
            out += [(f"{p}.self_attn.q_norm.weight", 2 * head_dim),
                    (f"{p}.self_attn.k_norm.weight", 2 * head_dim)]
        else:
            vd = lin_value_heads * lin_value_dim
            out += _mlx_parts(f"{p}.linear_attn.in_proj_qkv", conv, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.linear_attn.in_proj_z", vd, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.linear_attn.in_proj_b", lin_value_heads, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.linear_attn.in_proj_a", lin_value_heads, hidden, quant_bits, group)
            out += _mlx_parts(f"{p}.linear_attn.out_proj", hidden, vd, quant_bits, group)
            out += [(f"{p}.linear_attn.conv1d.weight", 2 * conv * conv_kernel),
                    (f"{p}.linear_attn.A_log", 2 * lin_value_heads),
                    (f"{p}.linear_attn.dt_bias", 2 * lin_value_heads),
                    (f"{p}.linear_attn.norm.weight", 2 * lin_value_dim)]
        out.append((f"{p}.post_attention_layernorm.weight", 2 * hidden))
        out += _mlx_parts(f"{p}.mlp.gate", experts, hidden, gate_bits, group)
        out += _mlx_parts(f"{p}.mlp.shared_expert_gate", 1, hidden, gate_bits, group)
        for part in ("gate_proj", "up_proj"):
            out += _mlx_parts(f"{p}.mlp.shared_expert.{part}", shared_intermediate, hidden, quant_bits, group)
        out += _mlx_parts(f"{p}.mlp.shared_expert.down_proj", hidden, shared_intermediate, quant_bits, group)
    out.append(("language_model.model.norm.weight", 2 * hidden))
    out += _mlx_parts("language_model.model.embed_tokens", vocab, hidden, quant_bits, group)
    out += _mlx_parts("language_model.lm_head", vocab, hidden, quant_bits, group)
    return out


def resident_placements(tensors):
    """{name: (offset, bytes)}: each tensor at the next 256-byte aligned offset, in order
    (HydraLayout.init, HydraLayout.swift:52-70)."""
    out, cursor = {}, 0
    for name, nbytes in tensors:
        cursor = F._align(cursor, F.TENSOR_ALIGNMENT)
        out[name] = (cursor, nbytes)
        cursor += nbytes
    return out


def family_resident_tensors(family: str, model: dict, desc: F.MoEDesc, dims: dict | None = None):
    """The resident tensor list of a .hydra installation of `family`, from the manifest's model
    counts (layers, hidden size, experts, vocabulary) and `dims`: the family function's other
    keyword arguments (attention geometry and so on; omitted ones take the published model's)."""
    dims = dict(dims or {})
    L, H, E = model["layerCount"], desc.hidden, desc.experts
    if family == "gpt-oss":
        return gpt_oss_resident_tensors(H, E, L, **dims)
    if family == "gemma4":
        dims.setdefault("vocab", model.get("vocabSize", 262_144))
        return gemma4_resident_tensors(hidden=H, experts=E, layers=L, **dims)
    if family == "qwen3.5-moe":
        dims.setdefault("vocab", model.get("vocabSize", 248_320))
        dims.setdefault("quant_bits", desc.bits)
        dims.setdefault("shared_intermediate", desc.shared_intermediate)
        dims.setdefault("group", desc.group_size)
        return qwen35_resident_tensors(hidden=H, experts=E, layers=L, **dims)
    raise CheckpointError(f"unknown family {family!r} (gpt-oss, gemma4, qwen3.5-moe)")


def load_hydra_layer(path: str, desc: F.MoEDesc, family: str, layer: int,
                     ctx: Context | None = None, device: int = 0, router_checkpoint=None,
                     attention=(64, 64, 8), resident_dims: dict | None = None) -> MoELayer:
    """The MoE half of layer `layer` of a .hydra installation, resident in HBM. The experts come
    from experts/layer_NN.bin as they are (checked against the manifest's count and stride and
    this build's blob layout). The router tensors (Qwen: also the shared expert and its gate)
    come from resident.bin at their placements in the family's resident order
    (HydraLayout.swift:52-70; GptOssConfig.swift:148-166, Gemma4Config.swift:175-225,
    Qwen35MoeConfig.swift:292-355), the model's shape from the manifest and `resident_dims`
    (GPT-OSS: `attention` = (heads, head_dim, kv_heads)); or, when `router_checkpoint` (a
    safetensors checkpoint or directory) is given, from that checkpoint, as load_moe_layer reads
    them."""
    m = hydra_manifest(path)
    model, lay_m = m["model"], m["layout"]
    lay = F.blob_layout(desc)
    if model["expertCount"] != desc.experts or model["hiddenSize"] != desc.hidden:
        raise CheckpointError(f"{path}: manifest has {model['expertCount']} experts of hidden "
                              f"{model['hiddenSize']}, the description {desc.experts} / {desc.hidden}")
    if lay_m["expertStrideBytes"] != lay.stride or lay_m["expertPayloadBytes"] != lay.payload:
        raise CheckpointError(f"{path}: expert stride/payload {lay_m['expertStrideBytes']}/"
                              f"{lay_m['expertPayloadBytes']} differ from the blob layout {lay.stride}/{lay.payload}")
    if not 0 <= layer < model["layerCount"]:
        raise CheckpointError(f"{path}: no layer {layer} (layerCount {model['layerCount']})")
    fn = os.path.join(path, "experts", f"layer_{layer:02d}.bin")
    if not os.path.exists(fn) or os.path.getsize(fn) != desc.experts * lay.stride:
        raise CheckpointError(f"{fn}: missing or not {desc.experts} blobs of {lay.stride} bytes")
    blobs = np.memmap(fn, dtype=np.uint8, mode="r", shape=(desc.experts, lay.stride))
    router_bits = 0
    if router_checkpoint is not None:
        ck = router_checkpoint if isinstance(router_checkpoint, Checkpoint) else Checkpoint(router_checkpoint)
        router_bits = _quantised_router_bits(ck, desc, family, layer)

        def fetch(name, dt, shape):
            return np.array(ck.tensor(name, dt, shape))

        def present(name):
            return name in ck
    else:
        dims = dict(resident_dims or {})
        if family == "gpt-oss":
            heads, head_dim, kv_heads = attention
            dims.update(heads=heads, head_dim=head_dim, kv_heads=kv_heads)
        place = resident_placements(family_resident_tensors(family, model, desc, dims))
        rfn = os.path.join(path, "resident.bin")
        res = np.memmap(rfn, dtype=np.uint8, mode="r")
        if family == "qwen3.5-moe":
            router_bits = dims.get("gate_bits", 8)
        npdt = {"BF16": np.uint16, "U32": np.uint32, "U8": np.uint8}

        def fetch(name, dt, shape):
            if name not in place:
                raise CheckpointError(f"{rfn}: no resident placement for {name}")
            off, nb = place[name]
            want = int(np.prod(shape)) * np.dtype(npdt[dt]).itemsize
            if nb != want:
                raise CheckpointError(f"{name}: {nb} resident bytes, the description needs {want}")
            if off + nb > res.size:
                raise CheckpointError(f"{rfn}: shorter than the placement of {name}")
            return np.array(res[off:off + nb]).view(npdt[dt]).reshape(shape)

        def present(name):
            return name in place
    tensors = {}
    for key, (name, dt, shape, req) in router_sources(desc, family, layer, router_bits).items():
        if req or present(name):
            tensors[key] = fetch(name, dt, shape)
    ctx = ctx or Context(device)
    dev = torch.device(f"cuda:{ctx.device}")
    torch.cuda.synchronize(dev)
    experts = torch.from_numpy(np.array(blobs)).to(dev)
    dt = {}
    for key, data in tensors.items():
        a = np.ascontiguousarray(data)
        if key.endswith("_words"):
            a = a.view(np.int32)
        elif a.dtype in (np.uint8, np.uint16):
            a = a.view(np.int16)
        dt[key] = torch.from_numpy(a.copy()).to(dev)
    if desc.shared_intermediate:
        slay = F.blob_layout(desc, desc.shared_intermediate)
        blob = np.zeros(slay.stride, np.uint8)
        for slot, name, dtn, shape in expert_sources(desc, family, layer, shared=True):
            blob[slay.offsets[slot]:slay.offsets[slot] + slay.sizes[slot]] = \
                np.asarray(fetch(name, dtn, shape)).view(np.uint8).reshape(-1)
        dt["shared_expert"] = torch.from_numpy(blob).to(dev)
    torch.cuda.synchronize(dev)
    return MoELayer.resident(desc, experts, lay.stride, dt, ctx, router_bits=router_bits)
