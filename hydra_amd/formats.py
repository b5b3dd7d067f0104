"""Layer descriptions and expert blob layouts of the MoE hot path.

Mirrors, for the hot path only, HydraCore's model configs (GptOssConfig.swift:60-86,
Qwen35MoeConfig.swift:73-136, Gemma4Config.swift:73-77) and its expert blob layouts
(ExpertBlobLayout.swift:78-103 MXFP4, :127-143 BF16, :193-223 MLX affine). The numeric
enum values are the ones of include/hydra_hip.h.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass

QUANT_MXFP4, QUANT_MLX4, QUANT_MLX8, QUANT_BF16 = 0, 1, 2, 3
ACT_SWIGLU_OAI, ACT_SILU, ACT_GELU_TANH = 0, 1, 2
ROUTER_TOPK_SOFTMAX, ROUTER_SOFTMAX_TOPK_RENORM, ROUTER_GEMMA = 0, 1, 2

TENSOR_ALIGNMENT = 256      # ExpertBlobLayout.tensorAlignment (ExpertBlobLayout.swift:48)
PAGE_ALIGNMENT = 16384      # ExpertBlobLayout.pageAlignment (ExpertBlobLayout.swift:38)
MAX_TOP_K = 8               # ForwardEncoder.maxRouterTopK (ForwardEncoder.swift:133)


@dataclass(frozen=True)
class MoEDesc:
    """One MoE layer's shape and conventions (the C struct hh_moe_desc)."""
    hidden: int
    intermediate: int
    experts: int
    top_k: int
    quant: int
    activation: int
    router: int
    shared_intermediate: int = 0
    group_size: int = 64
    expert_bias: int = 0
    swiglu_alpha: float = 1.702
    swiglu_limit: float = 7.0
    router_eps: float = 1e-6

    def replace(self, **kw) -> "MoEDesc":
        return dataclasses.replace(self, **kw)

    @property
    def bits(self) -> int:
        return {QUANT_MLX4: 4, QUANT_MLX8: 8}.get(self.quant, 0)


def _align(v: int, a: int) -> int:
    r = v % a
    return v if r == 0 else v + (a - r)


@dataclass(frozen=True)
class BlobLayout:
    offsets: tuple
    sizes: tuple
    payload: int
    stride: int


def blob_layout(desc: MoEDesc, intermediate: int | None = None) -> BlobLayout:
    """Sub-tensor offsets of one expert blob, in the reference's consumption order."""
    H = desc.hidden
    I = desc.intermediate if intermediate is None else intermediate
    if desc.quant == QUANT_MXFP4:
        sizes = [2 * I * (H // 32) * 16, 2 * I * (H // 32), 2 * I * 2,
                 H * (I // 32) * 16, H * (I // 32), H * 2]
    elif desc.quant == QUANT_BF16:
        sizes = [2 * I * H * 2, H * I * 2]
    else:
        vpw = 32 // desc.bits
        g = desc.group_size
        gw, gs = I * (H // vpw) * 4, I * (H // g) * 2
        dw, ds = H * (I // vpw) * 4, H * (I // g) * 2
        sizes = [gw, gs, gs, gw, gs, gs, dw, ds, ds]
    offsets, cursor = [], 0
    for s in sizes:
        cursor = _align(cursor, TENSOR_ALIGNMENT)
        offsets.append(cursor)
        cursor += s
    return BlobLayout(tuple(offsets), tuple(sizes), cursor, _align(cursor, PAGE_ALIGNMENT))


def expert_bytes(desc: MoEDesc, intermediate: int | None = None) -> int:
    """Bytes of one expert's source tensors (no padding): the algorithmic bytes an expert
    product streams."""
    return sum(blob_layout(desc, intermediate).sizes)


def streamed_expert_bytes(desc: MoEDesc, intermediate: int | None = None) -> int:
    """Bytes the expert products read for one expert: the source tensors minus any bias slots
    the layer does not use."""
    lay = blob_layout(desc, intermediate)
    total = sum(lay.sizes)
    if desc.quant == QUANT_MXFP4 and not desc.expert_bias:
        total -= lay.sizes[2] + lay.sizes[5]
    return total


# ---- named configurations --------------------------------------------

GPT_OSS_20B = MoEDesc(hidden=2880, intermediate=2880, experts=32, top_k=4, quant=QUANT_MXFP4,
                      activation=ACT_SWIGLU_OAI, router=ROUTER_TOPK_SOFTMAX, expert_bias=1)
GPT_OSS_120B = GPT_OSS_20B.replace(experts=128)
QWEN_35B_A3B_Q4 = MoEDesc(hidden=2048, intermediate=512, experts=256, top_k=8,
                          quant=QUANT_MLX4, activation=ACT_SILU,
                          router=ROUTER_SOFTMAX_TOPK_RENORM, shared_intermediate=512,
                          group_size=64)
QWEN_35B_A3B_Q8 = QWEN_35B_A3B_Q4.replace(quant=QUANT_MLX8)
GEMMA_BF16 = MoEDesc(hidden=2816, intermediate=704, experts=128, top_k=8, quant=QUANT_BF16,
                     activation=ACT_GELU_TANH, router=ROUTER_GEMMA, router_eps=1e-6)

CONFIGS = {
    "gpt-oss-20b": GPT_OSS_20B,
    "gpt-oss-120b": GPT_OSS_120B,
    "qwen-35b-a3b-q4": QWEN_35B_A3B_Q4,
    "qwen-35b-a3b-q8": QWEN_35B_A3B_Q8,
    "gemma-bf16": GEMMA_BF16,
}
