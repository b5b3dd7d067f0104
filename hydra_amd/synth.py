"""Deterministic synthetic layers and inputs, identical wherever they are generated.

One generator for CPU and GPU runs:
  * a splitmix64 stream per (seed, tensor name): state_i = key + i·γ, out = mix(state_i);
  * uniform doubles from the top 53 bits;
  * normals by Box–Muller over consecutive pairs;
  * rounding to bf16 by round-to-nearest-even (BF16.swift:27-31).

The value distributions are those of the benchmark configurations: MXFP4 nibbles uniform over
the 16 codes, e8m0 scale bytes uniform over 119..123 (2^-8..2^-4), biases bf16 N(0, 0.02),
router bf16 N(0, 1/√H) (so the logits are ≈ N(0, 1)), inputs bf16 N(0, 1).
"""
from __future__ import annotations

import hashlib

import numpy as np

from . import formats as F

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _key(seed: int, name: str) -> np.uint64:
    h = int.from_bytes(hashlib.sha256(f"{seed}/{name}".encode()).digest()[:8], "little")
    return np.uint64(h)


def u64(seed: int, name: str, n: int) -> np.ndarray:
    """n raw 64-bit draws of the (seed, name) stream."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(_key(seed, name) + i * _GAMMA)


def uniform(seed: int, name: str, n: int) -> np.ndarray:
    return (u64(seed, name, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, name: str, n: int) -> np.ndarray:
    m = (n + 1) // 2
    u = uniform(seed, name, 2 * m)
    u1, u2 = 1.0 - u[0::2], u[1::2]          # u1 in (0, 1]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * m)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:n]


def random_bytes(seed: int, name: str, n: int) -> np.ndarray:
    return u64(seed, name, (n + 7) // 8).view(np.uint8)[:n].copy()


def f32_to_bf16(a) -> np.ndarray:
    """Round-to-nearest-even float32 → bf16 bits, NaN quieted (BF16.fromFloat)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32)
    rounded = ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1)))
               >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        rounded[nan] = ((bits[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return rounded


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_normal(seed: int, name: str, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    return f32_to_bf16((mean + std * normal(seed, name, n)).astype(np.float32))


# ---- layers ----------------------------------------------------------------------------------

def _expert_tensors(desc: F.MoEDesc, seed: int, prefix: str, count: int, inter: int):
    """The source tensors of `count` experts, per blob slot, as uint8 arrays [count, bytes]."""
    lay = F.blob_layout(desc, inter)
    H, I = desc.hidden, inter
    out = []
    if desc.quant == F.QUANT_MXFP4:
        names = ["gate_up_blocks", "gate_up_scales", "gate_up_bias",
                 "down_blocks", "down_scales", "down_bias"]
        for slot, (name, size) in enumerate(zip(names, lay.sizes)):
            n = count * size
            if name.endswith("blocks"):
                data = random_bytes(seed, f"{prefix}/{name}", n)       # uniform nibbles
            elif name.endswith("scales"):
                data = (np.uint8(119) + (u64(seed, f"{prefix}/{name}", n) % np.uint64(5))
                        .astype(np.uint8))                             # 2^-8 .. 2^-4
            else:
                data = bf16_normal(seed, f"{prefix}/{name}", n // 2, 0.0, 0.02).view(np.uint8)
            out.append(data.reshape(count, size))
    elif desc.quant == F.QUANT_BF16:
        for name, size in zip(["gate_up", "down"], lay.sizes):
            data = bf16_normal(seed, f"{prefix}/{name}", count * size // 2, 0.0, 0.02)
            out.append(data.view(np.uint8).reshape(count, size))
    else:
        bits = desc.bits
        centre = 7.5 if bits == 4 else 127.5
        for mat in ["gate", "up", "down"]:
            rows, cols = (I, H) if mat != "down" else (H, I)
            nw = count * rows * cols * bits // 32
            words = random_bytes(seed, f"{prefix}/{mat}_words", nw * 4)
            ng = count * rows * cols // desc.group_size
            scales = bf16_normal(seed, f"{prefix}/{mat}_scales", ng, 0.01, 0.002)
            # Group bias −centre·scale centres the dequantised values on zero.
            biases = f32_to_bf16(-centre * bf16_to_f32(scales))
            out += [words.reshape(count, -1), scales.view(np.uint8).reshape(count, -1),
                    biases.view(np.uint8).reshape(count, -1)]
    return lay, out


def pack_blobs(lay: F.BlobLayout, tensors) -> np.ndarray:
    count = tensors[0].shape[0]
    blobs = np.zeros((count, lay.stride), dtype=np.uint8)
    for off, size, t in zip(lay.offsets, lay.sizes, tensors):
        assert t.shape == (count, size), (t.shape, size)
        blobs[:, off:off + size] = t
    return blobs


def zipf_router_bias(seed: int, experts: int, s: float = 1.1) -> np.ndarray:
    """Per-expert logit bias log(w_rank) with Zipf(s) rank weights over a seeded permutation:
    bias_e = −s·ln(1 + rank(e)). Skews the top-k load as a Zipf law."""
    rank = np.argsort(np.argsort(uniform(seed, "zipf_perm", experts)))
    return f32_to_bf16((-s * np.log1p(rank)).astype(np.float32))


def mlx_router_rows(seed: int, name: str, rows: int, hidden: int, bits: int):
    """An MLX-affine router matrix [rows][hidden] (group 64): uniform codes, scales chosen so
    the dequantised rows have std ≈ 1/√H (logits ≈ N(0, 1) for N(0, 1) inputs), group biases
    −centre·scale. Returns (words uint32 [rows][H·bits/32], scales, biases bf16 [rows][H/64])."""
    centre = 7.5 if bits == 4 else 127.5
    code_std = (2 ** bits - 1) / np.sqrt(12.0)
    nw = rows * hidden * bits // 32
    words = random_bytes(seed, f"{name}_words", nw * 4).view(np.uint32).reshape(rows, -1)
    ng = rows * hidden // 64
    s0 = 1.0 / (np.sqrt(hidden) * code_std)
    scales = f32_to_bf16(np.abs(s0 + 0.2 * s0 * normal(seed, f"{name}_scales", ng)).astype(np.float32))
    biases = f32_to_bf16(-centre * bf16_to_f32(scales))
    return words, scales.reshape(rows, -1), biases.reshape(rows, -1)


def make_layer(desc: F.MoEDesc, seed: int = 0, zipf: float | None = None,
               router_bits: int = 0) -> dict:
    """Synthetic weights of one layer as host arrays, in the reference blob layout. With
    `router_bits` 4 or 8 the router (and shared gate) are MLX-affine matrices, as Qwen's
    published builds store mlp.gate and mlp.shared_expert_gate (Qwen35MoeConfig.swift:340-342)."""
    H, E = desc.hidden, desc.experts
    lay, tens = _expert_tensors(desc, seed, "experts", E, desc.intermediate)
    layer = {"desc": desc, "layout": lay, "experts": pack_blobs(lay, tens)}
    if desc.shared_intermediate:
        slay, stens = _expert_tensors(desc, seed, "shared", 1, desc.shared_intermediate)
        layer["shared_expert"] = pack_blobs(slay, stens)[0]
        layer["shared_gate"] = bf16_normal(seed, "shared_gate", H, 0.0, 1.0 / np.sqrt(H))
    if router_bits:
        assert desc.router != F.ROUTER_GEMMA, "the GEMMA router takes a bf16 projection"
        layer["router_bits"] = router_bits
        (layer["router_words"], layer["router_scales"],
         layer["router_biases"]) = mlx_router_rows(seed, "router", E, H, router_bits)
        if desc.shared_intermediate:
            del layer["shared_gate"]
            (layer["shared_gate_words"], layer["shared_gate_scales"],
             layer["shared_gate_biases"]) = mlx_router_rows(seed, "shared_gate", 1, H, router_bits)
        if desc.expert_bias:
            layer["router_bias"] = bf16_normal(seed, "router_bias", E, 0.0, 0.02)
        return layer
    if desc.router == F.ROUTER_GEMMA:
        # Unit router scales: the normalised input has unit rms, so N(0, 1) projection rows
        # give ≈ N(0, 1) logits after the H^-½ factor.
        layer["router_weight"] = bf16_normal(seed, "router", E * H, 0.0, 1.0).reshape(E, H)
        layer["router_scale"] = f32_to_bf16(np.ones(H, np.float32))
        layer["router_expert_scale"] = f32_to_bf16(np.ones(E, np.float32))
    else:
        layer["router_weight"] = bf16_normal(seed, "router", E * H, 0.0,
                                             1.0 / np.sqrt(H)).reshape(E, H)
        if desc.expert_bias:
            layer["router_bias"] = (zipf_router_bias(seed, E, zipf) if zipf
                                    else bf16_normal(seed, "router_bias", E, 0.0, 0.02))
    return layer


def make_tokens(hidden: int, tokens: int, seed: int = 0, name: str = "x") -> np.ndarray:
    """Input hidden states, bf16 N(0, 1) [T][H]."""
    return bf16_normal(seed, name, tokens * hidden).reshape(tokens, hidden)
