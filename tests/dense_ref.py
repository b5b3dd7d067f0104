"""A second, independent fp64 formulation of the MoE layer for the tests.

Where the oracle (oracle/hh_oracle.c) walks rows in plain loops like HydraReference, this
module dequantises whole matrices with vectorised numpy and multiplies them with matmul, and
routes with lexsort. Agreement between the two pins the oracle's composition (dequant, blob
offsets, gate/up split, activation, routing, rank-ordered combine, shared expert) without
retyping its loops. Test infrastructure only.
"""
import numpy as np

from hydra_amd import formats as F

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def bf16(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits).view(np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def mxfp4_matrix(blocks, scales, rows, cols):
    b = np.frombuffer(blocks.tobytes(), np.uint8).reshape(rows, cols // 32, 16)
    vals = np.empty((rows, cols // 32, 32))
    vals[..., 0::2] = E2M1[b & 0x0F]
    vals[..., 1::2] = E2M1[b >> 4]
    s = np.frombuffer(scales.tobytes(), np.uint8).reshape(rows, cols // 32).astype(np.int64)
    return (vals * np.ldexp(1.0, s - 127)[..., None]).reshape(rows, cols)


def mlx_matrix(words, scales, biases, rows, cols, bits, group):
    w = np.frombuffer(words.tobytes(), np.uint32).reshape(rows, -1).astype(np.uint64)
    shifts = (np.arange(32 // bits) * bits).astype(np.uint64)
    q = ((w[..., None] >> shifts) & np.uint64((1 << bits) - 1)).reshape(rows, cols)
    s = np.repeat(bf16(scales).reshape(rows, cols // group), group, axis=1)
    bi = np.repeat(bf16(biases).reshape(rows, cols // group), group, axis=1)
    return q.astype(np.float64) * s + bi


def expert_matrices(desc, blob, inter):
    """(gate [I,H], up [I,H], down [H,I], gate_bias [I], up_bias [I], down_bias [H])."""
    lay = F.blob_layout(desc, inter)
    H, I = desc.hidden, inter
    sl = [blob[o:o + s] for o, s in zip(lay.offsets, lay.sizes)]
    zI, zH = np.zeros(I), np.zeros(H)
    if desc.quant == F.QUANT_MXFP4:
        gu = mxfp4_matrix(sl[0], sl[1], 2 * I, H)
        dn = mxfp4_matrix(sl[3], sl[4], H, I)
        if desc.expert_bias:
            gub, dnb = bf16(sl[2]), bf16(sl[5])
        else:
            gub, dnb = np.zeros(2 * I), zH
        return gu[0::2], gu[1::2], dn, gub[0::2], gub[1::2], dnb
    if desc.quant == F.QUANT_BF16:
        gu = bf16(sl[0]).reshape(2 * I, H)
        return gu[:I], gu[I:], bf16(sl[1]).reshape(H, I), zI, zI, zH
    bits, g = desc.bits, desc.group_size
    gate = mlx_matrix(sl[0], sl[1], sl[2], I, H, bits, g)
    up = mlx_matrix(sl[3], sl[4], sl[5], I, H, bits, g)
    dn = mlx_matrix(sl[6], sl[7], sl[8], H, I, bits, g)
    return gate, up, dn, zI, zI, zH


def activation(desc, g, u):
    if desc.activation == F.ACT_SWIGLU_OAI:
        g = np.minimum(g, desc.swiglu_limit)
        u = np.clip(u, -desc.swiglu_limit, desc.swiglu_limit)
        return g / (1.0 + np.exp(-desc.swiglu_alpha * g)) * (u + 1.0)
    if desc.activation == F.ACT_SILU:
        return g / (1.0 + np.exp(-g)) * u
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3))) * u


def expert_ffn(desc, blob, x, inter=None):
    inter = desc.intermediate if inter is None else inter
    gate, up, dn, gb, ub, db = expert_matrices(desc, blob, inter)
    a = activation(desc, gate @ x + gb, up @ x + ub)
    return dn @ a + db


def _topk(values, k):
    order = np.lexsort((np.arange(values.size), -values))
    return order[:k]


def route(desc, logits, per_expert_scale=None):
    k = desc.top_k
    if desc.router == F.ROUTER_TOPK_SOFTMAX:
        idx = _topk(logits, k)
        e = np.exp(logits[idx] - logits[idx].max())
        return idx, e / e.sum()
    p = np.exp(logits - logits.max())
    p /= p.sum()
    idx = _topk(p, k)
    w = p[idx] / p[idx].sum()
    if desc.router == F.ROUTER_GEMMA:
        w = w * per_expert_scale[idx]
    return idx, w


def logits(desc, layer, xr):
    W = bf16(layer["router_weight"]).reshape(desc.experts, desc.hidden)
    if desc.router == F.ROUTER_GEMMA:
        s = (np.mean(xr * xr) + desc.router_eps) ** -0.5
        v = xr * s * bf16(layer["router_scale"]) * desc.hidden ** -0.5
        return W @ v
    out = W @ xr
    if layer.get("router_bias") is not None:
        out = out + bf16(layer["router_bias"])
    return out


def moe_forward(layer, x_bf16, x_router=None):
    desc = layer["desc"]
    x = bf16(np.atleast_2d(x_bf16))
    xr_all = x if x_router is None else bf16(np.atleast_2d(x_router))
    T = x.shape[0]
    y = np.zeros((T, desc.hidden))
    idxs = np.zeros((T, desc.top_k), np.int64)
    ws = np.zeros((T, desc.top_k))
    pes = bf16(layer["router_expert_scale"]) if desc.router == F.ROUTER_GEMMA else None
    for t in range(T):
        idx, w = route(desc, logits(desc, layer, xr_all[t]), pes)
        idxs[t], ws[t] = idx, w
        for r in range(desc.top_k):
            y[t] += w[r] * expert_ffn(desc, layer["experts"][idx[r]], x[t])
        if desc.shared_intermediate:
            sc = 1.0 / (1.0 + np.exp(-(bf16(layer["shared_gate"]) @ x[t])))
            y[t] += sc * expert_ffn(desc, layer["shared_expert"], x[t], desc.shared_intermediate)
    return y, idxs, ws
