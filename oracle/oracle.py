"""ctypes front end of oracle/liboracle.so (fp64 restatement of HydraReference).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the cpu_baseline leg of
bench.py as the checker / CPU baseline. Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


class Desc(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("intermediate", C.c_int32), ("experts", C.c_int32),
                ("top_k", C.c_int32), ("shared_intermediate", C.c_int32), ("quant", C.c_int32),
                ("group_size", C.c_int32), ("activation", C.c_int32), ("router", C.c_int32),
                ("expert_bias", C.c_int32), ("swiglu_alpha", C.c_double),
                ("swiglu_limit", C.c_double), ("router_eps", C.c_double)]


class Weights(C.Structure):
    _fields_ = [("experts", C.c_void_p), ("expert_stride", C.c_size_t),
                ("shared_expert", C.c_void_p), ("router_weight", C.c_void_p),
                ("router_bias", C.c_void_p), ("router_scale", C.c_void_p),
                ("router_expert_scale", C.c_void_p), ("shared_gate", C.c_void_p),
                ("router_bits", C.c_int32), ("router_words", C.c_void_p),
                ("router_scales", C.c_void_p), ("router_biases", C.c_void_p),
                ("shared_gate_words", C.c_void_p), ("shared_gate_scales", C.c_void_p),
                ("shared_gate_biases", C.c_void_p)]


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _lib.hho_bf16_to_f32.restype = C.c_float
        _lib.hho_bf16_to_f32.argtypes = [C.c_uint16]
        _lib.hho_f32_to_bf16.restype = C.c_uint16
        _lib.hho_f32_to_bf16.argtypes = [C.c_float]
        _lib.hho_sigmoid.restype = C.c_double
        _lib.hho_sigmoid.argtypes = [C.c_double]
        _lib.hho_silu.restype = C.c_double
        _lib.hho_silu.argtypes = [C.c_double]
        _lib.hho_gelu_tanh.restype = C.c_double
        _lib.hho_gelu_tanh.argtypes = [C.c_double]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def to_desc(d) -> Desc:
    return Desc(d.hidden, d.intermediate, d.experts, d.top_k, d.shared_intermediate, d.quant,
                d.group_size, d.activation, d.router, d.expert_bias, d.swiglu_alpha,
                d.swiglu_limit, d.router_eps)


def bf16_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().hho_bf16_to_f32_array(_p(bits), _p(out), C.c_size_t(bits.size))
    return out


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().hho_f32_to_bf16_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def mxfp4_decode(packed, scales) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    assert packed.size == scales.size * 16
    out = np.empty(scales.size * 32, np.float32)
    lib().hho_mxfp4_decode(_p(packed), _p(scales), C.c_size_t(scales.size), _p(out))
    return out


def mlx_unpack(words, bits) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    out = np.empty(words.size * (32 // bits), np.int32)
    lib().hho_mlx_unpack(_p(words), C.c_size_t(words.size), C.c_int(bits), _p(out))
    return out


def mlx_dequant(words, scales, biases, cols, bits, group) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.float64)
    biases = np.ascontiguousarray(biases, dtype=np.float64)
    out = np.empty(cols, np.float64)
    lib().hho_mlx_dequant(_p(words), _p(scales), _p(biases), C.c_int(cols), C.c_int(bits),
                          C.c_int(group), _p(out))
    return out


def swiglu(row, alpha=1.702, limit=7.0) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.float64)
    out = np.empty(row.size // 2, np.float64)
    lib().hho_swiglu(_p(row), C.c_int(row.size // 2), C.c_double(alpha), C.c_double(limit),
                     _p(out))
    return out


def gelu_tanh(x: float) -> float:
    return lib().hho_gelu_tanh(float(x))


def silu(x: float) -> float:
    return lib().hho_silu(float(x))


def sigmoid(x: float) -> float:
    return lib().hho_sigmoid(float(x))


def _router(fn, logits, k):
    logits = np.ascontiguousarray(logits, dtype=np.float64)
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float64)
    fn(_p(logits), C.c_int(logits.size), C.c_int(k), _p(idx), _p(w))
    return idx, w


def router_topk_softmax(logits, k):
    return _router(lib().hho_router_topk_softmax, logits, k)


def router_softmax_topk_renorm(logits, k):
    return _router(lib().hho_router_softmax_topk_renorm, logits, k)


def router_gemma(hidden, projection, scale, per_expert_scale, k, eps):
    hidden = np.ascontiguousarray(hidden, dtype=np.float64)
    projection = np.ascontiguousarray(projection, dtype=np.float64)
    scale = np.ascontiguousarray(scale, dtype=np.float64)
    pes = np.ascontiguousarray(per_expert_scale, dtype=np.float64)
    E = projection.shape[0]
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float64)
    lib().hho_router_gemma(_p(hidden), C.c_int(hidden.size), _p(projection), _p(scale),
                           _p(pes), C.c_int(E), C.c_int(k), C.c_double(eps), _p(idx), _p(w))
    return idx, w


def blob_layout(desc, intermediate=None):
    off = (C.c_size_t * 9)()
    by = (C.c_size_t * 9)()
    payload, stride = C.c_size_t(), C.c_size_t()
    d = to_desc(desc)
    inter = desc.intermediate if intermediate is None else intermediate
    n = lib().hho_blob_layout(C.byref(d), C.c_int(inter), off, by, C.byref(payload),
                              C.byref(stride))
    return list(off[:n]), list(by[:n]), payload.value, stride.value


def _weights(layer):
    keep = []

    def arr(name, dtype):
        a = layer.get(name)
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return _p(a)

    w = Weights(arr("experts", np.uint8), C.c_size_t(layer["experts"].shape[1]),
                arr("shared_expert", np.uint8), arr("router_weight", np.uint16),
                arr("router_bias", np.uint16), arr("router_scale", np.uint16),
                arr("router_expert_scale", np.uint16), arr("shared_gate", np.uint16),
                int(layer.get("router_bits", 0)), arr("router_words", np.uint32),
                arr("router_scales", np.uint16), arr("router_biases", np.uint16),
                arr("shared_gate_words", np.uint32), arr("shared_gate_scales", np.uint16),
                arr("shared_gate_biases", np.uint16))
    return w, keep


def expert_ffn(desc, blob, x, intermediate=None) -> np.ndarray:
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(desc.hidden, np.float64)
    d = to_desc(desc)
    inter = desc.intermediate if intermediate is None else intermediate
    lib().hho_expert_ffn(C.byref(d), _p(blob), C.c_int(inter), _p(x), _p(out))
    return out


def router_logits(desc, layer, x_bf16) -> np.ndarray:
    """fp64 logits of each token [T][E] (GEMMA: after its normalisation and scales)."""
    w, keep = _weights(layer)
    d = to_desc(desc)
    x = bf16_to_f32(np.atleast_2d(x_bf16)).astype(np.float64)
    out = np.empty((x.shape[0], desc.experts), np.float64)
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t])
        lib().hho_router_logits(C.byref(d), C.byref(w), _p(xt), _p(out[t]))
    return out


def moe_forward(layer, x_bf16, x_router=None, nthreads=1):
    """The whole layer: returns (y fp64 [T][H], idx [T][K], w fp64 [T][K], shared_w [T])."""
    desc = layer["desc"]
    x_bf16 = np.ascontiguousarray(np.atleast_2d(x_bf16), dtype=np.uint16)
    T = x_bf16.shape[0]
    y = np.empty((T, desc.hidden), np.float64)
    idx = np.empty((T, desc.top_k), np.int32)
    wts = np.empty((T, desc.top_k), np.float64)
    sw = np.zeros(T, np.float64)
    w, keep = _weights(layer)
    xr = None if x_router is None else np.ascontiguousarray(x_router, dtype=np.uint16)
    d = to_desc(desc)
    rc = lib().hho_moe_forward(C.byref(d), C.byref(w), _p(x_bf16), _p(xr), C.c_int(T), _p(y),
                               _p(idx), _p(wts), _p(sw), C.c_int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle rejected the layer (code {rc})")
    return y, idx, wts, sw


QUANT_F64 = 100  # test-only fp64 gate/up/down matrices (oracle/hh_oracle.h)


class WeightsF64(C.Structure):
    _fields_ = [("experts", C.c_void_p), ("expert_stride", C.c_size_t),
                ("shared_expert", C.c_void_p), ("router_weight", C.c_void_p),
                ("router_bias", C.c_void_p), ("router_scale", C.c_void_p),
                ("router_expert_scale", C.c_void_p), ("shared_gate", C.c_void_p)]


def pack_f64_experts(desc, gates, ups, downs) -> np.ndarray:
    """fp64 expert matrices → blobs of the oracle's test-only fp64 layout."""
    off, by, payload, stride = blob_layout(desc)
    blobs = np.zeros((len(gates), stride), np.uint8)
    for e, mats in enumerate(zip(gates, ups, downs)):
        for o, b, m in zip(off, by, mats):
            m = np.ascontiguousarray(m, dtype=np.float64).view(np.uint8).ravel()
            assert m.size == b
            blobs[e, o:o + b] = m
    return blobs


def moe_forward_f64(desc, blobs, x, router_weight, x_router=None, router_bias=None,
                    router_scale=None, router_expert_scale=None, shared_blob=None,
                    shared_gate=None, nthreads=1):
    keep = []

    def arr(a, dtype):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return _p(a)

    w = WeightsF64(arr(blobs, np.uint8), C.c_size_t(blobs.shape[1]), arr(shared_blob, np.uint8),
                   arr(router_weight, np.float64), arr(router_bias, np.float64),
                   arr(router_scale, np.float64), arr(router_expert_scale, np.float64),
                   arr(shared_gate, np.float64))
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float64)
    xr = None if x_router is None else np.ascontiguousarray(np.atleast_2d(x_router), np.float64)
    T = x.shape[0]
    y = np.empty((T, desc.hidden), np.float64)
    idx = np.empty((T, desc.top_k), np.int32)
    wts = np.empty((T, desc.top_k), np.float64)
    sw = np.zeros(T, np.float64)
    d = to_desc(desc)
    rc = lib().hho_moe_forward_f64(C.byref(d), C.byref(w), _p(x), _p(xr), C.c_int(T), _p(y),
                                   _p(idx), _p(wts), _p(sw), C.c_int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle rejected the layer (code {rc})")
    return y, idx, wts, sw


def attention_decode(q, k_cache, v_cache, sinks, kv_heads, key_count, start_position=0,
                     ring_size=0, sm_scale=None):
    """fp64 decode attention with sinks (ReferenceLayer.swift:150-180). q [q_heads][d];
    caches [rows][kv_heads][d]; returns out [q_heads][d]."""
    q = np.ascontiguousarray(q, np.float64)
    qh, d = q.shape
    k = np.ascontiguousarray(k_cache, np.float64)
    v = np.ascontiguousarray(v_cache, np.float64)
    s = np.ascontiguousarray(sinks, np.float64)
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(d)
    out = np.zeros((qh, d), np.float64)
    L = lib()
    L.hho_attention_decode.argtypes = [C.c_void_p] * 4 + [C.c_int] * 6 + [C.c_double, C.c_void_p]
    L.hho_attention_decode(_p(q), _p(k), _p(v), _p(s), qh, kv_heads, d, key_count, ring_size,
                           start_position, float(sm_scale), _p(out))
    return out


# ---- the FFN block around the MoE layer (RMSNorm, residual, Gemma's branch norms) ------------

def rms_norm(x, weight, eps, pow_form=False) -> np.ndarray:
    """RMSNorm of each row in fp64: x·f·w with f = 1/√(mean(x²)+eps) (ReferenceOps.rmsNorm,
    ReferenceOps.swift:20-25) or, with `pow_form`, f = (mean(x²)+eps)^-½ (Gemma4ReferenceOps
    .rmsNorm, Gemma4ReferenceOps.swift:25-31); `weight` None = unscaled. The mean of squares is
    numpy's (pairwise) sum, which differs from the reference's left-to-right sum only in the
    last bits of fp64."""
    x = np.asarray(x, np.float64)
    m = np.mean(x * x, axis=-1, keepdims=True) + eps
    f = m ** -0.5 if pow_form else 1.0 / np.sqrt(m)
    out = x * f
    return out if weight is None else out * np.asarray(weight, np.float64)


def f64_to_bf16(x) -> np.ndarray:
    """fp64 → bf16 bits, one round to nearest even (NaN → quiet NaN). Normal results round
    the fp64 significand at bf16's last bit directly; results below bf16's normal range go
    through exact rational arithmetic."""
    from fractions import Fraction
    x = np.ascontiguousarray(x, np.float64)
    bits = x.view(np.uint64)
    lsb = (bits >> np.uint64(45)) & np.uint64(1)
    r = (bits + np.uint64((1 << 44) - 1) + lsb) & ~np.uint64((1 << 45) - 1)
    with np.errstate(over="ignore"):            # past bf16's range: inf, as RNE gives
        out = (r.view(np.float64).astype(np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)
    tiny = np.abs(x) < 2.0 ** -126
    for i in zip(*np.nonzero(tiny)):
        v = Fraction(float(x[i]))
        q = v / Fraction(2) ** -133            # bf16 subnormal step 2^-133
        n = int(q)                              # toward zero
        rem = q - n
        if abs(rem) > Fraction(1, 2) or (abs(rem) == Fraction(1, 2) and n % 2):
            n += 1 if q > 0 else -1
        out[i] = (0x8000 if (x[i] < 0 or (x[i] == 0 and np.signbit(x[i]))) else 0) | abs(n)
    out[np.isnan(x)] = 0x7FC0
    return out


def block_forward(desc, norms, hidden, moe, dense_out=None, bf16_input=True):
    """The FFN block around the MoE layer on an fp32/fp64 residual stream `hidden` [T][H]:
    returns (new hidden fp64 [T][H], idx, w, the layer input x).

    Pre-norm (no post_expert_norm; GPT-OSS ReferenceLayer.swift:189-202, Qwen
    QwenLayerRunner.swift:11-14): x = rmsnorm(hidden, pre_norm); hidden + moe(x).
    Gemma (Gemma4ReferenceLayer.swift:175-214): the router reads the residual, the experts
    x = rmsnorm(hidden, pre_norm); hidden + rmsnorm(rmsnorm(dense_out, post_dense_norm) +
    rmsnorm(moe(x), post_expert_norm), post_norm), times layer_scalar.

    `norms` holds fp64 weights (layer_scalar: one value, or None) and eps. `moe(x, x_router)`
    returns (y, idx, w). With `bf16_input` the layer input x (and the GEMMA router's residual)
    is rounded to bf16 bits, the format the layer's C ABI takes (x through f64_to_bf16, the
    fp32 residual through f32_to_bf16); without it the fp64 values go to `moe` as they are."""
    hidden = np.atleast_2d(np.asarray(hidden, np.float64))
    eps = float(norms["eps"])
    gemma_router = desc.router == 2
    xn = rms_norm(hidden, norms["pre_norm"], eps, pow_form=gemma_router)
    if bf16_input:
        x = f64_to_bf16(xn)
        xr = f32_to_bf16(hidden.astype(np.float32)) if gemma_router else None
    else:
        x, xr = xn, (hidden if gemma_router else None)
    y, idx, wts = moe(x, xr)
    if norms.get("post_expert_norm") is None:
        return hidden + y, idx, wts, x
    b1 = rms_norm(np.asarray(dense_out, np.float64), norms["post_dense_norm"], eps, pow_form=True)
    b2 = rms_norm(y, norms["post_expert_norm"], eps, pow_form=True)
    c = rms_norm(b1 + b2, norms["post_norm"], eps, pow_form=True)
    ls = 1.0 if norms.get("layer_scalar") is None else float(np.ravel(norms["layer_scalar"])[0])
    return (hidden + c) * ls, idx, wts, x


def block_forward_layer(layer, norms_bf16, hidden, dense_out=None, nthreads=1):
    """block_forward over a synthetic/quantised layer (moe_forward), with the norm weights
    given as bf16 bits, as the C ABI takes them."""
    desc = layer["desc"]
    to64 = lambda v: None if v is None else bf16_to_f32(v).astype(np.float64)
    norms = {k: (to64(v) if k != "eps" else v) for k, v in norms_bf16.items()}

    def moe(x, xr):
        y, idx, w, _ = moe_forward(layer, x, x_router=xr, nthreads=nthreads)
        return y, idx, w
    return block_forward(desc, norms, hidden, moe, dense_out)


def matvec(quant, rows, cols, weights, scales=None, biases=None, bias=None, x=None,
           group=64) -> np.ndarray:
    """y[t] = W·x[t] (+ bias) in fp64 with W dequantised exactly: MXFP4 through mxfp4_decode
    (MXFP4.swift:67-99), MLX through mlx_dequant (Gemma4ReferenceOps.swift:210-239), BF16
    widened; the projection of ReferenceLayer.matVec (ReferenceLayer.swift:104-113) and
    MLXAffine.matvec. x fp32/fp64 [T][cols] → y fp64 [T][rows]."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    if quant == 0:
        W = mxfp4_decode(np.asarray(weights, np.uint8).reshape(-1, 16),
                         np.asarray(scales, np.uint8).reshape(-1)).reshape(rows, cols).astype(np.float64)
    elif quant == 3:
        W = bf16_to_f32(np.asarray(weights, np.uint16).reshape(rows, cols)).astype(np.float64)
    else:
        bits = 4 if quant == 1 else 8
        wd = np.asarray(weights, np.uint32).reshape(rows, -1)
        sc = bf16_to_f32(np.asarray(scales, np.uint16)).astype(np.float64).reshape(rows, -1)
        bi = bf16_to_f32(np.asarray(biases, np.uint16)).astype(np.float64).reshape(rows, -1)
        W = np.stack([mlx_dequant(wd[r], sc[r], bi[r], cols, bits, group) for r in range(rows)])
    y = x @ W.T
    if bias is not None:
        y = y + bf16_to_f32(np.asarray(bias, np.uint16)).astype(np.float64)
    return y
