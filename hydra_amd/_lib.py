"""ctypes binding of libhydra_hip.so (the C ABI of include/hydra_hip.h).

There is no fallback: if the library is missing or fails to load, every entry point raises
HydraHIPError. Build it with `python -m hydra_amd.build`.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhydra_hip.so")

# Every function include/hydra_hip.h declares.
EXPORTS = [
    "hh_ctx_create", "hh_ctx_destroy", "hh_ctx_stream", "hh_ctx_synchronize", "hh_ctx_reserve",
    "hh_dispatch_count", "hh_last_error", "hh_desc_check", "hh_expert_blob_layout",
    "hh_moe_forward", "hh_mxfp4_dequant", "hh_mlx_dequant", "hh_router_topk", "hh_activation",
    "hh_permute", "hh_ctx_profile", "hh_ctx_profile_read", "hh_ctx_decode_fused", "hh_scatter_expert_tensor",
    "hh_ctx_capture_begin", "hh_ctx_capture_end", "hh_graph_launch", "hh_graph_destroy",
    "hh_attention_decode", "hh_moe_forward_noalloc", "hh_moe_block_forward",
    "hh_expert_gemv", "hh_expert_gemm", "hh_combine",
    "hh_runner_create", "hh_runner_destroy", "hh_runner_set_layer", "hh_runner_reserve",
    "hh_runner_forward", "hh_runner_capture",
]

# int (*hh_layer_hook)(void *user, int32_t layer, void *stream)
LAYER_HOOK = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32, C.c_void_p)

CODES = {0: "HH_OK", -1: "HH_EINVAL", -2: "HH_EALIGN", -3: "HH_ETOPK", -4: "HH_EHIP",
         -5: "HH_ENOMEM", -6: "HH_ESHAPE"}


class HydraHIPError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{CODES.get(code, code)}: {message}")
        self.code = code


class MoEDescC(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("intermediate", C.c_int32), ("experts", C.c_int32),
                ("top_k", C.c_int32), ("shared_intermediate", C.c_int32), ("quant", C.c_int32),
                ("group_size", C.c_int32), ("activation", C.c_int32), ("router", C.c_int32),
                ("expert_bias", C.c_int32), ("swiglu_alpha", C.c_float),
                ("swiglu_limit", C.c_float), ("router_eps", C.c_float)]


class MoEWeightsC(C.Structure):
    _fields_ = [("experts", C.c_void_p), ("expert_stride", C.c_size_t),
                ("shared_expert", C.c_void_p), ("router_weight", C.c_void_p),
                ("router_bias", C.c_void_p), ("router_scale", C.c_void_p),
                ("router_expert_scale", C.c_void_p), ("shared_gate", C.c_void_p),
                ("router_bits", C.c_int32), ("router_words", C.c_void_p),
                ("router_scales", C.c_void_p), ("router_biases", C.c_void_p),
                ("shared_gate_words", C.c_void_p), ("shared_gate_scales", C.c_void_p),
                ("shared_gate_biases", C.c_void_p)]


class BlockNormsC(C.Structure):
    _fields_ = [("pre_norm", C.c_void_p), ("post_expert_norm", C.c_void_p),
                ("post_dense_norm", C.c_void_p), ("post_norm", C.c_void_p),
                ("layer_scalar", C.c_void_p), ("eps", C.c_float)]


class MatrixC(C.Structure):
    _fields_ = [("quant", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32),
                ("group_size", C.c_int32), ("weights", C.c_void_p), ("scales", C.c_void_p),
                ("biases", C.c_void_p), ("bias", C.c_void_p)]


class BlobLayoutC(C.Structure):
    _fields_ = [("slot_count", C.c_int32), ("offset", C.c_size_t * 9), ("bytes", C.c_size_t * 9),
                ("payload_bytes", C.c_size_t), ("stride_bytes", C.c_size_t)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HydraHIPError(-4, f"{LIB_PATH} is not built; run `python -m hydra_amd.build`")
    L = C.CDLL(LIB_PATH)
    vp, i32, i64, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
    L.hh_last_error.restype = C.c_char_p
    L.hh_ctx_create.argtypes = [C.POINTER(vp), i32]
    L.hh_ctx_destroy.argtypes = [vp]
    L.hh_ctx_stream.argtypes = [vp]
    L.hh_ctx_stream.restype = vp
    L.hh_ctx_synchronize.argtypes = [vp]
    L.hh_ctx_reserve.argtypes = [vp, C.POINTER(MoEDescC), i32]
    L.hh_dispatch_count.argtypes = [vp]
    L.hh_dispatch_count.restype = i64
    L.hh_desc_check.argtypes = [C.POINTER(MoEDescC)]
    L.hh_expert_blob_layout.argtypes = [C.POINTER(MoEDescC), i32, C.POINTER(BlobLayoutC)]
    L.hh_moe_forward.argtypes = [vp, C.POINTER(MoEDescC), C.POINTER(MoEWeightsC), vp, vp, i32,
                                 vp, vp, vp]
    L.hh_moe_forward_noalloc.argtypes = L.hh_moe_forward.argtypes
    L.hh_moe_block_forward.argtypes = [vp, C.POINTER(MoEDescC), C.POINTER(MoEWeightsC),
                                       C.POINTER(BlockNormsC), vp, vp, i32, vp, vp]
    L.hh_expert_gemv.argtypes = [vp, C.POINTER(MatrixC), vp, vp]
    L.hh_expert_gemm.argtypes = [vp, C.POINTER(MatrixC), vp, i32, vp]
    L.hh_combine.argtypes = [vp, vp, vp, i32, i32, i32, vp]
    L.hh_runner_create.argtypes = [vp, i32, C.POINTER(vp)]
    L.hh_runner_destroy.argtypes = [vp]
    L.hh_runner_set_layer.argtypes = [vp, i32, C.POINTER(MoEDescC), C.POINTER(MoEWeightsC),
                                      C.POINTER(BlockNormsC), vp]
    L.hh_runner_reserve.argtypes = [vp, i32]
    L.hh_runner_forward.argtypes = [vp, vp, i32, LAYER_HOOK, vp]
    L.hh_runner_capture.argtypes = [vp, vp, i32, LAYER_HOOK, vp, C.POINTER(vp)]
    L.hh_mxfp4_dequant.argtypes = [vp, vp, vp, i64, vp]
    L.hh_mlx_dequant.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, vp]
    L.hh_router_topk.argtypes = [vp, C.POINTER(MoEDescC), C.POINTER(MoEWeightsC), vp, i32, vp,
                                 vp, vp, vp]
    L.hh_activation.argtypes = [vp, C.POINTER(MoEDescC), vp, vp, i64, vp]
    L.hh_permute.argtypes = [vp, vp, i32, i32, i32, vp, vp]
    L.hh_ctx_profile.argtypes = [vp, i32]
    L.hh_ctx_capture_begin.argtypes = [vp]
    L.hh_attention_decode.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, C.c_float, vp]
    L.hh_ctx_capture_end.argtypes = [vp, C.POINTER(vp)]
    L.hh_graph_launch.argtypes = [vp]
    L.hh_graph_destroy.argtypes = [vp]
    L.hh_scatter_expert_tensor.argtypes = [vp, C.POINTER(MoEDescC), i32, i32, i32, vp, i64, vp,
                                           C.c_uint64]
    L.hh_ctx_decode_fused.argtypes = [vp, i32]
    L.hh_ctx_profile_read.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)]
    for name in EXPORTS:
        if name not in ("hh_last_error", "hh_ctx_stream", "hh_dispatch_count"):
            getattr(L, name).restype = C.c_int
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise HydraHIPError(rc, lib().hh_last_error().decode(errors="replace"))


def desc_c(d) -> MoEDescC:
    return MoEDescC(d.hidden, d.intermediate, d.experts, d.top_k, d.shared_intermediate, d.quant,
                    d.group_size, d.activation, d.router, d.expert_bias, d.swiglu_alpha,
                    d.swiglu_limit, d.router_eps)


def blob_layout(d, intermediate=None):
    out = BlobLayoutC()
    inter = d.intermediate if intermediate is None else intermediate
    dc = desc_c(d)
    check(lib().hh_expert_blob_layout(C.byref(dc), inter, C.byref(out)))
    n = out.slot_count
    return list(out.offset[:n]), list(out.bytes[:n]), out.payload_bytes, out.stride_bytes
