"""Host-side MoE layer over the HydraHIP C ABI.

`MoELayer` plays the part of the reference's layer runners for the MoE half of a layer
(LayerRunner.encodeMixtureOfExperts, LayerRunner.swift:304-353; PrefillRunner.encodeExpert,
PrefillRunner.swift:252-302; QwenMixtureBlock, QwenMixtureBlock.swift:122-263;
Gemma4LayerRunner.encodeExpertGroup, Gemma4LayerRunner.swift:579-616): it owns the layer's
weights resident in HBM and runs router → dispatch → experts → combine on device through
`hh_moe_forward`, with no host synchronisation inside a call.

PyTorch is used only to own device memory and to wrap the context's stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import formats as F
from ._lib import LAYER_HOOK, BlockNormsC, MoEWeightsC, check, desc_c, lib


# Device tensors of a layer besides its expert blobs (absent ones are None).
TENSORS = ["shared_expert", "router_weight", "router_bias", "router_scale", "router_expert_scale",
           "shared_gate", "router_words", "router_scales", "router_biases", "shared_gate_words",
           "shared_gate_scales", "shared_gate_biases"]


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


class Context:
    """One hh_ctx: a device, its stream and the scratch arena."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().hh_ctx_create(C.byref(h), device))
        self.handle = h
        self.device = device
        self.stream = torch.cuda.ExternalStream(lib().hh_ctx_stream(h), device=f"cuda:{device}")

    def synchronize(self):
        check(lib().hh_ctx_synchronize(self.handle))

    def reserve(self, desc: F.MoEDesc, max_tokens: int):
        d = desc_c(desc)
        check(lib().hh_ctx_reserve(self.handle, C.byref(d), max_tokens))

    def decode_fused(self, enable: int):
        """MXFP4 decode launches: 2 two (router inside the gate-up launch), 1 one fused launch,
        0 three, -1 the default (HH_DECODE_FUSED in the environment, else 2)."""
        check(lib().hh_ctx_decode_fused(self.handle, int(enable)))

    def profile(self, enable: bool = True):
        check(lib().hh_ctx_profile(self.handle, 1 if enable else 0))

    def profile_read(self):
        """(per-phase summed ms [route, gate-up, down, combine], profiled calls)."""
        ms = (C.c_double * 4)()
        calls = C.c_int64()
        check(lib().hh_ctx_profile_read(self.handle, ms, C.byref(calls)))
        return list(ms), calls.value

    def capture(self, record) -> "Graph":
        """Runs `record()` (hh_moe_forward calls on this context) under graph capture and
        returns the graph; nothing runs until `Graph.launch`."""
        check(lib().hh_ctx_capture_begin(self.handle))
        try:
            record()
        except BaseException:
            # end the capture and drop what it recorded: a graph left alive would keep the
            # context's scratch from growing
            g = C.c_void_p()
            lib().hh_ctx_capture_end(self.handle, C.byref(g))
            lib().hh_graph_destroy(g)
            raise
        g = C.c_void_p()
        check(lib().hh_ctx_capture_end(self.handle, C.byref(g)))
        return Graph(g, self)

    @property
    def dispatches(self) -> int:
        return lib().hh_dispatch_count(self.handle)

    def close(self):
        if self.handle:
            lib().hh_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def block_norms_c(norms: dict) -> BlockNormsC:
    """hh_block_norms from {pre_norm, post_expert_norm, post_dense_norm, post_norm, layer_scalar:
    device bf16 tensors (absent = NULL), eps: float}."""
    return BlockNormsC(_ptr(norms.get("pre_norm")), _ptr(norms.get("post_expert_norm")),
                       _ptr(norms.get("post_dense_norm")), _ptr(norms.get("post_norm")),
                       _ptr(norms.get("layer_scalar")), float(norms.get("eps", 1e-5)))


class Runner:
    """hh_runner: the MoE halves (FFN blocks) of a layer stack on one context. `hook(layer)`
    (optional) runs before each layer's block, on the host, with torch's current stream set to
    the stream hh_runner hands it (the context's): torch work it enqueues is ordered with the
    MoE kernels and is recorded by `capture`. An exception raised by the hook stops the stack
    (hh_runner returns HH_EINVAL) and is re-raised by `forward` / `capture`."""

    def __init__(self, ctx: Context, layers: list):
        """layers: [(MoELayer, norms dict, dense_out tensor or None)]."""
        self.ctx = ctx
        h = C.c_void_p()
        check(lib().hh_runner_create(ctx.handle, len(layers), C.byref(h)))
        self.handle = h
        self._keep = []
        self._error = None
        for i, (ml, norms, dense) in enumerate(layers):
            nc = block_norms_c(norms)
            self._keep.append((ml, norms, dense, nc))
            check(lib().hh_runner_set_layer(h, i, C.byref(ml._desc_c), C.byref(ml._weights_c),
                                            C.byref(nc), _ptr(dense)))

    def reserve(self, max_tokens: int):
        check(lib().hh_runner_reserve(self.handle, max_tokens))

    def _hook(self, hook):
        self._error = None
        if hook is None:
            return LAYER_HOOK()
        dev = f"cuda:{self.ctx.device}"

        def fn(user, layer, stream):
            try:
                with torch.cuda.stream(torch.cuda.ExternalStream(stream, device=dev)):
                    hook(layer)
                return 0
            except BaseException as e:   # kept for the caller; the C side sees a failure
                self._error = e
                return -1
        return LAYER_HOOK(fn)

    def _check(self, rc):
        if rc != 0 and self._error is not None:
            err, self._error = self._error, None
            raise err
        check(rc)

    def forward(self, hidden: torch.Tensor, hook=None):
        cb = self._hook(hook)
        self._check(lib().hh_runner_forward(self.handle, _ptr(hidden), hidden.shape[0], cb, None))

    def capture(self, hidden: torch.Tensor, hook=None) -> "Graph":
        cb = self._hook(hook)
        g = C.c_void_p()
        self._check(lib().hh_runner_capture(self.handle, _ptr(hidden), hidden.shape[0], cb, None,
                                            C.byref(g)))
        return Graph(g, self.ctx)

    def close(self):
        if self.handle:
            lib().hh_runner_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """A recorded sequence of layer calls (hh_graph); `launch` replays it on the context's
    stream."""

    def __init__(self, handle, ctx: Context):
        self.handle, self.ctx = handle, ctx

    def launch(self):
        check(lib().hh_graph_launch(self.handle))

    def close(self):
        # A graph outlived by its context was freed with nothing: its context is gone.
        if self.handle and self.ctx.handle:
            lib().hh_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_device(a: np.ndarray | None, device) -> torch.Tensor | None:
    """Host array → device tensor of the same bytes (bf16 bit patterns travel as int16)."""
    if a is None:
        return None
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(device)


class MoELayer:
    """One MoE layer with its weights in HBM, in the reference's expert blob layout."""

    def __init__(self, layer: dict, ctx: Context | None = None, device: int = 0):
        self.desc: F.MoEDesc = layer["desc"]
        self.ctx = ctx or Context(device)
        dev = torch.device(f"cuda:{self.ctx.device}")
        torch.cuda.synchronize(dev)
        self.experts = to_device(layer["experts"], dev)
        self.expert_stride = int(layer["experts"].shape[1])
        self.tensors = {k: to_device(layer.get(k), dev) for k in TENSORS}
        self.router_bits = int(layer.get("router_bits", 0))
        torch.cuda.synchronize(dev)
        self._desc_c = desc_c(self.desc)
        self._weights_c = self.weights_c()

    @classmethod
    def resident(cls, desc: F.MoEDesc, experts: torch.Tensor, expert_stride: int,
                 tensors: dict, ctx: Context, router_bits: int = 0) -> "MoELayer":
        """A layer over weights already in HBM: `experts` uint8 [E][expert_stride] in the blob
        layout, `tensors` the device router / shared-expert tensors by name (absent = None)."""
        self = cls.__new__(cls)
        self.desc, self.ctx = desc, ctx
        self.experts, self.expert_stride = experts, int(expert_stride)
        self.tensors = {k: tensors.get(k) for k in TENSORS}
        self.router_bits = int(router_bits)
        self._desc_c = desc_c(desc)
        self._weights_c = self.weights_c()
        return self

    def weights_c(self, experts: torch.Tensor | None = None) -> MoEWeightsC:
        t = self.tensors
        ex = self.experts if experts is None else experts
        return MoEWeightsC(ex.data_ptr(), self.expert_stride, _ptr(t["shared_expert"]),
                           _ptr(t["router_weight"]), _ptr(t["router_bias"]),
                           _ptr(t["router_scale"]), _ptr(t["router_expert_scale"]),
                           _ptr(t["shared_gate"]), self.router_bits, _ptr(t["router_words"]),
                           _ptr(t["router_scales"]), _ptr(t["router_biases"]),
                           _ptr(t["shared_gate_words"]), _ptr(t["shared_gate_scales"]),
                           _ptr(t["shared_gate_biases"]))

    def forward_into(self, x: torch.Tensor, y: torch.Tensor, idx: torch.Tensor | None = None,
                     w: torch.Tensor | None = None, x_router: torch.Tensor | None = None,
                     weights_c: MoEWeightsC | None = None) -> None:
        """Enqueues the layer on the context's stream (no host synchronisation)."""
        T = x.shape[0]
        check(lib().hh_moe_forward(self.ctx.handle, C.byref(self._desc_c),
                                   C.byref(weights_c or self._weights_c), _ptr(x),
                                   _ptr(x_router), T, _ptr(y), _ptr(idx), _ptr(w)))

    def block_forward_into(self, norms: dict, hidden: torch.Tensor,
                           dense_out: torch.Tensor | None = None, idx: torch.Tensor | None = None,
                           w: torch.Tensor | None = None) -> None:
        """The FFN block on the fp32 residual stream `hidden` [T][H], updated in place
        (hh_moe_block_forward): `norms` maps pre_norm / post_expert_norm / post_dense_norm /
        post_norm / layer_scalar to device bf16 tensors (absent = NULL) and eps to a float."""
        nc = block_norms_c(norms)
        check(lib().hh_moe_block_forward(self.ctx.handle, C.byref(self._desc_c),
                                         C.byref(self._weights_c), C.byref(nc), _ptr(hidden),
                                         _ptr(dense_out), hidden.shape[0], _ptr(idx), _ptr(w)))

    def forward(self, x, x_router=None):
        """x: bf16 bits [T][H] (numpy uint16 or device int16). Returns (y fp32 [T][H],
        top-k indices [T][K], top-k weights [T][K]) as device tensors, synchronised."""
        dev = torch.device(f"cuda:{self.ctx.device}")
        if isinstance(x, np.ndarray):
            x = to_device(np.atleast_2d(x), dev)
        if isinstance(x_router, np.ndarray):
            x_router = to_device(np.atleast_2d(x_router), dev)
        T = x.shape[0]
        y = torch.empty((T, self.desc.hidden), dtype=torch.float32, device=dev)
        idx = torch.empty((T, self.desc.top_k), dtype=torch.int32, device=dev)
        w = torch.empty((T, self.desc.top_k), dtype=torch.float32, device=dev)
        torch.cuda.synchronize(dev)
        self.forward_into(x, y, idx, w, x_router)
        self.ctx.synchronize()
        return y, idx, w
