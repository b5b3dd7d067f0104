"""Decode attention with sinks over the HydraHIP C ABI (`hh_attention_decode`).

Mirrors ForwardEncoder.attention (ForwardEncoder.swift:1107-1160): one query token against a
key/value history held as fp16 rows [rows][kv_heads][head_dim], optionally a ring (sliding
window layers), with per-head bf16 sinks in the softmax denominator.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import check, lib
from .layer import Context


def attention_decode_into(ctx: Context, q: torch.Tensor, k_cache: torch.Tensor,
                          v_cache: torch.Tensor, sinks: torch.Tensor, key_count: int,
                          start_position: int = 0, ring_size: int = 0,
                          sm_scale: float | None = None, out: torch.Tensor | None = None):
    """Enqueues one call on the context's stream. q fp32 [q_heads][d]; caches fp16 (or int16
    bits) [rows][kv_heads][d]; sinks bf16 bits (int16) [q_heads]. Returns `out`."""
    qh, d = q.shape
    rows, kvh, d2 = k_cache.shape
    assert d2 == d and tuple(v_cache.shape) == tuple(k_cache.shape) and sinks.numel() == qh
    need = ring_size if ring_size > 0 else start_position + key_count
    assert rows >= need, "the caches hold fewer rows than the visible keys need"
    if out is None:
        out = torch.empty((qh, d), dtype=torch.float32, device=q.device)
    scale = (1.0 / d ** 0.5) if sm_scale is None else sm_scale
    check(lib().hh_attention_decode(ctx.handle, C.c_void_p(q.data_ptr()),
                                    C.c_void_p(k_cache.data_ptr()), C.c_void_p(v_cache.data_ptr()),
                                    C.c_void_p(sinks.data_ptr()), qh, kvh, d, key_count,
                                    ring_size, start_position, float(scale),
                                    C.c_void_p(out.data_ptr())))
    return out
