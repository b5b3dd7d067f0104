"""Decode attention with sinks (hh_attention_decode) against the fp64 oracle, which the
reference's sdpa fixtures pin (tests/test_oracle.py). Inputs are rounded to the kernel's
storage types (fp16 caches, bf16 sinks) before the oracle sees them; the kernel accumulates in
fp32, so outputs must agree within rel-L2 1e-4 (the layer bar, 1e-3, with margin)."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

REL_L2 = 1e-4

CASES = [
    # q_heads, kv_heads, d, key_count, start, ring
    (64, 8, 64, 1, 0, 0),           # GPT-OSS shape, first token
    (64, 8, 64, 300, 0, 0),          # ragged last tile
    (64, 8, 64, 4096, 0, 0),         # many chunks
    (64, 8, 64, 128, 1000, 128),     # sliding layer: window of 128 in a ring, wrapped
    (64, 8, 64, 0, 0, 0),            # no keys: the sink alone, output zero
    (16, 4, 128, 777, 5, 0),         # head_dim 128, q_mult 4, offset history
    (6, 6, 64, 513, 0, 0),           # q_mult 1
]


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.gpu
@pytest.mark.parametrize("qh,kvh,d,n,start,ring", CASES)
def test_attention_decode_matches_oracle(qh, kvh, d, n, start, ring):
    import torch
    from hydra_amd.attention import attention_decode_into
    from hydra_amd.layer import Context
    from hydra_amd import synth
    print(f"[gpu] attention qh={qh} kvh={kvh} d={d} n={n} start={start} ring={ring}", flush=True)
    rng = np.random.default_rng(qh * 1000 + n)
    rows = ring if ring > 0 else start + n + 3
    q = rng.standard_normal((qh, d)).astype(np.float32)
    k = rng.standard_normal((rows, kvh, d)).astype(np.float16)
    v = rng.standard_normal((rows, kvh, d)).astype(np.float16)
    sinks = synth.f32_to_bf16(rng.standard_normal(qh).astype(np.float32))
    ctx = Context(0)
    try:
        dev = "cuda:0"
        out = attention_decode_into(ctx, torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                    torch.from_numpy(v).to(dev),
                                    torch.from_numpy(sinks.view(np.int16)).to(dev), n, start, ring)
        torch.cuda.synchronize()
        ctx.synchronize()
        got = out.cpu().numpy()
    finally:
        ctx.close()
    ref = O.attention_decode(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                             synth.bf16_to_f32(sinks).astype(np.float64), kvh, n, start, ring)
    if n == 0:
        assert np.all(got == 0)
    else:
        assert rel_l2(got, ref) < REL_L2


def test_attention_shape_errors_need_no_gpu():
    """Shape checks run before any HIP call (NULL-free pointers are never dereferenced)."""
    from hydra_amd._lib import lib
    L, p = lib(), C.c_void_p(16)
    assert L.hh_attention_decode(None, p, p, p, p, 64, 8, 64, 10, 0, 0, 0.125, p) != 0
