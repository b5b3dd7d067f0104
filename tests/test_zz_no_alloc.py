"""hh_moe_forward_noalloc (the allocation-free layer entry, scratch in a static device array)
against hh_moe_forward, through the C ABI, bit for bit: two calls in a row per layer, the
second with fewer tokens, so a call that read scratch left by the previous, larger call would
show. Also: a call whose scratch plan exceeds the static array is refused with HH_ENOMEM."""
import ctypes as C

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth

pytestmark = pytest.mark.gpu

CASES = {
    "gpt-oss-20b": (F.GPT_OSS_20B, [8, 1]),
    "gpt-oss-small-prefill": (F.GPT_OSS_20B.replace(experts=8, top_k=2), [96, 17]),
    "qwen-q4": (F.QWEN_35B_A3B_Q4, [16, 3]),
    "gemma-bf16": (F.GEMMA_BF16, [40, 1]),
}


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_equals_forward(name):
    import torch
    from hydra_amd._lib import check, lib
    from hydra_amd.layer import Context, MoELayer, to_device
    desc, Ts = CASES[name]
    print(f"[gpu] noalloc {name} T={Ts}", flush=True)
    ctx = Context(0)
    try:
        L = MoELayer(synth.make_layer(desc, seed=81), ctx)
        for i, T in enumerate(Ts):
            x = to_device(synth.make_tokens(desc.hidden, T, seed=90 + i), "cuda:0")
            outs = []
            for fn in (lib().hh_moe_forward, lib().hh_moe_forward_noalloc):
                y = torch.full((T, desc.hidden), float("nan"), dtype=torch.float32, device="cuda:0")
                idx = torch.full((T, desc.top_k), -1, dtype=torch.int32, device="cuda:0")
                w = torch.full((T, desc.top_k), float("nan"), dtype=torch.float32, device="cuda:0")
                torch.cuda.synchronize()
                check(fn(ctx.handle, C.byref(L._desc_c), C.byref(L._weights_c), _p(x), None, T,
                         _p(y), _p(idx), _p(w)))
                ctx.synchronize()
                outs.append([v.cpu().numpy() for v in (y, idx, w)])
            (ya, ia, wa), (yb, ib, wb) = outs
            assert not np.isnan(yb).any(), (name, T)
            assert np.array_equal(ia, ib), (name, T)
            assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), (name, T)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (name, T)
    finally:
        ctx.close()


def test_noalloc_refuses_oversized_calls():
    import torch
    from hydra_amd._lib import lib
    from hydra_amd.layer import Context, MoELayer
    print("[gpu] noalloc oversized call", flush=True)
    desc = F.GPT_OSS_20B.replace(experts=8, top_k=4, intermediate=64)
    ctx = Context(0)
    try:
        L = MoELayer(synth.make_layer(desc, seed=82), ctx)
        T = 4096      # slot outputs alone: 4096 * 4 * 2880 * 4 B = 189 MB > 16 MiB
        x = torch.zeros((T, desc.hidden), dtype=torch.int16, device="cuda:0")
        y = torch.zeros((T, desc.hidden), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        rc = lib().hh_moe_forward_noalloc(ctx.handle, C.byref(L._desc_c), C.byref(L._weights_c),
                                          _p(x), None, T, _p(y), None, None)
        assert rc == -5, rc      # HH_ENOMEM, nothing enqueued
        assert b"scratch" in lib().hh_last_error()
        assert ctx.dispatches == 0
    finally:
        ctx.close()
