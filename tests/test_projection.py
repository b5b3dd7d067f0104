"""Operator-level expert projections (hh_expert_gemv / hh_expert_gemm) and the weighted combine
(hh_combine), through the C ABI, against the fp64 oracle.

Bars: rel-L2 1e-3 against the fp64 dequantise-then-dot oracle (observed: MXFP4 ~1e-5 with the
three-term fp8 activation operand, BF16/MLX ~1e-6); gemm row t equals gemv of x[t] bit for bit
(decode and prefill kernels alike); combine bit-exact against an fp32 emulation of
write_expert_scaled + sum_expert_slices."""
import ctypes as C

import numpy as np
import pytest

from hydra_amd import formats as F
from hydra_amd import synth
from oracle import oracle as O


def make_matrix(quant, rows, cols, seed, bias=False):
    """Host tensors of one matrix in the expert formats' value distributions."""
    out = {"quant": quant, "rows": rows, "cols": cols}
    if quant == F.QUANT_MXFP4:
        out["weights"] = synth.random_bytes(seed, "blocks", rows * cols // 2)
        out["scales"] = (np.uint8(119) + (synth.u64(seed, "scales", rows * cols // 32) % np.uint64(5)).astype(np.uint8))
        if bias:
            out["bias"] = synth.bf16_normal(seed, "bias", rows, 0.0, 0.02)
    elif quant == F.QUANT_BF16:
        out["weights"] = synth.bf16_normal(seed, "w", rows * cols, 0.0, 0.02)
    else:
        bits = 4 if quant == F.QUANT_MLX4 else 8
        centre = 7.5 if bits == 4 else 127.5
        out["weights"] = synth.random_bytes(seed, "words", rows * cols * bits // 8).view(np.uint32)
        sc = synth.bf16_normal(seed, "scales", rows * cols // 64, 0.01, 0.002)
        out["scales"] = sc
        out["biases"] = synth.f32_to_bf16(-centre * synth.bf16_to_f32(sc))
    return out


CASES = {
    "mxfp4-down-20b": (F.QUANT_MXFP4, 2880, 2880, True),
    "mxfp4-gate-up-20b": (F.QUANT_MXFP4, 5760, 2880, True),
    "mxfp4-nobias": (F.QUANT_MXFP4, 256, 640, False),
    "mlx4-gate": (F.QUANT_MLX4, 512, 2048, False),
    "mlx8-down": (F.QUANT_MLX8, 2048, 512, False),
    "bf16-gate-up": (F.QUANT_BF16, 1408, 2816, False),
    "bf16-down": (F.QUANT_BF16, 2816, 704, False),
    "bf16-small": (F.QUANT_BF16, 64, 256, False),
    "bf16-square": (F.QUANT_BF16, 256, 256, False),
    "mlx4-small": (F.QUANT_MLX4, 64, 256, False),
    "mxfp4-small": (F.QUANT_MXFP4, 64, 256, True),
}


def test_oracle_matvec_matches_layer_expert():
    """The oracle's matvec, composed as gate-up → activation → down over one expert blob's
    tensors, reproduces the oracle's whole-expert function (pinned elsewhere)."""
    desc = F.MoEDesc(hidden=128, intermediate=64, experts=2, top_k=1, quant=F.QUANT_MLX8,
                     activation=F.ACT_SILU, router=F.ROUTER_SOFTMAX_TOPK_RENORM, group_size=64)
    layer = synth.make_layer(desc, seed=4)
    lay = layer["layout"]
    blob = layer["experts"][1]
    sl = lambda k: blob[lay.offsets[k]:lay.offsets[k] + lay.sizes[k]]
    x = synth.bf16_to_f32(synth.make_tokens(128, 1, seed=5)).astype(np.float64)
    gate = O.matvec(2, 64, 128, sl(0).view(np.uint32), sl(1).view(np.uint16), sl(2).view(np.uint16), x=x)
    up = O.matvec(2, 64, 128, sl(3).view(np.uint32), sl(4).view(np.uint16), sl(5).view(np.uint16), x=x)
    h = gate / (1 + np.exp(-gate)) * up
    y = O.matvec(2, 128, 64, sl(6).view(np.uint32), sl(7).view(np.uint16), sl(8).view(np.uint16), x=h)
    ref = O.expert_ffn(desc, blob, x[0])
    assert np.max(np.abs(y[0] - ref)) <= 1e-12 * np.max(np.abs(ref))


def _mat_c(torch, m):
    from hydra_amd._lib import MatrixC
    dev = {}
    for k in ("weights", "scales", "biases", "bias"):
        if m.get(k) is not None:
            a = np.ascontiguousarray(m[k])
            a = a.view(np.int16) if a.dtype == np.uint16 else (a.view(np.int32) if a.dtype == np.uint32 else a)
            dev[k] = torch.from_numpy(a.copy()).to("cuda:0")
    p = lambda k: C.c_void_p(dev[k].data_ptr()) if k in dev else None
    return MatrixC(m["quant"], m["rows"], m["cols"], 64, p("weights"), p("scales"), p("biases"), p("bias")), dev


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_projection_against_oracle(name):
    import torch
    from hydra_amd._lib import check, lib
    from hydra_amd.layer import Context
    q, rows, cols, bias = CASES[name]
    print(f"[gpu] projection {name}", flush=True)
    ctx = Context(0)
    try:
        m = make_matrix(q, rows, cols, seed=31, bias=bias)
        mc, keep = _mat_c(torch, m)
        rng = np.random.default_rng(32)
        for T in (1, 5, 40):
            x = rng.standard_normal((T, cols)).astype(np.float32)
            xd = torch.from_numpy(x).to("cuda:0")
            y = torch.full((T, rows), float("nan"), dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            check(lib().hh_expert_gemm(ctx.handle, C.byref(mc), C.c_void_p(xd.data_ptr()), T,
                                       C.c_void_p(y.data_ptr())))
            ctx.synchronize()
            got = y.cpu().numpy()
            ref = O.matvec(q, rows, cols, m["weights"], m.get("scales"), m.get("biases"),
                           m.get("bias"), x)
            rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
            assert rel < 1e-3, (name, T, rel)
            for t in sorted({0, T - 1}):
                y1 = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda:0")
                x1 = torch.from_numpy(x[t].copy()).to("cuda:0")
                torch.cuda.synchronize()
                check(lib().hh_expert_gemv(ctx.handle, C.byref(mc), C.c_void_p(x1.data_ptr()),
                                           C.c_void_p(y1.data_ptr())))
                ctx.synchronize()
                assert np.array_equal(y1.cpu().numpy().view(np.uint32), got[t].view(np.uint32)), (name, T, t)
    finally:
        ctx.close()


@pytest.mark.gpu
def test_combine_bit_exact():
    import torch
    from hydra_amd._lib import check, lib
    from hydra_amd.layer import Context
    print("[gpu] combine", flush=True)
    ctx = Context(0)
    try:
        rng = np.random.default_rng(33)
        for T, K, H in [(1, 4, 2880), (7, 8, 2048), (33, 9, 704)]:
            slots = rng.standard_normal((T, K, H)).astype(np.float32)
            w = rng.uniform(0, 1, (T, K)).astype(np.float32)
            expect = np.zeros((T, H), np.float32)
            for r in range(K):
                expect = (expect + (w[:, r:r + 1] * slots[:, r]).astype(np.float32)).astype(np.float32)
            plain = np.zeros((T, H), np.float32)
            for r in range(K):
                plain = (plain + slots[:, r]).astype(np.float32)
            sd = torch.from_numpy(slots).to("cuda:0")
            wd = torch.from_numpy(w).to("cuda:0")
            for wp, ex in ((wd, expect), (None, plain)):
                y = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
                torch.cuda.synchronize()
                check(lib().hh_combine(ctx.handle, C.c_void_p(sd.data_ptr()),
                                       None if wp is None else C.c_void_p(wp.data_ptr()), T, K, H,
                                       C.c_void_p(y.data_ptr())))
                ctx.synchronize()
                assert np.array_equal(y.cpu().numpy().view(np.uint32), ex.view(np.uint32)), (T, K, H)
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("field", ["scales", "biases", "bias"])
def test_projection_refuses_unaligned_tensors(field):
    """Scales, MLX biases and the MXFP4 row bias read from an offset view (2 bytes past a
    16-byte boundary) are refused with HH_EALIGN before anything is enqueued; the aligned
    matrix then runs."""
    import torch
    from hydra_amd._lib import lib
    from hydra_amd.layer import Context
    print(f"[gpu] projection alignment {field}", flush=True)
    q = F.QUANT_MLX4 if field == "biases" else F.QUANT_MXFP4
    ctx = Context(0)
    try:
        m = make_matrix(q, 64, 256, seed=34, bias=True)
        mc, keep = _mat_c(torch, m)
        n = keep[field].numel() * keep[field].element_size()
        raw = torch.zeros(n + 16, dtype=torch.uint8, device="cuda:0")
        raw[2:2 + n].copy_(keep[field].view(torch.uint8).reshape(-1))
        setattr(mc, field, C.c_void_p(raw.data_ptr() + 2))
        x = torch.zeros((1, 256), dtype=torch.float32, device="cuda:0")
        y = torch.zeros((1, 64), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        rc = lib().hh_expert_gemm(ctx.handle, C.byref(mc), C.c_void_p(x.data_ptr()), 1,
                                  C.c_void_p(y.data_ptr()))
        assert rc == -2, rc      # HH_EALIGN
        setattr(mc, field, C.c_void_p(keep[field].data_ptr()))
        assert lib().hh_expert_gemm(ctx.handle, C.byref(mc), C.c_void_p(x.data_ptr()), 1,
                                    C.c_void_p(y.data_ptr())) == 0
        ctx.synchronize()
    finally:
        ctx.close()
