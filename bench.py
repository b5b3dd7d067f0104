"""Benchmark of the HydraHIP MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (`value`): GPT-OSS-20B-shaped MXFP4 MoE layer in decode at T=1 (BASELINE.json
configs[1]), whole-layer tokens/s (router + top-k + dispatch + gate-up + SwiGLU + down +
combine) with inputs already in HBM. A step is one layer over one token batch; steps cycle over
several resident copies of the layer (> 256 MB Infinity Cache) and over a bank of inputs, so
every step streams its experts from HBM as consecutive layers of a model would.

Also reported: decode at T=2, 4, 8; the GPT-OSS-120B-shaped Zipf-skewed chunked prefill at
T=512 and T=2048; the Qwen-shaped MLX 4-bit and 8-bit layers and the
BF16 GELU layer at T=1 and in chunked prefill; the roofline of the dominant kernel (the gate-up expert
product) from HIP events on the library's stream; and the fp64 CPU restatement of the
reference path timed on this host.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hydra_amd import formats as F  # noqa: E402
from hydra_amd import synth  # noqa: E402

METRIC = "MoE-layer tokens/s at T=1 and T=512; % HBM GB/s (decode), % MFMA peak (prefill)"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
MXFP4_MFMA_PEAK_TFLOPS = 10100.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def up_bytes(desc: F.MoEDesc) -> int:
    """Algorithmic bytes of one expert's gate-up product: the gate_up tensors (blocks, scales
    and, when used, bias)."""
    lay = F.blob_layout(desc)
    if desc.quant == F.QUANT_MXFP4:
        return lay.sizes[0] + lay.sizes[1] + (lay.sizes[2] if desc.expert_bias else 0)
    if desc.quant == F.QUANT_BF16:
        return lay.sizes[0]
    return sum(lay.sizes[:6])


def router_bytes(desc: F.MoEDesc, router_bits: int) -> int:
    """Bytes of the router matrix every decode step reads: bf16 [E][H], or MLX-affine codes
    plus a bf16 scale and bias per 64-column group."""
    E, H = desc.experts, desc.hidden
    if router_bits:
        return E * H * router_bits // 8 + E * (H // 64) * 4
    return E * H * 2


def flops_per_token(desc: F.MoEDesc) -> float:
    H, I, K = desc.hidden, desc.intermediate, desc.top_k
    f = 2.0 * K * (2 * I * H + H * I)
    if desc.shared_intermediate:
        f += 2.0 * 3 * desc.shared_intermediate * H
    return f


class Workload:
    """`copies` resident copies of one synthetic layer and, per token count, a bank of token
    batches already in HBM."""

    def __init__(self, torch, desc, copies, zipf=None, seed=0, router_bits=0):
        from hydra_amd.layer import Context, MoELayer
        self.torch, self.desc = torch, desc
        t0 = time.time()
        host = synth.make_layer(desc, seed=seed, zipf=zipf, router_bits=router_bits)
        self.router_bytes = router_bytes(desc, router_bits)
        log(f"{desc.experts}x{desc.hidden} layer generated in {time.time() - t0:.1f}s")
        self.ctx = Context(0)
        self.layer = MoELayer(host, self.ctx)
        del host
        self.copies = [self.layer.experts] + [self.layer.experts.clone() for _ in range(copies - 1)]
        self.wc = [self.layer.weights_c(e) for e in self.copies]
        torch.cuda.synchronize()

    def prepare(self, T, bank):
        from hydra_amd.layer import to_device
        torch, dev = self.torch, "cuda:0"
        self.T = T
        self.bank = [to_device(synth.make_tokens(self.desc.hidden, T, seed=1000 + i), dev)
                     for i in range(bank)]
        self.y = torch.empty((T, self.desc.hidden), dtype=torch.float32, device=dev)
        self.idx = torch.full((bank, T, self.desc.top_k), -1, dtype=torch.int32, device=dev)
        self.written = set()
        self.w = torch.empty((T, self.desc.top_k), dtype=torch.float32, device=dev)
        self.ctx.reserve(self.desc, T)
        torch.cuda.synchronize()

    def step(self, i):
        b = i % len(self.bank)
        self.written.add(b)
        self.layer.forward_into(self.bank[b], self.y, self.idx[b], self.w,
                                weights_c=self.wc[i % len(self.wc)])

    def run(self, steps, warmup):
        torch = self.torch
        for i in range(warmup):
            self.step(i)
        self.ctx.synchronize()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            self.step(i)
        self.ctx.synchronize()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    def profiled(self, steps):
        """Per-phase mean ms from HIP events on the library stream, over `steps` steps."""
        self.ctx.profile(True)
        for i in range(steps):
            self.step(i)
        ms, calls = self.ctx.profile_read()
        self.ctx.profile(False)
        return [m / max(calls, 1) for m in ms]

    def unique_experts(self):
        """Mean distinct experts per step over the routing of the bank entries this run has
        actually routed (entries never stepped hold -1 and are left out)."""
        idx = self.idx.cpu().numpy()
        rows = sorted(self.written)
        assert rows, "no step has run"
        assert all((idx[i] >= 0).all() for i in rows), "a routed bank entry holds no indices"
        return float(np.mean([np.unique(idx[i]).size for i in rows]))

    def close(self):
        self.copies = self.wc = self.bank = None
        self.layer = None
        self.ctx.close()
        self.torch.cuda.empty_cache()


def measure_decode(wl, T, steps, warmup, fused=False):
    """Decode at T tokens in the default launch structure: for MXFP4 layers two launches (the
    router's workgroups first in the gate-up launch, which selects the top-k itself; down with
    the rank-ordered combine), otherwise three (router logits, gate-up, down); or with `fused`
    the one-launch kernel (hh_ctx_decode_fused 1), whose profile records the whole layer as the
    route phase."""
    desc = wl.desc
    wl.ctx.decode_fused(1 if fused else -1)
    wl.prepare(T, bank=64)
    sec = wl.run(steps, warmup)
    phases = wl.profiled(min(steps, 200))
    U = wl.unique_experts()
    if T == 1:
        assert U == desc.top_k, f"T=1 must touch exactly top_k experts, got {U}"
    # the gate-up launch of the two-launch MXFP4 decode also reads the router
    router_in_up = desc.quant == F.QUANT_MXFP4 and wl.router_bytes == desc.experts * desc.hidden * 2 \
        and desc.router != F.ROUTER_GEMMA and desc.experts <= 128 and desc.hidden <= 4096
    up_b = U * up_bytes(desc) + T * desc.hidden * 2 + (wl.router_bytes if router_in_up else 0)
    layer_b = U * F.streamed_expert_bytes(desc) + wl.router_bytes
    wl.ctx.decode_fused(-1)
    if fused:
        return {"T": T, "tokens_per_s": T / sec, "ms_per_step": sec * 1e3, "unique_experts": U,
                "kernel_ms": phases[0], "layer_GBps": layer_b / sec / 1e9,
                "layer_hbm_frac": layer_b / sec / 1e9 / HBM_PEAK_GBS}
    return {
        "T": T, "tokens_per_s": T / sec, "ms_per_step": sec * 1e3,
        "unique_experts": U, "phase_ms": dict(zip(["route", "gate_up", "down", "combine"], phases)),
        "gate_up_GBps": up_b / (phases[1] * 1e-3) / 1e9,
        "down_GBps": U * (F.streamed_expert_bytes(desc) - up_bytes(desc)) / (phases[2] * 1e-3) / 1e9,
        "layer_GBps": layer_b / sec / 1e9,
        "layer_hbm_frac": layer_b / sec / 1e9 / HBM_PEAK_GBS,
        "up_bytes_per_launch": up_b, "router_in_gate_up_launch": router_in_up,
    }


def measure_stack(wl, T, layers, steps, warmup):
    """The MoE halves of a GPT-OSS-20B decode stack (24 layers) at T tokens through hh_runner:
    per layer the FFN block (RMSNorm, router, experts, residual) on one fp32 residual stream,
    layer l on weight copy l % copies, no host synchronisation between layers; run eagerly (the
    default decode structure, and three launches per block) and as one captured HIP graph (three
    launches per block). Returns µs per layer of each."""
    from hydra_amd.layer import MoELayer, Runner
    torch = wl.torch
    dev = "cuda:0"
    desc = wl.desc
    wl.ctx.decode_fused(0)   # capture takes the three-launch structure
    g = torch.Generator(device=dev).manual_seed(7)
    norm = {"pre_norm": (torch.rand(desc.hidden, device=dev, generator=g) + 0.5).bfloat16().view(torch.int16),
            "eps": 1e-5}
    mls = [MoELayer.resident(desc, wl.copies[l % len(wl.copies)], wl.layer.expert_stride,
                             wl.layer.tensors, wl.ctx) for l in range(layers)]
    runner = Runner(wl.ctx, [(ml, norm, None) for ml in mls])
    runner.reserve(T)
    hidden = torch.randn((T, desc.hidden), device=dev, generator=g) * 3
    base = hidden.clone()
    torch.cuda.synchronize()

    def timed(fn):
        for _ in range(warmup):
            fn()
        wl.ctx.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        wl.ctx.synchronize()
        return (time.perf_counter() - t0) / steps

    eager3 = timed(lambda: runner.forward(hidden))   # three launches per block, as the graph
    hidden.copy_(base)
    wl.ctx.decode_fused(-1)   # the default decode structure (two launches for one or two tokens)
    eager = timed(lambda: runner.forward(hidden))
    hidden.copy_(base)
    torch.cuda.synchronize()
    graph = runner.capture(hidden)
    replay = timed(graph.launch)
    graph.close()
    runner.close()
    return {"T": T, "layers": layers, "eager_us_per_layer": eager / layers * 1e6,
            "eager_three_launch_us_per_layer": eager3 / layers * 1e6,
            "graph_us_per_layer": replay / layers * 1e6, "graph_tokens_per_s": T / replay,
            "eager_tokens_per_s": T / eager,
            "what": "hh_runner FFN blocks (RMSNorm + MoE + residual) of 24 GPT-OSS-20B layers"}


def measure_attention(torch, keys, q_heads=64, kv_heads=8, head_dim=64, reps=50, steps=20):
    """Decode attention with sinks (hh_attention_decode) on GPT-OSS's attention shape over an
    fp16 history of `keys` positions: `steps` rounds of `reps` back-to-back calls, timed with
    events on the context's stream; a spin kernel queued ahead of each round lets the host
    enqueue the round's calls before the first runs, so the events bracket GPU work only.
    Bytes = the key and value rows read once (keys · kv_heads · head_dim · 2 B · 2)."""
    from hydra_amd.attention import attention_decode_into
    from hydra_amd.layer import Context
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(keys)
    ctx = Context(0)
    q = torch.randn((q_heads, head_dim), device=dev, generator=g)
    # Two histories used in turn, each larger than the 256 MB memory-side cache at 64k keys.
    caches = [(torch.randn((keys, kv_heads, head_dim), device=dev, generator=g).half(),
               torch.randn((keys, kv_heads, head_dim), device=dev, generator=g).half())
              for _ in range(2)]
    sinks = torch.randn(q_heads, device=dev, generator=g).bfloat16().view(torch.int16)
    out = torch.empty((q_heads, head_dim), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for i in range(4):
        attention_decode_into(ctx, q, *caches[i % 2], sinks, keys, out=out)
    ctx.synchronize()
    total = 0.0
    for _ in range(steps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(ctx.stream):
            torch.cuda._sleep(20_000_000)
            start.record(ctx.stream)
        for i in range(reps):
            attention_decode_into(ctx, q, *caches[i % 2], sinks, keys, out=out)
        stop.record(ctx.stream)
        stop.synchronize()
        total += start.elapsed_time(stop) * 1e-3
    sec = total / (steps * reps)
    ctx.close()
    by = keys * kv_heads * head_dim * 2 * 2
    return {"keys": keys, "q_heads": q_heads, "kv_heads": kv_heads, "head_dim": head_dim,
            "us_per_call": sec * 1e6, "GBps": by / sec / 1e9, "hbm_frac": by / sec / 1e9 / HBM_PEAK_GBS}


def measure_prefill(wl, T, steps, warmup):
    desc = wl.desc
    wl.prepare(T, bank=4)
    sec = wl.run(steps, warmup)
    phases = wl.profiled(min(steps, 20))
    U = wl.unique_experts()
    fl = flops_per_token(desc) * T
    by = U * F.streamed_expert_bytes(desc) + shared_bytes(desc)
    t_exp = (phases[1] + phases[2]) * 1e-3
    return {
        "T": T, "tokens_per_s": T / sec, "ms_per_step": sec * 1e3, "unique_experts": U,
        "phase_ms": dict(zip(["route", "gate_up", "down", "combine"], phases)),
        "expert_TFLOPs": fl / t_exp / 1e12,
        "mfma_frac_bf16": fl / t_exp / 1e12 / BF16_MFMA_PEAK_TFLOPS,
        "mfma_frac_mxfp4": fl / t_exp / 1e12 / MXFP4_MFMA_PEAK_TFLOPS,
        "expert_GBps": by / t_exp / 1e9,
        "hbm_frac": by / t_exp / 1e9 / HBM_PEAK_GBS,
    }


OTHER = [  # (name, desc, copies, prefill T, router bits): BASELINE configs[3] (both bit
    # widths; the router and shared gate 8-bit MLX-affine as the published Qwen checkpoints
    # store them, Qwen35MoeConfig.swift:340-342) and [4]
    ("qwen-35b-a3b-mlx4", F.QWEN_35B_A3B_Q4, 2, 1024, 8),
    ("qwen-35b-a3b-mlx8", F.QWEN_35B_A3B_Q8, 2, 1024, 8),
    ("gemma-bf16", F.GEMMA_BF16, 2, 2048, 0),
]


def shared_bytes(desc: F.MoEDesc) -> int:
    """Bytes of the always-on shared expert (Qwen) plus its gate row."""
    if not desc.shared_intermediate:
        return 0
    return F.streamed_expert_bytes(desc, desc.shared_intermediate) + desc.hidden * 2


def measure_other(torch, name, desc, copies, T_prefill, steps, prefill=True, decode_tokens=(1, 8),
                  router_bits=0):
    """Decode at the given batch sizes and one chunked prefill of another format: whole-layer tokens/s,
    layer GB/s on the bytes touched (distinct routed experts + shared expert + router),
    expert-product TFLOP/s for the prefill."""
    log(f"{name}: decode T={list(decode_tokens)}, prefill T={T_prefill}")
    wl = Workload(torch, desc, copies=copies, router_bits=router_bits)
    dec = {}
    for T in decode_tokens:
        d = measure_decode(wl, T, steps if T == 1 else max(50, steps // 4), 20)
        d["layer_GBps"] += shared_bytes(desc) / (d["ms_per_step"] * 1e-3) / 1e9
        d["layer_hbm_frac"] = d["layer_GBps"] / HBM_PEAK_GBS
        dec[str(T)] = d
    p = measure_prefill(wl, T_prefill, 10, 3) if prefill else None
    wl.close()
    return {"decode": dec, "prefill": {str(T_prefill): p} if p else {}}


def cpu_baseline(runs=5, seconds=2.5):
    """The fp64 restatement of the reference's CPU path (oracle/), GPT-OSS-20B shape
    (configs[0]), timed on this host: `runs` timed runs of T=16 tokens per call with OpenMP over
    rows (each about `seconds` long) and `runs` single-thread T=1 calls; the medians are
    reported."""
    from oracle import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    layer = synth.make_layer(F.GPT_OSS_20B, seed=0)
    x = synth.make_tokens(F.GPT_OSS_20B.hidden, 16, seed=0)
    O.moe_forward(layer, x[:1], nthreads=threads)           # warm
    omp, total = [], 0
    for _ in range(runs):
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            O.moe_forward(layer, x, nthreads=threads)
            done += 16
        omp.append(done / (time.perf_counter() - t0))
        total += done
    single = []
    for r in range(runs):
        t1 = time.perf_counter()
        O.moe_forward(layer, x[r:r + 1], nthreads=1)
        single.append(1.0 / (time.perf_counter() - t1))
    med = float(np.median(omp))
    return {"value": med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "runs": runs, "openmp_tokens_per_s": omp, "openmp_threads": threads,
            "single_thread_tokens_per_s": float(np.median(single)),
            "single_thread_runs": single,
            "sample": f"gpt-oss-20b MXFP4 MoE layer (BASELINE configs[0]), fp64 oracle: median of "
                      f"{runs} runs of T=16 calls with OpenMP over rows on {threads} threads "
                      f"({total} tokens in ~{runs * seconds:.0f}s), and median of {runs} "
                      f"single-thread T=1 calls"}


TRAFFIC = "profiles/traffic_up_small_mx_gptoss20b_T1.json"


def load_traffic():
    p = os.path.join(ROOT, TRAFFIC)
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=8, help="resident layer copies (decode)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--decode-tokens", default="1,8",
                    help="decode batch sizes of the --only-other measurement (comma list)")
    ap.add_argument("--only-t1", action="store_true", help="decode T=1 only (for profiling)")
    ap.add_argument("--no-other", action="store_true", help="skip the MLX and BF16 configs")
    ap.add_argument("--only-other", default=None,
                    help="run only the named other config (qwen-35b-a3b-mlx4, ...; for profiling)")
    ap.add_argument("--only-prefill", action="store_true", help="prefill only (for profiling)")
    ap.add_argument("--only-stack", action="store_true",
                    help="the 24-layer FFN-block decode stack only (for profiling)")
    ap.add_argument("--only-attention", action="store_true",
                    help="decode attention only (for profiling)")
    ap.add_argument("--one-launch", action="store_true",
                    help="also time the opt-in one-launch MXFP4 decode (hh_ctx_decode_fused)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one 256 MiB device-to-device copy and exit (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(expert/tensor parallel sharding is design-only). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        # A plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch should read
        # 262144 KiB each; the ratio scales the counters of the expert kernels.
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 256 << 20}))
        return
    from hydra_amd._lib import lib
    lib()  # fail loudly if the HIP library is missing

    if args.only_stack:
        wl = Workload(torch, F.GPT_OSS_20B, copies=args.copies)
        print(json.dumps({"decode_stack_24_layers": {"1": measure_stack(wl, 1, 24, args.steps, args.warmup)}}))
        wl.close()
        return
    if args.only_attention:
        print(json.dumps({"decode_attention_gpt_oss": {
            str(k): measure_attention(torch, k) for k in [4096, 32768, 131072]}}))
        return
    if args.only_other:
        name, desc, copies, Tp, rb = next(o for o in OTHER if o[0] == args.only_other)
        print(json.dumps({name: measure_other(torch, name, desc, copies, Tp, args.steps,
                                              prefill=not args.no_prefill,
                                              decode_tokens=[int(t) for t in args.decode_tokens.split(",") if t],
                                              router_bits=rb)}))
        return
    decode, fused, stack = {}, {}, {}
    if not args.only_prefill:
        wl = Workload(torch, F.GPT_OSS_20B, copies=args.copies)
        for T in ([1] if args.only_t1 else [1, 2, 4, 8]):
            log(f"decode T={T}")
            steps = args.steps if T == 1 else max(100, args.steps // 4)
            decode[T] = measure_decode(wl, T, steps, args.warmup if T == 1 else 10)
        if not args.only_t1:
            for T in [1, 8]:
                log(f"decode stack of 24 layers, T={T}: eager and one HIP graph")
                stack[T] = measure_stack(wl, T, 24, 40, 5)
            for T in ([1, 2, 4, 8] if args.one_launch else []):
                log(f"decode T={T}, one launch")
                fused[T] = measure_decode(wl, T, max(100, args.steps // 4), 10, fused=True)
        wl.close()
    attention = {}
    if not (args.only_t1 or args.only_prefill or args.no_other):
        for keys in [4096, 32768, 131072]:
            log(f"decode attention, {keys} keys")
            attention[keys] = measure_attention(torch, keys)
    prefill = {}
    if not args.no_prefill and not args.only_t1:
        wl = Workload(torch, F.GPT_OSS_120B, copies=2, zipf=1.1)
        for T in [512, 2048]:
            log(f"prefill T={T}")
            prefill[T] = measure_prefill(wl, T, 20 if T == 512 else 10, 3)
        wl.close()
    other = {}
    if not (args.no_other or args.only_t1 or args.only_prefill):
        for name, desc, copies, Tp, rb in OTHER:
            other[name] = measure_other(torch, name, desc, copies, Tp, max(100, args.steps // 4),
                                        router_bits=rb)
    cpu = None if args.no_cpu else cpu_baseline()
    if args.only_prefill:
        print(json.dumps({"prefill_gpt_oss_120b_zipf": {str(T): v for T, v in prefill.items()}}))
        return

    d1 = decode[1]
    achieved = d1["gate_up_GBps"]
    out = {
        "metric": METRIC,
        "value": d1["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": d1["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 weights x fp8-e4m3 activation terms (x: 2 terms, h: 3), fp32 accumulation",
        "data": "synthetic",
        "config": {"workload": "gpt-oss-20b-shaped MXFP4 MoE layer, decode T=1 (BASELINE configs[1])",
                   "hidden": 2880, "intermediate": 2880, "experts": 32, "top_k": 4,
                   "weights": "mxfp4 e2m1 + e8m0/32", "layer_copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "up_small_mx<24, true>: decode gate-up (MXFP4 weights on the "
                               "scaled MFMA, top-k selected in every workgroup)",
                     "bytes_per_launch": d1["up_bytes_per_launch"],
                     "avg_launch_ms": d1["phase_ms"]["gate_up"]},
        "cpu_baseline": cpu,
        "decode": {str(T): v for T, v in decode.items()},
        "decode_one_launch": {str(T): v for T, v in fused.items()},
        "decode_stack_24_layers": {str(T): v for T, v in stack.items()},
        "decode_attention_gpt_oss": {str(k): v for k, v in attention.items()},
        "prefill_gpt_oss_120b_zipf": {str(T): v for T, v in prefill.items()},
        "other_configs": other,
    }
    tr = load_traffic()
    if tr is not None:
        out["roofline"]["traffic"] = tr.get("bytes_per_launch")
        out["roofline"]["traffic_source"] = TRAFFIC
    print(json.dumps(out))


if __name__ == "__main__":
    main()
