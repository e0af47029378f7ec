#!/usr/bin/env python3
"""Benchmark: the Qwen3-30B-A3B W8 MoE layer on one MI355X.

    python bench.py [--steps K] [--warmup W] [--tokens T] [--copies R] [--sweep]
    python bench.py --copy-calibration MIB   # plain device copies of MIB MiB (counter calibration)

A step is one call of the whole MoE block (router, top-k, dispatch, SwiGLU
experts, combine) on T tokens, through the C ABI (kmoe_forward). Inputs and
weights are resident in HBM before timing starts. To measure HBM rather than
the 256 MB Infinity Cache, steps rotate over R independent weight copies
(R x 604 MB) and R activation batches.

Prints ONE JSON line on stdout (logs go to stderr):
  value        decode tokens/s at T (default 64) = T * steps / elapsed
  roofline     the dominant decode kernel (gate/up + SwiGLU), HBM-bound:
               algorithmic bytes per launch / mean launch time from HIP events
  prefill      the 4096-token prefill chunk: tokens/s and the MFMA roofline
               of its dominant kernel (the gate/up grouped GEMM), next to
               hipBLASLt bf16 GEMMs of the same shapes (library_reference)
  --sweep      also decode T in {1, 8, 32}, prefill T in {512, 2048}, and the
               235B-A22B-shaped layer (decode T=16, prefill T=2048)
  cpu_baseline the oracle (the C restatement of the reference algorithm),
               OpenMP on this host's cores, on a bounded sample
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "Qwen3-30B-A3B W8 MoE layer tokens/s; decode HBM GB/s; prefill MFMA % of peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Bound:
    """One layer copy with every C struct prebuilt, so a step is one ctypes call."""

    def __init__(self, layer, T, impl="ragged_jax", threshold=0):
        import torch

        from kappa_amd import _lib
        from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _desc
        from kappa_amd.qwen3.quant import weight_struct

        self.layer = layer
        dev = layer.router.device
        self.T = T
        # per-channel W8: the ragged program at every token count (ragged_jax, threshold 0)
        self.desc = _desc(T, layer.D, layer.E, layer.K, layer.I, torch.bfloat16, impl=impl, threshold=threshold)
        self.r, self._kr = weight_struct(layer.router, dev, n_out=layer.E, n_groups=None, name="router")
        self.g, self._kg = weight_struct(layer.gate, dev, n_out=layer.I, n_groups=layer.E, name="gate")
        self.u, self._ku = weight_struct(layer.up, dev, n_out=layer.I, n_groups=layer.E, name="up")
        self.d, self._kd = weight_struct(layer.down, dev, n_out=layer.D, n_groups=layer.E, name="down")
        self.packed = PACK_CACHE.get(layer.gate, layer.up, layer.down)
        PACK_CACHE.clear()
        self.p = self.packed.struct()
        n = ctypes.c_size_t()
        _lib.check(_lib.lib().kmoe_workspace_bytes(self.desc, ctypes.byref(n)))
        self.ws = torch.empty(n.value, dtype=torch.uint8, device=dev)


def make_copies(R, T, seed0=0):
    from moe_cases import make_layer

    return [Bound(make_layer("30b", seed=seed0 + i), T) for i in range(R)]


def time_forward(bounds, xs, outs, steps, warmup):
    """Whole-block steps through kmoe_forward; returns (seconds, per-step list unused)."""
    import torch

    from kappa_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    R = len(bounds)

    def step(i):
        b = bounds[i % R]
        st = L.kmoe_forward(
            b.desc, xs[i % len(xs)].data_ptr(), b.r, b.g, b.u, b.d, b.p, outs[i % len(outs)].data_ptr(),
            None, None, b.ws.data_ptr(), b.ws.numel(), stream,
        )  # fmt: skip
        if st:
            _lib.check(st)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        step(warmup + i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / 1e3


def time_block(bounds, hs, outs, scale, steps, warmup, fused: bool):
    """The MoE half of the layer, h + block(rms_norm(h)) (kappa/qwen3/block.py:196-207):
    fused = one kmoe_forward_block call; otherwise kmoe_rms_norm, kmoe_forward and a
    separate add, as the three steps run unfused. Returns seconds for `steps` steps."""
    import torch

    from kappa_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    R = len(bounds)
    h2 = torch.empty_like(hs[0])
    moe = torch.empty_like(hs[0])

    def step(i):
        b = bounds[i % R]
        h = hs[i % len(hs)]
        out = outs[i % len(outs)]
        if fused:
            st = L.kmoe_forward_block(
                b.desc, h.data_ptr(), scale.data_ptr(), _lib.DTYPE_BF16, 1e-6, b.r, b.g, b.u, b.d, b.p,
                out.data_ptr(), None, None, b.ws.data_ptr(), b.ws.numel(), stream,
            )  # fmt: skip
            if st:
                _lib.check(st)
            return
        _lib.check(L.kmoe_rms_norm(b.desc, h.data_ptr(), scale.data_ptr(), _lib.DTYPE_BF16, 1e-6, h2.data_ptr(), stream))
        st = L.kmoe_forward(
            b.desc, h2.data_ptr(), b.r, b.g, b.u, b.d, b.p, moe.data_ptr(), None, None, b.ws.data_ptr(), b.ws.numel(),
            stream,
        )  # fmt: skip
        if st:
            _lib.check(st)
        torch.add(h, moe, out=out)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        step(warmup + i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / 1e3


def time_gate_up(bounds, xs, steps, decode: bool):
    """Mean duration of the gate/up kernel (the dominant one) from HIP events on
    its stream around `steps` back-to-back launches that rotate over the weight
    copies (routing and dispatch for each copy are computed first, untimed).

    Returns (mean gate/up ms, mean active experts U)."""
    import torch

    from kappa_amd.qwen3 import moe_stages

    items = []
    actives = []
    for i, b in enumerate(bounds):
        lay = b.layer
        x = xs[i % len(xs)]
        r = moe_stages.route(x, lay.router, num_experts=lay.E, k=lay.K)
        dsp = moe_stages.dispatch(r["idx"], r["hist"], num_experts=lay.E)
        h = torch.empty((x.shape[0] * lay.K, 2 * lay.I), dtype=torch.bfloat16, device=x.device)  # hi, lo planes
        items.append((b, x, dsp, h))
        actives.append(dsp["active"][lay.E : lay.E + 1])
    for it in items:
        _gate_up_only(*it, decode)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        _gate_up_only(*items[i % len(items)], decode)
    e1.record()
    torch.cuda.synchronize()
    U = float(torch.cat(actives).float().mean().item())
    return e0.elapsed_time(e1) / steps, U


def _gate_up_only(b, x, dsp, h, decode):
    import torch

    from kappa_amd import _lib

    from kappa_amd.qwen3.ffn_moe import _desc

    lay = b.layer
    T = x.shape[0]
    desc = _desc(T, lay.D, lay.E, lay.K, lay.I, torch.bfloat16, impl="ragged_jax", threshold=0,
                 kernels=_lib.KERNELS_AUTO if decode else _lib.KERNELS_GROUPED)  # fmt: skip
    _lib.check(
        _lib.lib().kmoe_expert_gate_up(
            desc, x.data_ptr(), dsp["offsets"].data_ptr(), dsp["active"].data_ptr(), dsp["sorted_token"].data_ptr(),
            dsp["sorted_expert"].data_ptr(), b.g, b.u, b.p, h.data_ptr(), torch.cuda.current_stream().cuda_stream,
        )
    )  # fmt: skip
    return h


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload` from the rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE, copy-calibrated) committed under profiles/, or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_30b.md")
    try:
        for line in open(path):
            f = line.split()
            if len(f) >= 4 and f[0] == "traffic" and f[1] == kernel and f[2] == workload:
                return int(f[3])
    except OSError:
        pass
    return None


def bench_235b(bounds, xs, outs, args, dev):
    """The 235B-A22B-shaped W8 layer (D 4096, E 128, K 8, I 1536, ~2.4 GB of
    int8 experts): decode T=16 (HBM fraction) and prefill T=2048 (MFMA
    fraction), two weight copies in rotation. Frees the 30B copies first."""
    import torch

    from kappa_amd.qwen3 import moe_stages
    from moe_cases import make_layer

    bounds.clear()
    xs.clear()
    outs.clear()
    torch.cuda.empty_cache()
    log("bench: building 2 weight copies of the 235B-A22B W8 layer")
    big = [make_layer("235b", seed=40 + i) for i in range(2)]
    D, E, K, I = big[0].D, big[0].E, big[0].K, big[0].I
    res = {}
    for T, kind in ((16, "decode"), (2048, "prefill")):
        bb = [Bound(layer, T) for layer in big]
        g = torch.Generator(device=dev)
        g.manual_seed(13)
        xb = [torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(2)]
        ob = [torch.empty(T, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        steps = args.steps if kind == "decode" else max(10, args.steps // 5)
        secs = time_forward(bb, xb, ob, steps, args.warmup if kind == "decode" else 10)
        step_s = secs / steps
        if kind == "decode":
            us_ = [
                int(torch.unique(moe_stages.route(x, b.layer.router, num_experts=E, k=K)["idx"]).numel())
                for b, x in zip(bb, xb)
            ]
            U = sum(us_) / len(us_)
            lb = U * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 4 * T * D
            res["decode_T16"] = {
                "us_per_step": step_s * 1e6,
                "tokens_per_s": T / step_s,
                "layer_hbm_gbs": lb / step_s / 1e9,
                "layer_hbm_frac": lb / step_s / 1e9 / HBM_PEAK_GBS,
                "active_experts": U,
            }
        else:
            fl = 2.0 * T * K * 3 * D * I + 2.0 * T * D * E
            lb = E * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 4 * T * D
            res["prefill_T2048"] = {
                "us_per_step": step_s * 1e6,
                "tokens_per_s": T / step_s,
                "layer_tflops": fl / step_s / 1e12,
                "layer_mfma_frac": fl / step_s / 1e12 / BF16_PEAK_TFLOPS,
                "layer_hbm_frac": lb / step_s / 1e9 / HBM_PEAK_GBS,
            }
        log(f"bench: 235B {kind} T={T}: {step_s * 1e6:.1f} us/step")
        del bb, xb, ob
    del big
    torch.cuda.empty_cache()
    return res


def library_reference(T, D, I, E, K, reps=20):
    """hipBLASLt (torch.bmm / torch.mm, bf16) on the prefill expert shapes with
    uniform routing, M = T*K/E rows per expert, bf16 weights (no int8
    dequantisation, no gather, no SwiGLU): a vendor-library reference point
    for the grouped GEMMs, not part of the block."""
    import torch

    dev = torch.device("cuda:0")
    M = T * K // E
    out = {}
    for name, (bs, m, k, n) in (
        ("gate_up_bmm", (E, M, D, 2 * I)),
        ("down_bmm", (E, M, I, D)),
        ("gate_up_one_gemm", (1, T * K, D, 2 * I)),
    ):
        a = torch.randn(bs, m, k, device=dev).to(torch.bfloat16)
        b = torch.randn(bs, k, n, device=dev).to(torch.bfloat16).contiguous()
        for _ in range(3):
            torch.bmm(a, b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch.bmm(a, b)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        tf = 2.0 * bs * m * k * n / (us * 1e-6) / 1e12
        out[name] = {"shape": [bs, m, k, n], "us": us, "tflops": tf, "frac": tf / BF16_PEAK_TFLOPS}
        del a, b
    torch.cuda.empty_cache()
    return out


def cpu_baseline(layer, T, budget_s=12.0, max_reps=20):
    """Time the oracle (C, OpenMP) on the same workload; bounded sample."""
    import numpy as np

    import oracle

    host = layer.host()
    x = layer_x_host(T, layer.D)
    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    oracle.forward(x, host["router"], host["gate"], host["up"], host["down"], k=layer.K, act_bf16=True,
                   impl="ragged")  # warm  # fmt: skip
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        oracle.forward(x, host["router"], host["gate"], host["up"], host["down"], k=layer.K, act_bf16=True,
                       impl="ragged")  # fmt: skip
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    cpu = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": T / med,
        "unit": "tokens/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "sample": f"{len(times)} full layer calls at T={T} (30B-A3B W8, bf16), median {med * 1e3:.1f} ms; CPU: {cpu}",
    }


def layer_x_host(T, D, seed=99):
    import numpy as np

    from inputs import bf16_rne

    rng = np.random.default_rng(seed)
    return bf16_rne(rng.standard_normal((T, D)).astype(np.float32))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the first ~100 steps after the weight build run ~6% slower (clocks and
    # caches settling); 200 untimed steps cost ~25 ms
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--prefill-tokens", type=int, default=4096)
    ap.add_argument("--sweep", action="store_true", help="also time decode T in {1, 8, 32} and prefill T in {512, 2048}")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument(
        "--copy-calibration",
        type=int,
        default=0,
        metavar="MIB",
        help="only run 5 device-to-device copies of MIB MiB (the known-size kernel that scales the "
        "FETCH_SIZE / WRITE_SIZE counters) and exit",
    )
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the MoE block is not "
            "sharded across GPUs",
            file=sys.stderr,
        )
        sys.exit(1)

    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import torch

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20)
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: 5 copies of {args.copy_calibration} MiB ({n} bytes read and written each)")
        return

    from kappa_amd import _lib

    _lib.lib()
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T = args.tokens
    R = args.copies
    log(f"bench: building {R} weight copies of the 30B-A3B W8 layer")
    bounds = make_copies(R, T)
    lay0 = bounds[0].layer
    D, E, K, I = lay0.D, lay0.E, lay0.K, lay0.I
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    xs = [torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(R)]
    outs = [torch.empty(T, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]

    log(f"bench: decode T={T}: {args.warmup} warmup + {args.steps} timed steps")
    secs = time_forward(bounds, xs, outs, args.steps, args.warmup)
    ms_step = secs * 1e3 / args.steps
    tok_s = T * args.steps / secs
    log(f"bench: decode T={T}: {ms_step * 1e3:.1f} us/step, {tok_s:.0f} tokens/s")

    gu_ms, U = time_gate_up(bounds, xs, max(args.steps, 16), decode=True)
    M = T * K
    gu_bytes = U * (2 * D * I + 2 * I * 4) + T * D * 2 + M * I * 2
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    layer_bytes = U * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 2 * (2 * T * D)
    log(f"bench: gate/up kernel {gu_ms * 1e3:.1f} us, U={U:.1f}, {gu_gbs:.0f} GB/s")
    result = {
        "metric": METRIC,
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"qwen3-30b-a3b W8 MoE layer, decode batch T={T}",
            "tokens": T,
            "hidden": D,
            "experts": E,
            "top_k": K,
            "intermediate": I,
            "weights": "int8 per-output-channel fp32 scales, quantised from N(0,0.02)",
            "weight_copies_rotated": R,
        },
        "roofline": {
            "kernel": "k_gateup_decode",
            "bound": "hbm",
            "achieved": gu_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gu_gbs / HBM_PEAK_GBS,
            "traffic": measured_traffic("k_gateup_decode", f"decode_T{T}"),
            "algorithmic_bytes_per_launch": gu_bytes,
            "mean_launch_us": gu_ms * 1e3,
            "active_experts": U,
        },
        "layer_hbm_gbs": layer_bytes / (ms_step * 1e-3) / 1e9,
    }
    result["layer_hbm_frac"] = result["layer_hbm_gbs"] / HBM_PEAK_GBS

    # the steps either side of the block: rms_norm in, residual add out. The
    # fused call, the three separate calls and the bare MoE layer are timed in
    # interleaved rounds (the clock drifts over a run); medians are reported.
    scale = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    rounds = {"fused": [], "separate": [], "moe_only": []}
    n_round = max(args.steps // 5, 5)
    for _ in range(5):
        rounds["fused"].append(time_block(bounds, xs, outs, scale, n_round, 2, fused=True) / n_round)
        rounds["separate"].append(time_block(bounds, xs, outs, scale, n_round, 2, fused=False) / n_round)
        rounds["moe_only"].append(time_forward(bounds, xs, outs, n_round, 2) / n_round)
    med = {k: sorted(v)[len(v) // 2] * 1e6 for k, v in rounds.items()}
    result["block"] = {
        "workload": f"h + moe_layer(rms_norm(h)), decode T={T}",
        "fused_us_per_step": med["fused"],
        "separate_us_per_step": med["separate"],
        "moe_only_us_per_step": med["moe_only"],
        "rounds": f"5 interleaved rounds of {n_round} steps, medians",
    }
    log(f"bench: block {result['block']}")

    if args.sweep:
        sweep = {}
        for Ts in (1, 8, 32):
            bs = [Bound(b.layer, Ts) for b in bounds]
            xs_s = [x[:Ts].contiguous() for x in xs]
            o_s = [torch.empty(Ts, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
            s = time_forward(bs, xs_s, o_s, args.steps, args.warmup)
            gms, Us = time_gate_up(bs, xs_s, max(args.steps, 16), decode=True)
            gb = Us * (2 * D * I + 2 * I * 4) + Ts * D * 2 + Ts * K * I * 2
            lb = Us * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 2 * (2 * Ts * D)
            sweep[str(Ts)] = {
                "tokens_per_s": Ts * args.steps / s,
                "us_per_step": s * 1e6 / args.steps,
                "layer_hbm_gbs": lb / (s / args.steps) / 1e9,
                "gate_up_us": gms * 1e3,
                "gate_up_gbs": gb / (gms * 1e-3) / 1e9,
                "active_experts": Us,
            }
            log(f"bench: decode T={Ts}: {sweep[str(Ts)]}")
        result["decode_sweep"] = sweep

    if not args.no_prefill:
        Tp = args.prefill_tokens
        log(f"bench: prefill T={Tp}")
        bp = [Bound(b.layer, Tp) for b in bounds[:2]]
        gp = torch.Generator(device=dev)
        gp.manual_seed(11)
        xp = [torch.randn(Tp, D, generator=gp, device=dev).to(torch.bfloat16) for _ in range(2)]
        op = [torch.empty(Tp, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        psteps = max(10, args.steps // 5)
        s = time_forward(bp, xp, op, psteps, 10)
        gms, Up = time_gate_up(bp, xp, psteps, decode=False)
        Mp = Tp * K
        flops_gu = 2.0 * Mp * D * 2 * I
        flops_layer = 2.0 * Tp * K * 3 * D * I + 2.0 * Tp * D * E
        tf = flops_gu / (gms * 1e-3) / 1e12
        result["prefill"] = {
            "workload": f"qwen3-30b-a3b W8 MoE layer, prefill chunk T={Tp}",
            "tokens_per_s": Tp * psteps / s,
            "ms_per_step": s * 1e3 / psteps,
            "layer_tflops": flops_layer / (s / psteps) / 1e12,
            "layer_mfma_frac": flops_layer / (s / psteps) / 1e12 / BF16_PEAK_TFLOPS,
            "roofline": {
                "kernel": "k_gemm<true> (gate/up grouped GEMM + SwiGLU)",
                "bound": "mfma",
                "achieved": tf,
                "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": tf / BF16_PEAK_TFLOPS,
                "traffic": measured_traffic("k_gemm_gateup", f"prefill_T{Tp}"),
                "algorithmic_flops_per_launch": flops_gu,
                "mean_launch_us": gms * 1e3,
            },
        }
        result["prefill"]["library_reference"] = library_reference(Tp, D, I, E, K)
        if args.sweep:
            # the other prefill chunk sizes: whole-layer tokens/s and MFMA fraction
            psweep = {}
            for Tq in (512, 2048):
                bq = [Bound(b.layer, Tq) for b in bounds[:2]]
                xq = [x_[:Tq].contiguous() for x_ in xp]
                oq = [o_[:Tq] for o_ in op]
                sq = time_forward(bq, xq, oq, psteps, 10)
                fq = 2.0 * Tq * K * 3 * D * I + 2.0 * Tq * D * E
                # every expert is active at these sizes: the weight stream bounds T=512
                bq_ = E * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 4 * Tq * D
                psweep[str(Tq)] = {
                    "tokens_per_s": Tq * psteps / sq,
                    "us_per_step": sq * 1e6 / psteps,
                    "layer_tflops": fq / (sq / psteps) / 1e12,
                    "layer_mfma_frac": fq / (sq / psteps) / 1e12 / BF16_PEAK_TFLOPS,
                    "layer_hbm_frac": bq_ / (sq / psteps) / 1e9 / HBM_PEAK_GBS,
                }
                log(f"bench: prefill T={Tq}: {psweep[str(Tq)]}")
            result["prefill"]["sweep"] = psweep
        log(f"bench: prefill {result['prefill']}")

    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle)")
        result["cpu_baseline"] = cpu_baseline(bounds[0].layer, T)
        log(f"bench: cpu {result['cpu_baseline']}")
    else:
        result["cpu_baseline"] = None

    if args.sweep:
        result["layer_235b"] = bench_235b(bounds, xs, outs, args, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
