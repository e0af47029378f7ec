#!/usr/bin/env python3
"""Benchmark: the Qwen3-30B-A3B W8 MoE layer on one MI355X, and the other
workloads of the same metric.

    python bench.py [--steps K] [--warmup W] [--copies R] [--quick] [--no-cpu-baseline]
    python bench.py --copy-calibration MIB   # plain device copies of MIB MiB (counter calibration)

A step is one call of the whole MoE block (router, top-k, dispatch, SwiGLU
experts, combine) on T tokens, through the C ABI (kmoe_forward). Inputs and
weights are resident in HBM before timing starts. To measure HBM rather than
the 256 MB Infinity Cache, steps rotate over R independent weight copies
(R x 604 MB) and R activation batches.

The layers hold per-output-channel W8 weights, which the reference runs with
its ragged program (moe_impl ragged_jax; decode threshold 0 for the decode
batches): that is the program every timed call follows. The gather program
(the reference default, per-tensor W8) is timed beside it at decode T=64.

Prints ONE JSON line on stdout (logs go to stderr):
  value          decode tokens/s at T=64 (the headline workload)
  roofline       the dominant decode kernel (gate/up + SwiGLU), HBM-bound:
                 algorithmic bytes per launch / mean launch time from HIP events
  decode         T in {1, 8, 32, 64}: us/step, tokens/s, layer HBM fraction,
                 the gate/up kernel's time and HBM fraction
  prefill        T in {512, 2048, 4096}: us/step, tokens/s, layer MFMA and HBM
                 fractions; the MFMA roofline of the gate/up grouped GEMM at 4096
  skew           the Zipf(1.2)-skewed router at T=4096 and T=64, with the share of
                 assignments the 8 hottest experts receive
  layer_235b     the 235B-A22B-shaped layer: decode T=16, prefill T=2048
  gather_decode  the gather program on per-tensor W8 at T=64
  block          h + block(rms_norm(h)) fused in one call vs the separate steps
  cpu_baseline   the oracle (the C restatement of the reference programs),
                 OpenMP on this host's cores, on bounded samples (decode T=64 and
                 a T=512 prefill chunk)
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

    def __init__(self, layer, T, impl="ragged_jax", threshold=0, router=None):
        import torch

        from kappa_amd import _lib
        from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _desc
        from kappa_amd.qwen3.quant import weight_struct

        self.layer = layer
        self.router = layer.router if router is None else router
        dev = layer.router.device
        self.T = T
        self.desc = _desc(T, layer.D, layer.E, layer.K, layer.I, torch.bfloat16, impl=impl, threshold=threshold)
        self.r, self._kr = weight_struct(self.router, dev, n_out=layer.E, n_groups=None, name="router")
        self.g, self._kg = weight_struct(layer.gate, dev, n_out=layer.I, n_groups=layer.E, name="gate")
        self.u, self._ku = weight_struct(layer.up, dev, n_out=layer.I, n_groups=layer.E, name="up")
        self.d, self._kd = weight_struct(layer.down, dev, n_out=layer.D, n_groups=layer.E, name="down")
        self.packed = PACK_CACHE.get(layer.gate, layer.up, layer.down)
        self.p = self.packed.struct()
        n = ctypes.c_size_t()
        _lib.check(_lib.lib().kmoe_workspace_bytes(self.desc, ctypes.byref(n)))
        self.ws = torch.empty(n.value, dtype=torch.uint8, device=dev)


def time_forward(bounds, xs, outs, steps, warmup):
    """Whole-block steps through kmoe_forward, rotating over the weight copies;
    seconds for `steps` steps between two HIP events on the launch stream."""
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


def time_forward_graph(bounds, xs, outs, steps, warmup):
    """The same steps captured once in a HIP graph (one step per weight copy, in
    rotation) and replayed, as a serving loop runs a decode step: the host
    launches nothing per step. Returns seconds per step."""
    import torch

    from kappa_amd import _lib

    L = _lib.lib()
    R = len(bounds)

    def one_round(stream):
        for i, b in enumerate(bounds):
            st = L.kmoe_forward(
                b.desc, xs[i % len(xs)].data_ptr(), b.r, b.g, b.u, b.d, b.p, outs[i % len(outs)].data_ptr(),
                None, None, b.ws.data_ptr(), b.ws.numel(), stream,
            )  # fmt: skip
            if st:
                _lib.check(st)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        one_round(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        one_round(torch.cuda.current_stream().cuda_stream)
    reps = max(1, steps // R)
    for _ in range(max(1, warmup // R)):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / 1e3 / (reps * R)


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
        r = moe_stages.route(x, b.router, num_experts=lay.E, k=lay.K)
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


def active_experts(bounds, xs):
    """Mean number of experts with at least one assignment (U), over the copies."""
    import torch

    from kappa_amd.qwen3 import moe_stages

    us = []
    for i, b in enumerate(bounds):
        lay = b.layer
        idx = moe_stages.route(xs[i % len(xs)], b.router, num_experts=lay.E, k=lay.K)["idx"]
        us.append(int(torch.unique(idx).numel()))
    return sum(us) / len(us)


def hot_share(bounds, xs, top=8):
    """Share of the assignments that the `top` most-chosen experts receive."""
    import torch

    from kappa_amd.qwen3 import moe_stages

    b, x = bounds[0], xs[0]
    lay = b.layer
    idx = moe_stages.route(x, b.router, num_experts=lay.E, k=lay.K)["idx"]
    counts = torch.bincount(idx.reshape(-1).long(), minlength=lay.E)
    return float(torch.topk(counts, top).values.sum().item() / idx.numel())


def decode_bytes(layer, T, U):
    """Algorithmic HBM bytes of one layer call with U active experts."""
    D, E, I = layer.D, layer.E, layer.I
    return U * (3 * D * I + 4 * (2 * I + D)) + 2 * D * E + 4 * T * D


def prefill_flops(layer, T):
    return 2.0 * T * layer.K * 3 * layer.D * layer.I + 2.0 * T * layer.D * layer.E


def make_x_list(T, D, n, seed, dev, skew=False):
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    xs = [torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    if skew:
        for x in xs:
            x[:, 0] = 1.0
    return xs


def decode_point(layers, T, args, dev, router_fn=None, impl="ragged_jax", threshold=0, seed=7):
    """us/step, tokens/s, layer HBM fraction and the gate/up kernel at decode size T."""
    import torch

    bounds = [Bound(lay, T, impl=impl, threshold=threshold, router=router_fn(lay) if router_fn else None)
              for lay in layers]  # fmt: skip
    xs = make_x_list(T, layers[0].D, len(layers), seed + T, dev, skew=router_fn is not None)
    outs = [torch.empty(T, layers[0].D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    secs = time_forward(bounds, xs, outs, args.steps, args.warmup)
    step_s = secs / args.steps
    U = active_experts(bounds, xs)
    lb = decode_bytes(layers[0], T, U)
    res = {
        "us_per_step": step_s * 1e6,
        "tokens_per_s": T / step_s,
        "layer_hbm_gbs": lb / step_s / 1e9,
        "layer_hbm_frac": lb / step_s / 1e9 / HBM_PEAK_GBS,
        "active_experts": U,
    }
    # the same steps replayed from a HIP graph (steps and warm-up rounded to whole rotations)
    g_s = time_forward_graph(bounds, xs, outs, max(args.steps, 8 * len(bounds)), args.warmup)
    res["graph_us_per_step"] = g_s * 1e6
    res["graph_tokens_per_s"] = T / g_s
    if impl == "ragged_jax":
        gu_ms, _ = time_gate_up(bounds, xs, max(args.steps, 16), decode=True)
        lay = layers[0]
        gu_bytes = U * (2 * lay.D * lay.I + 2 * lay.I * 4) + T * lay.D * 2 + T * lay.K * lay.I * 4
        res["gate_up_us"] = gu_ms * 1e3
        res["gate_up_gbs"] = gu_bytes / (gu_ms * 1e-3) / 1e9
        res["gate_up_hbm_frac"] = res["gate_up_gbs"] / HBM_PEAK_GBS
        res["_gate_up_bytes"] = gu_bytes
    if router_fn is not None:
        res["hot8_share"] = hot_share(bounds, xs)
    log(f"bench: decode T={T} ({impl}{', skewed' if router_fn else ''}): {res['us_per_step']:.1f} us/step "
        f"({res['graph_us_per_step']:.1f} from a graph), layer HBM {res['layer_hbm_frac']:.3f}")  # fmt: skip
    return res


def prefill_point(layers, T, args, dev, router_fn=None, roofline=False, seed=11):
    import torch

    bounds = [Bound(lay, T, router=router_fn(lay) if router_fn else None) for lay in layers]
    xs = make_x_list(T, layers[0].D, len(layers), seed + T, dev, skew=router_fn is not None)
    outs = [torch.empty(T, layers[0].D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    steps = max(10, args.steps // 2)
    secs = time_forward(bounds, xs, outs, steps, max(args.warmup, 3))
    step_s = secs / steps
    lay = layers[0]
    fl = prefill_flops(lay, T)
    lb = decode_bytes(lay, T, lay.E)  # every expert is active at these sizes
    res = {
        "us_per_step": step_s * 1e6,
        "tokens_per_s": T / step_s,
        "layer_tflops": fl / step_s / 1e12,
        "layer_mfma_frac": fl / step_s / 1e12 / BF16_PEAK_TFLOPS,
        "layer_hbm_frac": lb / step_s / 1e9 / HBM_PEAK_GBS,
    }
    if router_fn is not None:
        res["hot8_share"] = hot_share(bounds, xs)
    if roofline:
        gms, _ = time_gate_up(bounds, xs, steps, decode=False)
        flops_gu = 2.0 * T * lay.K * lay.D * 2 * lay.I
        tf = flops_gu / (gms * 1e-3) / 1e12
        res["roofline"] = {
            "kernel": "k_gemm<true> (gate/up grouped GEMM + SwiGLU)",
            "bound": "mfma",
            "achieved": tf,
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": tf / BF16_PEAK_TFLOPS,
            "traffic": measured_traffic("k_gemm_gateup", f"prefill_T{T}"),
            "algorithmic_flops_per_launch": flops_gu,
            "mean_launch_us": gms * 1e3,
        }
    log(f"bench: prefill T={T}{' (skewed)' if router_fn else ''}: {res['us_per_step']:.1f} us/step, "
        f"MFMA {res['layer_mfma_frac']:.3f}")  # fmt: skip
    return res


def near_ties(router, xs, K, exact_products=True):
    """Tokens whose canonical K-th / (K+1)-th logit gap another fp32 summation order
    could close (the reference sums the router product in XLA's order,
    kappa/qwen3/ffn_moe.py:50): any order of the D products is within
    gamma * S_e of the exact sum, S_e = sum_d |x_d r_de|, gamma = n u / (1 - n u),
    u = 2^-24, n = D (D + 1 when the products round: f32 inputs); two orders are
    within 2 gamma S_e of each other. A token with gap <= 2 gamma (S_K + S_K+1) may
    select a different K-th expert under XLA's order; the others cannot."""
    import torch

    from kappa_amd.qwen3 import moe_stages

    D, E = router.shape
    n = D if exact_products else D + 1
    u = 2.0**-24
    gamma = n * u / (1.0 - n * u)
    within, total, worst, differs = 0, 0, float("inf"), 0
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    for x in xs:
        lg = moe_stages.route(x, router, num_experts=E, k=K)["logits"]
        S = x.abs().float() @ router.abs().float()
        vals, order = torch.sort(lg, dim=1, descending=True, stable=True)
        gap = (vals[:, K - 1] - vals[:, K]).double()
        bound = 2.0 * gamma * (S.gather(1, order[:, K - 1 : K]) + S.gather(1, order[:, K : K + 1])).double()[:, 0]
        within += int((gap <= bound).sum())
        total += x.shape[0]
        worst = min(worst, float((gap / bound).min()))
        # the same products summed in another order: torch's f32 GEMM
        alt = torch.sort(x.float() @ router.float(), dim=1, descending=True, stable=True)[1][:, :K]
        differs += int((alt != order[:, :K]).any(dim=1).sum())
    torch.backends.cuda.matmul.allow_tf32 = prev
    return {"tokens": total, "within_order_bound": within, "min_gap_over_bound": worst,
            "topk_differs_under_f32_gemm_order": differs}  # fmt: skip


def library_reference(T, D, I, E, K, reps=10):
    """hipBLASLt (torch.bmm, bf16) on the prefill expert shapes with uniform
    routing, M = T*K/E rows per expert, bf16 weights (no int8 conversion, no
    gather, no SwiGLU): a vendor-library reference point for the grouped GEMMs,
    not part of the block."""
    import torch

    dev = torch.device("cuda:0")
    M = T * K // E
    out = {}
    for name, (bs, m, k, n) in (("gate_up_bmm", (E, M, D, 2 * I)), ("down_bmm", (E, M, I, D))):
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


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(layer, T_decode, T_prefill, budget_s=10.0):
    """The oracle (C, OpenMP) on the ragged program, on bounded samples of the same
    workloads: full layer calls at decode T_decode, then at a prefill chunk
    T_prefill (a per-expert GEMM loop, which is what the ragged program's
    ragged_dot computes)."""
    import oracle

    host = layer.host()
    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    res = {}
    for kind, T, max_reps in (("decode", T_decode, 20), ("prefill", T_prefill, 5)):
        x = layer_x_host(T, layer.D)
        oracle.forward(x, host["router"], host["gate"], host["up"], host["down"], k=layer.K, act_bf16=True,
                       impl="ragged")  # warm  # fmt: skip
        times = []
        t_start = time.perf_counter()
        while len(times) < max_reps and (time.perf_counter() - t_start) < budget_s:
            t0 = time.perf_counter()
            oracle.forward(x, host["router"], host["gate"], host["up"], host["down"], k=layer.K, act_bf16=True,
                           impl="ragged")  # fmt: skip
            times.append(time.perf_counter() - t0)
        res[kind] = (T, statistics.median(times), len(times))
    Td, md, nd = res["decode"]
    Tp, mp, npf = res["prefill"]
    return {
        "value": Td / md,
        "unit": "tokens/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "sample": (f"{nd} full layer calls at decode T={Td} (30B-A3B W8, bf16, ragged program), median "
                   f"{md * 1e3:.1f} ms; CPU: {_cpu_name()}"),  # fmt: skip
        "prefill": {
            "value": Tp / mp,
            "unit": "tokens/s",
            "sample": f"{npf} full layer calls at a prefill chunk of T={Tp}, median {mp * 1e3:.1f} ms",
        },
    }


def layer_x_host(T, D, seed=99):
    import numpy as np

    from inputs import bf16_rne

    rng = np.random.default_rng(seed)
    return bf16_rne(rng.standard_normal((T, D)).astype(np.float32))


def bench_235b(args, dev):
    """The 235B-A22B-shaped W8 layer (D 4096, E 128, K 8, I 1536, ~2.4 GB of
    int8 experts): decode T=16 (HBM fraction) and prefill T=2048 (MFMA
    fraction), two weight copies in rotation."""
    import torch

    from moe_cases import make_layer

    log("bench: building 2 weight copies of the 235B-A22B W8 layer")
    big = [make_layer("235b", seed=40 + i) for i in range(2)]
    res = {"decode_T16": decode_point(big, 16, args, dev), "prefill_T2048": prefill_point(big, 2048, args, dev)}
    res["routing_near_ties"] = {
        "decode_T16": near_ties(big[0].router, make_x_list(16, big[0].D, 8, 7 + 16, dev), big[0].K),
        "prefill_T2048": near_ties(big[0].router, make_x_list(2048, big[0].D, 2, 11 + 2048, dev), big[0].K),
    }
    for v in res.values():
        v.pop("_gate_up_bytes", None)
    del big
    torch.cuda.empty_cache()
    return res


def floor_probe():
    """What a kernel costs before it does any work, and how fast a cold stream of
    the T=1 layer's weight sizes moves, on this device: a one-element fill (one
    block) launched 200 times back to back, eagerly and from a graph; and
    elementwise passes (bitwise not: one read and one write per byte, a launch
    grid per size) whose sources rotate over enough buffers (> 256 MB) that every
    pass reads from HBM, with the traffic of the T=1 layer's weights (12.6 MB,
    the down weights of 8 experts; 25.2 MB, their gate and up weights; 37.7 MB,
    all three)."""
    import torch

    dev = torch.device("cuda:0")
    t = torch.zeros(1, device=dev)

    def per_launch(fn, n=200, graph=False):
        if graph:
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                fn()
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    for _ in range(n):
                        fn()
            torch.cuda.current_stream().wait_stream(s)
            run = g.replay
        else:

            def run():
                for _ in range(n):
                    fn()

        run()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            run()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / n)
        return best

    res = {
        "fill_1_element_us_eager": per_launch(lambda: t.fill_(1.0)),
        "fill_1_element_us_graph": per_launch(lambda: t.fill_(1.0), graph=True),
        "cold_stream": {},
    }
    for mb, what in ((12.6, "down weights of 8 experts"), (25.2, "gate/up weights of 8 experts"),
                     (37.7, "all weights of 8 experts")):  # fmt: skip
        n = int(mb * 1e6 / 2) // 256 * 256  # n bytes read and n written
        nbuf = max(2, int(400e6 // n) + 1)
        srcs = [torch.full((n,), i, dtype=torch.uint8, device=dev) for i in range(nbuf)]
        dst = torch.empty(n, dtype=torch.uint8, device=dev)
        times = []
        for r in range(3 * nbuf):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            torch.bitwise_not(srcs[r % nbuf], out=dst)
            e1.record()
            torch.cuda.synchronize()
            if r >= nbuf:
                times.append(e0.elapsed_time(e1) * 1e3)
        times.sort()
        us = times[len(times) // 2]
        res["cold_stream"][f"{mb}MB"] = {"traffic_bytes": 2 * n, "us": us, "GBps": 2 * n / us / 1e3, "as": what}
        del srcs, dst
    log(f"bench: floor {res}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    # the first ~100 steps after the weight build run ~6% slower (clocks and
    # caches settling); 100 untimed steps cost ~12 ms
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--quick", action="store_true", help="only the 30B decode and prefill points")
    ap.add_argument(
        "--only-235b",
        action="store_true",
        help="only the 235B-A22B layer's decode T=16 and prefill T=2048 points (for kernel traces)",
    )
    ap.add_argument("--decode", default="1,8,32,64", help="decode token counts; the largest is the headline")
    ap.add_argument("--prefill", default="512,2048,4096", help="prefill token counts ('' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument(
        "--copy-calibration",
        type=int,
        default=0,
        metavar="MIB",
        help="only run 5 device-to-device copies of MIB MiB (the known-size kernel that scales the "
        "FETCH_SIZE / WRITE_SIZE counters) and exit",
    )
    ap.add_argument(
        "--floor",
        action="store_true",
        help="only time the floors the small decode batches are measured against (a one-block kernel, "
        "back to back and in a graph; cold streams of the T=1 layer's weight sizes) and exit",
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

    if args.floor:
        print(json.dumps({"floor": floor_probe()}), flush=True)
        return

    from kappa_amd import _lib
    from moe_cases import make_layer, skew_router

    _lib.lib()
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only_235b:
        print(json.dumps({"layer_235b": bench_235b(args, dev)}), flush=True)
        return
    R = args.copies
    log(f"bench: building {R} weight copies of the 30B-A3B W8 layer")
    layers = [make_layer("30b", seed=i) for i in range(R)]
    lay0 = layers[0]
    D, E, K, I = lay0.D, lay0.E, lay0.K, lay0.I

    # headline: the largest decode batch asked for (T=64 by default)
    dall = sorted({int(v) for v in args.decode.split(",") if v})
    T = dall[-1]
    dh = decode_point(layers, T, args, dev)
    gu_bytes = dh.pop("_gate_up_bytes")
    result = {
        "metric": METRIC,
        "value": dh["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dh["us_per_step"] / 1e3,
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
            "program": "moe_impl ragged_jax, decode threshold 0 (_moe_ragged rounding points)",
            "weight_copies_rotated": R,
        },
        "roofline": {
            "kernel": "k_gateup_decode",
            "bound": "hbm",
            "achieved": dh["gate_up_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dh["gate_up_hbm_frac"],
            "traffic": measured_traffic("k_gateup_decode", f"decode_T{T}"),
            "algorithmic_bytes_per_launch": gu_bytes,
            "mean_launch_us": dh["gate_up_us"],
            "active_experts": dh["active_experts"],
        },
        "layer_hbm_gbs": dh["layer_hbm_gbs"],
        "layer_hbm_frac": dh["layer_hbm_frac"],
    }
    decode = {str(T): dh}
    for Ts in dall[:-1]:
        p = decode_point(layers, Ts, args, dev)
        p.pop("_gate_up_bytes", None)
        decode[str(Ts)] = p
    result["decode"] = {str(k): decode[str(k)] for k in dall}

    # the steps either side of the block: rms_norm in, residual add out. The
    # fused call, the three separate calls and the bare MoE layer are timed in
    # interleaved rounds (the clock drifts over a run); medians are reported.
    bounds = [Bound(lay, T) for lay in layers]
    xs = make_x_list(T, D, R, 77, dev)
    outs = [torch.empty(T, D, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    scale = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    rounds = {"fused": [], "separate": [], "moe_only": []}
    n_round = max(args.steps // 3, 5)
    for _ in range(3):
        rounds["fused"].append(time_block(bounds, xs, outs, scale, n_round, 2, fused=True) / n_round)
        rounds["separate"].append(time_block(bounds, xs, outs, scale, n_round, 2, fused=False) / n_round)
        rounds["moe_only"].append(time_forward(bounds, xs, outs, n_round, 2) / n_round)
    med = {k: sorted(v)[len(v) // 2] * 1e6 for k, v in rounds.items()}
    result["block"] = {
        "workload": f"h + moe_layer(rms_norm(h)), decode T={T}",
        "fused_us_per_step": med["fused"],
        "separate_us_per_step": med["separate"],
        "moe_only_us_per_step": med["moe_only"],
        "rounds": f"3 interleaved rounds of {n_round} steps, medians",
    }
    del bounds

    # prefill chunks on two copies (the weights stream once per call; MFMA-bound at 4096)
    pl = layers[:2]
    prefill = {}
    for Tp in sorted({int(v) for v in args.prefill.split(",") if v}):
        prefill[str(Tp)] = prefill_point(pl, Tp, args, dev, roofline=(Tp == 4096))
    if prefill:
        top = prefill[str(max(int(k) for k in prefill))]
        result["prefill"] = {
            "workload": "qwen3-30b-a3b W8 MoE layer, prefill chunks (ragged program)",
            "tokens_per_s": top["tokens_per_s"],
            "ms_per_step": top["us_per_step"] / 1e3,
            "layer_tflops": top["layer_tflops"],
            "layer_mfma_frac": top["layer_mfma_frac"],
            "roofline": top.pop("roofline", None),
            "chunks": prefill,
        }

    if not args.quick:
        # Zipf(1.2)-skewed routing: the bias enters through x[:, 0] = 1 and router row 0
        skewed = {id(lay): skew_router(lay.router, lam=1.5) for lay in layers}

        def sk(lay):
            return skewed[id(lay)]

        s64 = decode_point(layers, 64, args, dev, router_fn=sk)
        s64.pop("_gate_up_bytes", None)
        result["skew"] = {"decode_T64": s64, "prefill_T4096": prefill_point(pl, 4096, args, dev, router_fn=sk)}
        del skewed
        # the gather program (the reference's default) on per-tensor W8 at decode T=64
        gl = [make_layer("30b", seed=100 + i, per_tensor=True) for i in range(min(R, 4))]
        gd = decode_point(gl, 64, args, dev, impl="gather_einsum", threshold=64)
        gd["program"] = "moe_impl gather_einsum, per-tensor W8 (bf16 scale)"
        result["gather_decode_T64"] = gd
        del gl
        if "prefill" in result:
            result["prefill"]["library_reference"] = library_reference(4096, D, I, E, K)

    if not args.quick:
        # routing near ties against another summation order, per measured
        # workload (the inputs of the timed points above)
        from inputs import GOLDEN_SPECS, make_inputs

        margins = {}
        for Td in dall:
            margins[f"30b_decode_T{Td}"] = near_ties(lay0.router, make_x_list(Td, D, 8, 7 + Td, dev), K)
        for Tp in sorted({int(v) for v in args.prefill.split(",") if v}):
            margins[f"30b_prefill_T{Tp}"] = near_ties(lay0.router, make_x_list(Tp, D, 2, 11 + Tp, dev), K)
        sr = skew_router(lay0.router, lam=1.5)
        margins["30b_skew_decode_T64"] = near_ties(sr, make_x_list(64, D, 8, 7 + 64, dev, skew=True), K)
        margins["30b_skew_prefill_T4096"] = near_ties(sr, make_x_list(4096, D, 2, 11 + 4096, dev, skew=True), K)
        toy = next(sp for sp in GOLDEN_SPECS if sp.name == "toy_f32")
        ti = make_inputs(toy)
        margins["toy_f32_T64"] = near_ties(torch.from_numpy(ti["router"]).to(dev), [torch.from_numpy(ti["x"]).to(dev)],
                                           toy.K, exact_products=False)  # fmt: skip
        result["routing_near_ties"] = margins
        log(f"bench: routing near ties {margins}")

    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle)")
        result["cpu_baseline"] = cpu_baseline(lay0, 64, 512)
        log(f"bench: cpu {result['cpu_baseline']}")
    else:
        result["cpu_baseline"] = None

    if not args.quick:
        del layers, pl, lay0
        from kappa_amd.qwen3.ffn_moe import PACK_CACHE

        PACK_CACHE.clear()
        torch.cuda.empty_cache()
        result["layer_235b"] = bench_235b(args, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
