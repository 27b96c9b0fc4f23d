#!/usr/bin/env python3
"""Benchmark of the W8A8 fused-MoE layer on one MI355X.

Default workload (the metric's config): W8A8 INT8
decode MoE layer, DeepSeek-V3/V4 shape -- T=64 tokens, H=7168, I=2048, 256
routed experts top-8 (softmax, renormalise, x2.5) + 1 shared expert,
weights N(0, 0.02) bf16 quantised per output channel, dynamic per-token int8
activations. A step is one call of ``fused_moe_w8a8_tiled_with_shared`` on
inputs resident in HBM. Prints ONE JSON line.

``--config c3`` / ``c4`` run the prefill configs, ``c1`` / ``c0`` the BF16
ones and ``c1w8`` the W8A16 one; ``--tokens`` overrides a config's token
count. The default C2 line also carries, as ``secondary`` entries, decode at
T=1 and T=2 on the C2 layer (timed over at least 1000 steps), C3 and C4
prefill, and C1 (BF16), each with its own kernel roofline, layer roofline and
sampled bit-exact parity check.

roofline: the dominant kernel (largest GPU time per step among the grouped
GEMM tile-class launches) is timed live with hipEvents recorded by libfcmoe
on the launch stream (fcmoe_stage_timing_*); its algorithmic bytes/ops come
from the realised routing: active experts' weight and scale bytes plus the
stage's activation rows in and out (ops: 2 x MACs).
cpu_baseline: the repo tests' PyTorch eager reference (tests/test_moe_w8a8.py:
40-69, restated grouped per expert with float64 GEMMs) on this host's torch
threads, timed on a seeded uniform sample of the active experts and scaled to
the layer; cpu_baseline_oracle: the C oracle (oracle/, OpenMP) on the same
sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
CLASS_BM = (16, 32, 64, 128, 192, 256)

CONFIGS = {
    "c0": dict(kind="bf16", T=32, H=1024, I=512, E=8, k=2, shared=False, scale=1.0, skew=None,
               desc="C0 BF16 fused MoE plumbing: T=32 H=1024 I=512 E=8 top-2"),
    "c1": dict(kind="bf16", T=32, H=7168, I=2048, E=256, k=8, shared=True, scale=2.5, skew=None,
               desc="C1 BF16 DSv3 decode: T=32 H=7168 I=2048 E=256 top-8 +1 shared"),
    "c2": dict(kind="w8a8", T=64, H=7168, I=2048, E=256, k=8, shared=True, scale=2.5, skew=None,
               desc="C2 W8A8 DSv3 decode: T=64 H=7168 I=2048 E=256 top-8 +1 shared"),
    "c3": dict(kind="w8a8", T=4096, H=7168, I=2048, E=256, k=8, shared=True, scale=2.5, skew=1.2,
               desc="C3 W8A8 DSv3 prefill: T=4096 Zipf(1.2) routing, +1 shared"),
    "c4": dict(kind="w8a8", T=8192, H=7168, I=2048, E=384, k=8, shared=True, scale=2.5, skew=None,
               desc="C4 W8A8 prefill: T=8192 H=7168 I=2048 E=384 top-8 +1 shared"),
    # not a BASELINE config: the C1 decode shape on the W8A16 path (int8 weights, bf16 activations)
    "c1w8": dict(kind="w8a16", T=32, H=7168, I=2048, E=256, k=8, shared=True, scale=2.5, skew=None,
                 desc="C1 shape on W8A16: T=32 H=7168 I=2048 E=256 top-8 +1 shared, int8 weights"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_routing(cfg, seed: int = 0):
    """Router of the config text: softmax top-k renormalised x scale; C3 Zipf-skewed."""
    rng = np.random.default_rng(seed)
    T, E, k = cfg["T"], cfg["E"], cfg["k"]
    if cfg["skew"] is None:
        logits = rng.standard_normal((T, E)).astype(np.float32)
        z = np.exp(logits - logits.max(1, keepdims=True))
        p = z / z.sum(1, keepdims=True)
        ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
        w = np.take_along_axis(p, ids, 1)
        w = w / w.sum(1, keepdims=True)
        return ids.astype(np.int64), w.astype(np.float32), None
    # Zipf popularity over a random expert permutation, Gumbel-top-k without
    # replacement; sharpened (tau) until some expert receives no token.
    for tau in (1.0, 0.5, 0.25):
        perm = rng.permutation(E)
        pz = np.empty(E)
        pz[perm] = np.arange(1, E + 1, dtype=np.float64) ** (-cfg["skew"])
        pz /= pz.sum()
        g = np.log(pz)[None, :] / tau + rng.gumbel(size=(T, E))
        ids = np.argsort(-g, axis=1, kind="stable")[:, :k]
        if (np.bincount(ids.reshape(-1), minlength=E) == 0).any():
            break
    sel = np.take_along_axis(g, ids, 1)
    w = np.exp(sel - sel.max(1, keepdims=True))
    w = w / w.sum(1, keepdims=True)
    return ids.astype(np.int64), w.astype(np.float32), tau


def make_x(cfg, device):
    """Token rows x ~ N(0, 1) as bf16 on the device (seed 7)."""
    import torch

    rng = np.random.default_rng(7)
    return torch.from_numpy(rng.standard_normal((cfg["T"], cfg["H"])).astype(np.float32)).to(device).to(torch.bfloat16)


def build_layer(cfg, device, keep_host_int8: bool, keep_device_int8: bool = False):
    """Random N(0, 0.02) bf16 experts (+shared), quantised per channel and packed on the GPU.

    Returns (prepared weights, host int8 copy or None); with keep_device_int8 a
    third item holds the unpacked device tensors (q13, s13, q2, s2)."""
    import torch

    from fused_cpp_amd import cabi
    from fused_cpp_amd.moe import PreparedW8A8TiledFusedMoEWeights, PreparedW8A8TiledRoutedSharedMoEWeights

    L = cabi.lib()
    stream = cabi.stream_handle()
    E = cfg["E"] + (1 if cfg["shared"] else 0)
    H, I = cfg["H"], cfg["I"]
    g = torch.Generator(device=device).manual_seed(1234)
    q13 = torch.empty((E, 2 * I, H), dtype=torch.int8, device=device)
    q2 = torch.empty((E, H, I), dtype=torch.int8, device=device)
    s13 = torch.empty((E, 2 * I), dtype=torch.float32, device=device)
    s2 = torch.empty((E, H), dtype=torch.float32, device=device)
    for e in range(E):
        for q, s, shape in ((q13, s13, (2 * I, H)), (q2, s2, (H, I))):
            w = (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * 0.02).to(torch.bfloat16)
            cabi.check(L.fcmoe_quantize_weight_rows(w.data_ptr(), shape[0], shape[1], q[e].data_ptr(),
                                                    s[e].data_ptr(), stream), "quantize")
    per13 = L.fcmoe_packed_expert_bytes(1, 2 * I, H, 2)
    per2 = L.fcmoe_packed_expert_bytes(1, H, I, 1)
    p13 = torch.empty((E, per13), dtype=torch.int8, device=device)
    p2 = torch.empty((E, per2), dtype=torch.int8, device=device)
    cabi.check(L.fcmoe_pack_experts(q13.data_ptr(), 1, E, 2 * I, H, 2, p13.data_ptr(), stream), "pack13")
    cabi.check(L.fcmoe_pack_experts(q2.data_ptr(), 1, E, H, I, 1, p2.data_ptr(), stream), "pack2")
    torch.cuda.synchronize()
    packed = PreparedW8A8TiledFusedMoEWeights(w13=(p13, H, 2 * I, s13), w2=(p2, I, H, s2))
    host = None
    if keep_host_int8:
        host = (q13.cpu().numpy(), s13.cpu().numpy(), q2.cpu().numpy(), s2.cpu().numpy())
    dev_int8 = (q13, s13, q2, s2) if keep_device_int8 else None
    del q13, q2
    torch.cuda.empty_cache()
    if cfg["shared"]:
        weights = PreparedW8A8TiledRoutedSharedMoEWeights(packed=packed, routed_experts=cfg["E"],
                                                          shared_expert_id=cfg["E"])
    else:
        weights = packed
    if keep_device_int8:
        return weights, host, dev_int8
    return weights, host


def build_bf16_layer(cfg, device, keep_device: bool = False):
    """Random N(0, 0.02) bf16 experts (+shared), packed on the GPU; with
    keep_device the unpacked (w13, w2) device tensors are returned as well."""
    import torch

    from fused_cpp_amd.moe import (PreparedBF16TiledRoutedSharedMoEWeights, prepare_fused_moe_bf16_tiled_weights)

    E = cfg["E"] + (1 if cfg["shared"] else 0)
    H, I = cfg["H"], cfg["I"]
    g = torch.Generator(device=device).manual_seed(1234)
    w13 = (torch.randn((E, 2 * I, H), generator=g, device=device) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device=device) * 0.02).to(torch.bfloat16)
    packed = prepare_fused_moe_bf16_tiled_weights(w13, w2, fuse_silu=True)
    kept = (w13, w2) if keep_device else None
    del w13, w2
    torch.cuda.empty_cache()
    if cfg["shared"]:
        packed = PreparedBF16TiledRoutedSharedMoEWeights(packed=packed, routed_experts=cfg["E"],
                                                         shared_expert_id=cfg["E"])
    return (packed, kept) if keep_device else packed


def expert_counts(cfg, ids):
    E = cfg["E"] + (1 if cfg["shared"] else 0)
    counts = np.bincount(ids.reshape(-1), minlength=E).astype(np.int64)
    if cfg["shared"]:
        counts[cfg["E"]] += cfg["T"]
    return counts


CLASS_BM_PREFILL = (16, 128, 192, 256)  # W8A8 / BF16 prefill tile classes
CLASS_BM_W8 = (16, 32, 128, 192, 256)  # W8A16 tile classes


def class_of(c: int, decode: bool, kind: str = "w8a8") -> int:
    """Tile class (its index in CLASS_BM) the GPU selector assigns to an expert
    with c rows (fcmoe_api.hip select_classes; W8A16 uses its own class set)."""
    if decode:
        return 0
    bms = CLASS_BM_W8 if kind == "w8a16" else CLASS_BM_PREFILL
    for bm in bms:
        if c <= bm:
            return CLASS_BM.index(bm)
    return CLASS_BM.index(bms[-1])


def prefill_plan(counts) -> tuple[str, int]:
    """The W8A8 prefill launch plan the device picks for these expert row
    counts ("mixed", "classic" or "partitioned" with its CUs for the 256-row
    class), from the library's own rule (fcmoe_w8a8_prefill_plan). Tile
    counts: one tile per expert of 1-192 rows, ceil(rows / 256) above."""
    from fused_cpp_amd import cabi

    counts = np.asarray(counts)
    t = [int(((counts > 0) & (counts <= 16)).sum()), int(((counts > 16) & (counts <= 128)).sum()),
         int(((counts > 128) & (counts <= 192)).sum()), int(np.ceil(counts[counts > 192] / 256).sum())]
    return cabi.w8a8_prefill_plan(t)


def algorithmic(cfg, counts):
    """Algorithmic HBM bytes and ops of the layer and of each GEMM stage class.

    Layer bytes = active experts' weights + scales, x in, out, ids + weights;
    ops = 2 * MACs = routed rows * 6 * H * I (int8 or bf16)."""
    H, I = cfg["H"], cfg["I"]
    eb = 1 if cfg["kind"] in ("w8a8", "w8a16") else 2
    sb = 4 if cfg["kind"] in ("w8a8", "w8a16") else 0
    active = counts > 0
    rows = int(counts.sum())
    T = cfg["T"]
    layer_bytes = int(active.sum()) * (3 * H * I * eb + (2 * I + H) * sb) + T * H * 2 * 2 + T * cfg["k"] * 12
    layer_ops = rows * 6 * H * I
    stages = {}
    decode = rows <= 8 * len(counts)
    for c in range(len(CLASS_BM)):
        sel = (counts > 0) & (np.array([class_of(int(x), decode, cfg["kind"]) for x in counts]) == c)
        n_exp, r = int(sel.sum()), int(counts[sel].sum())
        if n_exp == 0:
            continue
        stages[f"w13_bm{CLASS_BM[c]}"] = dict(
            bytes=n_exp * (2 * I * H * eb + 2 * I * sb) + r * H * eb + r * I * 2, ops=r * 2 * (2 * I) * H,
            experts=n_exp, rows=r)
        stages[f"w2_bm{CLASS_BM[c]}"] = dict(
            bytes=n_exp * (H * I * eb + H * sb) + r * I * eb + r * H * 4, ops=r * 2 * H * I, experts=n_exp, rows=r)
    if cfg["kind"] == "w8a8" and not decode:
        # The mixed prefill plan's two launches: the persistent MFMA launch
        # (every expert above 16 rows) and the 16-row streaming launch.
        for name, sel in (("mixed_mfma", counts > 16), ("mixed_stream", (counts > 0) & (counts <= 16))):
            n_exp, r = int(sel.sum()), int(counts[sel].sum())
            if n_exp == 0:
                continue
            stages[f"w13_{name}"] = dict(
                bytes=n_exp * (2 * I * H * eb + 2 * I * sb) + r * H * eb + r * I * 2, ops=r * 2 * (2 * I) * H,
                experts=n_exp, rows=r)
            stages[f"w2_{name}"] = dict(
                bytes=n_exp * (H * I * eb + H * sb) + r * I * eb + r * H * 4, ops=r * 2 * H * I, experts=n_exp,
                rows=r)
        # the partitioned classic plan's persistent launch: the 256-row class
        for st in ("w13", "w2"):
            if f"{st}_bm256" in stages:
                stages[f"{st}_part256"] = stages[f"{st}_bm256"]
    return layer_bytes, layer_ops, stages


_LAYERS: dict = {}


def get_layer(cfg, device):
    """Prepared weights for cfg's shape, built once per (kind, shape) and shared
    by every workload of that shape (C2, C3 and the small-batch decode lines
    use the same seeded E=256 layer). Entries also hold the unpacked device
    tensors (int8 + scales, or the bf16 weights), from which parity checks and
    the CPU baselines copy the experts they touch."""
    kind = "w8" if cfg["kind"] in ("w8a8", "w8a16") else "bf16"
    key = (kind, cfg["E"], cfg["H"], cfg["I"], cfg["shared"])
    if key not in _LAYERS:
        import gc

        import torch

        for k in list(_LAYERS):  # one layer resident at a time
            del _LAYERS[k]
        gc.collect()
        torch.cuda.empty_cache()
        t0 = time.time()
        if kind == "w8":
            weights, _, dev = build_layer(cfg, device, False, keep_device_int8=True)
        else:
            weights, dev = build_bf16_layer(cfg, device, keep_device=True)
        log(f"[bench] {cfg['desc']}: weights ready in {time.time() - t0:.1f}s")
        _LAYERS[key] = (weights, dev)
    return _LAYERS[key]


def run_gpu(cfg, steps: int, warmup: int, device, graph: bool = False):
    import torch

    from fused_cpp_amd import cabi
    from fused_cpp_amd import moe
    from fused_cpp_amd.moe import fused_moe_bf16_tiled_with_shared, fused_moe_tiled, fused_moe_w8a8_tiled_with_shared

    ids, w, tau = make_routing(cfg)
    x = make_x(cfg, device)
    ids_d = torch.from_numpy(ids).to(device)
    w_d = torch.from_numpy(w).to(device)
    weights, dev_int8 = get_layer(cfg, device)
    if cfg["kind"] == "w8a8":
        if cfg["shared"]:
            def step(out):
                return fused_moe_w8a8_tiled_with_shared(x, weights, w_d, ids_d, routed_scaling_factor=cfg["scale"],
                                                        out=out)
        else:
            def step(out):
                return fused_moe_tiled(x, weights, w_d, ids_d, swiglu_limit=10.0, out=out)
    elif cfg["kind"] == "w8a16":
        p = weights.packed
        w16 = moe.PreparedW8A16TiledRoutedSharedMoEWeights(
            packed=moe.PreparedW8A16TiledFusedMoEWeights(w13=p.w13, w2=p.w2), routed_experts=weights.routed_experts,
            shared_expert_id=weights.shared_expert_id)

        def step(out):
            return moe.fused_moe_w8a16_tiled_with_shared(x, w16, w_d, ids_d, routed_scaling_factor=cfg["scale"],
                                                         out=out)
    else:
        if cfg["shared"]:
            def step(out):
                return fused_moe_bf16_tiled_with_shared(x, weights, w_d, ids_d, routed_scaling_factor=cfg["scale"],
                                                        out=out)
        else:
            def step(out):
                return fused_moe_tiled(x, weights, w_d, ids_d, out=out)
    out = torch.empty_like(x)
    for _ in range(max(warmup, 1)):
        step(out)
    torch.cuda.synchronize()
    run = step
    if graph:
        # One whole forward captured into a HIP graph and replayed per step: the
        # same kernels on the same HBM-resident inputs, without per-launch host cost.
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(out)
        g.replay()
        torch.cuda.synchronize()

        def run(o):
            g.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cabi.stage_timing_read()  # clear
    start.record()
    for _ in range(steps):
        run(out)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # Per-stage kernel durations: a separate pass with event pairs around each launch.
    cabi.stage_timing_enable(True)
    for _ in range(steps):
        step(out)
    torch.cuda.synchronize()
    stages = cabi.stage_timing_read()
    cabi.stage_timing_enable(False)
    return dict(ms=ms, stages=stages, ids=ids, w=w, tau=tau, x=x, out=out, dev_int8=dev_int8)


def _host_experts(dev_int8, experts: np.ndarray):
    """Host copies (numpy) of the given experts' int8 weights and scales."""
    import torch

    q13, s13, q2, s2 = dev_int8
    sel = torch.from_numpy(np.ascontiguousarray(experts, np.int64)).to(q13.device)
    return tuple(t.index_select(0, sel).cpu().numpy() for t in (q13, s13, q2, s2))


def _expert_sample(cfg, ids, budget_experts: int, seed: int = 5):
    """A seeded uniform sample of the active experts (shared one included with
    its share of probability): timing a uniform subset of experts and scaling
    by active/sampled estimates the whole layer without bias."""
    counts = expert_counts(cfg, ids)
    active = np.nonzero(counts > 0)[0]
    rng = np.random.default_rng(seed)
    n = min(budget_experts, len(active))
    return np.sort(rng.choice(active, n, replace=False)), len(active), counts


def _expert_routes(cfg, ids, experts: np.ndarray):
    """For each expert: its flat routes (t*kt + s) in ascending order."""
    kt = cfg["k"] + (1 if cfg["shared"] else 0)
    T = cfg["T"]
    routes = []
    for e in experts:
        if cfg["shared"] and e == cfg["E"]:
            r = np.arange(T, dtype=np.int64) * kt + cfg["k"]
        else:
            t, s = np.nonzero(ids == e)
            r = np.sort(t.astype(np.int64) * kt + s)
        routes.append(r)
    return routes, kt


def torch_eager_expert_layer(x_bf16, ids, w, cfg, experts, host, routes):
    """Grouped per-expert restatement, in PyTorch eager on the CPU, of the
    reference test's W8A8 reference (tests/test_moe_w8a8.py:40-69): per-token
    quantisation (round half to even, as torch.round), int8 GEMMs accumulated
    exactly in float64, fp32 dequantisation, clamped SiLU-mul to bf16,
    requantisation, the down GEMM, and the routing-weighted sum over slots in
    fp32. Returns the fp32 [T, H] partial output of the given experts."""
    import torch

    q13, s13, q2, s2 = (torch.from_numpy(a) for a in host)
    T, Hd = x_bf16.shape
    I = q2.shape[2]
    kt = cfg["k"] + (1 if cfg["shared"] else 0)
    xf = x_bf16.float()
    xs = (xf.abs().amax(1) / 127.0).clamp_min(1.0e-30)
    xq = (xf / xs[:, None]).round().clamp(-127, 127).double()
    wt = torch.from_numpy(w)
    out = torch.zeros((T, Hd), dtype=torch.float32)
    for j, e in enumerate(experts):
        r = torch.from_numpy(routes[j])
        if r.numel() == 0:
            continue
        tok, slot = r // kt, r % kt
        if cfg["shared"] and e == cfg["E"]:
            rw = torch.ones(r.numel(), dtype=torch.float32)
        else:
            rw = wt[tok, slot] * cfg["scale"] if cfg["shared"] else wt[tok, slot]
        acc = (xq[tok] @ q13[j].double().T).float() * xs[tok][:, None] * s13[j]
        gate = acc[:, :I].clamp(max=10.0)
        up = acc[:, I:].clamp(-10.0, 10.0)
        act = (gate * up / (1.0 + torch.exp(-gate))).to(torch.bfloat16).float()
        s_act = (act.abs().amax(1) / 127.0).clamp_min(1.0e-30)
        aq = (act / s_act[:, None]).round().clamp(-127, 127).double()
        route = (aq @ q2[j].double().T).float() * s_act[:, None] * s2[j]
        out.index_add_(0, tok, route * rw[:, None])
    return out


def cpu_threads() -> tuple[int, int]:
    """(host CPUs as os.cpu_count() reports them, CPUs this process may run
    on). The CPU baselines run torch on the second: on a shared GPU box the
    affinity mask is the host share this job holds."""
    n_host = os.cpu_count() or 1
    try:
        n_use = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n_use = n_host
    return n_host, max(1, min(n_use, n_host))


def _set_torch_threads() -> tuple[int, int]:
    import torch

    n_host, n_use = cpu_threads()
    torch.set_num_threads(n_use)
    return n_host, torch.get_num_threads()


def _median_time(fn, reps: int = 3) -> float:
    fn()  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_baseline_torch(cfg, res, budget_experts: int):
    """The north-star CPU baseline: the repo tests' PyTorch eager reference
    (grouped per expert, float64 accumulation) on this host's cores, timed on
    a seeded uniform sample of the active experts and scaled to the layer;
    median of 3 after 1 warmup."""
    import torch

    experts, n_active, _ = _expert_sample(cfg, res["ids"], budget_experts)
    host = _host_experts(res["dev_int8"], experts)
    routes, _ = _expert_routes(cfg, res["ids"], experts)
    x = res["x"].cpu()
    n_host, threads = _set_torch_threads()
    t = _median_time(lambda: torch_eager_expert_layer(x, res["ids"], res["w"], cfg, experts, host, routes))
    layer_s = t * n_active / len(experts)
    rows = sum(len(r) for r in routes)
    return {
        "value": round(cfg["T"] / layer_s, 2),
        "unit": "tokens/s",
        "cores": threads,
        "host_cpus": n_host,
        "kind": "torch_eager",
        "sample": f"PyTorch eager grouped restatement of tests/test_moe_w8a8.py:40-69 (float64 GEMMs, "
                  f"torch.set_num_threads({threads}), host os.cpu_count() = {n_host}) on a seeded uniform sample "
                  f"of {len(experts)} of the {n_active} active experts ({rows} routes), median of 3 = {t:.2f}s "
                  f"after 1 warmup, scaled by {n_active}/{len(experts)} to the full layer ({layer_s:.2f}s/layer)",
    }


def _bf16_host_experts(cfg, dev, experts: np.ndarray, exact: bool = False):
    """Host copies of the given experts' [2I, H] and [H, I] weights: the bf16
    layer's own weights, or for W8A16 the int8 weights dequantised, q * s: in
    fp32 with exact=True (the W8A16 tests' reference: the kernel applies the
    fp32 scale to the fp32 accumulator), else rounded to bf16 for the CPU
    baseline's bf16 F.linear."""
    import torch

    sel = torch.from_numpy(np.ascontiguousarray(experts, np.int64))
    if cfg["kind"] == "w8a16":
        q13, s13, q2, s2 = (t.index_select(0, sel.to(t.device)).cpu() for t in dev)
        d13, d2 = q13.float() * s13[..., None], q2.float() * s2[..., None]
        return (d13, d2) if exact else (d13.to(torch.bfloat16), d2.to(torch.bfloat16))
    w13, w2 = dev
    return tuple(t.index_select(0, sel.to(t.device)).cpu() for t in (w13, w2))


def torch_naive_bf16_layer(x_bf16, ids, w, cfg, w13, w2, routes):
    """Grouped per-expert restatement, in PyTorch eager on the CPU, of the
    reference's fused_moe_naive (src/fused_cpp/moe/naive.py:161-272): F.linear
    of each expert's token rows in bf16, SiLU(gate) * up, F.linear, then the
    [T, slots, H] route rows times the routing weights in fp32, summed over
    slots and cast to bf16. Routed+shared calls add the shared expert as one
    more slot of weight 1 with the routed weights scaled (bf16_tiled.py:807-828)."""
    import torch
    import torch.nn.functional as F

    T, Hd = x_bf16.shape
    kt = cfg["k"] + (1 if cfg["shared"] else 0)
    new_x = torch.zeros((T * kt, Hd), dtype=torch.bfloat16)
    for j in range(len(routes)):
        r = torch.from_numpy(routes[j])
        if r.numel() == 0:
            continue
        gate_up = F.linear(x_bf16.index_select(0, r // kt), w13[j])
        d = gate_up.shape[1] // 2
        new_x[r] = F.linear(F.silu(gate_up[:, :d]) * gate_up[:, d:], w2[j])
    wt = torch.from_numpy(w).float() * (cfg["scale"] if cfg["shared"] else 1.0)
    if cfg["shared"]:
        wt = torch.cat([wt, torch.ones((T, 1))], 1)
    return (new_x.view(T, kt, Hd).float() * wt[:, :, None]).sum(1).to(torch.bfloat16)


def cpu_baseline_bf16(cfg, res, budget_experts: int):
    """CPU baseline of the BF16 / W8A16 lines: the reference's PyTorch naive
    MoE (naive.py:161-272, grouped F.linear in bf16) on this host's cores, on a
    seeded uniform sample of the active experts scaled to the layer; median
    of 3 after 1 warmup."""
    experts, n_active, _ = _expert_sample(cfg, res["ids"], budget_experts)
    w13, w2 = _bf16_host_experts(cfg, res["dev_int8"], experts)
    routes, _ = _expert_routes(cfg, res["ids"], experts)
    x = res["x"].cpu()
    n_host, threads = _set_torch_threads()
    t = _median_time(lambda: torch_naive_bf16_layer(x, res["ids"], res["w"], cfg, w13, w2, routes))
    layer_s = t * n_active / len(experts)
    deq = " on the int8 weights dequantised to bf16 (outside the timed region)" if cfg["kind"] == "w8a16" else ""
    return {
        "value": round(cfg["T"] / layer_s, 2),
        "unit": "tokens/s",
        "cores": threads,
        "host_cpus": n_host,
        "kind": "torch_eager",
        "sample": f"PyTorch eager grouped restatement of fused_moe_naive (src/fused_cpp/moe/naive.py:161-272; "
                  f"bf16 F.linear per expert{deq}; torch.set_num_threads({threads}), host os.cpu_count() = "
                  f"{n_host}) on a seeded uniform sample of {len(experts)} of the {n_active} active experts, "
                  f"median of 3 = {t:.3f}s after 1 warmup, scaled by {n_active}/{len(experts)} to the layer "
                  f"({layer_s:.3f}s/layer)",
    }


def bf16_parity(cfg, res, n: int = 4, tol: float = 2e-2, cos_min: float = 0.9999) -> dict:
    """BF16 / W8A16 outputs of n tokens (the first n-1 and the last) against
    the fp32 oracle (oracle.bf16_moe_reference, the naive semantics; for
    W8A16 on the dequantised weights with the activation output rounded to
    bf16, as its tests do) on the experts they touch; north-star bar max-abs
    <= 2e-2, cosine >= 0.9999."""
    import torch

    import oracle

    T = cfg["T"]
    tok = np.unique(np.array(list(range(min(n - 1, T))) + [T - 1]))
    ids = res["ids"][tok]
    wts = res["w"][tok].astype(np.float32)
    if cfg["shared"]:
        ids = np.concatenate([ids, np.full((len(tok), 1), cfg["E"])], 1)
        wts = np.concatenate([wts * np.float32(cfg["scale"]), np.ones((len(tok), 1), np.float32)], 1)
    touched = np.unique(ids)
    w13, w2 = (t.float().numpy() for t in _bf16_host_experts(cfg, res["dev_int8"], touched, exact=True))
    tk = torch.from_numpy(tok).to(res["x"].device)
    x = res["x"][tk].float().cpu().numpy()
    ref = oracle.bf16_moe_reference(x, w13, w2, wts, np.searchsorted(touched, ids),
                                    round_intermediate=cfg["kind"] == "w8a16")
    got = res["out"][tk].float().cpu().numpy().astype(np.float64)
    return _tolerance_report(got, ref, len(tok), tol, cos_min)


def _bf16_half_ulp(x):
    """Half a bf16 ulp at each |x|: the rounding a correctly rounded bf16
    output carries against an fp32 reference (0.031 at |x| >= 8)."""
    _, e = np.frexp(np.abs(np.asarray(x, np.float64)))
    return np.ldexp(1.0, e - 9)


def _tolerance_report(got, ref, n: int, tol: float = 2e-2, cos_min: float = 0.9999) -> dict:
    """max-abs error against the fp32 reference, raw and beyond the bf16
    output's own rounding (half an ulp of the reference value; the bound
    applies to this part), and the cosine."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    excess = float((diff - _bf16_half_ulp(ref)).max())
    cos = float((got * ref).sum() / np.sqrt((got * got).sum() * (ref * ref).sum() + 1e-300))
    return {"tokens_checked": int(n), "max_abs": round(float(diff.max()), 6),
            "max_abs_beyond_bf16_rounding": round(excess, 6), "cosine": round(cos, 7),
            "tolerance": f"max-abs beyond the bf16 output rounding <= {tol}, cosine >= {cos_min}",
            "within_tolerance": bool(excess <= tol and cos >= cos_min)}


def cpu_baseline_oracle(cfg, res, budget_experts: int):
    """The C oracle (oracle/, OpenMP), grouped per expert, on the same kind of
    expert sample as cpu_baseline_torch, scaled to the layer."""
    import oracle

    experts, n_active, _ = _expert_sample(cfg, res["ids"], budget_experts)
    host = _host_experts(res["dev_int8"], experts)
    routes, kt = _expert_routes(cfg, res["ids"], experts)
    offsets = np.zeros(len(experts) + 1, np.int64)
    offsets[1:] = np.cumsum([len(r) for r in routes])
    sorted_routes = np.concatenate(routes).astype(np.int64)
    x_bits = res["x"].cpu().view(__import__("torch").int16).numpy().view(np.uint16)
    route_out = np.zeros((cfg["T"] * kt, cfg["H"]), np.float32)
    q13, s13, q2, s2 = host
    oracle.w8a8_expert_range(x_bits, sorted_routes, offsets, kt, q13, s13, q2, s2, 0, min(2, len(experts)),
                             route_out)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.w8a8_expert_range(x_bits, sorted_routes, offsets, kt, q13, s13, q2, s2, 0, len(experts), route_out)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    layer_s = t * n_active / len(experts)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(cfg["T"] / layer_s, 2),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"C oracle grouped W8A8 (OpenMP, {threads} threads) on the same {len(experts)}-of-{n_active} "
                  f"expert sample, median of 3 = {t:.2f}s, scaled to the layer ({layer_s:.2f}s/layer)",
    }


def parity_check(cfg, res, n: int = 4) -> dict:
    """Bit-exact check of n tokens (the first n-1 and the last) against the
    oracle, on host copies of only the experts they touch."""
    import oracle

    T = cfg["T"]
    tok = np.unique(np.array(list(range(min(n - 1, T))) + [T - 1]))
    sid = cfg["E"] if cfg["shared"] else -1
    touched = np.unique(res["ids"][tok])
    local = np.searchsorted(touched, res["ids"][tok])
    experts = np.append(touched, sid) if sid >= 0 else touched
    q13, s13, q2, s2 = _host_experts(res["dev_int8"], experts)
    import torch

    tk = torch.from_numpy(tok).to(res["x"].device)
    x_bits = res["x"][tk].cpu().view(torch.int16).numpy().view(np.uint16)
    ref = oracle.w8a8_forward(x_bits, local, res["w"][tok], q13, s13, q2, s2,
                              shared_id=len(experts) - 1 if sid >= 0 else -1, routed_scale=cfg["scale"])
    got = res["out"][tk].cpu().view(torch.int16).numpy().view(np.uint16)
    return {"tokens_checked": int(len(tok)), "bit_exact": bool(np.array_equal(ref, got))}


def measured_traffic(config: str, stage: str):
    """HBM bytes per launch of `stage` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (calibrated against a plain copy), if that workload was profiled."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"w8a8_decode_{config}_traffic.json")
    if not os.path.exists(path):
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"w8a8_prefill_{config}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][stage]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def kernel_roofline(workload: str, best, st_alg, peak_ops):
    """Roofline of the dominant GEMM stage: its algorithmic bytes or ops over its
    average launch time (library hipEvents on the launch stream)."""
    name, tot, n = best
    avg_ms = tot / n
    a = st_alg[name]
    t_bytes = a["bytes"] / (HBM_PEAK_GBPS * 1e9)
    t_ops = a["ops"] / (peak_ops * 1e12)
    if t_bytes >= t_ops:
        achieved = a["bytes"] / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4)}
    else:
        achieved = a["ops"] / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak_ops, "unit": "TFLOP/s",
                "frac": round(achieved / peak_ops, 4)}
    traffic = measured_traffic(workload, name)
    roof.update({"kernel": f"grouped_gemm {name}", "avg_launch_ms": round(avg_ms, 4), "traffic": traffic,
                 "algorithmic_bytes": a["bytes"], "algorithmic_ops": a["ops"], "experts": a["experts"],
                 "rows": a["rows"]})
    return roof


# Decode secondaries (a few tokens, ~0.07-0.13 ms per step) time at least this
# many steps: every timed region carries a fixed ~75 us ramp out of idle, 5% of
# a 20-step one-token region (C2 at T=1: 0.0732 ms at 20 steps, 0.0727 at 50,
# 0.0703 at 200, 0.0694 at 1000; T=2 0.1318 -> 0.1291). The main line times
# exactly --steps.
DECODE_MIN_STEPS = 1000


def measure(cfg, workload: str, args, device, want_cpu: bool, min_steps: int = 0, with_oracle: bool = False):
    steps = max(args.steps, min_steps)
    res = run_gpu(cfg, steps, args.warmup, device, graph=args.graph)
    counts = expert_counts(cfg, res["ids"])
    layer_bytes, layer_ops, st_alg = algorithmic(cfg, counts)
    ms = res["ms"]
    plan = None
    if cfg["kind"] == "w8a8" and counts.sum() > 8 * len(counts):
        plan, part = prefill_plan(counts)
        if plan == "partitioned":  # the persistent launch ran the 256-row class, not the mixed plan
            res["stages"] = {k.replace("_mixed_mfma", "_part256"): v for k, v in res["stages"].items()}
    # dominant kernel: largest per-step GPU time among GEMM stages
    best = None
    for name, (tot, n) in res["stages"].items():
        if name in st_alg and (best is None or tot > best[1]):
            best = (name, tot, n)
    peak_ops = INT8_PEAK_TOPS if cfg["kind"] == "w8a8" else BF16_PEAK_TFLOPS
    roof = None
    if best is not None:  # stage classes outside this model (W8A16 at prefill): no kernel roofline
        roof = kernel_roofline(workload, best, st_alg, peak_ops)
    layer_roof_s = max(layer_bytes / (HBM_PEAK_GBPS * 1e9), layer_ops / (peak_ops * 1e12))
    layer = {
        "bytes": layer_bytes, "ops": layer_ops, "active_experts": int((counts > 0).sum()),
        "zero_token_experts": int((counts[: cfg["E"]] == 0).sum()),
        "hbm_TBps": round(layer_bytes / (ms * 1e-3) / 1e12, 3),
        "ops_TOPS": round(layer_ops / (ms * 1e-3) / 1e12, 2),
        "int8_mfma_frac": round(layer_ops / (ms * 1e-3) / 1e12 / peak_ops, 4),
        "roofline_ms": round(layer_roof_s * 1e3, 4),
        "roofline_frac": round(layer_roof_s * 1e3 / ms, 4),
        "stage_ms_per_step": {k: round(v[0] / steps, 4) for k, v in res["stages"].items()},
    }
    if cfg["kind"] != "w8a8":
        layer["bf16_mfma_frac"] = layer.pop("int8_mfma_frac")
    if res.get("tau") is not None:
        layer["zipf_tau"] = res["tau"]
    if plan is not None:
        layer["prefill_plan"] = plan if plan != "partitioned" else f"partitioned ({part} CUs for the 256-row class)"
    out = {"ms": ms, "steps": steps, "tokens_per_s": cfg["T"] / (ms * 1e-3), "roofline": roof, "layer": layer}
    out["parity"] = parity_check(cfg, res) if cfg["kind"] == "w8a8" else bf16_parity(cfg, res)
    if want_cpu:
        if cfg["kind"] == "w8a8":
            out["cpu_baseline"] = cpu_baseline_torch(cfg, res, args.cpu_experts)
            if with_oracle:
                out["cpu_baseline_oracle"] = cpu_baseline_oracle(cfg, res, args.cpu_experts)
        else:
            out["cpu_baseline"] = cpu_baseline_bf16(cfg, res, args.cpu_experts)
    del res
    return out


# Extra workloads measured by default after the headline one, each on its own
# layer: decode at small batches, the same C2 layer and T=1 with the id check
# off (FUSED_CPP_AMD_VALIDATE_IDS=0; every other line runs the operators'
# default, the check on), the prefill configs, the BF16 configs, W8A16 at the
# C1 shape and at T=4096. (workload, config, tokens, validate_ids)
SECONDARY = [("c2_t1", "c2", 1, True), ("c2_t2", "c2", 2, True), ("c2_t8", "c2", 8, True),
             ("c2_t32", "c2", 32, True), ("c2_no_validate_ids", "c2", 0, False),
             ("c2_t1_no_validate_ids", "c2", 1, False),
             ("c3", "c3", 0, True), ("c4", "c4", 0, True), ("c1", "c1", 0, True), ("c0", "c0", 0, True),
             ("c1w8", "c1w8", 0, True), ("c1w8_t4096", "c1w8", 4096, True)]

# The other operators of the drop-in surface, at DeepSeek-V3.2-shaped sizes
# (public model config: hidden 7168, q_lora_rank 1536, main Q projection
# 128 heads x 192 = 24576, indexer Q projection 64 heads x 128 = 8192, output
# projection 128 x 128 = 16384 -> 7168): the i8gemm pair (one quantisation,
# two GEMMs; deepseek_v4_w8a8.py:114-132), the single i8gemm (wo_b,
# :135-143), both at decode (64 rows) and prefill (4096 rows), and the BF16
# shared MLP (bf16_tiled.py:1805-1873) at T=64. (workload, op, M, K, N list)
OP_SECONDARY = [("i8gemm_pair_q_m64", "pair", 64, 1536, (24576, 8192)),
                ("i8gemm_pair_q_m4096", "pair", 4096, 1536, (24576, 8192)),
                ("i8gemm_wo_b_m64", "single", 64, 16384, (7168,)),
                ("i8gemm_wo_b_m128", "single", 128, 16384, (7168,)),
                ("i8gemm_wo_b_m512", "single", 512, 16384, (7168,)),
                ("i8gemm_wo_b_m4096", "single", 4096, 16384, (7168,)),
                ("shared_mlp_t64", "shared_mlp", 64, 7168, (2048,)),
                ("shared_mlp_t128", "shared_mlp", 128, 7168, (2048,))]


def _time_op(fn, steps: int, warmup: int):
    """ms per call of fn on the current stream (torch events), then one pass
    with the library's stage timing on: {stage: (total ms, launches)}."""
    import torch

    from fused_cpp_amd import cabi

    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    cabi.stage_timing_read()
    cabi.stage_timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    stages = cabi.stage_timing_read()
    cabi.stage_timing_enable(False)
    return ms, stages


def _op_roofline(stages, steps: int, names, alg_bytes: int, alg_ops: int, peak_ops: float, kernel: str):
    """Roofline of an operator's GEMM launches (stage names `names`): their
    algorithmic bytes / ops per step over their GPU time per step."""
    tot = sum(stages[n][0] for n in names if n in stages)
    launches = sum(stages[n][1] for n in names if n in stages)
    if not launches:
        return None
    t_s = tot / steps * 1e-3
    if alg_bytes / (HBM_PEAK_GBPS * 1e9) >= alg_ops / (peak_ops * 1e12):
        ach = alg_bytes / t_s / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBPS, 4)}
    else:
        ach = alg_ops / t_s / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": peak_ops, "unit": "TFLOP/s",
                "frac": round(ach / peak_ops, 4)}
    roof.update({"kernel": kernel, "avg_launch_ms": round(tot / launches, 4), "launches_per_step": launches // steps,
                 "traffic": None, "algorithmic_bytes": alg_bytes, "algorithmic_ops": alg_ops})
    return roof


def measure_op(wl: str, op: str, M: int, K: int, Ns, args, device, want_cpu: bool) -> dict:
    """One operator secondary: time, kernel roofline, parity (i8gemm bit-exact
    vs the oracle on 4 rows; shared MLP within the north-star tolerance of the
    fp32 reference) and a CPU baseline (PyTorch eager on the host)."""
    import torch
    import torch.nn.functional as F

    import oracle
    from fused_cpp_amd import i8gemm as ig
    from fused_cpp_amd.moe import prepare_shared_mlp_bf16_tiled_weights, shared_mlp_bf16_tiled

    g = torch.Generator(device=device).manual_seed(99)
    x = torch.randn((M, K), generator=g, device=device).to(torch.bfloat16)
    steps = max(args.steps, 100 if M <= 128 else 0)
    entry = {"workload": wl}
    if op == "shared_mlp":
        I = Ns[0]
        w13 = (torch.randn((1, 2 * I, K), generator=g, device=device) * 0.02).to(torch.bfloat16)
        w2 = (torch.randn((1, K, I), generator=g, device=device) * 0.02).to(torch.bfloat16)
        prepared = prepare_shared_mlp_bf16_tiled_weights(w13[0], w2[0])
        out = torch.empty_like(x)

        def fn():
            return shared_mlp_bf16_tiled(x, prepared, out=out)

        ms, stages = _time_op(fn, steps, args.warmup)
        gemm = [n for n in stages if n.startswith(("w13_", "w2_"))]
        alg_b = 3 * K * I * 2 + 2 * M * K * 2
        alg_o = 6 * M * K * I
        entry.update({"workload": f"BF16 shared MLP (one dense SwiGLU expert), T={M}, H={K}, I={I}",
                      "dtype": "bf16", "tokens_per_s": round(M / (ms * 1e-3), 1)})
        roof = _op_roofline(stages, steps, gemm, alg_b, alg_o, BF16_PEAK_TFLOPS, "grouped_gemm (W13 + W2 launches)")
        tok = np.unique(np.array([0, 1, M // 2, M - 1]).clip(0, M - 1))
        xs = x[torch.from_numpy(tok).to(device)].float().cpu().numpy()
        ref = oracle.bf16_moe_reference(xs, w13.float().cpu().numpy(), w2.float().cpu().numpy(),
                                        np.ones((len(tok), 1), np.float32), np.zeros((len(tok), 1), np.int64))
        got = out[torch.from_numpy(tok).to(device)].float().cpu().numpy()
        entry["parity"] = _tolerance_report(got, ref, len(tok))
        if want_cpu:
            hx, h13, h2 = x.cpu(), w13[0].cpu(), w2[0].cpu()
            n_host, threads = _set_torch_threads()

            def cpu():
                gu = F.linear(hx, h13)
                return F.linear(F.silu(gu[:, :I]) * gu[:, I:], h2)

            t = _median_time(cpu)
            entry["cpu_baseline"] = {
                "value": round(M / t, 2), "unit": "tokens/s", "cores": threads, "host_cpus": n_host,
                "kind": "torch_eager",
                "sample": f"the whole op: PyTorch eager bf16 F.linear -> SiLU * up -> F.linear (naive.py:161-272 "
                          f"with one expert, weight 1), torch.set_num_threads({threads}), median of 3 = {t * 1e3:.2f} "
                          f"ms after 1 warmup"}
    else:
        ws, preps = [], []
        for n in Ns:
            w = torch.randint(-127, 128, (n, K), generator=g, device=device, dtype=torch.int8)
            sc = torch.rand((n,), generator=g, device=device) * 0.004 + 0.0005
            ws.append((w, sc))
            preps.append(ig.prepare(w, sc))
        if op == "pair":
            fn = lambda: ig.dynamic_scaled_mm_pair(x, preps[0], preps[1])  # noqa: E731
        else:
            fn = lambda: ig.dynamic_scaled_mm(x, preps[0])  # noqa: E731
        ms, stages = _time_op(fn, steps, args.warmup)
        outs = fn()
        outs = outs if isinstance(outs, tuple) else (outs,)
        torch.cuda.synchronize()
        gemm = [n for n in stages if n.startswith("w13_")]
        alg_b = sum(n * K + 4 * n + M * K + M * n * 2 for n in Ns)
        alg_o = sum(2 * M * K * n for n in Ns)
        shape = " + ".join(f"[{n}, {K}]" for n in Ns)
        entry.update({"workload": f"i8gemm {'dynamic_scaled_mm_pair' if op == 'pair' else 'dynamic_scaled_mm'}: "
                                  f"x [{M}, {K}] bf16 against {shape} int8, bf16 out",
                      "dtype": "int8", "rows_per_s": round(M / (ms * 1e-3), 1)})
        roof = _op_roofline(stages, steps, gemm, alg_b, alg_o, INT8_PEAK_TOPS, "grouped_gemm (i8gemm GEMM launches)")
        rows = np.unique(np.array([0, 1, M // 2, M - 1]).clip(0, M - 1))
        xr = x[torch.from_numpy(rows).to(device)].cpu().view(torch.int16).numpy().view(np.uint16)
        ok = True
        for (w, sc), o in zip(ws, outs):
            ref = oracle.i8gemm(xr, w.cpu().numpy(), sc.cpu().numpy(), None, True)
            got = o[torch.from_numpy(rows).to(device)].cpu().view(torch.int16).numpy().view(np.uint16)
            ok = ok and bool(np.array_equal(ref, got))
        entry["parity"] = {"rows_checked": len(rows), "bit_exact": ok}
        if want_cpu:
            hx = x.cpu()
            hw = [(w.cpu().double(), sc.cpu()) for w, sc in ws]
            n_host, threads = _set_torch_threads()

            def cpu():
                # tests/test_deepseek_v4_w8a8.py:19-50: per-row scale max|x|/127, round
                # half to even, clamp +-127, exact integer GEMM (float64), fp32 scales, bf16
                f = hx.float()
                m = f.abs().amax(1, keepdim=True)
                s_x = torch.where(m > 0, m / 127.0, torch.ones_like(m))
                q = (f / s_x).round().clamp(-127, 127).double()
                return [((q @ w.T).float() * s_x * sc).to(torch.bfloat16) for w, sc in hw]

            t = _median_time(cpu)
            entry["cpu_baseline"] = {
                "value": round(M / t, 2), "unit": "rows/s", "cores": threads, "host_cpus": n_host,
                "kind": "torch_eager",
                "sample": f"the whole op: PyTorch eager restatement of tests/test_deepseek_v4_w8a8.py:19-50 "
                          f"(quantise once, float64 integer GEMMs), torch.set_num_threads({threads}), median of 3 "
                          f"= {t * 1e3:.1f} ms after 1 warmup"}
    entry.update({"ms_per_step": round(ms, 4), "steps": steps, "roofline": roof,
                  "stage_ms_per_step": {k: round(v[0] / steps, 4) for k, v in stages.items()}})
    return entry


def int_mm_reference() -> int:
    """hipBLASLt int8 GEMM throughput at the shapes of C3/C4's large experts:
    W13 of a 4096/2048/1792-row expert ([M, 7168] x [7168, 4096]), W2 of the
    shared expert ([4096, 2048] x [2048, 7168]) and C4's shared W13 (8192 rows)."""
    import torch

    dev = torch.device("cuda", 0)
    out = []
    for m, k, n in [(4096, 7168, 4096), (2048, 7168, 4096), (1792, 7168, 4096), (4096, 2048, 7168),
                    (8192, 7168, 4096)]:
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev)
        b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev).t()
        for _ in range(3):
            torch._int_mm(a, b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch._int_mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        out.append({"m": m, "k": k, "n": n, "us": round(ms * 1e3, 1), "TOPS": round(2 * m * k * n / ms / 1e9)})
    print(json.dumps({"int_mm_reference": out}))
    return 0


def probe_lib():
    """libfcmoe_probe.so (fused_cpp_amd/csrc/fcmoe_probe.h): the measurement
    probes, built beside libfcmoe.so but not part of the operator library."""
    import ctypes

    from fused_cpp_amd import build as fbuild

    if not fbuild.PROBE_LIB.exists():
        raise RuntimeError(f"{fbuild.PROBE_LIB} is not built (python -m fused_cpp_amd.build)")
    lib = ctypes.CDLL(str(fbuild.PROBE_LIB))
    P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    for name, args in {"fcmoe_probe_stream": [P, I64, I, I, I, I, P, P], "fcmoe_probe_mfma": [I, I, I, I, P, P],
                       "fcmoe_probe_mix": [P, I64, I, I, I, I, P, P], "fcmoe_probe_fence": [P, I64, I, I, I, P, P, P],
                       "fcmoe_probe_ring": [P, I64, P, I64, I, I, I, I, P, P],
                       "fcmoe_probe_loop_dma": [P, I64, I, I, P, P]}.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = I, args
    return lib


def probes() -> int:
    """Chip figures the design relies on, from the probe kernels
    (libfcmoe_probe.so, fused_cpp_amd/csrc/fcmoe_probe.h): HBM streaming by launch shape (loads to
    VGPRs and LDS-DMA), the MFMA + LDS-fragment loop by wave tile and waves per
    SIMD, MFMA waves beside streaming waves on one CU, one agent-scope
    release per workgroup, and the prefill GEMM's weight + A-row load mix. Best of 5 launches after 1 warmup (torch events on
    the launch stream)."""
    import torch

    from fused_cpp_amd import cabi

    L = probe_lib()
    cabi.lib()
    dev = torch.device("cuda", 0)
    stream = cabi.stream_handle()
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    src = torch.ones(2 << 30, dtype=torch.uint8, device=dev)
    counters = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    rows = torch.empty(64 << 20, dtype=torch.uint8, device=dev)

    def best_ms(launch, reps=5, before=None):
        times = []
        for r in range(reps + 1):
            if before:
                before()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            cabi.check(launch(), "probe")
            b.record()
            torch.cuda.synchronize()
            if r:
                times.append(a.elapsed_time(b))
        return min(times)

    out = {"stream": [], "mfma": [], "mix": [], "fence": []}
    for nbytes, wgs, waves, mode, pad in [(2 << 30, 256, 8, 0, 0), (2 << 30, 256, 8, 1, 0), (2 << 30, 144, 8, 0, 98304),
                                          (2 << 30, 128, 8, 0, 98304), (2 << 30, 128, 8, 1, 98304),
                                          (2 << 30, 64, 8, 0, 98304), (2 << 30, 64, 8, 1, 98304),
                                          (2 << 30, 1152, 1, 0, 0), (2 << 30, 4096, 8, 0, 0),
                                          (264 << 20, 256, 8, 0, 0), (264 << 20, 144, 8, 0, 0)]:
        ms = best_ms(lambda: L.fcmoe_probe_stream(src.data_ptr(), nbytes, wgs, waves, mode, pad, sink.data_ptr(),
                                                  stream))
        moved = nbytes // 1024 // (wgs * waves) * (wgs * waves) * 1024
        out["stream"].append({"bytes": moved, "workgroups": wgs, "waves": waves,
                              "path": "lds_dma" if mode else "vgpr_nontemporal", "lds_pad": pad,
                              "us": round(ms * 1e3, 1), "TBps": round(moved / ms / 1e9, 3),
                              "GBps_per_busy_cu": round(moved / ms / 1e6 / min(wgs, 256), 1)})
    for tile, name, waves in [(0, "128x96", 8), (0, "128x96", 4), (1, "128x64", 8), (1, "128x64", 12),
                              (2, "96x80", 12), (3, "64x96", 12), (4, "64x64", 8), (4, "64x64", 16)]:
        fm, fn = [int(v) // 16 for v in name.split("x")]
        iters = 20000 // (fm * fn) * 8
        ms = best_ms(lambda: L.fcmoe_probe_mfma(tile, waves, 256, iters, sink.data_ptr(), stream))
        ops = 256 * waves * iters * fm * fn * 32768
        out["mfma"].append({"wave_tile": name, "waves_per_cu": waves, "reads_per_mfma": round((fm + fn) / (fm * fn), 3),
                            "us": round(ms * 1e3, 1), "POPS": round(ops / ms / 1e12, 3)})
    iters = 4000
    for nc, ns, smfma in [(8, 0, 0), (0, 4, 0), (0, 8, 0), (8, 4, 0), (8, 8, 0), (8, 8, 1), (4, 4, 0), (4, 0, 0)]:
        ms = best_ms(lambda: L.fcmoe_probe_mix(src.data_ptr(), 2 << 30, nc, ns, iters, smfma, sink.data_ptr(), stream))
        moved = (2 << 30) // 1024 // (256 * ns) // 8 * 8 * 1024 * 256 * ns if ns else 0
        ops = 256 * nc * iters * 7 * 32768
        out["mix"].append({"compute_waves": nc, "stream_waves": ns, "stream_mfma": bool(smfma),
                           "us": round(ms * 1e3, 1), "POPS": round(ops / ms / 1e12, 3),
                           "TBps": round(moved / ms / 1e9, 3)})
    for wgs, waves, rel in [(144, 8, 0), (144, 8, 1), (3552, 8, 0), (3552, 8, 1)]:
        ms = best_ms(lambda: L.fcmoe_probe_fence(src.data_ptr(), 264 << 20, wgs, waves, rel, counters.data_ptr(),
                                                 rows.data_ptr(), stream), before=counters.zero_)
        out["fence"].append({"workgroups": wgs, "waves": waves, "release_per_workgroup": bool(rel),
                             "bytes": 264 << 20, "us": round(ms * 1e3, 1)})
    arows = torch.ones(16 << 20, dtype=torch.uint8, device=dev)
    big = torch.ones(3 << 30, dtype=torch.uint8, device=dev)
    out["ring"] = []
    for wgs in (256, 96):
        for la, na, bar in [(2, 0, 1), (2, 2, 1), (4, 2, 1), (6, 2, 1), (2, 2, 0)]:
            nbytes = 3 << 30 if wgs == 256 else 1 << 30
            ms = best_ms(lambda: L.fcmoe_probe_ring(big.data_ptr(), nbytes,
                                                    arows.data_ptr(), arows.numel(), wgs, la, na, bar, sink.data_ptr(), stream))
            chunks = nbytes // (wgs * 8 * 4 * 1024)
            wb, ab = wgs * chunks * 32768, wgs * chunks * 8 * na * 1024
            out["ring"].append({"workgroups": wgs, "lookahead": la, "a_kib_per_chunk": 8 * na, "barrier": bool(bar),
                                "us": round(ms * 1e3, 1), "weights_TBps": round(wb / ms / 1e9, 3),
                                "GBps_per_cu": round((wb + ab) / ms / 1e6 / wgs, 1)})
    out["loop_dma"] = []
    iters = 4000
    for mode in (0, 1, 2, 3, 7):
        ms = best_ms(lambda: L.fcmoe_probe_loop_dma(src.data_ptr(), 1 << 20, mode, iters, sink.data_ptr(), stream))
        ops = 256 * 8 * iters * 32 * 32768
        out["loop_dma"].append({"barrier": bool(mode & 1), "lds_dma_kib_per_cu": 32 if mode & 2 else 0,
                                "wait_before_barrier": bool(mode & 4), "us": round(ms * 1e3, 1),
                                "POPS": round(ops / ms / 1e12, 3)})
    print(json.dumps({"probes": out}))
    return 0


def item_trace(cfg) -> int:
    """Per-item timing of the persistent LDS launches (W13 and W2 epilogues)
    of one forward, from a diagnostic build's item trace: per row-count class
    the mean K-loop and epilogue microseconds, the launch span, the idle
    fraction of the workgroups' time and the per-XCD end times. Once with the
    production launch path, once with the serial stage-timing path."""
    import ctypes

    import torch

    from fused_cpp_amd import cabi
    from fused_cpp_amd.moe import fused_moe_w8a8_tiled_with_shared

    L = cabi.lib()
    if not hasattr(L, "fcmoe_diag_item_trace"):
        print(json.dumps({"error": "libfcmoe.so is not a diagnostic build with the item trace (--diag 4)",
                          "lib": str(cabi.LIB_PATH)}))
        return 2
    fn = L.fcmoe_diag_item_trace
    fn.restype, fn.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]
    dev = torch.device("cuda", 0)
    weights, _ = get_layer(cfg, dev)
    ids, w, _ = make_routing(cfg)
    x = make_x(cfg, dev)
    ids_d, w_d = torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)
    out = torch.empty_like(x)

    def forward():
        fused_moe_w8a8_tiled_with_shared(x, weights, w_d, ids_d, routed_scaling_factor=cfg["scale"], out=out)

    for _ in range(3):
        forward()
    torch.cuda.synchronize()
    buf = np.zeros(2 * 256 * 64 * 4, dtype=np.uint64)
    res = {"workload": cfg["desc"], "clock_MHz": 100}
    for mode in ("production", "serial"):
        cabi.stage_timing_enable(mode == "serial")
        zeros = np.zeros_like(buf)
        cabi.check(fn(zeros.ctypes.data, 1), "item trace clear")
        forward()
        torch.cuda.synchronize()
        cabi.stage_timing_read()
        cabi.check(fn(buf.ctypes.data, 0), "item trace read")
        t = buf.reshape(2, 256, 64, 4).astype(np.int64)
        valid = t[..., 0] > 0
        t0 = t[..., 0][valid].min() if valid.any() else 0
        launches = {}
        for e, name in ((0, "w13"), (1, "w2")):
            v = valid[e]
            if not v.any():
                continue
            T = (t[e, :, :, :3] - t0) / 100.0  # us
            rows = (t[e, :, :, 3] >> 32) & 0xFFFF
            ends = np.where(v, T[:, :, 2], -np.inf).max(1)
            starts = np.where(v, T[:, :, 0], np.inf).min(1)
            used = v.any(1)
            span = float(ends[used].max() - starts[used].min())
            busy = ((T[:, :, 2] - T[:, :, 0]) * v).sum(1)[used]
            kl, ep, r = (T[:, :, 1] - T[:, :, 0])[v], (T[:, :, 2] - T[:, :, 1])[v], rows[v]
            classes = {}
            for lo, hi in ((1, 16), (17, 128), (129, 192), (193, 255), (256, 256)):
                m = (r >= lo) & (r <= hi)
                if m.any():
                    classes[f"{lo}-{hi}"] = {"items": int(m.sum()), "kloop_us": round(float(kl[m].mean()), 1),
                                             "epilogue_us": round(float(ep[m].mean()), 1),
                                             "cu_us_per_wg": round(float((kl + ep)[m].sum() / used.sum()), 1)}
            xe = [round(float(ends[x::8][used[x::8]].max()), 1) if used[x::8].any() else None for x in range(8)]
            launches[name] = {"workgroups": int(used.sum()), "span_us": round(span, 1),
                              "idle_frac": round(1 - float(busy.mean()) / span, 3), "xcd_end_us": xe,
                              "rows_classes": classes}
        res[mode] = launches
    cabi.stage_timing_enable(False)
    print(json.dumps({"item_trace": res}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--tokens", type=int, default=0,
                    help="override the config's token count (e.g. small-batch decode on the C2 shape)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="measure only the selected config (by default the C2 line also carries C3, C4, decode "
                         "at T=1 and T=2, and C1 as 'secondary' entries)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of one forward captured into a HIP graph (removes per-launch host cost)")
    ap.add_argument("--cpu-experts", type=int, default=24,
                    help="active experts in the seeded sample the CPU baselines are timed on")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (scale reference for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--int-mm-reference", action="store_true",
                    help="only time the vendor int8 GEMM (torch._int_mm -> hipBLASLt, int32 out, no gather "
                         "or epilogue) at the prefill experts' shapes, as a reference point for the grouped "
                         "kernels' TOPS")
    ap.add_argument("--probe", action="store_true",
                    help="only run the library's measurement probes (streaming ceiling, MFMA loop rates, MFMA "
                         "beside streaming waves, release-fence cost) and print them as one JSON line")
    ap.add_argument("--ops", action="store_true",
                    help="only run the operator entries (i8gemm, i8gemm pair, shared MLP at the DeepSeek V4 "
                         "shapes) and print them as one JSON line")
    ap.add_argument("--item-trace", action="store_true",
                    help="only trace the persistent prefill launches' items (a diagnostic build: python -m "
                         "fused_cpp_amd.build --diag 4 --out DIR, run with LD_LIBRARY_PATH=DIR FCMOE_LIB_DIR=DIR) "
                         "for one production and one serial forward of --config; prints one JSON line")
    args = ap.parse_args()
    if args.item_trace:
        return item_trace(CONFIGS[args.config])
    if args.ops:
        if args.gpus != 1:
            print(json.dumps({"error": "this build measures one GPU only: run with --gpus 1"}))
            return 2
        import torch

        device = torch.device("cuda", 0)
        ops = [dict(measure_op(wl, op, M, K, Ns, args, device, want_cpu=not args.no_cpu_baseline), name=wl)
               for wl, op, M, K, Ns in OP_SECONDARY]
        print(json.dumps({"ops": ops}), flush=True)
        return 0
    if args.probe:
        return probes()
    if args.int_mm_reference:
        return int_mm_reference()
    if args.copy_calibration:
        import torch

        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 256 << 20, "launches": 5}))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: every box has one MI355X; "
                                   "run with --gpus 1"}))
        return 2
    # the operators' default: the id check on (it waits only for each call's
    # route launch)
    os.environ.setdefault("FUSED_CPP_AMD_VALIDATE_IDS", "1")
    import torch

    device = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    if args.tokens > 0:
        cfg = dict(cfg, T=args.tokens, desc=f"{cfg['desc']} (T overridden to {args.tokens})")
    workload = args.config if args.tokens <= 0 else f"{args.config}_t{args.tokens}"
    res = measure(cfg, workload, args, device, want_cpu=not args.no_cpu_baseline, with_oracle=True)
    line = {
        "metric": {"w8a8": "W8A8", "w8a16": "W8A16", "bf16": "BF16"}[cfg["kind"]] + " MoE-layer tokens/s",
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if cfg["kind"] == "w8a8" else "bf16",
        "data": "synthetic (seeded random N(0,0.02) weights, N(0,1) activations and router logits)",
        "config": {"workload": cfg["desc"], "tokens": cfg["T"], "hidden": cfg["H"], "intermediate": cfg["I"],
                   "routed_experts": cfg["E"], "top_k": cfg["k"], "shared_experts": int(cfg["shared"]),
                   "routed_scaling": cfg["scale"], "parallelism": "single GPU",
                   "validate_ids": os.environ.get("FUSED_CPP_AMD_VALIDATE_IDS", "1") != "0",
                   "launch": "hip_graph_replay" if args.graph else "eager"},
        "roofline": res["roofline"],
        "layer": res["layer"],
    }
    if "parity" in res:
        line["parity"] = res["parity"]
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
        line["cpu_baseline_oracle"] = res["cpu_baseline_oracle"]
    if args.config == "c2" and args.tokens <= 0 and not args.no_secondary:
        line["secondary"] = []
        for wl, name, tokens, validate in SECONDARY:
            c = CONFIGS[name] if tokens <= 0 else dict(CONFIGS[name], T=tokens,
                                                       desc=f"{CONFIGS[name]['desc']}, run at T={tokens}")
            if not validate:
                c = dict(c, desc=f"{c['desc']}, id check off (FUSED_CPP_AMD_VALIDATE_IDS=0)")
            log(f"[bench] secondary {wl}: {c['desc']}")
            default_validate = os.environ["FUSED_CPP_AMD_VALIDATE_IDS"]
            os.environ["FUSED_CPP_AMD_VALIDATE_IDS"] = "1" if validate else "0"
            try:
                sec = measure(c, wl, args, device, want_cpu=not args.no_cpu_baseline,
                              min_steps=DECODE_MIN_STEPS if c["T"] <= 8 else 0)
            finally:
                os.environ["FUSED_CPP_AMD_VALIDATE_IDS"] = default_validate
            entry = {"workload": c["desc"], "name": wl, "validate_ids": validate,
                     "dtype": "int8" if c["kind"] == "w8a8" else "bf16",
                     "tokens_per_s": round(sec["tokens_per_s"], 1), "ms_per_step": round(sec["ms"], 4), "steps": sec["steps"],
                     "roofline": sec["roofline"], "layer": sec["layer"]}
            for key in ("parity", "cpu_baseline"):
                if key in sec:
                    entry[key] = sec[key]
            line["secondary"].append(entry)
        for wl, op, M, K, Ns in OP_SECONDARY:
            log(f"[bench] secondary {wl}")
            line["secondary"].append(dict(measure_op(wl, op, M, K, Ns, args, device,
                                                     want_cpu=not args.no_cpu_baseline), name=wl))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
