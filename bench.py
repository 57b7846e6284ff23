#!/usr/bin/env python3
"""bench.py — routed-MoE decode layer on one MI355X.

One step = one routed-MoE layer at decode (mxfp4_moe_layer): device gating of
N(0,1) logits over 256 experts (top-8, sigmoid weights renormalised) with the
routing tables, then stage A (W1/W3 + SiLU) and stage B (W2 + weighted combine)
of the expert-indexed MXFP4 grouped GEMV, reading the routed experts in place
from HBM-resident per-layer tensors. At T=1 the gating runs inside stage A
(two launches); for T>1 it is a launch of its own. The K timed steps are timed
twice over all K steps: issued from the host loop, and captured in a HIP graph
and replayed; the faster is the headline (`timing` names it). Inputs are
resident in HBM before the timed region, and the steps cycle over --layers
layers of 256 experts (4 x 3.42 GB) with fresh logits each step, so weights
come from HBM, not the 256 MB MALL.

Prints ONE JSON line. `value` is the layer's algorithmic HBM bytes per step
(unique routed experts x 13,369,344 B + activations + routing) divided by the
step time, in GB/s. `roofline` covers the dominant kernel of that step, the
gated one-token stage A (moe_swiglu_t1_kernel with the gating folded in), timed
alone over back-to-back launches with HIP events on the launch stream;
`stage_b_roofline` the same for stage B. `configs` holds the other
configurations measured in the same run (config 3 at T=4 and T=16, the
reference's routed dispatch, config 4's 43-layer decode sweep and its 512-token
prefill chunk), `kernels` the other drop-in kernels at BASELINE.json's shapes
and the engine's FP8 shapes. `cpu_baseline` times the CPU oracle (dequant +
fp32 matmul, the reference's CPU path) on one step. `read_floor` streams the
byte counts of stage A, stage B and the whole layer once with a read-only
kernel: what the HBM delivers for that many bytes in one pass, beside the
kernels' times (`copy_ceiling_gbs` is torch's 1 GiB copy); the prefill entry
of `configs` has the same for its weight bytes.

    python bench.py [--steps K] [--warmup W] [--tokens T] [--layers L]
                    [--no-configs] [--no-kernels] [--no-cpu-baseline]
    python bench.py --counters     # a short fixed sequence for rocprofv3 counter passes
"""
from __future__ import annotations

import argparse
import json
import re
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "dsv4-flash-gb10-runtime_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "MoE-layer decode µs + MXFP4 grouped GEMV HBM GB/s (% of MI355X peak)"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
E, K, H, O, TOPK = 256, 4096, 2048, 4096, 8
EXPERT_BYTES = 3 * (H * K // 2 + H * K // 32)          # 13,369,344 B (W1 + W3 + W2, packed + scales)
STAGE_A_EXPERT_BYTES = 2 * (H * K // 2 + H * K // 32)  # 8,912,896 B (W1 + W3)
STAGE_B_EXPERT_BYTES = O * H // 2 + O * H // 32         # 4,456,448 B (W2)
MALL_DEFEAT_BYTES = 512 << 20                           # rotate weight copies over >= 2x the 256 MB MALL


VERBOSE = False


def log(msg: str) -> None:
    """Progress on stderr with --verbose only: the driver keeps the last
    2,000 characters of stdout + stderr, which belong to the JSON line."""
    if VERBOSE:
        print(f"[bench] {msg}", file=sys.stderr, flush=True)


def topk_ids(logits: np.ndarray, k: int = TOPK) -> np.ndarray:
    return np.argsort(-logits.astype(np.float64), axis=1, kind="stable")[:, :k]


CSRC = os.path.join(PKG, "csrc")


def source_sha(name: str) -> str:
    """First 12 hex digits of the SHA-256 of a kernel source file (csrc/)."""
    import hashlib
    with open(os.path.join(CSRC, name), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:12]


def _profile_lines(tag: str):
    """Machine-readable lines of profiles/*.md: `SOURCE <file> <sha12>` (the
    kernel sources the profile was taken from) and `<tag> <key> <value> ...
    <file>[,<file>...]`. Yields (key, fields, profile file, stale) where stale
    says that one of the line's source files changed since the profile."""
    d = os.path.join(REPO, "profiles")
    if not os.path.isdir(d):
        return
    for name in sorted(os.listdir(d)):
        if not name.endswith(".md"):
            continue
        with open(os.path.join(d, name)) as f:
            lines = [ln.split() for ln in f]
        shas = {p[1]: p[2] for p in lines if len(p) == 3 and p[0] == "SOURCE"}
        for p in lines:
            if len(p) >= 4 and p[0] == tag:
                files = p[-1].split(",")
                stale = any(fn not in shas or not os.path.exists(os.path.join(CSRC, fn))
                            or source_sha(fn) != shas[fn] for fn in files)
                yield p[1], p[2:-1], "profiles/" + name, stale


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` ("name@T<tokens>") from the rocprofv3
    counter summaries in profiles/*.md (lines `TRAFFIC <kernel>@T<tokens>
    <bytes> <source files>`); returns (bytes, file), or (None, None) when no
    profile has the kernel or its sources changed since the profile."""
    for key, fields, src, stale in _profile_lines("TRAFFIC"):
        if key == kernel and not stale:
            return int(fields[0]), src
    return None, None


def profiled_duration(kernel: str):
    """rocprofv3 kernel-trace average duration (µs) of `kernel`'s launches in
    the bench's own roofline timing (lines `DURATION <kernel>@T<tokens> <µs>
    <dispatches> <source files>` of profiles/*.md); (µs, file) or (None, None)
    when absent or stale."""
    for key, fields, src, stale in _profile_lines("DURATION"):
        if key == kernel and not stale:
            return float(fields[0]), src
    return None, None


def gbs(nbytes: float, us: float) -> float:
    return nbytes / (us * 1e-6) / 1e9


class Timer:
    """HIP events on torch's current stream, which is the stream every
    binding launches on."""

    def __init__(self, torch):
        self.torch = torch
        self.e0 = torch.cuda.Event(enable_timing=True)
        self.e1 = torch.cuda.Event(enable_timing=True)

    def ms(self, fn) -> float:
        self.torch.cuda.synchronize()
        self.e0.record()
        fn()
        self.e1.record()
        self.torch.cuda.synchronize()
        return self.e0.elapsed_time(self.e1)

    def graph_us_per_call(self, fn, n_calls: int, reps: int = 2) -> float:
        """Capture fn() (n_calls launches) once, replay; µs per call."""
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        us = self.ms(lambda: [g.replay() for _ in range(reps)]) * 1e3 / (reps * n_calls)
        del g
        return us


# ------------------------------------------------------------ config 3 ------

def moe_layer_case(torch, dev, layers, T: int, steps: int, warmup: int, seed: int, stages: bool = True) -> dict:
    """Config 3 at T tokens: the layer step (graph and host-issued, the faster
    is reported) and, with `stages`, each launch alone over back-to-back
    launches: the gating + stage A launch(es) (mxfp4_moe_gate_swiglu), stage A
    on given tables (mxfp4_moe_swiglu) and stage B (mxfp4_moe_down)."""
    from runtime import moe, synth
    from runtime import mxfp4_grouped_gemv_binding as gb

    L = len(layers)
    tm = Timer(torch)
    n = warmup + steps
    mods = [moe.RoutedMoELayer(w, topk=TOPK, max_tokens=max(16, T), check=False) for w in layers]
    x = torch.from_numpy(synth.normal_bf16(seed, (T, K)).view(np.int16)).view(torch.bfloat16).to(dev)
    logits_h = synth.gating_logits(seed + 1, n * T, E).reshape(n, T, E)
    logits = torch.from_numpy(logits_h).to(dev)
    uniq = np.array([len(np.unique(topk_ids(logits_h[i]))) for i in range(n)])
    step_bytes = uniq * EXPERT_BYTES + 2 * T * K * 2 + T * TOPK * 8 + T * E * 4

    def step(i):
        mods[i % L].forward(x, logits=logits[i])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graph_us = tm.graph_us_per_call(lambda: [step(i) for i in range(warmup, n)], steps, reps=1)
    host_us = tm.ms(lambda: [step(i) for i in range(warmup, n)]) * 1e3 / steps
    us = min(graph_us, host_us)
    timed_bytes = float(step_bytes[warmup:].mean())
    out = {
        "tokens": T,
        "moe_layer_us": round(us, 3),
        "moe_layer_us_graph": round(graph_us, 3),
        "moe_layer_us_host_issued": round(host_us, 3),
        "timing": "HIP graph replay" if graph_us <= host_us else "launches issued from the host loop",
        "gbs": round(gbs(timed_bytes, us), 1),
        "hbm_frac_of_peak": round(gbs(timed_bytes, us) / HBM_PEAK_GBS, 4),
        "mean_unique_experts": round(float(uniq[warmup:].mean()), 3),
        "algorithmic_bytes_per_step": int(round(timed_bytes)),
    }
    if not stages:
        return out
    # Each launch alone: R steps' worth of routing states, launched back to back.
    R = min(32, n)
    sts = []
    for i in range(R):
        st = gb.MoEStages(layers[i % L].W1, layers[i % L].W3, layers[i % L].W2, T, TOPK, dev)
        st.gate_swiglu(x, logits[i])
        sts.append(st)
    yo = torch.empty(T, O, dtype=torch.bfloat16, device=dev)
    for st in sts:
        st.down(yo)
    torch.cuda.synchronize()
    a_gate_us = tm.graph_us_per_call(lambda: [st.gate_swiglu(x, logits[i]) for i, st in enumerate(sts)], R, reps=4)
    a_us = tm.graph_us_per_call(lambda: [st.swiglu(x) for st in sts], R, reps=2)
    b_us = tm.graph_us_per_call(lambda: [st.down(yo) for st in sts], R, reps=4)
    a_bytes = float(np.mean(uniq[:R] * STAGE_A_EXPERT_BYTES + T * K * 2 + T * E * 4))
    b_bytes = float(np.mean(uniq[:R] * STAGE_B_EXPERT_BYTES + T * O * 2))
    out["stage_us"] = {"gate_swiglu_A": round(a_gate_us, 3), "swiglu_A_tables_given": round(a_us, 3),
                       "down_B": round(b_us, 3)}
    out["stage_gbs"] = {"gate_swiglu_A": round(gbs(a_bytes, a_gate_us), 1),
                        "swiglu_A_tables_given": round(gbs(a_bytes, a_us), 1),
                        "down_B": round(gbs(b_bytes, b_us), 1)}
    out["_stage_bytes"] = (a_bytes, b_bytes)
    del sts
    return out


def routed_dispatch_case(torch, dev, layers, steps: int, warmup: int) -> dict:
    """The reference engine's routed dispatch on the device
    (mxfp4_moe_routed_dispatch: router GEMV over a bf16 [256, 4096] gate,
    sqrt-softplus top-6 x 1.5, expert-indexed grouped GEMV) at T=1, cycling
    over the resident layers; replaces kernel/cpp-engine-mxfp4/routed.cu:373-503
    (host sync, 36 pack copies, grouped GEMV)."""
    from runtime import fill, moe, synth

    L = len(layers)
    k = 6
    tm = Timer(torch)
    gates = []
    for l in range(L):
        # bf16 gate rows of seeded random bits, masked to finite values below
        # 2^-5 (sign bit cleared; timing does not depend on the values)
        g = torch.empty(E, K, dtype=torch.bfloat16, device=dev)
        fill.fill_uniform_u8(g.view(torch.uint8), 5000 + l, 0, 0, 255)
        g.view(torch.int16).bitwise_and_(0x3CFF)
        gates.append(g)
    mods = [moe.RoutedMoELayer(w, topk=k, max_tokens=1, check=False, router_gate=gates[l])
            for l, w in enumerate(layers)]
    n = warmup + steps
    xs = torch.from_numpy(synth.normal_bf16(3500, (n, 1, K)).view(np.int16)).view(torch.bfloat16).to(dev)

    def step(i):
        mods[i % L].forward(xs[i])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graph_us = tm.graph_us_per_call(lambda: [step(i) for i in range(warmup, n)], steps, reps=1)
    host_us = tm.ms(lambda: [step(i) for i in range(warmup, n)]) * 1e3 / steps
    us = min(graph_us, host_us)
    nbytes = k * EXPERT_BYTES + E * K * 2 + 2 * K * 2 + k * 8
    return {
        "tokens": 1, "topk": k, "routed_scale": 1.5,
        "us": round(us, 3), "us_graph": round(graph_us, 3), "us_host_issued": round(host_us, 3),
        "algorithmic_bytes_per_step": int(nbytes),
        "gbs": round(gbs(nbytes, us), 1), "hbm_frac_of_peak": round(gbs(nbytes, us) / HBM_PEAK_GBS, 4),
        "launches": 3,
        "kernels": "router GEMV (mxfp4_moe_router_logits' kernel), gated stage A with sqrt-softplus scoring, stage B",
    }


# ------------------------------------------------------------ config 4 ------

def config4_case(torch, dev, steps: int, warmup: int, n_layers: int = 43) -> dict:
    """a decode sweep over n_layers layers whose 256
    MXFP4 experts are all resident in HBM (147 GB at 43 layers). Each layer
    has a seeded Zipf(1.1) expert popularity; each step routes one token per
    layer by Gumbel-top-8 (runtime.synth.zipf_routing). One step = the
    n_layers routed layers (ids given: mxfp4_moe_grouped_gemv, two launches
    per layer), the layer's input being the previous layer's output (a
    chained decode). Then one 512-token prefill chunk per layer through the
    MFMA grouped GEMM."""
    from runtime import moe, synth
    from runtime import mxfp4_grouped_gemv_binding as gb

    tm = Timer(torch)
    t0 = time.perf_counter()
    log(f"configs[4]: allocating and filling {n_layers} layers x {E} experts "
        f"({n_layers * E * EXPERT_BYTES / 1e9:.1f} GB)")
    layers = [moe.make_moe_weights(40000 + 100 * l, E, K, H, O, dev) for l in range(n_layers)]
    torch.cuda.synchronize()
    fill_s = time.perf_counter() - t0
    n = warmup + steps
    mods = [moe.RoutedMoELayer(w, topk=TOPK, max_tokens=1, check=False) for w in layers]
    ids_h, ids_d, w_d = [], [], []
    for l in range(n_layers):
        ids, w = synth.zipf_routing(4000, n, E, TOPK, 1.1, layer=l)
        ids_h.append(ids)
        ids_d.append(torch.from_numpy(ids).to(dev))
        w_d.append(torch.from_numpy(w).to(dev))
    x0 = torch.from_numpy(synth.normal_bf16(4001, (1, K)).view(np.int16)).view(torch.bfloat16).to(dev)

    def step(i):
        # layer l reads layer l-1's output in place (each layer owns its output buffer)
        x = x0
        for l in range(n_layers):
            x = mods[l].forward(x, ids=ids_d[l][i:i + 1], weights=w_d[l][i:i + 1])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graph_ms = tm.graph_us_per_call(lambda: [step(i) for i in range(warmup, n)], steps, reps=1) / 1e3
    host_ms = tm.ms(lambda: [step(i) for i in range(warmup, n)]) / steps
    ms = min(graph_ms, host_ms)
    uniq = sum(len(np.unique(ids_h[l][i])) for l in range(n_layers) for i in range(warmup, n))
    step_bytes = uniq / steps * EXPERT_BYTES + n_layers * (2 * K * 2 + TOPK * 8)
    decode = {
        "layers": n_layers, "tokens": 1, "steps": steps,
        "ms_per_step": round(ms, 4), "us_per_layer": round(ms * 1e3 / n_layers, 3),
        "us_per_layer_graph": round(graph_ms * 1e3 / n_layers, 3),
        "us_per_layer_host_issued": round(host_ms * 1e3 / n_layers, 3),
        "timing": "HIP graph replay" if graph_ms <= host_ms else "launches issued from the host loop",
        "algorithmic_bytes_per_step": int(step_bytes),
        "gbs": round(gbs(step_bytes, ms * 1e3), 1),
        "hbm_frac_of_peak": round(gbs(step_bytes, ms * 1e3) / HBM_PEAK_GBS, 4),
        "resident_gb": round(n_layers * E * EXPERT_BYTES / 1e9, 2),
        "fill_seconds": round(fill_s, 1),
        "note": "a chained decode: each layer reads the previous layer's output",
    }
    # One 512-token prefill chunk per layer (MFMA grouped GEMM), graph-replayed.
    TP = 512
    xp = torch.from_numpy(synth.normal_bf16(4002, (TP, K)).view(np.int16)).view(torch.bfloat16).to(dev)
    pre_ids, pre_w, pre_uniq = [], [], 0
    for l in range(n_layers):
        ids, w = synth.zipf_routing(4003, TP, E, TOPK, 1.1, layer=l)
        pre_uniq += len(np.unique(ids))
        pre_ids.append(torch.from_numpy(ids).to(dev))
        pre_w.append(torch.from_numpy(w).to(dev))
    ws = torch.empty(gb.prefill_workspace_bytes(TP, TOPK, E, H, O), dtype=torch.uint8, device=dev)
    yout = torch.empty(TP, O, dtype=torch.bfloat16, device=dev)

    def prefill_all():
        for l in range(n_layers):
            gb.mxfp4_moe_prefill(xp, layers[l].W1, layers[l].W3, layers[l].W2, pre_ids[l], pre_w[l],
                                 out=yout, workspace=ws)

    prefill_all()
    torch.cuda.synchronize()
    pre_us = tm.graph_us_per_call(prefill_all, n_layers, reps=1)
    pre_bytes = pre_uniq / n_layers * EXPERT_BYTES + TP * K * 2 + TP * O * 2
    pre_flop = 2.0 * TP * TOPK * (2 * K * H + H * O)
    prefill = {
        "tokens": TP, "layers": n_layers, "us_per_layer": round(pre_us, 2),
        "mean_unique_experts": round(pre_uniq / n_layers, 2),
        "algorithmic_bytes_per_layer": int(pre_bytes),
        "gbs": round(gbs(pre_bytes, pre_us), 1),
        "hbm_frac_of_peak": round(gbs(pre_bytes, pre_us) / HBM_PEAK_GBS, 4),
        "tflops": round(pre_flop / (pre_us * 1e-6) / 1e12, 1),
        "mfma_frac_of_bf16_peak": round(pre_flop / (pre_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "kernel": "v_mfma_f32_16x16x32_bf16 on exactly dequantised MXFP4 weights (4 launches per layer)",
    }
    del layers, mods, ws
    torch.cuda.empty_cache()
    return {"decode": decode, "prefill": prefill}


# ------------------------------------------------------- dense kernels ------

def dense_kernels(torch, dev, cpu: bool, counters: bool = False) -> dict:
    """The other drop-in kernels at BASELINE.json's shapes (dense MXFP4
    configs[0], FP8 configs[2] at T in {1, 8}, RMSNorm + residual configs[1] at
    T in {1, 8, 64}), the FP8 launches at the reference engine's MLA shapes
    (dsv4_engine_mxfp4_wire.cu:395-501), the fused FP8 call sites and the
    router GEMV. Each case replays a HIP graph of at most 2,048 launches that
    rotate over weight copies totalling >= 512 MB (so weights come from HBM),
    µs per launch (launch floor included), algorithmic GB/s and the fraction
    of 8 TB/s, with the CPU oracle's time for one call beside it (cpu=True).
    counters=True runs 32 eager launches per case instead (rocprofv3 counter
    passes)."""
    from oracle import mx  # CPU baseline only
    from runtime import fill
    from runtime import fp8_e4m3_gemv_binding as fp8b
    from runtime import mxfp4_gemv_binding as mxb
    from runtime import mxfp4_grouped_gemv_binding as gb
    from runtime import rmsnorm_fuse_binding as rb
    from runtime import synth

    tm = Timer(torch)

    def u8(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(dev)

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(torch.bfloat16).to(dev)

    def rep(t, n):
        return t.unsqueeze(0).repeat(n, *([1] * t.dim()))

    def n_copies(nbytes_per_copy):
        return max(2, -(-MALL_DEFEAT_BYTES // nbytes_per_copy))

    def copies(t, nbytes_per_copy):
        n = n_copies(nbytes_per_copy)
        return rep(t, n), n

    def time_launches(fn, n_cop):
        if counters:
            for i in range(32):
                fn(i % n_cop)
            torch.cuda.synchronize()
            return float("nan")
        fn(0)
        torch.cuda.synchronize()
        n = min(max(n_cop, 64), 2048)
        return tm.graph_us_per_call(lambda: [fn(i % n_cop) for i in range(n)], n, reps=4)

    def cpu_us(fn):
        if not cpu or counters:
            return None
        t0 = time.perf_counter()
        fn()
        return round((time.perf_counter() - t0) * 1e6, 1)

    def entry(us, nbytes, cpu_time, extra=None):
        g = gbs(nbytes, us)
        e = {"us": round(us, 3), "algorithmic_bytes": int(nbytes), "gbs": round(g, 1),
             "frac_of_peak": round(g / HBM_PEAK_GBS, 4), "cpu_oracle_us": cpu_time}
        if extra:
            e.update(extra)
        return e

    out = {}
    # MXFP4 dense 2048 x 4096
    N0, K0 = 2048, 4096
    p, s = synth.mxfp4_weight(1000, N0, K0)
    x0 = synth.normal_bf16(1001, (K0,))
    P, nP = copies(u8(p[0]), N0 * K0 // 2 + N0 * K0 // 32)
    S = rep(u8(s[0]), nP)
    xd = bf(x0)
    y = torch.empty(N0, dtype=torch.bfloat16, device=dev)
    us = time_launches(lambda i: mxb.mxfp4_gemv(P[i], S[i], xd, out=y), nP)
    out["mxfp4_gemv_m1 2048x4096"] = entry(us, N0 * K0 // 2 + N0 * K0 // 32 + 2 * K0 + 2 * N0,
                                            cpu_us(lambda: mx.mxfp4_gemv(x0, p[0], s[0])))
    del P, S
    # FP8 GEMVs, T in {1, 8}
    for (N, Kf) in ((1536, 4096), (576, 4096), (4096, 4096), (4096, 2048)):
        w, ws = synth.fp8_weight(1002 + N + Kf, N, Kf)
        wbytes = N * Kf + ws.size
        W, nW = copies(u8(w), wbytes)
        WS = rep(u8(ws), nW)
        for T in (1, 8):
            xh = synth.normal_bf16(2002 + T, (T, Kf))
            xdt = bf(xh) if T > 1 else bf(xh[0])
            y = torch.empty((T, N) if T > 1 else (N,), dtype=torch.bfloat16, device=dev)
            us = time_launches(lambda i: fp8b.fp8_e4m3_gemv(W[i], WS[i], xdt, out=y), nW)
            out[f"fp8_e4m3_gemv {N}x{Kf} T={T}"] = entry(us, wbytes + T * (2 * Kf + 2 * N),
                                                          cpu_us(lambda: mx.fp8_gemv(xh, w, ws)))
        del W, WS
    # configs[2] with its literal scale format: one fp32 scale per 128x128
    # block (fp8_e4m3_gemv_f32s; the reference ABI above carries E8M0 bytes)
    for (N, Kf) in ((1536, 4096), (576, 4096), (4096, 4096), (4096, 2048)):
        w, wsf = synth.fp8_weight_f32s(1702 + N + Kf, N, Kf)
        wbytes = N * Kf + 4 * wsf.size
        W, nW = copies(u8(w), wbytes)
        WS = rep(torch.from_numpy(wsf).to(dev), nW)
        for T in (1, 8):
            xh = synth.normal_bf16(2002 + T, (T, Kf))
            xdt = bf(xh) if T > 1 else bf(xh[0])
            y = torch.empty((T, N) if T > 1 else (N,), dtype=torch.bfloat16, device=dev)
            us = time_launches(lambda i: fp8b.fp8_e4m3_gemv_f32s(W[i], WS[i], xdt, out=y), nW)
            out[f"fp8_e4m3_gemv_f32s {N}x{Kf} T={T}"] = entry(us, wbytes + T * (2 * Kf + 2 * N),
                                                               cpu_us(lambda: mx.fp8_gemv_f32s(xh, w, wsf)))
        del W, WS
    # Rows longer than the tile set (K up to the reference's 16384 cap) with
    # several tokens: each weight byte is read once for all tokens.
    for (N, Kf) in ((2048, 6144), (1024, 12288)):
        w, ws = synth.fp8_weight(1502 + N + Kf, N, Kf)
        wbytes = N * Kf + ws.size
        W, nW = copies(u8(w), wbytes)
        WS = rep(u8(ws), nW)
        T = 8
        xdt = bf(synth.normal_bf16(2102 + Kf, (T, Kf)))
        y = torch.empty((T, N), dtype=torch.bfloat16, device=dev)
        us = time_launches(lambda i: fp8b.fp8_e4m3_gemv(W[i], WS[i], xdt, out=y), nW)
        out[f"fp8_e4m3_gemv {N}x{Kf} T={T}"] = entry(us, wbytes + T * (2 * Kf + 2 * N), None)
        del W, WS

    # The engine's MLA shapes (kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu):
    # wq_a 1024x4096 and wkv 512x4096 on one activation (one multi launch
    # against two single launches), wq_b 32768x1024, wo_b 4096x8192. Weights
    # are device-filled E4M3 codes (positive, finite) with E8M0 tile scales.
    def fp8_dev(seed, N, Kf):
        w = torch.empty(N, Kf, dtype=torch.uint8, device=dev)
        fill.fill_uniform_u8(w, seed, 0, 0, 0x7E)
        s = torch.empty((N + 127) // 128, Kf // 128, dtype=torch.uint8, device=dev)
        fill.fill_uniform_u8(s, seed + 1, 0, 119, 125)
        return w, s

    xe = bf(synth.normal_bf16(2100, (8, 8192)))
    for name, N, Kf in (("wq_b", 32768, 1024), ("wo_b", 4096, 8192)):
        w, s = fp8_dev(2200 + N, N, Kf)
        wbytes = N * Kf + s.numel()
        n = n_copies(wbytes)
        W, WS = rep(w, n), rep(s, n)
        for T in (1, 8):
            xdt = xe[:T, :Kf].contiguous() if T > 1 else xe[0, :Kf].contiguous()
            y = torch.empty((T, N) if T > 1 else (N,), dtype=torch.bfloat16, device=dev)
            us = time_launches(lambda i: fp8b.fp8_e4m3_gemv(W[i], WS[i], xdt, out=y), n)
            out[f"fp8_e4m3_gemv {name} {N}x{Kf} T={T}"] = entry(us, wbytes + T * (2 * Kf + 2 * N), None)
        del W, WS
    wa, sa = fp8_dev(2300, 1024, 4096)
    wk, sk = fp8_dev(2301, 512, 4096)
    wbytes = wa.numel() + sa.numel() + wk.numel() + sk.numel()
    n = n_copies(wbytes)
    WA, SA, WK, SK = rep(wa, n), rep(sa, n), rep(wk, n), rep(sk, n)
    xa = xe[0, :4096].contiguous()
    ya = torch.empty(1024, dtype=torch.bfloat16, device=dev)
    yk = torch.empty(512, dtype=torch.bfloat16, device=dev)
    us = time_launches(lambda i: fp8b.fp8_e4m3_gemv_multi([(WA[i], SA[i]), (WK[i], SK[i])], xa, outs=[ya, yk]), n)
    out["fp8_e4m3_gemv_multi wq_a 1024x4096 + wkv 512x4096 T=1"] = entry(us, wbytes + 2 * 4096 + 2 * 1536, None)

    def two_single(i):
        fp8b.fp8_e4m3_gemv(WA[i], SA[i], xa, out=ya)
        fp8b.fp8_e4m3_gemv(WK[i], SK[i], xa, out=yk)

    us = time_launches(two_single, n)
    out["fp8_e4m3_gemv_m1 x 2 wq_a + wkv (reference call pattern)"] = entry(us, wbytes + 2 * 4096 + 2 * 1536, None)
    del WA, SA, WK, SK

    # Extensions on the FP8 path: the grouped output projection wo_a (8 groups
    # of 1024 x 4096 in one launch) and the shared expert's gate + up + SwiGLU.
    G, N, Kf = 8, 1024, 4096
    w, ws = synth.fp8_weight(1100, G * N, Kf)
    wbytes = G * N * Kf + ws.size
    W, nW = copies(u8(w), wbytes)
    WS = rep(u8(ws), nW)
    xh = synth.normal_bf16(1101, (G, Kf))
    xdt = bf(xh)
    y = torch.empty(G, N, dtype=torch.bfloat16, device=dev)
    us = time_launches(lambda i: fp8b.fp8_e4m3_gemv_grouped(W[i], WS[i], xdt, G, out=y), nW)
    out["fp8_e4m3_gemv_grouped wo_a 8x1024x4096 T=1"] = entry(
        us, wbytes + 2 * G * Kf + 2 * G * N, cpu_us(lambda: mx.fp8_gemv_grouped(xh, w, ws, G)))
    del W, WS
    N, Kf = 2048, 4096
    w1, s1 = synth.fp8_weight(1102, N, Kf)
    w3, s3 = synth.fp8_weight(1103, N, Kf)
    wbytes = N * Kf + s1.size
    W1, nW = copies(u8(w1), 2 * wbytes)
    S1 = rep(u8(s1), nW)
    W3, S3 = rep(u8(w3), nW), rep(u8(s3), nW)
    xh = synth.normal_bf16(1104, (Kf,))
    xdt = bf(xh)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev)
    us = time_launches(lambda i: fp8b.fp8_e4m3_swiglu_gemv(W1[i], S1[i], W3[i], S3[i], xdt, 10.0, True, out=y), nW)
    out["fp8_e4m3_swiglu_gemv shared expert 2x2048x4096 T=1"] = entry(
        us, 2 * wbytes + 2 * Kf + 2 * N, cpu_us(lambda: mx.fp8_swiglu(xh, w1, s1, w3, s3, 10.0, True)))
    del W1, S1, W3, S3
    # RMSNorm + residual folded into the wq_a GEMV (1536 x 4096).
    N, Kf = 1536, 4096
    w, ws = synth.fp8_weight(1105, N, Kf)
    wbytes = N * Kf + ws.size
    W, nW = copies(u8(w), wbytes)
    WS = rep(u8(ws), nW)
    hh, rh = synth.normal_bf16(1106, (Kf,)), synth.normal_bf16(1107, (Kf,), 0.0, 0.5)
    gh = synth.normal_bf16(1108, (Kf,), 1.0, 0.1)
    hd, rd, gd = bf(hh), bf(rh), bf(gh)
    xn = torch.empty(Kf, dtype=torch.bfloat16, device=dev)
    nr = torch.empty(Kf, dtype=torch.bfloat16, device=dev)
    y = torch.empty(N, dtype=torch.bfloat16, device=dev)
    us = time_launches(lambda i: fp8b.fp8_e4m3_rmsnorm_gemv(W[i], WS[i], hd, gd, rd), nW)
    nbytes = wbytes + 3 * 2 * Kf + 2 * Kf + 2 * 2 * Kf + 2 * N
    out["fp8_e4m3_rmsnorm_gemv residual+norm+wq_a 1536x4096 T=1"] = entry(us, nbytes, None)

    def two_launches(i):
        rb.rmsnorm_fuse_residual_add(hd, rd, gd, out_norm=xn, out_new_residual=nr)
        fp8b.fp8_e4m3_gemv(W[i], WS[i], xn, out=y)

    us = time_launches(two_launches, nW)
    out["rmsnorm_fuse_residual_add + fp8_e4m3_gemv_m1 (two launches)"] = entry(us, nbytes, None)
    del W, WS
    # Router gate GEMV of the routed dispatch: bf16 [256, 4096] x one token.
    wg = torch.empty(E, K, dtype=torch.bfloat16, device=dev)
    fill.fill_uniform_u8(wg.view(torch.uint8), 2400, 0, 0, 255)
    wg.view(torch.int16).bitwise_and_(0x3CFF)
    nbytes = E * K * 2
    n = n_copies(nbytes)
    WG = rep(wg, n)
    xr = xe[0, :K].contiguous()
    lo = torch.empty(1, E, dtype=torch.float32, device=dev)
    us = time_launches(lambda i: gb.router_logits(xr, WG[i], out=lo), n)
    out["router_logits bf16 256x4096 T=1"] = entry(us, nbytes + 2 * K + 4 * E, None)
    del WG
    # RMSNorm + residual, H = 4096
    Hn = 4096
    g = synth.normal_bf16(1203, (Hn,), 1.0, 0.1)
    gdn = bf(g)
    for T in (1, 8, 64):
        h = synth.normal_bf16(1201 + T, (T, Hn))
        r = synth.normal_bf16(1301 + T, (T, Hn), 0.0, 0.5)
        nb = 4 * T * Hn * 2
        # at most 2,048 activation copies per case (64 MB at T = 1): the
        # activations are small enough that the launch floor, not HBM, bounds
        # these launches
        ncop = min(n_copies(nb), 2048)
        Hc, Rc = rep(bf(h), ncop), rep(bf(r), ncop)
        yo = torch.empty(T, Hn, dtype=torch.bfloat16, device=dev)
        ro = torch.empty(T, Hn, dtype=torch.bfloat16, device=dev)
        us = time_launches(lambda i: rb.rmsnorm_fuse_residual_add(Hc[i], Rc[i], gdn, out_norm=yo,
                                                                  out_new_residual=ro), ncop)
        out[f"rmsnorm_fuse_residual_add T={T}x{Hn}"] = entry(us, nb + 2 * Hn,
                                                             cpu_us(lambda: mx.rmsnorm_residual(h, r, g)))
        del Hc, Rc
    add_traffic(out)
    if not counters:
        # the read floor for each line's bytes, timed the same way (graph replay)
        rf = read_floor_case(torch, dev, {k: (e["algorithmic_bytes"], e["us"]) for k, e in out.items()
                                          if e["algorithmic_bytes"] >= 16}, graph=True)
        for k, e in out.items():
            if k in rf:
                e["read_floor_us"] = rf[k]["floor_us"]
                e["kernel_over_floor"] = rf[k]["kernel_over_floor"]
    return out


def traffic_key(name: str):
    """The `TRAFFIC` key of profiles/*.md for a dense-kernel line of the
    bench (None for the reference-call-pattern comparison lines)."""
    m = re.match(r"fp8_e4m3_gemv (?:wq_b |wo_b )?(\d+)x(\d+) T=(\d+)$", name)
    if m:
        return f"fp8_gemv_{m.group(1)}x{m.group(2)}@T{m.group(3)}"
    m = re.match(r"fp8_e4m3_gemv_f32s (\d+)x(\d+) T=(\d+)$", name)
    if m:
        return f"fp8_gemv_f32s_{m.group(1)}x{m.group(2)}@T{m.group(3)}"
    m = re.match(r"rmsnorm_fuse_residual_add T=(\d+)x\d+$", name)
    if m:
        return f"rmsnorm_fuse_residual_add@T{m.group(1)}"
    fixed = {"mxfp4_gemv_m1 2048x4096": "mxfp4_gemv_m1@T1",
             "fp8_e4m3_gemv_multi wq_a 1024x4096 + wkv 512x4096 T=1": "fp8_gemv_multi_wqa_wkv@T1",
             "fp8_e4m3_gemv_grouped wo_a 8x1024x4096 T=1": "fp8_gemv_grouped_wo_a@T1",
             "fp8_e4m3_swiglu_gemv shared expert 2x2048x4096 T=1": "fp8_swiglu_gemv@T1",
             "fp8_e4m3_rmsnorm_gemv residual+norm+wq_a 1536x4096 T=1": "fp8_rmsnorm_gemv@T1",
             "router_logits bf16 256x4096 T=1": "router_logits@T1"}
    return fixed.get(name)


def add_traffic(kernels: dict) -> None:
    """Attach the rocprof-measured HBM bytes per launch (profiles/*.md) and
    the GB/s they make at the measured time to each dense-kernel line."""
    for name, e in kernels.items():
        key = traffic_key(name)
        if key is None or not e.get("us"):
            continue
        tb, src = profiled_traffic(key)
        if tb is not None:
            e["traffic_bytes"] = tb
            e["traffic_gbs"] = round(gbs(tb, e["us"]), 1)
            e["traffic_source"] = src


# ----------------------------------------------------------- CPU baseline ---

def read_floor_case(torch, dev, cases: dict, graph: bool = False) -> dict:
    """The HBM read floor for the byte counts of the timed launches: a
    read-only kernel (runtime.fill.read_floor: contiguous chunk per workgroup,
    16-byte loads, 8 in flight per thread) streams the same number of bytes,
    rotating over 1 GiB so that they come from HBM; the fastest of five
    launch shapes (256 to 2,048 workgroups of 256 or 512 threads), 200
    launches issued back to back by the library and
    timed by HIP events (graph=True: captured in a HIP graph and replayed, as
    the dense-kernel lines are timed). cases maps a name to (bytes, the
    kernel's measured µs)."""
    from runtime import fill
    pool = 1 << 30
    largest = max(int(nbytes) // 16 * 16 for nbytes, _ in cases.values())
    buf = torch.empty(max(pool, largest), dtype=torch.uint8, device=dev)
    fill.fill_uniform_u8(buf, 4242)
    sink = torch.empty(2048 * 512, dtype=torch.int32, device=dev)
    tm = Timer(torch)
    out = {"kernel": "dsv4_read_floor (libdsv4_fill.so)"}
    for name, (nbytes, kernel_us) in cases.items():
        nb = int(nbytes) // 16 * 16
        nrot = max(1, pool // nb)          # ranges past 1 GiB are read from one place (beyond the MALL anyway)
        best = float("inf")
        for wgs, thr in ((256, 256), (512, 256), (1024, 256), (1024, 512), (2048, 512)):
            fill.read_floor(buf, nb, wgs, sink, nrot, 10, thr)
            reps = 200
            if graph:
                us = tm.graph_us_per_call(lambda: fill.read_floor(buf, nb, wgs, sink, nrot, reps, thr), reps, reps=4)
            else:
                us = tm.ms(lambda: fill.read_floor(buf, nb, wgs, sink, nrot, reps, thr)) * 1e3 / reps
            best = min(best, us)
        out[name] = {"bytes": nb, "floor_us": round(best, 3), "floor_gbs": round(gbs(nb, best), 1),
                     "kernel_us": round(kernel_us, 3), "kernel_over_floor": round(kernel_us / best, 3)}
    del buf, sink
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_quota_cores():
    """CPUs granted by the cgroup v2 quota (cpu.max), or None without one."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, p = f.read().split()[:2]
        return None if q == "max" else round(int(q) / int(p), 2)
    except (OSError, ValueError):
        return None


def cpu_baseline(torch, layer, x, logits_h, T: int, step_bytes: float) -> dict:
    """The CPU oracle (the reference's CPU path: unpack + E8M0 -> bf16 dequant,
    fp32 matmul, bf16 casts) on one step of the headline workload, on every
    core of the host (os.cpu_count() BLAS threads), and the same layer on
    weights dequantised beforehand."""
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import mx

    cache = {}

    def expert(e):
        if e not in cache:
            cache[e] = tuple((m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy())
                             for m in (layer.W1, layer.W3, layer.W2))
        return cache[e]

    ids_t, w_t = mx.route_sigmoid_topk(logits_h, TOPK)
    xh = x.view(torch.int16).cpu().numpy().view(np.uint16)
    for e in np.unique(ids_t):
        expert(int(e))
    threads = os.cpu_count() or 1
    with threadpool_limits(limits=threads):
        blas = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
        log(f"cpu baseline: oracle moe layer, {threads} BLAS threads")
        t0 = time.perf_counter()
        n_calls = 0
        while True:
            mx.moe_layer(xh, expert, ids_t, w_t, O)
            n_calls += 1
            if time.perf_counter() - t0 > 10.0 or n_calls >= 3:
                break
        cpu_s = (time.perf_counter() - t0) / n_calls
        dq = {int(e): mx.dequant_expert_f32(expert(int(e))) for e in np.unique(ids_t)}
        t0 = time.perf_counter()
        n_mm = 0
        while True:
            mx.moe_layer_dequantised(xh, dq.__getitem__, ids_t, w_t, O)
            n_mm += 1
            if time.perf_counter() - t0 > 5.0 or n_mm >= 20:
                break
        mm_s = (time.perf_counter() - t0) / n_mm
    return {
        "value": round(step_bytes / cpu_s / 1e9, 4),
        "unit": "GB/s",
        "us_per_layer": round(cpu_s * 1e6, 1),
        "matmul_only_us_per_layer": round(mm_s * 1e6, 1),
        "cores": int(blas[0]) if blas else threads,
        "kind": "port",
        "nproc": os.cpu_count(),
        "cpu_quota_cores": cpu_quota_cores(),
        "cpu_model": cpu_model(),
        "sample": (f"{n_calls} oracle moe_layer call(s), T={T}, {len(np.unique(ids_t))} experts "
                   f"(dequant+fp32 matmul); matmul_only: {n_mm} call(s) on pre-dequantised weights"),
    }


# -------------------------------------------------------------- counters ----

def counters_run(torch, dev) -> int:
    """A short fixed sequence for rocprofv3 --pmc passes (no HIP graphs, a
    bounded number of dispatches): 24 one-token layers (gated stage A + stage
    B) on 4 resident layers, 8 T=4 and 8 T=16 layers, two 512-token prefill
    chunks, then 32 launches of each dense case and four 1 GiB copies (the
    counters' calibration). Kernel names and grid sizes identify the cases in
    the counter output."""
    from runtime import moe, synth

    layers = [moe.make_moe_weights(20000 + 100 * l, E, K, H, O, dev) for l in range(4)]
    for T, n in ((1, 24), (4, 8), (16, 8)):
        mods = [moe.RoutedMoELayer(w, topk=TOPK, max_tokens=16, check=False) for w in layers]
        x = torch.from_numpy(synth.normal_bf16(3001, (T, K)).view(np.int16)).view(torch.bfloat16).to(dev)
        lg = torch.from_numpy(synth.gating_logits(3002, n * T, E).reshape(n, T, E)).to(dev)
        for i in range(n):
            mods[i % 4].forward(x, logits=lg[i])
        torch.cuda.synchronize()
        log(f"counters: {n} layers at T={T}")
    # one 512-token prefill chunk on each of two layers (MFMA grouped GEMM)
    from runtime import mxfp4_grouped_gemv_binding as gb
    TP = 512
    xp = torch.from_numpy(synth.normal_bf16(4002, (TP, K)).view(np.int16)).view(torch.bfloat16).to(dev)
    ws = torch.empty(gb.prefill_workspace_bytes(TP, TOPK, E, H, O), dtype=torch.uint8, device=dev)
    for l in range(2):
        ids, w = synth.zipf_routing(4003, TP, E, TOPK, 1.1, layer=l)
        gb.mxfp4_moe_prefill(xp, layers[l].W1, layers[l].W3, layers[l].W2, torch.from_numpy(ids).to(dev),
                             torch.from_numpy(w).to(dev), workspace=ws)
    torch.cuda.synchronize()
    log("counters: 2 prefill chunks of 512 tokens")
    del layers, ws
    torch.cuda.empty_cache()
    dense_kernels(torch, dev, cpu=False, counters=True)
    torch.cuda.synchronize()
    log("counters: dense cases done")
    # calibration: torch's copy kernel over 1 GiB (reads 1 GiB, writes 1 GiB)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("counters: calibration copies done")
    return 0


# ------------------------------------------------------------------ main ----

def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=1, help="decode tokens per step of the headline (1, 4, 16)")
    ap.add_argument("--layers", type=int, default=4, help="resident layers cycled over (MALL defeat)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernels", action="store_true", help="skip the dense / FP8 / RMSNorm per-kernel lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations (config 3 at T=4/16, dispatch, config 4)")
    ap.add_argument("--c4-layers", type=int, default=43, help="layers of the config-4 sweep")
    ap.add_argument("--counters", action="store_true", help="short fixed sequence for rocprofv3 --pmc")
    ap.add_argument("--verbose", action="store_true", help="progress lines on stderr")
    args = ap.parse_args()
    global VERBOSE
    VERBOSE = args.verbose or args.counters
    if args.gpus != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(the routed MoE would shard by experts, or by the ff dimension with one all-reduce "
              "of the layer output per step)", file=sys.stderr)
        return 2

    import torch

    from runtime import moe

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.counters:
        return counters_run(torch, dev)
    t_start = time.perf_counter()
    T, L = args.tokens, args.layers

    log(f"allocating {L} layers x {E} experts ({L * E * EXPERT_BYTES / 1e9:.2f} GB)")
    layers = [moe.make_moe_weights(20000 + 100 * l, E, K, H, O, dev) for l in range(L)]
    torch.cuda.synchronize()
    log(f"headline: config 3, T={T}, {args.steps} steps")
    head = moe_layer_case(torch, dev, layers, T, args.steps, args.warmup, 3001)
    a_bytes, b_bytes = head.pop("_stage_bytes")
    value = head["gbs"]

    configs = None
    if not args.no_configs:
        configs = {}
        for Tc in (1, 4, 16):
            if Tc == T:
                continue
            log(f"config 3 at T={Tc}")
            c = moe_layer_case(torch, dev, layers, Tc, 20, 3, 3101 + Tc)
            c.pop("_stage_bytes")
            # rocprof HBM bytes per launch of the stage kernels (profiles/*.md)
            kn = ("moe_swiglu_t1_kernel_gated", "moe_down_t1_kernel") if Tc == 1 else \
                ("moe_swiglu_tn_kernel", "moe_down_tn_kernel")
            st = {}
            for stage, kname, us_key in (("A", kn[0], "swiglu_A_tables_given" if Tc > 1 else "gate_swiglu_A"),
                                         ("B", kn[1], "down_B")):
                tb, src = profiled_traffic(f"{kname}@T{Tc}")
                if tb is not None:
                    st[stage] = {"kernel": kname, "traffic_bytes": tb, "source": src,
                                 "traffic_gbs": round(gbs(tb, c["stage_us"][us_key]), 1)}
            if st:
                c["stage_traffic"] = st
            configs[f"cfg3_T{Tc}"] = c
        log("routed dispatch (reference routing) at T=1")
        configs["routed_dispatch_T1"] = routed_dispatch_case(torch, dev, layers, 20, 3)

    cpu = None
    if not args.no_cpu_baseline:
        from runtime import synth
        xh = torch.from_numpy(synth.normal_bf16(3001, (T, K)).view(np.int16)).view(torch.bfloat16).to(dev)
        lg0 = synth.gating_logits(3002, T, E)
        cpu = cpu_baseline(torch, layers[0], xh, lg0, T, float(head["algorithmic_bytes_per_step"]))

    del layers
    torch.cuda.empty_cache()
    if configs is not None:
        log(f"config 4: {args.c4_layers}-layer decode sweep and 512-token prefill")
        c4 = config4_case(torch, dev, 8, 2, args.c4_layers)
        configs["cfg4_decode"] = c4["decode"]
        configs["cfg4_prefill"] = c4["prefill"]
        del c4
        torch.cuda.empty_cache()
        pf = configs["cfg4_prefill"]
        pf["read_floor"] = read_floor_case(torch, dev, {
            "layer_bytes": (pf["algorithmic_bytes_per_layer"], pf["us_per_layer"])})

    kernels = None
    if not args.no_kernels:
        log("per-kernel lines: dense MXFP4, FP8, RMSNorm, router")
        kernels = dense_kernels(torch, dev, cpu=not args.no_cpu_baseline)

    a_kernel = "moe_swiglu_t1_kernel_gated" if T == 1 else "moe_swiglu_tn_kernel"
    b_kernel = "moe_down_t1_kernel" if T == 1 else "moe_down_tn_kernel"
    a_us = head["stage_us"]["gate_swiglu_A"] if T == 1 else head["stage_us"]["swiglu_A_tables_given"]
    b_us = head["stage_us"]["down_B"]
    a_traffic, a_src = profiled_traffic(f"{a_kernel}@T{T}")
    b_traffic, b_src = profiled_traffic(f"{b_kernel}@T{T}")

    def roof(kernel, desc, us, nbytes, traffic, src):
        # achieved / frac: this run's HIP-event average per launch; rocprof_*:
        # the kernel-trace average of the same timing launches in
        # profiles/ (null when the kernel's sources changed since)
        rp_us, rp_src = profiled_duration(f"{kernel}@T{T}")
        return {"kernel": f"{kernel} ({desc})", "bound": "hbm", "achieved": round(gbs(nbytes, us), 2),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs(nbytes, us) / HBM_PEAK_GBS, 4),
                "traffic": traffic, "traffic_source": src, "algorithmic_bytes_per_launch": int(round(nbytes)),
                "avg_launch_us": round(us, 3),
                "rocprof_avg_us": rp_us,
                "rocprof_frac": round(gbs(nbytes, rp_us) / HBM_PEAK_GBS, 4) if rp_us else None,
                "rocprof_source": rp_src}

    result = {
        "metric": METRIC,
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["moe_layer_us"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4-e2m1/e8m0 weights, bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded SplitMix64 weights filled on device, N(0,1) activations/logits)",
        "config": {
            "workload": f"configs[3]: routed MoE layer decode, T={T}, top-{TOPK} of {E} MXFP4 experts "
                        f"(W1/W3 {H}x{K}, W2 {O}x{H}), device sigmoid gating, {L} resident layers",
            "tokens": T, "experts": E, "topk": TOPK, "layers_cycled": L,
            "mean_unique_experts": head["mean_unique_experts"],
            "algorithmic_bytes_per_step": head["algorithmic_bytes_per_step"],
        },
        "timing": head["timing"] + " (the faster of the two over the same K steps; HIP events on the launch stream)",
        "moe_layer_us": head["moe_layer_us"],
        "moe_layer_us_graph": head["moe_layer_us_graph"],
        "moe_layer_us_host_issued": head["moe_layer_us_host_issued"],
        "hbm_frac_of_peak": head["hbm_frac_of_peak"],
        "stage_us": head["stage_us"],
        "stage_gbs": head["stage_gbs"],
        "roofline": roof(a_kernel, "stage A of the timed step: gating + W1/W3 MXFP4 GEMV + SiLU" if T == 1
                         else "stage A: W1/W3 MXFP4 GEMV + SiLU", a_us, a_bytes, a_traffic, a_src),
        "stage_b_roofline": roof(b_kernel, "stage B: W2 MXFP4 GEMV + weighted combine", b_us, b_bytes,
                                 b_traffic, b_src),
        "cpu_baseline": cpu,
        "kernels": kernels,
        "configs": configs,
    }
    # the measured device-copy ceiling (torch's copy over 1 GiB, read + write)
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    dst.copy_(src)
    copy_ms = Timer(torch).ms(lambda: [dst.copy_(src) for _ in range(5)]) / 5
    result["copy_ceiling_gbs"] = round(2 * src.numel() / (copy_ms * 1e-3) / 1e9, 1)
    del src, dst
    # the HBM read floor for the same byte counts (one pass of a read-only kernel)
    result["read_floor"] = read_floor_case(torch, dev, {
        "stage_A": (a_bytes, a_us), "stage_B": (b_bytes, b_us),
        "layer_one_pass": (a_bytes + b_bytes, result["moe_layer_us"])})
    result["bench_seconds"] = round(time.perf_counter() - t_start, 1)
    # last key: every configuration in a few characters, so that it falls in
    # the tail of the output that a driver keeps
    result["summary"] = summary(result)
    print(json.dumps(result, separators=(",", ":")), flush=True)
    return 0


def summary(r: dict) -> dict:
    """[µs, fraction of 8 TB/s (algorithmic bytes / time), kernel time over
    the read floor for the same bytes] per configuration and kernel; prefill
    adds the fraction of the bf16 MFMA peak; stage A/B add the rocprof average
    from profiles/ (µs) and the fraction it gives."""
    def r3(v):
        return None if v is None else round(v, 3)

    rf = r.get("read_floor", {})
    s = {"cols": "us,frac_hbm,over_floor"}
    s["cfg3_T%d" % r["config"]["tokens"]] = [r3(r["moe_layer_us"]), r3(r["hbm_frac_of_peak"]),
                                              r3(rf.get("layer_one_pass", {}).get("kernel_over_floor"))]
    for tag, key in (("A", "roofline"), ("B", "stage_b_roofline")):
        ro = r[key]
        floor = rf.get("stage_" + tag, {}).get("kernel_over_floor")
        s["stage" + tag] = [r3(ro["avg_launch_us"]), r3(ro["frac"]), r3(floor), ro["rocprof_avg_us"],
                            r3(ro["rocprof_frac"])]
    c = r.get("configs") or {}
    for k in ("cfg3_T1", "cfg3_T4", "cfg3_T16"):
        if k in c:
            s[k] = [r3(c[k]["moe_layer_us"]), r3(c[k]["hbm_frac_of_peak"])]
    if "routed_dispatch_T1" in c:
        s["dispatch_T1"] = [r3(c["routed_dispatch_T1"]["us"]), r3(c["routed_dispatch_T1"]["hbm_frac_of_peak"])]
    if "cfg4_decode" in c:
        d = c["cfg4_decode"]
        s["cfg4_decode_layer"] = [r3(d["us_per_layer"]), r3(d["hbm_frac_of_peak"])]
    if "cfg4_prefill" in c:
        p = c["cfg4_prefill"]
        s["cfg4_prefill_layer"] = [round(p["us_per_layer"], 1), r3(p["hbm_frac_of_peak"]),
                                   r3(p.get("read_floor", {}).get("layer_bytes", {}).get("kernel_over_floor")),
                                   r3(p["mfma_frac_of_bf16_peak"])]
    short = {"mxfp4_gemv_m1 2048x4096": "cfg0_mxfp4",
             "fp8_e4m3_gemv_multi wq_a 1024x4096 + wkv 512x4096 T=1": "fp8_multi_wqa_wkv",
             "fp8_e4m3_gemv_grouped wo_a 8x1024x4096 T=1": "fp8_grouped_wo_a",
             "fp8_e4m3_swiglu_gemv shared expert 2x2048x4096 T=1": "fp8_swiglu_shared",
             "fp8_e4m3_rmsnorm_gemv residual+norm+wq_a 1536x4096 T=1": "fp8_rmsnorm_wqa",
             "router_logits bf16 256x4096 T=1": "router_gemv"}
    for name, e in (r.get("kernels") or {}).items():
        m = re.match(r"fp8_e4m3_gemv (?:(wq_b|wo_b) )?(\d+)x(\d+) T=(\d+)$", name)
        mf = re.match(r"fp8_e4m3_gemv_f32s (\d+)x(\d+) T=(\d+)$", name)
        if m:
            key = f"fp8_{m.group(2)}x{m.group(3)}_T{m.group(4)}"
        elif mf:
            key = f"fp8f32s_{mf.group(1)}x{mf.group(2)}_T{mf.group(3)}"
        else:
            m = re.match(r"rmsnorm_fuse_residual_add T=(\d+)x\d+$", name)
            key = f"cfg1_rmsnorm_T{m.group(1)}" if m else short.get(name)
        if key:
            s[key] = [r3(e["us"]), r3(e["frac_of_peak"]), r3(e.get("kernel_over_floor"))]
    if r.get("cpu_baseline"):
        cb = r["cpu_baseline"]
        s["cpu_baseline"] = [cb["us_per_layer"], cb["cores"]]
    return s


if __name__ == "__main__":
    sys.exit(main())
