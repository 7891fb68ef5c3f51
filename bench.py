#!/usr/bin/env python3
"""Benchmark of the MI355X linear-layer GEMM path (one JSON line on stdout).

Headline workload (the metric's "f16, M=1024"): all
per-layer Qwen3-0.6B decoder projections for 28 layers at M = 1024 tokens, in
the reference's fused layout and order (src/decoder.rs:1321-1657):
    qkv    [1024,1024] x [4096,1024]^T
    o      [1024,2048] x [1024,2048]^T  + residual
    gate|up[1024,1024] x [6144,1024]^T  + SiLU.up  -> act [1024,3072]
    down   [1024,3072] x [1024,3072]^T  + residual
f16, random-init weights ~ N(0, 0.02), activations RMSNorm'd N(0,1) (the
norms and attention between the projections are not part of this path; their
outputs are fixed synthetic inputs).  A step is one pass over the 112 GEMMs,
launched as one captured hipGraph on the context's stream; inputs and weights
are resident in HBM before timing starts.

`value` is TFLOP/s over the whole step (2*M*N*K per GEMM, host clock around
exactly --steps steps with the stream synchronized on both sides).
`roofline` prices the dominant kernel (the gate|up GEMM, 40% of the FLOPs)
against the published MI355X dense FP16 peak, from its average kernel
duration over eager passes of the same layer sequence, each launch stamping
start and end HIP events from its own dispatch (qa_time_next_launch, on the
launching stream).  `cpu_baseline`
times the oracle (the C restatement of the reference CPU path) on a bounded
sample of the same workload on this host's cores.  `detail` carries the
other BASELINE configs (1, 2, 4) as kernel-level figures.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2516.6  # MI355X dense FP16/BF16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0
METRIC = "GEMM TFLOP/s + % MFMA peak (f16, M=1024); aligner forward ms per 300 s audio"

DEC = dict(layers=28, hidden=1024, q_dim=2048, kv_dim=1024, inter=3072, nqh=16, nkvh=8, hd=128)
PREFILL_ROWS = (1024, 4352)  # config 3's M; config 5's ~300 s prefill (~4.3 k tokens)
ENC = dict(layers=18, d_model=896, ffn=3584, conv_k=128 * 9)
COPY_CAL_BYTES = 512 << 20
COUNTER_PROFILE = os.path.join(ROOT, "profiles", "gemm_sites_counters.json")


def measured_counters(site: str):
    """From the committed rocprofv3 --pmc passes over `bench.py --site <site>`
    (cold weights): L2 <-> fabric bytes per launch (FETCH_SIZE / WRITE_SIZE
    scaled by the copy calibration), the kernel, and the MFMA-busy share
    SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x duration x 2.4 GHz); Nones when
    the profile is missing."""
    try:
        entry = json.load(open(COUNTER_PROFILE))["sites"][f"{site}/cold"]
        return (int(entry["hbm_bytes"]), entry["kernel"], entry["mfma_busy_pct_duration_2p4GHz"],
                entry["mfma_busy_pct_gui"])
    except (OSError, KeyError, ValueError):
        return None, None, None, None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


SETTLE_MS = 100.0  # untimed replays ahead of the W warm-up steps (see settled)


def settled(timer, warmup, steps):
    """timer(warmup, steps) -> (event ms, wall ms) per step over `steps` timed
    graph replays after `warmup` untimed ones.  The GPU reaches its steady
    clocks after ~70 ms of continuous work: with 5 warm-up steps of config 3
    (7 ms) the timed steps ran ~2.5% slower than after 50.  So a 2-step probe
    gives the step time, and the timed call replays the graph for at least
    SETTLE_MS more, untimed, ahead of its `warmup` steps.  Returns (event ms,
    wall ms, settle steps)."""
    ev, wall = timer(1, 2)
    settle = int(np.ceil(SETTLE_MS / max(ev, wall, 1e-3)))
    ev, wall = timer(warmup + settle, steps)
    return ev, wall, settle


def rmsnormed(host, seed, tid, shape, dtype):
    """N(0,1) rows scaled to unit RMS (RMSNorm with weight 1), as 16-bit bits."""
    x = host.synth_normal_f32(seed, tid, shape).astype(np.float64)
    x /= np.sqrt((x * x).mean(axis=-1, keepdims=True) + 1e-6)
    return host.narrow(x.astype(np.float32), dtype)


def decoder_weights(host, li, dtype=0, seed=0):
    h, q, kv, it = DEC["hidden"], DEC["q_dim"], DEC["kv_dim"], DEC["inter"]
    shapes = dict(q=(q, h), k=(kv, h), v=(kv, h), o=(h, q), gate=(it, h), up=(it, h), down=(h, it))
    return {name: host.synth_normal(seed, 1000 + li * 16 + i, shp, 0.0, 0.02, dtype)
            for i, (name, shp) in enumerate(shapes.items())}


def dec_flops(m):
    h, q, kv, it = DEC["hidden"], DEC["q_dim"], DEC["kv_dim"], DEC["inter"]
    per = {"qkv": 2 * m * (q + 2 * kv) * h, "o": 2 * m * h * q, "gu": 2 * m * 2 * it * h,
           "down": 2 * m * h * it}
    return per, sum(per.values()) * DEC["layers"]


def cpu_baseline(orc, host, m, budget_s):
    """Oracle (f32 GEMM + the reference's rounding points) over whole decoder
    layers of the same workload until `budget_s` of CPU time is spent."""
    per, _ = dec_flops(m)
    layer_flops = sum(per.values())
    normed = rmsnormed(host, 0, 1, (m, DEC["hidden"]), 0)
    attn = rmsnormed(host, 0, 2, (m, DEC["q_dim"]), 0)
    norm2 = rmsnormed(host, 0, 3, (m, DEC["hidden"]), 0)
    h = host.synth_normal(0, 4, (m, DEC["hidden"]))
    done, t_used, li = 0, 0.0, 0
    while li < DEC["layers"] and (li == 0 or t_used < budget_s):
        w = decoder_weights(host, li)
        qkv_w = np.concatenate([w["q"], w["k"], w["v"]])
        gu_w = np.concatenate([w["gate"], w["up"]])
        t0 = time.perf_counter()
        orc.linear(0, normed, qkv_w, np.zeros((m, qkv_w.shape[0]), np.uint16))
        orc.linear(0, attn, w["o"], h, flags=orc.ACCUMULATE)
        act = orc.linear(0, norm2, gu_w, np.zeros((m, DEC["inter"]), np.uint16),
                         flags=orc.EPI_SILU_MUL)
        orc.linear(0, act, w["down"], h, flags=orc.ACCUMULATE)
        t_used += time.perf_counter() - t0
        done += 1
        li += 1
    threads = orc.num_threads()
    # the same layer's qkv projection on one thread
    orc.set_threads(1)
    try:
        w = decoder_weights(host, 0)
        qkv_w = np.concatenate([w["q"], w["k"], w["v"]])
        t0 = time.perf_counter()
        orc.linear(0, normed, qkv_w, np.zeros((m, qkv_w.shape[0]), np.uint16))
        t1 = time.perf_counter() - t0
    finally:
        orc.set_threads(threads)
    per_config = cpu_other_configs(orc, host)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(done * layer_flops / t_used / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} of 28 decoder layers (4 projections each, M={m}, f16 in/out, f32 "
                  f"accumulate) through oracle/qa_oracle.c on {threads} OpenMP threads; "
                  f"{t_used:.1f} s",
        "value_1thread": round(per["qkv"] / t1 / 1e12, 4),
        "sample_1thread": f"layer 0's qkv projection ({per['qkv'] / 1e9:.2f} GFLOP) on 1 thread; "
                          f"{t1:.2f} s",
        "cpu_model": cpu_model,
        "nproc": os.cpu_count(),
        "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
        "per_config": per_config,
    }


def cpu_other_configs(orc, host):
    """The oracle on BASELINE configs 1, 2 and 4 and a bounded sample of
    config 5, on the same threads: config 1 and 2 whole; config 4 as one
    encoder layer at M = 3750 (bf16; qkv, o, fc1 + GELU, fc2) plus the conv
    GEMM, extrapolated to 18 layers; config 5 as one decoder layer at
    s = 4334 (norms, projections, RoPE, causal attention), one tower layer
    at 3900 tokens with the post-projection, and the conv stem over 10 of the
    300 chunks, extrapolated to 28 decoder layers, 18 tower layers and 300
    chunks (the log-mel and the head are left out: under 1% of the forward).
    The decoder layer's causal attention is timed on its last 512 query rows
    (exact for those rows) and scaled by the causal area those rows cover."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from chains import EPS, HD, INTER, NKVH, NQH, oracle_tower, perm_conv
    from qwen3_aligner_wgpu_amd import synthetic as syn
    out, z = {}, lambda r, c: np.zeros((r, c), np.uint16)  # noqa: E731
    # config 1
    a, w = host.synth_normal(0, 11, (256, 1024)), host.synth_normal(0, 12, (3072, 1024), 0, 0.02)
    t0 = time.perf_counter()
    for _ in range(5):
        orc.linear(0, a, w, z(256, 3072))
    t = (time.perf_counter() - t0) / 5
    out["config1"] = {"ms": round(t * 1e3, 2), "tflops": round(2 * 256 * 3072 * 1024 / t / 1e12, 4)}
    # config 2
    x = host.synth_normal(0, 21, (512, 1024))
    wgu, wd = host.synth_normal(0, 22, (6144, 1024), 0, 0.02), host.synth_normal(0, 23, (1024, 3072), 0, 0.02)
    t0 = time.perf_counter()
    act = orc.linear(0, x, wgu, z(512, 3072), flags=orc.EPI_SILU_MUL)
    orc.linear(0, act, wd, x.copy(), flags=orc.ACCUMULATE)
    t = time.perf_counter() - t0
    out["config2"] = {"ms": round(t * 1e3, 2), "tflops": round(9.664e9 / t / 1e12, 4)}
    # config 4: one layer + the conv GEMM, extrapolated
    m, d, f, ck = 3750, ENC["d_model"], ENC["ffn"], ENC["conv_k"]
    g = lambda tid, shp, std: host.synth_normal(1, tid, shp, 0.0, std, 1)  # noqa: E731
    xin, h = g(2, (m, d), 1.0), g(5, (m, d), 1.0)
    t0 = time.perf_counter()
    orc.linear(1, g(1, (m, ck), 1.0), g(4000, (d, ck), 0.02), z(m, d), flags=orc.EPI_GELU,
               bias=g(4001, (d,), 0.01))
    tc = time.perf_counter() - t0
    t0 = time.perf_counter()
    orc.linear(1, xin, g(5000, (3 * d, d), 0.02), z(m, 3 * d), bias=g(5001, (3 * d,), 0.01))
    h = orc.linear(1, xin, g(5002, (d, d), 0.02), h, flags=orc.ACCUMULATE, bias=g(5003, (d,), 0.01))
    act = orc.linear(1, xin, g(5004, (f, d), 0.02), z(m, f), flags=orc.EPI_GELU, bias=g(5005, (f,), 0.01))
    orc.linear(1, act, g(5006, (d, f), 0.02), h, flags=orc.ACCUMULATE, bias=g(5007, (d,), 0.01))
    tl = time.perf_counter() - t0
    t4 = tc + ENC["layers"] * tl
    out["config4"] = {"ms_extrapolated": round(t4 * 1e3, 1),
                      "tflops": round(1308.3e9 / t4 / 1e12, 4),
                      "sample": f"conv GEMM {tc:.2f} s + one layer {tl:.2f} s, x 18 layers"}
    # config 5 sample
    w5 = syn.aligner_weights(0, 1, 1, 5)
    s = 4334
    hd_in = host.synth_normal(5, 9, (s, 1024))
    cap = (s + 63) // 64 * 64
    import __graft_entry__ as entry
    cos, sin = entry.load_package().rope_tables(cap, 128, 1e6, 0)
    lw = w5["dec"][0]
    t0 = time.perf_counter()
    normed = orc.rms_norm(0, hd_in, lw["iln"], EPS)
    qkv_w = np.ascontiguousarray(np.concatenate([lw["q"], lw["k"], lw["v"]]))
    qkv = orc.linear(0, normed, qkv_w, z(s, qkv_w.shape[0]))
    kc, vc = np.zeros((NKVH, cap, HD), np.uint16), np.zeros((NKVH, HD, cap), np.uint16)
    q = orc.qk_norm_rope(0, qkv, NQH, NKVH, HD, lw["qn"], lw["kn"], cos, sin, 0, EPS, kc, vc, 0)
    t_lin = time.perf_counter() - t0
    tail = 512
    t0 = time.perf_counter()
    attn = orc.attention(0, np.ascontiguousarray(q[:, s - tail:]), kc, vc, s - tail)
    t_att = (time.perf_counter() - t0) * (s * (s + 1) / 2) / (tail * (2 * s - tail + 1) / 2)
    attn = np.ascontiguousarray(np.concatenate([np.zeros((s - tail, attn.shape[1]), np.uint16), attn]))
    t0 = time.perf_counter()
    h2 = orc.linear(0, attn, lw["o"], hd_in.copy(), flags=orc.ACCUMULATE)
    norm2 = orc.rms_norm(0, h2, lw["pln"], EPS)
    gu_w = np.ascontiguousarray(np.concatenate([lw["gate"], lw["up"]]))
    act = orc.linear(0, norm2, gu_w, z(s, INTER), flags=orc.EPI_SILU_MUL)
    orc.linear(0, act, lw["down"], h2, flags=orc.ACCUMULATE)
    t_lin += time.perf_counter() - t0
    t_dec = t_lin + t_att
    n_tok = 3900
    t0 = time.perf_counter()
    oracle_tower(orc, 0, w5["enc"], None, n_tok, start="h", h0=host.synth_normal(5, 10, (n_tok, 896)))
    t_tow = time.perf_counter() - t0
    b = 10
    mel = host.synth_normal(5, 11, (b, 128, 100, 1), 0, 1.0)
    (c1w, c1b), (c2w, c2b), (c3w, c3b) = w5["enc"]["conv"]
    t0 = time.perf_counter()
    y1 = orc.conv3x3s2(0, mel, perm_conv(c1w), c1b)
    y2 = orc.conv3x3s2(0, y1.reshape(b, 64, 50, 480), perm_conv(c2w), c2b)
    orc.conv3x3s2(0, y2.reshape(b, 32, 25, 480), perm_conv(c3w), c3b, token_major=True)
    t_stem = time.perf_counter() - t0
    t5 = 28 * t_dec + 18 * t_tow + 30 * t_stem
    out["config5"] = {"s_extrapolated": round(t5, 1),
                      "sample": f"one decoder layer at s={s} {t_dec:.1f} s (attention {t_att:.1f} s "
                                f"scaled from its last {tail} rows), one tower layer + "
                                f"post at {n_tok} tokens {t_tow:.1f} s, stem over {b} chunks "
                                f"{t_stem:.1f} s; x 28, x 18, x 30"}
    return out


def bench_decoder(pkg, host, ctx, m, warmup, steps, tdec=None):
    """Config 3 (the headline).  When `tdec` (a host.TextDecoder) is given, the
    same weights are loaded into it too, with unit norm weights."""
    dec = host.DecoderLinears(ctx, pkg.F16, DEC["layers"], m, DEC["hidden"], DEC["q_dim"],
                              DEC["kv_dim"], DEC["inter"])
    t0 = time.perf_counter()
    ones_h = np.ones(DEC["hidden"], np.float32)
    ones_d = np.ones(DEC["hd"], np.float32)
    for li in range(DEC["layers"]):
        w = decoder_weights(host, li)
        dec.load_layer(li, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"])
        if tdec is not None:
            tdec.load_layer(li, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"],
                            ones_h, ones_h, ones_d, ones_d)
    dec.set_inputs(m, rmsnormed(host, 0, 1, (m, DEC["hidden"]), 0),
                   rmsnormed(host, 0, 2, (m, DEC["q_dim"]), 0),
                   rmsnormed(host, 0, 3, (m, DEC["hidden"]), 0),
                   host.synth_normal(0, 4, (m, DEC["hidden"])))
    log(f"[bench] decoder weights generated and resident in {time.perf_counter() - t0:.1f} s")
    ev_ms, wall_ms, settle = settled(lambda w, s: dec.time(m, w, s, use_graph=True), warmup, steps)
    sites = dec.profile_sites(m, max(2, steps // 4))
    return dec, ev_ms, wall_ms, sites, settle


# ---- per-launch timing protocol: >= 200 back-to-back launches after 20
# warm-ups, median and p10 / p90 of the per-launch durations; "warm" repeats
# one weight matrix (L2 / MALL resident), "cold" cycles through copies that
# together exceed the 256 MB MALL, so every launch fetches its W from HBM ----

def dist(ms):
    """Per-launch ms -> {median, p10, p90} in microseconds."""
    us = np.asarray(ms, np.float64) * 1e3
    return {"median": round(float(np.median(us)), 2), "p10": round(float(np.percentile(us, 10)), 2),
            "p90": round(float(np.percentile(us, 90)), 2), "launches": int(us.size)}


# site -> (n rows of W, k, flags name, output columns); fused as the reference
# runs them (src/decoder.rs:1321-1657) and unfused as its CPU path does
# (q, k, v and gate, up separately, src/cpu_decoder.rs:416-512)
def dec_sites(unfused):
    h, q, kv, it = DEC["hidden"], DEC["q_dim"], DEC["kv_dim"], DEC["inter"]
    if unfused:
        return {"q": (q, h, 0), "k": (kv, h, 0), "v": (kv, h, 0), "o": (h, q, 1),
                "gate": (it, h, 0), "up": (it, h, 0), "down": (h, it, 1)}
    return {"qkv": (q + 2 * kv, h, 0), "o": (h, q, 1), "gu": (2 * it, h, 2), "down": (h, it, 1)}


class SiteSet:
    """Device copies of every decoder layer's weights for the per-site
    protocol (fused or unfused layout) plus the fixed activations, and one
    qa_linear descriptor per (site, layer)."""

    def __init__(self, pkg, host, ctx, m, layers, unfused):
        self.pkg, self.ctx, self.m, self.unfused = pkg, ctx, m, unfused
        self.sites = dec_sites(unfused)
        self.bufs = []
        h, q, it = DEC["hidden"], DEC["q_dim"], DEC["inter"]
        put = lambda a: self._keep(ctx.to_device(a))  # noqa: E731
        self.x = {"h": put(rmsnormed(host, 0, 1, (m, h), 0)), "q": put(rmsnormed(host, 0, 2, (m, q), 0)),
                  "it": put(host.synth_normal(0, 5, (m, it), 0, 0.5))}
        self.out = {"wide": self._keep(ctx.alloc(m * 2 * it * 2)),
                    "res": put(host.synth_normal(0, 4, (m, h)))}
        self.descs = {s: [] for s in self.sites}
        for li in range(layers):
            w = decoder_weights(host, li)
            mats = dict(q=w["q"], k=w["k"], v=w["v"], o=w["o"], gate=w["gate"], up=w["up"],
                        down=w["down"]) if unfused else dict(
                qkv=np.concatenate([w["q"], w["k"], w["v"]]), o=w["o"],
                gu=np.concatenate([w["gate"], w["up"]]), down=w["down"])
            for s, (n, k, fl) in self.sites.items():
                dw = put(np.ascontiguousarray(mats[s]))
                a = self.x["q"] if k == q else self.x["it"] if k == it else self.x["h"]
                if fl == 1:
                    d = pkg.linear_desc(pkg.F16, m, n, k, a, dw, self.out["res"], flags=pkg.ACCUMULATE)
                elif fl == 2:
                    d = pkg.linear_desc(pkg.F16, m, n, k, a, dw, self.out["wide"], flags=pkg.EPI_SILU_MUL)
                else:
                    d = pkg.linear_desc(pkg.F16, m, n, k, a, dw, self.out["wide"])
                self.descs[s].append(d)

    def _keep(self, b):
        self.bufs.append(b)
        return b

    def flops(self, site):
        n, k, fl = self.sites[site]
        return 2 * self.m * n * k

    def close(self):
        for b in self.bufs:
            b.free()
        self.bufs = []


def site_protocol(host, ctx, ss, warm_iters=200, cold_iters=280):
    """Per site: cold (cycling through every layer's W, 880 MB fused) and warm
    (layer 0's W repeated) per-launch distributions; and one back-to-back pass
    over the layers' sites in the reference's order, ms per 28-layer step."""
    out = {}
    for s, descs in ss.descs.items():
        cold = dist(host.time_linears_each(ss.ctx, descs, 20, cold_iters))
        warm = dist(host.time_linears_each(ss.ctx, descs[:1], 20, warm_iters))
        cold_k = dist(host.time_linears_stamped(ss.ctx, descs, 20, cold_iters))
        warm_k = dist(host.time_linears_stamped(ss.ctx, descs[:1], 20, warm_iters))
        out[s] = {"cold": cold, "warm": warm, "cold_kernel": cold_k, "warm_kernel": warm_k,
                  "tflops_cold_median": round(ss.flops(s) / (cold["median"] * 1e-6) / 1e12, 1),
                  "tflops_cold_kernel_median":
                      round(ss.flops(s) / (cold_k["median"] * 1e-6) / 1e12, 1)}
    seq = [ss.descs[s][li] for li in range(DEC["layers"]) for s in ss.sites]
    ms = host.time_linears_each(ss.ctx, seq, 20, 2 * len(seq))
    step_ms = float(ms.sum()) / 2
    flops = sum(ss.flops(s) for s in ss.sites) * DEC["layers"]
    return out, {"step_ms_back_to_back": round(step_ms, 4),
                 "tflops": round(flops / (step_ms * 1e-3) / 1e12, 1),
                 "note": "eager launches, no graph: each site's GEMM in layer order over 28 "
                         "layers, ms summed over per-launch events"}


COLD_BYTES = 320 << 20  # weight copies a cold --site run cycles through: > the 256 MB MALL


def site_descs(pkg, host, ctx, site, warm):
    """One GEMM site for counter runs (rocprofv3 --pmc over bench.py --site):
    config-3 sites (qkv, o, gu, down; q, k, v, gate, up unfused) at M = 1024,
    config1 (x [256,1024] . W[3072,1024]^T) or config2_gu / config2_down (the
    MLP block at M = 512).  warm: one weight matrix repeated (L2 / MALL
    resident); cold: distinct copies of it totalling COLD_BYTES, cycled, so
    every launch fetches its W from HBM.  Returns (descriptors, FLOPs per
    launch)."""
    h, q, kv, it = DEC["hidden"], DEC["q_dim"], DEC["kv_dim"], DEC["inter"]
    sites = dict(dec_sites(False), **dec_sites(True))
    if site == "config1":
        m, n, k, fl, xk = 256, 3072, 1024, 0, None
    elif site == "config2_gu":
        m, n, k, fl, xk = 512, 2 * it, h, 2, None
    elif site == "config2_down":
        m, n, k, fl, xk = 512, h, it, 1, None
    elif site == "config2_mlp":
        return config2_pair_descs(pkg, host, ctx, warm)
    elif site in sites:
        (n, k, fl), m = sites[site], 1024
        xk = k
    else:
        raise SystemExit(f"bench.py: unknown --site {site}")
    a = ctx.to_device(rmsnormed(host, 0, 31, (m, k), 0) if xk is not None
                      else host.synth_normal(0, 32, (m, k), 0, 0.5))
    nout = n // 2 if fl == 2 else n
    c = ctx.to_device(host.synth_normal(0, 33, (m, nout)))
    copies = 1 if warm else -(-COLD_BYTES // (n * k * 2))
    w0 = host.synth_normal(0, 34, (n, k), 0, 0.02)
    descs = []
    for i in range(copies):
        w = ctx.to_device(w0)  # identical values, distinct buffers: only the addresses rotate
        flags = {0: 0, 1: pkg.ACCUMULATE, 2: pkg.EPI_SILU_MUL}[fl]
        descs.append(pkg.linear_desc(pkg.F16, m, n, k, a, w, c, flags=flags, ldc=nout))
    return descs, 2 * m * n * k


def phase_stamps(pkg, host, ctx, warmup, steps):
    """Config 3 in a graph replay on the measurement build: the per-block
    s_memrealtime records (100 MHz) of the last 8 GEMM launches (the last two
    layers: qkv, o, gate|up, down), reduced per launch to medians over its
    blocks (us): gap from the previous launch's last block end, start skew
    (first to last block start), fill (start to ring stage 0 in), main loop,
    park (accumulators to LDS), stores (first store to block end), span; and
    the fill split at the first DMA-issuing thread's prologue points: kernel
    arguments in, tile enumeration, issue of the first ring stages, wait for
    stage 0."""
    L = pkg.lib()
    L.qa_phase_stamps_read.argtypes = [ctypes.c_void_p] * 4
    slots, blocks, words = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    L.qa_phase_stamps_read(None, ctypes.byref(slots), ctypes.byref(blocks), ctypes.byref(words))
    m = 1024
    dec = host.DecoderLinears(ctx, pkg.F16, DEC["layers"], m, DEC["hidden"], DEC["q_dim"],
                              DEC["kv_dim"], DEC["inter"])
    for li in range(DEC["layers"]):
        w = decoder_weights(host, li)
        dec.load_layer(li, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"])
    dec.set_inputs(m, rmsnormed(host, 0, 1, (m, DEC["hidden"]), 0),
                   rmsnormed(host, 0, 2, (m, DEC["q_dim"]), 0),
                   rmsnormed(host, 0, 3, (m, DEC["hidden"]), 0),
                   host.synth_normal(0, 4, (m, DEC["hidden"])))
    dec.time(m, max(1, warmup), 1, use_graph=True)  # capture; the records' slots are fixed then
    pkg.check(L.qa_phase_stamps_clear())
    ms, _ = dec.time(m, 0, max(1, steps), use_graph=True)
    rec = np.zeros((slots.value, blocks.value, words.value), np.uint64)
    pkg.check(L.qa_phase_stamps_read(rec.ctypes.data, None, None, None))
    dec.close()
    names = {(4096, 1024): "qkv", (1024, 2048): "o", (6144, 1024): "gu", (1024, 3072): "down"}
    launches = []
    for sl in range(slots.value):
        r = rec[sl][rec[sl][:, 0] > 0].astype(np.int64)
        if len(r):
            launches.append(r)
    launches.sort(key=lambda r: int(r[:, 0].min()))
    out, prev_end = [], None
    med = lambda x: round(float(np.median(x)) / 100.0, 2)  # noqa: E731  (100 MHz ticks -> us)
    for r in launches:
        t = [r[:, i] for i in range(5)]
        out.append({"site": names.get((int(r[0, 6]), int(r[0, 7])), f"N{r[0, 6]}K{r[0, 7]}"),
                    "blocks": int(len(r)),
                    "gap": None if prev_end is None else round((int(t[0].min()) - prev_end) / 100.0, 2),
                    "start_skew": round(int(t[0].max() - t[0].min()) / 100.0, 2),
                    "fill": med(t[1] - t[0]), "loop": med(t[2] - t[1]), "park": med(t[3] - t[2]),
                    "stores": med(t[4] - t[3]),
                    "span": round(int(t[4].max() - t[0].min()) / 100.0, 2),
                    "fill_args": med(r[:, 8] - t[0]), "fill_tile_enum": med(r[:, 9] - r[:, 8]),
                    "fill_issue": med(r[:, 10] - r[:, 9]), "fill_stage0_wait": med(t[1] - r[:, 10])})
        prev_end = int(t[4].max())
    return {"phase_stamps_config3": out, "step_ms": round(ms, 4),
            "note": "measurement build (-DQA_PHASE_STAMPS); medians over blocks, us; the last "
                    "two layers of the last graph replay"}


def phase_stamps_prefill(pkg, host, ctx, launches=3):
    """The 300 s forward's large GEMM shapes (decoder prefill at 4352 rows,
    the tower's fc1 at 3900) on the measurement build: eager back-to-back
    launches of one shape, the per-block records of the last one, split by
    the round of tiles each block ran in (one block per CU at a time, started
    in dispatch order); per round, medians over its blocks (us from the
    launch's first block start)."""
    L = pkg.lib()
    L.qa_phase_stamps_read.argtypes = [ctypes.c_void_p] * 4
    slots, blocks, words = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    L.qa_phase_stamps_read(None, ctypes.byref(slots), ctypes.byref(blocks), ctypes.byref(words))
    ncu = 256
    cases = [("qkv", 4352, 4096, 1024, 0, False), ("o", 4352, 1024, 2048, pkg.ACCUMULATE, False),
             ("gate|up", 4352, 6144, 1024, pkg.EPI_SILU_MUL, False),
             ("down", 4352, 1024, 3072, pkg.ACCUMULATE, False),
             ("tower fc1", 3900, 3584, 896, pkg.EPI_GELU, True)]
    out = []
    for name, m, n, k, flags, bias in cases:
        a = host.synth_normal(0, 1, (m, k))
        w = host.synth_normal(0, 2, (n, k), 0, 0.02)
        nout = n // 2 if flags & pkg.EPI_SILU_MUL else n
        da, dw = ctx.to_device(a), ctx.to_device(w)
        dc = ctx.to_device(host.synth_normal(0, 4, (m, nout)))
        db = ctx.to_device(host.synth_normal(0, 3, (n,), 0, 0.01)) if bias else None
        desc = pkg.linear_desc(pkg.F16, m, n, k, da, dw, dc, flags=flags, bias=db, ldc=nout)
        for _ in range(10):
            ctx.linear(desc)
        ctx.sync()
        pkg.check(L.qa_phase_stamps_clear())
        for _ in range(launches):
            ctx.linear(desc)
        ctx.sync()
        rec = np.zeros((slots.value, blocks.value, words.value), np.uint64)
        pkg.check(L.qa_phase_stamps_read(rec.ctypes.data, None, None, None))
        for b in (da, dw, dc, db):
            if b is not None:
                b.free()
        runs = [rec[s][rec[s][:, 0] > 0].astype(np.int64) for s in range(slots.value)]
        r = sorted([x for x in runs if len(x)], key=lambda x: int(x[:, 0].min()))[-1]
        t = [(r[:, i] - r[:, 0].min()) / 100.0 for i in range(5)]  # 100 MHz ticks -> us
        # blocks start in dispatch order as CUs free up: the i-th block to
        # start ran in round i // (one block per CU)
        rnd = np.empty(len(r), int)
        rnd[np.argsort(t[0], kind="stable")] = np.arange(len(r)) // ncu
        rounds = []
        for q in sorted(set(rnd.tolist())):
            s = rnd == q
            med = lambda x: round(float(np.median(x[s])), 2)  # noqa: E731
            rounds.append({"blocks": int(s.sum()), "start": med(t[0]), "fill": med(t[1] - t[0]),
                           "loop": med(t[2] - t[1]), "park": med(t[3] - t[2]),
                           "stores": med(t[4] - t[3]), "last_end": round(float(t[4][s].max()), 2)})
        out.append({"site": name, "m": m, "n": n, "k": k, "blocks": int(len(r)),
                    "span": round(float(t[4].max()), 2), "rounds": rounds})
    return {"phase_stamps_prefill": out,
            "note": "measurement build (-DQA_PHASE_STAMPS), f16, eager launches; per round of "
                    "tiles, medians over its blocks, us from the first block start"}


def config2_pair_descs(pkg, host, ctx, warm):
    """Config 2's MLP block as launch pairs (gate|up + SiLU.up, then down +
    residual, M = 512): warm one weight set, cold 16 distinct sets (320 MB).
    Returns (descriptors in launch order, FLOPs per pair)."""
    m, hid, it = 512, DEC["hidden"], DEC["inter"]
    x = ctx.to_device(host.synth_normal(0, 21, (m, hid)))
    act = ctx.alloc(m * it * 2)
    descs = []
    for i in range(1 if warm else 16):
        gu = ctx.to_device(host.synth_normal(0, 22 if i == 0 else 2200 + 2 * i, (2 * it, hid), 0, 0.02))
        dn = ctx.to_device(host.synth_normal(0, 23 if i == 0 else 2201 + 2 * i, (hid, it), 0, 0.02))
        descs += [pkg.linear_desc(pkg.F16, m, 2 * it, hid, x, gu, act, flags=pkg.EPI_SILU_MUL),
                  pkg.linear_desc(pkg.F16, m, hid, it, act, dn, x, flags=pkg.ACCUMULATE)]
    return descs, 2 * m * 2 * it * hid + 2 * m * hid * it


def config1_protocol(pkg, host, ctx):
    """Config 1 (x [256,1024] . W[3072,1024]^T, HBM-bound): warm (one W) and
    cold (48 copies of W, 302 MB > the 256 MB MALL), with the algorithmic
    bytes over the median launch."""
    m, n, k = 256, 3072, 1024
    a = ctx.to_device(host.synth_normal(0, 11, (m, k)))
    c = ctx.alloc(m * n * 2)
    ws = [ctx.to_device(host.synth_normal(0, 12 if i == 0 else 1200 + i, (n, k), 0, 0.02))
          for i in range(48)]
    descs = [pkg.linear_desc(pkg.F16, m, n, k, a, w, c) for w in ws]
    warm = dist(host.time_linears_each(ctx, descs[:1], 20, 200))
    cold = dist(host.time_linears_each(ctx, descs, 20, 288))
    warm_k = dist(host.time_linears_stamped(ctx, descs[:1], 20, 200))
    cold_k = dist(host.time_linears_stamped(ctx, descs, 20, 288))
    algo = 2 * (m * k + n * k + m * n)
    for b in [a, c] + ws:
        b.free()
    f = 2 * m * n * k
    return {"warm": warm, "cold": cold, "warm_kernel": warm_k, "cold_kernel": cold_k,
            "algorithmic_bytes": algo,
            "hbm_gbs_cold_median": round(algo / (cold["median"] * 1e-6) / 1e9, 1),
            "hbm_frac_cold_median": round(algo / (cold["median"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "hbm_gbs_cold_kernel_median": round(algo / (cold_k["median"] * 1e-6) / 1e9, 1),
            "hbm_frac_cold_kernel_median":
                round(algo / (cold_k["median"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "tflops_cold_median": round(f / (cold["median"] * 1e-6) / 1e12, 1),
            "tflops_warm_median": round(f / (warm["median"] * 1e-6) / 1e12, 1),
            "note": "cold / warm: event-to-event intervals of back-to-back launches (each with its "
                    "share of the launch gap); *_kernel: the same launches timed by the kernel's "
                    "own dispatch (qa_time_next_launch), kernel time alone"}


def config2_protocol(pkg, host, ctx):
    """Config 2 (the MLP block at M = 512: gate|up + SiLU.up, then down +
    residual): per-launch distributions of the pair, warm and cold (16 weight
    sets, 320 MB)."""
    m, hid, it = 512, 1024, 3072
    x = ctx.to_device(host.synth_normal(0, 21, (m, hid)))
    act = ctx.alloc(m * it * 2)
    sets = [(ctx.to_device(host.synth_normal(0, 22 if i == 0 else 2200 + 2 * i, (2 * it, hid), 0, 0.02)),
             ctx.to_device(host.synth_normal(0, 23 if i == 0 else 2201 + 2 * i, (hid, it), 0, 0.02)))
            for i in range(16)]
    descs = []
    for gu, dn in sets:
        descs += [pkg.linear_desc(pkg.F16, m, 2 * it, hid, x, gu, act, flags=pkg.EPI_SILU_MUL),
                  pkg.linear_desc(pkg.F16, m, hid, it, act, dn, x, flags=pkg.ACCUMULATE)]
    warm = host.time_linears_each(ctx, descs[:2], 20, 400)
    cold = host.time_linears_each(ctx, descs, 20, 416)
    warm_k = host.time_linears_stamped(ctx, descs[:2], 20, 400)
    cold_k = host.time_linears_stamped(ctx, descs, 20, 416)
    pair = lambda ms: ms[0::2] + ms[1::2]  # noqa: E731
    f = 2 * m * 2 * it * hid + 2 * m * hid * it
    out = {"warm": dist(pair(warm)), "cold": dist(pair(cold)),
           "gu_cold": dist(cold[0::2]), "down_cold": dist(cold[1::2]),
           "warm_kernel": dist(pair(warm_k)), "cold_kernel": dist(pair(cold_k)),
           "gu_cold_kernel": dist(cold_k[0::2]), "down_cold_kernel": dist(cold_k[1::2])}
    out["tflops_cold_median"] = round(f / (out["cold"]["median"] * 1e-6) / 1e12, 1)
    for b in [x, act] + [b for s in sets for b in s]:
        b.free()
    return out


def dec_layer_flops(s):
    """Per-layer FLOPs of a prefill of s tokens: the four projections plus the
    causal attention (QK^T and PV over the s(s+1)/2 visible pairs per head)."""
    per, _ = dec_flops(s)
    attn = 4 * DEC["hd"] * DEC["nqh"] * s * (s + 1) // 2
    return sum(per.values()), attn


def bench_prefill(host, tdec, rows, warmup, steps):
    """Whole decoder layers (norms, qkv, RoPE + KV write, attention, o,
    gate|up + SiLU, down) over `rows` tokens, 28 layers, one hipGraph per step."""
    h = rmsnormed(host, 2, 7, (rows, DEC["hidden"]), 0)
    tdec.set_hidden(h)
    ev_ms, wall_ms, _ = settled(lambda w, s: tdec.time(rows, w, s, use_graph=True), warmup, steps)
    ops = tdec.profile_ops(rows, 2)
    lin_f, attn_f = dec_layer_flops(rows)
    t_attn = ops["attention"]
    return {
        "ms": round(max(ev_ms, wall_ms), 3),
        "tflops": round(DEC["layers"] * (lin_f + attn_f) / (max(ev_ms, wall_ms) * 1e-3) / 1e12, 1),
        "per_layer_op_us": {k: round(v * 1e3, 2) for k, v in ops.items()},
        "attention_tflops": round(attn_f / (t_attn * 1e-3) / 1e12, 1),
    }


AUDIO = dict(layers=18, n_mels=128, cs=100, c_conv=480, d_model=896, nh=14, ffn=3584,
             out_dim=1024, wlen=104, chunks=300)  # 300 s of 16 kHz audio: 30000 mel frames


def bench_audio_tower(host, ctx, dtype, warmup, steps):
    """The whole audio tower (GpuAudioEncoder::encode) over 300 s of audio:
    300 mel chunks -> conv stem -> conv_out + position add -> 18 windowed
    layers -> projector, 3900 tokens, one hipGraph per step; random weights."""
    A = AUDIO
    enc = host.AudioEncoder(ctx, dtype, A["layers"], A["chunks"], A["n_mels"], A["cs"],
                            A["c_conv"], A["d_model"], A["nh"], A["ffn"], A["out_dim"], A["wlen"])
    g = lambda tid, shape, std: host.synth_normal(9, tid, shape, 0.0, std, dtype)  # noqa: E731
    cc, dm, ff = A["c_conv"], A["d_model"], A["ffn"]
    enc.load_conv(0, g(1, (cc, 1, 3, 3), 1 / 3.0), g(2, (cc,), 0.05))
    enc.load_conv(1, g(3, (cc, cc, 3, 3), (9 * cc) ** -0.5), g(4, (cc,), 0.05))
    enc.load_conv(2, g(5, (cc, cc, 3, 3), (9 * cc) ** -0.5), g(6, (cc,), 0.05))
    enc.load_conv_out(g(7, (dm, cc * 16), (cc * 16) ** -0.5), g(8, (dm,), 0.02))
    ones, zeros = np.ones(dm, np.float32), np.zeros(dm, np.float32)
    for li in range(A["layers"]):
        b = 100 + 16 * li
        enc.load_layer(li, ones, zeros, g(b, (3 * dm, dm), 0.02), g(b + 1, (3 * dm,), 0.02),
                       g(b + 2, (dm, dm), 0.02), g(b + 3, (dm,), 0.02), ones, zeros,
                       g(b + 4, (ff, dm), 0.02), g(b + 5, (ff,), 0.02), g(b + 6, (dm, ff), 0.02),
                       g(b + 7, (dm,), 0.02))
    enc.load_post(ones, zeros, g(20, (dm, dm), 0.02), g(21, (dm,), 0.02),
                  g(22, (A["out_dim"], dm), 0.02), g(23, (A["out_dim"],), 0.02))
    enc.set_mel(host.synth_normal(9, 30, (A["chunks"], A["n_mels"], A["cs"]), 0.0, 1.0, dtype))
    ev_ms, wall_ms, _ = settled(lambda w, s: enc.time(A["chunks"], 0, w, s, use_graph=True),
                                warmup, steps)
    prof = enc.profile(A["chunks"], 0, 2)
    n = enc.tokens(A["chunks"], 0)
    enc.close()
    px = [A["chunks"] * 64 * 50, A["chunks"] * 32 * 25, A["chunks"] * 16 * 13]
    conv_f = [2 * px[0] * cc * 9, 2 * px[1] * cc * 9 * cc, 2 * px[2] * cc * 9 * cc]
    lin_f = 2 * n * (A["layers"] * (4 * dm * dm + 2 * dm * ff) + cc * 16 * dm + dm * dm
                     + dm * A["out_dim"])
    return {
        "ms": round(max(ev_ms, wall_ms), 3),
        "tokens": n,
        "tflops_total": round((sum(conv_f) + lin_f) / (max(ev_ms, wall_ms) * 1e-3) / 1e12, 1),
        "phase_ms": {k: round(v, 3) for k, v in prof.items()},
        "conv2_tflops": round(conv_f[1] / (prof["conv2"] * 1e-3) / 1e12, 1),
        "conv3_tflops": round(conv_f[2] / (prof["conv3"] * 1e-3) / 1e12, 1),
        "conv1_out_gbs": round(px[0] * cc * 2 / (prof["conv1"] * 1e-3) / 1e9, 1),
    }


E2E = dict(seconds=300.0, words=120, enc_layers=18, dec_layers=28, dtype=0, seed=5)
E2E_GOLDEN = os.path.join(ROOT, "tests", "golden", "e2e_300s.json")


def bench_e2e(pkg, ctx, warmup, steps):
    """the whole aligner forward over 300 s of synthetic
    audio and 120 synthetic words, f16, random-init 0.6B-shaped weights:
    log-mel -> 18-layer audio tower -> embedding gather + audio scatter ->
    28-layer decoder prefill -> timestamp head, one hipGraph per step with
    the samples and the assembled input resident in HBM.  Also times the
    eager forward with the classes' readback and the host repair, the same
    forward with single-rounded probabilities (the reference GPU's softmax
    storage, `p16_ms`), and
    compares the classes with the oracle's (the committed fixture made from
    the same seeded inputs by tests/golden/make_e2e_golden.py)."""
    from qwen3_aligner_wgpu_amd import synthetic as syn
    c = E2E
    w = syn.aligner_weights(c["dtype"], c["enc_layers"], c["dec_layers"], c["seed"])
    x = syn.synthetic_audio(c["seconds"], c["seed"])
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(c["words"], c["seed"])]
    al, enc, dec = syn.build_aligner(pkg, ctx, c["dtype"], w, c["seconds"] + 0.01, max(PREFILL_ROWS))
    del w
    try:
        info = al.prepare(x, words)
        ev_ms, wall_ms, _ = settled(lambda w, s: al.time(w, s, use_graph=True), warmup, steps)
        phases = al.profile(2)
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            al.forward()
            al.result()
        eager_ms = (time.perf_counter() - t0) * 1e3 / reps
        classes = al.read("classes")
        # the same forward with the probabilities rounded once to 16 bits before
        # P.V, as the reference's own GPU softmax stores them (QA_ATTN_P16)
        dec.set_attention_flags(pkg.QA_ATTN_P16)
        ev16, wall16, _ = settled(lambda w, s: al.time(w, s, use_graph=True), warmup, steps)
        al.forward()
        classes16 = al.read("classes")
        dec.set_attention_flags(0)
    finally:
        al.close()
        enc.close()
        dec.close()
    out = {
        "ms": round(max(ev_ms, wall_ms), 3),
        "event_ms": round(ev_ms, 3),
        "wall_ms": round(wall_ms, 3),
        "eager_with_readback_ms": round(eager_ms, 3),
        "phase_ms": {k: round(v, 3) for k, v in phases.items()},
        "seq": info["seq"], "audio_tokens": info["n_audio"], "slots": info["slots"],
        "p16_ms": round(max(ev16, wall16), 3),
    }
    try:
        gold = json.load(open(E2E_GOLDEN))
        if gold["config"] == c:
            want = np.array(gold["classes"])
            clear = np.array(gold["gap"]) > 2.0 ** -8 * np.array(gold["logit_rms"])
            out["argmax_identical_slots"] = int((classes == want).sum())
            out["argmax_clear_margin_slots"] = int(clear.sum())
            out["argmax_identical_at_clear_slots"] = bool((classes == want)[clear].all())
            out["p16_argmax_identical_slots"] = int((classes16 == want).sum())
    except (OSError, KeyError, ValueError):
        out["argmax_identical_slots"] = None
    return out


def attention_stamps(pkg, host, ctx):
    """The decoder attention at s = 4352 (16 q heads, 8 kv heads, hd 128, f16,
    synthetic q / K / V) on the measurement build, in both probability modes:
    every wave's s_memtime cycles by phase (qa_attn_stamps_read), as medians
    over the waves -- per MFMA phase and per VALU phase, and each phase
    kind's share of a wave's cycles."""
    L = pkg.lib()
    L.qa_attn_stamps_read.argtypes = [ctypes.c_void_p] * 4
    nb, nw, nwd = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    pkg.check(L.qa_attn_stamps_read(None, ctypes.byref(nb), ctypes.byref(nw), ctypes.byref(nwd)))
    rows, nqh, nkvh, hd = 4352, 16, 8, 128
    q = ctx.to_device(host.synth_normal(0, 1, (nqh, rows, hd), 0, 0.3))
    kc = ctx.to_device(host.synth_normal(0, 2, (nkvh, rows, hd)))
    vc = ctx.to_device(host.synth_normal(0, 3, (nkvh, hd, rows)))
    out = ctx.alloc(rows * nqh * hd * 2)
    res = {}
    for name, flags in (("two-term P (default)", 0), ("single-rounded P", pkg.QA_ATTN_P16)):
        desc = pkg.AttentionDesc(dtype=pkg.F16, flags=flags, rows=rows, nqh=nqh, nkvh=nkvh, hd=hd,
                                 q=int(q), k_cache=int(kc), v_cache=int(vc), cap=rows, q0=0,
                                 out=int(out), ldo=nqh * hd)
        for _ in range(3):
            ctx.attention_prefill(desc)
        ctx.sync()
        pkg.check(L.qa_attn_stamps_clear())
        ctx.attention_prefill(desc)
        ctx.sync()
        rec = np.zeros((nb.value, nw.value, nwd.value), np.uint64)
        pkg.check(L.qa_attn_stamps_read(rec.ctypes.data, None, None, None))
        r = rec.reshape(-1, nwd.value).astype(np.float64)
        r = r[r[:, 7] > 0]  # waves that ran at least one MFMA phase
        tot = r[:, :7].sum(axis=1)
        med = lambda x: round(float(np.median(x)), 3)  # noqa: E731
        res[name] = {
            "waves": int(len(r)),
            "cycles_per_mfma_phase": med(r[:, 1] / r[:, 7]),
            "cycles_per_valu_phase": med(r[r[:, 8] > 0, 2] / r[r[:, 8] > 0, 8]),
            "share": {k: med(r[:, i] / tot) for i, k in enumerate(
                ("prologue", "mfma_phases", "valu_phases", "no_work_phases", "barrier",
                 "merge_and_output", "dma_lds_waits"))},
            "mfma_phases_per_wave": med(r[:, 7]),
            "wave_cycles": med(tot),
        }
    for b in (q, kc, vc, out):
        b.free()
    return res


def e2e_eager(pkg, ctx, warmup, steps, p16=False):
    """The config-5 forward of bench_e2e, launched eagerly (no hipGraph):
    `warmup` then `steps` forwards, timed by HIP events and the host clock.
    For kernel traces: each kernel then appears once per forward, in launch
    order, with no graph machinery in the process.  p16: the attention's
    probabilities rounded once to 16 bits (QA_ATTN_P16)."""
    from qwen3_aligner_wgpu_amd import synthetic as syn
    c = E2E
    w = syn.aligner_weights(c["dtype"], c["enc_layers"], c["dec_layers"], c["seed"])
    x = syn.synthetic_audio(c["seconds"], c["seed"])
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(c["words"], c["seed"])]
    al, enc, dec = syn.build_aligner(pkg, ctx, c["dtype"], w, c["seconds"] + 0.01, max(PREFILL_ROWS))
    del w
    try:
        al.prepare(x, words)
        if p16:
            dec.set_attention_flags(pkg.QA_ATTN_P16)
        ev_ms, wall_ms = al.time(warmup, steps, use_graph=False)
    finally:
        al.close()
        enc.close()
        dec.close()
    return {"eager_ms": round(max(ev_ms, wall_ms), 3), "event_ms": round(ev_ms, 3),
            "wall_ms": round(wall_ms, 3), "warmup": warmup, "steps": steps, "attn_p16": p16}


def bench_encoder(pkg, host, ctx, m, warmup, steps):
    dt = pkg.BF16
    d, f, ck = ENC["d_model"], ENC["ffn"], ENC["conv_k"]
    enc = host.EncoderLinears(ctx, dt, ENC["layers"], m, d, f, ck)
    for li in range(ENC["layers"]):
        g = lambda i, shp, std: host.synth_normal(1, 5000 + li * 16 + i, shp, 0.0, std, dt)
        enc.load_layer(li, g(0, (3 * d, d), 0.02), g(1, (3 * d,), 0.01), g(2, (d, d), 0.02),
                       g(3, (d,), 0.01), g(4, (f, d), 0.02), g(5, (f,), 0.01), g(6, (d, f), 0.02),
                       g(7, (d,), 0.01))
    enc.load_conv(host.synth_normal(1, 4000, (d, ck), 0.0, 0.02, dt),
                  host.synth_normal(1, 4001, (d,), 0.0, 0.01, dt))
    enc.set_inputs(m, host.synth_normal(1, 1, (m, ck), 0, 1, dt), rmsnormed(host, 1, 2, (m, d), dt),
                   rmsnormed(host, 1, 3, (m, d), dt), rmsnormed(host, 1, 4, (m, d), dt),
                   host.synth_normal(1, 5, (m, d), 0, 1, dt))
    ev_ms, wall_ms, _ = settled(lambda w, s: enc.time(m, w, s, use_graph=True), warmup, steps)
    sites = enc.profile_sites(m, 2)
    enc.close()
    flops = 2 * m * (ENC["layers"] * (3 * d * d + d * d + 2 * d * f) + d * ck)
    return ev_ms, wall_ms, sites, flops


def vs_hipblaslt(pkg, ctx, launches):
    """The decoder's four projections at M = 1024 (config 3) and M = 4352 (the
    300 s prefill), f16, warm weights (one W), `launches` back-to-back launches
    each: first through qa_linear, then through torch's f16 GEMM (hipBLASLt on
    this image): `addmm_` (beta = 1) where qa_linear adds the residual, a plain
    `mm` for gate|up, which gets no SiLU.up epilogue in the library (its output
    is twice as wide).  Only launches: the durations come from a kernel trace
    of this run (rocprofv3 --kernel-trace), in the order returned."""
    import torch
    shapes = []
    for m in (1024, 4352):
        shapes += [(f"qkv/{m}", m, DEC["q_dim"] + 2 * DEC["kv_dim"], DEC["hidden"], 0),
                   (f"o/{m}", m, DEC["hidden"], DEC["q_dim"], 1),
                   (f"gu/{m}", m, 2 * DEC["inter"], DEC["hidden"], 2),
                   (f"down/{m}", m, DEC["hidden"], DEC["inter"], 1)]
    order = []
    for name, m, n, k, fl in shapes:
        rng = np.random.default_rng(0)
        a = rng.standard_normal((m, k)).astype(np.float16)
        w = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
        nout = n // 2 if fl == 2 else n
        c = rng.standard_normal((m, nout)).astype(np.float16)
        da, dw, dc = (ctx.to_device(x.view(np.uint16)) for x in (a, w, c))
        flags = {0: 0, 1: pkg.ACCUMULATE, 2: pkg.EPI_SILU_MUL}[fl]
        d = pkg.linear_desc(pkg.F16, m, n, k, da, dw, dc, flags=flags, ldc=nout)
        for _ in range(launches):
            ctx.linear(d)
        ctx.sync()
        for b in (da, dw, dc):
            b.free()
        ta, tw = torch.from_numpy(a).cuda(), torch.from_numpy(w).cuda()
        tc = torch.from_numpy(c if fl != 2 else np.zeros((m, n), np.float16)).cuda()
        torch.cuda.synchronize()
        for _ in range(launches):
            if fl == 1:
                tc.addmm_(ta, tw.t())
            else:
                torch.mm(ta, tw.t(), out=tc)
        torch.cuda.synchronize()
        order.append(dict(shape=name, m=m, n=n, k=k, launches=launches))
    return {"vs_hipblaslt": order, "blas": str(torch.backends.cuda.preferred_blas_library())}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of oracle work for cpu_baseline (0 disables)")
    ap.add_argument("--no-detail", action="store_true", help="skip configs 1, 2, 4")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the config-5 aligner forward (for profiling); prints its detail")
    ap.add_argument("--e2e-eager", action="store_true",
                    help="only the config-5 forward, launched eagerly without a graph, --warmup "
                         "then --steps times (for kernel traces); prints one JSON line")
    ap.add_argument("--attn-stamps", action="store_true",
                    help="the decoder attention at s = 4352 on the measurement build (make -C "
                         "qwen3-aligner-wgpu_amd/csrc stamps): each wave's cycles by phase, both "
                         "probability modes (one JSON line)")
    ap.add_argument("--attn-p16", action="store_true",
                    help="with --e2e-eager: the attention's probabilities rounded once to 16 bits")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB copy 3 times (calibrates FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--site", default=None,
                    help="only launch one GEMM site --launches times (for rocprofv3 counter runs): "
                         "qkv, o, gu, down (fused), q, k, v, gate, up (unfused) over the 28 layers' "
                         "weights, config1, config2_gu, config2_down, or config2_mlp (gate|up, down "
                         "pairs; --launches counts launches, the figures are per pair)")
    ap.add_argument("--launches", type=int, default=56)
    ap.add_argument("--phase-stamps", action="store_true",
                    help="config 3 on the measurement build (make -C qwen3-aligner-wgpu_amd/csrc "
                         "stamps): per-block phase timestamps of the last two layers' GEMMs in a "
                         "graph replay, as a table of medians (one JSON line)")
    ap.add_argument("--phase-stamps-prefill", action="store_true",
                    help="the 300 s forward's prefill GEMM shapes and the tower's fc1 on the "
                         "measurement build: per-block phase timestamps of one launch each, split "
                         "by round of tiles (one JSON line)")
    ap.add_argument("--warm", action="store_true",
                    help="with --site: repeat layer 0's (or config 1's first) W instead of cycling")
    ap.add_argument("--vs-hipblaslt", action="store_true",
                    help="only launch the decoder projections at M = 1024 and 4352 through "
                         "qa_linear, then through torch's f16 GEMM (hipBLASLt), --launches each, "
                         "for a kernel trace")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this path has no multi-GPU form (the GEMMs shard by "
              "token rows with no exchange; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.phase_stamps or args.phase_stamps_prefill or args.attn_stamps:
        os.environ["QA_BUILD"] = "stamps"  # before the package loads its libraries
    if args.vs_hipblaslt:
        # torch's own HIP runtime and BLAS libraries first: loaded after this
        # package's, torch's hipBLASLt / rocBLAS handles fail to initialise
        import torch  # noqa: F401
    import __graft_entry__ as entry

    pkg = entry.load_package()
    from qwen3_aligner_wgpu_amd import host

    if args.attn_stamps:
        with pkg.Context(0) as ctx:
            print(json.dumps(attention_stamps(pkg, host, ctx)), flush=True)
        return

    if args.e2e_eager:
        with pkg.Context(0) as ctx:
            print(json.dumps(e2e_eager(pkg, ctx, args.warmup, args.steps, args.attn_p16)), flush=True)
        return

    if args.copy_calibration:
        with pkg.Context(0) as ctx:
            host.copy_calibration(ctx, COPY_CAL_BYTES, 3)
        log(f"[bench] copied {COPY_CAL_BYTES} bytes x3")
        return

    if args.site:
        with pkg.Context(0) as ctx:
            descs, flops = site_descs(pkg, host, ctx, args.site, args.warm)
            ms = host.time_linears_each(ctx, descs, 0, args.launches)
            if args.site == "config2_mlp":  # launch pairs: per-pair figures
                ms = ms[0::2] + ms[1::2]
            print(json.dumps({"site": args.site, "warm": args.warm, "weight_sets": len(descs),
                              "flops_per_launch": flops, "per_launch": dist(ms)}), flush=True)
        return

    if args.vs_hipblaslt:
        with pkg.Context(0) as ctx:
            print(json.dumps(vs_hipblaslt(pkg, ctx, args.launches)), flush=True)
        return

    if args.phase_stamps:
        with pkg.Context(0) as ctx:
            print(json.dumps(phase_stamps(pkg, host, ctx, args.warmup, args.steps)), flush=True)
        return

    if args.phase_stamps_prefill:
        with pkg.Context(0) as ctx:
            print(json.dumps(phase_stamps_prefill(pkg, host, ctx)), flush=True)
        return

    if args.e2e_only:
        with pkg.Context(0) as ctx:
            print(json.dumps({"e2e_300s": bench_e2e(pkg, ctx, args.warmup, args.steps)}), flush=True)
        return

    m = 1024
    ctx = pkg.Context(0)
    per, total_flops = dec_flops(m)
    tdec = None
    if not args.no_detail:
        tdec = host.TextDecoder(ctx, pkg.F16, DEC["layers"], max(PREFILL_ROWS), DEC["hidden"],
                                DEC["nqh"], DEC["nkvh"], DEC["hd"], DEC["inter"])
        tdec.set_rope(*pkg.rope_tables(max(PREFILL_ROWS), DEC["hd"], 1e6, pkg.F16))
    dec, ev_ms, wall_ms, sites, settle = bench_decoder(pkg, host, ctx, m, args.warmup, args.steps,
                                                       tdec)
    ms_per_step = max(ev_ms, wall_ms)
    value = total_flops / (ms_per_step * 1e-3) / 1e12
    gu_ms = sites["gu"]
    achieved = per["gu"] / (gu_ms * 1e-3) / 1e12
    log(f"[bench] config3: {ms_per_step:.3f} ms/step (events {ev_ms:.3f}, wall {wall_ms:.3f}) "
        f"{value:.1f} TFLOP/s; sites ms {sites}")

    detail = {
        "config3_sites_us": {k: round(v * 1e3, 2) for k, v in sites.items()},
        "config3_sites_tflops": {k: round(per[k] / (v * 1e-3) / 1e12, 1) for k, v in sites.items()},
        "config3_event_ms_per_step": round(ev_ms, 4),
        "config3_wall_ms_per_step": round(wall_ms, 4),
    }
    if not args.no_detail:
        # config 1: one up-projection, M=256
        a = host.synth_normal(0, 11, (256, 1024))
        w = host.synth_normal(0, 12, (3072, 1024), 0, 0.02)
        da, dw, dc = ctx.to_device(a), ctx.to_device(w), ctx.alloc(256 * 3072 * 2)
        t1 = host.time_linear(ctx, pkg.linear_desc(pkg.F16, 256, 3072, 1024, da, dw, dc), 5, 50)
        f1 = 2 * 256 * 3072 * 1024
        detail["config1_us"] = round(t1 * 1e3, 2)
        detail["config1_tflops"] = round(f1 / (t1 * 1e-3) / 1e12, 1)
        detail["config1_hbm_gbs"] = round(2 * (256 * 1024 + 3072 * 1024 + 256 * 3072) / (t1 * 1e-3) / 1e9, 1)
        for b in (da, dw, dc):
            b.free()
        # config 2: the fused MLP block, M=512
        x = host.synth_normal(0, 21, (512, 1024))
        wgu = host.synth_normal(0, 22, (6144, 1024), 0, 0.02)
        wd = host.synth_normal(0, 23, (1024, 3072), 0, 0.02)
        dx, dgu, dwd, dact = ctx.to_device(x), ctx.to_device(wgu), ctx.to_device(wd), ctx.alloc(512 * 3072 * 2)
        gu_d = pkg.linear_desc(pkg.F16, 512, 6144, 1024, dx, dgu, dact, flags=pkg.EPI_SILU_MUL)
        dn_d = pkg.linear_desc(pkg.F16, 512, 1024, 3072, dact, dwd, dx, flags=pkg.ACCUMULATE)
        t2 = host.time_linear(ctx, gu_d, 5, 50) + host.time_linear(ctx, dn_d, 5, 50)
        f2 = 2 * 512 * 6144 * 1024 + 2 * 512 * 1024 * 3072
        detail["config2_us"] = round(t2 * 1e3, 2)
        detail["config2_tflops"] = round(f2 / (t2 * 1e-3) / 1e12, 1)
        for b in (dx, dgu, dwd, dact):
            b.free()
        # the per-launch protocol: each config-3 site fused and unfused, cold and
        # warm, and configs 1 and 2 cold and warm
        for unf, key in ((False, "config3_sites_protocol"), (True, "config3_unfused_protocol")):
            ss = SiteSet(pkg, host, ctx, m, DEC["layers"], unf)
            sites_d, step_d = site_protocol(host, ctx, ss)
            ss.close()
            detail[key] = {"sites": sites_d, **step_d}
            log(f"[bench] {key}: {step_d}; " +
                ", ".join(f"{s} {v['cold']['median']}/{v['warm']['median']} us" for s, v in sites_d.items()))
        detail["config1_protocol"] = config1_protocol(pkg, host, ctx)
        detail["config2_protocol"] = config2_protocol(pkg, host, ctx)
        log(f"[bench] config1: {detail['config1_protocol']}")
        log(f"[bench] config2: {detail['config2_protocol']}")
    dec.close()
    if tdec is not None:
        # whole decoder layers: config 3's 1024 tokens and config 5's prefill length
        for rows in PREFILL_ROWS:
            r = bench_prefill(host, tdec, rows, 2, 5)
            detail[f"decoder_prefill_{rows}"] = r
            log(f"[bench] decoder prefill s={rows}: {r}")
        tdec.close()
    if not args.no_detail:
        # config 4: 18-layer audio-tower linear stack, bf16, M=3750, + conv GEMM
        ev4, wall4, sites4, f4 = bench_encoder(pkg, host, ctx, 3750, 2, 5)
        t4 = max(ev4, wall4)
        detail["config4_ms"] = round(t4, 4)
        detail["config4_tflops"] = round(f4 / (t4 * 1e-3) / 1e12, 1)
        detail["config4_sites_us"] = {k: round(v * 1e3, 2) for k, v in sites4.items()}
        # the whole audio tower over 300 s (config 5's encoder), f16
        r = bench_audio_tower(host, ctx, pkg.F16, 1, 3)
        detail["audio_tower_300s"] = r
        log(f"[bench] audio tower 300 s: {r}")
    e2e = {"ms": None}
    if not args.no_detail:
        e2e = bench_e2e(pkg, ctx, 2, 5)
        detail["e2e_300s"] = e2e
        log(f"[bench] aligner forward 300 s: {e2e}")
    ctx.close()

    traffic, traffic_kernel, busy_pct, _ = measured_counters("gu")
    cpu = None
    if args.cpu_budget > 0:
        orc = entry.load_oracle()
        cpu = cpu_baseline(orc, host, m, args.cpu_budget)
        log(f"[bench] cpu_baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        # untimed graph replays ahead of the warm-up steps, >= SETTLE_MS of them
        # (the GPU's clocks settle after ~70 ms of continuous work)
        "settle_steps": settle,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded SplitMix64/Box-Muller; weights N(0,0.02), activations "
                "RMSNorm'd N(0,1))",
        "config": {
            "workload": "config3: 28 Qwen3-0.6B decoder layers x {qkv 1024->4096, o 2048->1024 "
                        "+res, gate|up 1024->6144 +SiLU.up, down 3072->1024 +res}, M=1024 tokens, "
                        "one hipGraph per step",
            "tokens": m,
            "layers": DEC["layers"],
            "gemms_per_step": 4 * DEC["layers"],
            "gflop_per_step": round(total_flops / 1e9, 2),
        },
        "pct_mfma_peak": round(100 * value / PEAK_F16_TFLOPS, 2),
        "e2e_ms_per_300s_audio": e2e["ms"],
        "roofline": {
            "bound": "mfma",
            "kernel": "gate|up GEMM + SiLU.up epilogue, [1024,1024]x[6144,1024]^T",
            "achieved": round(achieved, 2),
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_kernel": traffic_kernel,
            "mfma_busy_pct": busy_pct,
            "counter_source": "profiles/gemm_sites_counters.md" if traffic else None,
        },
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
