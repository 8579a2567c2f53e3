#!/usr/bin/env python
"""Benchmark of the MI355X ring-attention compute path.

Headline (BASELINE.json ``metric``): the simulated P=8 zigzag-causal ring of
configs[2] (S=131072, 16384 tokens per rank as two 8192 chunks, H=16 MHA, D=128,
bf16) forward + backward on ONE GPU, reported as TFLOP/s of algorithmic work
(FA2 convention: 4*D*H per attended pair forward, 10*D*H backward; masked pairs
are not counted). One step = one full emulated ring forward + reverse-ring
backward over synthetic inputs already resident in HBM.

The JSON line also carries the roofline of the dominant kernel (HIP events around
every launch on the launching stream), the per-kernel breakdown, the HBM-bound
kernels (zigzag shard of q/k/v at configs[2], standalone LSE merge at configs[1],
cp_linear_scan fwd+bwd at configs[4]) and the CPU baseline: the oracle (torch CPU
fp32 restatement of the reference ``math`` path) timed on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time

import torch

BF16_PEAK_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 4096 FLOP/clk x 2.4 GHz)
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E


def _sync():
    torch.cuda.synchronize()


def _gen(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


def _time(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    _sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    _sync()
    return (time.perf_counter() - t0) / steps * 1e3


def _time_gpu(fn, steps, warmup):
    """Mean ms per call from HIP events recorded on the current stream around ``steps``
    back-to-back calls (the GPU's time, launch gaps included, not the host's)."""
    for _ in range(warmup):
        fn()
    _sync()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    _sync()
    return e0.elapsed_time(e1) / steps


class ClockSampler:
    """Samples the GPU's current shader clock (``rocm-smi --showclocks``, read from sysfs, no
    GPU work) from a background thread while a timed region runs: the clock under load, which
    the power limit holds below the 2.4 GHz of the peak figure."""

    def __init__(self, period_s=0.25):
        self.period, self.mhz = period_s, []
        self._stop = None

    def _read(self):
        try:
            out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True,
                                 timeout=10).stdout
        except Exception:
            return None
        for ln in out.splitlines():
            if "sclk" in ln and "Mhz" in ln:
                try:
                    return int(ln.rsplit("(", 1)[1].split("Mhz")[0])
                except (IndexError, ValueError):
                    return None
        return None

    def __enter__(self):
        import threading

        self._stop = threading.Event()

        def run():
            while not self._stop.is_set():
                v = self._read()
                if v is not None:
                    self.mhz.append(v)
                self._stop.wait(self.period)

        self._t = threading.Thread(target=run, daemon=True)
        self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._t.join(timeout=15)
        return False

    def summary(self):
        if not self.mhz:
            return None
        v = sorted(self.mhz)
        return {"samples": len(v), "min_mhz": v[0], "median_mhz": v[len(v) // 2],
                "max_mhz": v[-1], "source": "rocm-smi --showclocks sampled during the timed steps"}


def gemm_ceiling(steps=20, warmup=5):
    """The library bf16 GEMM rate on this GPU (torch.matmul -> hipBLASLt), the practical MFMA
    ceiling the attention kernels are compared with, at 8192^3 and 16384^3, and the clock
    during it."""
    out = {}
    for n in (8192, 16384):
        a = _gen((n, n), 11)
        b = _gen((n, n), 12)
        with ClockSampler() as clk:
            ms = _time(lambda: torch.matmul(a, b), steps, warmup)
        tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
        out[f"bf16_{n}^3"] = {"ms": round(ms, 3), "TFLOP/s": round(tf, 1),
                              "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                              "sclk_under_load": clk.summary()}
        del a, b
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- configs[2] ring
def ring_workload(steps, warmup):
    from ringmaster_amd.ring.schedule import ring_pairs_per_rank
    from ringmaster_amd.ring.zigzag import KernelTimer, zigzag_ring_attention

    P, S, H, D = 8, 131072, 16, 128
    L = S // P
    q = _gen((P, 1, H, L, D), 1).requires_grad_(True)
    k = _gen((P, 1, H, L, D), 2).requires_grad_(True)
    v = _gen((P, 1, H, L, D), 3).requires_grad_(True)
    dout = _gen((P, 1, L, H, D), 4)
    pairs = P * ring_pairs_per_rank(P, L)
    assert pairs == S * (S + 1) // 2
    flops = 14 * D * H * pairs
    timer = KernelTimer()

    def step(t=None):
        out = zigzag_ring_attention(q, k, v, timer=t)
        torch.autograd.grad(out, (q, k, v), dout)

    for _ in range(warmup):
        step()
    _sync()
    with ClockSampler() as clk:
        t0 = time.perf_counter()
        for _ in range(steps):
            step(timer)
        _sync()
        ms = (time.perf_counter() - t0) / steps * 1e3
    # per-kernel averages over the timed region; algorithmic FLOPs per launch:
    # each launch is one ring step over all P ranks = pairs / P
    per_launch_pairs = pairs / P
    kern = {}
    credit = {"attn_fwd": 4, "attn_bwd_dkdv": 8, "attn_bwd_dq": 2}
    for name in ("attn_fwd", "attn_bwd_dkdv", "attn_bwd_dq", "attn_bwd_delta"):
        m = timer.mean_ms(name)
        if m is None:
            continue
        n = timer.count(name) // steps
        entry = {"mean_ms": round(m, 4), "launches_per_step": n,
                 "ms_per_step": round(m * n, 3)}
        if name in credit:
            tf = credit[name] * D * H * per_launch_pairs / (m * 1e-3) / 1e12
            entry["algorithmic_tflops"] = round(tf, 1)
            entry["frac_bf16_peak"] = round(tf / BF16_PEAK_TFLOPS, 4)
        kern[name] = entry
    dom = max((n for n in credit if n in kern), key=lambda n: kern[n]["ms_per_step"])
    roof = {"kernel": dom, "bound": "mfma", "achieved": kern[dom]["algorithmic_tflops"],
            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": kern[dom]["frac_bf16_peak"], "traffic": None,
            "algorithmic_flop_per_launch": credit[dom] * D * H * per_launch_pairs}
    return {"ms": ms, "flops": flops, "kernels": kern, "roofline": roof,
            "peak_mem_gib": round(torch.cuda.max_memory_allocated() / 2**30, 2),
            "sclk_under_load": clk.summary()}


def per_rank_workload(steps, warmup):
    """One simulated GPU of configs[2] at its real grid: the blocks one rank computes, step
    by step (8 forward and 16 backward launches), without the other ranks' blocks in the
    same launch: the per-GPU compute of a real 8-GPU ring. Zigzag (ranks 0 and 7: equal
    work) and DistFlash on contiguous chunks (workers 0, 3, 4, 7: 4.5 blocks of 8192^2...
    16384^2 for workers 0-3, 3.5 for workers 4-7, schedule.distflash_work)."""
    from ringmaster_amd.ring.zigzag import KernelTimer, ring_backward, ring_forward

    P, S, H, D = 8, 131072, 16, 128
    L = S // P
    q, k, v = _gen((P, 1, H, L, D), 1), _gen((P, 1, H, L, D), 2), _gen((P, 1, H, L, D), 3)
    dout = _gen((P, 1, L, H, D), 4)
    scale = 1.0 / math.sqrt(D)
    res = {}
    for layout, ranks in (("zigzag", (0, 7)), ("distflash", (0, 3, 4, 7))):
        # the global out / lse the backward reads
        _, lse, out32 = ring_forward(q, k, v, scale, layout=layout)
        per_layout = {}
        for r in ranks:
            only = {r}

            def step(t=None):
                ring_forward(q, k, v, scale, timer=t, layout=layout, only_ranks=only)
                ring_backward(dout, q, k, v, out32, lse, scale, timer=t, layout=layout,
                              only_ranks=only)

            for _ in range(warmup):
                step()
            _sync()
            timer = KernelTimer()
            t0 = time.perf_counter()
            for _ in range(steps):
                step(timer)
            _sync()
            ms = (time.perf_counter() - t0) / steps * 1e3
            per = {}
            for name in ("attn_fwd", "attn_bwd_dkdv", "attn_bwd_dq"):
                spans = timer.events[name]
                per[name] = [round(sum(a.elapsed_time(b) for a, b in spans[i::P]) / steps, 3)
                             for i in range(P)]
            per_layout[f"rank{r}"] = {"ms_fwd_bwd": round(ms, 3),
                                      "fwd_ms_per_step": per["attn_fwd"],
                                      "dkdv_ms_per_step": per["attn_bwd_dkdv"],
                                      "dq_ms_per_step": per["attn_bwd_dq"]}
        res[layout] = per_layout
        del lse, out32
        torch.cuda.empty_cache()
    return res


def distflash_workload(steps, warmup):
    """The DistFlash (contiguous, load-balanced causal) ring at the configs[2] shape: P=8,
    S=131072 (16384 contiguous tokens per rank), H=16, D=128, bf16, fwd+bwd. Same attended
    pairs as the zigzag ring; on one GPU step d runs the blocks (i, i - d), i >= d."""
    from ringmaster_amd.ring import distflash_attention

    P, S, H, D = 8, 131072, 16, 128
    L = S // P
    q = _gen((P, 1, H, L, D), 1).requires_grad_(True)
    k = _gen((P, 1, H, L, D), 2).requires_grad_(True)
    v = _gen((P, 1, H, L, D), 3).requires_grad_(True)
    dout = _gen((P, 1, L, H, D), 4)
    flops = 14 * D * H * (S * (S + 1) // 2)

    def step():
        out = distflash_attention(q, k, v, scaling=None)
        torch.autograd.grad(out, (q, k, v), dout)

    ms = _time(step, steps, warmup)
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 3), "flops": flops, "TFLOP/s": round(tf, 1),
            "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}


def varlen_docs(total, seed=5, median=2048, sigma=1.0, lo=128, hi=16384):
    """configs[3] document lengths: clip(round(exp(ln median + sigma z)), lo, hi), z ~ N(0, 1)
    from ``seed``, drawn until they cover ``total``; the last one is cut to the remainder."""
    g = torch.Generator().manual_seed(seed)
    lens, acc = [], 0
    while acc < total:
        z = torch.randn(1, generator=g).item()
        n = int(min(max(round(math.exp(math.log(median) + sigma * z)), lo), hi))
        n = min(n, total - acc)
        lens.append(n)
        acc += n
    return lens


def varlen_workload(steps, warmup):
    """packed lognormal documents under P=4 zigzag CP, S=65536, Hq=32/Hkv=8,
    D=128, bf16, fwd+bwd (document-masked blocks)."""
    from ringmaster_amd.ring.zigzag import KernelTimer, zigzag_ring_attention

    P, S, Hq, Hkv, D = 4, 65536, 32, 8, 128
    L = S // P
    lens = varlen_docs(S)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    pairs = sum(n * (n + 1) // 2 for n in lens)
    q = _gen((P, 1, Hq, L, D), 1).requires_grad_(True)
    k = _gen((P, 1, Hkv, L, D), 2).requires_grad_(True)
    v = _gen((P, 1, Hkv, L, D), 3).requires_grad_(True)
    dout = _gen((P, 1, L, Hq, D), 4)
    cu_dev = cu.cuda()
    timer = KernelTimer()

    def step(t=None):
        out = zigzag_ring_attention(q, k, v, cu_seqlens=cu_dev, timer=t)
        torch.autograd.grad(out, (q, k, v), dout)

    for _ in range(warmup):
        step()
    _sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(timer)
    _sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    flops = 14 * D * Hq * pairs
    tf = flops / (ms * 1e-3) / 1e12
    kern = {}
    for name in ("attn_fwd", "attn_bwd_dkdv", "attn_bwd_dq"):
        m = timer.mean_ms(name)
        if m is not None:
            kern[name] = {"mean_ms": round(m, 4), "launches_per_step": timer.count(name) // steps}
    return {"ms": round(ms, 3), "docs": len(lens), "attended_pairs": pairs, "flops": flops,
            "TFLOP/s": round(tf, 1), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
            "kernels": kern}


# ---------------------------------------------------------------- HBM-bound kernels
def shard_workload(steps, warmup):
    from ringmaster_amd.shard import zigzag_shard

    P, S, H, D = 8, 131072, 16, 128
    xs = [_gen((1, S, H, D), i) for i in (1, 2, 3)]
    nbytes = 3 * 2 * xs[0].numel() * 2
    ms = _time_gpu(lambda: [zigzag_shard(x, P) for x in xs], steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del xs
    return {"ms": round(ms, 4), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def merge_workload(steps, warmup):
    from ringmaster_amd.ring.merge import update_out_and_lse

    S, H, D = 16384, 32, 128
    out = _gen((1, S, H, D), 6, torch.float32)
    lse = _gen((1, S, H, 1), 7, torch.float32)
    blk = _gen((1, S, H, D), 8)
    blk_lse = _gen((1, H, S), 9, torch.float32)
    nbytes = 677_380_096
    ms = _time_gpu(lambda: update_out_and_lse(out, lse, blk, blk_lse), steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def scan_workload(steps, warmup):
    from ringmaster_amd.strategies.state_passing import linear_scan_backward, linear_scan_forward

    L, d, G, P = 256, 64 * 64 * 128, 64, 8
    g = torch.Generator(device="cuda").manual_seed(5)
    A = -torch.exp(torch.rand(G, generator=g, device="cuda") * math.log(16.0))
    dt = torch.nn.functional.softplus(torch.randn(1, L, G, generator=g, device="cuda"))
    a = torch.exp(A * dt).contiguous()                   # per-chunk, per-head decay
    b = torch.randn(1, L, d, generator=g, device="cuda")  # chunk states
    dh = torch.randn(1, L, d, generator=g, device="cuda")
    h = linear_scan_forward(a, b, P)
    fwd_ms = _time_gpu(lambda: linear_scan_forward(a, b, P), steps, warmup)
    bwd_ms = _time_gpu(lambda: linear_scan_backward(a, h, dh, P), steps, warmup)
    fb, bb = 1_073_807_360, 1_610_612_736
    tot = fb + bb
    gbs = tot / ((fwd_ms + bwd_ms) * 1e-3) / 1e9
    return {"fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4), "bytes": tot,
            "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "fwd_GB/s": round(fb / (fwd_ms * 1e-3) / 1e9, 1),
            "bwd_GB/s": round(bb / (bwd_ms * 1e-3) / 1e9, 1)}


def scan_long_workload(steps, warmup):
    """The L-parallel (chained) cp_linear_scan on long sequences: a token-level recurrence
    over configs[2]'s 131072 tokens with 4096 channels (32 decay groups), and the long-L /
    small-d shape L=65536, d=256 (8 groups). Algorithmic bytes: fwd reads b, writes h;
    bwd reads h, dh, writes db (a, da: 1/128 of that or less)."""
    from ringmaster_amd.strategies.state_passing import linear_scan_backward, linear_scan_forward

    res = {}
    for (B, L, d, G) in ((1, 131072, 4096, 32), (1, 65536, 256, 8)):
        g = torch.Generator(device="cuda").manual_seed(5)
        a = 1.0 - 0.01 * torch.rand(B, L, G, generator=g, device="cuda")
        b = torch.randn(B, L, d, generator=g, device="cuda")
        dh = torch.randn(B, L, d, generator=g, device="cuda")
        h = linear_scan_forward(a, b, algo="chunked")
        fwd_ms = _time_gpu(lambda: linear_scan_forward(a, b, algo="chunked"), steps, warmup)
        bwd_ms = _time_gpu(lambda: linear_scan_backward(a, h, dh, algo="chunked"), steps, warmup)
        n = B * L * d * 4
        fb, bb = 2 * n + a.numel() * 4, 3 * n + 2 * a.numel() * 4
        res[f"B{B}_L{L}_d{d}_G{G}"] = {
            "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
            "fwd_GB/s": round(fb / (fwd_ms * 1e-3) / 1e9, 1),
            "bwd_GB/s": round(bb / (bwd_ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round((fb + bb) / ((fwd_ms + bwd_ms) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del a, b, dh, h
        torch.cuda.empty_cache()
    return res


def mamba_workload(steps, warmup):
    """configs[4] Mamba2 CP output correction: 8 shards of 8192 tokens stacked on the
    batch axis, nheads=64, headdim=64, d_state=128, strong decay; one launch through the C
    ABI ("ms"). "wrapper_ms" times the Python op, which also checks whether h_prev is all
    zero (the reference returns its inputs then): a reduction and a host synchronisation."""
    from ringmaster_amd import abi
    from ringmaster_amd.strategies.mamba import mamba2_cp_correction

    P, T, H, D, N = 8, 8192, 64, 64, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    out = _gen((P, T, H * D), 10)
    C = _gen((P, T, 1, N), 11)
    A = -torch.exp(torch.rand(H, generator=g, device="cuda") * math.log(16.0))
    dt = torch.nn.functional.softplus(torch.randn(P, T, H, generator=g, device="cuda"))
    cum_A = torch.cumsum(A * dt, dim=1)
    h_prev = _gen((P, H, D, N), 12, torch.float32)
    h_final = _gen((P, H, D, N), 13, torch.float32)
    y, hf_out = torch.empty_like(out), torch.empty_like(h_final)
    lib, stream = abi.lib(), abi.stream_of(out)

    def run():
        abi.check(lib.rmx_mamba2_cp_correction(
            out.data_ptr(), y.data_ptr(), h_final.data_ptr(), hf_out.data_ptr(), C.data_ptr(),
            cum_A.data_ptr(), h_prev.data_ptr(), None, P, T, H, D, 1, N, stream))

    ms = _time_gpu(run, steps, warmup)
    wrapper_ms = _time_gpu(lambda: mamba2_cp_correction(out, h_final, C, cum_A, h_prev, H, D),
                           steps, warmup)
    # read out + write y (bf16), read C, cum_A, h_prev, read + write h_final
    nbytes = 2 * out.numel() * 2 + C.numel() * 2 + cum_A.numel() * 4 + 3 * h_prev.numel() * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "wrapper_ms": round(wrapper_ms, 4)}


def chunk_state_workload(steps, warmup):
    """configs[4] Mamba2 shard final state (rmx_mamba2_chunk_state and its backward): 8
    shards of 8192 tokens, nheads=64, headdim=64, ngroups=1, d_state=128. Algorithmic
    bytes: fwd reads x, B, e, cum_A and writes the fp32 state; bwd reads x, B, e, cum_A
    and the state gradient and writes g_x, g_B (bf16), g_e, g_cum_A (fp32)."""
    from ringmaster_amd import abi

    P, T, H, D, G, N = 8, 8192, 64, 64, 1, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    x = _gen((P, T, H, D), 30)
    B = _gen((P, T, G, N), 31)
    A = -torch.exp(torch.rand(H, generator=g, device="cuda") * math.log(16.0))
    e = torch.nn.functional.softplus(torch.randn(P, T, H, generator=g, device="cuda") - 2.0)
    cum = torch.cumsum(A * e, dim=1)
    state = torch.empty((P, H, D, N), dtype=torch.float32, device="cuda")
    gst = _gen((P, H, D, N), 32, torch.float32)
    g_x, g_B = torch.empty_like(x), torch.empty_like(B)
    g_e, g_cum = torch.empty_like(e), torch.empty_like(e)
    lib, st = abi.lib(), abi.stream_of(x)

    def fwd():
        abi.check(lib.rmx_mamba2_chunk_state(x.data_ptr(), B.data_ptr(), e.data_ptr(),
                                             cum.data_ptr(), None, state.data_ptr(), P, T, H,
                                             D, G, N, st))

    ws_bytes = lib.rmx_mamba2_chunk_state_bwd_workspace(P, H, D, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") if ws_bytes else None

    def bwd():
        abi.check(lib.rmx_mamba2_chunk_state_bwd(
            x.data_ptr(), B.data_ptr(), e.data_ptr(), cum.data_ptr(), None, gst.data_ptr(),
            g_x.data_ptr(), g_B.data_ptr(), g_e.data_ptr(), g_cum.data_ptr(), P, T, H, D, G, N,
            abi.ptr(ws), ws_bytes, st))

    fwd_ms = _time_gpu(fwd, steps, warmup)
    bwd_ms = _time_gpu(bwd, steps, warmup)
    small = e.numel() * 4
    fwd_bytes = x.numel() * 2 + B.numel() * 2 + 2 * small + state.numel() * 4
    bwd_bytes = 2 * x.numel() * 2 + 2 * B.numel() * 2 + 4 * small + gst.numel() * 4
    flops = 2 * P * T * H * D * N
    out = {}
    for name, ms, nb, fl in (("fwd", fwd_ms, fwd_bytes, flops), ("bwd", bwd_ms, bwd_bytes, 2 * flops)):
        gbs = nb / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "bytes": nb, "GB/s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                     "TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 1)}
    return out


def conv_workload(steps, warmup):
    """configs[4] Mamba2 CP causal conv1d with the halo, fwd and bwd: 8 shards of 8192
    tokens, conv channels = nheads * headdim + 2 * ngroups * d_state = 4352, width 4,
    silu, bias. Algorithmic bytes: fwd reads x and writes y (bf16); bwd reads x and dy
    and writes dx (the weight / bias gradients are 4352 x 5 floats)."""
    from ringmaster_amd.strategies.mamba import causal_conv1d_cp

    P, T, C, W = 8, 8192, 64 * 64 + 2 * 128, 4
    x = _gen((P, 1, C, T), 14).requires_grad_(True)
    w = _gen((C, W), 15, scale=0.5).requires_grad_(True)
    b = _gen((C,), 16).requires_grad_(True)
    dy = _gen((P, 1, C, T), 17)
    fwd_ms = _time_gpu(lambda: causal_conv1d_cp(x, w, b, "silu"), steps, warmup)
    y = causal_conv1d_cp(x, w, b, "silu")
    tot_ms = _time_gpu(lambda: torch.autograd.grad(causal_conv1d_cp(x, w, b, "silu"), (x, w, b), dy),
                   steps, warmup)
    bwd_ms = tot_ms - fwd_ms
    n = x.numel() * 2
    fwd_bytes, bwd_bytes = 2 * n, 3 * n
    return {"fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
            "bytes": fwd_bytes + bwd_bytes,
            "GB/s": round((fwd_bytes + bwd_bytes) / (tot_ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round((fwd_bytes + bwd_bytes) / (tot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "fwd_GB/s": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9, 1),
            "bwd_GB/s": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1)}


def mamba_bwd_workload(steps, warmup):
    """configs[4] Mamba2 CP correction backward (dC, dcumA, dh_prev from dL/dy and
    dL/dh_final_out) through the C ABI with a preallocated workspace; one launch
    sequence. Algorithmic bytes: read dy, C, cum_A, h_prev, dh_final; write dC, dcumA,
    dh_prev. MFMA work executed: the dh_prev product with a two-part G e (2 x 2 T H d n) and
    P = G H_in with a three-part H_in (3 x 2 T H d n; dC and dcumA both contract it).
    "seven_pass_TFLOP/s" divides the 7 x 2 T H d n of the earlier form (S recomputed in
    three parts, dC in two) by the same time, the figure earlier runs reported."""
    from ringmaster_amd import abi

    P, T, H, D, N = 8, 8192, 64, 64, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    gy = _gen((P, T, H * D), 14)
    C = _gen((P, T, 1, N), 11)
    A = -torch.exp(torch.rand(H, generator=g, device="cuda") * math.log(16.0))
    dt = torch.nn.functional.softplus(torch.randn(P, T, H, generator=g, device="cuda"))
    cum_A = torch.cumsum(A * dt, dim=1)
    h_prev = _gen((P, H, D, N), 12, torch.float32)
    ghf = _gen((P, H, D, N), 15, torch.float32)
    gC, gA, gH = torch.empty_like(C), torch.empty_like(cum_A), torch.empty_like(h_prev)
    lib = abi.lib()
    ws_bytes = lib.rmx_mamba2_cp_correction_bwd_workspace(P, T, H, D, 1, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    stream = abi.stream_of(gy)

    def run():
        abi.check(lib.rmx_mamba2_cp_correction_bwd(
            gy.data_ptr(), ghf.data_ptr(), C.data_ptr(), cum_A.data_ptr(), h_prev.data_ptr(),
            None, gC.data_ptr(), gA.data_ptr(), gH.data_ptr(), ws.data_ptr(), ws_bytes,
            P, T, H, D, 1, N, stream))

    ms = _time_gpu(run, steps, warmup)
    nbytes = gy.numel() * 2 + 2 * C.numel() * 2 + 2 * cum_A.numel() * 4 + 3 * h_prev.numel() * 4
    unit = 2 * P * T * H * D * N
    return {"ms": round(ms, 4), "bytes": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "TFLOP/s": round(5 * unit / (ms * 1e-3) / 1e12, 1),
            "seven_pass_TFLOP/s": round(7 * unit / (ms * 1e-3) / 1e12, 1)}


def block_workload(steps, warmup, D=128):
    """one non-causal ring step, Hq=32/Hkv=8, 16384^2, D=128, fwd+bwd, merged
    into a running fp32 (out, lse) from a prior step. With D=256 the same step at head dim
    256 with half the heads (Hq=16/Hkv=4: the same FLOPs), on the head-dim-256 kernels."""
    from ringmaster_amd import abi
    from ringmaster_amd.ring import ops

    S = 16384
    Hq, Hkv = (32, 8) if D == 128 else (16, 4)
    sc = 1.0 / math.sqrt(D)
    q, k, v = _gen((1, S, Hq, D), 1, scale=sc), _gen((1, S, Hkv, D), 2, scale=sc), \
        _gen((1, S, Hkv, D), 3, scale=sc)
    dout = _gen((1, S, Hq, D), 4)
    acc = _gen((1, S, Hq, D), 6, torch.float32)
    acc_lse = _gen((1, Hq, S), 7, torch.float32)
    out = torch.empty((1, S, Hq, D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((1, Hq, S), device="cuda")
    delta = torch.empty((1, Hq, S), device="cuda")
    nlse = torch.empty((1, Hq, S), device="cuda")
    dq = torch.empty((1, S, Hq, D), device="cuda")
    dk = torch.empty((1, S, Hkv, D), device="cuda")
    dv = torch.empty_like(dk)

    def step():
        ops.attn_fwd([ops.FwdJob(q=q, k=k, v=v, mode=abi.FWD_ACC_FINAL, out=out, lse=lse,
                                 acc_out=acc, acc_lse=acc_lse)], scale=sc, mask=abi.MASK_FULL)
        # fp32 final out left in acc by ACC_FINAL
        ops.attn_bwd_delta(acc, dout, delta, Hkv, lse=lse, nlse=nlse)
        ops.attn_bwd([ops.BwdJob(q=q, k=k, v=v, dout=dout, lse=lse, delta=delta, nlse=nlse,
                                 dq_mode=abi.GRAD_WRITE_F32, dkv_mode=abi.GRAD_WRITE_F32,
                                 dq_acc=dq, dk_acc=dk, dv_acc=dv)], scale=sc, mask=abi.MASK_FULL)

    ms = _time(step, steps, warmup)
    flops = 14 * D * Hq * S * S
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 3), "flops": flops, "TFLOP/s": round(tf, 1),
            "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(heads=1):
    """Oracle (torch CPU fp32 restatement of the reference ``math`` block path) on a
    bounded sample of configs[2]: rank 0's ring-step-0 block (its 16384 queries x its
    own 16384 keys, causal) and one remote ring-step block (its late 8192 queries x a
    remote rank's 16384 keys), forward + backward, ``heads`` head(s). Those are the two
    block shapes every rank's ring is made of (1 + 7 blocks), so the per-pair rate is
    the job's rate."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import ring_math as rm

    L, D = 16384, 128
    h = L // 2
    scale = 1.0 / math.sqrt(D)
    g = torch.Generator().manual_seed(1)
    mk = lambda n: torch.randn(1, n, heads, D, generator=g)  # noqa: E731
    q, k, v, dout = mk(L), mk(L), mk(L), mk(L)
    kr, vr = mk(L), mk(L)
    t0 = time.perf_counter()
    # ring step 0: the local 2h x 2h block, bottom-right causal
    m = rm.causal_mask(L, L)
    out, lse = rm.masked_block_fwd(q, k, v, m, scale)
    rm.masked_block_bwd(dout, q, k, v, out, lse, m, scale)
    del m
    # a ring step s > r: late query half x the visiting rank's whole KV block
    out1, lse1 = rm.masked_block_fwd(q[:, h:], kr, vr, 0.0, scale)
    rm.masked_block_bwd(dout[:, h:], q[:, h:], kr, vr, out1, lse1, 0.0, scale)
    sec = time.perf_counter() - t0
    cpu_model = None
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                             None)
    except OSError:
        pass
    pairs = L * (L + 1) // 2 + h * L
    flops = 14 * D * heads * pairs
    return {"value": round(flops / sec / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle (torch CPU fp32) fwd+bwd of rank 0's ring-step-0 block (16384x16384 "
                      f"causal) and one remote step block (8192x16384), {heads} head(s), D=128: "
                      f"{pairs} pairs = 2 of the 8 blocks of one rank of configs[2] "
                      f"({sec:.1f} s; os.cpu_count()={os.cpu_count()})",
            "seconds": round(sec, 2), "cpu_model": cpu_model}


# ---------------------------------------------------------------- profiling mode
def profile_workload():
    """One warm-up and one configs[2] ring fwd+bwd step, then a 1 GiB device-to-device
    copy (3 times): the calibration kernel for the rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (bytes counted for a copy of known size give the counter's scale)."""
    from ringmaster_amd.ring.zigzag import zigzag_ring_attention

    P, S, H, D = 8, 131072, 16, 128
    L = S // P
    q = _gen((P, 1, H, L, D), 1).requires_grad_(True)
    k = _gen((P, 1, H, L, D), 2).requires_grad_(True)
    v = _gen((P, 1, H, L, D), 3).requires_grad_(True)
    dout = _gen((P, 1, L, H, D), 4)
    for i in range(2):
        out = zigzag_ring_attention(q, k, v)
        torch.autograd.grad(out, (q, k, v), dout)
        _sync()
        print(f"profile: ring step {i} done", flush=True)
    del q, k, v, dout, out
    torch.cuda.empty_cache()
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    _sync()
    print("profile: calibration copies of 1073741824 bytes done", flush=True)


def profile_hbm_workload():
    """The HBM-bound kernels at their bench shapes (shard q/k/v, the standalone merge, the
    configs[4] scan fwd/bwd, the long-L chained scans, the Mamba2 correction fwd/bwd, the CP
    conv fwd/bwd and the shard state fwd/bwd), each launched a few times, then the 1 GiB
    copy calibration: the run the rocprofv3 FETCH_SIZE / WRITE_SIZE passes count."""
    for name, fn in (("shard", shard_workload), ("merge", merge_workload),
                     ("scan", scan_workload), ("scan_long", scan_long_workload),
                     ("mamba_fwd", mamba_workload), ("mamba_bwd", mamba_bwd_workload),
                     ("conv", conv_workload), ("chunk_state", chunk_state_workload)):
        fn(2, 1)
        torch.cuda.empty_cache()
        print(f"profile-hbm: {name} done", flush=True)
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    _sync()
    print("profile-hbm: calibration copies of 1073741824 bytes done", flush=True)


def _traffic(kernel):
    """HBM bytes per launch of ``kernel`` measured by rocprofv3 (profiles/traffic.json), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    entry = data.get("kernels", {}).get(kernel)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def _attach_counters(extras):
    """Each HBM extra gets the rocprofv3-counted bytes of its call and their ratio to the
    algorithmic bytes (profiles/traffic.json "hbm_kernels"; a key "x.fwd" goes to
    extras["x"] with a "_fwd" suffix)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            calls = json.load(f)["hbm_kernels"]["calls"]
    except (OSError, ValueError, KeyError):
        return
    for key, c in calls.items():
        parts = key.split(".")
        suffix = ""
        if parts[-1] in ("fwd", "bwd"):
            suffix = "_" + parts.pop()
        node = extras
        for p in parts:
            node = node.get(p) if isinstance(node, dict) else None
        if isinstance(node, dict):
            node["counter_bytes" + suffix] = c["hbm_bytes"]
            node["counter_over_algorithmic" + suffix] = c["counter_over_algorithmic"]


def _clocks():
    try:
        out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True,
                             timeout=20).stdout
        return [ln.strip() for ln in out.splitlines() if "sclk" in ln or "mclk" in ln][:4]
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-extras", action="store_true", help="skip the HBM-bound kernels")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=1)
    ap.add_argument("--profile", action="store_true",
                    help="one ring step + copy calibration, for rocprofv3 counter passes")
    ap.add_argument("--profile-hbm", action="store_true",
                    help="the HBM-bound kernels + copy calibration, for rocprofv3 counter passes")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="time torch bf16 GEMMs (hipBLASLt) at 8192^3 and 16384^3 and exit")
    ap.add_argument("--per-rank", action="store_true",
                    help="time single simulated GPUs of configs[2] (zigzag, DistFlash) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              "and emulates the P-rank ring inside one process (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.profile:
        profile_workload()
        return
    if args.profile_hbm:
        profile_hbm_workload()
        return
    if args.gemm_ceiling:
        print(json.dumps({"gemm_ceiling": gemm_ceiling()}))
        return
    if args.per_rank:
        print(json.dumps({"per_rank_configs2": per_rank_workload(args.steps, args.warmup)}))
        return

    ring = ring_workload(args.steps, args.warmup)
    ring["roofline"]["traffic"] = _traffic(ring["roofline"]["kernel"])
    torch.cuda.empty_cache()
    extras = {}
    if not args.no_extras:
        # sub-millisecond kernels: enough warm-up and timed calls for the steady rate (the
        # first tens of calls after other work run up to 15% slower)
        extras["shard_qkv_configs2"] = shard_workload(100, 10)
        torch.cuda.empty_cache()
        extras["lse_merge_configs1"] = merge_workload(200, 20)
        torch.cuda.empty_cache()
        extras["cp_linear_scan_configs4"] = scan_workload(100, 10)
        torch.cuda.empty_cache()
        extras["cp_linear_scan_long_L"] = scan_long_workload(10, 2)
        torch.cuda.empty_cache()
        extras["mamba2_correction_configs4"] = mamba_workload(300, 30)
        torch.cuda.empty_cache()
        extras["mamba2_correction_bwd_configs4"] = mamba_bwd_workload(100, 10)
        torch.cuda.empty_cache()
        extras["mamba2_conv_cp_configs4"] = conv_workload(100, 10)
        torch.cuda.empty_cache()
        extras["mamba2_chunk_state_configs4"] = chunk_state_workload(100, 10)
        torch.cuda.empty_cache()
        extras["block_configs1"] = block_workload(3, 1)
        torch.cuda.empty_cache()
        extras["block_configs1_d256"] = block_workload(3, 1, D=256)
        torch.cuda.empty_cache()
        extras["varlen_configs3"] = varlen_workload(3, 1)
        torch.cuda.empty_cache()
        extras["distflash_configs2_shape"] = distflash_workload(2, 1)
        torch.cuda.empty_cache()
        extras["per_rank_configs2"] = per_rank_workload(3, 1)
        torch.cuda.empty_cache()
    _attach_counters(extras)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_heads)

    value = ring["flops"] / (ring["ms"] * 1e-3) / 1e12
    line = {
        "metric": "ring fwd+bwd TFLOP/s (% bf16 MFMA peak) at 16k/rank P=8 zigzag, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ring["ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 q/k/v/dout generated on device (seeds 1-4)",
        "config": {"workload": "configs[2]: simulated P=8 zigzag-causal ring fwd+bwd, S=131072 "
                               "(16384/rank as two 8192 chunks), H=16 MHA, D=128, bf16",
                   "world": 8, "seq_len": 131072, "heads": 16, "head_dim": 128,
                   "global_batch": 1, "parallelism": "emulated ring P=8 on 1 GPU"},
        "frac_bf16_peak": round(value / BF16_PEAK_TFLOPS, 4),
        "roofline": ring["roofline"],
        "cpu_baseline": cpu,
        "kernels": ring["kernels"],
        "extras": extras,
        "peak_mem_gib": ring["peak_mem_gib"],
        "sclk_under_load": ring["sclk_under_load"],
        "clocks_after_run": _clocks(),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
