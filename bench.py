#!/usr/bin/env python3
"""Benchmark of Mote's Relation hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-decode]

Headline (BASELINE.json `metric`, the config it is quoted on): the Mote-96M Relation stack,
bf16 forward + backward, B = 1, a 16384-byte window with Bernoulli(1/3.3) chunk boundaries
(seed 2, ~4965 chunks), 12 layers. One step = for every layer: RoPE/Givens prologue, fused
forward, fused backward (one pass), prologue backward. Inputs (the layer's fused projection
output and dY) are synthetic, resident in HBM before timing. FLOPs follow the reference's causal
convention: 7 * H * dh * T^2 per layer (fwd 2x, bwd 5x), projections and RoPE/Givens excluded.

Also reported: the decode step (12 layers, cache prefilled to 4096 chunks, one chunk per step,
256 steps, batch 1 and 16, HIP-graph replayed; batch 1 rotates 4 independent caches so the
Infinity Cache cannot hold them), the roofline of the dominant kernel (HIP events around that
kernel's launches) and the CPU oracle timed on the host cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import socket
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Relation fwd+bwd TFLOP/s & decode µs/step at Mote-96M shape; % of roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
D_MODEL, N_HEADS, D_HEAD, N_LAYERS = 768, 8, 96, 12   # Mote-96M main network (mote/config.py)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rmsnorm(x, eps=1e-5):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def chunk_count(seed: int, nbytes: int, batch: int = 1) -> int:
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand(batch, nbytes, generator=g) < (1.0 / 3.3)
    mask[:, 0] = True
    return int(mask.sum(-1).max())


# ------------------------------------------------------------------------------------------------
# fwd + bwd (C3)
# ------------------------------------------------------------------------------------------------
class StackInputs:
    """Per layer: the fused projection output of RMSNorm'd N(0,1) hidden states through random-init
    FullRelation weights (bf16, [B, T, 3 D]) and an N(0,1) upstream gradient dY, resident on the GPU."""

    def __init__(self, T: int, seed: int, dev, B: int = 1, d_model: int = D_MODEL, heads: int = N_HEADS,
                 layers: int = N_LAYERS):
        from mote_amd.relation import FullRelation

        torch.manual_seed(seed)
        x = rmsnorm(torch.randn(B, T, d_model))
        dh = d_model // heads
        self.layers = []
        for li in range(layers):
            m = FullRelation(d_model, heads, li)
            with torch.no_grad():
                m.theta.uniform_(-0.3, 0.3)
            w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).detach()
            qkv = (x @ w.t()).to(torch.bfloat16).to(dev)
            dy = torch.randn(B, heads, T, dh).to(torch.bfloat16).to(dev)
            self.layers.append(dict(qkv=qkv, dy=dy, theta=m.theta.detach().to(dev), lam=m.lam.detach().to(dev),
                                    inv=m.inv_freq.to(dev), parity=li % 2, heads=heads))
        self.T = T


def stack_step(inp: StackInputs, timers=None):
    """One fwd+bwd pass of the layer stack through the HIP ops; returns the last layer's Y and
    d(qkv), d(theta) (for the graph-replay check)."""
    ops = torch.ops.mote
    out = None
    for L in inp.layers:
        p1, p2, info = ops.rope_givens(L["qkv"], L["inv"], L["theta"], L["heads"], L["parity"], 0)
        if timers is not None:
            timers["fwd"][0].append(torch.cuda.Event(enable_timing=True))
            timers["fwd"][0][-1].record()
        y, g, ibar, lse = ops.relation_fwd(p1, p2, info, L["lam"], 2.0, 0)
        if timers is not None:
            timers["fwd"][1].append(torch.cuda.Event(enable_timing=True))
            timers["fwd"][1][-1].record()
            dp = staged_bwd(p1, p2, info, ibar, lse, g, L["dy"], timers)
        else:
            dp = ops.relation_bwd(p1, p2, info, ibar, lse, g, L["dy"], 2.0, 0)
        dqkv, dth = ops.rope_givens_bwd(dp[0], dp[1], dp[2], L["qkv"], L["inv"], L["theta"], L["heads"], L["parity"], 0)
        out = (y, dqkv, dth, dp[3])
    return out


def capture_stack(inp: StackInputs):
    """The whole stack step as one HIP graph (torch.cuda.CUDAGraph): every launch of every layer
    replays without the per-op Python dispatch. Returns (graph, the graph's output tensors)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack_step(inp)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(gr, stream=side):
            outs = stack_step(inp)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return gr, outs


def check_replays(gr, outs, ref, n: int = 3):
    """Replays `gr` n times with eager work and synchronisations between the replays; every replay
    must reproduce the eager outputs bit for bit (the kernels are deterministic)."""
    for r in range(n):
        for t in outs:
            t.fill_(float("nan")) if t.is_floating_point() else t.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            if not torch.equal(a, b):
                raise RuntimeError(f"graph replay {r} differs from the eager step")


def bwd_stage_args(p1, p2, info, ibar, lse, g, dy):
    """The backward's argument block with its outputs and workspace allocated, for a caller that
    issues the stages (rows, keys, queries, finish) one launch at a time; returns (args, keep-alive)."""
    from mote_amd import _lib as Lb
    from mote_amd.flash_relation import _token_major

    B, H, TQ, D = p1.shape
    dp1 = _token_major(B, H, TQ, D, p1, p1.dtype)
    dp2 = _token_major(B, H, TQ, D, p1, p1.dtype)
    dinfo = _token_major(B, H, TQ, D, p1, p1.dtype)
    dlam = torch.empty((), device=p1.device, dtype=torch.float32)
    a = Lb.BwdArgs()
    a.dtype, a.B, a.H, a.TQ, a.TK, a.D, a.q_start = Lb.dtype_code(p1), B, H, TQ, TQ, D, 0
    a.tau_s, a.deterministic = 2.0, 0
    a.p1, a.p2, a.info, a.dy = Lb.view(p1), Lb.view(p2), Lb.view(info), Lb.view(dy)
    a.ibar, a.lse, a.g = ibar.data_ptr(), lse.data_ptr(), g.data_ptr()
    a.dp1, a.dp2, a.dinfo, a.dlam = Lb.view(dp1), Lb.view(dp2), Lb.view(dinfo), dlam.data_ptr()
    ws = torch.empty(int(Lb.lib().mote_relation_bwd_workspace(a)), device=p1.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    return a, (dp1, dp2, dinfo, dlam, ws)


def run_stage(a, stage: int, stream) -> None:
    from mote_amd import _lib as Lb

    a.stages = stage
    Lb.check(Lb.lib().mote_relation_bwd(a, stream), f"bwd stage {stage}")


def staged_bwd(p1, p2, info, ibar, lse, g, dy, timers):
    """The one-pass backward issued stage by stage through the ABI's `stages` field, with events
    around the key + query work: rows; keys and queries in one call (the fused launch, after the
    small clear of its control words that a call without the rows stage adds); finish. Then the same
    backward again in the two-launch form (keys, then queries, each bracketed), for comparison."""
    from mote_amd import _lib as Lb

    a, (dp1, dp2, dinfo, dlam, ws) = bwd_stage_args(p1, p2, info, ibar, lse, g, dy)
    st = Lb.stream_of(p1)

    def stage(bits, what):
        a.stages = bits
        Lb.check(Lb.lib().mote_relation_bwd(a, st), what)

    def timed(key, bits, what):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        stage(bits, what)
        e1.record()
        timers[key][0].append(e0)
        timers[key][1].append(e1)

    stage(Lb.MOTE_BWD_ROWS, "bwd rows")
    timed("bwd_kq", Lb.MOTE_BWD_KEYS | Lb.MOTE_BWD_QUERIES, "bwd keys + queries")
    stage(Lb.MOTE_BWD_FINISH, "bwd finish")
    stage(Lb.MOTE_BWD_ROWS, "bwd rows")
    timed("bwd_keys", Lb.MOTE_BWD_KEYS, "bwd keys")
    timed("bwd_queries", Lb.MOTE_BWD_QUERIES, "bwd queries")
    stage(Lb.MOTE_BWD_FINISH, "bwd finish")
    return dp1, dp2, dinfo, dlam


def bench_stack(steps: int, warmup: int, dev):
    T = chunk_count(2, 16384)
    log(f"[bench] Mote-96M stack: T = {T} chunks, {N_LAYERS} layers, bf16 fwd+bwd")
    inp = StackInputs(T, 2, dev)
    for _ in range(warmup):
        stack_step(inp)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    t0.record()
    for _ in range(steps):
        stack_step(inp)
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = t0.elapsed_time(t1) / steps
    flops = N_LAYERS * 7.0 * N_HEADS * D_HEAD * T * T
    # kernel-level timing pass (same work, stages bracketed by events)
    timers = {"fwd": ([], []), "bwd_kq": ([], []), "bwd_keys": ([], []), "bwd_queries": ([], [])}
    for _ in range(max(1, min(steps, 3))):
        stack_step(inp, timers)
    torch.cuda.synchronize()
    clock = stack_clock(inp, ms)
    avg = {k: sum(a.elapsed_time(b) for a, b in zip(*v)) / len(v[0]) for k, v in timers.items()}
    # per-kernel work (units of H*dh*T^2, one per causal product): forward U and P I~ (2); the fused
    # key + query launch U, dW, dV, dK and dQ (5); in the two-launch form the key kernel's 4 and the
    # query kernel's dQ (1), which reads the key kernel's dU^T tiles and is HBM-bound
    unit = N_HEADS * D_HEAD * T * T
    dq_bytes = dq_kernel_bytes(T)
    res = dict(T=T, ms_per_step=ms, wall_s=wall, tflops=flops / (ms * 1e-3) / 1e12, flops_per_step=flops,
               kq_ms=avg["bwd_kq"], kq_tflops=5.0 * unit / (avg["bwd_kq"] * 1e-3) / 1e12,
               keys_ms=avg["bwd_keys"], queries_ms=avg["bwd_queries"], fwd_ms=avg["fwd"],
               keys_tflops=4.0 * unit / (avg["bwd_keys"] * 1e-3) / 1e12,
               queries_tflops=1.0 * unit / (avg["bwd_queries"] * 1e-3) / 1e12,
               queries_bytes=dq_bytes, queries_gbs=dq_bytes / (avg["bwd_queries"] * 1e-3) / 1e9,
               fwd_tflops=2.0 * unit / (avg["fwd"] * 1e-3) / 1e12, clock=clock, dut=dut_residency(inp))
    log(f"[bench] stack: {ms:.3f} ms/step = {res['tflops']:.1f} TFLOP/s; fwd kernel {avg['fwd']*1e3:.1f} us "
        f"({res['fwd_tflops']:.1f} TF/s), bwd key + query launch {avg['bwd_kq']*1e3:.1f} us ({res['kq_tflops']:.1f} TF/s); "
        f"two-launch form: key kernel {avg['bwd_keys']*1e3:.1f} us ({res['keys_tflops']:.1f} TF/s), "
        f"dQ kernel {avg['bwd_queries']*1e3:.1f} us ({res['queries_gbs']:.0f} GB/s of dU^T tiles + P2 + dP1); "
        f"shader clock during a step {clock['sclk_mhz']} MHz {clock['sclk_mhz_runs']}; dQ kernel {res['dut']['dq_us_hot']} us right after the key kernel, "
        f"{res['dut']['dq_us_after_sweep']} us after a {res['dut']['sweep_MiB']} MiB sweep")
    return res


def gpu_identity(dev) -> dict:
    """Which GPU and host the line was measured on."""
    p = torch.cuda.get_device_properties(dev)
    ident = {"name": p.name, "arch": getattr(p, "gcnArchName", ""), "cus": p.multi_processor_count,
             "host": socket.gethostname()}
    for k in ("uuid", "pci_bus_id", "pci_device_id", "pci_domain_id"):
        v = getattr(p, k, None)
        if v is not None:
            ident[k] = str(v)
    return ident


class ClockProbe:
    """mote_clock_probe launches on the current stream: each workgroup counts shader-clock ticks
    (s_memtime) against the constant 100 MHz clock (s_memrealtime) over a short loop, so the shader
    clock at that moment is 100 MHz x the ratio, with no host timing involved."""

    def __init__(self, dev, max_workgroups: int = 256):
        self.out = torch.zeros(3 * max_workgroups, dtype=torch.int64, device=dev)
        self.max_workgroups = max_workgroups
        self.samples = []  # (workgroups, snapshot of out) per launch

    def launch(self, workgroups: int = 8, iters: int = 512, keep: bool = True) -> None:
        from mote_amd import _lib as Lb

        assert workgroups <= self.max_workgroups
        Lb.check(Lb.lib().mote_clock_probe(self.out.data_ptr(), workgroups, iters, Lb.stream_of(self.out)),
                 "mote_clock_probe")
        if keep:
            self.samples.append(self.out[: 3 * workgroups].clone())

    def mhz(self) -> list:
        """Shader clock of every kept launch (the mean over its workgroups)."""
        out = []
        for o in self.samples:
            o = o.view(-1, 3).double().cpu()
            out.append(float((100.0 * o[:, 0] / o[:, 1].clamp(min=1)).mean()))
        return out


def stack_clock(inp: "StackInputs", step_ms: float, reps: int = 3) -> dict:
    """The shader clock the stack's kernels run at: while a stack step runs on the current stream, 8
    probe workgroups on a second stream (one per XCD, a few wave slots of the chip) count shader-clock
    ticks against the 100 MHz clock over a loop sized to end inside the step. The clock reacts to the
    load within microseconds, so a probe run between kernels or alone reads a different clock than
    the kernels see; this pass runs after the timed steps and its step time is not reported."""
    dev = inp.layers[0]["qkv"].device
    probe = ClockProbe(dev, 8)
    side = torch.cuda.Stream()
    iters = 1000
    res = []
    for r in range(reps + 1):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            probe.launch(8, iters)
        stack_step(inp)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        o = probe.samples[-1].view(-1, 3).double().cpu()
        span_ms = float(o[:, 1].max()) / 1e5
        if r == 0:  # size the loop to about 70 % of a step from the first probe's pace
            iters = max(1000, int(iters * 0.7 * step_ms / max(span_ms, 1e-3)))
            continue
        res.append((float((100.0 * o[:, 0] / o[:, 1].clamp(min=1)).mean()), span_ms))
    mhz = [m for m, _ in res]
    return {"sclk_mhz": round(sum(mhz) / len(mhz), 1), "sclk_mhz_runs": [round(m, 1) for m in mhz],
            "probe_span_ms": [round(t, 3) for _, t in res], "step_ms": round(step_ms, 3),
            "method": "8 workgroups of mote_clock_probe on a second stream beside a stack step: s_memtime "
                      "ticks over s_memrealtime (100 MHz) ticks", **shader_clock_check(dev)}


def shader_clock_check(dev) -> dict:
    """The probe's constant counter against HIP event time over a longer launch: both must advance
    at 100 MHz for the probe's clock figures to mean what they say."""
    pr = ClockProbe(dev)
    pr.launch(256, 20000, keep=False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    pr.launch(256, 20000)
    e1.record()
    torch.cuda.synchronize()
    o = pr.samples[0].view(-1, 3).double().cpu()
    real_ms = float(o[:, 1].max()) / 1e5
    return {"probe_event_ms": round(e0.elapsed_time(e1), 3), "probe_realtime_ms": round(real_ms, 3),
            "sclk_mhz_probe_alone": round(pr.mhz()[0], 1)}


def dut_residency(inp: "StackInputs", reps: int = 5, sweep_mib: int = 1024) -> dict:
    """Where the dQ kernel finds the dU^T tiles the key kernel wrote just before it: the dQ launch
    timed right after the key kernel (tiles possibly still in the 256 MB Infinity Cache) and after a
    read of `sweep_mib` MiB in between (which leaves none of them there). Both issue the same launch
    on the same data; the difference is what the round trip through HBM costs."""
    from mote_amd import _lib as Lb

    ops = torch.ops.mote
    L = inp.layers[0]
    p1, p2, info = ops.rope_givens(L["qkv"], L["inv"], L["theta"], L["heads"], L["parity"], 0)
    y, g, ibar, lse = ops.relation_fwd(p1, p2, info, L["lam"], 2.0, 0)
    a, keep = bwd_stage_args(p1, p2, info, ibar, lse, g, L["dy"])
    st = Lb.stream_of(p1)
    sweep = torch.ones(sweep_mib << 18, dtype=torch.float32, device=p1.device)
    times = {"hot": [], "after_sweep": []}
    for r in range(2 * reps + 2):
        kind = "hot" if r % 2 == 0 else "after_sweep"
        run_stage(a, Lb.MOTE_BWD_ROWS, st)
        run_stage(a, Lb.MOTE_BWD_KEYS, st)
        if kind == "after_sweep":
            sweep.sum()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run_stage(a, Lb.MOTE_BWD_QUERIES, st)
        e1.record()
        torch.cuda.synchronize()
        if r >= 2:
            times[kind].append(e0.elapsed_time(e1) * 1e3)
    hot, cold = (sum(v) / len(v) for v in (times["hot"], times["after_sweep"]))
    tile_bytes = N_HEADS * pair_total(inp.T) * 8192
    del sweep, keep
    return {"dq_us_hot": round(hot, 2), "dq_us_after_sweep": round(cold, 2), "sweep_MiB": sweep_mib,
            "dut_tile_bytes": tile_bytes, "reps": reps,
            "note": "dQ launch right after the key kernel vs after a read of sweep_MiB in between"}


def pair_total(TQ: int, q_start: int = 0) -> int:
    """Visible (query block, key block) pairs of 64 x 64 per head (the backward's dU^T tile count)."""
    if TQ <= 0:
        return 0
    nqb = (TQ + 63) // 64
    A = (q_start + 126) // 64
    last = nqb - 1
    qlast = min(TQ, 64 * last + 64) - 1
    return last * (last - 1) // 2 + A * last + (q_start + qlast + 63) // 64


def dq_kernel_bytes(T: int) -> float:
    """Algorithmic HBM bytes of one dQ-kernel launch at the stack shape: the dU^T tiles (8 KB per
    visible 64 x 64 pair and head, written by the key kernel), P2 read once and dP1 written once."""
    return N_HEADS * (pair_total(T) * 8192 + 2 * T * D_HEAD * 2)


def copy_calibration(dev, mib: int = 1024):
    """One plain device-to-device copy of `mib` MiB (reads and writes that many bytes), run once
    outside every timed region, so that an HBM counter pass over this program (rocprofv3 --pmc
    FETCH_SIZE, then WRITE_SIZE) holds a dispatch of known traffic to scale the counters by."""
    a = torch.ones(mib << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


# The device sources each recorded kernel figure depends on: a figure read from profiles/ counts only
# while these files are unchanged since it was measured (their fingerprint is recorded beside it).
_COMMON = ("common.hpp", "params.hpp")
KERNEL_SOURCES = {
    "bwd_kvq_kernel": ("relation_bwd_tiles.hip", "tiles.hpp", "bwd.hpp") + _COMMON,
    "bwd_kv_kernel": ("relation_bwd_tiles.hip", "tiles.hpp", "bwd.hpp") + _COMMON,
    "bwd_dq_kernel": ("relation_bwd_tiles.hip", "tiles.hpp", "bwd.hpp") + _COMMON,
    "relation_fwd_tile_kernel": ("relation_fwd.hip", "tiles.hpp") + _COMMON,
    "bwd_rows_kernel": ("relation_bwd.hip", "bwd.hpp") + _COMMON,
    "rope_givens_fwd_stream_kernel": ("rope_givens.hip",) + _COMMON,
    "rope_givens_bwd_stream_kernel": ("rope_givens.hip",) + _COMMON,
    "relation_decode_kernel": ("relation_decode.hip",) + _COMMON,
    "qkv_rope_kernel": ("qkv_rope.hip", "tiles.hpp") + _COMMON,
}


def _code_only(text: str) -> str:
    """C++ source without its comments and blank space at line ends (string literals kept whole), so
    that an edit of comments alone leaves a kernel's fingerprint unchanged."""
    out, i, n = [], 0, len(text)
    while i < n:
        c = text[i]
        if c == '"':  # string literal, escapes included
            j = i + 1
            while j < n and text[j] != '"':
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        elif text.startswith("//", i):
            j = text.find("\n", i)
            i = n if j < 0 else j
        elif text.startswith("/*", i):
            j = text.find("*/", i + 2)
            i = n if j < 0 else j + 2
        else:
            out.append(c)
            i += 1
    lines = [ln.rstrip() for ln in "".join(out).split("\n")]
    return "\n".join(ln for ln in lines if ln)


def source_fingerprint(kernel: str) -> str:
    """12 hex digits of sha256 over the code of the kernel's device sources, comments excluded
    (decode figures share one entry)."""
    import hashlib

    base = kernel.split("@")[0]
    base = "relation_decode_kernel" if base.startswith("relation_decode_kernel") else base
    h = hashlib.sha256()
    for f in KERNEL_SOURCES[base]:
        with open(os.path.join(ROOT, "mote_amd", "csrc", f), encoding="utf-8") as fh:
            h.update(_code_only(fh.read()).encode())
    return h.hexdigest()[:12]


def _recorded(fname: str, kernel: str):
    """(fields after the kernel name, whether they were measured on the current sources) from a
    profiles/ file of lines "<kernel> <fields...> src=<fingerprint>", or (None, None)."""
    path = os.path.join(ROOT, "profiles", fname)
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and parts[0] == kernel and parts[-1].startswith("src="):
                    return parts[1:-1], parts[-1][4:] == source_fingerprint(kernel)
    except OSError:
        pass
    return None, None


TRAFFIC_KIND = ("bytes between L2 and the memory fabric per launch (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known "
                "size); Infinity Cache hits are included, so this is an upper bound on the bytes that reach HBM")


def measured_traffic(kernel: str):
    """Bytes per launch of `kernel` between L2 and the memory fabric at this workload, from the two
    counter passes recorded in profiles/hbm_traffic.txt, with where it came from; the bytes are null
    when the kernel's sources changed after the measurement (the record is then stale, not this
    build's). The counters see requests leaving L2, hits in the Infinity Cache included."""
    fields, current = _recorded("hbm_traffic.txt", kernel)
    if fields is None:
        return None, {"recorded": None}
    note = {"recorded": "profiles/hbm_traffic.txt", "sources_match": bool(current), "kind": TRAFFIC_KIND}
    return (int(float(fields[0])) if current else None), note


def _traffic(kernel: str) -> dict:
    b, note = measured_traffic(kernel)
    return {"traffic": b, "traffic_source": note}


def measured_counters(kernel: str):
    """MFMA busy, VALU busy and MFMA/VALU co-execution (fractions) of `kernel` from the counter
    passes recorded in profiles/kernel_counters.txt; null when the sources changed since."""
    fields, current = _recorded("kernel_counters.txt", kernel)
    if fields is None:
        return {"recorded": None}
    out = {"recorded": "profiles/kernel_counters.txt", "sources_match": bool(current)}
    for f in fields:
        k, _, v = f.partition("=")
        out[k] = float(v) if current else None
    return out


def summarize_counters(base: str) -> None:
    """Print profiles/ lines from rocprofv3 counter-collection CSVs under `base`: <cfg>_A / <cfg>_B
    (SQ counter passes of `--kernels-only <cfg>`) -> kernel_counters.txt lines; fetch / write
    (FETCH_SIZE / WRITE_SIZE passes over the default workload) -> hbm_traffic.txt lines. Each line
    ends with the fingerprint of the sources it was measured on."""
    import csv
    import glob
    import re

    def load(d):
        per, name = {}, {}
        for f in glob.glob(os.path.join(base, d, "*counter_collection.csv")):
            for r in csv.DictReader(open(f)):
                k = int(r["Dispatch_Id"])
                per.setdefault(k, {})[r["Counter_Name"]] = float(r["Counter_Value"])
                name[k] = re.sub(r"^void |mote::|\(.*$", "", r["Kernel_Name"]).split("<")[0]
        return per, name

    known = tuple(KERNEL_SOURCES)
    for cfg in ("c3", "c2", "c5"):
        agg = {}
        for pas in ("A", "B"):
            per, name = load(f"{cfg}_{pas}")
            for k, cs in per.items():
                if name[k] not in known:
                    continue
                for c, v in cs.items():
                    agg.setdefault(name[k], {}).setdefault(c, []).append(v)
        for kern, cs in sorted(agg.items()):
            av = {c: sum(v) / len(v) for c, v in cs.items()}
            cyc = av.get("SQ_BUSY_CYCLES", 0.0) / 32.0  # summed over the 32 shader engines
            if not cyc or "SQ_VALU_MFMA_BUSY_CYCLES" not in av:
                continue
            mfma = av["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * 1024)          # per SIMD
            valu = av.get("SQ_ACTIVE_INST_VALU", 0.0) / (cyc * 256)       # quad-cycles per CU
            coex = av.get("SQ_VALU_MFMA_COEXEC_CYCLES", 0.0) / max(av["SQ_VALU_MFMA_BUSY_CYCLES"], 1.0)
            print(f"{kern}@{cfg} mfma_busy={mfma:.4f} valu_busy={valu:.4f} mfma_valu_coexec={coex:.4f} "
                  f"src={source_fingerprint(kern)}")
    fetch, fname = load("fetch")
    write, _ = load("write")
    cal = [k for k, n in fname.items() if "copyBuffer" in n]
    if fetch and cal:
        big = max(cal, key=lambda k: fetch[k].get("FETCH_SIZE", 0))
        sf = 1048576.0 / fetch[big]["FETCH_SIZE"]
        sw = 1048576.0 / write[big]["WRITE_SIZE"] if big in write else 1.0
        tot = {}
        for k, cs in fetch.items():
            if fname[k] in known and k in write:
                b = (cs["FETCH_SIZE"] * sf + write[k]["WRITE_SIZE"] * sw) * 1024
                tot.setdefault(fname[k], []).append(b)
        for kern, v in sorted(tot.items()):
            groups = {kern: v}
            if kern == "relation_decode_kernel":  # batch 1 (~14 MB per launch) and batch 16 (~200 MB)
                groups = {kern + "_b1": [b for b in v if b < 5e7], kern + "_b16": [b for b in v if b >= 5e7]}
            for kn, vv in groups.items():
                if vv:
                    print(f"{kn} {sum(vv) / len(vv):.0f} src={source_fingerprint(kn)}   "
                          f"# scale FETCH x{sf:.3f}, WRITE x{sw:.3f}")


# ------------------------------------------------------------------------------------------------
# decode (C4)
# ------------------------------------------------------------------------------------------------
def bench_decode(batch: int, steps: int, dev, copies: int):
    from mote_amd.arena import RelationArena
    from mote_amd.decode import decode_workspace, relation_decode
    from mote_amd.relation import FullRelation, rope_givens

    S0 = 4096
    cap = S0 + steps + 256
    torch.manual_seed(3)
    mods = []
    for li in range(N_LAYERS):
        m = FullRelation(D_MODEL, N_HEADS, li)
        with torch.no_grad():
            m.theta.uniform_(-0.3, 0.3)
        mods.append(m)
    arenas, Ss = [], []
    for c in range(copies):
        ar = RelationArena(N_LAYERS, N_HEADS, cap, D_HEAD, dev, torch.bfloat16, batch=batch)
        for li, m in enumerate(mods):
            w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).detach().to(dev, torch.bfloat16)
            for b0 in range(batch):
                x = rmsnorm(torch.randn(1, S0, D_MODEL, device=dev)).to(torch.bfloat16)
                qkv = x @ w.t()
                _, p2, info = rope_givens(qkv, N_HEADS, m.inv_freq.to(dev), m.theta.detach().to(dev), li, 0)
                ar.p2(li)[b0, :, :S0] = p2[0]
                ar.info(li)[b0, :, :S0] = info[0]
        arenas.append(ar)
        Ss.append(torch.full((batch,), S0, device=dev, dtype=torch.int64))
    lam = [m.lam.detach().float().to(dev) for m in mods]
    theta = [m.theta.detach().float().to(dev) for m in mods]
    inv = [m.inv_freq.to(dev) for m in mods]
    ins = [torch.randn(batch, 3, N_HEADS, D_HEAD, device=dev).to(torch.bfloat16) for _ in range(N_LAYERS)]
    ws = [decode_workspace(batch, N_HEADS, D_HEAD, cap, dev) for _ in range(copies)]
    ys = [torch.empty(batch, N_HEADS, D_HEAD, device=dev, dtype=torch.bfloat16) for _ in range(N_LAYERS)]
    gs = [torch.empty(batch, N_HEADS, device=dev) for _ in range(N_LAYERS)]

    def step(c):
        for li in range(N_LAYERS):
            q = ins[li]
            relation_decode(q[:, 0], q[:, 1], q[:, 2], Ss[c], arenas[c].p2(li), arenas[c].info(li), lam[li], 2.0,
                            inv[li], theta[li], li, advance=(li == N_LAYERS - 1), workspace=ws[c], y=ys[li], g=gs[li])

    # eager per-launch timing of the decode kernel (for the roofline), then restore S
    ev = []
    for c in range(copies):
        for li in range(N_LAYERS):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            q = ins[li]
            relation_decode(q[:, 0], q[:, 1], q[:, 2], Ss[c], arenas[c].p2(li), arenas[c].info(li), lam[li], 2.0,
                            inv[li], theta[li], li, advance=False, workspace=ws[c], y=ys[li], g=gs[li])
            e1.record()
            ev.append((e0, e1))
    torch.cuda.synchronize()
    kern_ms = sum(a.elapsed_time(b) for a, b in ev[copies:]) / max(1, len(ev) - copies)
    # graphs: one per cache copy
    graphs = []
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in range(copies):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=side):
                step(c)
            graphs.append(gr)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for c in range(copies):  # capture does not run the kernels; positions are still S0
        assert int(Ss[c][0]) == S0
    for i in range(3 * copies):  # warm-up replays
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    s_begin = [int(s[0]) for s in Ss]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        graphs[i % copies].replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / steps
    # algorithmic bytes: rows [0, S] of P2 and I~ per layer and sequence
    rows = 0
    for i in range(steps):
        c = i % copies
        s = s_begin[c] + i // copies
        rows += (s + 1)
    bytes_per_step = rows / steps * 2 * N_HEADS * D_HEAD * 2 * N_LAYERS * batch
    s_avg = rows / steps - 1
    kern_bytes = (S0 + 1) * 2 * N_HEADS * D_HEAD * 2 * batch  # the eager launches ran at S = S0
    # one launch inside the replayed graph: the step's time over its 12 launches (gaps included)
    launch_us = us / N_LAYERS
    floor_us = launch_floor(dev, N_LAYERS, 256, steps)
    res = dict(batch=batch, us_per_step=us, gbs=bytes_per_step / (us * 1e-6) / 1e9, bytes_per_step=bytes_per_step,
               avg_S=s_avg, kernel_us=launch_us, kernel_gbs=bytes_per_step / N_LAYERS / (launch_us * 1e-6) / 1e9,
               eager_us=kern_ms * 1e3, eager_gbs=kern_bytes / (kern_ms * 1e-3) / 1e9, copies=copies,
               launch_floor_us=floor_us)
    log(f"[bench] decode b{batch}: {us:.1f} us/step ({res['gbs']:.0f} GB/s over the step), "
        f"{launch_us:.2f} us per launch in the graph (launch floor {floor_us:.2f} us), "
        f"one eager launch {res['eager_us']:.1f} us")
    return res


def launch_floor(dev, launches: int, workgroups: int, replays: int) -> float:
    """The per-launch cost of a chain of `launches` dependent near-empty launches of `workgroups`
    workgroups (mote_clock_probe with one loop step: the decode kernel's grid, no memory traffic)
    captured in one HIP graph and replayed like the decode step: the floor under a decode launch."""
    probe = ClockProbe(dev, workgroups)

    def chain():
        for _ in range(launches):
            probe.launch(workgroups, 1, keep=False)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=side):
            chain()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for _ in range(8):
        gr.replay()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / replays / launches


# ------------------------------------------------------------------------------------------------
# C2 (Mote-32M stack) and C5 (Mote-138M ragged prefill): reported beside the headline
# ------------------------------------------------------------------------------------------------
def bench_decode_engine(batch: int, steps: int, dev):
    """The decode engine's per-token Relation work for the 12-layer Mote-96M stack: per layer the
    fused projection (hipBLASLt), the decode kernel (RoPE / Givens, append at the device position S,
    the sweep over rows [0, S]) and `wo` (graph.py:151-187 through mote_amd.decode.RelationDecodeStep),
    layer outputs chained into the next layer's input, the whole token captured as one HIP graph
    that advances S itself. Caches prefilled to 4096 rows as in bench_decode; `steps` tokens timed."""
    from mote_amd.arena import RelationArena
    from mote_amd.decode import RelationDecodeStep
    from mote_amd.relation import FullRelation, rope_givens

    S0 = 4096
    cap = S0 + steps + 256
    torch.manual_seed(7)
    arena = RelationArena(N_LAYERS, N_HEADS, cap, D_HEAD, dev, torch.bfloat16, batch=batch)
    mods, dsteps = [], []
    for li in range(N_LAYERS):
        m = FullRelation(D_MODEL, N_HEADS, li)
        with torch.no_grad():
            m.theta.uniform_(-0.3, 0.3)
        m = m.to(dev)
        with torch.no_grad():
            w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).to(torch.bfloat16)
            for b0 in range(batch):
                x = rmsnorm(torch.randn(1, S0, D_MODEL, device=dev)).to(torch.bfloat16)
                _, p2, info = rope_givens(x @ w.t(), N_HEADS, m.inv_freq, m.theta, li, 0)
                arena.p2(li)[b0, :, :S0] = p2[0]
                arena.info(li)[b0, :, :S0] = info[0]
        for lin in (m.w1, m.w2, m.wi, m.wo):
            lin.to(torch.bfloat16)  # bf16 weights; lam, theta and the RoPE frequencies stay fp32
        mods.append(m)
        dsteps.append(RelationDecodeStep(m, arena, li))
    S = torch.full((batch,), S0, device=dev, dtype=torch.int64)
    x0 = torch.randn(batch, 1, D_MODEL, device=dev).to(torch.bfloat16)

    def token():
        x = x0
        for li, st in enumerate(dsteps):
            x, _ = st(x, S, advance=(li == N_LAYERS - 1))
        return x

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        token()  # warm-up on the capture stream (S advances once)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(gr, stream=side):
            token()
    torch.cuda.current_stream().wait_stream(side)
    S.fill_(S0)
    torch.cuda.synchronize()
    for _ in range(3):
        gr.replay()
    S.fill_(S0)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / steps
    if int(S[0]) != S0 + steps:
        raise RuntimeError(f"decode engine: S = {int(S[0])} after {steps} tokens from {S0}")
    log(f"[bench] decode engine b{batch}: {us:.1f} us per token for the 12 Relation layers (projections, decode, wo)")
    del gr
    return dict(workload=f"Mote-96M Relation decode step with projections and wo, 12 layers chained, batch {batch}, "
                         f"cache 4096 -> {S0 + steps} rows, one HIP graph per token", batch=batch,
                us_per_token=round(us, 2), tokens=steps)


def bench_c2(steps: int, warmup: int, dev):
    """Mote-32M Relation stack (d_model 512, 8 heads, dh 64, 8 layers), bf16 fwd+bwd, B = 4, a
    2048-byte window with Bernoulli(1/3.3) chunk boundaries (seed 1): every sequence padded to the
    longest (T = max M_b); FLOPs count the real rows only, 7 H dh sum_b M_b^2 per layer."""
    g = torch.Generator().manual_seed(1)
    mask = torch.rand(4, 2048, generator=g) < (1.0 / 3.3)
    mask[:, 0] = True
    M = mask.sum(-1).tolist()
    T = max(M)
    inp = StackInputs(T, 1, dev, B=4, d_model=512, heads=8, layers=8)
    for _ in range(warmup):
        stack_step(inp)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        stack_step(inp)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    flops = 8 * 7.0 * 8 * 64 * sum(m * m for m in M)
    # the same step as one HIP graph: at T ~ 650 the eager step is bound by per-op dispatch
    ref = [t.clone() for t in stack_step(inp)]
    torch.cuda.synchronize()
    gr, outs = capture_stack(inp)
    check_replays(gr, outs, ref)
    for _ in range(warmup):
        gr.replay()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(steps):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_g = t0.elapsed_time(t1) / steps
    del gr, outs
    log(f"[bench] C2 Mote-32M stack: chunks {M} (T = {T}), eager {ms:.3f} ms/step = {flops / ms / 1e9:.1f} TFLOP/s, "
        f"HIP graph {ms_g:.3f} ms/step = {flops / ms_g / 1e9:.1f} TFLOP/s")
    return dict(workload="Mote-32M Relation stack fwd+bwd (8 layers, B=4, 2048-byte window, seed 1)", chunks=M,
                T_padded=T, ms_per_step=round(ms, 4), tflops=round(flops / (ms * 1e-3) / 1e12, 2),
                flop_per_step=flops, frac_bf16_peak=round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                graph=dict(ms_per_step=round(ms_g, 4), tflops=round(flops / (ms_g * 1e-3) / 1e12, 2),
                           frac_bf16_peak=round(flops / (ms_g * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                           replays_checked=3))


def bench_c5(steps: int, warmup: int, dev):
    """Mote-138M Relation prefill (d_model 768, 8 heads, dh 96, 18 layers), bf16 forward over a
    ragged packed batch: 8 sequences of U[1000, 5000] chunks (seed 4) in cu_seqlens layout. Per layer
    the varlen core (mote::relation_fwd_varlen) on resident P1 / P2 / I~ ([H, total, dh] views of
    [total, H, dh] memory from RMSNorm'd N(0,1) hidden states through random-init projections, RoPE
    restarting at 0 for every sequence, Givens). FLOPs: 2 H dh sum_i T_i^2 per layer."""
    from mote_amd.relation import FullRelation, rope_givens

    lens = torch.randint(1000, 5001, (8,), generator=torch.Generator().manual_seed(4)).tolist()
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    total = int(cu[-1])
    torch.manual_seed(4)
    x = rmsnorm(torch.randn(total, D_MODEL))
    layers = []
    for li in range(18):
        m = FullRelation(D_MODEL, N_HEADS, li)
        with torch.no_grad():
            m.theta.uniform_(-0.3, 0.3)
        w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).detach()
        qkv = (x @ w.t()).to(torch.bfloat16).to(dev)
        bufs = [torch.empty(total, N_HEADS, D_HEAD, device=dev, dtype=torch.bfloat16) for _ in range(3)]
        for b, n in enumerate(lens):  # RoPE positions restart at every sequence
            r0 = int(cu[b])
            outs = rope_givens(qkv[None, r0:r0 + n], N_HEADS, m.inv_freq.to(dev), m.theta.detach().to(dev), li, 0)
            for dst, o in zip(bufs, outs):
                dst[r0:r0 + n] = o[0].transpose(0, 1)
        layers.append(([t.permute(1, 0, 2) for t in bufs], m.lam.detach().to(dev)))
    cud = cu.to(dev)
    ops = torch.ops.mote

    def step():
        for (p1, p2, info), lam in layers:
            ops.relation_fwd_varlen(p1, p2, info, lam, cud, max(lens), 2.0)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    flops = 18 * 2.0 * N_HEADS * D_HEAD * sum(n * n for n in lens)
    log(f"[bench] C5 Mote-138M prefill: lens {lens} (total {total}), {ms:.3f} ms/step = "
        f"{flops / ms / 1e9:.1f} TFLOP/s")
    return dict(workload="Mote-138M Relation prefill, varlen core forward (18 layers, 8 ragged sequences, seed 4)",
                lens=lens, total_chunks=total, ms_per_step=round(ms, 4), tflops=round(flops / (ms * 1e-3) / 1e12, 2),
                flop_per_step=flops, frac_bf16_peak=round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4))


# ------------------------------------------------------------------------------------------------
# fused add + RMSNorm (the pre-norm of every H-Net block)
# ------------------------------------------------------------------------------------------------
def bench_norm(rows: int, dev, copies: int, launches: int = 24):
    """mote::add_rms_norm / _bwd at the H-Net block's pre-norm: x bf16 [rows, 768] plus the fp32
    residual stream, prenorm (y bf16 and the new fp32 stream out); backward with the gradients of
    both outputs. Each direction is a HIP graph of `launches` launches rotating over `copies` input
    sets (so that the 256 MB Infinity Cache cannot hold them); time per launch = replay time / launches.
    Algorithmic bytes per row: forward 2D + 4D in, 2D + 4D out, 4 (rstd); backward 2D + 4D + 4D + 4
    in (dy, d stream, s, rstd), 2D + 4D out (dx, d residual)."""
    import mote_amd.norm  # noqa: F401  (registers the ops)

    D = D_MODEL
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (torch.randn(D, generator=g) * 0.2 + 1.0).to(dev)
    sets = []
    for _ in range(copies):
        x = torch.randn(rows, D, generator=g).to(torch.bfloat16).to(dev)
        res = torch.randn(rows, D, generator=g).to(dev)
        y, s_, rstd = torch.ops.mote.add_rms_norm(x, w, res, 1e-5, True, True)
        dy = torch.randn(rows, D, generator=g).to(torch.bfloat16).to(dev)
        dro = torch.randn(rows, D, generator=g).to(dev)
        sets.append((x, res, s_, rstd, dy, dro))
    torch.cuda.synchronize()
    ops = torch.ops.mote

    def fwd(i):
        x, res = sets[i % copies][:2]
        ops.add_rms_norm(x, w, res, 1e-5, True, True)

    def bwd(i):
        _, _, s_, rstd, dy, dro = sets[i % copies]
        ops.add_rms_norm_bwd(dy, dro, s_, rstd, w, torch.bfloat16, True, torch.float32)

    out = {}
    side = torch.cuda.Stream()
    for name, fn, per_row in (("fwd", fwd, 12 * D + 4), ("bwd", bwd, 16 * D + 4)):
        for i in range(copies):
            fn(i)
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(gr, stream=side):
                for i in range(launches):
                    fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for _ in range(2):
            gr.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        t0.record()
        for _ in range(reps):
            gr.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / (reps * launches)
        gbs = rows * per_row / (us * 1e-6) / 1e9
        out[name] = dict(us_per_launch=round(us, 2), bytes_per_launch=rows * per_row, GBs=round(gbs, 1),
                         frac_hbm=round(gbs / PEAK_HBM_GBS, 4))
        del gr
    log(f"[bench] add_rms_norm rows {rows} x {D}: fwd {out['fwd']['us_per_launch']:.2f} us "
        f"({out['fwd']['GBs']:.0f} GB/s), bwd {out['bwd']['us_per_launch']:.2f} us ({out['bwd']['GBs']:.0f} GB/s)")
    return dict(workload=f"add+RMSNorm pre-norm, {rows} rows x {D} (bf16 x, fp32 residual stream), HIP graph "
                         f"of {launches} launches over {copies} input sets", rows=rows, D=D, **out)


# ------------------------------------------------------------------------------------------------
# fused projection prologue (QKV product with RoPE / Givens in the epilogue)
# ------------------------------------------------------------------------------------------------
def bench_qkv(rows: int, dev, copies: int, launches: int = 20):
    """mote::qkv_rope at the Mote-96M shape (x bf16 [rows, 768], w = [w1; w2; wi] [2304, 768], an odd
    layer: RoPE on p1 / p2, Givens pairs (1,2),...,(7,0)) against the unfused path (hipBLASLt product
    + mote::rope_givens), each a HIP graph of `launches` launches over `copies` inputs. The fused
    path's cos / sin table is memoised across calls (as every layer of a step shares it), so the
    graph reuses the table its warm-up wrote. Work: 2 rows D 3D FLOP (the product; the rotations are
    elementwise)."""
    from mote_amd.relation import FullRelation, qkv_rope, rope_givens

    D, H = D_MODEL, N_HEADS
    torch.manual_seed(6)
    m = FullRelation(D, H, 1)
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
    w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).detach().to(torch.bfloat16).to(dev)
    inv, th = m.inv_freq.to(dev), m.theta.detach().to(dev)
    xs = [torch.randn(1, rows, D).to(torch.bfloat16).to(dev) for _ in range(copies)]

    def fused(i):
        return qkv_rope(xs[i % copies], w, H, inv, th, 1, 0)

    def unfused(i):
        return rope_givens(torch.nn.functional.linear(xs[i % copies], w), H, inv, th, 1, 0)

    out = {}
    side = torch.cuda.Stream()
    flops = 2.0 * rows * D * 3 * D
    with torch.no_grad():
        a, b = fused(0), unfused(0)
        diff = max(float((u.float() - v.float()).abs().max()) / max(float(v.float().abs().max()), 1e-3)
                   for u, v in zip(a, b))
        for name, fn in (("fused", fused), ("unfused", unfused)):
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):  # warm-up on the capture stream (fills the RoPE table memo)
                for i in range(copies):
                    fn(i)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(gr, stream=side):
                    for i in range(launches):
                        fn(i)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            for _ in range(2):
                gr.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            t0.record()
            for _ in range(reps):
                gr.replay()
            t1.record()
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) * 1e3 / (reps * launches)
            tf = flops / (us * 1e-6) / 1e12
            out[name] = dict(us_per_launch=round(us, 2), tflops=round(tf, 1), frac_bf16_peak=round(tf / PEAK_BF16_TFLOPS, 4))
            del gr
    log(f"[bench] qkv prologue rows {rows}: fused {out['fused']['us_per_launch']:.1f} us "
        f"({out['fused']['tflops']:.0f} TF/s), unfused {out['unfused']['us_per_launch']:.1f} us; rel diff {diff:.2e}")
    return dict(workload=f"QKV product + RoPE/Givens, {rows} rows x {D} -> 3 x {H} heads x {D // H} (bf16, odd layer), "
                         f"HIP graph of {launches} launches over {copies} inputs", rows=rows, flop_per_launch=flops,
                rel_diff_fused_vs_unfused=diff, **out)


def bench_wgrad(rows: int, dev, copies: int, launches: int = 20):
    """mote::wgrad, the prologue's weight gradient dW = dqkv^T x at the Mote-96M shape (dqkv bf16
    [rows, 2304], x bf16 [rows, 768]), against the GEMM library's dqkv^T x (torch.matmul of the
    transposed view, what the unfused backward runs); each a HIP graph of `launches` launches over
    `copies` input sets. Work: 2 rows 3D D FLOP."""
    from mote_amd.relation import _wgrad

    D = D_MODEL
    g = torch.Generator(device="cpu").manual_seed(9)
    sets = [(torch.randn(rows, 3 * D, generator=g).to(torch.bfloat16).to(dev),
             torch.randn(rows, D, generator=g).to(torch.bfloat16).to(dev)) for _ in range(copies)]
    fns = {"mote_wgrad": lambda i: _wgrad(*sets[i % copies]),
           "library": lambda i: torch.matmul(sets[i % copies][0].t(), sets[i % copies][1])}
    a, b = fns["mote_wgrad"](0), fns["library"](0)
    diff = float((a.float() - b.float()).abs().max()) / max(float(b.float().abs().max()), 1e-3)
    flops = 2.0 * rows * 3 * D * D
    out = {}
    side = torch.cuda.Stream()
    for name, fn in fns.items():
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(copies):
                fn(i)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(gr, stream=side):
                for i in range(launches):
                    fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for _ in range(2):
            gr.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        t0.record()
        for _ in range(reps):
            gr.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / (reps * launches)
        tf = flops / (us * 1e-6) / 1e12
        out[name] = dict(us_per_launch=round(us, 2), tflops=round(tf, 1), frac_bf16_peak=round(tf / PEAK_BF16_TFLOPS, 4))
        del gr
    log(f"[bench] prologue dW rows {rows}: mote_wgrad {out['mote_wgrad']['us_per_launch']:.1f} us "
        f"({out['mote_wgrad']['tflops']:.0f} TF/s), library {out['library']['us_per_launch']:.1f} us; rel diff {diff:.2e}")
    return dict(workload=f"prologue weight gradient dqkv^T x, {rows} rows, [{rows}, {3 * D}]^T [{rows}, {D}] (bf16), "
                         f"HIP graph of {launches} launches over {copies} inputs", rows=rows, flop_per_launch=flops,
                rel_diff_vs_library=diff, **out)


# ------------------------------------------------------------------------------------------------
# chunk gather and EMA dechunk (either side of the main network)
# ------------------------------------------------------------------------------------------------
def bench_dc(B: int, dev, copies: int, launches: int = 20):
    """mote::chunk_route / chunk_gather / chunk_gather_bwd / dechunk / dechunk_bwd at the Mote-96M
    shape: B windows of 16384 bytes, Bernoulli(1/3.3) boundaries (seed 2, first byte forced), D0 = 512,
    bf16 hidden states, fp32 boundary probabilities, chunk rows padded to a multiple of 64. Each op is a
    HIP graph of `launches` launches rotating over `copies` input sets. Algorithmic bytes per launch:
    route L (mask) + 8 L (cum, perm); gather 2 M D 2 (rows in and out); gather_bwd M D 2 + L D 2;
    dechunk M D 2 (x) + L D 2 (bytes out) + M D 4 (z kept) + 8 M (p and positions); dechunk_bwd L D 2
    (dout) + M D 2 (x) + M D 4 (z) + M D 2 (dx) + 16 L (dprob) + 8 M."""
    from mote_amd import dc

    Ln, D = 16384, 512
    g = torch.Generator().manual_seed(2)
    sets = []
    for _ in range(copies):
        mask = torch.rand(B, Ln, generator=g) < (1.0 / 3.3)
        mask[:, 0] = True
        mask = mask.to(dev)
        x = torch.randn(B, Ln, D, generator=g).to(torch.bfloat16).to(dev)
        prob = torch.rand(B, Ln, 2, generator=g).to(dev)
        cum, perm, num, _ = dc.chunk_route(mask)
        M = min(Ln, -(-int(num.max()) // 64) * 64)
        hc = dc.chunk_gather(x, perm, num, mask, cum, M)
        out, w = dc.dechunk(hc, prob, perm, num, mask, cum, 1e-4, None)
        dy = torch.randn(B, Ln, D, generator=g).to(torch.bfloat16).to(dev)
        sets.append(dict(mask=mask, x=x, prob=prob, cum=cum, perm=perm, num=num, M=M, hc=hc, w=w, dy=dy))
    torch.cuda.synchronize()
    Ms = sorted({s_["M"] for s_ in sets})
    M = sum(s_["M"] for s_ in sets) / copies
    ops = {
        "route": (lambda s_: dc.chunk_route(s_["mask"]), B * Ln * 9),
        "gather": (lambda s_: dc.chunk_gather(s_["x"], s_["perm"], s_["num"], s_["mask"], s_["cum"], s_["M"]),
                   2 * B * M * D * 2),
        "gather_bwd": (lambda s_: dc.chunk_gather_bwd(s_["hc"], s_["mask"], s_["cum"], s_["num"], Ln),
                       B * M * D * 2 + B * Ln * D * 2),
        "dechunk": (lambda s_: dc.dechunk(s_["hc"], s_["prob"], s_["perm"], s_["num"], s_["mask"], s_["cum"], 1e-4,
                                          None), B * (M * D * 2 + Ln * D * 2 + M * D * 4 + 8 * M)),
        "dechunk_bwd": (lambda s_: dc.dechunk_bwd(s_["dy"], s_["hc"], s_["prob"], s_["perm"], s_["num"], s_["mask"],
                                                  s_["cum"], s_["w"], 1e-4),
                        B * (Ln * D * 2 + M * D * 2 + M * D * 4 + M * D * 2 + 16 * Ln + 8 * M)),
    }
    res = {}
    side = torch.cuda.Stream()
    for name, (fn, nbytes) in ops.items():
        for s_ in sets:
            fn(s_)
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(gr, stream=side):
                for i in range(launches):
                    fn(sets[i % copies])
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        t0.record()
        for _ in range(reps):
            gr.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / (reps * launches)
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = dict(us_per_launch=round(us, 2), bytes_per_launch=int(nbytes), GBs=round(gbs, 1),
                         frac_hbm=round(gbs / PEAK_HBM_GBS, 4))
        del gr
    log(f"[bench] chunk/dechunk B={B} (M {Ms}): " + ", ".join(f"{k} {v['us_per_launch']:.1f} us" for k, v in res.items()))
    return dict(workload=f"chunk gather + EMA dechunk, {B} x 16384 bytes, D0 = 512 (bf16 hidden, fp32 p), bucket 64, "
                         f"HIP graph of {launches} launches over {copies} input sets", B=B, L=Ln, D=D, M=Ms, **res)


# ------------------------------------------------------------------------------------------------
# CPU baseline: the oracle on the host cores
# ------------------------------------------------------------------------------------------------
def _cpu_times(fn, warmup: int = 1, reps: int = 3):
    """Seconds of `reps` timed calls of fn after `warmup` untimed ones (time.perf_counter)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return ts


def bench_cpu(T: int):
    """The CPU baselines of the build's own restatement of the reference (the test oracle: fp32,
    materialized scores, autograd for the backward) on the host cores, each one warm-up and three
    timed runs over a bounded sample of its workload:
    c3: one Mote-96M layer fwd+bwd at T (the 12-layer step extrapolated), TFLOP/s;
    c2: the Mote-32M stack, 8 layers fwd+bwd over the 4 sequences' real rows, TFLOP/s;
    c5: one Mote-138M layer forward over the 8 ragged sequences, one at a time (18 layers
        extrapolated), TFLOP/s;
    decode_b1 / decode_b16: one 12-layer decode step at S = 4096 (the new rows' RoPE / Givens, the
        append and the read of rows [0, S]), microseconds per step."""
    from oracle import relation as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    res = {}

    def fwd_bwd(p1, p2, info, lam, dy):
        y, _ = O.relation_reference(p1, p2, info, lam, 2.0, 0)
        torch.autograd.grad((y * dy).sum(), [p1, p2, info, lam])

    def leaves(g, B, H, Tn, D):
        return [torch.randn(B, H, Tn, D, generator=g).requires_grad_(True) for _ in range(3)]

    # C3: one layer fwd + bwd
    g = torch.Generator().manual_seed(2)
    p1, p2, info = leaves(g, 1, N_HEADS, T, D_HEAD)
    lam = torch.tensor(0.5, requires_grad=True)
    dy = torch.randn(1, N_HEADS, T, D_HEAD, generator=g)
    ts = _cpu_times(lambda: fwd_bwd(p1, p2, info, lam, dy))
    dt = sum(ts) / len(ts)
    res["c3"] = dict(value=7.0 * N_HEADS * D_HEAD * T * T / dt / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                     sample=f"one Mote-96M Relation layer fwd+bwd (T={T}, H=8, dh=96, fp32, materialized oracle with "
                            f"autograd), 1 warm-up + 3 timed: {', '.join(f'{t:.2f}' for t in ts)} s; the 12-layer "
                            f"step would take {12 * dt:.1f} s", seconds=ts, cpu=cpu)
    del p1, p2, info, dy
    # C2: the Mote-32M stack, real rows of each sequence
    gm = torch.Generator().manual_seed(1)
    mask = torch.rand(4, 2048, generator=gm) < (1.0 / 3.3)
    mask[:, 0] = True
    M = mask.sum(-1).tolist()
    layers = [[(leaves(g, 1, 8, m, 64), torch.randn(1, 8, m, 64, generator=g)) for m in M] for _ in range(8)]
    lam2 = torch.tensor(0.5, requires_grad=True)

    def c2_step():
        for lay in layers:
            for (q, k, v), d in lay:
                fwd_bwd(q, k, v, lam2, d)
    ts = _cpu_times(c2_step)
    dt = sum(ts) / len(ts)
    res["c2"] = dict(value=8 * 7.0 * 8 * 64 * sum(m * m for m in M) / dt / 1e12, unit="TFLOP/s", cores=cores,
                     kind="port", sample=f"the Mote-32M stack (8 layers, B=4, chunks {M}, H=8, dh=64) fwd+bwd over "
                     f"each sequence's real rows, 1 warm-up + 3 timed: {', '.join(f'{t:.2f}' for t in ts)} s per step",
                     seconds=ts)
    del layers
    # C5: one layer forward over the 8 ragged sequences
    lens = torch.randint(1000, 5001, (8,), generator=torch.Generator().manual_seed(4)).tolist()
    seqs = [[torch.randn(1, N_HEADS, n, D_HEAD, generator=g) for _ in range(3)] for n in lens]

    def c5_layer():
        with torch.no_grad():
            for q, k, v in seqs:
                O.relation_reference(q, k, v, torch.tensor(0.5), 2.0, 0)
    ts = _cpu_times(c5_layer)
    dt = sum(ts) / len(ts)
    res["c5"] = dict(value=2.0 * N_HEADS * D_HEAD * sum(n * n for n in lens) / dt / 1e12, unit="TFLOP/s", cores=cores,
                     kind="port", sample=f"one Mote-138M Relation layer forward over 8 ragged sequences {lens} (one at a "
                     f"time, fp32 materialized), 1 warm-up + 3 timed: {', '.join(f'{t:.2f}' for t in ts)} s; the "
                     f"18-layer prefill would take {18 * dt:.1f} s", seconds=ts)
    del seqs
    # C4: one 12-layer decode step at S = 4096, batch 1 and 16 (bf16 caches as the GPU's)
    S0, cap = 4096, 4097
    inv = O.rope_inv_freq(D_HEAD, 10000.0)
    for batch in (1, 16):
        caches = [[(torch.randn(batch, N_HEADS, cap, D_HEAD, generator=g) * 0.7).to(torch.bfloat16) for _ in range(2)]
                  for _ in range(N_LAYERS)]
        raws = [[(torch.randn(batch, N_HEADS, D_HEAD, generator=g) * 0.7).to(torch.bfloat16) for _ in range(3)]
                for _ in range(N_LAYERS)]
        theta = torch.rand(N_HEADS // 2, generator=g) * 0.6 - 0.3
        Sv = torch.full((batch,), S0, dtype=torch.int64)

        def dec_step():
            with torch.no_grad():
                for li in range(N_LAYERS):
                    kc, vc = caches[li]
                    q, k, v = O.decode_rows_ref(*raws[li], Sv, inv, theta, li, torch.bfloat16)
                    kc[:, :, S0], vc[:, :, S0] = k, v
                    O.relation_decode_ref(q, kc, vc, Sv, torch.tensor(0.4), 2.0)
        ts = _cpu_times(dec_step)
        dt = sum(ts) / len(ts)
        res[f"decode_b{batch}"] = dict(value=dt * 1e6, unit="us/step", cores=cores, kind="port",
                                       sample=f"one 12-layer decode step, batch {batch}, S = 4096, bf16 caches (new rows, "
                                       f"append, fp32 read of rows [0, S]), 1 warm-up + 3 timed: "
                                       f"{', '.join(f'{t * 1e3:.1f}' for t in ts)} ms", seconds=ts)
        del caches
    log(f"[bench] CPU oracle on {cores} threads ({cpu}): " +
        ", ".join(f"{k} {v['value']:.4g} {v['unit']}" for k, v in res.items()))
    return res


def profile_kernels(which: str, dev, steps: int = 3) -> None:
    """A short run of one configuration's kernels for rocprofv3 counter passes (no timing, no JSON):
    c3 = the Mote-96M stack step, c2 = the Mote-32M stack step, c5 = the Mote-138M varlen prefill,
    each `steps` times after one warm-up."""
    if which == "c3":
        inp = StackInputs(chunk_count(2, 16384), 2, dev)
    elif which == "c2":
        inp = StackInputs(chunk_count(1, 2048, 4), 1, dev, B=4, d_model=512, heads=8, layers=8)
    elif which == "c5":
        bench_c5(steps, 1, dev)
        torch.cuda.synchronize()
        return
    else:
        raise SystemExit(f"--kernels-only takes c2, c3 or c5, not {which!r}")
    for _ in range(steps + 1):
        stack_step(inp)
    torch.cuda.synchronize()
    log(f"[bench] profiled {which}: {steps + 1} stack steps")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the C2 / C5 / add+RMSNorm / dechunk lines")
    ap.add_argument("--engine-only", action="store_true",
                    help="only the decode-engine lines (batch 1 and 16, --decode-steps tokens), for profiling")
    ap.add_argument("--dc-only", action="store_true",
                    help="only the chunk route / gather / EMA dechunk lines (1 and 8 windows), for profiling")
    ap.add_argument("--kernels-only", choices=("c2", "c3", "c5"), default=None,
                    help="only run one configuration's kernels a few times, for rocprofv3 counter passes")
    ap.add_argument("--summarize-counters", metavar="DIR", default=None,
                    help="print profiles/ lines from rocprofv3 counter CSVs under DIR and exit (no GPU)")
    args = ap.parse_args()
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the Relation path is built and measured on a single GPU "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import mote_amd.flash_relation as fr  # noqa: F401  (registers the ops)
    import mote_amd.relation  # noqa: F401

    if not fr.HAS_HIP:
        raise SystemExit("bench.py needs libmote_relation.so and a GPU")
    dev = torch.device("cuda")
    if args.kernels_only:
        profile_kernels(args.kernels_only, dev)
        return
    if args.engine_only:
        print(json.dumps({k: bench_decode_engine(b, args.decode_steps, dev) for k, b in (("b1", 1), ("b16", 16))}),
              flush=True)
        return
    if args.dc_only:
        print(json.dumps({"B1": bench_dc(1, dev, copies=8), "B8": bench_dc(8, dev, copies=1)}), flush=True)
        return
    copy_calibration(dev)
    st = bench_stack(args.steps, args.warmup, dev)
    dec = {}
    if not args.no_decode:
        dec["b1"] = bench_decode(1, args.decode_steps, dev, copies=4)
        dec["b16"] = bench_decode(16, args.decode_steps, dev, copies=1)
        dec_engine = {k: bench_decode_engine(b, args.decode_steps, dev) for k, b in (("b1", 1), ("b16", 16))}
    extra = {}
    if not args.no_extra:
        extra["c2_mote32m_stack"] = bench_c2(args.steps, args.warmup, dev)
        extra["c5_mote138m_prefill"] = bench_c5(max(3, args.steps // 4), min(args.warmup, 2), dev)
        extra["qkv_prologue"] = {"T": bench_qkv(st["T"], dev, copies=8), "16T": bench_qkv(16 * st["T"], dev, copies=1)}
        extra["prologue_wgrad"] = {"T": bench_wgrad(st["T"], dev, copies=8), "16T": bench_wgrad(16 * st["T"], dev, copies=1)}
        extra["add_rms_norm"] = {"T": bench_norm(st["T"], dev, copies=8),
                                 "16T": bench_norm(16 * st["T"], dev, copies=1)}
        extra["chunk_dechunk"] = {"B1": bench_dc(1, dev, copies=8), "B8": bench_dc(8, dev, copies=1)}
    cpu = None if args.no_cpu else bench_cpu(st["T"])
    out = {
        "metric": METRIC,
        "value": round(st["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(st["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) hidden states, random-init weights, Bernoulli(1/3.3) chunk boundaries, seed 2)",
        "config": {"workload": "Mote-96M Relation stack fwd+bwd (12 layers, B=1, 16384-byte window)",
                   "T_chunks": st["T"], "heads": N_HEADS, "d_head": D_HEAD, "layers": N_LAYERS,
                   "flop_convention": "7*H*dh*T^2 per layer (causal; fwd 2x, bwd 5x)"},
        "roofline": {"kernel": "bwd_kvq_kernel (backward key + query work in one launch: U, dW, dV, dK, dQ)",
                     "bound": "mfma", "achieved": round(st["kq_tflops"], 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(st["kq_tflops"] / PEAK_BF16_TFLOPS, 4), **_traffic("bwd_kvq_kernel"),
                     "counters": measured_counters("bwd_kvq_kernel@c3"),
                     "flop_per_launch": 5.0 * N_HEADS * D_HEAD * st["T"] ** 2, "avg_launch_ms": round(st["kq_ms"], 4),
                     "timed_with": "the clear of the launch's control words (one small kernel) inside the events"},
        "two_launch_form": {
            "bwd_kv_kernel": {"bound": "mfma", "achieved": round(st["keys_tflops"], 2), "unit": "TFLOP/s",
                              "frac": round(st["keys_tflops"] / PEAK_BF16_TFLOPS, 4),
                              "flop_per_launch": 4.0 * N_HEADS * D_HEAD * st["T"] ** 2,
                              "avg_launch_ms": round(st["keys_ms"], 4), **_traffic("bwd_kv_kernel")},
            "bwd_dq_kernel": {"bound": "hbm", "achieved": round(st["queries_gbs"], 1), "unit": "GB/s",
                              "frac": round(st["queries_gbs"] / PEAK_HBM_GBS, 4), "bytes_per_launch": st["queries_bytes"],
                              "avg_launch_ms": round(st["queries_ms"], 4), **_traffic("bwd_dq_kernel")},
            "note": "the same backward as two launches (MOTE_BWD_SPLIT=1 or separate key / query stages)"},
        "roofline_fwd": {"kernel": "relation_fwd_tile_kernel", "bound": "mfma", "achieved": round(st["fwd_tflops"], 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(st["fwd_tflops"] / PEAK_BF16_TFLOPS, 4),
                         **_traffic("relation_fwd_tile_kernel"),
                         "counters": measured_counters("relation_fwd_tile_kernel@c3"),
                         "flop_per_launch": 2.0 * N_HEADS * D_HEAD * st["T"] ** 2, "avg_launch_ms": round(st["fwd_ms"], 4)},
        "stack_frac_of_peak": round(st["tflops"] / PEAK_BF16_TFLOPS, 4),
        "gpu": {**gpu_identity(dev), **st["clock"]},
        "dut_residency": st["dut"],
    }
    if dec:
        out["decode"] = {
            k: {"batch": v["batch"], "us_per_step": round(v["us_per_step"], 2), "layers": N_LAYERS,
                "avg_S": round(v["avg_S"], 1), "step_GBs": round(v["gbs"], 1),
                "step_frac_hbm": round(v["gbs"] / PEAK_HBM_GBS, 4), "kernel_us": round(v["kernel_us"], 2),
                "kernel_GBs": round(v["kernel_gbs"], 1), "kernel_frac_hbm": round(v["kernel_gbs"] / PEAK_HBM_GBS, 4),
                "eager_launch_us": round(v["eager_us"], 2), "launch_floor_us": round(v["launch_floor_us"], 2),
                **_traffic(f"relation_decode_kernel_{k}"),
                "cache_copies_rotated": v["copies"]}
            for k, v in dec.items()}
    if dec:
        out["decode_engine"] = dec_engine
    if "qkv_prologue" in extra:
        q = extra["qkv_prologue"]["T"]
        out["roofline_qkv_prologue"] = {
            "kernel": "qkv_rope_kernel (QKV product with RoPE / Givens in the epilogue, 4964 tokens)", "bound": "mfma",
            "achieved": q["fused"]["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": q["fused"]["frac_bf16_peak"], "flop_per_launch": q["flop_per_launch"],
            "avg_launch_ms": round(q["fused"]["us_per_launch"] / 1e3, 5)}
    out.update(extra)
    if cpu is not None:
        out["cpu_baseline"] = {k: cpu["c3"][k] for k in ("value", "unit", "cores", "kind", "sample")}
        out["cpu_baselines"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
