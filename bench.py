#!/usr/bin/env python3
"""Benchmark of the MI355X Gated DeltaNet hot path (one GPU).

A "step" is one batched decode update of one GDN layer at B=64, T=1
(Hk=16, Hv=32, Dk=Dv=128): the state of every row is read, advanced by one
token and written back in place, and the next step reads it again (state
carried across back-to-back steps, inputs redrawn per step).  ``value`` is
the algorithmic state+I/O bytes per step over the measured step time (GB/s);
the JSON line also carries the other workloads of the path measured in the
same run (decode B=1, MTP verify+commit, chunked prefill T=4096 with the
fused conv prologue, a mixed continuous-batching launch set, and the
full-attention layers of the hybrid trunk and the MTP draft head), the
roofline of the dominant kernel and a CPU baseline.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA, TFLOP/s
Hk, Hv, Dk, Dv, KT = 16, 32, 128, 128, 4
C_DIM = 2 * Hk * Dk + Hv * Dv
CHUNK = 64
METRIC = "GDN decode state GB/s (% HBM peak) at B=64; chunked-prefill tokens/s"


# ------------------------------------------------------------ work models

def state_bytes(B):
    return B * Hv * Dv * Dk * 4


def io_bytes(B, T):
    # q, k read; v read, y written (bf16); a, b read (bf16)
    return B * T * (2 * Hk * Dk * 2 + 2 * Hv * Dv * 2 + 2 * Hv * 2)


def decode_bytes(B, T=1):
    """State read + written once, plus the per-token I/O."""
    return 2 * state_bytes(B) + io_bytes(B, T)


def chunk_flops(C=CHUNK):
    """Algorithmic FLOPs per (chunk, head): KK^T, solve, W, U, 3 state products, QK^T, attn V."""
    return 2 * C * C * Dk + (2.0 / 3.0) * C ** 3 + 2 * C * C * Dk + 2 * C * C * Dv + 6 * C * Dk * Dv \
        + 2 * C * C * Dk + 2 * C * C * Dv


def prefill_flops(lengths):
    return sum(math.ceil(n / CHUNK) for n in lengths) * Hv * chunk_flops()


# ----------------------------------------------------------------- inputs

def draw(gen, B, T, torch, dev, state=True, dtype=None):
    """Seeded inputs: q,k ~ N(0,1) L2-normalised per head (q also / sqrt(Dk)),
    v ~ N(0,1), a, b ~ N(0,1), A_log ~ U(0, ln 16), dt_bias ~ U(-1, 1),
    S0 ~ N(0, 0.02); drawn on the CPU, then copied to ``dev``."""
    dtype = dtype or torch.bfloat16
    q = torch.randn(B, T, Hk, Dk, generator=gen)
    k = torch.randn(B, T, Hk, Dk, generator=gen)
    q = q / q.norm(dim=-1, keepdim=True) / math.sqrt(Dk)
    k = k / k.norm(dim=-1, keepdim=True)
    d = dict(
        q=q.to(dtype), k=k.to(dtype), v=torch.randn(B, T, Hv, Dv, generator=gen).to(dtype),
        a=torch.randn(B, T, Hv, generator=gen).to(dtype), b=torch.randn(B, T, Hv, generator=gen).to(dtype),
        A_log=torch.rand(Hv, generator=gen) * math.log(16.0), dt_bias=torch.rand(Hv, generator=gen) * 2 - 1,
        state=(torch.randn(B, Hv, Dv, Dk, generator=gen) * 0.02) if state else None,
    )
    return {kk: (None if vv is None else vv.to(dev)) for kk, vv in d.items()}


# ---------------------------------------------------------------- timing

class Timer:
    """HIP-event timing on torch's current stream (where every launch goes)."""

    def __init__(self, torch):
        self.torch = torch

    def settle(self, fn, ms=100.0, batch=50):
        """Untimed launches of ``fn`` until ``ms`` of device time has passed:
        a GPU that was idle (input generation on the host) runs its first few
        milliseconds at lower clocks, which a handful of warmup launches does
        not cover.  Returns the launches made."""
        t = self.torch
        spent, n = 0.0, 0
        while spent < ms:
            s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            s.record()
            for i in range(batch):
                fn(n + i)
            e.record()
            t.cuda.synchronize()
            spent += s.elapsed_time(e)
            n += batch
        return n

    def total_ms(self, fn, iters, settle_ms=20.0):
        """Device time of ``iters`` back-to-back calls, after ``settle_ms`` of
        untimed calls (steady clocks whatever ran, or idled, before)."""
        t = self.torch
        if settle_ms:
            self.settle(fn, settle_ms, batch=max(1, min(iters, 50)))
        t.cuda.synchronize()
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record()
        for i in range(iters):
            fn(i)
        e.record()
        t.cuda.synchronize()
        return s.elapsed_time(e)

    def per_launch_ms(self, fn, iters, settle_ms=20.0):
        """Mean of event pairs placed tightly around each launch."""
        t = self.torch
        if settle_ms:
            self.settle(fn, settle_ms, batch=max(1, min(iters, 50)))
        evs = [(t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)) for _ in range(iters)]
        t.cuda.synchronize()
        for i, (s, e) in enumerate(evs):
            s.record()
            fn(i)
            e.record()
        t.cuda.synchronize()
        ds = sorted(s.elapsed_time(e) for s, e in evs)
        return sum(ds) / len(ds), ds[len(ds) // 2]


def read_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, or None."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    vals = {}
    for line in p.read_text().splitlines():
        if "=" in line and line.split("=", 1)[0].strip() in ("fetch_bytes_per_launch", "write_bytes_per_launch"):
            k, v = line.split("=", 1)
            vals[k.strip()] = float(v.split()[0])
    if len(vals) != 2:
        return None
    return vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"]


def read_kernel_avg_us(name, kernel_prefix):
    """Average duration (us) of a kernel in a committed rocprofv3 summary
    table (``| kernel | calls | average (ns) | ...``), or None."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0].startswith(kernel_prefix):
            try:
                return float(cells[2]) / 1e3
            except ValueError:
                continue
    return None


# ------------------------------------------------------------- workloads

def bench_decode_b64(torch, mx, dev, steps, warmup, timer):
    gen = torch.Generator().manual_seed(1001)
    B = 64
    n = max(steps, warmup, 1)
    d = draw(gen, B, n, torch, dev)
    # one contiguous [B,1,...] slab per step
    per = {k: [d[k][:, s:s + 1].contiguous() for s in range(n)] for k in ("q", "k", "v", "a", "b")}
    state = d["state"]
    plans = [mx.prepare_recurrent(per["q"][s], per["k"][s], per["v"][s], per["a"][s], per["b"][s], d["A_log"],
                                  d["dt_bias"], state, state_out=state) for s in range(n)]
    for i in range(warmup):
        plans[i % n].launch()
    timer.settle(lambda i: plans[i % n].launch())
    total = timer.total_ms(lambda i: plans[i % n].launch(), steps)
    per_launch, median = timer.per_launch_ms(lambda i: plans[i % n].launch(), steps)
    ok = bool(torch.isfinite(state).all())
    return dict(ms_per_step=total / steps, kernel_ms=per_launch, kernel_ms_median=median, finite=ok)


def bench_decode_b1(torch, mx, dev, timer, iters=200):
    gen = torch.Generator().manual_seed(1000)
    d = draw(gen, 1, 1, torch, dev)
    plan = mx.prepare_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], d["state"],
                                state_out=d["state"])
    for _ in range(20):
        plan.launch()
    total = timer.total_ms(lambda i: plan.launch(), iters)
    per, med = timer.per_launch_ms(lambda i: plan.launch(), iters)
    # the same steps captured in one HIP graph: device time per step without
    # the host's per-launch cost
    graph, n = torch.cuda.CUDAGraph(), 50
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream(dev)
        for _ in range(n):
            plan.launch(cap)
    graph.replay()
    t_graph = timer.total_ms(lambda i: graph.replay(), 4) / (4 * n)
    # us_event_pair_per_launch: event pairs around each launch, which at this
    # size mostly time the events themselves (the kernel trace gives the kernel)
    return dict(us_per_step=1e3 * total / iters, us_event_pair_per_launch=1e3 * per,
                us_per_step_graph=1e3 * t_graph, bytes=decode_bytes(1))


def bench_verify(torch, mx, dev, timer, iters=50):
    gen = torch.Generator().manual_seed(1002)
    B, T = 32, 4
    d = draw(gen, B, T, torch, dev)
    n_b = torch.randint(1, T + 1, (B,), generator=gen, dtype=torch.int32).to(dev)
    verify = mx.prepare_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], d["state"],
                                  write_state=False)
    commit = mx.prepare_recurrent(None, d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], d["state"],
                                  y=False, commit_len=n_b, state_out=torch.empty_like(d["state"]))
    snap = mx.prepare_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], d["state"],
                                write_state=False, snapshots=True)
    # The commit folded into the next round (gated_delta_commit_verify): one
    # launch over [this round's drafts, the next round's drafts], the rejected
    # drafts masked, the state written after this round's tokens.
    nxt = draw(gen, B, T, torch, dev, state=False)
    cat = {n: torch.cat([d[n], nxt[n]], dim=1).contiguous() for n in ("q", "k", "v", "a", "b")}
    keep = torch.cat([torch.arange(T, device=dev)[None, :] < n_b[:, None],
                      torch.ones(B, T, dtype=torch.bool, device=dev)], dim=1)
    fused = mx.prepare_recurrent(cat["q"], cat["k"], cat["v"], cat["a"], cat["b"], d["A_log"], d["dt_bias"],
                                 d["state"], keep, commit_len=torch.full((B,), T, dtype=torch.int32, device=dev),
                                 state_out=torch.empty_like(d["state"]), y_from=T)

    def round_commit(i):
        verify.launch()
        commit.launch()

    for _ in range(5):
        round_commit(0)
        snap.launch()
        fused.launch()
    t_commit = timer.total_ms(round_commit, iters) / iters
    t_verify, _ = timer.per_launch_ms(lambda i: verify.launch(), iters)
    t_snap = timer.total_ms(lambda i: snap.launch(), iters) / iters
    t_fused = timer.total_ms(lambda i: fused.launch(), iters) / iters
    credited = 2 * state_bytes(B) + io_bytes(B, T)
    return dict(ms_verify_plus_commit=t_commit, ms_verify=t_verify, ms_snapshot_verify=t_snap,
                credited_bytes=credited, gbs=credited / (t_commit * 1e-3) / 1e9,
                frac=credited / (t_commit * 1e-3) / 1e9 / HBM_PEAK_GBS,
                ms_commit_verify_one_pass=t_fused, gbs_one_pass=credited / (t_fused * 1e-3) / 1e9,
                frac_one_pass=credited / (t_fused * 1e-3) / 1e9 / HBM_PEAK_GBS)


def bench_prefill(torch, mx, dev, timer, iters=50):
    gen = torch.Generator().manual_seed(1003)
    T = 4096
    qkv = torch.randn(1, T, C_DIM, generator=gen).to(torch.bfloat16).to(dev)
    w = (torch.randn(C_DIM, KT, generator=gen) * 0.1).to(torch.bfloat16).to(dev)
    cs = torch.zeros(1, KT - 1, C_DIM, dtype=torch.bfloat16, device=dev)
    a = torch.randn(1, T, Hv, generator=gen).to(torch.bfloat16).to(dev)
    b = torch.randn(1, T, Hv, generator=gen).to(torch.bfloat16).to(dev)
    A_log = (torch.rand(Hv, generator=gen) * math.log(16.0)).to(dev)
    dt_bias = (torch.rand(Hv, generator=gen) * 2 - 1).to(dev)
    ws = torch.empty(mx.chunk_workspace_bytes(1, T, Hv, Dk, Dv), dtype=torch.uint8, device=dev)
    # prepared launches (validated once, as a serving loop issues them): the
    # prologue's q/k/v buffers are the chunked pass's inputs
    pro = mx.prepare_conv_prologue(qkv, w, Hk, Hv, Dk, Dv, cs)
    q, k, v, _ = pro.outputs
    gdn = mx.prepare_chunked(q, k, v, a, b, A_log, dt_bias, None, workspace=ws)
    out = {"S": gdn.outputs[1]}
    # the mixer's path: the prologue inside the chunked pass's prep (one
    # call, two launches), bit-identical to the two calls above
    wsf = torch.empty(mx.conv_chunk_workspace_bytes(1, T, Hv, Dk, Dv), dtype=torch.uint8, device=dev)
    fused = mx.prepare_conv_chunked(qkv, w, Hk, Hv, Dk, Dv, a, b, A_log, dt_bias, None, cs, workspace=wsf)

    def step(i):
        fused.launch()

    def unfused(i):
        pro.launch()
        gdn.launch()

    def gdn_only(i):
        gdn.launch()

    def pro_only(i):
        pro.launch()

    for _ in range(3):
        step(0)
        unfused(0)
    t_all = timer.total_ms(step, iters) / iters
    t_unfused = timer.total_ms(unfused, iters) / iters
    t_gdn = timer.total_ms(gdn_only, iters) / iters
    t_pro = timer.total_ms(pro_only, iters) / iters
    flops = prefill_flops([T])
    torch.cuda.synchronize()
    same = bool(torch.equal(fused.outputs[1], out["S"]))
    return dict(ms_total=t_all, ms_unfused=t_unfused, ms_gdn=t_gdn, ms_prologue=t_pro,
                tokens_per_s=T / (t_all * 1e-3),
                gdn_tflops=flops / (t_gdn * 1e-3) / 1e12, mfma_frac=flops / (t_gdn * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                mfma_frac_with_prologue=flops / (t_all * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                flops=flops, finite=bool(torch.isfinite(out["S"]).all()), fused_equals_unfused=same)


def mixed_bytes(lens, n_dec=48, n_ver=16, t_ver=4):
    """Credited HBM bytes of the mixed step: the packed prefills' I/O and
    prefix states (read + written), the decode rows' states and I/O, and the
    verify rows' state read + one committed write and I/O."""
    n_seq = len(lens)
    prefill = io_bytes(1, sum(lens)) + 2 * state_bytes(n_seq)
    return prefill, decode_bytes(n_dec) + 2 * state_bytes(n_ver) + io_bytes(n_ver, t_ver)


def bench_mixed(torch, mx, dev, timer, iters=50):
    """One continuous-batching step (``multiplex_amd.MixedStep``): the packed
    prefills' prep and scan on the current stream; the decode, verify and
    commit launches (independent rows and states) on a second stream beside
    the scan, once the prep is done; the step ends when both are done.  For
    comparison, the same launches on one stream."""
    gen = torch.Generator().manual_seed(1004)
    lens = [1024, 2560, 7168]
    n_tok = sum(lens)
    cu = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(3)], dtype=torch.int32)
    pf = draw(gen, 1, n_tok, torch, dev, state=False)
    pf_state = (torch.randn(3, Hv, Dv, Dk, generator=gen) * 0.02).to(dev)
    dec = draw(gen, 48, 1, torch, dev)
    ver = draw(gen, 16, 4, torch, dev)
    n_b = torch.randint(1, 5, (16,), generator=gen, dtype=torch.int32).to(dev)
    ws = torch.empty(mx.chunk_workspace_bytes(3, n_tok, Hv, Dk, Dv), dtype=torch.uint8, device=dev)
    dplan = mx.prepare_recurrent(dec["q"], dec["k"], dec["v"], dec["a"], dec["b"], dec["A_log"],
                                 dec["dt_bias"], dec["state"], state_out=dec["state"])
    vplan = mx.prepare_recurrent(ver["q"], ver["k"], ver["v"], ver["a"], ver["b"], ver["A_log"],
                                 ver["dt_bias"], ver["state"], write_state=False)
    cplan = mx.prepare_recurrent(None, ver["k"], ver["v"], ver["a"], ver["b"], ver["A_log"], ver["dt_bias"],
                                 ver["state"], y=False, commit_len=n_b, state_out=torch.empty_like(ver["state"]))
    pplan = mx.prepare_chunked(pf["q"], pf["k"], pf["v"], pf["a"], pf["b"], pf["A_log"], pf["dt_bias"], pf_state,
                               cu_seqlens=cu, workspace=ws, state_out=torch.empty_like(pf_state))
    # verify and commit first, the decode last: with the decode first the
    # step took about 3 us longer (332.5 against 329.4 us, four alternating
    # runs); the launches are independent, so the outputs are the same
    step = mx.MixedStep(pplan, [vplan, cplan, dplan])

    for _ in range(3):
        step.launch()
        step.launch_overlapped()
    timer.settle(lambda i: step.launch())
    # the two schedules timed alternately, twice each (best of each), so
    # neither gains from running second
    tt, ts = [], []
    for _ in range(2):
        tt.append(timer.total_ms(lambda i: step.launch_overlapped(), iters) / iters)
        ts.append(timer.total_ms(lambda i: step.launch_serial(), iters) / iters)
    t, t_serial = min(tt), min(ts)
    flops = prefill_flops(lens)
    pf_bytes, dv_bytes = mixed_bytes(lens)
    hbm = pf_bytes + dv_bytes
    bound_ms = max(flops / (MFMA_BF16_PEAK_TFLOPS * 1e12), hbm / (HBM_PEAK_GBS * 1e9)) * 1e3
    toks = n_tok + 48 + 64
    return dict(ms=t, ms_one_stream=t_serial, tokens_per_s=toks / (t * 1e-3), prefill_gflop=flops / 1e9,
                prefill_bytes=pf_bytes, decode_verify_bytes=dv_bytes,
                mfma_frac=round(flops / (t * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                hbm_frac=round(hbm / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                lower_bound_ms=round(bound_ms, 5), bound_frac=round(bound_ms / t, 4), streams=2)


def bench_decode_past_mall(torch, mx, dev, timer, B=256, steps=50):
    """Decode at B=256: a 512 MiB state, twice the 256 MB last-level cache
    (MALL), so no step can be served from it; GB/s as for B=64."""
    gen = torch.Generator().manual_seed(1011)
    d = draw(gen, B, 1, torch, dev)
    plan = mx.prepare_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], d["state"],
                                state_out=d["state"])
    for _ in range(5):
        plan.launch()
    timer.settle(lambda i: plan.launch())
    t = timer.total_ms(lambda i: plan.launch(), steps) / steps
    gbs = decode_bytes(B) / (t * 1e-3) / 1e9
    del d, plan
    torch.cuda.empty_cache()
    return dict(B=B, state_bytes=state_bytes(B), ms_per_step=round(t, 5), gbs=round(gbs, 1),
                hbm_frac=round(gbs / HBM_PEAK_GBS, 4))


def bench_epilogue(torch, mx, dev, timer, iters=50):
    """The mixer epilogue's gated RMSNorm at the decode (B=64) and prefill
    (T=4096) row counts: the fused HIP kernel, and for comparison the same
    formula as separate torch ops (what the epilogue cost before fusion)."""
    gen = torch.Generator().manual_seed(1005)
    res = {}
    for name, rows in (("decode_b64", 64 * Hv), ("prefill_t4096", 4096 * Hv)):
        x = torch.randn(rows, Dv, generator=gen).to(torch.bfloat16).to(dev)
        z = torch.randn(rows, Dv, generator=gen).to(torch.bfloat16).to(dev)
        w = (1 + 0.1 * torch.randn(Dv, generator=gen)).to(torch.bfloat16).to(dev)
        plan = mx.prepare_gated_rms_norm(x, z, w, 1e-6)

        def fused(i):
            plan.launch()

        def unfused(i):
            xf = x.float()
            n = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
            (w * n * torch.nn.functional.silu(z.float())).to(torch.bfloat16)

        for _ in range(5):
            fused(0)
            unfused(0)
        t = timer.total_ms(fused, iters) / iters
        t_ref = timer.total_ms(unfused, iters) / iters
        nbytes = 3 * rows * Dv * 2
        res[name] = dict(rows=rows, us=round(1e3 * t, 3), bytes=nbytes, gbs=round(nbytes / (t * 1e-3) / 1e9, 1),
                         hbm_frac=round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         unfused_torch_us=round(1e3 * t_ref, 3))
    return res


def bench_pool(torch, mx, dev, timer, iters=20):
    """Pooled states: a batch-membership change (64 rows -> keep 48 -> add 16
    fresh rows) done densely (index_select + cat of the fp32 states, as the
    engine's filter / merge do) and through a StatePool (slot lists only);
    and B=64 decode steps reading and writing pool slots."""
    gen = torch.Generator().manual_seed(1006)
    B = 64
    keep = sorted(torch.randperm(B, generator=gen)[:48].tolist())
    dense = (torch.randn(B, Hv, Dv, Dk, generator=gen) * 0.02).to(dev)
    keep_t = torch.tensor(keep, device=dev)

    def dense_change(i):
        s = dense.index_select(0, keep_t)
        torch.cat([s, torch.zeros(16, Hv, Dv, Dk, device=dev)])

    pool = mx.StatePool(2 * B, Hv, Dv, Dk, device=dev)

    def pooled_change(i):
        batch = mx.PooledBatch(pool, pool.alloc(B, zero=False))
        batch.filter(keep)
        batch = mx.PooledBatch.merge([batch, mx.PooledBatch.new(pool, 16)])
        batch.index  # the int32 slot table the next launch reads
        batch.release()

    for _ in range(3):
        dense_change(0)
        pooled_change(0)
    t_dense = timer.total_ms(dense_change, iters) / iters
    t_pool = timer.total_ms(pooled_change, iters) / iters

    d = draw(gen, B, 1, torch, dev, state=False)
    slots = pool.alloc(B, zero=False)
    pool.states.copy_((torch.randn(pool.states.shape, generator=gen) * 0.02).to(dev))
    plan = mx.prepare_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], pool.states,
                                state_index=pool.index(slots), state_out=pool.states)
    for _ in range(10):
        plan.launch()
    timer.settle(lambda i: plan.launch())
    t_dec = timer.total_ms(lambda i: plan.launch(), 100) / 100
    return dict(change_dense_us=round(1e3 * t_dense, 2), change_pooled_us=round(1e3 * t_pool, 2),
                dense_bytes_moved=(48 + 48 + 64) * state_bytes(1),
                decode_b64_pooled_ms=round(t_dec, 5),
                decode_b64_pooled_gbs=round(decode_bytes(B) / (t_dec * 1e-3) / 1e9, 1))


def bench_prefix_state(torch, mx, dev, layers=24):
    """Prefix-cache state records: a snapshot of ``layers`` GDN layers (conv
    state [1,3,8192] bf16 + recurrent state [1,32,128,128] fp32 each) staged
    device -> pinned host asynchronously, encoded (SHA-256 content keys) and
    uploaded back."""
    from multiplex_amd import prefix_state as ps

    gen = torch.Generator().manual_seed(1007)
    snap = [[torch.randn(1, KT - 1, C_DIM, generator=gen).to(torch.bfloat16).to(dev),
             (torch.randn(1, Hv, Dv, Dk, generator=gen) * 0.02).to(dev)] for _ in range(layers)]
    nbytes = sum(t.numel() * t.element_size() for layer in snap for t in layer)
    side = torch.cuda.Stream(dev)
    ps.stage_to_host(snap, side).wait()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    host = ps.stage_to_host(snap, side).wait()
    t_d2h = time.perf_counter() - t0
    t0 = time.perf_counter()
    spec, blobs = ps.encode_tree(host)
    t_enc = time.perf_counter() - t0
    t0 = time.perf_counter()
    back = ps.load_tree(spec, blobs.__getitem__, dev)
    torch.cuda.synchronize()
    t_h2d = time.perf_counter() - t0
    ok = all(torch.equal(a, b) for la, lb in zip(snap, back) for a, b in zip(la, lb))
    return dict(layers=layers, bytes=nbytes, d2h_ms=round(1e3 * t_d2h, 3), d2h_gbs=round(nbytes / t_d2h / 1e9, 1),
                encode_ms=round(1e3 * t_enc, 1), decode_upload_ms=round(1e3 * t_h2d, 1), round_trip_equal=ok)


def bench_mixer_layer(torch, mx, dev, timer, iters=20, hidden=2048):
    """One whole GatedDeltaNet mixer layer at the benchmark head layout with
    hidden size 2048 (in_proj GEMMs, fused prologue, GDN kernel, fused gated
    RMSNorm, out_proj GEMM), eager from Python and graph-replayed: decode
    B=64 and B=8 (one token per row, states in a StatePool updated in place;
    at B=8 the norm runs inside out_proj, and the unfused B=8 step is timed
    beside it) and prefill T=4096."""
    gen = torch.Generator().manual_seed(1008)
    m = mx.GatedDeltaNet(hidden, Hk, Hv, Dk, Dv, device=dev)
    m.reset_parameters(gen)
    res = {"hidden": hidden}

    def decode(B, tag):
        pool = mx.StatePool(B, Hv, Dv, Dk, device=dev)
        cache = mx.ArraysCache()
        cache[1] = mx.PooledBatch.new(pool, B)
        x = torch.randn(B, 1, hidden, generator=gen).to(torch.bfloat16).to(dev)
        for _ in range(3):
            m(x, None, cache)
        t = timer.total_ms(lambda i: m(x, None, cache), iters) / iters
        res[f"decode_{tag}_us"] = round(1e3 * t, 2)
        # the same step captured once in a HIP graph and replayed (pooled
        # decode updates the conv state in place, so the captured step reads
        # and writes the same buffers every replay)
        cs_in = cache[0]

        def step():
            m(x, None, cache)
            if cache[0] is not cs_in:  # a new conv state: hand it back to the captured buffer
                cs_in.copy_(cache[0])
                cache[0] = cs_in

        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(3):
            graph.replay()
        t = timer.total_ms(lambda i: graph.replay(), iters) / iters
        res[f"decode_{tag}_graph_us"] = round(1e3 * t, 2)
        # eight steps in one graph (as a captured multi-layer forward pass
        # issues its layers): per-step time without a graph launch per step
        graph8 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph8):
            for _ in range(8):
                step()
        for _ in range(3):
            graph8.replay()
        t8 = timer.total_ms(lambda i: graph8.replay(), iters) / (8 * iters)
        res[f"decode_{tag}_graph8_us_per_step"] = round(1e3 * t8, 2)

    with torch.no_grad():
        decode(64, "b64")
        # at 8 rows the gated norm runs inside out_proj's operand load; the
        # same step with the separate norm kernel and the library GEMM beside it
        decode(8, "b8")
        fused = m.fused_norm_max_rows
        m.fused_norm_max_rows = 0
        decode(8, "b8_unfused")
        m.fused_norm_max_rows = fused
        xp = torch.randn(1, 4096, hidden, generator=gen).to(torch.bfloat16).to(dev)
        for _ in range(2):
            m(xp, None, mx.ArraysCache())
        t = timer.total_ms(lambda i: m(xp, None, mx.ArraysCache()), max(3, iters // 4)) / max(3, iters // 4)
        res["prefill_t4096_ms"] = round(t, 4)
        res["prefill_t4096_tokens_per_s"] = round(4096 / (t * 1e-3), 1)
    return res


# ------------------------------------------------------------ CPU baseline

QWEN35_ATTN = dict(hidden_size=4096, num_attention_heads=16, num_key_value_heads=4, head_dim=256,
                   intermediate_size=12288, rms_norm_eps=1e-6, partial_rotary_factor=0.25, rope_theta=1.0e7)


def bench_attention(torch, mx, dev, timer, iters=20, L=4096):
    """The full-attention path at Qwen3.5's attention shapes (Hq=16, Hkv=4,
    D=256): GQA attention over a 4096-position KV cache for decode (B=64,
    T=1) and draft verify (B=32, T=4) -- HBM-bound on the cache read -- and a
    causal prefill of 4096 tokens (MFMA-bound); then one MTP draft step of a
    one-layer head at hidden 4096 over the same cache length (weights plus
    cache read per step).  Synthetic bf16 data, random weights."""
    from multiplex_amd import attention as att

    a = mx.AttentionArgs(**QWEN35_ATTN)
    Hq, Hkv, D = a.num_attention_heads, a.num_key_value_heads, a.head_dim
    gen = torch.Generator().manual_seed(1006)
    res = {}

    def kv(B, cap):
        k = torch.randn(B, Hkv, cap, D, generator=gen).to(torch.bfloat16).to(dev)
        return k, torch.randn(B, Hkv, cap, D, generator=gen).to(torch.bfloat16).to(dev)

    for name, B, T in (("decode_b64", 64, 1), ("verify_b32_t4", 32, 4)):
        kc, vc = kv(B, L)
        q = torch.randn(B, T, Hq, D, generator=gen).to(torch.bfloat16).to(dev)
        gate = torch.randn(B, T, Hq * 2 * D, generator=gen).to(torch.bfloat16).to(dev)
        pos0 = torch.full((B,), L - T, dtype=torch.int32, device=dev)
        layer = mx.Attention(a, device=dev)
        ns = layer._splits(B, T, L)
        ws = torch.empty(max(1, int(mx._lib.load().gdn_attn_workspace_bytes(B, T, Hq, Hkv, D, ns))),
                         dtype=torch.uint8, device=dev)
        out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
        fn = lambda i: att.attn_fwd(q, kc, vc, pos0, L, gate=gate, n_split=ns, workspace=ws, out=out)
        for i in range(3):
            fn(i)
        ms = timer.total_ms(fn, iters) / iters
        byts = 2 * B * Hkv * L * D * 2 + 2 * q.numel() * 2 + gate.numel() * 2
        res[f"attn_{name}"] = {"ms": round(ms, 5), "n_split": ns, "bytes": byts,
                               "GB/s": round(byts / (ms * 1e-3) / 1e9, 1),
                               "hbm_frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del kc, vc

    T = 4096
    kc, vc = kv(1, T)
    q = torch.randn(1, T, Hq, D, generator=gen).to(torch.bfloat16).to(dev)
    pos0 = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    fn = lambda i: att.attn_fwd(q, kc, vc, pos0, T, out=out)
    for i in range(3):
        fn(i)
    ms = timer.total_ms(fn, iters) / iters
    flops = 4.0 * Hq * D * T * (T + 1) / 2
    res["attn_prefill_t4096"] = {"ms": round(ms, 5), "gflop": round(flops / 1e9, 2),
                                 "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                 "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    del kc, vc

    B = 64
    head = mx.MTPHead(a, n_layers=1, device=dev)
    cache = head.make_cache(B, L + 8)
    c = cache[0]
    c.keys.normal_()
    c.values.normal_()
    c.advance(L - 1)
    H = a.hidden_size
    emb = torch.randn(B, 1, H, generator=gen).to(torch.bfloat16).to(dev)
    hid = torch.randn(B, 1, H, generator=gen).to(torch.bfloat16).to(dev)

    def step(i):
        head(emb, hid, cache)
        c.trim(1)

    for i in range(3):
        step(i)
    ms = timer.total_ms(step, iters) / iters
    wbytes = sum(p.numel() * p.element_size() for p in head.parameters())
    byts = wbytes + 2 * B * Hkv * L * D * 2
    res["mtp_draft_step_b64"] = {"ms": round(ms, 5), "weight_bytes": wbytes, "kv_bytes": 2 * B * Hkv * L * D * 2,
                                 "GB/s": round(byts / (ms * 1e-3) / 1e9, 1),
                                 "hbm_frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    res["shapes"] = dict(QWEN35_ATTN, cache_len=L)
    return res


def cpu_model_name():
    """The host CPU's model name (as ``lscpu`` reports it), from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(torch, budget_s=10.0):
    """The reference's ops path (fp32 port, oracle/ops_path.py) on host cores,
    with ``os.cpu_count()`` threads.

    Samples: decode steps at B=64 until ``budget_s`` seconds have passed (at
    least 2), reported as algorithmic GB/s like ``value``; the T=4096 prefill
    with its conv prologue; 20 decode steps at B=1; one B=32, T=4 verify with
    the reference's restore + replay rollback; and the mixed step (the three
    packed prefills run one sequence at a time, since the ops path has no
    packed form, plus 48 decode rows and 16 verify rows with rollback).
    """
    sys.path.insert(0, str(ROOT))
    from oracle import ops_path

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(1001)
    d = draw(gen, 64, 1, torch, "cpu")
    S = d["state"].float()
    done, t0 = 0, time.perf_counter()
    while done < 2 or (time.perf_counter() - t0 < budget_s and done < 50):
        _, S = ops_path.gated_delta_update(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"], d["dt_bias"], S)
        done += 1
    dt = (time.perf_counter() - t0) / done

    def prefill(T, seed, state=None):
        g = torch.Generator().manual_seed(seed)
        qkv = torch.randn(1, T, C_DIM, generator=g).to(torch.bfloat16)
        w = (torch.randn(C_DIM, KT, generator=g) * 0.1).to(torch.bfloat16)
        a = torch.randn(1, T, Hv, generator=g).to(torch.bfloat16)
        b = torch.randn(1, T, Hv, generator=g).to(torch.bfloat16)
        A_log = torch.rand(Hv, generator=g) * math.log(16.0)
        dt_bias = torch.rand(Hv, generator=g) * 2 - 1
        s0 = torch.zeros(1, Hv, Dv, Dk) if state is None else state
        t1 = time.perf_counter()
        q, k, v, _ = ops_path.conv_prologue(qkv, w, Hk, Hv, Dk, Dv, torch.zeros(1, KT - 1, C_DIM))
        ops_path.gated_delta_update(q, k, v, a, b, A_log, dt_bias, s0)
        return time.perf_counter() - t1

    T = 4096
    tp = prefill(T, 1003)
    # decode B=1: median of 20 steps
    gen = torch.Generator().manual_seed(1000)
    d1 = draw(gen, 1, 1, torch, "cpu")
    S1, times = d1["state"].float(), []
    for _ in range(20):
        t2 = time.perf_counter()
        _, S1 = ops_path.gated_delta_update(d1["q"], d1["k"], d1["v"], d1["a"], d1["b"], d1["A_log"], d1["dt_bias"], S1)
        times.append(time.perf_counter() - t2)
    t_b1 = sorted(times)[len(times) // 2]

    def verify_rollback(B, seed):
        # MTP verify at T=4, then the reference's rollback: restore the
        # snapshot and replay each row's accepted prefix (engine.py:337-359)
        g = torch.Generator().manual_seed(seed)
        dv = draw(g, B, 4, torch, "cpu")
        n_b = torch.randint(1, 5, (B,), generator=g)
        t3 = time.perf_counter()
        S0 = dv["state"].float().clone()
        ops_path.gated_delta_update(dv["q"], dv["k"], dv["v"], dv["a"], dv["b"], dv["A_log"], dv["dt_bias"], S0)
        for n in sorted(set(n_b.tolist())):
            rows = (n_b == n).nonzero().flatten()
            sl = lambda t: t[rows][:, :n]
            ops_path.gated_delta_update(sl(dv["q"]), sl(dv["k"]), sl(dv["v"]), sl(dv["a"]), sl(dv["b"]), dv["A_log"],
                                        dv["dt_bias"], S0[rows])
        return time.perf_counter() - t3

    t_ver = verify_rollback(32, 1002)
    # the mixed step: prefills of 1024, 2560 and 7168 tokens from prefix
    # states, 48 decode rows, 16 verify rows with rollback
    g = torch.Generator().manual_seed(1004)
    t_mix = sum(prefill(n, 2000 + n, torch.randn(1, Hv, Dv, Dk, generator=g) * 0.02) for n in (1024, 2560, 7168))
    dd = draw(g, 48, 1, torch, "cpu")
    t4 = time.perf_counter()
    ops_path.gated_delta_update(dd["q"], dd["k"], dd["v"], dd["a"], dd["b"], dd["A_log"], dd["dt_bias"],
                                dd["state"].float())
    t_mix += time.perf_counter() - t4 + verify_rollback(16, 1005)
    model = cpu_model_name()
    return dict(value=decode_bytes(64) / dt / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"{done} decode steps at B=64 (ops-path port, fp32, torch CPU), "
                       f"{dt * 1e3:.1f} ms/step; prefill T=4096 with conv prologue: {T / tp:.0f} tokens/s; "
                       f"decode B=1 {t_b1 * 1e6:.0f} us/step; verify B=32 T=4 + replay rollback {t_ver * 1e3:.1f} ms; "
                       f"mixed step (1024+2560+7168 prefill, 48 decode, 16 verify + rollback) {t_mix * 1e3:.0f} ms; "
                       f"{threads} threads on {model}",
                ms_per_step=dt * 1e3, prefill_tokens_per_s=T / tp, decode_b1_us=t_b1 * 1e6, verify_ms=t_ver * 1e3,
                mixed_ms=t_mix * 1e3, cpu=model)


# ------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--decode-only", action="store_true", help="only the B=64 decode workload")
    ap.add_argument("--decode-b1-only", action="store_true", help="only the B=1 decode workload")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device-to-device copy (counter calibration) and exit")
    ap.add_argument("--prefill-only", action="store_true", help="only the T=4096 prefill workload")
    ap.add_argument("--mixed-only", action="store_true", help="only the mixed continuous-batching step")
    ap.add_argument("--epilogue-only", action="store_true", help="only the gated RMSNorm epilogue workloads")
    ap.add_argument("--verify-only", action="store_true", help="only the B=32, T=4 verify + commit workload")
    ap.add_argument("--mixer-only", action="store_true", help="only the whole-mixer-layer workloads")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the full-attention (trunk attention layer, MTP draft head) workloads")
    ap.add_argument("--pool-only", action="store_true",
                    help="only the pooled-state and prefix-cache state-record workloads")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only time in-place streaming updates (read + write) of 128 MiB and 1 GiB fp32 "
                         "with a library elementwise kernel, the practical HBM ceiling the decode kernel is "
                         "compared against, and exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the GDN path runs on a single MI355X "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        sys.exit(2)

    import torch

    sys.path.insert(0, str(ROOT))
    import multiplex_amd as mx

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    timer = Timer(torch)
    if args.copy_calibration:
        # A plain streaming kernel of known size (read 256 MiB, write 256
        # MiB): what HBM byte counters read for it calibrates their reading
        # of the GDN kernels.  (A same-dtype copy_ would go to the DMA
        # engines, not to a kernel the counters see.)
        src = torch.randn(64 * 1024 * 1024, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": 2 * src.numel() * 4, "launches": args.steps}), flush=True)
        return
    if args.hbm_ceiling:
        res = {}
        for mib in (128, 1024):
            x = torch.zeros(mib * 1024 * 1024 // 4, device=dev)
            for _ in range(5):
                x.mul_(0.5)
            t = timer.total_ms(lambda i: x.mul_(0.5), 50) / 50
            res[f"{mib}MiB"] = {"ms": round(t, 5), "GB/s": round(2 * x.numel() * 4 / (t * 1e-3) / 1e9, 1)}
            del x
        print(json.dumps({"inplace_stream": res, "peak_GB/s": HBM_PEAK_GBS}), flush=True)
        return
    if args.mixer_only:
        print(json.dumps({"mixer_layer": bench_mixer_layer(torch, mx, dev, timer, iters=args.steps)}), flush=True)
        return
    if args.decode_b1_only:
        print(json.dumps({"decode_b1": bench_decode_b1(torch, mx, dev, timer, iters=args.steps)}), flush=True)
        return
    if args.attention_only:
        print(json.dumps({"attention": bench_attention(torch, mx, dev, timer, iters=args.steps)}), flush=True)
        return
    if args.verify_only:
        print(json.dumps({"verify_b32_t4": bench_verify(torch, mx, dev, timer, iters=args.steps)}), flush=True)
        return
    if args.pool_only:
        print(json.dumps({"state_pool": bench_pool(torch, mx, dev, timer),
                          "prefix_state": bench_prefix_state(torch, mx, dev)}), flush=True)
        return
    if args.epilogue_only:
        print(json.dumps({"epilogue_gated_rmsnorm": bench_epilogue(torch, mx, dev, timer, iters=args.steps)}),
              flush=True)
        return
    if args.prefill_only:
        p = bench_prefill(torch, mx, dev, timer, iters=args.steps)
        print(json.dumps({"prefill_t4096": p}), flush=True)
        return
    if args.mixed_only:
        print(json.dumps({"mixed": bench_mixed(torch, mx, dev, timer, iters=args.steps)}), flush=True)
        return

    dec = bench_decode_b64(torch, mx, dev, args.steps, args.warmup, timer)
    step_bytes = decode_bytes(64)
    value = step_bytes / (dec["ms_per_step"] * 1e-3) / 1e9
    # One launch of the decode kernel per step: its average duration is the
    # timed region's HIP-event span over the steps (back-to-back launches).
    achieved = value
    configs = {}
    if not args.decode_only:
        configs["decode_b1"] = bench_decode_b1(torch, mx, dev, timer)
        configs["verify_b32_t4"] = bench_verify(torch, mx, dev, timer)
        configs["prefill_t4096"] = bench_prefill(torch, mx, dev, timer)
        configs["mixed"] = bench_mixed(torch, mx, dev, timer)
        configs["decode_b256_past_mall"] = bench_decode_past_mall(torch, mx, dev, timer)
        configs["epilogue_gated_rmsnorm"] = bench_epilogue(torch, mx, dev, timer)
        configs["state_pool"] = bench_pool(torch, mx, dev, timer)
        configs["prefix_state"] = bench_prefix_state(torch, mx, dev)
        configs["mixer_layer"] = bench_mixer_layer(torch, mx, dev, timer)
        configs["attention"] = bench_attention(torch, mx, dev, timer)
    base = None if args.no_cpu else cpu_baseline(torch)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "GDN decode B=64 T=1 Hk=16 Hv=32 Dk=Dv=128, fp32 state carried in place over back-to-back steps",
            "B": 64, "T": 1, "Hk": Hk, "Hv": Hv, "Dk": Dk, "Dv": Dv, "io_dtype": "bf16",
            "bytes_per_step": step_bytes, "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic("decode_b64_traffic.txt"),
            "kernel": "recurrent_kernel<128, bf16, GF_IO_F32, kDecodeLean>",
            # achieved = bytes per launch / (event-timed span of the back-to-back launches / launches)
            "ms_per_launch_event_span": round(dec["ms_per_step"], 5),
            "ms_per_launch_event_pairs": round(dec["kernel_ms"], 5),
            "kernel_us_rocprof_committed": read_kernel_avg_us("decode_b64_kernel_trace.md", "recurrent_kernel"),
        },
        "cpu_baseline": None if base is None else {k: base[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "prefill": None,
        "configs": configs,
    }
    if base is not None:
        if "decode_b1" in configs:
            configs["decode_b1"]["cpu_us_per_step"] = round(base["decode_b1_us"], 1)
        if "verify_b32_t4" in configs:
            configs["verify_b32_t4"]["cpu_ms_verify_plus_rollback"] = round(base["verify_ms"], 2)
        if "mixed" in configs:
            configs["mixed"]["cpu_ms"] = round(base["mixed_ms"], 1)
    if "prefill_t4096" in configs:
        p = configs["prefill_t4096"]
        line["prefill"] = {"tokens_per_s": round(p["tokens_per_s"], 1), "ms": round(p["ms_total"], 4),
                           "unfused_ms": round(p["ms_unfused"], 4), "gdn_ms": round(p["ms_gdn"], 4),
                           "mfma_frac": round(p["mfma_frac"], 4),
                           "cpu_tokens_per_s": None if base is None else round(base["prefill_tokens_per_s"], 1)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
