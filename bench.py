#!/usr/bin/env python3
"""Benchmark of the HTile hot path on one MI355X.

Default workload (the configuration BASELINE.json's metric is quoted on,
configs[1]): causal bf16 prefill flash-attention B=4 H=32 S=4096 D=128 with
per-row logsumexp, inputs ~ 0.5 N(0,1) resident in HBM. A step is one
neptune_attn_fwd launch over that batch. The JSON line also carries, under
"secondary", the split-K GQA decode (bf16 and fp8 KV, contiguous and paged)
and selective-scan configurations measured the same way (GB/s against HBM),
config 1 (fp32 single-head attention, latency-bound, TFLOP/s) and the
reference's own tile program (f16 non-causal [1, 32, 4096, 128] through the
HTile front end), each with its own cpu_baseline, and a bf16 GEMM
(hipBLASLt) that calibrates the dense MFMA rate this box sustains: the
headline's prefill_over_gemm is the prefill's rate over that GEMM's.

Each workload first runs untimed for SPINUP_S seconds (so the GPU is at its
working clocks), then W warmup steps, then exactly K timed steps.
roofline.achieved = algorithmic FLOPs (or bytes) per launch / mean launch
duration from HIP events on the launch stream; cpu_baseline = the CPU oracle
(oracle/, OpenMP) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "mlir-toy_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "attention TFLOP/s (% MFMA peak); decode/scan GB/s (% HBM peak), 1 GPU"
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_HBM_GBS = 8000.0       # HBM3E
PEAK_FP32_TFLOPS = 157.3    # dense fp32 MFMA
# Selective-scan VALU roofline: a state update is one v_exp_f32 (1.8 FMA
# issue slots on gfx950, measured) plus two multiplies and two FMAs, 5.8
# slots; a wave64 VALU op takes one 16-lane slot per SIMD per clock:
# 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz / 5.8 slots.
SCAN_SLOTS_PER_UPDATE = 5.8
PEAK_SCAN_TUPS = 256 * 4 * 16 * 2.4e9 / SCAN_SLOTS_PER_UPDATE / 1e12


def prefill_flops(B, H, S, D):
    # exact count of unmasked (query, key) pairs under the causal mask, two
    # GEMMs of 2*D FLOPs each per pair
    return 4.0 * B * H * D * S * (S + 1) / 2


SPINUP_S = 1.0  # untimed run of each workload before its warmup steps
CPU_BUDGET_S = 3.0  # CPU oracle seconds per secondary workload


def _host_bits(t):
    """A device tensor's storage as the numpy type the oracle takes."""
    import numpy as np
    import torch

    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _timed(fn):
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def _cpu_sample(run, units, per_unit, unit, scale, budget_s, what):
    """cpu_baseline from run(i) -> seconds over units 0, 1, ... until
    budget_s of CPU time or all units are spent; per_unit is the
    algorithmic work (bytes or FLOPs) of one unit."""
    import oracle

    done, elapsed = 0, 0.0
    while elapsed < budget_s and done < units:
        elapsed += run(done)
        done += 1
    return {"value": per_unit * done / elapsed / scale, "unit": unit,
            "cores": oracle.num_threads(), "kind": "port",
            "sample": f"{done} {what} ({elapsed:.1f} s of CPU oracle time)"}


def spin_up(fn, seconds, rotate=1):
    """Run fn, untimed, until `seconds` of wall time have passed. An idle
    MI355X takes tens of milliseconds of load to reach its working clocks;
    without this the first workload's timed steps run partly below them
    (measured: ~605 us against ~555 us steady state for the prefill)."""
    import torch

    t0, i = time.perf_counter(), 0
    while True:
        fn(i % rotate)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= seconds:
                return i


def time_launches(fn, steps, warmup, rotate=1, spinup=None):
    """Spin up, run warmup + steps launches; returns (wall seconds for the
    timed steps, mean seconds per step from one pair of HIP events around
    the timed steps on the current stream). The steps run back to back, as
    a serving loop issues them: a timing marker between steps would add its
    own dispatch latency (some 5 us) to every step."""
    import torch

    spinup = SPINUP_S if spinup is None else spinup
    if spinup > 0:
        spin_up(fn, spinup, rotate)
    for i in range(warmup):
        fn(i % rotate)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        fn(i % rotate)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev = start.elapsed_time(stop) / steps / 1e3
    return wall, ev


def bench_prefill(ops, torch, steps, warmup, B=4, H=32, S=4096, D=128):
    g = torch.Generator(device="cuda").manual_seed(2)
    q, k, v = (torch.randn((B, H, S, D), device="cuda", generator=g).mul_(0.5).to(torch.bfloat16)
               for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")

    def step(_):
        ops.attention(q, k, v, causal=True, out=out, lse=lse)

    wall, ev = time_launches(step, steps, warmup)
    flops = prefill_flops(B, H, S, D)
    return {"q": q, "k": k, "v": v, "wall": wall, "event_s": ev, "flops": flops}


def bench_htile_reference(torch, steps, warmup, B=1, H=32, S=4096, D=128):
    """The reference's own tile program: the flash-attention HTile program
    (f16, non-causal MHA [1, 32, 4096, 128], 128-row query blocks, 64-key
    blocks, pipeline_stages 2) bound by this backend's HTile front end
    (neptune_hip.htile.translate_source) and launched as the reference's
    functional test launches the generated kernel,
    flash_attention_htile[(32, 32, 1)](q, k, v, out)
    (tests/test_translators.py:184-194). The program text comes from
    tests/htile_gen.py, which writes it for a given shape and dtype."""
    if str(ROOT / "tests") not in sys.path:
        sys.path.insert(0, str(ROOT / "tests"))
    from htile_gen import program

    from neptune_hip import htile

    kern = htile.translate_source(program(B=B, H=H, S=S, D=D, dtype="f16")).flash_attention_htile
    grid = kern.program.grid
    g = torch.Generator(device="cuda").manual_seed(6)
    q, k, v = (torch.randn((B, H, S, D), device="cuda", generator=g).to(torch.float16)
               for _ in range(3))
    out = torch.empty_like(q)
    launch = kern[grid]
    wall, ev = time_launches(lambda _: launch(q, k, v, out), steps, warmup)
    flops = 4.0 * B * H * S * S * D  # every (query, key) pair: two GEMMs of 2 D FLOPs
    name = (f"reference tile program flash_attention_htile f16 [{B},{H},{S},{D}] non-causal, "
            f"grid {grid} via htile.translate_source")

    def cpu(budget_s):
        """The oracle (HTile policy) on whole heads of the same inputs."""
        import oracle

        per_head = flops / (B * H)

        def run(i):
            b, h = divmod(i, H)
            qs, ks, vs = (_host_bits(t[b:b + 1, h:h + 1]) for t in (q, k, v))
            t0 = time.perf_counter()
            oracle.attn_fwd(qs, ks, vs, oracle.F16)
            return time.perf_counter() - t0

        return _cpu_sample(run, B * H, per_head, "TFLOP/s", 1e12, budget_s,
                           "heads of the same tile-program attention")

    return name, wall, ev, flops, cpu


def bench_decode(ops, torch, steps, warmup, fp8):
    B, Hq, Hk, L, D, splits = 16, 32, 8, 32768, 128, 16
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((B, Hq, D), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((B, Hk, L, D), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((B, Hk, L, D), device="cuda", generator=g).to(torch.bfloat16)
    ks = vs = None
    if fp8:
        k, ks = ops.kv_quantize_fp8(k)
        v, vs = ops.kv_quantize_fp8(v)
    ws = torch.empty(ops.decode_workspace_bytes(q, k, num_splits=splits, fp8=fp8),
                     dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    def step(_):
        ops.decode_splitk(q, k, v, k_scale=ks, v_scale=vs, num_splits=splits, workspace=ws)

    wall, ev = time_launches(step, steps, warmup)
    kv_bytes = 2 * B * Hk * L * D * (1 if fp8 else 2)
    scale_bytes = 2 * B * Hk * (L // 64) * 4 if fp8 else 0
    nbytes = kv_bytes + scale_bytes + 2 * B * Hq * D * 2
    name = "config5 fp8-KV split-K GQA decode" if fp8 else "config3 bf16 split-K GQA decode"

    def cpu(budget_s):
        """The oracle on whole batch rows of the same inputs, in order."""
        import oracle

        kvt = oracle.FP8 if fp8 else oracle.BF16
        per_row = nbytes / B

        def run(b):
            sl = slice(b, b + 1)
            args = [_host_bits(t[sl]) for t in (q, k, v)]
            sc = [_host_bits(t[sl]) for t in (ks, vs)] if fp8 else [None, None]
            t0 = time.perf_counter()
            oracle.decode_splitk(*args, kvt, *sc, num_splits=splits)
            return time.perf_counter() - t0

        return _cpu_sample(run, B, per_row, "GB/s", 1e9, budget_s,
                           "batch rows of the same decode")

    return name, wall, ev, nbytes, cpu


def bench_decode_paged(ops, torch, steps, warmup, page_size=64, fp8=False):
    """Config 3 (fp8: config 5) with K/V held in a shuffled page pool and a
    random block table: same bytes as contiguous decode, scattered in HBM.
    bf16 pages are token-major [pages, page_size, Hkv, D] (seen as
    [pages, Hkv, page_size, D]). fp8 pages are head-major
    [pages, Hkv, page_size, D], hold finite positive E4M3 codes and one scale
    per (page, kv head): a token-major fp8 page leaves each kv head only a
    128-byte run per token, which HBM serves at about 0.66 of peak against
    0.73 for head-major pages."""
    B, Hq, Hk, L, D, splits = 16, 32, 8, 32768, 128, 16
    per = L // page_size
    npages = B * per
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((B, Hq, D), device="cuda", generator=g).to(torch.bfloat16)
    pshape = (npages, Hk, page_size, D) if fp8 else (npages, page_size, Hk, D)
    if fp8:
        k_pool = torch.randint(0, 0x7f, pshape, device="cuda", generator=g, dtype=torch.uint8)
        v_pool = torch.randint(0, 0x7f, pshape, device="cuda", generator=g, dtype=torch.uint8)
        scales = {n: torch.rand((npages, Hk), device="cuda", generator=g) / 448 + 1e-3
                  for n in ("k_scales", "v_scales")}
    else:
        k_pool = torch.randn(pshape, device="cuda", generator=g).to(torch.bfloat16)
        v_pool = torch.randn(pshape, device="cuda", generator=g).to(torch.bfloat16)
        scales = {}
    kp, vp = (k_pool, v_pool) if fp8 else (k_pool.permute(0, 2, 1, 3), v_pool.permute(0, 2, 1, 3))
    table = torch.randperm(npages, device="cuda", generator=g).to(torch.int32).view(B, per)
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    k_meta = torch.empty((B, Hk, L, D), dtype=torch.bfloat16, device="meta")
    ws = torch.empty(ops.decode_workspace_bytes(q, k_meta, num_splits=splits),
                     dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    def step(_):
        ops.decode_paged(q, kp, vp, table, lens, max_seq_len=L, num_splits=splits, workspace=ws,
                         **scales)

    wall, ev = time_launches(step, steps, warmup)
    esize = 1 if fp8 else 2
    nbytes = 2 * B * Hk * L * D * esize + B * per * 4 + 2 * B * Hq * D * 2
    if fp8:
        nbytes += 2 * B * per * Hk * 4  # the scales of every page read

    def cpu(budget_s):
        """The oracle's paged decode on one sequence at a time: that
        sequence's pages (as the table orders them) form the pool it reads."""
        import oracle

        def run(b):
            pages = table[b].long()
            kq, vq = (_host_bits(pool.index_select(0, pages)) for pool in (k_pool, v_pool))
            if not fp8:  # token-major storage, read through [pages, Hk, page, D] views
                kq, vq = kq.transpose(0, 2, 1, 3), vq.transpose(0, 2, 1, 3)
            sc = {n: _host_bits(t.index_select(0, pages)) for n, t in scales.items()}
            tab = np.arange(per, dtype=np.int32)[None, :]
            t0 = time.perf_counter()
            oracle.decode_paged(_host_bits(q[b:b + 1]), kq, vq, tab, np.array([L], np.int32),
                                max_seq_len=L, num_splits=splits, **sc)
            return time.perf_counter() - t0

        return _cpu_sample(run, B, nbytes / B, "GB/s", 1e9, budget_s,
                           "sequences of the same paged decode")

    if fp8:
        return ("config5 fp8-KV split-K GQA decode, paged KV (64-token head-major pages)", wall,
                ev, nbytes, cpu)
    return "config3 bf16 split-K GQA decode, paged KV (64-token pages)", wall, ev, nbytes, cpu


def bench_scan(ops, torch, steps, warmup, rotate=2):
    Bn, L, Dm, N = 4, 2048, 5120, 16
    sets = []
    for r in range(rotate):
        g = torch.Generator(device="cuda").manual_seed(100 + r)

        def rn(shape, dtype=torch.bfloat16):
            return torch.randn(shape, device="cuda", generator=g).to(dtype)

        u, dr, z = rn((Bn, Dm, L)), rn((Bn, Dm, L)), rn((Bn, Dm, L))
        Bm, Cm = rn((Bn, N, L)), rn((Bn, N, L))
        A = -torch.exp(rn((Dm, N), torch.float32))
        Dv, bias = rn((Dm,), torch.float32), rn((Dm,), torch.float32)
        sets.append((u, dr, A, Bm, Cm, Dv, z, bias))

    def step(i):
        ops.selective_scan(*sets[i])

    wall, ev = time_launches(step, steps, warmup, rotate)
    nbytes = 4 * Bn * Dm * L * 2 + 2 * Bn * N * L * 2 + Dm * N * 4 + 2 * Dm * 4

    def cpu(budget_s, chunk=256):
        """The oracle (fp64 recurrence) on 256-channel blocks of the first
        input set, in order; bytes counted per channel (8 B per step, plus
        its A, D and bias)."""
        import oracle

        u, dr, A, Bm, Cm, Dv, z, bias = sets[0]
        Bh, Ch = _host_bits(Bm), _host_bits(Cm)
        per_chunk = chunk * (L * 8 + N * 4 + 8)

        def run(i):
            b, c0 = divmod(i * chunk, Dm)
            ch = slice(c0, c0 + chunk)
            args = [_host_bits(t[b:b + 1, ch]) for t in (u, dr)]
            t0 = time.perf_counter()
            oracle.selective_scan(*args, _host_bits(A[ch]), Bh[b:b + 1], Ch[b:b + 1],
                                  _host_bits(Dv[ch]), _host_bits(z[b:b + 1, ch]),
                                  _host_bits(bias[ch]))
            return time.perf_counter() - t0

        return _cpu_sample(run, Bn * Dm // chunk, per_chunk, "GB/s", 1e9, budget_s,
                           "256-channel blocks of the same scan")

    return "config4 Mamba-1 selective scan", wall, ev, nbytes, cpu


def scan_valu_roofline(ev, Bn=4, L=2048, Dm=5120, N=16):
    """The scan against its vector-ALU bound (state updates per second)."""
    tups = Bn * Dm * L * N / ev / 1e12
    return {"bound": "valu", "achieved": round(tups, 3), "peak": round(PEAK_SCAN_TUPS, 3),
            "unit": "T state-updates/s", "frac": round(tups / PEAK_SCAN_TUPS, 4),
            "basis": f"{SCAN_SLOTS_PER_UPDATE} VALU issue slots per state update (v_exp_f32 "
                     "1.8 + two mul + two fma), 16 lanes x 1024 SIMDs x 2.4 GHz"}


def bench_config1(ops, torch, steps, warmup, per_graph=100):
    """Config 1: single-head fp32 attention B=1 H=1 S=128 D=64, non-causal,
    the reference's CPU-runnable case. One launch is a few microseconds, far
    less than the host's per-call cost, so a step replays a HIP graph of
    `per_graph` captured launches and the figures are per launch."""
    S, D = 128, 64
    g = torch.Generator(device="cuda").manual_seed(1)
    q, k, v = (torch.randn((1, 1, S, D), device="cuda", generator=g) for _ in range(3))
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # the first call loads the library off the capture
        ops.attention(q, k, v, out=out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            ops.attention(q, k, v, out=out)

    wall, ev = time_launches(lambda _: graph.replay(), steps, warmup)
    wall, ev = wall / per_graph, ev / per_graph
    flops = 4.0 * S * S * D

    def cpu(budget_s):
        import oracle

        qh, kh, vh = (_host_bits(t) for t in (q, k, v))
        return _cpu_sample(lambda _: _timed(lambda: oracle.attn_fwd(qh, kh, vh, oracle.F32)),
                           10**9, flops, "TFLOP/s", 1e12, budget_s,
                           "repeated runs of the same config-1 attention")

    return "config1 fp32 attention B1 H1 S128 D64 (latency-bound)", wall, ev, flops, cpu


def cpu_baseline_prefill(res, budget_s=15.0, max_slices=64):
    """CPU oracle (HTile policy, OpenMP) on whole (batch, head) slices of the
    same inputs, in order, until the time budget is spent."""
    import numpy as np
    import torch

    import oracle

    B, H, S, D = res["q"].shape
    per_head = prefill_flops(1, 1, S, D)

    def b16(t):
        return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

    done, elapsed = 0, 0.0
    while elapsed < budget_s and done < min(max_slices, B * H):
        b, h = divmod(done, H)
        sl = (slice(b, b + 1), slice(h, h + 1))
        qs, ks, vs = b16(res["q"][sl]), b16(res["k"][sl]), b16(res["v"][sl])
        t0 = time.perf_counter()
        oracle.attn_fwd(qs, ks, vs, oracle.BF16, causal=True)
        elapsed += time.perf_counter() - t0
        done += 1
    return {
        "value": per_head * done / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": oracle.num_threads(),
        "kind": "port",
        "sample": f"{done} of {B * H} (batch, head) slices of the same causal prefill "
                  f"({elapsed:.1f} s of CPU oracle time)",
    }


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.txt"
# roofline.traffic is not measured by this run: it is the byte count of a
# separate rocprofv3 counter pass, summarised in that file
TRAFFIC_SOURCE = ("profiles/hbm_traffic.txt: L2 fetch and write bytes to the data fabric (HBM or "
                  "the MALL in front of it) from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes "
                  "over the same workload, scaled by a 1 GiB copy's counts; not this run")


def measured_traffic():
    """Bytes per launch between L2 and the data fabric (HBM, or the MALL in
    front of it) per workload, from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes summarised in profiles/hbm_traffic.txt (lines 'workload bytes');
    {} when that summary is absent."""
    out = {}
    if TRAFFIC_FILE.is_file():
        for line in TRAFFIC_FILE.read_text().splitlines():
            parts = line.split("#", 1)[0].split()
            if len(parts) == 2:
                out[parts[0]] = float(parts[1])
    return out


def bench_copy(torch, steps, warmup, nbytes=1 << 30):
    """A plain device-to-device copy of known size: the calibration kernel
    for the HBM byte counters."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    wall, ev = time_launches(lambda _: dst.copy_(src), steps, warmup)
    return "copy 1 GiB", wall, ev, 2 * nbytes, None


def bench_gemm(torch, steps, warmup, n=8192):
    """A bf16 n^3 GEMM through torch.matmul (hipBLASLt): the vendor's own dense
    MFMA rate on this box, under the same power cap as the prefill. It
    calibrates what fraction of the nominal MFMA peak dense bf16 work reaches
    here; the default run carries it as a secondary entry and puts the
    prefill's rate over it on the headline (prefill_over_gemm)."""
    a = torch.randn((n, n), device="cuda").to(torch.bfloat16)
    b = torch.randn((n, n), device="cuda").to(torch.bfloat16)
    c = torch.empty((n, n), device="cuda", dtype=torch.bfloat16)
    wall, ev = time_launches(lambda _: torch.matmul(a, b, out=c), steps, warmup)
    return f"bf16 GEMM {n}^3 (torch.matmul, hipBLASLt)", wall, ev, 2.0 * n ** 3, None


def mfma_entry(name, wall, ev, flops, steps, cpu=None):
    """A 16-bit MFMA-bound workload (the same dense peak for f16 and bf16)."""
    tf = flops / ev / 1e12
    return {
        "workload": name,
        "value": round(flops * steps / wall / 1e12, 1),
        "unit": "TFLOP/s",
        "us_per_step": round(ev * 1e6, 2),
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


def hbm_entry(key, name, wall, ev, nbytes, steps, traffic, cpu=None):
    gbs = nbytes / ev / 1e9
    return {
        "workload": name,
        "value": round(nbytes * steps / wall / 1e9, 1),
        "unit": "GB/s",
        "us_per_step": round(ev * 1e6, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": traffic.get(key),
                     "traffic_source": TRAFFIC_SOURCE if key in traffic else None},
        "cpu_baseline": cpu,
    }


def config1_entry(name, wall, ev, flops, steps, cpu=None):
    tf = flops / ev / 1e12
    return {
        "workload": name,
        "value": round(flops * steps / wall / 1e12, 4),
        "unit": "TFLOP/s",
        "us_per_step": round(ev * 1e6, 2),
        "roofline": {"bound": "mfma", "achieved": round(tf, 4), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / PEAK_FP32_TFLOPS, 6),
                     "traffic": None},
        "cpu_baseline": cpu,
    }


def short_kernel_name(name):
    """A kernel name without its namespaces, return type and argument list,
    template arguments kept (they tell the instantiations apart)."""
    n = name.replace("void ", "").replace("(anonymous namespace)::", "").replace("neptune::", "")
    depth = 0
    for i, ch in enumerate(n):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            n = n[:i]
            break
    return n[:90]


def trace_summary(path, last):
    """Markdown table of a rocprofv3 kernel-trace CSV: per kernel, every
    launch, and the last `last` launches alone (the timed steps of a
    single-workload run, after its spin-up and warmup launches)."""
    import csv

    runs = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            t0, t1 = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
            runs.setdefault(row["Kernel_Name"], []).append((t0, t1 - t0))
    print(f"| kernel | launches | avg µs (all) | last {last}: avg µs | min µs | max µs |")
    print("|---|---|---|---|---|---|")
    for name, rs in sorted(runs.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        rs.sort()
        tail = [d / 1e3 for _, d in rs[-last:]]
        allv = sum(d for _, d in rs) / len(rs) / 1e3
        print(f"| `{short_kernel_name(name)}` | {len(rs)} | {allv:.1f} | {sum(tail) / len(tail):.1f} | "
              f"{min(tail):.1f} | {max(tail):.1f} |")


def main():
    global SPINUP_S
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the decode/scan configurations")
    ap.add_argument("--workload", default="all",
                    choices=["all", "prefill", "decode", "decode_fp8", "decode_paged",
                             "decode_paged_fp8", "scan", "config1", "copy", "gemm",
                             "htile_ref"],
                    help="run one configuration only (for profiling); 'copy' is a plain "
                         "1 GiB device copy used to calibrate HBM byte counters, 'gemm' a "
                         "bf16 8192^3 torch.matmul that calibrates the dense MFMA rate")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--spinup", type=float, default=SPINUP_S,
                    help="untimed seconds of each workload before its warmup steps "
                         "(0 for counter-collection runs, which need no steady clocks)")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel-trace CSV (no GPU work) and exit")
    ap.add_argument("--last", type=int, default=20,
                    help="with --trace-summary: launches per kernel counted as timed steps")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.last)
        return
    SPINUP_S = args.spinup

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this backend runs on one GPU only: the multi-GPU "
                          "sharding of this path is a design note, no collectives are built",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from neptune_hip import ops

    torch.cuda.set_device(0)
    arch = torch.cuda.get_device_properties(0).gcnArchName
    print(f"# device {torch.cuda.get_device_name(0)} {arch}", file=sys.stderr, flush=True)
    traffic = measured_traffic()

    single = {
        "decode": lambda: bench_decode(ops, torch, args.steps, args.warmup, fp8=False),
        "decode_fp8": lambda: bench_decode(ops, torch, args.steps, args.warmup, fp8=True),
        "decode_paged": lambda: bench_decode_paged(ops, torch, args.steps, args.warmup),
        "decode_paged_fp8": lambda: bench_decode_paged(ops, torch, args.steps, args.warmup,
                                                       fp8=True),
        "scan": lambda: bench_scan(ops, torch, args.steps, args.warmup),
        "copy": lambda: bench_copy(torch, args.steps, args.warmup),
        "gemm": lambda: bench_gemm(torch, args.steps, args.warmup),
        "config1": lambda: bench_config1(ops, torch, args.steps, args.warmup),
        "htile_ref": lambda: bench_htile_reference(torch, args.steps, args.warmup),
    }
    if args.workload in single:
        name, wall, ev, work, cpu = single[args.workload]()
        if args.workload == "config1":
            entry = config1_entry(name, wall, ev, work, args.steps)
        elif args.workload in ("gemm", "htile_ref"):
            entry = mfma_entry(name, wall, ev, work, args.steps)
        else:
            entry = hbm_entry(args.workload, name, wall, ev, work, args.steps, traffic)
        if args.workload == "scan":
            entry["roofline_valu"] = scan_valu_roofline(ev)
        print(json.dumps(entry), flush=True)
        return

    res = bench_prefill(ops, torch, args.steps, args.warmup)
    value = res["flops"] * args.steps / res["wall"] / 1e12
    achieved = res["flops"] / res["event_s"] / 1e12
    print(f"# prefill done: {res['event_s'] * 1e6:.1f} us/launch, {achieved:.1f} TFLOP/s",
          file=sys.stderr, flush=True)

    secondary = []
    gemm_tf = None
    if not args.no_secondary and args.workload == "all":
        del res["k"], res["v"]
        torch.cuda.empty_cache()
        sec_steps, sec_warm = min(args.steps, 20), min(args.warmup, 3)
        for key, fn in (("decode", lambda: bench_decode(ops, torch, sec_steps, sec_warm, False)),
                        ("decode_fp8", lambda: bench_decode(ops, torch, sec_steps, sec_warm,
                                                            True)),
                        ("decode_paged", lambda: bench_decode_paged(ops, torch, sec_steps,
                                                                    sec_warm)),
                        ("decode_paged_fp8", lambda: bench_decode_paged(ops, torch, sec_steps,
                                                                        sec_warm, fp8=True)),
                        ("scan", lambda: bench_scan(ops, torch, sec_steps, sec_warm)),
                        ("config1", lambda: bench_config1(ops, torch, sec_steps, sec_warm)),
                        ("htile_ref", lambda: bench_htile_reference(torch, sec_steps, sec_warm)),
                        ("gemm", lambda: bench_gemm(torch, sec_steps, sec_warm))):
            name, wall, ev, work, cpu_fn = fn()
            cpu = None if (args.no_cpu or cpu_fn is None) else cpu_fn(CPU_BUDGET_S)
            if key in ("htile_ref", "gemm"):
                secondary.append(mfma_entry(name, wall, ev, work, sec_steps, cpu))
                if key == "gemm":
                    gemm_tf = work / ev / 1e12
                print(f"# {name}: {ev * 1e6:.1f} us, {work / ev / 1e12:.1f} TFLOP/s",
                      file=sys.stderr, flush=True)
            elif key == "config1":  # wall and ev are per launch: steps x launches per graph
                secondary.append(config1_entry(name, wall, ev, work, sec_steps, cpu))
                print(f"# {name}: {ev * 1e6:.1f} us, {work / ev / 1e12:.3f} TFLOP/s",
                      file=sys.stderr, flush=True)
            else:
                secondary.append(hbm_entry(key, name, wall, ev, work, sec_steps, traffic, cpu))
                if key == "scan":
                    secondary[-1]["roofline_valu"] = scan_valu_roofline(ev)
                print(f"# {name}: {ev * 1e6:.1f} us, {work / ev / 1e9:.0f} GB/s",
                      file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
        # the prefill inputs are needed again for the CPU sample
        g = torch.Generator(device="cuda").manual_seed(2)
        shape = res["q"].shape
        res["q"], res["k"], res["v"] = (
            torch.randn(shape, device="cuda", generator=g).mul_(0.5).to(torch.bfloat16)
            for _ in range(3))

    cpu = None if args.no_cpu else cpu_baseline_prefill(res)
    # the prefill's rate over the vendor GEMM's, both timed in this run: how
    # close the fused attention (softmax included) comes to dense bf16 MFMA
    # work under the same power cap
    prefill_over_gemm = None if gemm_tf is None else {
        "ratio": round(achieved / gemm_tf, 4), "gemm_achieved": round(gemm_tf, 1),
        "gemm_frac": round(gemm_tf / PEAK_BF16_TFLOPS, 4), "unit": "TFLOP/s",
        "gemm": "bf16 8192^3 torch.matmul (hipBLASLt), secondary entry 'gemm'"}

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "spinup_s": SPINUP_S,
        "ms_per_step": round(res["wall"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config2 causal prefill flash-attention bf16 in / fp32 "
                               "accumulate, output bf16 + per-row LSE fp32",
                   "batch": 4, "heads": 32, "seq_len": 4096, "head_dim": 128,
                   "causal": True, "flops_per_step": res["flops"]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic.get("prefill"),
                     "traffic_source": TRAFFIC_SOURCE if "prefill" in traffic else None},
        "prefill_over_gemm": prefill_over_gemm,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
