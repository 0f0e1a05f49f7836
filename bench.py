#!/usr/bin/env python3
"""Benchmark of the fused-attention hot path on one MI355X.

Headline (the benchmark metric, config C2): Llama-3-8B GQA decode
(32 query / 8 KV heads, head_dim 128, 4096-position f16 cache, batch 1). A
step is one decoded token through a 32-layer stack: 32 decode-attention
launches, each over its own layer's KV cache, so the 537 MB touched per step
is more than twice the 256 MB Infinity Cache and the bytes come from HBM. The
step is captured once in a HIP graph and replayed (no host work in the timed
region). `value` = algorithmic bytes (2 * kv * tk * hd * 2 per layer, the
reference's bench_attn.rs:167 formula) / step time.

Secondary lines (prefill TFLOP/s, Whisper, batched Q8_0 decode) are measured
the same way and reported under `secondary`. The CPU baseline is the oracle's
C restatement of the reference's scalar decode chain, timed on this host.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
F16_PEAK_TFLOPS = 2500.0     # MI355X dense f16 MFMA, TFLOP/s
LLC_BYTES = 256 * 2 ** 20    # Infinity Cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="", metavar="NAME",
                    help="run one workload alone and print its line, for profiling runs: c2_decode, "
                         "c3_prefill_512, c3_prefill_128, c3_prefill_8192_steady, c4_encoder, c4_cross_decode, "
                         "c4_self_decode_224_f32, c5_q8_batch_decode, practical_peaks, reference_rows")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB a few times (the known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def rotate_layers(bytes_per_layer: int, want: int) -> int:
    """Layers so that one step touches at least 2x the last-level cache."""
    return max(want, math.ceil(2 * LLC_BYTES / max(1, bytes_per_layer)))


class Timer:
    """Captures `fn` (one step) in a HIP graph, checks a replay against the
    eager result, then times `steps` replays with HIP events on the capture
    stream (the stream every launch of the step is made on)."""

    def __init__(self, torch, fn, check=None):
        self.torch = torch
        self.fn = fn
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            eager = fn()  # first call: scratch allocation happens here, outside capture
            torch.cuda.synchronize()
            eager = [t.clone() for t in eager] if eager else []
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=s):
                self.outs = fn()
        torch.cuda.current_stream().wait_stream(s)
        self.stream = s
        self.graph.replay()
        torch.cuda.synchronize()
        if eager:
            for a, b in zip(eager, self.outs):
                if not torch.equal(a, b):
                    raise RuntimeError("graph replay differs from the eager step")

    def time(self, steps: int, warmup: int) -> float:
        torch = self.torch
        for _ in range(warmup):
            self.graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            for _ in range(steps):
                self.graph.replay()
            e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps  # ms per step


def rand_f16(torch, n, gen):
    return torch.randn(n, generator=gen, device="cuda", dtype=torch.float32).to(torch.float16)


def bench_decode_f16(torch, g, heads, kv, hd, tk, cap, scale_q, steps, warmup, layers, f32_cache=False,
                     tiled=False):
    """One decode launch per layer over distinct per-layer caches. tiled: the
    fragment-order f16 cache (llmtie_attn_decode_t16); else the reference
    layout (llmtie_attn_decode_f16 / llmtie_attn_decode)."""
    from ttsxabe_amd.gpu import DecodeScratch, TiledCache16
    gen = torch.Generator(device="cuda").manual_seed(1234)
    esz = 4 if f32_cache else 2
    bytes_layer = 2 * kv * tk * hd * esz
    L = rotate_layers(2 * kv * cap * hd * esz, layers)
    qs = [torch.randn(heads * hd, generator=gen, device="cuda") for _ in range(L)]
    scratch = DecodeScratch()
    scale = hd ** -0.5
    if tiled:
        caches = []
        for _ in range(L):
            c = TiledCache16(kv, hd, cap, zero=False)
            c.data.copy_(rand_f16(torch, c.data.numel(), gen))
            caches.append(c)

        def step():
            return [g.attn_decode_t16(qs[l], caches[l], heads, tk, scale, scale_q, scratch) for l in range(L)]
    else:
        if f32_cache:
            ks = [torch.randn(kv * cap * hd, generator=gen, device="cuda") for _ in range(L)]
            vs = [torch.randn(kv * cap * hd, generator=gen, device="cuda") for _ in range(L)]
        else:
            ks = [rand_f16(torch, kv * cap * hd, gen) for _ in range(L)]
            vs = [rand_f16(torch, kv * cap * hd, gen) for _ in range(L)]
        fn_ = g.attn_decode if f32_cache else g.attn_decode_f16

        def step():
            return [fn_(qs[l], ks[l], vs[l], heads, kv, hd, tk, cap, scale, scale_q, scratch) for l in range(L)]

    ms = Timer(torch, step).time(steps, warmup)
    per_launch_us = ms * 1e3 / L
    gbs = bytes_layer / (per_launch_us * 1e-6) / 1e9
    return dict(layers=L, layout="tiled f16" if tiled else ("reference f32" if f32_cache else "reference f16"),
                ms_per_step=ms, us_per_launch=per_launch_us, bytes_per_launch=bytes_layer, gbs=gbs,
                frac=gbs / HBM_PEAK_GBS)


def bench_prefill(torch, g, tq, heads, kv, hd, steps, warmup, layers, tiled=True):
    """Causal GQA prefill of tq tokens, one launch per layer over distinct
    per-layer caches (tiled: llmtie_flash_attn_t16; else llmtie_flash_attn_f16)."""
    from ttsxabe_amd.gpu import TiledCache16
    gen = torch.Generator(device="cuda").manual_seed(99)
    cap = tq
    flop = 4 * hd * heads * (tq * (tq + 1) // 2)  # bench_flash.rs:107-112, causal
    L = max(1, min(layers, rotate_layers(2 * kv * cap * hd * 2 + 2 * tq * heads * hd * 4, layers)))
    qs = [torch.randn(tq * heads * hd, generator=gen, device="cuda") for _ in range(L)]
    scale = hd ** -0.5
    if tiled:
        caches = []
        for _ in range(L):
            c = TiledCache16(kv, hd, cap, zero=False)
            c.data.copy_(rand_f16(torch, c.data.numel(), gen))
            caches.append(c)

        def step():
            return [g.flash_attn_t16(qs[l], caches[l], tq, 0, heads, scale, True) for l in range(L)]
    else:
        ks = [rand_f16(torch, kv * cap * hd, gen) for _ in range(L)]
        vs = [rand_f16(torch, kv * cap * hd, gen) for _ in range(L)]

        def step():
            return [g.flash_attn_f16(qs[l], ks[l], vs[l], tq, 0, heads, kv, hd, cap, scale, True) for l in range(L)]

    ms = Timer(torch, step).time(steps, warmup)
    us = ms * 1e3 / L
    tf = flop / (us * 1e-6) / 1e12
    return dict(tq=tq, layers=L, layout="tiled f16" if tiled else "reference f16", us_per_launch=us,
                flop_per_launch=flop, tflops=tf, frac=tf / F16_PEAK_TFLOPS)


def bench_encoder(torch, g, t, heads, hd, steps, warmup, layers):
    gen = torch.Generator(device="cuda").manual_seed(7)
    d = heads * hd
    flop = 4 * hd * heads * t * t  # non-causal
    L = rotate_layers(t * 3 * d * 4, layers)
    qkvs = [torch.randn(t * 3 * d, generator=gen, device="cuda") for _ in range(L)]
    scale = hd ** -0.5

    def step():
        return [g.flash_attn_rows(qkvs[l], t, heads, hd, scale) for l in range(L)]

    ms = Timer(torch, step).time(steps, warmup)
    us = ms * 1e3 / L
    tf = flop / (us * 1e-6) / 1e12
    return dict(layers=L, us_per_launch=us, flop_per_launch=flop, tflops=tf, frac=tf / F16_PEAK_TFLOPS)


def bench_q8_batch(torch, g, steps, warmup):
    """C5: 32 sequences, one launch over a tiled Q8_0 cache; lengths from the
    seeded U[256, 8192] draw. Eight layers' caches (4.6 GB, far beyond the
    LLC) are decoded in turn, one launch each, per graph replay, as a model's
    layers are: with fewer launches per replay the replay's own gap would be
    spread over too few of them."""
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    from tests import configs
    nseq, heads, kv, hd, cap = 32, 32, 8, 128, 8192
    tk = configs.c5_lengths(nseq=nseq)
    bytes_layer = 2 * kv * (hd + 2 * hd // 32) * int(tk.sum())  # 272 * 8 * sum(tk)
    L = max(8, math.ceil(2 * LLC_BYTES / bytes_layer))
    gen = torch.Generator(device="cuda").manual_seed(5)
    caches = []
    nb = hd // 32
    for _ in range(L):
        c = KvCacheQ8(nseq, kv, hd, cap)
        nblocks = nseq * kv * (cap // 32)
        blocks = c.data.view(nblocks, -1)
        blocks[:, : 64 * hd].copy_(torch.randint(-128, 128, (nblocks, 64 * hd), generator=gen, device="cuda",
                                                 dtype=torch.int8))
        sc = (torch.randn(nblocks, 64 * nb, generator=gen, device="cuda").abs() * 0.02).half()
        blocks[:, 64 * hd:].copy_(sc.view(torch.int8))
        caches.append(c)
    q = [torch.randn(nseq * heads * hd, generator=gen, device="cuda") for _ in range(L)]
    tk_d = torch.from_numpy(tk).to("cuda")
    slot_d = torch.arange(nseq, dtype=torch.int32, device="cuda")
    scratch = DecodeScratch()

    def step():
        return [g.attn_decode_q8_batch(q[l], caches[l], tk_d, slot_d, cap, heads, hd ** -0.5, False, scratch)
                for l in range(L)]

    ms = Timer(torch, step).time(steps, warmup)
    us = ms * 1e3 / L
    gbs = bytes_layer / (us * 1e-6) / 1e9
    return dict(layers=L, us_per_launch=us, bytes_per_launch=bytes_layer, sum_tk=int(tk.sum()), gbs=gbs,
                frac=gbs / HBM_PEAK_GBS, tokens_per_s=nseq / (us * 1e-6))


# The reference's own published rows for this path (one Quadro RTX 8000;
# docs/KERNELS.md:1396-1403, :1253-1256, docs/BENCHMARKS.md:2197-2199), as
# (name, kind, shape, published ms). Decode rows are ms per 32 layers of one
# step; prefill rows are ms per layer.
REFERENCE_ROWS = [
    ("chat 8B decode, 128 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=128), 0.42),
    ("chat 8B decode, 512 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=512), 0.45),
    ("chat 8B decode, 1024 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=1024), 0.60),
    ("chat 8B decode, 2048 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=2048), 1.17),
    ("chat 8B decode, 4096 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=4096), 1.522),
    ("chat 8B decode, 8192 ctx", "decode", dict(heads=32, kv=8, hd=128, tk=8192), 2.548),
    ("translator 13B decode, 128 ctx", "decode", dict(heads=40, kv=40, hd=128, tk=128), 0.44),
    ("translator 13B decode, 1024 ctx", "decode", dict(heads=40, kv=40, hd=128, tk=1024), 1.61),
    ("translator 13B decode, 4000 ctx", "decode", dict(heads=40, kv=40, hd=128, tk=4000), 5.390),
    ("Whisper self decode, 40 of 448 (f32 cache)", "decode", dict(heads=20, kv=20, hd=64, tk=40, cap=448, f32=True,
                                                                  scale_q=True), 0.18),
    ("Whisper cross decode, 1500", "decode", dict(heads=20, kv=20, hd=64, tk=1500, scale_q=True), 0.76),
    ("chat 8B prefill, 2048 positions", "prefill", dict(heads=32, kv=8, hd=128, tq=2048), 0.95),
    ("chat 8B prefill, 8192 positions", "prefill", dict(heads=32, kv=8, hd=128, tq=8192), 11.0),
    ("translator 13B prefill, 3968 positions", "prefill", dict(heads=40, kv=40, hd=128, tq=3968), 3.25),
    ("Whisper encoder, 1500 frames", "encoder", dict(t=1500, heads=20, hd=64), 0.43),
]


def bench_reference_rows(torch, g, steps, warmup):
    """Each published row of the reference at its own shape, through the
    drop-in entry points on the reference's own layouts (f16 K [kv][cap][hd],
    V [kv][hd][cap]; the f32 cache where it keeps one), timed as the other
    lines are (HIP-graph replays over caches rotated past the LLC)."""
    out = {}
    for name, kind, c, ref_ms in REFERENCE_ROWS:
        if kind == "decode":
            r = bench_decode_f16(torch, g, c["heads"], c["kv"], c["hd"], c["tk"], c.get("cap", c["tk"]),
                                 c.get("scale_q", False), steps, warmup, 32, f32_cache=c.get("f32", False))
            ms = r["us_per_launch"] * 32 / 1e3
            row = dict(ms_32_layers=round(ms, 4), gbs=round(r["gbs"], 1), frac=round(r["frac"], 4))
        elif kind == "prefill":
            r = bench_prefill(torch, g, c["tq"], c["heads"], c["kv"], c["hd"], max(3, steps // 4), 2,
                              4 if c["tq"] >= 4096 else 32, tiled=False)
            ms = r["us_per_launch"] / 1e3
            row = dict(ms_per_layer=round(ms, 4), tflops=round(r["tflops"], 1), frac=round(r["frac"], 4))
        else:
            r = bench_encoder(torch, g, c["t"], c["heads"], c["hd"], steps, warmup, 32)
            ms = r["us_per_launch"] / 1e3
            row = dict(ms_per_layer=round(ms, 4), tflops=round(r["tflops"], 1), frac=round(r["frac"], 4))
        row["reference_rtx8000_ms"] = ref_ms
        row["speedup_vs_reference"] = round(ref_ms / ms, 2)
        out[name] = row
    return out


def practical_peaks(torch):
    """What this box sustains outside the hot path, measured in the same run
    as context for the spec peaks the fractions use: an 8192^3 f16 GEMM
    through torch.matmul (the vendor GEMM library), a 1 GiB device copy
    (bytes read + written), and this repository's two probes
    (ttsxabe_amd/csrc/peaks.hip): back-to-back 16x16x32 f16 MFMAs from
    registers on every SIMD (the MFMA rate at the clock the part holds under
    dense work; it runs power-limited below its 2.4 GHz peak clock) and a
    streaming read of 1 GiB (the HBM read rate a kernel can reach)."""
    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps * 1e-3
    n = 8192
    x = torch.randn(n, n, device="cuda", dtype=torch.float16)
    y = torch.randn(n, n, device="cuda", dtype=torch.float16)
    t_gemm = timed(lambda: torch.matmul(x, y), 20)
    del x, y
    src = torch.ones(2 ** 29, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    t_copy = timed(lambda: dst.copy_(src), 20)
    del dst
    import ctypes
    from ttsxabe_amd.build import PEAKS_LIB
    pk = ctypes.CDLL(str(PEAKS_LIB))
    pk.llmtie_peak_mfma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    pk.llmtie_peak_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(max(cus, 1) * 8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    iters = 20000
    t_mfma = timed(lambda: pk.llmtie_peak_mfma(st, sink.data_ptr(), cus, iters), 5)
    nbytes = src.numel() * 2
    t_read = timed(lambda: pk.llmtie_peak_read(st, src.data_ptr(), nbytes, sink.data_ptr(), cus * 8), 10)
    return {"f16_gemm_8192_tflops": round(2 * n ** 3 / t_gemm / 1e12, 1),
            "copy_1gib_gbs": round(2 * src.numel() * 2 / t_copy / 1e9, 1),
            "mfma_f16_loop_tflops": round(cus * 8 * iters * 8 * 16384 / t_mfma / 1e12, 1),
            "hbm_read_1gib_gbs": round(nbytes / t_read / 1e9, 1)}


def cpu_baseline(seconds: float):
    """The oracle's restatement of the reference's scalar decode chain
    (crates/llmtie-cuda/tests/kernels.rs:2733-2780 over an f16 cache), on a
    C2 layer-step, at 1 thread, repeated for about `seconds`."""
    import numpy as np
    import oracle
    heads, kv, hd, tk = 32, 8, 128, 4096
    rng = np.random.default_rng(3)
    q = rng.standard_normal(heads * hd, dtype=np.float32)
    k = oracle.f32_to_f16(rng.standard_normal(kv * tk * hd, dtype=np.float32))
    v = oracle.f32_to_f16(rng.standard_normal(kv * tk * hd, dtype=np.float32))
    bytes_layer = 2 * kv * tk * hd * 2
    n = 0
    t0 = time.perf_counter()
    while True:
        oracle.decode_f16(q, k, v, heads, kv, hd, tk, tk, hd ** -0.5, False, threads=1)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    out = dict(value=round(bytes_layer * n / el / 1e9, 4), unit="GB/s", cores=1, kind="port",
               sample=f"{n} C2 decode layer-steps (32/8/128 GQA, 4096-position f16 cache) through the oracle's "
                      f"scalar f32 chain, 1 thread, {el:.1f} s",
               ms_per_layer_step=round(el / n * 1e3, 2))
    # The same chain with the query heads spread over the host's cores
    # (OpenMP), about a fifth of the time budget.
    threads = min(heads, os.cpu_count() or 1)
    if oracle.has_openmp() and threads > 1:
        n2, t0 = 0, time.perf_counter()
        while True:
            oracle.decode_f16(q, k, v, heads, kv, hd, tk, tk, hd ** -0.5, False, threads=threads)
            n2 += 1
            el2 = time.perf_counter() - t0
            if el2 >= seconds / 5:
                break
        out["all_cores"] = dict(value=round(bytes_layer * n2 / el2 / 1e9, 4), unit="GB/s", threads=threads,
                                ms_per_layer_step=round(el2 / n2 * 1e3, 2))
    return out


def cpu_c1(seconds=3.0):
    """Config 1 (f32 causal MHA prefill 8/8/64, 128 tokens) on the CPU path."""
    import oracle
    from tests import configs
    c = configs.c1_cpu()
    flop = 4 * c["hd"] * c["heads"] * (c["t"] * (c["t"] + 1) // 2)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.prefill_f32(c["q"], c["k"], c["v"], c["t"], c["heads"], c["heads"], c["hd"], c["scale"], True, 1)
        n += 1
    el = time.perf_counter() - t0
    return dict(gflops=round(flop * n / el / 1e9, 3), ms=round(el / n * 1e3, 3), threads=1)


def traffic_from_profiles(name: str):
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, calibrated)."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU (--gpus > 1) is out of scope: attention "
                                   "shards by kv head and sequence with no exchange inside attention"}))
        sys.exit(2)
    import torch
    if a.copy_calibration:
        n = a.copy_calibration * 2 ** 20 // 2
        src = torch.ones(n, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 2 * n, "launches": 5}), flush=True)
        return
    from ttsxabe_amd.gpu import Gpu
    g = Gpu(0)
    if a.only:
        only = {
            "c2_decode": lambda: bench_decode_f16(torch, g, 32, 8, 128, 4096, 4096, False, a.steps, a.warmup,
                                                  a.layers, tiled=True),
            "c4_cross_decode": lambda: bench_decode_f16(torch, g, 20, 20, 64, 1500, 1500, True, a.steps, a.warmup,
                                                        a.layers, tiled=True),
            "c4_self_decode_224_f32": lambda: bench_decode_f16(torch, g, 20, 20, 64, 224, 448, True, a.steps,
                                                               a.warmup, a.layers, f32_cache=True),
            "c3_prefill_128": lambda: bench_prefill(torch, g, 128, 32, 8, 128, a.steps, a.warmup, a.layers),
            "c3_prefill_8192_steady": lambda: bench_prefill(torch, g, 8192, 32, 8, 128, 5, 2, 4),
            "c3_prefill_512": lambda: bench_prefill(torch, g, 512, 32, 8, 128, a.steps, a.warmup, a.layers),
            "c3_prefill_512_reference_layout": lambda: bench_prefill(torch, g, 512, 32, 8, 128, a.steps, a.warmup,
                                                                     a.layers, tiled=False),
            "c4_cross_decode_reference_layout": lambda: bench_decode_f16(torch, g, 20, 20, 64, 1500, 1500, True,
                                                                         a.steps, a.warmup, a.layers),
            "c4_encoder": lambda: bench_encoder(torch, g, 1500, 20, 64, a.steps, a.warmup, a.layers),
            "c5_q8_batch_decode": lambda: bench_q8_batch(torch, g, a.steps, a.warmup),
            "practical_peaks": lambda: practical_peaks(torch),
            "reference_rows": lambda: bench_reference_rows(torch, g, a.steps, a.warmup),
        }
        if a.only not in only:
            print(json.dumps({"error": f"--only takes one of {sorted(only)}"}))
            sys.exit(2)
        print(json.dumps({"only": a.only, **only[a.only]()}), flush=True)
        return
    print("bench: C2 decode", file=sys.stderr, flush=True)
    c2 = bench_decode_f16(torch, g, 32, 8, 128, 4096, 4096, False, a.steps, a.warmup, a.layers, tiled=True)
    line = {
        "metric": "decode attn HBM GB/s + prefill attn TFLOP/s (% roofline), 1×MI355X",
        "value": round(c2["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(c2["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) f16 KV caches, f32 queries)",
        "config": {"workload": "C2: Llama-3-8B GQA decode, 32 q / 8 kv heads, head_dim 128, 4096-position f16 "
                               "KV cache (tiled fragment-order layout), batch 1; one step = one token through %d "
                               "layers (distinct caches, HIP-graph replay)" % c2["layers"],
                   "heads": 32, "kv_heads": 8, "head_dim": 128, "context": 4096, "layers": c2["layers"],
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(c2["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(c2["frac"], 4), "traffic": traffic_from_profiles("attn_decode_c2.md"),
                     "kernel": "attn_decode_kernel<128, KV_T16> (split merge by the last-arriving workgroup, one kernel per launch)",
                     "bytes_per_launch": c2["bytes_per_launch"],
                     "us_per_launch": round(c2["us_per_launch"], 3)},
    }
    if not a.no_secondary:
        sec = {}
        steps = max(5, a.steps // 2)
        print("bench: C3 prefill", file=sys.stderr, flush=True)
        for tq in (512, 128):
            sec[f"c3_prefill_{tq}"] = bench_prefill(torch, g, tq, 32, 8, 128, steps, a.warmup, a.layers)
        sec["c3_prefill_512_reference_layout"] = bench_prefill(torch, g, 512, 32, 8, 128, steps, a.warmup, a.layers,
                                                               tiled=False)
        # Four layers a step: one 0.6 ms launch per graph replay would time
        # the replay gaps too.
        sec["c3_prefill_8192_steady"] = bench_prefill(torch, g, 8192, 32, 8, 128, max(3, steps // 5), 2, 4)
        sec["c2_decode_reference_layout"] = bench_decode_f16(torch, g, 32, 8, 128, 4096, 4096, False, steps,
                                                             a.warmup, a.layers)
        print("bench: C4", file=sys.stderr, flush=True)
        sec["c4_encoder"] = bench_encoder(torch, g, 1500, 20, 64, steps, a.warmup, a.layers)
        sec["c4_cross_decode"] = bench_decode_f16(torch, g, 20, 20, 64, 1500, 1500, True, steps, a.warmup,
                                                  a.layers, tiled=True)
        sec["c4_cross_decode_reference_layout"] = bench_decode_f16(torch, g, 20, 20, 64, 1500, 1500, True, steps,
                                                                   a.warmup, a.layers)
        sec["c4_self_decode_224_f32"] = bench_decode_f16(torch, g, 20, 20, 64, 224, 448, True, steps, a.warmup,
                                                         a.layers, f32_cache=True)
        print("bench: C5", file=sys.stderr, flush=True)
        sec["c5_q8_batch_decode"] = bench_q8_batch(torch, g, steps, a.warmup)
        for v in sec.values():
            for k2 in list(v):
                if isinstance(v[k2], float):
                    v[k2] = round(v[k2], 4)
        print("bench: the reference's published shapes", file=sys.stderr, flush=True)
        sec["reference_rows"] = bench_reference_rows(torch, g, steps, a.warmup)
        # The peak the secondary numbers are fractions of, for reading them,
        # and what the box sustains outside the hot path.
        sec["peaks"] = {"hbm_gbs": HBM_PEAK_GBS, "f16_mfma_tflops": F16_PEAK_TFLOPS}
        print("bench: practical peaks", file=sys.stderr, flush=True)
        sec["practical_peaks"] = practical_peaks(torch)
        line["secondary"] = sec
    if not a.no_cpu:
        print("bench: CPU baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
        line["cpu_baseline"]["c1_cpu_prefill_f32"] = cpu_c1()
        line["cpu_baseline"]["host_cpus"] = os.cpu_count()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
