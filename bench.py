"""Benchmark of the MI355X quantized-weight matrix path (one GPU).

A "step" is one pass of the hot path over one batch: one launch of the decode
GEMV (or W8A8 linear) on weights already resident in HBM. The headline workload
is BASELINE.json configs[1]: the group-wise int4 GEMV at the Qwen2.5-1.5B
down-proj shape (M=1, K=8960, N=1536, fp16 x/y, fp16 group scales, g=32).

Timing: W warm-up launches (at least 2000 for the sweep entries, whose
compute-bound GEMMs are still speeding up after 20), then K launches captured
in one HIP graph (so the GPU runs them back to back, free of host launch gaps)
and replayed inside a pair of HIP events recorded on the launch stream;
ms_per_step = region / K.
The weights rotate over enough copies (>= 512 MiB in total) that each launch
streams them from HBM rather than from the 256 MiB Infinity Cache. Bytes are
algorithmic: every operand once (weights + scales + x + y).

One JSON line on stdout; `--sweep` (default on) adds the other BASELINE configs
under "sweep". The CPU baseline times the reference's own AVX2+OpenMP
linear_q4g (oracle/_ref, built from the reference sources) — or the C
restatement when that build is absent — on a bounded sample of the same
workload, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
ROTATE_BYTES = 512 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default="", help="comma list of sweep entries to run (debug)")
    p.add_argument("--shape-sweep", action="store_true",
                   help="only time the dispatch over a grid of common model shapes (one JSON line)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a device-to-device copy of MIB MiB (FETCH_SIZE/WRITE_SIZE calibration)")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def measured_traffic(workload):
    """HBM bytes per launch for `workload` from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(workload, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the path is single-GPU by design", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        a = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n}))
        return

    from nanoinfer_amd import _lib
    from nanoinfer_amd import quant as nq

    lib = _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261201)

    def rnd(shape, std, dtype=torch.float32):
        return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dtype)

    def copies_for(nbytes):
        """Weight copies that make >= 512 MiB; a multiple of --steps when there
        are more copies than steps, so time_graph's windows tile the rotation."""
        c = max(2, math.ceil(ROTATE_BYTES / max(nbytes, 1)))
        if c > args.steps:
            c = math.ceil(c / args.steps) * args.steps
        return c

    def time_graph(launches, steps, warmup, replays=None):
        """launches: zero-arg callables over rotating weight copies (each copy
        one launch's operands). Returns the median ms per launch over timed
        replays of a HIP graph of exactly `steps` back-to-back launches.

        The copies are split into windows of `steps` consecutive launches (one
        graph each; a single window of launches[i % r] when steps >= r) and the
        graphs replay in a cycle, so every launch reads a copy last touched a
        whole rotation (>= 512 MiB of other weights) earlier: the timed reads
        come from HBM, not from the 256 MiB Infinity Cache, whatever `steps`
        is. Each replay is timed on its own between two events on the launch
        stream; at least 5 replays and 50 timed launches."""
        r = len(launches)
        warmup = max(warmup, 10)
        if replays is None:
            replays = max(5, math.ceil(50 / steps))
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for i in range(max(warmup, r)):
                launches[i % r]()
        torch.cuda.synchronize()
        if steps >= r:
            windows = [[launches[i % r] for i in range(steps)]]
        else:
            nw = math.ceil(r / steps)
            windows = [[launches[(j * steps + i) % r] for i in range(steps)] for j in range(nw)]
        graphs = []
        for win in windows:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for f in win:
                    f()
            graphs.append(g)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            for g in graphs:                             # untimed cycle (first-replay setup)
                g.replay()
        torch.cuda.synchronize()
        times = []
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
        with torch.cuda.stream(s):
            for t in range(replays):
                e0, e1 = ev[t]
                e0.record(s)
                graphs[t % len(graphs)].replay()
                e1.record(s)
        torch.cuda.synchronize()
        times = sorted(e0.elapsed_time(e1) / steps for e0, e1 in ev)
        del graphs
        return times[len(times) // 2]

    def stream_ptr():
        return torch.cuda.current_stream().cuda_stream

    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    # ---------------- workloads ----------------------------------------------------------
    def q4g_gemv(m, n, k, g=32):
        x = rnd((m, k), 1.0, torch.float16)
        w = rnd((n, k), 0.02)
        t = nq.quantize_q4g(w, g, scale_dtype=torch.float16)
        del w
        wbytes = t.q.numel() + t.scale.numel() * 2
        nb = wbytes + x.numel() * 2 + m * n * 2
        qs = [t.q] + [t.q.clone() for _ in range(copies_for(wbytes) - 1)]
        ss = [t.scale] + [t.scale.clone() for _ in range(len(qs) - 1)]
        y = torch.empty((m, n), dtype=torch.float16, device=dev)
        wsb = lib.nq_linear_wq_workspace_size(m, n, k)  # split-K planes (0: none)
        work = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev) if wsb else None

        def mk(i):
            return lambda: lib.nq_linear_q4g_ws(P(x), 1, P(qs[i]), P(ss[i]), 1, g, None, P(y), 1, m, n, k,
                                                P(work), wsb, stream_ptr())
        return [mk(i) for i in range(len(qs))], nb, 2 * m * n * k

    def q8_gemv(m, n, k, xdt):
        x = rnd((m, k), 1.0, xdt)
        w = rnd((n, k), 0.02)
        t = nq.quantize_q8(w)
        del w
        wbytes = t.q.numel() + t.scale.numel() * 4
        esz = 2 if xdt == torch.float16 else 4
        nb = wbytes + x.numel() * esz + m * n * esz
        qs = [t.q] + [t.q.clone() for _ in range(copies_for(wbytes) - 1)]
        ss = [t.scale] + [t.scale.clone() for _ in range(len(qs) - 1)]
        y = torch.empty((m, n), dtype=xdt, device=dev)
        dt = 1 if xdt == torch.float16 else 0
        wsb = lib.nq_linear_wq_workspace_size(m, n, k)
        work = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev) if wsb else None

        def mk(i):
            return lambda: lib.nq_linear_q8_ws(P(x), dt, P(qs[i]), P(ss[i]), None, P(y), dt, m, n, k, P(work), wsb,
                                               stream_ptr())
        return [mk(i) for i in range(len(qs))], nb, 2 * m * n * k

    def quantize(kind, n, k, g=32):
        """Load-time weight quantize (quant.cpp:88-108 / :295-321): fp32 [n, k]
        read once, codes + scales written once (q4g: fp16 scales)."""
        ws = [rnd((n, k), 0.02) for _ in range(copies_for(n * k * 4))]
        if kind == "q8":
            q = torch.empty((n, k), dtype=torch.int8, device=dev)
            s = torch.empty(n, dtype=torch.float32, device=dev)
            nb = n * k * 4 + n * k + n * 4

            def mk(i):
                return lambda: lib.nq_quantize_q8(P(ws[i]), n, k, P(q), P(s), stream_ptr())
        else:
            q = torch.empty((n, (k + 1) // 2), dtype=torch.uint8, device=dev)
            s = torch.empty((n, (k + g - 1) // g), dtype=torch.float16, device=dev)
            nb = n * k * 4 + q.numel() + s.numel() * 2

            def mk(i):
                return lambda: lib.nq_quantize_q4g(P(ws[i]), n, k, g, P(q), P(s), 1, stream_ptr())
        return [mk(i) for i in range(len(ws))], nb, 0

    def q8_lmhead_argmax(m, n, k, xdt):
        """LM head with the greedy argmax fused in: no logits are written, so
        the algorithmic bytes are weights + scales + x + the int64 ids."""
        x = rnd((m, k), 1.0, xdt)
        w = rnd((n, k), 0.02)
        t = nq.quantize_q8(w)
        del w
        wbytes = t.q.numel() + t.scale.numel() * 4
        esz = 2 if xdt == torch.float16 else 4
        nb = wbytes + x.numel() * esz + m * 8
        qs = [t.q] + [t.q.clone() for _ in range(copies_for(wbytes) - 1)]
        ss = [t.scale] + [t.scale.clone() for _ in range(len(qs) - 1)]
        ids = torch.empty(m, dtype=torch.int64, device=dev)
        wsb = lib.nq_lm_head_argmax_q8_workspace_size(m, n, k)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
        dt = 1 if xdt == torch.float16 else 0

        def mk(i):
            return lambda: lib.nq_lm_head_argmax_q8(P(x), dt, P(qs[i]), P(ss[i]), None, P(ids), m, n, k, P(ws),
                                                    ws.numel(), stream_ptr())
        return [mk(i) for i in range(len(qs))], nb, 2 * m * n * k

    def w8a8_linear(m, n, k, gemm_only=False):
        x = rnd((m, k), 1.0, torch.float16)
        w = rnd((n, k), 0.02)
        t = nq.quantize_q8(w)
        del w
        wbytes = t.q.numel() + t.scale.numel() * 4
        nb = wbytes + (m * k if gemm_only else 2 * m * k) + 2 * m * n
        qs = [t.q] + [t.q.clone() for _ in range(copies_for(wbytes) - 1)]
        ss = [t.scale] + [t.scale.clone() for _ in range(len(qs) - 1)]
        y = torch.empty((m, n), dtype=torch.float16, device=dev)
        if gemm_only:
            xq, a_s = nq.act_quant(x)
            wsb = lib.nq_gemm_w8a8_workspace_size(m, n, k)
            ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)

            def mk(i):
                return lambda: lib.nq_gemm_w8a8(P(xq), P(a_s), P(qs[i]), P(ss[i]), None, P(y), 1, m, n, k,
                                                P(ws), ws.numel(), 0, stream_ptr())
        else:
            wsb = lib.nq_linear_w8a8_workspace_size(m, n, k)
            ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)

            def mk(i):
                return lambda: lib.nq_linear_w8a8(P(x), 1, P(qs[i]), P(ss[i]), None, P(y), 1, m, n, k,
                                                  P(ws), ws.numel(), 0, stream_ptr())
        return [mk(i) for i in range(len(qs))], nb, 2 * m * n * k

    # Sweep entries warm up for at least 2000 launches: the compute-bound GEMMs
    # read ~4% slower after 20 (config 5a: 42.2 vs 40.6-40.9 us after 2000 or
    # 20000), the latency-bound GEMVs do not change.
    sweep_warmup = max(args.warmup, 2000)

    def entry(name, launches, nb, ops, bound):
        ms = time_graph(launches, args.steps, sweep_warmup)
        gbs = nb / (ms * 1e-3) / 1e9
        tops = ops / (ms * 1e-3) / 1e12
        e = {"name": name, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "TOPS": round(tops, 2),
             "bytes": nb, "ops": ops, "bound": bound,
             "frac": round(gbs / HBM_PEAK_GBS if bound == "hbm"
                           else tops / (FP16_PEAK_TFLOPS if bound == "mfma_f16" else INT8_PEAK_TOPS), 4),
             "warmup": sweep_warmup}
        return e

    if args.shape_sweep:
        print(json.dumps({"shape_sweep": shape_sweep(args, time_graph, q4g_gemv, q8_gemv, w8a8_linear, entry,
                                                     copies_for, stream_ptr)}), flush=True)
        return

    # ---------------- headline: configs[1] int4 GEMV ------------------------------------------
    M, N, K, G = 1, 1536, 8960, 32
    launches, nbytes, ops = q4g_gemv(M, N, K, G)
    ms = time_graph(launches, args.steps, args.warmup)
    del launches
    torch.cuda.empty_cache()
    gbs = nbytes / (ms * 1e-3) / 1e9

    # Context for the headline: one device-to-device copy of the same number of
    # bytes (torch's copy kernel; it reads and writes them), rotated and timed
    # the same way. A single launch that touches ~8 MB is bound by launch and
    # memory latency, not by bandwidth.
    srcs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(copies_for(2 * nbytes))]
    dsts = [torch.empty_like(t) for t in srcs]
    copy_ms = time_graph([lambda i=i: dsts[i].copy_(srcs[i]) for i in range(len(srcs))], args.steps, args.warmup)
    del srcs, dsts
    # The read floor: one streaming read of the same bytes (libnq_bench.so's
    # probe: the GEMV's 16-byte non-temporal loads), rotated the same way, over
    # workgroup sizes and loads in flight per lane; the best is the floor. The
    # best shape again with the headline's 3 KB y store at the end.
    import ctypes
    blib = ctypes.CDLL(os.path.join(ROOT, "nanoinfer_amd", "libnq_bench.so"))
    blib.nq_probe_read_cfg.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    rbytes = (nbytes + 15) // 16 * 16
    rsrc = [torch.empty(rbytes, dtype=torch.uint8, device=dev) for _ in range(copies_for(rbytes))]
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    yout = torch.empty(M * N * 2, dtype=torch.uint8, device=dev)

    def probe(th, u, ob):
        return time_graph([lambda i=i: blib.nq_probe_read_cfg(P(rsrc[i]), rbytes, th, u, P(yout), ob, P(sink),
                                                              stream_ptr())
                           for i in range(len(rsrc))], args.steps, args.warmup)
    probe_sweep = {}
    for th, us in ((256, (1, 2, 4, 8)), (512, (1, 2, 4, 8)), (1024, (1, 2, 4))):
        for u in us:
            probe_sweep[f"{th}x{u}"] = round(probe(th, u, 0) * 1e3, 3)
    best = min(probe_sweep, key=probe_sweep.get)
    read_ms = probe_sweep[best] * 1e-3
    bth, bu = (int(v) for v in best.split("x"))
    read_store_ms = probe(bth, bu, M * N * 2)
    del rsrc
    torch.cuda.empty_cache()

    sweep = []
    if not args.no_sweep:
        only = set(filter(None, args.only.split(",")))

        def want(n):
            return not only or n in only
        if want("q8_gemv_cfg1"):
            sweep.append(entry("q8_gemv_cfg1 M=1 K=896 N=4864 fp32", *q8_gemv(1, 4864, 896, torch.float32), "hbm"))
            torch.cuda.empty_cache()
        if want("lmhead_cfg5b"):
            sweep.append(entry("q8_lmhead_cfg5b M=1 K=1536 N=151936 fp16", *q8_gemv(1, 151936, 1536, torch.float16), "hbm"))
            torch.cuda.empty_cache()
            sweep.append(entry("q8_lmhead_argmax_cfg5b M=1 K=1536 N=151936 fp16 (greedy id, no logits)",
                               *q8_lmhead_argmax(1, 151936, 1536, torch.float16), "hbm"))
        torch.cuda.empty_cache()
        if want("lmhead_prefill"):
            # the LM head over prefill rows: weight-only int8 (fp16 MFMA) against
            # the opt-in W8A8 route on the same codes (use_w8a8_lmhead,
            # cuda_quant.cu:362-372), incl. the activation quant
            for m in (128, 512):
                sweep.append(entry(f"q8_lmhead_prefill M={m} K=1536 N=151936 fp16 (weight-only)",
                                   *q8_gemv(m, 151936, 1536, torch.float16), "mfma_f16"))
                torch.cuda.empty_cache()
                sweep.append(entry(f"w8a8_lmhead_prefill M={m} K=1536 N=151936 fp16 (use_w8a8_lmhead, incl. act quant)",
                                   *w8a8_linear(m, 151936, 1536), "mfma"))
                torch.cuda.empty_cache()
        if want("w8a8_cfg3"):
            for m in (8, 16, 32, 64):
                for nm, (n, k) in (("qo", (1536, 1536)), ("kv", (256, 1536)), ("gateup", (8960, 1536)),
                                   ("down", (1536, 8960))):
                    sweep.append(entry(f"w8a8_cfg3 {nm} M={m} K={k} N={n}", *w8a8_linear(m, n, k), "hbm"))
                    torch.cuda.empty_cache()
        if want("prefill_cfg5a"):
            sweep.append(entry("w8a8_gemm_cfg5a M=2048 K=1536 N=8960 (pre-quantized x)",
                               *w8a8_linear(2048, 8960, 1536, gemm_only=True), "mfma"))
            sweep.append(entry("w8a8_linear_cfg5a M=2048 K=1536 N=8960 (incl. act quant)",
                               *w8a8_linear(2048, 8960, 1536), "mfma"))
        if want("wq_prefill"):
            # weight-only prefill (fp16 activations, fp16 MFMA): the caller-side
            # shape of config 5a in the q8 / q4g quant modes
            sweep.append(entry("q8_weight_only_prefill M=2048 K=1536 N=8960 fp16",
                               *q8_gemv(2048, 8960, 1536, torch.float16), "mfma_f16"))
            torch.cuda.empty_cache()
            sweep.append(entry("q4g_weight_only_prefill M=2048 K=1536 N=8960 g=32 fp16",
                               *q4g_gemv(2048, 8960, 1536, 32), "mfma_f16"))
            torch.cuda.empty_cache()
        if want("wq_batched"):
            # weight-only at a batch of 64 on config 2's weight shape: few weight
            # rows and long K, split K over the workspace
            sweep.append(entry("q8_weight_only_batched M=64 K=8960 N=1536 fp16 (split K)",
                               *q8_gemv(64, 1536, 8960, torch.float16), "hbm"))
            torch.cuda.empty_cache()
            sweep.append(entry("q4g_weight_only_batched M=64 K=8960 N=1536 g=32 fp16 (split K)",
                               *q4g_gemv(64, 1536, 8960, 32), "hbm"))
            torch.cuda.empty_cache()
        if want("quantize"):
            # load-time quantize of the configs' weights, HBM-bound (fp32 in)
            for kind, n, k, nm in (("q8", 151936, 1536, "lm head cfg5b"), ("q8", 8960, 1536, "gate/up cfg5a"),
                                   ("q4g", 1536, 8960, "down cfg2, g=32")):
                sweep.append(entry(f"quantize_{kind} {nm} N={n} K={k} fp32 in", *quantize(kind, n, k), "hbm"))
                torch.cuda.empty_cache()
        if want("decoder_cfg4"):
            sweep.append(decoder_layer_cfg4(rnd, time_graph, args, w8a8_linear, entry))
        torch.cuda.empty_cache()

    # ---------------- CPU baseline (rank 0, N=1) --------------------------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(M, N, K, G, nbytes, args.cpu_seconds)

    out = {
        "metric": "int8/int4 GEMV HBM GB/s (% peak); W8A8 GEMM int8 TOPS (% MFMA peak)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": max(args.warmup, 10),
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, fp16 x/y, fp32 accumulate",
        "data": "synthetic (weights N(0,0.02) quantized on device, x N(0,1)); weights rotated over "
                f">= {ROTATE_BYTES >> 20} MiB of copies, every timed launch on a copy last read a full "
                "rotation earlier",
        "config": {"workload": "configs[1]: int4 group GEMV, Qwen2.5-1.5B down-proj",
                   "M": M, "K": K, "N": N, "group": G, "scale_dtype": "fp16", "x_dtype": "fp16",
                   "algorithmic_bytes": nbytes, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic("q4g_gemv_cfg2")},
        "cpu_baseline": cpu,
        "context": {"copy_same_bytes_us": round(copy_ms * 1e3, 3),
                    "copy_same_bytes_note": "device copy of the headline's algorithmic bytes (read + write), "
                                            "same graph timing",
                    "read_same_bytes_us": round(read_ms * 1e3, 3),
                    "read_same_bytes_GB/s": round(rbytes / (read_ms * 1e-3) / 1e9, 1),
                    "read_same_bytes_note": "nq_probe_read_cfg: one streaming read of the headline's algorithmic "
                                            "bytes with 16-byte non-temporal loads, same graph timing; the best "
                                            f"of the sweep ({best}: lanes per workgroup x loads per lane): the "
                                            "single-launch floor at this size",
                    "read_probe_sweep_us": probe_sweep,
                    "read_then_store_y_us": round(read_store_ms * 1e3, 3),
                    "read_then_store_y_note": f"the {best} probe plus the headline's {M * N * 2}-byte y store"},
        "timing": {"method": "HIP graph of exactly `steps` launches, windows of distinct weight copies "
                             "replayed in a cycle (each copy last read >= 512 MiB earlier); median over timed "
                             "replays, each between two events on the launch stream",
                   "timed_replays": max(5, math.ceil(50 / args.steps)), "warmup_launches": max(args.warmup, 10)},
    }
    if sweep:
        out["sweep"] = sweep
    print(json.dumps(out), flush=True)


# (model, projection, n, k): the projections of Llama-3-8B, Qwen2.5-7B and
# Qwen2.5-1.5B (q|k|v and gate|up fused by rows as this library runs them) and
# two LM heads, none of which the dispatch thresholds were tuned on except
# Qwen2.5-1.5B's.
SWEEP_SHAPES = [
    ("llama3-8b", "qkv", 6144, 4096), ("llama3-8b", "o", 4096, 4096), ("llama3-8b", "gate|up", 28672, 4096),
    ("llama3-8b", "down", 4096, 14336), ("llama3-8b", "lm_head", 128256, 4096),
    ("qwen2.5-7b", "qkv", 4608, 3584), ("qwen2.5-7b", "o", 3584, 3584), ("qwen2.5-7b", "gate|up", 37888, 3584),
    ("qwen2.5-7b", "down", 3584, 18944),
    ("qwen2.5-1.5b", "qkv", 2048, 1536), ("qwen2.5-1.5b", "o", 1536, 1536), ("qwen2.5-1.5b", "gate|up", 17920, 1536),
    ("qwen2.5-1.5b", "down", 1536, 8960),
]


def shape_sweep(args, time_graph, q4g_gemv, q8_gemv, w8a8_linear, entry, copies_for, stream_ptr):
    """Decode (m = 1) GEMVs in the three quant modes over SWEEP_SHAPES, each
    beside a streaming read of the same weight bytes (the single-launch floor
    at that size), batched decode at m = 8 and 64, and the prefill GEMMs at m =
    128, 256 and 512: evidence that the dispatch holds up away from the shapes
    it was tuned on."""
    import ctypes

    import torch
    dev = torch.device("cuda:0")
    blib = ctypes.CDLL(os.path.join(ROOT, "nanoinfer_amd", "libnq_bench.so"))
    blib.nq_probe_read_cfg.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.zeros(64, dtype=torch.int32, device=dev)

    def read_us(nbytes):
        rb = (nbytes + 15) // 16 * 16
        src = [torch.empty(rb, dtype=torch.uint8, device=dev) for _ in range(copies_for(rb))]
        best = None
        for th, u in ((256, 4), (512, 2), (1024, 1)):
            ms = time_graph([lambda i=i: blib.nq_probe_read_cfg(src[i].data_ptr(), rb, th, u, None, 0,
                                                                sink.data_ptr(), stream_ptr())
                             for i in range(len(src))], args.steps, 10)
            best = ms if best is None else min(best, ms)
        del src
        torch.cuda.empty_cache()
        return round(best * 1e3, 3)

    out = []
    for model, proj, n, k in SWEEP_SHAPES:
        row = {"model": model, "proj": proj, "n": n, "k": k}
        for kind, mk in (("q4g_g32_m1", lambda: q4g_gemv(1, n, k, 32)),
                         ("q8_m1", lambda: q8_gemv(1, n, k, torch.float16)),
                         ("w8a8_m1", lambda: w8a8_linear(1, n, k))):
            e = entry(kind, *mk(), "hbm")
            torch.cuda.empty_cache()
            wbytes = n * k // 2 + n * (k // 32) * 2 if kind.startswith("q4g") else n * k + n * 4
            e["read_floor_us"] = read_us(wbytes)
            e["floor_ratio"] = round(e["read_floor_us"] / e["us"], 3)
            row[kind] = {key: e[key] for key in ("us", "GB/s", "frac", "read_floor_us", "floor_ratio")}
        for mb in (8, 64):  # batched decode: HBM-bound, beside the same read floor
            for kind, mk in ((f"q4g_g32_m{mb}", lambda: q4g_gemv(mb, n, k, 32)),
                             (f"q8_m{mb}", lambda: q8_gemv(mb, n, k, torch.float16)),
                             (f"w8a8_m{mb}", lambda: w8a8_linear(mb, n, k))):
                e = entry(kind, *mk(), "hbm")
                torch.cuda.empty_cache()
                floor = row[kind.replace(f"_m{mb}", "_m1")]["read_floor_us"]
                row[kind] = {"us": e["us"], "GB/s": e["GB/s"], "floor_ratio": round(floor / e["us"], 3)}
        for mp in (128, 256, 512):  # prefill chunks: the MFMA GEMMs' tile and split plans
            for kind, mk, bound in ((f"w8a8_m{mp}", lambda: w8a8_linear(mp, n, k, gemm_only=True), "mfma"),
                                    (f"q8_m{mp}", lambda: q8_gemv(mp, n, k, torch.float16), "mfma_f16"),
                                    (f"q4g_g32_m{mp}", lambda: q4g_gemv(mp, n, k, 32), "mfma_f16")):
                e = entry(kind, *mk(), bound)
                torch.cuda.empty_cache()
                row[kind] = {key: e[key] for key in ("us", "TOPS", "frac")}
        print(json.dumps(row), file=sys.stderr, flush=True)  # progress
        out.append(row)
    return out


def decoder_layer_cfg4(rnd, time_graph, args, w8a8_linear, entry):
    """one Qwen2.5-1.5B decoder layer, M=512 prefill, all seven
    projections W8A8 on libnq_hip.so (q|k|v and gate|up fused into two GEMMs,
    activation quant fused into rmsnorm and silu*up), fp16 activations, RoPE and
    causal GQA attention in torch. Layers with distinct weights are chained
    (>= 512 MiB of weights) so each layer streams its own weights."""
    import torch

    from nanoinfer_amd import model as nm
    from nanoinfer_amd import quant as nq
    cfg = nm.qwen25_15b()
    shapes = nm.proj_shapes(cfg)
    layer_bytes = sum(o * i for o, i in shapes.values())
    L = max(2, math.ceil(ROTATE_BYTES / layer_bytes))
    w = {"embed_tokens.weight": torch.zeros(8, cfg.hidden), "norm.weight": torch.ones(cfg.hidden)}
    for li in range(L):
        p = f"layers.{li}."
        for name, (o, i) in shapes.items():
            w[p + name + ".weight"] = rnd((o, i), 0.02)
        for b in ("q_proj", "k_proj", "v_proj"):
            w[p + f"self_attn.{b}.bias"] = rnd((shapes[f"self_attn.{b}"][0],), 0.02)
        w[p + "input_layernorm.weight"] = 1.0 + rnd((cfg.hidden,), 0.02)
        w[p + "post_attention_layernorm.weight"] = 1.0 + rnd((cfg.hidden,), 0.02)
    mdl = nm.Model(cfg, w, nq.QuantMode.W8A8, "cuda", act_dtype=torch.float16, quantize_embed=False, layers=L)
    del w
    m = 512
    x0 = rnd((m, cfg.hidden), 1.0, torch.float16)

    def run_layers():
        return mdl.run_layers(x0)
    steps = max(2, args.steps // L)
    ms = time_graph([run_layers], steps, max(1, max(args.warmup, 2000) // L)) / L
    proj_ops = sum(2 * m * o * i for o, i in shapes.values())
    del mdl
    torch.cuda.empty_cache()
    # The layer's causal GQA attention is torch's scaled_dot_product_attention
    # (AOTriton on ROCm), outside this path: timed alone at the layer's shape and
    # reported as non-product time.
    hq = torch.randn((cfg.heads, m, cfg.head_dim), device="cuda").half()
    hk = torch.randn((cfg.kv_heads, m, cfg.head_dim), device="cuda").half()
    hv = torch.randn((cfg.kv_heads, m, cfg.head_dim), device="cuda").half()
    attn_ms = time_graph([lambda: nm.attention(hq, hk, hv, cfg.heads // cfg.kv_heads)], args.steps,
                         max(args.warmup, 200))
    del hq, hk, hv
    e = {"name": f"decoder_layer_cfg4 M={m} Qwen2.5-1.5B: the 7 W8A8 projections (4 fused GEMMs on this path)",
         "layer_us": round(ms * 1e3, 3), "layers_chained": L,
         "layer_note": "whole layer: projections + fused act quants + RoPE (this path) + torch SDPA attention "
                       "(non-product)",
         "attention_us_nonproduct": round(attn_ms * 1e3, 3),
         "attention_note": "torch.nn.functional.scaled_dot_product_attention (AOTriton attn_fwd on ROCm), "
                           "timed alone at the layer's shape; not part of the quantized path"}
    torch.cuda.empty_cache()
    # The layer runs q|k|v and gate|up as fused GEMMs on pre-quantized input
    # (activation quant fused into rmsnorm / silu*up); these are timed as GEMMs.
    fused = {"qkv_proj": (shapes["self_attn.q_proj"][0] + 2 * shapes["self_attn.k_proj"][0], cfg.hidden),
             "o_proj": shapes["self_attn.o_proj"],
             "gate_up_proj": (2 * cfg.intermediate, cfg.hidden),
             "down_proj": shapes["mlp.down_proj"]}
    projs = []
    for name, (o, i) in fused.items():
        pe = entry(f"{name} M={m} K={i} N={o} (GEMM on pre-quantized x)", *w8a8_linear(m, o, i, gemm_only=True), "mfma")
        projs.append(pe)
        torch.cuda.empty_cache()
    e["projections"] = projs
    pus = sum(p["us"] for p in projs)
    # the config-4 figure: the seven projections' GEMM time and its MFMA fraction
    e.update({"us": round(pus, 3), "ops": proj_ops, "TOPS": round(proj_ops / (pus * 1e-6) / 1e12, 2),
              "bound": "mfma", "frac": round(proj_ops / (pus * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
              "layer_TOPS_incl_nonproduct": round(proj_ops / (ms * 1e-3) / 1e12, 2)})
    return e


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_calls(fn, seconds, min_calls=3):
    """Median wall time of repeated fn() calls over about `seconds` (after one warm call)."""
    import numpy as np
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(m, n, k, g, nbytes, seconds):
    """Time the reference's CPU path (oracle/_ref: the reference's own quant.cpp,
    AVX2 + OpenMP) — or the C restatement where that build is absent — on this
    host's cores: the headline linear_q4g (quant.cpp:337-389) on the same shape,
    plus bounded samples of the other configs' CPU ops (linear_q8 :136-163 at
    config 1 and the LM head, linear_w8a8 :165-210 at configs 3 and 5a)."""
    import numpy as np

    import oracle
    impl = oracle.reference()
    kind = "reference"
    if impl is None:
        impl = oracle.oracle()
        kind = "port"
    rng = np.random.default_rng(7)
    x = rng.standard_normal((m, k)).astype(np.float16).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = impl.quantize_q4g(w, g)
    s = s.astype(np.float16).astype(np.float32)      # the fp16 storage variant's scales, widened
    med, calls = _time_calls(lambda: impl.linear_q4g(x, q, s, g), seconds)
    # The load-time quantize of the same weight (quant.cpp:295-321, serial in
    # the reference): fp32 read once, packed codes + fp32 scales written once.
    qmed, qcalls = _time_calls(lambda: impl.quantize_q4g(w, g), max(1.0, seconds / 5))
    qbytes = n * k * 4 + n * ((k + 1) // 2) + n * ((k + g - 1) // g) * 4
    del w, q, s

    # Other configs, same algorithmic-byte / op accounting as the GPU sweep.
    others = []
    per = max(1.0, seconds / 4)

    def q8_case(name, mm, nn, kk, xdt):
        xx = rng.standard_normal((mm, kk), dtype=np.float32).astype(xdt).astype(np.float32)
        ww = rng.standard_normal((nn, kk), dtype=np.float32) * np.float32(0.02)
        qq, ss = impl.quantize_q8(ww)
        del ww
        t, c = _time_calls(lambda: impl.linear_q8(xx, qq, ss), per)
        esz = 2 if xdt == np.float16 else 4
        nb = nn * kk + 4 * nn + esz * mm * kk + esz * mm * nn
        others.append({"op": f"linear_q8 {name} M={mm} K={kk} N={nn}", "ms": round(t * 1e3, 3),
                       "GB/s": round(nb / t / 1e9, 3), "calls": c})

    def w8a8_case(name, mm, nn, kk, bound):
        xx = rng.standard_normal((mm, kk), dtype=np.float32).astype(np.float16).astype(np.float32)
        ww = rng.standard_normal((nn, kk), dtype=np.float32) * np.float32(0.02)
        qq, ss = impl.quantize_q8(ww)
        del ww
        t, c = _time_calls(lambda: impl.linear_w8a8(xx, qq, ss), per, min_calls=1)
        nb = nn * kk + 4 * nn + 2 * mm * kk + 2 * mm * nn
        e = {"op": f"linear_w8a8 {name} M={mm} K={kk} N={nn}", "ms": round(t * 1e3, 3), "calls": c,
             "TOPS": round(2 * mm * nn * kk / t / 1e12, 4)}
        if bound == "hbm":
            e["GB/s"] = round(nb / t / 1e9, 3)
        others.append(e)

    q8_case("cfg1", 1, 4864, 896, np.float32)
    q8_case("lm head cfg5b", 1, 151936, 1536, np.float16)
    w8a8_case("gate/up cfg3", 8, 8960, 1536, "hbm")
    w8a8_case("prefill cfg5a", 2048, 8960, 1536, "mfma")
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": impl.max_threads(),
            "kind": kind, "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "sample": f"{calls} calls of linear_q4g M={m} K={k} N={n} g={g} (median {med * 1e3:.2f} ms), "
                      f"~{seconds:.0f}s of CPU work, same algorithmic bytes",
            "quantize": {"op": f"quantize_q4g N={n} K={k} g={g} (load time)", "ms": round(qmed * 1e3, 3),
                         "GB/s": round(qbytes / qmed / 1e9, 3), "calls": qcalls},
            "other_configs": others}


if __name__ == "__main__":
    main()
