"""Quantized-linear benchmark on one MI355X.

Default workload (one JSON line on stdout): GGUF block-decode linear, K = N = 4096, M in {1, 8, 64},
one call per (type, M) for Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS -- 21 linear calls per step.
Weights are N(0, 0.02) quantized with the standard GGUF block layouts, activations fp16 N(0, 1),
everything resident in HBM before the timed region.  Each step reads a different copy of every
weight from a pool of >= 1 GiB (4x the 256 MiB Infinity Cache) so the bytes come from HBM.  The
steps are captured once in a HIP graph and replayed, so launch overhead from Python is not timed.

value = whole-step algorithmic bytes (packed weights + fp16 x + fp16 y) / step time, in GB/s.
roofline: the kernel with the largest share of the step (by time), its algorithmic bytes per launch over
its average launch duration (HIP events around graph replays of that call alone), against the 8 TB/s
HBM peak; `traffic` is its measured HBM bytes per launch from the committed counter summary.
cpu_baseline: the oracle's dequantize-then-matmul on the host (C decode, fp32 BLAS matmul).

Other suites (--suite int8|w4a8|w6a8|dit|lora|grad|all) print their own JSON lines to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mac-kernels-public_amd")]

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
METRIC = "quantized-linear TFLOP/s + HBM GB/s (% of MI355X roofline), M=1..4096"
GGUF_SUITE = ("Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS")
POOL_BYTES = 1 << 30


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gguf_bytes(name, n, k):
    from qlin.gguf import GGUF_TYPES
    _, qk, ts = GGUF_TYPES[name]
    return n * (k // qk) * ts


def quantized_base(name, n, k, seed=0):
    """One N(0, 0.02) weight quantized on the host to GGUF `name` (uint8 [n, row_bytes])."""
    import torch
    from qlin.quantize import quantize_gguf
    base = (torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02).numpy()
    return torch.from_numpy(quantize_gguf(base, name))


def make_gguf_weights(name, n, k, copies, seed=0, raw=None):
    """`copies` independent weights of one type (quantized on the host, then resident on the GPU)."""
    import numpy as np
    import torch
    out = []
    if raw is None:
        raw = quantized_base(name, n, k, seed)
    for c in range(copies):
        # distinct bytes per copy: permute the block rows (still valid blocks) so no two copies alias
        perm = torch.from_numpy(np.random.default_rng(seed + 100 + c).permutation(n))
        out.append(raw[perm].contiguous().to("cuda"))
    return out


def time_graph(fn_step, steps, warmup, stream=None):
    """Capture `fn_step` once into a HIP graph, replay warmup + steps times, return ms per replay."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn_step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn_step()
    torch.cuda.synchronize()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, g


def suite_gguf(steps, warmup, n=4096, k=4096, ms=(1, 8, 64)):
    import torch
    import qlin
    per_step_bytes = sum(gguf_bytes(t, n, k) for t in GGUF_SUITE) * len(ms)
    copies = max(1, -(-POOL_BYTES // per_step_bytes))
    log(f"[gguf] building pool: {copies} copies x {per_step_bytes / 2**20:.0f} MiB per step")
    bases = {t: quantized_base(t, n, k, seed=i) for i, t in enumerate(GGUF_SUITE)}
    weights = {t: make_gguf_weights(t, n, k, copies * len(ms), seed=i, raw=bases[t]) for i, t in enumerate(GGUF_SUITE)}
    g = torch.Generator().manual_seed(1)
    xs = {m: torch.randn(m, k, generator=g).half().cuda() for m in ms}
    calls = []
    for c in range(copies):
        for t in GGUF_SUITE:
            for j, m in enumerate(ms):
                calls.append((t, m, weights[t][c * len(ms) + j]))
    tid = {t: qlin.GGUF_TYPES[t][0] for t in GGUF_SUITE}

    def step_all():
        for t, m, w in calls:
            qlin.gguf_linear(xs[m], w, tid[t], (n, k))

    log(f"[gguf] {len(calls)} calls per graph replay ({copies} pool passes)")
    ms_replay, _ = time_graph(step_all, max(1, steps), warmup)
    ms_step = ms_replay / copies
    alg_bytes = sum(gguf_bytes(t, n, k) + m * k * 2 + m * n * 2 for t in GGUF_SUITE for m in ms)
    flops = sum(2 * m * n * k for _ in GGUF_SUITE for m in ms)
    gbs = alg_bytes / (ms_step * 1e-3) / 1e9

    # per (type, M): a graph of the same call over its own >= 1 GiB pool of that weight, so that
    # every launch reads HBM (a few copies would sit in the 256 MiB Infinity Cache)
    del weights
    detail = {}
    for i, t in enumerate(GGUF_SUITE):
        nc = -(-POOL_BYTES // gguf_bytes(t, n, k))
        ws = make_gguf_weights(t, n, k, nc, seed=i, raw=bases[t])
        for j, m in enumerate(ms):
            def one(ws=ws, m=m, t=t):
                for w in ws:
                    qlin.gguf_linear(xs[m], w, tid[t], (n, k))

            msr, _ = time_graph(one, 10, 2)
            us = msr / nc * 1e3
            b = gguf_bytes(t, n, k) + m * k * 2 + m * n * 2
            detail[f"{t}/M{m}"] = {"us": round(us, 2), "bytes": b, "GBps": round(b / (us * 1e-6) / 1e9, 1),
                                   "TFLOPs": round(2 * m * n * k / (us * 1e-6) / 1e12, 2)}
            log(f"[gguf] {t:7s} M={m:3d}: {us:7.2f} us  {detail[f'{t}/M{m}']['GBps']:8.1f} GB/s")
    return {
        "ms_per_step": ms_step, "value": gbs, "alg_bytes": alg_bytes, "flops": flops,
        "launches": len(GGUF_SUITE) * len(ms), "detail": detail, "copies": copies,
    }


def cpu_baseline_gguf(n=4096, k=4096, ms=(1, 8, 64), rows=None):
    """Oracle decode (C, one thread) + fp32 matmul (torch, all host threads) for the same 21 calls.
    `rows`: decode only that many weight rows per call (bounded sample), scaled up to N."""
    import numpy as np
    import torch

    import oracle as O
    from qlin.quantize import quantize_gguf
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows = rows or n
    rng = np.random.default_rng(0)
    total_s, dec_s, mm_s, alg = 0.0, 0.0, 0.0, 0
    for t in GGUF_SUITE:
        w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
        raw = quantize_gguf(w, t)
        for m in ms:
            x = torch.randn(m, k).half().float()
            t0 = time.perf_counter()
            wd = torch.from_numpy(O.gguf_dequantize(raw, t, (rows, k)))
            t1 = time.perf_counter()
            y = x @ wd.T
            t2 = time.perf_counter()
            del y
            dec_s += (t1 - t0) * n / rows
            mm_s += (t2 - t1) * n / rows
            alg += gguf_bytes(t, n, k) + m * k * 2 + m * n * 2
    total_s = dec_s + mm_s
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(alg / total_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"one pass of the 21 calls (7 types x M in {{1,8,64}}, K=N=4096); decode of {rows} of "
                   f"{n} rows per call by the C oracle on 1 thread, fp32 torch matmul on {threads} threads, "
                   f"scaled to N={n}"),
        "decode_ms": round(dec_s * 1e3, 1), "matmul_ms": round(mm_s * 1e3, 1), "cpu_model": cpu_model,
        "decode_threads": 1,
    }


SPLIT_PATH = "gguf_split_kernel+gguf_split_reduce_kernel"


def kernel_of(t, m):
    """Kernel(s) that serve a K=N=4096 GGUF call of type t with M activation rows (the dispatch in
    the C ABI).  The K-split path is two launches per call: the split kernel and its reduction."""
    if m == 1:
        return "gguf_gemv_kernel"
    return SPLIT_PATH if m >= (5 if t == "Q6_K" else 17) else "gguf_smallm_kernel"


def kernel_breakdown(detail):
    """Per kernel (or two-kernel path): calls, algorithmic bytes per call and the average call
    duration, from the per-(type, M) graph timings (HIP events on the replay stream)."""
    out = {}
    for key, d in detail.items():
        t, m = key.split("/M")
        k = kernel_of(t, int(m))
        e = out.setdefault(k, {"launches": 0, "bytes": 0, "us_total": 0.0})
        e["launches"] += 1
        e["bytes"] += d["bytes"]
        e["us_total"] += d["us"]
    for k, e in out.items():
        e["bytes_per_launch"] = round(e["bytes"] / e["launches"])
        e["us_per_launch"] = round(e["us_total"] / e["launches"], 3)
        e["GBps"] = round(e["bytes"] / (e["us_total"] * 1e-6) / 1e9, 1)
        e["us_total"] = round(e["us_total"], 2)
        del e["bytes"]
    return out


def measured_traffic(kernel):
    """HBM bytes per call of `kernel` (a '+'-joined path adds its kernels) from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (counter runs cannot happen inside the timed
    process); None when the summary has no line for one of them."""
    path = os.path.join(ROOT, "profiles", "gguf_linear_k4096_counters.md")
    per = {}
    try:
        for line in open(path):
            if line.startswith("traffic "):
                f = line.split()
                per[f[1]] = int(f[2])
    except OSError:
        return None
    parts = kernel.split("+")
    return sum(per[k] for k in parts) if all(k in per for k in parts) else None


def profile_pass(n=4096, k=4096, ms=(1, 8, 64), reps=3):
    """Eager launches for counter collection (each dispatch is profiled on its own)."""
    import torch
    import qlin
    weights = {t: make_gguf_weights(t, n, k, reps * len(ms), seed=i) for i, t in enumerate(GGUF_SUITE)}
    g = torch.Generator().manual_seed(1)
    xs = {m: torch.randn(m, k, generator=g).half().cuda() for m in ms}
    for t in GGUF_SUITE:
        tid = qlin.GGUF_TYPES[t][0]
        for j, m in enumerate(ms):
            for r in range(reps):
                qlin.gguf_linear(xs[m], weights[t][r * len(ms) + j], tid, (n, k))
    # reference kernel of known traffic: an elementwise pass reading and writing 64 MiB each
    src = torch.ones(16 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log("[profile] done")


def other_suites(which, steps, warmup):
    """INT8-ConvRot, W4A8, W6A8 and the DiT layer stack at their benchmark shapes (stderr JSON lines)."""
    import torch
    import qlin
    from qlin.quantize import quantize_int8_convrot_weight, quantize_w4a8_int8_weight
    out = []
    gen = torch.Generator().manual_seed(0)

    def weight(n, k):
        return (torch.randn(n, k, generator=gen) * 0.02).numpy()

    def timed(name, fn, flops, nbytes, peak, unit):
        msr, _ = time_graph(fn, steps, warmup)
        tfl = flops / (msr * 1e-3) / 1e12
        gbs = nbytes / (msr * 1e-3) / 1e9
        rec = {"suite": name, "ms": round(msr, 4), unit: round(tfl, 1), "GBps": round(gbs, 1),
               "frac_peak": round(tfl / peak, 4), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        log(json.dumps(rec))
        out.append(rec)

    if which in ("int8", "all"):
        m, n, k = 256, 3072, 3072
        q, s = quantize_int8_convrot_weight(weight(n, k), 128)
        qd, sd = torch.from_numpy(q).cuda(), torch.from_numpy(s).half().cuda()
        x = torch.randn(m, k).half().cuda()
        timed("int8_convrot M256 K3072 N3072", lambda: qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=128),
              2 * m * n * k, n * k + n * 2 + m * k * 2 + m * n * 2, FP16_PEAK_TFLOPS, "TFLOPs")
    if which in ("w4a8", "all"):
        m, n, k = 4096, 12288, 3072
        log("[w4a8] quantizing 12288x3072 ...")
        q, sr, sc, cb = quantize_w4a8_int8_weight(weight(n, k), bits=4, group_size=128, convrot_groupsize=128,
                                                  codebook=None, s_rel_dtype=torch.float16)
        qd, srd, scd = q.cuda(), sr.cuda(), sc.cuda()
        g = torch.Generator().manual_seed(2)
        x = torch.randn(m, k, generator=g)
        x = torch.where(torch.rand(m, k, generator=g) < 0.01, 20.0 * torch.sign(x), x).half().cuda()
        timed("w4a8 M4096 K3072 N12288", lambda: qlin.w4a8_int8_linear(x, qd, srd, scd, None, None, None, 128, 128),
              2 * m * n * k, q.numel() + sr.numel() * 2 + n * 4 + m * k * 2 + m * n * 2, INT8_PEAK_TOPS, "TOPs")
    if which in ("w6a8", "all"):
        packed = {}
        for (n, k) in ((13824, 5120), (5120, 13824)):
            log(f"[w6a8] quantizing {n}x{k} ...")
            q, sr, sc, cb = quantize_w4a8_int8_weight(weight(n, k), bits=6, group_size=64, convrot_groupsize=256,
                                                      codebook=None, s_rel_dtype=torch.float16)
            packed[(n, k)] = (q, sr, sc)
        for m in (1024, 9504):
            for (n, k), (q, sr, sc) in packed.items():
                qd, srd, scd = q.cuda(), sr.cuda(), sc.cuda()
                x = torch.randn(m, k).half().cuda()
                timed(f"w6a8 M{m} K{k} N{n}", lambda: qlin.w4a8_int8_linear(x, qd, srd, scd, None, None, None, 64, 256),
                      2 * m * n * k, q.numel() + sr.numel() * 2 + n * 4 + m * k * 2 + m * n * 2, INT8_PEAK_TOPS, "TOPs")
    if which in ("dit", "all"):
        m, h = 4608, 3072
        shapes = [(9216, 3072), (3072, 3072), (12288, 3072), (3072, 12288)]
        layer = []
        for (n, k) in shapes:
            q, s = quantize_int8_convrot_weight(weight(n, k), 128)
            layer.append((torch.from_numpy(q).cuda(), torch.from_numpy(s).half().cuda(),
                          torch.randn(m, k).half().cuda()))
        dense = [(torch.randn(n, k).half().cuda() * 0.02, torch.randn(m, k).half().cuda()) for (n, k) in shapes]

        def qstep():
            for qd, sd, x in layer:
                qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=128)

        def dstep():
            for w, x in dense:
                torch.nn.functional.linear(x, w)

        fl = sum(2 * m * n * k for n, k in shapes)
        nb = sum(n * k for n, k in shapes)
        timed("dit_layer int8_convrot (4 linears, M4608)", qstep, fl, nb, FP16_PEAK_TFLOPS, "TFLOPs")
        timed("dit_layer fp16 torch F.linear (resident weights)", dstep, fl, nb * 2, FP16_PEAK_TFLOPS, "TFLOPs")
    if which in ("lora", "all"):
        # unmerged LoRA beside the quantized linears at the reference's LoRA benchmark shape
        # (M, K, N) = (4608, 6144, 6144), rank 64, bf16 in and out, ConvRot on: the base call, the
        # call with lora_down / lora_up, and the LoRA as two separate bf16 GEMMs on the base output
        m, n, k, r = 4608, 6144, 6144, 64
        x = torch.randn(m, k).to(torch.bfloat16).cuda()
        down = (torch.randn(r, k) * 0.02).to(torch.bfloat16).cuda()
        up = (torch.randn(n, r) * 0.02).to(torch.bfloat16).cuda()
        q, s = quantize_int8_convrot_weight(weight(n, k), 256)
        qd, sd = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
        log("[lora] quantizing 6144x6144 (6-bit) ...")
        q6, sr6, sc6, _ = quantize_w4a8_int8_weight(weight(n, k), bits=6, group_size=64, convrot_groupsize=256,
                                                    codebook=None, s_rel_dtype=torch.float16)
        q6, sr6, sc6 = q6.cuda(), sr6.cuda(), sc6.cuda()
        calls = {
            "int8_convrot": lambda **kw: qlin.int8_linear(x, qd, sd, None, torch.bfloat16, convrot=True,
                                                          convrot_groupsize=256, **kw),
            "w6a8": lambda **kw: qlin.w4a8_int8_linear(x, q6, sr6, sc6, None, None, None, 64, 256, torch.bfloat16, **kw),
        }
        fl, flr = 2 * m * n * k, 2 * m * r * (k + n)
        for fmt, f in calls.items():
            peak, unit = (FP16_PEAK_TFLOPS, "TFLOPs") if fmt == "int8_convrot" else (INT8_PEAK_TOPS, "TOPs")
            timed(f"lora base {fmt} M{m} K{k} N{n}", lambda f=f: f(), fl, n * k + m * k * 2 + m * n * 2, peak, unit)
            timed(f"lora fused {fmt} r{r}", lambda f=f: f(lora_down=down, lora_up=up, lora_scale=0.8), fl + flr,
                  n * k + m * k * 2 + m * n * 4, peak, unit)

            def unfused(f=f):
                y = f()
                y.addmm_(torch.nn.functional.linear(x, down), up.t(), alpha=0.8)
            timed(f"lora unfused {fmt} r{r} (bf16 addmm beside the call)", unfused, fl + flr,
                  n * k + m * k * 2 + m * n * 4, peak, unit)
    if which in ("grad", "all"):
        # frozen-weight input gradient at the reference's training shapes: 1056 tokens, Krea 2
        # layers attn.wq 6144->6144, attn.wk 6144->1536, mlp.up 6144->16384, mlp.down 16384->6144;
        # fp16 dy, INT8-ConvRot weights.  Beside it: torch's dense fp16 dy @ W on a resident fp16
        # weight, and dequantizing the whole layer to fp16 before that GEMM.
        m = 1056
        for name, k, n in (("attn.wq", 6144, 6144), ("attn.wk", 6144, 1536), ("mlp.up", 6144, 16384),
                           ("mlp.down", 16384, 6144)):
            q, s = quantize_int8_convrot_weight(weight(n, k), 256)
            qd, sd = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
            dy = torch.randn(m, n).half().cuda()
            wd = qlin.dequantize_int8_convrot_weight(qd, sd, 256).half()
            fl = 2 * m * n * k
            timed(f"grad int8_convrot {name} M{m} K{k} N{n}", lambda: qlin.int8_linear_grad_input(dy, qd, sd, True, 256),
                  fl, n * k + m * n * 2 + m * k * 2, FP16_PEAK_TFLOPS, "TFLOPs")
            timed(f"grad dense fp16 torch {name}", lambda: dy @ wd, fl, n * k * 2 + m * n * 2 + m * k * 2,
                  FP16_PEAK_TFLOPS, "TFLOPs")
            timed(f"grad dequantize-then-gemm {name}", lambda: dy @ (qd.half() * sd.half()[:, None]), fl,
                  n * k * 5 + m * n * 2 + m * k * 2, FP16_PEAK_TFLOPS, "TFLOPs")
            del wd
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--suite", default="gguf", choices=["gguf", "int8", "w4a8", "w6a8", "dit", "lora", "grad", "all"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-rows", type=int, default=1024, help="weight rows decoded per call for the CPU baseline")
    ap.add_argument("--profile", action="store_true",
                    help="eager launches for rocprofv3 counter runs (no timing, no JSON): each GGUF call three "
                         "times on distinct weights, then a 64 MiB device copy as the byte-counter reference")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported: the linear shards by weight "
              "rows with no exchange between GPUs, so one GPU's throughput is the figure of merit",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import qlin  # noqa: F401
    from qlin import _lib
    _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"

    if a.profile:
        profile_pass()
        return
    if a.suite != "gguf":
        other_suites(a.suite, a.steps, a.warmup)
        if a.suite != "all":
            return
    r = suite_gguf(a.steps, a.warmup)
    kernels = kernel_breakdown(r["detail"])
    dom = max(kernels, key=lambda k: kernels[k]["us_total"])
    dk = kernels[dom]
    line = {
        "metric": METRIC,
        "value": round(r["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "gguf_decode_linear K=N=4096, M in {1,8,64}, types Q4_0 Q8_0 Q4_K Q5_K Q6_K IQ4_NL IQ4_XS "
                        "(21 calls per step, weights cycled through a >=1 GiB pool, HIP-graph replay)",
            "K": 4096, "N": 4096, "M": [1, 8, 64], "types": list(GGUF_SUITE), "pool_copies": r["copies"],
            "tflops_step": round(r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12, 3),
        },
        "roofline": {
            "bound": "hbm", "achieved": dk["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dk["GBps"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
            "kernel": dom, "launches": dk["launches"],
            "bytes_per_launch": dk["bytes_per_launch"], "us_per_launch": dk["us_per_launch"],
            "step_GBps": round(r["value"], 1),
        },
        "kernels": kernels,
        "detail": r["detail"],
    }
    if not a.no_cpu:
        log("[cpu] oracle dequantize-then-matmul baseline ...")
        line["cpu_baseline"] = cpu_baseline_gguf(rows=a.cpu_rows)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
