"""Quantized-linear benchmark on one MI355X.

One JSON line on stdout.  Its headline (`value`) is the GGUF block-decode linear, K = N = 4096,
M in {1, 8, 64}, one call per (type, M) for Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS -- 21
linear calls per step.  Weights are N(0, 0.02) quantized with the standard GGUF block layouts,
activations fp16 N(0, 1), everything resident in HBM before the timed region.  Each step reads a
different copy of every weight from a pool of >= 1 GiB (4x the 256 MiB Infinity Cache) so the
bytes come from HBM.  The steps are captured once in a HIP graph and replayed, so launch
overhead from Python is not timed.

value = whole-step algorithmic bytes (packed weights + fp16 x + fp16 y) / step time, in GB/s.
roofline: the kernel path with the largest share of the step (by time), its algorithmic bytes per
call over its average call duration (HIP events around graph replays of that call alone, on the
replay stream), against the 8 TB/s HBM peak; `traffic` is its measured HBM bytes per call from the
committed counter summary.
cpu_baseline: the oracle's dequantize-then-matmul on the host (C decode on all host threads,
fp32 torch matmul on all host threads), median of 5 after 2 warm-ups.

`configs` holds the other workloads at their real shapes, each with its own throughput, roofline
and CPU baseline: INT8-ConvRot M256 K=N=3072; W4A8 M4096 K3072 N12288; W6A8 M in {1024, 9504} for
5120 -> 13824 and 13824 -> 5120; and one INT8-ConvRot DiT block layer (4 linears at 4608 tokens),
reported per layer and x60 beside torch's fp16 F.linear on resident fp16 weights.

Other suites (--suite lora|grad|residual|floors) print their own JSON lines to stderr.
"""
import argparse
import concurrent.futures as cf
import json
import os
import statistics
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
DIT_LAYERS = 60


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_threads():
    """Host threads for the CPU baseline: every CPU this process may use, capped by
    OMP_NUM_THREADS when it is set (the share of a shared host)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


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


def time_graph(fn_step, steps, warmup):
    """Capture `fn_step` once into a HIP graph, replay warmup + steps times, return ms per replay.
    The events are recorded on the stream the replays run on."""
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


def time_eager(fn, calls=200, warmup=20):
    """Microseconds per call issued eagerly from Python (descriptors, workspace and launch on every
    call), back to back on the current stream: when the host is slower than the kernels this is the
    host's time per call."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(calls):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / calls * 1e3


def median_ms(fn, reps=5, warm=2):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e3


class HostPool:
    """Row-parallel CPU decode: the oracle's C routines run in threads (ctypes releases the GIL)."""

    def __init__(self, threads):
        self.threads = threads
        self.ex = cf.ThreadPoolExecutor(threads)

    def rows(self, fn, n):
        """fn(r0, r1) -> array of rows r0..r1; returns their concatenation."""
        import numpy as np
        step = -(-n // self.threads)
        spans = [(r, min(n, r + step)) for r in range(0, n, step)]
        return np.concatenate(list(self.ex.map(lambda sp: fn(*sp), spans)))


# ------------------------------------------------------------------------------------------------
# GGUF decode-linear (the headline)
# ------------------------------------------------------------------------------------------------

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
    # The step runs its calls M-major, all M = 1 calls, then M = 8, then M = 64, as a model's decode
    # or prefill step runs its linears at one M; the type-major order (each type's three M in a row)
    # switches kernel families on every call and is timed beside it for reference.
    calls, calls_tm = [], []
    for c in range(copies):
        for j, m in enumerate(ms):
            for t in GGUF_SUITE:
                calls.append((t, m, weights[t][c * len(ms) + j]))
        for t in GGUF_SUITE:
            for j, m in enumerate(ms):
                calls_tm.append((t, m, weights[t][c * len(ms) + j]))
    tid = {t: qlin.GGUF_TYPES[t][0] for t in GGUF_SUITE}

    def step_of(order):
        def step():
            for t, m, w in order:
                qlin.gguf_linear(xs[m], w, tid[t], (n, k))
        return step

    step_all = step_of(calls)
    log(f"[gguf] {len(calls)} calls per graph replay ({copies} pool passes)")
    ms_replay, _ = time_graph(step_all, max(1, steps), warmup)
    ms_step = ms_replay / copies
    ms_tm = time_graph(step_of(calls_tm), max(1, steps), warmup)[0] / copies
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
        if t == "Q4_K":  # eager calls from Python, beside the graph figure
            for m in ms:
                us = time_eager(lambda m=m: qlin.gguf_linear(xs[m], ws[0], tid[t], (n, k)))
                detail[f"{t}/M{m}"]["eager_us"] = round(us, 2)
                detail[f"{t}/M{m}"]["eager_host_overhead_us"] = round(us - detail[f"{t}/M{m}"]["us"], 2)
                log(f"[gguf] {t:7s} M={m:3d}: eager {us:7.2f} us per call")
        del ws
    return {
        "ms_per_step": ms_step, "value": gbs, "alg_bytes": alg_bytes, "flops": flops,
        "launches": len(GGUF_SUITE) * len(ms), "detail": detail, "copies": copies, "bases": bases,
        "type_major": {"ms_per_step": round(ms_tm, 5), "GBps": round(alg_bytes / (ms_tm * 1e-3) / 1e9, 1)},
    }


def cpu_baseline_gguf(pool, bases, n=4096, k=4096, ms=(1, 8, 64)):
    """The oracle's dequantize (C, row-parallel over all host threads) then fp32 torch matmul for
    the same 21 calls on the same packed weights, each timed as the median of 5 after 2 warm-ups."""
    import torch

    import oracle as O
    torch.set_num_threads(pool.threads)
    dec_ms, mm_ms, alg = 0.0, 0.0, 0
    for t in GGUF_SUITE:
        raw = bases[t].numpy()
        wd = None

        def decode(raw=raw, t=t):
            nonlocal wd
            wd = torch.from_numpy(pool.rows(lambda r0, r1: O.gguf_dequantize(raw[r0:r1], t, (r1 - r0, k)), n))

        dms = median_ms(decode)
        for m in ms:
            x = torch.randn(m, k).half().float()
            mms = median_ms(lambda: x @ wd.T)
            dec_ms += dms
            mm_ms += mms
            alg += gguf_bytes(t, n, k) + m * k * 2 + m * n * 2
    total = dec_ms + mm_ms
    return {
        "value": round(alg / (total * 1e-3) / 1e9, 3), "unit": "GB/s", "cores": pool.threads, "kind": "port",
        "sample": (f"the 21 calls (7 types x M in {{1,8,64}}, K=N=4096) in full: oracle C decode of the whole "
                   f"weight row-parallel on {pool.threads} threads, then fp32 torch matmul on {pool.threads} "
                   "threads; each leg the median of 5 after 2 warm-ups"),
        "decode_ms": round(dec_ms, 2), "matmul_ms": round(mm_ms, 2), "total_ms": round(total, 2),
        "cpu_model": cpu_model(), "threads": pool.threads,
    }


SPLIT_PATH = "gguf_split_kernel+gguf_split_reduce_kernel"


def kernel_of(t, m):
    """Kernel(s) that serve a K=N=4096 GGUF call of type t with M activation rows (the dispatch in
    the C ABI).  The K-split path is two launches per call: the split kernel and its reduction."""
    if m == 1:
        return "gguf_gemv_kernel"
    return SPLIT_PATH if m >= (3 if t == "Q6_K" else 17) else "gguf_smallm_kernel"


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


def measured_traffic(kernel, summary="gguf_linear_k4096_counters.md"):
    """HBM bytes per call of `kernel` (a '+'-joined path adds its kernels) from a committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (counter runs cannot happen inside the timed
    process); None when the summary has no line for one of them."""
    path = os.path.join(ROOT, "profiles", summary)
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


def config_traffic(name, summary="linear_configs_counters.md"):
    """HBM bytes per call of config `name` (every kernel of the call) from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE summary; None when it has no line for the config."""
    try:
        for line in open(os.path.join(ROOT, "profiles", summary)):
            f = line.split()
            if len(f) >= 3 and f[0] == "traffic_call" and f[1] == name:
                return int(f[2])
    except OSError:
        pass
    return None


# ------------------------------------------------------------------------------------------------
# INT8-ConvRot, W4A8, W6A8 and the DiT layer at their benchmark shapes
# ------------------------------------------------------------------------------------------------

# name -> workload.  INT8: weights N(0, 0.02) rotated by the 128-point block Hadamard and quantized
# per output channel by the host quantizer, fp16 scales.  W4/W6: random legal symmetric codes and
# fp16 group scales inside the int8 grid (the offline quantizer takes minutes at these sizes; no
# kernel's time depends on code values).  Activations fp16 N(0, 1) (W4A8: 1% outliers at 20).
CONFIGS = {
    "int8_convrot_m256_k3072_n3072": dict(kind="int8", m=256, k=3072, n=3072, g=128),
    "int8_convrot_m1_k3072_n3072": dict(kind="int8", m=1, k=3072, n=3072, g=128, bound="hbm"),
    "w4a8_m4096_k3072_n12288": dict(kind="a8", bits=4, gs=128, g=128, m=4096, k=3072, n=12288, outliers=True),
    "w6a8_m1024_k5120_n13824": dict(kind="a8", bits=6, gs=64, g=256, m=1024, k=5120, n=13824),
    "w6a8_m1024_k13824_n5120": dict(kind="a8", bits=6, gs=64, g=256, m=1024, k=13824, n=5120),
    "w6a8_m9504_k5120_n13824": dict(kind="a8", bits=6, gs=64, g=256, m=9504, k=5120, n=13824),
    "w6a8_m9504_k13824_n5120": dict(kind="a8", bits=6, gs=64, g=256, m=9504, k=13824, n=5120),
    "dit_layer_int8_convrot_m4608": dict(kind="dit", m=4608, g=128,
                                         linears=((9216, 3072), (3072, 3072), (12288, 3072), (3072, 12288))),
    # a GGUF prefill: 512 activation rows (the split kernel's 64-row m-tiles, the weight decoded in
    # the load stage; one split at this size)
    "gguf_q4_k_m512_k4096_n4096": dict(kind="gguf", type="Q4_K", m=512, k=4096, n=4096),
}

# The launches a call makes at these shapes (the C ABI's dispatch), named as in the kernel traces.
CONFIG_KERNELS = {
    "int8_convrot_m256_k3072_n3072": "prologue_kernel+gemm_wo_dmas_kernel<64,64,256,3>",
    "int8_convrot_m1_k3072_n3072": "int8_gemv_kernel<1,3,2>",
    "w4a8_m4096_k3072_n12288": "a8_prepass_kernel+gemm_i8dma_kernel<256,256>",
    "w6a8_m1024_k5120_n13824": "prologue_kernel+a8_grid_kernel+gemm_i8dma_kernel<256,256>",
    "w6a8_m1024_k13824_n5120": "prologue_kernel+a8_grid_kernel+gemm_i8dma_kernel<128,160,2x5 waves>",
    "w6a8_m9504_k5120_n13824": "a8_prepass_kernel+gemm_i8dma_kernel<256,256>",
    "w6a8_m9504_k13824_n5120": "a8_prepass_kernel+gemm_i8dma_kernel<256,256>",
    "dit_layer_int8_convrot_m4608": "4x (prologue_kernel+gemm_wo_dma_kernel<256,3>)",
    "gguf_q4_k_m512_k4096_n4096": "gguf_split_kernel<Q4_K,MT=2,32x32> (8 m-tiles, one split)",
}


def int8_weight(n, k, g, seed):
    import torch
    from qlin.quantize import quantize_int8_convrot_weight
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02).numpy()
    q, s = quantize_int8_convrot_weight(w, g)
    return torch.from_numpy(q), torch.from_numpy(s).half()


def a8_weight(n, k, bits, gs, seed):
    """Random legal symmetric codes (4-bit 1..15, 6-bit 1..63), packed; fp16 group scales that keep
    level * s_rel inside the int8 grid; fp32 channel scales."""
    import torch
    from qlin.quantize import pack_codes
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(1, (15 if bits == 4 else 63) + 1, (n, k), generator=g, dtype=torch.int32)
    lo, hi = (8.0, 18.0) if bits == 4 else (2.0, 4.1)
    s_rel = (lo + (hi - lo) * torch.rand(n, k // gs, generator=g)).half()
    s_ch = (torch.rand(n, generator=g) * 2e-4 + 1e-4).float()
    return pack_codes(codes, bits), s_rel, s_ch


def permuted_copies(tensors, n, copies, seed):
    """`copies` weights on the GPU made by permuting the rows of `tensors` alike (distinct bytes,
    still a valid packed weight)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    dev = [t.cuda() for t in tensors]
    out = [tuple(dev)]
    for _ in range(copies - 1):
        p = torch.randperm(n, generator=g).cuda()
        out.append(tuple(t[p].contiguous() for t in dev))
    return out


def gpu_activations(m, k, seed, outliers=False):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g)
    if outliers:
        mask = torch.rand(m, k, device="cuda", generator=g) < 0.01
        x = torch.where(mask, 20.0 * torch.sign(x), x)
    return x.half()


def cpu_linear_baseline(pool, name, m, k, n, decode_rows, rows_n=None, rows_m=None):
    """Dequantize-then-matmul on the host for one call: the oracle's C decode of `rows_n` weight
    rows (all N by default; row-parallel on all host threads), then an fp32 torch matmul of `rows_m`
    activation rows (all M by default) against them; each leg the median of 5 after 2 warm-ups,
    scaled to the full M and N when sampled."""
    import torch
    torch.set_num_threads(pool.threads)
    rows_n = min(rows_n or n, n)
    rows_m = min(rows_m or m, m)
    wd = {}

    def decode():
        wd["w"] = torch.from_numpy(pool.rows(decode_rows, rows_n))

    dms = median_ms(decode)
    x = torch.randn(rows_m, k).half().float()
    mms = median_ms(lambda: x @ wd["w"].T)
    dec_full = dms * n / rows_n
    mm_full = mms * (m / rows_m) * (n / rows_n)
    total = dec_full + mm_full
    return {
        "value": round(2 * m * n * k / (total * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "cores": pool.threads,
        "kind": "port",
        "sample": (f"{name}: oracle C decode of {rows_n} of {n} weight rows to fp32 (original basis) on "
                   f"{pool.threads} threads, fp32 torch matmul of {rows_m} of {m} activation rows against them "
                   f"on {pool.threads} threads; medians of 5 after 2 warm-ups"
                   + ("" if (rows_m, rows_n) == (m, n) else f", scaled to M={m}, N={n}")),
        "decode_ms": round(dec_full, 2), "matmul_ms": round(mm_full, 2), "total_ms": round(total, 2),
    }


def run_configs(names, steps, warmup, pool):
    """Time each named workload; `pool` (a HostPool) also runs its CPU baseline, None skips it."""
    import torch
    import qlin

    import oracle as O
    out = {}
    for name in names:
        cfg = CONFIGS[name]
        log(f"[{name}] building ...")
        if cfg["kind"] == "int8":
            m, k, n, g = cfg["m"], cfg["k"], cfg["n"], cfg["g"]
            q, s = int8_weight(n, k, g, seed=7)
            copies = max(1, -(-POOL_BYTES // (n * k)))
            ws = permuted_copies((q, s), n, copies, seed=8)
            x = gpu_activations(m, k, seed=9)

            def step():
                for qd, sd in ws:
                    qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=g)

            msr, _ = time_graph(step, steps, warmup)
            us = msr / copies * 1e3
            eager = time_eager(lambda: qlin.int8_linear(x, ws[0][0], ws[0][1], convrot=True, convrot_groupsize=g))
            flops, nbytes = 2 * m * n * k, n * k + n * 2 + m * k * 2 + m * n * 2
            tfl = flops / (us * 1e-6) / 1e12
            qn, sn = q.numpy(), s.float().numpy()
            cpu = pool and cpu_linear_baseline(pool, name, m, k, n,
                                               lambda r0, r1: O.rotate(O.dequantize_int8(qn[r0:r1], sn[r0:r1]), g), n)
            gbs = nbytes / (us * 1e-6) / 1e9
            if cfg.get("bound") == "hbm":
                roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_frac": round(tfl / FP16_PEAK_TFLOPS, 4)}
            else:
                roof = {"bound": "mfma", "achieved": round(tfl, 2), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tfl / FP16_PEAK_TFLOPS, 4), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            roof.update({"kernel": CONFIG_KERNELS[name], "flops_per_call": flops, "bytes_per_call": nbytes,
                         "traffic": config_traffic(name)})
            rec = {"us_per_call": round(us, 2), "eager_us_per_call": round(eager, 2),
                   "eager_host_overhead_us": round(eager - us, 2), "TFLOPs": round(tfl, 2),
                   "GBps": round(gbs, 1), "pool_copies": copies, "roofline": roof, "cpu_baseline": cpu}
        elif cfg["kind"] == "a8":
            m, k, n, bits, gs, g = cfg["m"], cfg["k"], cfg["n"], cfg["bits"], cfg["gs"], cfg["g"]
            q, sr, sc = a8_weight(n, k, bits, gs, seed=11)
            wbytes = q.numel() + sr.numel() * 2 + n * 4
            copies = max(1, -(-POOL_BYTES // wbytes))
            ws = permuted_copies((q, sr, sc), n, copies, seed=12)
            x = gpu_activations(m, k, seed=13, outliers=cfg.get("outliers", False))

            def step():
                for qd, srd, scd in ws:
                    qlin.w4a8_int8_linear(x, qd, srd, scd, None, None, None, gs, g)

            msr, _ = time_graph(step, steps, warmup)
            us = msr / copies * 1e3
            flops, nbytes = 2 * m * n * k, wbytes + m * k * 2 + m * n * 2
            tops = flops / (us * 1e-6) / 1e12
            qn, srn, scn = q.view(torch.uint8).numpy(), sr.float().numpy(), sc.numpy()
            cpu = pool and cpu_linear_baseline(
                pool, name, m, k, n,
                lambda r0, r1: O.dequantize_w4a8(qn[r0:r1], srn[r0:r1], scn[r0:r1], None, gs, g, bits=bits))
            rec = {"us_per_call": round(us, 2), "TOPs": round(tops, 2),
                   "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "pool_copies": copies,
                   "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                                "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                                "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                "kernel": CONFIG_KERNELS[name], "ops_per_call": flops, "bytes_per_call": nbytes,
                                "traffic": config_traffic(name)},
                   "cpu_baseline": cpu}
        elif cfg["kind"] == "gguf":
            t, m, k, n = cfg["type"], cfg["m"], cfg["k"], cfg["n"]
            raw = quantized_base(t, n, k, seed=14)
            copies = max(1, -(-POOL_BYTES // raw.numel()))
            ws = make_gguf_weights(t, n, k, copies, seed=14, raw=raw)
            x = gpu_activations(m, k, seed=15)
            tid = qlin.GGUF_TYPES[t][0]

            def step():
                for wd in ws:
                    qlin.gguf_linear(x, wd, tid, (n, k))

            msr, _ = time_graph(step, steps, warmup)
            us = msr / copies * 1e3
            flops, nbytes = 2 * m * n * k, raw.numel() + m * k * 2 + m * n * 2
            tfl = flops / (us * 1e-6) / 1e12
            rn = raw.numpy()
            cpu = pool and cpu_linear_baseline(pool, name, m, k, n,
                                               lambda r0, r1: O.gguf_dequantize(rn[r0:r1], t, (r1 - r0, k)))
            rec = {"us_per_call": round(us, 2), "TFLOPs": round(tfl, 2),
                   "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "pool_copies": copies,
                   "roofline": {"bound": "mfma", "achieved": round(tfl, 2), "peak": FP16_PEAK_TFLOPS,
                                "unit": "TFLOP/s", "frac": round(tfl / FP16_PEAK_TFLOPS, 4),
                                "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                "kernel": CONFIG_KERNELS[name], "flops_per_call": flops, "bytes_per_call": nbytes,
                                "traffic": config_traffic(name)},
                   "cpu_baseline": cpu}
        else:  # one DiT block layer: QKV, O, MLP up, MLP down
            m, g = cfg["m"], cfg["g"]
            layer_bytes = sum(n * k for n, k in cfg["linears"])
            copies = max(1, -(-POOL_BYTES // layer_bytes))
            lin = []
            for i, (n, k) in enumerate(cfg["linears"]):
                q, s = int8_weight(n, k, g, seed=20 + i)
                lin.append((n, k, q, s, permuted_copies((q, s), n, copies, seed=30 + i), gpu_activations(m, k, 40 + i)))

            def step():
                for c in range(copies):
                    for n, k, _, _, ws, x in lin:
                        qlin.int8_linear(x, ws[c][0], ws[c][1], convrot=True, convrot_groupsize=g)

            msr, _ = time_graph(step, steps, warmup)
            layer_ms = msr / copies
            per_linear = {}
            for n, k, _, _, ws, x in lin:
                def one(ws=ws, x=x):
                    for qd, sd in ws:
                        qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=g)
                mo, _ = time_graph(one, steps, warmup)
                per_linear[f"{k}->{n}"] = round(mo / copies * 1e3, 2)
            flops = sum(2 * m * n * k for n, k in cfg["linears"])
            tfl = flops / (layer_ms * 1e-3) / 1e12
            # torch's fp16 F.linear on resident fp16 weights, the same pool size in weights
            dense_copies = max(1, -(-POOL_BYTES // (2 * layer_bytes)))
            dense = [[(torch.randn(n, k, device="cuda").half() * 0.02) for n, k in cfg["linears"]]
                     for _ in range(dense_copies)]
            xs = [x for *_, x in lin]

            def dstep():
                for c in range(dense_copies):
                    for w, x in zip(dense[c], xs):
                        torch.nn.functional.linear(x, w)

            dms, _ = time_graph(dstep, steps, warmup)
            dense_ms = dms / dense_copies
            del dense
            # CPU: one layer, each linear sampled as for the single-linear configs, times 60
            cpu = None
            if pool:
                parts = []
                for n, k, q, s, _, _ in lin:
                    qn, sn = q.numpy(), s.float().numpy()
                    parts.append(cpu_linear_baseline(
                        pool, f"{k}->{n}", m, k, n,
                        lambda r0, r1, qn=qn, sn=sn: O.rotate(O.dequantize_int8(qn[r0:r1], sn[r0:r1]), g)))
                layer = sum(p["total_ms"] for p in parts)
                cpu = {"value": round(flops / (layer * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "cores": pool.threads,
                       "kind": "port",
                       "sample": (f"one layer's four linears in full, each: oracle C decode of all its weight "
                                  f"rows to fp32 (original basis) on {pool.threads} threads, fp32 torch matmul of "
                                  f"all {m} activation rows against them on {pool.threads} threads; medians of 5 "
                                  f"after 2 warm-ups; x{DIT_LAYERS} for the stack"),
                       "decode_ms": round(sum(p["decode_ms"] for p in parts), 2),
                       "matmul_ms": round(sum(p["matmul_ms"] for p in parts), 2),
                       "layer_ms": round(layer, 2), "stack_ms": round(layer * DIT_LAYERS, 1)}
            rec = {"ms_per_layer": round(layer_ms, 4), "ms_60_layers": round(layer_ms * DIT_LAYERS, 2),
                   "layers": DIT_LAYERS, "us_per_linear": per_linear, "TFLOPs": round(tfl, 2),
                   "fp16_torch_ms_per_layer": round(dense_ms, 4),
                   "vs_fp16_dense": round(layer_ms / dense_ms, 3), "pool_copies": copies,
                   "roofline": {"bound": "mfma", "achieved": round(tfl, 2), "peak": FP16_PEAK_TFLOPS,
                                "unit": "TFLOP/s", "frac": round(tfl / FP16_PEAK_TFLOPS, 4),
                                "kernel": CONFIG_KERNELS[name], "flops_per_layer": flops, "traffic": config_traffic(name)},
                   "cpu_baseline": cpu}
        if rec["cpu_baseline"] is None:
            del rec["cpu_baseline"]
        out[name] = rec
        log(f"[{name}] " + json.dumps({k: v for k, v in rec.items() if k != "cpu_baseline"}))
        ws = lin = None
        torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------------------------------------
# profiling passes and the optional suites
# ------------------------------------------------------------------------------------------------

def profile_pass(which, reps=3, n=4096, k=4096, ms=(1, 8, 64)):
    """Eager launches for rocprofv3 kernel-trace and counter runs: `which` is "gguf" or a config
    name; each call `reps` times on distinct weights, then an elementwise pass over 64 MiB in and
    64 MiB out as the byte-counter reference."""
    import torch
    import qlin
    if which == "residual":
        # the residual keyword on large-M calls: INT8-ConvRot M4608 K=N=3072 G=128 (a DiT output
        # projection with its residual stream) and W6A8 M1024 K5120 N13824 group 64
        q, s = int8_weight(3072, 3072, 128, seed=20)
        x = gpu_activations(4608, 3072, 40)
        r = gpu_activations(4608, 3072, 41)
        for qd, sd in permuted_copies((q, s), 3072, reps, seed=30):
            qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=128, residual=r)
        qa, sr, sc = a8_weight(13824, 5120, 6, 64, seed=11)
        xa = gpu_activations(1024, 5120, 13)
        ra = gpu_activations(1024, 13824, 14)
        for qd, srd, scd in permuted_copies((qa, sr, sc), 13824, reps, seed=12):
            qlin.w4a8_int8_linear(xa, qd, srd, scd, None, None, None, 64, 256, residual=ra)
        torch.cuda.synchronize()
        log("[profile] done")
        return
    if which == "gguf":
        weights = {t: make_gguf_weights(t, n, k, reps * len(ms), seed=i) for i, t in enumerate(GGUF_SUITE)}
        g = torch.Generator().manual_seed(1)
        xs = {m: torch.randn(m, k, generator=g).half().cuda() for m in ms}
        for t in GGUF_SUITE:
            tid = qlin.GGUF_TYPES[t][0]
            for j, m in enumerate(ms):
                for r in range(reps):
                    qlin.gguf_linear(xs[m], weights[t][r * len(ms) + j], tid, (n, k))
    else:
        cfg = CONFIGS[which]
        if cfg["kind"] == "gguf":
            tid = qlin.GGUF_TYPES[cfg["type"]][0]
            x = gpu_activations(cfg["m"], cfg["k"], 15)
            for wd in make_gguf_weights(cfg["type"], cfg["n"], cfg["k"], reps, seed=14):
                qlin.gguf_linear(x, wd, tid, (cfg["n"], cfg["k"]))
        elif cfg["kind"] == "a8":
            q, sr, sc = a8_weight(cfg["n"], cfg["k"], cfg["bits"], cfg["gs"], seed=11)
            ws = permuted_copies((q, sr, sc), cfg["n"], reps, seed=12)
            x = gpu_activations(cfg["m"], cfg["k"], 13, cfg.get("outliers", False))
            for qd, srd, scd in ws:
                qlin.w4a8_int8_linear(x, qd, srd, scd, None, None, None, cfg["gs"], cfg["g"])
        else:
            lins = ((cfg["n"], cfg["k"]),) if cfg["kind"] == "int8" else cfg["linears"]
            for i, (n_, k_) in enumerate(lins):
                q, s = int8_weight(n_, k_, cfg["g"], seed=20 + i)
                x = gpu_activations(cfg["m"], k_, 40 + i)
                for qd, sd in permuted_copies((q, s), n_, reps, seed=30 + i):
                    qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=cfg["g"])
    src = torch.ones(16 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log("[profile] done")


def floors_suite(steps, warmup):
    """Hardware floors on this GPU (libqlin_floors.so, built from probe/floors.hip), one JSON line on
    stderr: the issue rate of the four MFMA shapes the kernels use (2 waves per SIMD, independent
    accumulators, no memory traffic); a streaming read of one GGUF weight's size (9 MiB Q4_K and
    18 MiB Q8_0 at K = N = 4096) from a >= 1 GiB pool, so every read misses the caches, and of a
    whole GiB; a 512 MiB copy; and an empty launch.  Reads, copies and empty launches are
    HIP-graph replays (the bench's own timing); MFMA rates are the median of 5 event-timed
    launches after 2 warm-ups."""
    import ctypes
    import torch
    L = ctypes.CDLL(os.path.join(ROOT, "mac-kernels-public_amd", "qlin", "libqlin_floors.so"))
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(16 * cus * 256, dtype=torch.float32, device="cuda")
    rec = {"suite": "floors", "cus": cus}

    def check(rc):
        assert rc == 0, f"floors launch failed: {rc}"

    # MFMA: kind -> (name, operations per instruction, accumulators per round)
    shapes = {0: ("mfma_f32_32x32x16_f16", 2 * 32 * 32 * 16, 4), 1: ("mfma_f32_16x16x32_f16", 2 * 16 * 16 * 32, 8),
              2: ("mfma_i32_32x32x32_i8", 2 * 32 * 32 * 32, 4), 3: ("mfma_i32_16x16x64_i8", 2 * 16 * 16 * 64, 8)}
    blocks, iters = 2 * cus, 4000
    mf = {}
    for kind, (name, ops, acc) in shapes.items():
        def launch(kind=kind):
            check(L.qlin_floor_mfma(kind, blocks, iters, ctypes.c_void_p(out.data_ptr()), cur()))
        def timed(launch=launch):
            st = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            launch()
            e1.record(st)
            torch.cuda.synchronize()
            t.append(e0.elapsed_time(e1))
        t = []
        for _ in range(7):
            timed()
        ms = statistics.median(t[2:])
        total = blocks * 4 * iters * acc * ops
        mf[name] = {"T_per_s": round(total / (ms * 1e-3) / 1e12, 1), "ms": round(ms, 4)}
    rec["mfma"] = mf

    pool = torch.empty(POOL_BYTES, dtype=torch.uint8, device="cuda")
    words = torch.empty(16 * cus * 256, dtype=torch.int32, device="cuda")
    rd = {}
    for label, nbytes in (("read_9MiB", 9437184), ("read_18MiB", 18874368), ("read_1GiB", POOL_BYTES)):
        copies = max(1, POOL_BYTES // nbytes)
        rblocks = 4 * cus

        def step(nbytes=nbytes, copies=copies, rblocks=rblocks):
            for c in range(copies):
                check(L.qlin_floor_read(ctypes.c_void_p(pool.data_ptr() + c * nbytes), ctypes.c_int64(nbytes),
                                        rblocks, ctypes.c_void_p(words.data_ptr()), cur()))
        ms, _ = time_graph(step, max(2, steps // 4), warmup)
        us = ms / copies * 1e3
        rd[label] = {"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    half = POOL_BYTES // 2

    def copy_step():
        check(L.qlin_floor_copy(ctypes.c_void_p(pool.data_ptr()), ctypes.c_void_p(pool.data_ptr() + half),
                                ctypes.c_int64(half), 4 * cus, cur()))
    ms, _ = time_graph(copy_step, max(2, steps // 4), warmup)
    rd["copy_512MiB"] = {"bytes_moved": 2 * half, "us": round(ms * 1e3, 1),
                         "GBps": round(2 * half / (ms * 1e-3) / 1e9, 1)}

    def empty_step():
        for _ in range(100):
            check(L.qlin_floor_empty(cus, ctypes.c_void_p(words.data_ptr()), cur()))
    ms, _ = time_graph(empty_step, steps, warmup)
    rd["empty_launch_us"] = round(ms / 100 * 1e3, 3)
    rec["memory"] = rd
    log(json.dumps(rec))
    return rec


def other_suites(which, steps, warmup):
    """LoRA beside the quantized linears, the residual epilogue and the frozen-weight input gradient
    (stderr JSON lines)."""
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
        # GGUF Q4_K at K = N = 4096 (the decode shape and a prefill), rank 64, fp16: the base call, the
        # call with the LoRA in the K-split reduction, and torch's fp16 LoRA beside the call
        n = k = 4096
        raw = make_gguf_weights("Q4_K", n, k, 1, seed=5)[0]
        tid = qlin.GGUF_TYPES["Q4_K"][0]
        d16 = (torch.randn(r, k, generator=gen) * 0.02).half().cuda()
        u16 = (torch.randn(n, r, generator=gen) * 0.02).half().cuda()
        for m in (64, 256):
            xg = torch.randn(m, k, generator=gen).half().cuda()
            g = lambda **kw: qlin.gguf_linear(xg, raw, tid, (n, k), **kw)
            fl, flr, nb = 2 * m * n * k, 2 * m * r * (k + n), gguf_bytes("Q4_K", n, k) + m * k * 2 + m * n * 2
            timed(f"lora base gguf_q4_k M{m} K{k} N{n}", lambda: g(), fl, nb, FP16_PEAK_TFLOPS, "TFLOPs")
            timed(f"lora fused gguf_q4_k M{m} r{r}", lambda: g(lora_down=d16, lora_up=u16, lora_scale=0.8), fl + flr,
                  nb, FP16_PEAK_TFLOPS, "TFLOPs")

            def unfused_g(xg=xg, g=g):
                y = g()
                y.addmm_(torch.nn.functional.linear(xg, d16), u16.t(), alpha=0.8)
            timed(f"lora unfused gguf_q4_k M{m} r{r} (fp16 addmm beside the call)", unfused_g, fl + flr, nb,
                  FP16_PEAK_TFLOPS, "TFLOPs")
    if which in ("residual", "all"):
        # the residual keyword at large M: y = residual + residual_scale * (x W^T + b) applied in the
        # GEMM epilogue, beside the plain call and the two-kernel route (the linear in fp32, then the
        # residual epilogue kernel) that the fused epilogue replaces
        from qlin import _lib
        q, s = int8_weight(3072, 3072, 128, seed=20)
        qd, sd = q.cuda(), s.cuda()
        x = gpu_activations(4608, 3072, 40)
        r = gpu_activations(4608, 3072, 41)
        rs = torch.full((3072,), 0.5, device="cuda").half()
        m, n, k = 4608, 3072, 3072
        fl = 2 * m * n * k
        plain = lambda: qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=128)
        timed(f"residual base int8_convrot M{m} K{k} N{n}", plain, fl, n * k + m * k * 2 + m * n * 2,
              FP16_PEAK_TFLOPS, "TFLOPs")
        timed("residual fused int8_convrot", lambda: qlin.int8_linear(x, qd, sd, convrot=True, convrot_groupsize=128,
                                                                    residual=r, residual_scale=rs),
              fl, n * k + m * k * 2 + m * n * 4, FP16_PEAK_TFLOPS, "TFLOPs")

        def two_kernels():
            base = qlin.int8_linear(x, qd, sd, None, torch.float32, convrot=True, convrot_groupsize=128)
            y = torch.empty(m, n, dtype=torch.float16, device="cuda")
            _lib.load().qlin_residual_epilogue(_lib.desc(base), _lib.desc(r), _lib.desc(rs), _lib.desc(y),
                                               _lib.stream_of(y.device))
        timed("residual two-kernel int8_convrot (fp32 linear, then the residual kernel)", two_kernels, fl,
              n * k + m * k * 2 + m * n * 4, FP16_PEAK_TFLOPS, "TFLOPs")
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
    ap.add_argument("--suite", default="main", choices=["main", "lora", "grad", "residual", "floors", "all"],
                    help="main: the JSON line (GGUF headline + configs); lora / grad / residual / floors: extra "
                         "suites on stderr (floors: MFMA issue rates, HBM read / copy floors, empty launch)")
    ap.add_argument("--configs", default="all",
                    help="comma-separated names from CONFIGS for the `configs` object, 'all' or 'none'")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--profile", default=None, choices=["gguf", "residual", *CONFIGS],
                    help="eager launches of one workload for rocprofv3 kernel-trace / counter runs (no timing, "
                         "no JSON): each call three times on distinct weights, then a 64 MiB elementwise pass as "
                         "the byte-counter reference")
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
        profile_pass(a.profile)
        return
    if a.suite in ("floors", "all"):
        floors_suite(a.steps, a.warmup)
    if a.suite not in ("main", "floors"):
        other_suites(a.suite, a.steps, a.warmup)
    if a.suite != "main" and a.suite != "all":
        return
    pool = None if a.no_cpu else HostPool(host_threads())
    r = suite_gguf(a.steps, a.warmup)
    kernels = kernel_breakdown(r["detail"])
    dom = max(kernels, key=lambda k: kernels[k]["us_total"])
    dk = kernels[dom]
    names = list(CONFIGS) if a.configs == "all" else ([] if a.configs == "none" else a.configs.split(","))
    configs = run_configs(names, a.steps, a.warmup, pool) if names else {}
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
        "data": ("synthetic: GGUF weights N(0, 0.02) quantized on the host; INT8 weights N(0, 0.02) rotated and "
                 "quantized on the host; W4/W6 random legal codes and group scales; activations fp16 N(0, 1)"),
        "config": {
            "workload": "gguf_decode_linear K=N=4096, M in {1,8,64}, types Q4_0 Q8_0 Q4_K Q5_K Q6_K IQ4_NL IQ4_XS "
                        "(21 calls per step, M-major: the 7 types at M=1, then at M=8, then at M=64; weights "
                        "cycled through a >=1 GiB pool, HIP-graph replay)",
            "K": 4096, "N": 4096, "M": [1, 8, 64], "types": list(GGUF_SUITE), "pool_copies": r["copies"],
            "tflops_step": round(r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12, 3),
            "type_major_step": r["type_major"],
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
        "configs": configs,
    }
    if pool:
        log("[cpu] oracle dequantize-then-matmul baseline for the headline ...")
        line["cpu_baseline"] = cpu_baseline_gguf(pool, r["bases"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
