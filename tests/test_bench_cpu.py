"""The benchmark's host side, without a GPU: the one-GPU contract of `bench.py --gpus N`, the kernel
map of the headline against the C ABI's dispatch thresholds, and the committed rocprofv3 summaries
that `bench.py` reads for `roofline.traffic` (every kernel and config it reports has its line)."""
import os
import subprocess
import sys

import pytest

import bench
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADLINE_TYPES = ["Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS"]


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused_before_any_device_call(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and r.stdout == ""


def test_headline_kernel_map_follows_the_dispatch():
    """bench.kernel_of names the kernels of each headline call; the C ABI's workspace query tells
    the K-split path apart (it alone asks for fp32 partials, S x M x N x 4 bytes beyond the
    activations and exponents), so the map is checked against the library's own dispatch."""
    from qlin import _lib
    L = _lib.load()
    a = lambda v: (v + 255) // 256 * 256
    n = k = 4096
    for t in HEADLINE_TYPES:
        tid = O.GGUF_TYPES[t][0]
        for m in (1, 2, 3, 4, 5, 8, 16, 17, 64):
            size = L.qlin_workspace_size(_lib.OP_GGUF_LINEAR, m, n, k, tid, _lib.DT_F16)
            split = size > a(m * k * 2) + a(m * 4) + a(n * 4)
            kern = bench.kernel_of(t, m)
            assert (kern == bench.SPLIT_PATH) == split, (t, m, kern, size)
            if m == 1:
                assert kern == "gguf_gemv_kernel"


def test_gguf_bytes_are_the_block_layout():
    for t in HEADLINE_TYPES:
        _, qk, ts = O.GGUF_TYPES[t]
        assert bench.gguf_bytes(t, 4096, 4096) == 4096 * (4096 // qk) * ts


def test_committed_traffic_summaries_cover_every_reported_kernel_and_config():
    for k in ("gguf_gemv_kernel", "gguf_smallm_kernel", bench.SPLIT_PATH):
        v = bench.measured_traffic(k)
        assert v is not None and v > 0, k
    # algorithmic bytes of a K = N = 4096 Q4_K call are ~9.5 MB; the counters cannot read less than
    # the weight itself
    assert bench.measured_traffic("gguf_gemv_kernel") > 0.9 * bench.gguf_bytes("Q4_0", 4096, 4096)
    for name in bench.CONFIGS:
        v = bench.config_traffic(name)
        assert v is not None and v > 0, name
