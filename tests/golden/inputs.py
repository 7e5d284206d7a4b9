"""Seeded self-test weights, restated from the reference's ``selftest_inputs``
(roblennon/mac-kernels-public ``modal/weight_error_app.py:421-436``).

They are built from integer draws of a seeded ``torch.Generator`` and exact arithmetic, so they
are bit-identical across platforms; each is checked against the reference's ``input_sha256``.
"""
import numpy as np
import torch


def _hadamard_256_f64():
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < 256:
        h = np.kron(h, h4)
    return h / 16.0


def selftest_inputs(which=("gauss_96x1024", "heavy_96x1024", "chunked_4200x1024")):
    g = torch.Generator().manual_seed(1234)

    def gauss(n, k):  # sum of 12 uniform integers, centred; std 1/64
        u = torch.randint(0, 65536, (12, n, k), generator=g, dtype=torch.int64).sum(0) - 6 * 65535
        return (u.double() * 2.0 ** -22).float().to(torch.bfloat16).float()

    out = {}
    wa = gauss(96, 1024)
    u = torch.randint(0, 256, (4, 96, 1024), generator=g, dtype=torch.int64).sum(0) - 510
    cubes = (u.double() ** 3).numpy()  # integers below 2^28: the +-1 Hadamard sums are exact in float64
    rot = (cubes * 16.0).reshape(96, 4, 256) @ _hadamard_256_f64().T  # exact: integer sums times 1/16
    wb = torch.from_numpy(rot.reshape(96, 1024) / 256.0 * 2.0 ** -30).float().to(torch.bfloat16).float()
    out["gauss_96x1024"] = wa.numpy()
    out["heavy_96x1024"] = wb.numpy()
    if "chunked_4200x1024" in which:
        out["chunked_4200x1024"] = gauss(4200, 1024).numpy()
    return {k: v for k, v in out.items() if k in which}
