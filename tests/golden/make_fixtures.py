"""Write the golden fixtures from the reference's own result file (data only).

Source: roblennon/mac-kernels-public ``modal/results/2026-11-09-weight-error-selftest-container.json``
(the reference's in-container self-test vectors: sha256 of every stored tensor and of its
dequantization, plus base64 raw bytes of the stored tensors for the two 96x1024 cases).

Run in the build container, where the reference is mounted:
    python tests/golden/make_fixtures.py [/root/reference]
Outputs (committed): tests/golden/selftest_raw.npz, tests/golden/selftest_sha256.json
"""
import base64
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "modal/results/2026-11-09-weight-error-selftest-container.json"


def main(ref_root="/root/reference"):
    with open(os.path.join(ref_root, SRC)) as f:
        data = json.load(f)
    raw = {}
    meta = {"source": SRC, "torch": data.get("torch"), "gguf": data.get("gguf"),
            "ggml_version": data.get("ggml_version"), "cases": {}}
    shapes = {"gauss_96x1024": (96, 1024), "heavy_96x1024": (96, 1024), "chunked_4200x1024": (4200, 1024)}
    for case, entry in data["cases"].items():
        n, k = shapes[case]
        cmeta = {"input_sha256": entry["input_sha256"], "shape": [n, k], "formats": {}}
        for fmt, e in entry["formats"].items():
            fm = {key: val for key, val in e.items()
                  if isinstance(val, str) and not key.endswith("_b64")}
            fm["rel_fro"] = e.get("rel_fro")
            fm["max_abs"] = e.get("max_abs")
            cmeta["formats"][fmt] = fm
            for key, val in e.items():
                if key.endswith("_b64"):
                    buf = np.frombuffer(base64.b64decode(val), dtype=np.uint8)
                    raw[f"{case}/{fmt}/{key[:-4]}"] = buf
        meta["cases"][case] = cmeta
    np.savez_compressed(os.path.join(HERE, "selftest_raw.npz"), **raw)
    with open(os.path.join(HERE, "selftest_sha256.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print(f"wrote {len(raw)} raw tensors")


if __name__ == "__main__":
    main(*sys.argv[1:])
