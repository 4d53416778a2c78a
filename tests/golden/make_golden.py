"""Writes the fixtures under tests/golden/ (run from the repo root).

scale_kats.json  the reference's E8M0 known-answer tests (scale_correctness.py
                 tests 2-4: inputs and expected values at :228, :310, :391)
c1_golden.json   config 1: SHA-256 of the seeded bf16
                 input and of the oracle's RCEIL payload/scale bytes, plus a probe
                 of the oracle's grouped forward output
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "mxfp8-grouped-gemm_amd")]
from mxfp8gg import workloads  # noqa: E402
from oracle import oracle as O  # noqa: E402

HERE = Path(__file__).resolve().parent


def bits(x):
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    kats = {
        "scale_bypass": {  # scale_correctness.py:181-251
            "M": 64, "N": 32, "K": 64, "E": 2, "a_scale_row": [128, 127], "ends": [32, 64],
            "expected": 96.0,
        },
        "application_order": {  # scale_correctness.py:258-337
            "M": 64, "N": 32, "K": 64, "E": 1, "a_scale_row": [128, 126],
            "w_scale_row": [129, 127], "ends": [64], "expected": 272.0,
        },
        "scale_layout": {  # scale_correctness.py:344-401, expected 32*2^m + 32
            "M": 64, "N": 32, "K": 64, "E": 1, "ends": [64],
        },
    }
    (HERE / "scale_kats.json").write_text(json.dumps(kats, indent=1) + "\n")

    x, w, sizes = workloads.c1("cpu")
    xq, xs = O.quant_dim0(bits(x), O.RCEIL)
    wq, ws = O.quant_dim0(bits(w.reshape(-1, 256)), O.RCEIL)
    y = O.grouped_fwd(xq, xs, wq.reshape(4, 512, 256), ws.reshape(4, 512, 8),
                      workloads.ends_of(sizes))
    rng = np.random.default_rng(0)
    idx = np.stack([rng.integers(0, 320, 64), rng.integers(0, 512, 64)], 1)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    fx = {
        "config": "BASELINE.json configs[0]",
        "x_sha256": h(bits(x)),
        "xq_sha256": h(xq), "xs_sha256": h(xs), "wq_sha256": h(wq), "ws_sha256": h(ws),
        "y_probe_index": idx.tolist(),
        "y_probe": [float(v) for v in y[idx[:, 0], idx[:, 1]]],
    }
    (HERE / "c1_golden.json").write_text(json.dumps(fx, indent=1) + "\n")


if __name__ == "__main__":
    main()
