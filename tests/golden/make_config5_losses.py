"""Writes config5_cnn_losses.json: the CPU oracle's per-step losses for 100
SGD-momentum steps of BASELINE config 5 (the CIFAR-100-shaped CNN at batch
128), so the device test can compare every step without re-running ~6 minutes
of oracle work on the GPU box.

The oracle (oracle/vkml_oracle.c) is deterministic for any thread count
(OpenMP over outputs only), and the inputs come from a seeded numpy
generator, so the file is a function of the seed and the restated reference
algorithms. tests/test_config5_fixture.py re-derives its first steps live.

Usage: python tests/golden/make_config5_losses.py
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

import numpy as np  # noqa: E402

from conftest import (CONFIG5_BATCH, CONFIG5_LOSSES, CONFIG5_LR, CONFIG5_MOMENTUM,  # noqa: E402
                      CONFIG5_STEPS, SEED, config5_train)
from oracle import OracleBackend  # noqa: E402


def main() -> None:
    t0 = time.time()
    losses = config5_train(OracleBackend())
    data = {
        "what": "CPU-oracle loss per step, BASELINE config 5 CNN, fresh U[-1,1) batch per step",
        "seed": SEED + CONFIG5_BATCH, "model_seed": SEED, "batch": CONFIG5_BATCH,
        "steps": CONFIG5_STEPS, "lr": CONFIG5_LR, "momentum": CONFIG5_MOMENTUM,
        "losses_f32_bits": [f"{int(b):08x}" for b in losses.view(np.uint32)],
        "losses": [float(v) for v in losses],
    }
    CONFIG5_LOSSES.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {CONFIG5_LOSSES} ({time.time() - t0:.0f} s): first {losses[0]:.6f} last {losses[-1]:.6f}")


if __name__ == "__main__":
    main()
