"""Writes the CPU oracle's per-step loss trajectories of BASELINE configs 1
and 5 (100 SGD-momentum steps each, the streams of streams.py) as fixtures:

  config1_mlp_losses.json       config 1, the oracle's named exp/log methods
  config5_cnn_losses.json       config 5, the same (about 6 minutes on 8 cores)
  config*_libm.json             the same loops with the oracle's exp/log routed
                                to the platform libm's expf/logf, which is what
                                the reference's std::exp / std::log on float
                                call (kernels_reduce.cpp:233,240)

The device tests compare every step against these without re-running the
oracle on the GPU box, and bench.py reports each timed loop's drift from them.
The two trajectories of one config differ only in the last bit of some
exponentials and logarithms: their distance is how far the reference's own CPU
arithmetic moves between two valid libm builds.

The oracle (oracle/vkml_oracle.c) is deterministic for any thread count
(OpenMP over outputs only) and the inputs come from seeded numpy generators, so
each file is a function of the seeds, the restated reference algorithms and (for
the _libm files) the libm recorded in it. tests/test_config5_fixture.py
re-derives the first steps of each live.

Usage: python tests/golden/make_training_losses.py [--config 1|5] [--libm]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent.parent))

import numpy as np  # noqa: E402

import oracle as O  # noqa: E402
from streams import CONFIGS, fixture_path, train  # noqa: E402


def libm_name() -> str:
    try:
        return os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        return "unknown"


def write(num: int, libm: bool) -> None:
    cfg = CONFIGS[num]
    t0 = time.time()
    backend = O.OracleBackend()
    if libm:
        with O.libm_math():
            losses = train(cfg, backend)
    else:
        losses = train(cfg, backend)
    data = {
        "what": f"CPU-oracle loss per step, BASELINE config {num} ({cfg.key}), fresh batch per step",
        "seed": cfg.data_seed, "model_seed": cfg.model_seed, "batch": cfg.batch,
        "steps": cfg.steps, "lr": cfg.lr, "momentum": cfg.momentum,
        "exp_log": (f"platform libm expf/logf ({libm_name()})" if libm
                    else "oracle named methods (correctly rounded, vkml_oracle.c or_expf/or_logf)"),
        "losses_f32_bits": [f"{int(b):08x}" for b in losses.view(np.uint32)],
        "losses": [float(v) for v in losses],
    }
    path = fixture_path(cfg, libm)
    path.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {path.name} ({time.time() - t0:.0f} s): first {losses[0]:.6f} "
          f"last {losses[-1]:.6f}", flush=True)


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--config", type=int, choices=sorted(CONFIGS), action="append")
    p.add_argument("--libm", action="store_true", help="write the libm trajectory only")
    args = p.parse_args()
    for num in args.config or sorted(CONFIGS):
        write(num, args.libm)


if __name__ == "__main__":
    main()
