"""The committed CPU-oracle loss trajectories of configs 1 and 5
(tests/golden/config*_losses*.json, written by
tests/golden/make_training_losses.py) against live runs of the CPU oracle:
their first steps must be the same bits, so the fixtures the device tests and
bench.py compare against are the oracle's, not stale copies. CPU only."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import streams as S
from oracle import OracleBackend


@pytest.mark.parametrize("num", [1, 5])
@pytest.mark.parametrize("libm", [False, True])
def test_fixture_describes_the_config(num, libm):
    cfg = S.CONFIGS[num]
    data = S.fixture(cfg, libm)
    assert (data["seed"], data["model_seed"], data["batch"], data["steps"]) == \
        (cfg.data_seed, cfg.model_seed, cfg.batch, cfg.steps)
    assert (data["lr"], data["momentum"]) == (cfg.lr, cfg.momentum)
    assert ("libm" in data["exp_log"]) == libm
    losses = S.oracle_losses(cfg, libm)
    assert losses.shape == (cfg.steps,) and np.all(np.isfinite(losses))
    # the decimal copy is the same numbers
    assert np.array(data["losses"], np.float32).tobytes() == losses.tobytes()
    # cross-entropy over C classes starts near log(C)
    assert abs(float(losses[0]) - np.log(cfg.classes)) < 0.1


def test_config1_fixture_matches_a_live_oracle_run():
    got = S.train(S.CONFIG1, OracleBackend())
    assert got.tobytes() == S.oracle_losses(S.CONFIG1).tobytes()


def test_config1_libm_fixture_matches_a_live_oracle_run():
    with O.libm_math():
        got = S.train(S.CONFIG1, OracleBackend())
    assert got.tobytes() == S.oracle_losses(S.CONFIG1, libm=True).tobytes()


@pytest.mark.parametrize("libm", [False, True])
def test_config5_fixture_matches_a_live_oracle_run(libm):
    if libm:
        with O.libm_math():
            got = S.train(S.CONFIG5, OracleBackend(), steps=2)
    else:
        got = S.train(S.CONFIG5, OracleBackend(), steps=2)
    assert got.tobytes() == S.oracle_losses(S.CONFIG5, libm)[:2].tobytes()


def test_libm_switch_changes_only_exp_and_log():
    """The switch reaches exp/log and nothing else: a matmul and a sum are the
    same bits either way, exp differs from the named method on a small
    fraction of inputs, never by more than one ulp."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((17, 40)).astype(np.float32)
    b = rng.standard_normal((40, 9)).astype(np.float32)
    x = rng.uniform(-30, 30, 200_000).astype(np.float32)
    named = (O.matmul(a, b), O.sum(a, [1]), O.expf(x), O.logf(np.abs(x) + 1e-3))
    with O.libm_math():
        libm = (O.matmul(a, b), O.sum(a, [1]), O.expf(x), O.logf(np.abs(x) + 1e-3))
    assert named[0].tobytes() == libm[0].tobytes()
    assert named[1].tobytes() == libm[1].tobytes()
    for n_, l_ in zip(named[2:], libm[2:]):
        ulps = np.abs(n_.view(np.int32).astype(np.int64) - l_.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1 and 0 < np.count_nonzero(ulps) < x.size // 100
    # and the switch is off again outside the context
    assert O.expf(x).tobytes() == named[2].tobytes()


def test_oracle_trajectories_separate_with_the_libm():
    """How far two valid builds of the reference's CPU arithmetic move the
    training trajectories (the oracle's named exp/log against glibc's
    expf/logf, everything else the same bits). Config 1's MLP is stable: the
    two stay within 1e-6 for 100 steps. Config 5's CNN is chaotic at the
    rounding level: bit-identical for the first 11 steps, past the north
    star's 1e-4 from step 24, ~1.8e-3 apart at step 86. This spread is the
    envelope the device's fast numerics are held to over 100 steps of config
    5 (tests/test_gpu_training.py)."""
    c1 = S.max_drift(S.oracle_losses(S.CONFIG1), S.oracle_losses(S.CONFIG1, libm=True))
    assert c1[0] <= 1e-6
    a, b = S.oracle_losses(S.CONFIG5), S.oracle_losses(S.CONFIG5, libm=True)
    d = np.abs(a.astype(np.float64) - b.astype(np.float64))
    assert a[:11].tobytes() == b[:11].tobytes() and a[11] != b[11]
    assert int(np.argmax(d > 1e-4)) == 24
    assert S.max_drift(a, b) == (d.max(), 86) and 1.5e-3 < d.max() < 2.5e-3
