"""DynamicLossScale (product) vs the reference's known answers and the oracle."""
import json
import random

import pytest

from morph_amd.precision import DynamicLossScale


def test_reference_kat_overflow_halves(golden_dir):
    """tests/test_fp16.py:59-72: first attempt at 128 overflows, retry at 64, stored 64."""
    kat = json.loads((golden_dir / "loss_scale.json").read_text())["reference_kat"]
    s = DynamicLossScale()
    seen = [s.scale]
    s.overflow()
    seen.append(s.scale)
    assert seen == kat["scales_seen"]
    s.success()
    assert s.state_dict()["scale"] == kat["stored_scale"]


def test_config4_sequence(golden_dir):
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    s = DynamicLossScale(cfg["initial"], cfg["growth_interval"])
    seen = []
    for step in range(1, cfg["steps"] + 1):
        seen.append(s.scale)
        s.overflow() if step in cfg["overflow_steps"] else s.success()
    assert seen == cfg["scale_before_step"]
    assert s.scale == cfg["final_scale"]


def test_growth_cap_and_floor():
    s = DynamicLossScale(16384., growth_interval=3)
    for _ in range(3):
        s.success()
    assert s.scale == 32768. and s.good_steps == 0
    for _ in range(9):
        s.success()
    assert s.scale == 65536.  # capped
    s = DynamicLossScale(2., growth_interval=5)
    s.overflow()
    assert s.scale == 1.
    with pytest.raises(FloatingPointError):
        s.overflow()
    assert s.scale == 1. and s.good_steps == 0


def test_matches_oracle_restatement_on_random_sequences(oracle):
    rng = random.Random(0)
    for trial in range(200):
        init = rng.choice([1., 2., 3., 128., 65536., 1000.])
        interval = rng.choice([1, 2, 3, 2000])
        a, b = DynamicLossScale(init, interval), oracle.LossScale(init, interval)
        for _ in range(rng.randint(1, 60)):
            if rng.random() < .3:
                ra = rb = None
                try:
                    a.overflow()
                except FloatingPointError as e:
                    ra = e
                try:
                    b.overflow()
                except FloatingPointError as e:
                    rb = e
                assert (ra is None) == (rb is None)
            else:
                a.success()
                b.success()
            assert a.state_dict() == b.state_dict()


def test_state_dict_roundtrip():
    s = DynamicLossScale(512., 7)
    s.success()
    t = DynamicLossScale()
    t.load_state_dict(s.state_dict())
    assert t.state_dict() == {"scale": 512., "good_steps": 1, "growth_interval": 7}


def test_bench_config4_expectation_matches_the_golden_sequence(golden_dir):
    """The overflow bench checks the device against bench.expected_config4_scales(): that
    expectation is the golden config-4 sequence (steps, overflow steps, scales, final state)."""
    import bench
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    assert bench.CONFIG4_STEPS == cfg["steps"]
    assert list(bench.CONFIG4_OVERFLOW) == cfg["overflow_steps"]
    assert bench.LOSS_SCALE == cfg["initial"]
    scales, state = bench.expected_config4_scales()
    assert scales == cfg["scale_before_step"]
    assert state["scale"] == cfg["final_scale"]
