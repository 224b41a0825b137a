"""Pins the oracle's 16-bit conversions and non-finite test against numpy/torch."""
import numpy as np
import pytest
import torch


def test_f32_to_f16_matches_numpy_rounding(oracle, golden_dir):
    """export.py:33 writes astype('<f2'); the golden cases hold numpy's rounding."""
    z = np.load(golden_dir / "f16_cases.npz")
    got = oracle.f32_to_f16(z["x"])
    assert (got == z["f16_bits"]).all()


def test_f32_to_f16_exhaustive_halfway_points(oracle):
    """Every midpoint between adjacent finite halves (ties to even) and its neighbours."""
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2)[:-1]
    x = np.concatenate([mid, -mid]).astype(np.float32)
    x = np.concatenate([x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))])
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    assert (oracle.f32_to_f16(x) == expect).all()


def test_f32_to_bf16_matches_torch(oracle):
    rng = np.random.RandomState(1)
    x = rng.randint(0, 2 ** 32, size=300000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x[np.isfinite(x)], np.array([np.inf, -np.inf, 0.0, -0.0], np.float32)])
    expect = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (oracle.f32_to_bf16(x) == expect).all()


def test_nan_conversions_are_quiet_nans(oracle):
    x = np.array([np.nan, -np.nan], np.float32)
    assert np.isnan(oracle.f32_to_f16(x).view(np.float16)).all()
    assert (oracle.f32_to_bf16(x) == 0x7FC0).all()  # torch c10::BFloat16
    assert torch.isnan(torch.from_numpy(oracle.f32_to_bf16(x).view(np.int16)).view(torch.bfloat16)).all()


@pytest.mark.parametrize("dtype", [np.float32, np.float16, "bf16"])
def test_nonfinite_any_matches_torch_isfinite(oracle, dtype):
    """Restates optimizer.py:49-51: any(not isfinite(g))."""
    rng = np.random.RandomState(0)
    for trial in range(40):
        n = int(rng.randint(1, 5000))
        g = rng.randn(n).astype(np.float32) * 10 ** rng.uniform(-8, 4)
        k = int(rng.randint(0, 4))
        for _ in range(k):
            g[rng.randint(n)] = rng.choice([np.inf, -np.inf, np.nan])
        if dtype == "bf16":
            t = torch.from_numpy(g).to(torch.bfloat16)
            arr = t.view(torch.int16).numpy().view(np.uint16)
            got = oracle.nonfinite_any(arr, oracle.DTYPE_BF16)
        else:
            with np.errstate(over="ignore"):
                arr = g.astype(dtype)
            t = torch.from_numpy(arr)
            got = oracle.nonfinite_any(arr)
        assert got == (not bool(torch.isfinite(t).all()))


def test_nonfinite_fp16_boundaries(oracle):
    finite = np.array([65504.0, -65504.0, 6e-8, 0.0], np.float16)
    assert not oracle.nonfinite_any(finite)
    assert oracle.nonfinite_any(np.array([1.0, np.inf], np.float16))
    assert oracle.nonfinite_any(np.array([np.nan, 1.0], np.float16))


def test_norm_decision_equals_element_decision(oracle):
    """disk.py:466-468 decides on sqrt(sum(g.double()**2)); that is non-finite iff an element is."""
    rng = np.random.RandomState(5)
    g = (rng.randn(10000) * 1e37).astype(np.float32)  # huge but finite: double sum stays finite
    g = g[np.isfinite(g)]
    norm = np.sqrt(sum(float(np.square(p.astype(np.float64)).sum()) for p in np.array_split(g, 7)))
    assert np.isfinite(norm) and not oracle.nonfinite_any(g)
    g[17] = np.inf
    norm = np.sqrt(float(np.square(g.astype(np.float64)).sum()))
    assert not np.isfinite(norm) and oracle.nonfinite_any(g)
