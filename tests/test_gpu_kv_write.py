"""GPU KV write (al_set_rows_f32_f16) bit-exact against the oracle's
restatement of nnml_compute_forward_set_rows_f32 (ops.cpp:135-181), and the
f32 -> f16 RNE conversion against numpy."""
import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _special_f32(rng, n):
    x = rng.standard_normal(n).astype(np.float32) * rng.choice([1e-6, 1e-3, 1, 100, 6e4], n).astype(np.float32)
    bits = rng.integers(0, 2**32, size=n // 4, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x[: n // 4] = bits            # arbitrary patterns: NaN, inf, subnormal, huge
    ties = np.float32(1.0) + np.float32(2.0 ** -11) * rng.integers(1, 1000, n // 8).astype(np.float32)
    x[n // 4: n // 4 + n // 8] = ties
    x[-6:] = [65504.0, 65519.99, 65520.0, 2.0 ** -25, 2.0 ** -24 * 1.5, -0.0]
    return x


def test_f32_to_f16_bits_match_numpy(gpu):
    from arclight_amd import device
    from arclight_amd._lib import call
    rng = np.random.default_rng(0)
    x = _special_f32(rng, 1 << 20)
    print("\n[case] f32_to_f16 1M", flush=True)
    dx = device.DeviceBuffer(x.nbytes)
    dx.upload(x)
    dh = device.DeviceBuffer(x.size * 2)
    call("al_util_f32_to_f16", dh.ptr, dx.ptr, x.size, None)
    got = np.empty(x.size, dtype=np.uint16)
    dh.download(got)
    with np.errstate(over="ignore"):                                  # values past f16 range round to inf
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got[nan].view(np.float16)).all()


@pytest.mark.parametrize("idx_dtype", [np.int64, np.int32])
def test_set_rows_matches_oracle(gpu, idx_dtype):
    from arclight_amd import device, fattn
    rng = np.random.default_rng(1)
    n_cells, nc, n = 1000, 1024, 37          # a Qwen3 layer: 8 kv heads x 128
    cache = rng.standard_normal((n_cells, nc)).astype(np.float16).view(np.uint16)
    rows = _special_f32(rng, n * nc).reshape(n, nc)
    idx = rng.choice(n_cells, size=n, replace=False).astype(idx_dtype)
    want = O.set_rows(cache, rows, idx)
    print(f"\n[case] set_rows {idx_dtype.__name__}", flush=True)
    dcache = device.DeviceTensor.from_numpy(cache)
    drows = device.DeviceTensor.from_numpy(rows)
    didx = device.DeviceTensor.from_numpy(idx)
    fattn.set_rows(dcache, drows, didx)
    device.synchronize()
    fattn.device_errors()
    got = dcache.numpy(np.uint16)
    nanw = np.isnan(want.view(np.float16))
    assert np.array_equal(np.isnan(got.view(np.float16)), nanw)
    assert np.array_equal(got[~nanw], want[~nanw])


def test_set_rows_reports_bad_index(gpu):
    from arclight_amd import device, fattn
    from arclight_amd._lib import ArclightError
    cache = np.zeros((16, 128), dtype=np.uint16)
    rows = np.ones((2, 128), dtype=np.float32)
    idx = np.array([3, 16], dtype=np.int64)
    print("\n[case] set_rows bad index", flush=True)
    dcache = device.DeviceTensor.from_numpy(cache)
    fattn.set_rows(dcache, device.DeviceTensor.from_numpy(rows), device.DeviceTensor.from_numpy(idx))
    device.synchronize()
    with pytest.raises(ArclightError) as ei:
        fattn.device_errors()
    assert ei.value.status == abi.AL_ERR_INVALID
    fattn.device_errors()                    # cleared
    got = dcache.numpy(np.uint16).view(np.float16)
    assert (got[3] == 1).all() and (np.delete(got, 3, axis=0) == 0).all()
