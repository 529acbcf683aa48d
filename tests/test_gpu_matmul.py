"""GPU parity of the WO projection (al_mul_mat_q4_0_f32) against the oracle's
restatement of nnml's Q4_0 x Q8_0 mul_mat (quantize_row_q8_0,
nnml_vec_dot_q4_0_q8_0: nnml/src/ops/arm/arm.cpp:1819-1848, 401;
forward_mul_mat_generic: nnml/src/ops/arm/common.cpp:120).

Bars: the activation quantization and every block's integer dot product are
exact, so with unit scales the device result equals the oracle's bit for bit.
With real scales only the float32 summation order differs (the oracle sums
blocks in order, the device per lane then across the wavefront), so both lie
within (K / 32 + 16) * 2^-23 * sum_k |w_k x_k| of the exact product of the
dequantized operands, and that is the bar between them.
"""
import numpy as np
import pytest

from arclight_amd import abi
from oracle import oracle as O
from tests.test_oracle_q4 import abs_bound, dequant_q4_0, dequant_q8_0

pytestmark = pytest.mark.gpu
EPS32 = 2.0 ** -24


def _case(name):
    print(f"\n[case] {name}", flush=True)


def _run(w, x, x_pad=0, y_pad=0):
    from arclight_amd import device, fattn, matmul
    N, nb = w.shape
    K = 32 * nb
    T = x.shape[0]
    wm = matmul.Q4_0Matrix(w.view(np.uint8), K, N)
    xs = np.zeros((T, K + x_pad), np.float32)
    xs[:, :K] = x
    xb = device.DeviceTensor.from_numpy(xs)
    xd = device.DeviceTensor(xb.buf, abi.AL_TYPE_F32, (T, K), ((K + x_pad) * 4, 4))
    yb = device.DeviceTensor.empty((T, N + y_pad), np.float32)
    yd = device.DeviceTensor(yb.buf, abi.AL_TYPE_F32, (T, N), ((N + y_pad) * 4, 4))
    matmul.mul_mat_q4_0(wm, xd, yd)
    device.synchronize()
    fattn.device_errors()
    return yb.numpy(np.float32)[:, :N]


def _activations(rng, T, K):
    # attention outputs: per-token magnitude spread, a few outliers per row
    x = rng.standard_normal((T, K)) * rng.uniform(0.02, 3.0, (T, 1))
    x[rng.random((T, K)) < 1e-3] *= 40.0
    return x.astype(np.float32)


@pytest.mark.parametrize("K,N,T", [(4096, 2560, 1), (4096, 2560, 4), (4096, 2560, 8), (4096, 2560, 64),
                                   (8192, 5120, 1), (8192, 5120, 5), (12288, 130, 3), (16384, 257, 64)])
def test_wo_matches_oracle(gpu, K, N, T):
    _case(f"wo K={K} N={N} T={T}")
    rng = np.random.default_rng(K * 7 + N * 3 + T)
    w = O.random_q4_0(rng, N, K)
    x = _activations(rng, T, K)
    got = _run(w, x)
    want = O.mul_mat_q4_0(w, x)
    bound = (K // 32 + 16) * 2 * EPS32 * abs_bound(dequant_q4_0(w), dequant_q8_0(O.quantize_q8_0(x)))
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), f"worst {err.max():.3e} at {np.unravel_index((err - bound).argmax(), err.shape)}"
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-6, rel


@pytest.mark.parametrize("K,N,T", [(4096, 301, 1), (4096, 301, 2), (4096, 301, 8), (8192, 77, 5), (8192, 77, 9)])
def test_wo_unit_scales_bit_exact(gpu, K, N, T):
    """Unit weight scales and activations whose every block has step 1:
    the result is the integer dot product, which both sides must hit
    exactly; half-integer activations check the device's ties-to-even.
    T = 1 (quarter blocks per thread), 2..8 (whole blocks per thread, one
    launch) and 9 (the quantization launch) each quantize differently; a
    block of zeros and one of negative zeros (scale 0) are among them."""
    _case(f"wo exact K={K} N={N} T={T}")
    rng = np.random.default_rng(N + T)
    w = O.random_q4_0(rng, N, K)
    w["d"] = np.float16(1.0).view(np.uint16)
    x = (rng.integers(-253, 254, size=(T, K)) / 2.0).astype(np.float32)
    x[:, ::32] = 127.0
    x[T - 1, 32:64] = 0.0
    x[0, 96:128] = -0.0
    got = _run(w, x, x_pad=4, y_pad=3)
    want = O.mul_mat_q4_0(w, x)
    assert np.array_equal(got, want)
    q = O.quantize_q8_0(x)
    nib = np.concatenate([(w["qs"] & 0x0F).astype(np.int64) - 8, (w["qs"] >> 4).astype(np.int64) - 8], -1)
    ints = q["qs"].reshape(T, -1).astype(np.int64) @ nib.reshape(N, -1).T
    assert np.array_equal(got, ints.astype(np.float32))


def test_wo_repeated_calls_reuse_scratch(gpu):
    """A large call then a small one: the small call's result does not see
    the earlier call's quantized activations."""
    _case("wo scratch reuse")
    rng = np.random.default_rng(5)
    big_w, big_x = O.random_q4_0(rng, 64, 16384), _activations(rng, 64, 16384)
    small_w, small_x = O.random_q4_0(rng, 2560, 4096), _activations(rng, 1, 4096)
    _run(big_w, big_x)
    got = _run(small_w, small_x)
    want = O.mul_mat_q4_0(small_w, small_x)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.parametrize("K,N,T,status", [(2048, 64, 1, abi.AL_ERR_UNSUPPORTED), (20480, 64, 1, abi.AL_ERR_UNSUPPORTED),
                                          (4096, 64, 65, abi.AL_ERR_UNSUPPORTED)])
def test_wo_rejects_unsupported_shapes(gpu, K, N, T, status):
    from arclight_amd import _lib, device, matmul
    rng = np.random.default_rng(0)
    wm = matmul.Q4_0Matrix(O.random_q4_0(rng, N, K).view(np.uint8), K, N)
    x = device.DeviceTensor.empty((T, K), np.float32)
    with pytest.raises(_lib.ArclightError) as e:
        matmul.mul_mat_q4_0(wm, x)
    assert e.value.status == status


def test_wo_rejects_mismatched_operands(gpu):
    from arclight_amd import _lib, device, matmul
    rng = np.random.default_rng(1)
    wm = matmul.Q4_0Matrix(O.random_q4_0(rng, 32, 4096).view(np.uint8), 4096, 32)
    x = device.DeviceTensor.empty((2, 4096), np.float32)
    y = device.DeviceTensor.empty((3, 32), np.float32)
    with pytest.raises(_lib.ArclightError) as e:
        matmul.mul_mat_q4_0(wm, x, y)
    assert e.value.status == abi.AL_ERR_INVALID
    xh = device.DeviceTensor.empty((2, 4096), np.float16)
    with pytest.raises(_lib.ArclightError) as e:
        matmul.mul_mat_q4_0(wm, xh)
    assert e.value.status == abi.AL_ERR_UNSUPPORTED


def test_q8_scale_inverse_equals_division(gpu):
    """The quantization's 1 / d (v_rcp_f32 and one Newton step for d in
    [2^-126, 2^126), the division elsewhere) equals the IEEE quotient for
    every non-negative float up to +inf, bit for bit."""
    from arclight_amd import matmul
    _case("Q8_0 scale inverse over every float")
    assert matmul.check_inverse() == 0
