"""Shared helpers for the flash-attention parity tests."""
import numpy as np

from arclight_amd import abi

MAX_ABS = 2e-3      # parity bar on the fp32 output: max-abs error ...
REL_L2 = 1e-3       # ... and relative L2 error, against oracle O2


def rel_l2(a, b):
    m = np.isfinite(b)
    return float(np.linalg.norm((a - b)[m]) / max(np.linalg.norm(b[m]), 1e-30))


def assert_parity(got, ref, max_abs=MAX_ABS, rel=REL_L2, what=""):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{what}: NaN pattern differs"
    m = ~nan_ref
    if m.any():
        err = float(np.abs(got[m] - ref[m]).max())
        r = rel_l2(got[m], ref[m])
        assert err <= max_abs, f"{what}: max-abs {err:.3e} > {max_abs:.1e} (rel-L2 {r:.3e})"
        assert r <= rel, f"{what}: rel-L2 {r:.3e} > {rel:.1e} (max-abs {err:.3e})"


def run_gpu(q, k, v, mask=None, sinks=None, *, scale, max_bias=0.0, logit_softcap=0.0, kv_len=0,
            causal_pos0=-1, prec=abi.AL_PREC_F32, workspace=None):
    """Uploads host operands, runs al_fattn_f16 on the default stream, returns dst."""
    from arclight_amd import device, fattn
    dq = fattn.upload_q(q)
    dk = fattn.upload_kv(k)
    dv = fattn.upload_kv(v)
    dm = fattn.upload_mask(mask) if mask is not None else None
    ds = fattn.upload_sinks(sinks) if sinks is not None else None
    dst = fattn.flash_attn_ext(dq, dk, dv, dm, ds, scale=scale, max_bias=max_bias, logit_softcap=logit_softcap,
                               kv_len=kv_len, causal_pos0=causal_pos0, prec=prec, workspace=workspace)
    device.synchronize()
    fattn.device_errors()                  # no kernel recorded an error (raises if one did)
    return dst.numpy(np.float32)
