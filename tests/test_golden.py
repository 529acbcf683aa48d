"""Known-answer vectors (tests/golden/fattn_golden.npz, expected outputs from
the float64 brute-force oracle) checked on the CPU against the parity oracle
and on the GPU against the HIP path through the C ABI."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.fattn_cases import assert_parity, run_gpu
from tests.golden.make_golden import digest

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "fattn_golden.npz")


def load_cases():
    z = np.load(FIXTURE)
    meta = json.loads(z["meta"].tobytes().decode())
    out = []
    for m in meta:
        q, k, v = O.make_inputs(m["seed"], **m["shape"])
        assert digest(q, k, v) == m["qkv_sha256"], f"{m['name']}: input generator changed"
        out.append(dict(name=m["name"], q=q, k=k, v=v,
                        mask=z[m["name"] + ".mask"] if m["has_mask"] else None,
                        sinks=z[m["name"] + ".sinks"] if m["has_sinks"] else None,
                        kw=m["kw"], want=z[m["name"] + ".expected"]))
    return out


CASES = load_cases()
IDS = [c["name"] for c in CASES]


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_oracle_o2_reproduces_golden(c):
    got = O.attention(c["q"], c["k"], c["v"], c["mask"], c["sinks"], **c["kw"])
    assert_parity(got, c["want"], max_abs=2e-5, rel=1e-5, what=c["name"])


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_hip_path_reproduces_golden(gpu, c):
    got = run_gpu(c["q"], c["k"], c["v"], c["mask"], c["sinks"], **c["kw"])
    assert_parity(got, c["want"], what=c["name"])
