"""The committed golden vectors (tests/golden/*.npz, written by
tests/golden/make_golden.py from the fp64 token recurrence) against both CPU
oracles, plus the recorded input digests."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import cpu as coracle
from oracle import gdn_ref as R

HERE = os.path.join(os.path.dirname(__file__), "golden")
FIXTURES = ["cfg0.npz", "varlen_h0.npz"]


def _load(name):
    z = np.load(os.path.join(HERE, name))
    f = lambda b: (b.astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    a = dict(q=f(z["q_bf16"]), k=f(z["k_bf16"]), v=f(z["v_bf16"]), g=z["g"], beta=z["beta"],
             initial_state=z["h0"] if "h0" in z else None,
             cu_seqlens=z["cu_seqlens"] if "cu_seqlens" in z else None)
    return z, a


@pytest.mark.parametrize("name", FIXTURES)
def test_input_digest(name):
    z = np.load(os.path.join(HERE, name))
    h = hashlib.sha256()
    for key in sorted(k for k in z.files if k not in ("o", "state")):
        h.update(np.ascontiguousarray(z[key]).tobytes())
    with open(os.path.join(HERE, "sha256.json")) as f:
        assert json.load(f)[name] == h.hexdigest()


@pytest.mark.parametrize("name", FIXTURES)
def test_numpy_oracle_reproduces_golden(name):
    z, a = _load(name)
    o, S = R.recurrent(**a, dtype=np.float64)
    np.testing.assert_allclose(o, z["o"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(S, z["state"], rtol=1e-6, atol=1e-7)
    oc, Sc = R.chunked(**a)
    np.testing.assert_allclose(oc, z["o"], rtol=1e-4, atol=1e-5)
    assert np.linalg.norm(Sc - z["state"]) / np.linalg.norm(z["state"]) < 1e-5


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("kind", ["chunk", "recurrent"])
def test_c_oracle_reproduces_golden(name, kind):
    z, a = _load(name)
    o, S = coracle.run(kind, **a, threads=2)
    np.testing.assert_allclose(o, z["o"], rtol=1e-4, atol=1e-5)
    assert np.linalg.norm(S - z["state"]) / np.linalg.norm(z["state"]) < 1e-5


def test_cfg0_shape_matches_baseline_config():
    z, a = _load("cfg0.npz")
    assert a["q"].shape == (1, 256, 4, 64) and a["v"].shape == (1, 256, 4, 64)
    assert z["state"].shape == (1, 4, 64, 64) and a["initial_state"] is None
