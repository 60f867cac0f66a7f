"""The oracle (oracle/nd_oracle.c) against golden vectors written by the
reference engine's own code (tests/golden/gen_golden.py): bit-exact."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import ndoracle as O  # noqa: E402
from gen_golden import SESSIONS, run_session  # noqa: E402

G = np.load(os.path.join(HERE, "golden", "golden.npz"))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_exp_pairs_fixture_bit_exact():
    """nd_expf_pair on the 1024 captured softmax argument pairs
    (esp32/main/exp_pairs.h) - the pair form equals two scalar calls."""
    xin, ref = G["exp_pairs_in"], G["exp_pairs_out"]
    got = np.array([O.lib().ndo_expf(float(x)) for x in xin], np.float32)
    assert np.array_equal(bits(got), bits(ref))


def test_exp_and_sigmoid_sweep_bit_exact():
    xs = G["exp_in"]
    e = np.array([O.lib().ndo_expf(float(x)) for x in xs], np.float32)
    s = np.array([O.lib().ndo_sigmoid(float(x)) for x in xs], np.float32)
    assert np.array_equal(bits(e), bits(G["exp_out"]))
    assert np.array_equal(bits(s), bits(G["sig_out"]))


def test_kv_store_rows_bit_exact():
    for row, n, codes, sc in zip(G["store_rows"], G["store_len"], G["store_codes"], G["store_scales"]):
        x = np.ascontiguousarray(row[:n], np.float32)
        d = np.zeros(n, np.int8)
        got_sc = O.lib().ndo_kv_quant_row(x, n, d)
        assert np.float32(got_sc).view(np.uint32) == np.float32(sc).view(np.uint32)
        assert np.array_equal(d, codes[:n])


@pytest.mark.parametrize("name", sorted(SESSIONS))
def test_session_bit_exact(name):
    spec = SESSIONS[name]
    S = O.OracleSession(*spec["geom"])
    out, saved = run_session(S, spec)
    for p in saved.values():
        O.lib().ndo_prefix_free(p)
    assert out.shape == G["sess_" + name].shape
    assert np.array_equal(bits(out), bits(G["sess_" + name]))
    k, v, ks, vs = S.cache()
    kvsum = [int(k.astype(np.int64).sum()), int(v.astype(np.int64).sum()),
             int(np.abs(k.astype(np.int64)).sum()), int(np.abs(v.astype(np.int64)).sum())]
    assert kvsum == list(G["sess_" + name + "_kvsum"])
    if "front" in spec:
        from gen_golden import hist_blob
        assert np.array_equal(bits(hist_blob(S)), bits(G["sess_" + name + "_hist"]))
