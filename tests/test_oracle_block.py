"""Pins the oracle's fused block (oracle_moe_block: out = x1 +
MoE(RMSNorm(x1) * gamma)) and its RMSNorm restatement before they are
trusted.

1. Golden vectors: bit-for-bit agreement with the reference's own ln2
   RMSNormLayer -> MoELayer -> Tensor::add_into (oracle/_ref/ref_driver
   block; layers/TransformerBlock.cpp:42-46) on every fixture in
   tests/golden/block/: out, the normalised rows, the per-token 1/rms and
   the routing (digests; full arrays where small).  cfg3 is checked through
   the same router/dispatch restatement and per-token rows.
2. Mathematics: gamma = 1 equals the unscaled restatement; a power-of-two
   gamma scales the output exactly; a constant row a has 1/rms =
   1/sqrt(a^2 + eps); rows of any scale normalise to RMS 1 (up to eps).
"""
import glob
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

BLK = os.path.join(os.path.dirname(__file__), "golden", "block")
FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(BLK, "*.npz")))


def canonical_digest(a):
    a = np.array(a, copy=True)
    if a.dtype == np.float32:
        a[np.isnan(a)] = np.float32("nan")
    return wl.digest(a)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_every_block_case_has_a_fixture():
    assert sorted(C.BLOCK_CASES) == FIXTURES


@pytest.mark.parametrize("name", [n for n in FIXTURES if n != "cfg3"])
def test_block_matches_reference(name):
    case = C.ALL_CASES[name]
    fx = np.load(os.path.join(BLK, name + ".npz"), allow_pickle=False)
    inp, x1, gamma = C.build_block_inputs(case)
    out = O.block(inp, x1, gamma, C.BLOCK_EPS)
    for n in ("out", "xn", "rstd", "idx", "topp", "perm"):
        assert canonical_digest(out[n]) == str(fx["sha_" + n]), n
    assert np.array_equal(out["counts"], fx["counts"])
    assert same_bits(out["rstd"], fx["rstd"])
    rows = fx["rows"]
    assert same_bits(out["out"][rows], fx["out_rows"])
    assert same_bits(out["xn"][rows], fx["xn_rows"])


def test_block_cfg3_matches_reference():
    case = C.ALL_CASES["cfg3"]
    fx = np.load(os.path.join(BLK, "cfg3.npz"), allow_pickle=False)
    inp, x1, gamma = C.build_block_inputs(case)
    xn, rstd = O.rmsnorm_scaled(x1, gamma, C.BLOCK_EPS)
    assert canonical_digest(xn) == str(fx["sha_xn"])
    assert same_bits(rstd, fx["rstd"])
    probs = O.softmax(O.router_logits(xn, inp.Wr, inp.br))
    idx, topp = O.topk(probs, case.cfg.k)
    counts, _, perm = O.dispatch(idx, case.cfg.E)
    assert np.array_equal(counts, fx["counts"])
    for n, a in (("idx", idx), ("topp", topp), ("perm", perm)):
        assert canonical_digest(a) == str(fx["sha_" + n]), n
    rows = fx["rows"]
    xin = wl.MoEInputs(case.cfg, xn, inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd,
                       inp.bd, inp.raw)
    y = O.tokens(xin, idx, topp, rows)
    assert same_bits(x1[rows] + y, fx["out_rows"])


def test_rmsnorm_unit_gamma_is_the_unscaled_restatement():
    x = wl.normal_f32(5, 1, 64 * 192).reshape(64, 192) * np.float32(3.0)
    out, _ = O.rmsnorm_scaled(x, np.ones(192, np.float32))
    assert same_bits(out, O.rmsnorm(x))


def test_rmsnorm_closed_forms():
    x = wl.normal_f32(6, 1, 32 * 128).reshape(32, 128)
    g = np.float32(1.0) + np.float32(0.3) * wl.normal_f32(7, 1, 128)
    out, r = O.rmsnorm_scaled(x, g)
    out2, r2 = O.rmsnorm_scaled(x, g * np.float32(2.0))
    assert same_bits(r, r2) and same_bits(out2, out * np.float32(2.0))   # power-of-two gamma
    a = np.full((3, 64), [[0.5], [2.0], [-3.0]], np.float32)
    _, ra = O.rmsnorm_scaled(a, np.ones(64, np.float32), 1e-5)
    want = (1.0 / np.sqrt(np.array([0.25, 4.0, 9.0]) + 1e-5)).astype(np.float32)
    assert np.allclose(ra, want, rtol=2e-7, atol=0)
    xs = x * np.exp2(np.arange(32, dtype=np.float32) % 7 - 3)[:, None]
    n1, _ = O.rmsnorm_scaled(xs, np.ones(128, np.float32))
    rms = np.sqrt(np.mean(n1.astype(np.float64) ** 2, axis=1))
    ms = np.mean(xs.astype(np.float64) ** 2, axis=1)
    assert np.allclose(rms, np.sqrt(ms / (ms + 1e-5)), rtol=1e-5)
