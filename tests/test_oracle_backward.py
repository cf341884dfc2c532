"""Pins the CPU oracle's MoE backward (oracle_moe_backward) before it is trusted.

1. Golden vectors: bit-for-bit agreement (NaN payloads aside) of dx and all
   2+6E parameter gradients with the reference's own CPU backward
   (oracle/_ref/ref_driver backward: MoELayer::forward_into then
   backward_into, layers/MoELayer.cpp:130-223) on every fixture in
   tests/golden/backward/, including dout = 1 on the shape of the
   reference's backward test (tests/networkTest/moeTests.cpp:22-39).
2. Mathematics: central finite differences of an independent float64
   forward of the loss the reference differentiates,
       L = sum(dy * y) + 0.01 * E * sum_e f_e * mean_t P[t, e],
   with f_e = counts_e / N held fixed (the load-balance term whose gradient
   layers/MoELayer.cpp:193-200 adds), against every gradient the oracle
   returns; softmax-Jacobian and routing invariants.
3. Planted mistakes: copies of the oracle built with one ORACLE_PLANT_*
   macro each are rejected by both checks above.
"""
import glob
import os
import subprocess

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

BWD = os.path.join(os.path.dirname(__file__), "golden", "backward")
NAMES = ("dx",) + O.GRAD_NAMES
FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(BWD, "*.npz")))


def canonical_digest(a):
    a = np.array(a, dtype=np.float32, copy=True)
    a[np.isnan(a)] = np.float32("nan")
    return wl.digest(a)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))


def test_every_backward_case_has_a_fixture():
    assert sorted(C.BACKWARD_CASES) == FIXTURES


@pytest.mark.parametrize("name", FIXTURES)
def test_backward_matches_reference(name):
    case = C.ALL_CASES[name]
    fx = np.load(os.path.join(BWD, name + ".npz"), allow_pickle=False)
    inp = C.build_inputs(case)
    out = O.backward(inp, C.build_dy(case))
    for n in NAMES:
        assert canonical_digest(out[n]) == str(fx["sha_" + n]), n
        if n in fx.files:
            assert same_bits(out[n], fx[n]), n
    assert same_bits(out["dx"][fx["rows"]], fx["dx_rows"])
    for n in O.GRAD_NAMES:
        assert same_bits(out[n].reshape(-1)[fx[n + "_at"]], fx[n + "_val"]), n


# ------------------------------------------------------------ mathematics
def _small_problem(seed=3, N=10, Cc=6, H=5, E=4, k=2):
    rng = np.random.default_rng(seed)
    cfg = wl.MoEConfig("fd", N, Cc, E, k, H, "f32", "f32", "normal")
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    inp = wl.MoEInputs(cfg, f(N, Cc), 0.6 * f(Cc, E), 0.3 * f(E), 0.5 * f(E, Cc, H),
                       0.2 * f(E, H), 0.5 * f(E, Cc, H), 0.2 * f(E, H), 0.5 * f(E, H, Cc),
                       0.2 * f(E, Cc), None)
    return inp, f(N, Cc)


def _loss64(p, dy, k, counts):
    """float64 forward of the differentiated loss; routing by a stable sort
    of (-P, expert id), gates are the unnormalised top-k probabilities."""
    x, Wr, br, Wg, bg, Wu, bu, Wd, bd = p
    N, E = x.shape[0], Wr.shape[1]
    lg = x @ Wr + br
    P = np.exp(lg - lg.max(axis=1, keepdims=True))
    P /= P.sum(axis=1, keepdims=True)
    idx = np.argsort(-P, axis=1, kind="stable")[:, :k]
    y = np.zeros_like(x)
    for t in range(N):
        for e in idx[t]:
            g = x[t] @ Wg[e] + bg[e]
            u = x[t] @ Wu[e] + bu[e]
            y[t] += P[t, e] * (((g / (1 + np.exp(-g))) * u) @ Wd[e] + bd[e])
    f = counts / N
    return float(np.sum(dy * y) + 0.01 * E * np.sum(f * P.mean(axis=0))), P, idx


def _fd_mismatches(library=None):
    """Names of the gradients on which the oracle (or a planted copy)
    disagrees with float64 central differences of the loss."""
    inp, dy = _small_problem()
    cfg = inp.cfg
    fwd = O.forward(inp)
    out = O.backward(inp, dy, library)
    p64 = [np.asarray(a, np.float64).copy() for a in
           (inp.x, inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd, inp.bd)]
    counts = fwd["counts"].astype(np.float64)
    _, P, idx = _loss64(p64, dy.astype(np.float64), cfg.k, counts)
    # routing must be the oracle's and far from a tie, so no perturbation flips it
    assert np.array_equal(np.sort(idx, 1), np.sort(fwd["idx"], 1))
    srt = -np.sort(-P, axis=1)
    assert np.min(srt[:, cfg.k - 1] - srt[:, cfg.k]) > 1e-3
    assert np.min(P) > 1e-6   # no clamped probability (the clamp is 1e-7)
    h = 1e-6
    bad = []
    for pi, name in enumerate(NAMES):
        arr = p64[pi]
        fd = np.empty(arr.size)
        flat = arr.reshape(-1)
        for i in range(arr.size):
            keep = flat[i]
            flat[i] = keep + h
            lp = _loss64(p64, dy.astype(np.float64), cfg.k, counts)[0]
            flat[i] = keep - h
            lm = _loss64(p64, dy.astype(np.float64), cfg.k, counts)[0]
            flat[i] = keep
            fd[i] = (lp - lm) / (2 * h)
        got = np.asarray(out[name], np.float64).reshape(-1)
        scale = max(1.0, float(np.max(np.abs(fd))))
        if not np.allclose(got, fd, rtol=2e-4, atol=2e-5 * scale):
            bad.append(name)
    return bad


def test_backward_matches_finite_differences():
    assert _fd_mismatches() == []


PLANTS = {
    # macro: gradients the mistake must corrupt
    "ORACLE_PLANT_NO_LOAD_BALANCE": ("dx", "dWr", "dbr"),
    "ORACLE_PLANT_SILU_SIGN": ("dx", "dWg", "dbg"),
    "ORACLE_PLANT_UNGATED": ("dx", "dWg", "dWu", "dWd", "dbd"),
}


@pytest.mark.parametrize("macro", sorted(PLANTS))
def test_planted_mistakes_are_detected(macro, tmp_path):
    """Each planted copy of the oracle fails the finite-difference check on
    the gradients the mistake feeds, and the golden comparison."""
    so = tmp_path / "planted.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-std=c11", "-fPIC", "-shared",
                    "-D" + macro, "-o", str(so), os.path.join(O.ORACLE_DIR, "moe_oracle.c"),
                    "-lm"], check=True)
    planted = O.load_variant(str(so))
    bad = _fd_mismatches(planted)
    for name in PLANTS[macro]:
        assert name in bad, (macro, name, bad)
    case = C.ALL_CASES["ragged_k3"]
    fx = np.load(os.path.join(BWD, case.name + ".npz"), allow_pickle=False)
    out = O.backward(C.build_inputs(case), C.build_dy(case), planted)
    assert canonical_digest(out["dx"]) != str(fx["sha_dx"])


def test_router_bias_gradient_sums_to_zero():
    # Each row of the softmax Jacobian-vector product sums to
    # sum(dP*P) * (1 - sum(P)), which is rounding-level when no probability
    # is clamped; dbr is the sum of those rows.
    inp, dy = _small_problem(seed=5, N=64, E=8, k=3)
    out = O.backward(inp, dy)
    assert abs(float(out["dbr"].sum())) < 1e-5 * float(np.abs(out["dbr"]).sum())


def test_unchosen_experts_get_no_gradient():
    inp, dy = _small_problem(seed=7, N=32, E=6, k=2)
    inp.br[:] = np.array([9, 8, -9, -9, -9, -9], np.float32)   # experts 0, 1 always win
    fwd = O.forward(inp)
    assert list(fwd["counts"]) == [32, 32, 0, 0, 0, 0]
    out = O.backward(inp, dy)
    for n in ("dWg", "dbg", "dWu", "dbu", "dWd", "dbd"):
        assert np.all(out[n][2:] == 0) and np.any(out[n][:2] != 0), n


def test_single_expert_has_no_router_gradient_from_the_task():
    # E = k = 1: p = 1 for every token, so dL = p * (dP - dP*p) = 0 exactly
    # apart from the load-balance term, which is (0.01 * 1 * 1)/N for every
    # token and also cancels: dWr and dbr are exactly zero.
    case = C.ALL_CASES["single_expert"]
    out = O.backward(C.build_inputs(case), C.build_dy(case))
    assert np.all(out["dWr"] == 0) and np.all(out["dbr"] == 0)
