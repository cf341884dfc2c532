"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted.

1. Golden vectors: bit-for-bit agreement with the reference's own CPU MoE
   forward (oracle/_ref/ref_driver on the unmodified reference sources) on
   every committed fixture in tests/golden/.
2. Known answers from the reference's tests and mathematics: the matmul KAT
   of tests/utilsTest/tensorTests.cpp:228-242, softmax([1,2,3]) and its
   properties (:383-391), uniform / clamped / NaN rows (utils/Tensor.cpp:
   861-881), one-hot router weights, single-expert (p = 1) and
   all-experts-identical invariants, fp64 textbook SwiGLU.
3. Brute force: top-k as a stable sort of (-p, e); dispatch as a stable
   argsort of the flat expert ids.
4. Planted mistakes: a dropped router bias, the opposite tie rule and a
   renormalised gate are each shown to break the golden comparison, so the
   fixtures are sensitive to exactly those errors.
"""
import glob
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def fixture(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else a.dtype)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        nan = np.isnan(a) & np.isnan(b)
        return a.shape == b.shape and bool(np.all((bits(a) == bits(b)) | nan))
    return a.shape == b.shape and np.array_equal(a, b)


FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))
SMALL = [n for n in FIXTURES if C.ALL_CASES[n].full_arrays]
LARGE = [n for n in FIXTURES if not C.ALL_CASES[n].full_arrays]


@pytest.mark.parametrize("name", SMALL)
def test_oracle_matches_reference_small(name):
    case = C.ALL_CASES[name]
    fx = fixture(name)
    inp = C.build_inputs(case)
    out = O.forward(inp)
    for key in ("idx", "topp", "logits", "probs", "perm", "counts", "offsets"):
        assert same_bits(out[key].reshape(fx[key].shape), fx[key]), key
    for key in ("idx", "topp", "perm", "logits", "probs", "y"):
        if key == "y" and case.tweak == "nan_rows":
            continue   # NaN payload bits are not part of the contract
        assert wl.digest(out[key]) == str(fx["sha_" + key]), key
    rows = fx["rows"]
    assert same_bits(out["y"][rows], fx["y_rows"])


@pytest.mark.parametrize("name", LARGE)
def test_oracle_matches_reference_large(name):
    """Full-size configs: routing digests and counts bit-exact; sampled
    output rows bit-exact (computed per token, which equals the full run)."""
    case = C.ALL_CASES[name]
    fx = fixture(name)
    inp = C.build_inputs(case)
    logits = O.router_logits(inp.x, inp.Wr, inp.br)
    probs = O.softmax(logits)
    idx, topp = O.topk(probs, case.cfg.k)
    counts, offsets, perm = O.dispatch(idx, case.cfg.E)
    assert np.array_equal(counts, fx["counts"])
    assert np.array_equal(offsets, fx["offsets"])
    for key, arr in (("logits", logits), ("probs", probs), ("idx", idx), ("topp", topp),
                     ("perm", perm)):
        assert wl.digest(arr) == str(fx["sha_" + key]), key
    rows = fx["rows"]
    y = O.tokens(inp, idx, topp, rows)
    assert same_bits(y, fx["y_rows"])


# ----------------------------------------------------------- known answers
def test_matmul_known_answer():
    # tests/utilsTest/tensorTests.cpp:228-242: [2x3] . [3x2] = [[31,19],[85,55]]
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    W = np.array([[7, 8], [9, 1], [2, 3]], np.float32)
    out = O.router_logits(x, W, np.zeros(2, np.float32))
    assert np.array_equal(out, np.array([[31, 19], [85, 55]], np.float32))
    out = O.router_logits(x, W, np.array([0.5, -1], np.float32))
    assert np.array_equal(out, np.array([[31.5, 18], [85.5, 54]], np.float32))


def test_router_one_hot_weights_select_features():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((40, 16)).astype(np.float32)
    W = np.zeros((16, 5), np.float32)
    W[[3, 0, 7, 15, 9], range(5)] = 1.0
    b = rng.standard_normal(5).astype(np.float32)
    out = O.router_logits(x, W, b)
    assert np.array_equal(out, x[:, [3, 0, 7, 15, 9]] + b)


def test_router_sequential_sum_order():
    # (1e8 + 1) - 1e8 in sequential fp32 order is 0 (the 1 is absorbed);
    # a pairwise or reordered sum would give 1.
    x = np.array([[1e8, 1.0, -1e8]], np.float32)
    W = np.ones((3, 1), np.float32)
    assert O.router_logits(x, W, np.zeros(1, np.float32))[0, 0] == 0.0


def test_softmax_known_values():
    p = O.softmax(np.array([[1.0, 2.0, 3.0]], np.float32))[0]
    assert np.allclose(p, [0.0900306, 0.2447285, 0.6652410], atol=1e-7)
    assert abs(p.sum() - 1.0) < 1e-6 and p[2] > p[1] > p[0]
    # uniform logits -> exactly fl(1/E)
    for E in (1, 3, 8, 64):
        p = O.softmax(np.full((1, E), 0.37, np.float32))[0]
        assert np.all(p == np.float32(1.0) / np.float32(E))
    # clamps: a gap of 20 gives exp(-20) ~ 2e-9 -> 1e-7; the winner -> 1
    p = O.softmax(np.array([[0.0, -20.0, -30.0]], np.float32))[0]
    assert p[0] == np.float32(1.0) and p[1] == np.float32(1e-7) and p[2] == np.float32(1e-7)
    # a NaN logit anywhere makes the sum NaN -> inv = 1/1e-15; NaN at 0 -> every p = 1e-7
    p = O.softmax(np.array([[np.nan, 1.0, 2.0]], np.float32))[0]
    assert np.all(p == np.float32(1e-7))


def brute_topk(p, k):
    order = np.lexsort((np.broadcast_to(np.arange(p.shape[1]), p.shape), -p), axis=1)
    idx = order[:, :k].astype(np.int32)
    return idx, np.take_along_axis(p, idx, 1)


@pytest.mark.parametrize("E,k", [(4, 2), (8, 3), (16, 8), (64, 6), (5, 5), (1, 1)])
def test_topk_is_stable_sort(E, k):
    rng = np.random.default_rng(E * 10 + k)
    # coarse values force many exact ties
    p = (rng.integers(0, 6, size=(500, E)) / 8.0 + 1e-7).astype(np.float32)
    idx, val = O.topk(p, k)
    bi, bv = brute_topk(p, k)
    assert np.array_equal(idx, bi) and np.array_equal(val, bv)


@pytest.mark.parametrize("E,k,N", [(4, 2, 100), (64, 6, 333), (8, 8, 17), (1, 1, 5)])
def test_dispatch_is_stable_counting_sort(E, k, N):
    rng = np.random.default_rng(N)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    counts, offsets, perm = O.dispatch(idx, E)
    flat = idx.reshape(-1)
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]))
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))


# ------------------------------------------------------------- invariants
def _ffn64(x, Wg, bg, Wu, bu, Wd, bd):
    x = x.astype(np.float64)
    g = x @ Wg.astype(np.float64) + bg
    u = x @ Wu.astype(np.float64) + bu
    h = g / (1.0 + np.exp(-g)) * u
    return h @ Wd.astype(np.float64) + bd


def test_experts_match_fp64_swiglu():
    case = C.ALL_CASES["small_f32"]
    inp = C.build_inputs(case)
    out = O.forward(inp)
    y64 = np.zeros((case.cfg.N, case.cfg.C))
    for t in range(case.cfg.N):
        for j in range(case.cfg.k):
            e = out["idx"][t, j]
            y64[t] += out["topp"][t, j] * _ffn64(inp.x[t], inp.Wg[e], inp.bg[e], inp.Wu[e],
                                                 inp.bu[e], inp.Wd[e], inp.bd[e])
    err = np.linalg.norm(out["y"] - y64) / np.linalg.norm(y64)
    assert err < 1e-6


def test_single_expert_is_dense_swiglu():
    case = C.ALL_CASES["single_expert"]
    inp = C.build_inputs(case)
    out = O.forward(inp)
    assert np.all(out["topp"] == 1.0) and np.all(out["idx"] == 0)
    # y = 0 + FFN(x)*1 exactly equals the expert's own output row
    e_only = O.tokens(inp, out["idx"], np.ones_like(out["topp"]), np.arange(case.cfg.N))
    assert same_bits(out["y"], e_only)


def test_identical_experts_scale_by_gate_sum():
    """All experts equal and biases shared: y = (sum_j p_j) * FFN(x)."""
    cfg = wl.MoEConfig("ident", 40, 64, 6, 3, 64, "f32", "f32", "normal")
    inp = wl.make_inputs(cfg, 7, bias_std=0.05)
    for arr in (inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd, inp.bd):
        arr[:] = arr[0]
    out = O.forward(inp)
    single = wl.MoEConfig("ident1", 40, 64, 1, 1, 64, "f32", "f32", "zero")
    inp1 = wl.MoEInputs(single, inp.x, np.zeros((64, 1), np.float32), np.zeros(1, np.float32),
                        inp.Wg[:1], inp.bg[:1], inp.Wu[:1], inp.bu[:1], inp.Wd[:1], inp.bd[:1])
    ffn = O.forward(inp1)["y"]
    expect = out["topp"].sum(axis=1, dtype=np.float64)[:, None] * ffn.astype(np.float64)
    assert np.allclose(out["y"], expect, rtol=1e-5, atol=1e-6)


def test_nan_input_routes_to_first_experts():
    """F16: a NaN (or +-inf) input makes every logit non-finite or the sum
    NaN, so every probability clamps to 1e-7 and the tie rule picks experts
    0..k-1 (utils/Tensor.cpp:879, :1321)."""
    case = C.ALL_CASES["nan_rows"]
    inp = C.build_inputs(case)
    out = O.forward(inp, with_y=False)
    for t in (3, 5, 9, 11):
        assert np.all(out["probs"][t] == np.float32(1e-7)), t
        assert list(out["idx"][t]) == list(range(case.cfg.k)), t
    finite = [t for t in range(case.cfg.N) if t not in (3, 5, 9, 11)]
    assert np.all(np.isfinite(out["probs"][finite]))


# --------------------------------------------------------- planted mistakes
def test_dropped_router_bias_is_detected():
    case = C.ALL_CASES["ragged_k3"]
    fx = fixture(case.name)
    inp = C.build_inputs(case)
    probs = O.softmax(O.router_logits(inp.x, inp.Wr, np.zeros_like(inp.br)))
    idx, _ = O.topk(probs, case.cfg.k)
    assert not np.array_equal(idx, fx["idx"])


def test_reversed_tie_rule_is_detected():
    for name in ("ties_ones", "clamp_ties"):
        fx = fixture(name)
        probs = fx["probs"]
        k = fx["idx"].shape[1]
        # ">=" insertion = higher expert id wins ties
        order = np.lexsort((-np.broadcast_to(np.arange(probs.shape[1]), probs.shape), -probs),
                           axis=1)
        assert not np.array_equal(order[:, :k], fx["idx"]), name


def test_renormalised_gate_is_detected():
    case = C.ALL_CASES["small_f32"]
    fx = fixture(case.name)
    inp = C.build_inputs(case)
    out = O.forward(inp)
    renorm = out["topp"] / out["topp"].sum(axis=1, keepdims=True)
    y = O.tokens(inp, out["idx"], renorm, fx["rows"])
    assert not np.allclose(y, fx["y_rows"], rtol=1e-3)
