"""Pins the training-sequence fixtures (tests/golden/train/) on the CPU.

The fixtures hold what the compiled reference computes for the Trainer's
step (pipeline/Trainer.cpp:303-386: zero grads, MoELayer::forward_into,
backward_into, AdamWOptimizer::step) repeated cases.TRAIN_STEPS times, then
a last forward.  Here the same sequence is rebuilt from independent parts
and must give the fixture's bits:
  * forward and backward: the oracle (bit-exact with the reference's layer,
    tests/test_oracle.py, tests/test_oracle_backward.py);
  * the optimizer: AdamW restated in float32 numpy from
    Tensor::adamw_step's CPU branch (utils/Tensor.cpp:683-701) with the
    optimizer's defaults (optimisers/AdamWOptimiser.h:20-22).
A forward that ignored the step (stale weights) or an optimizer that dropped
the weight decay or the bias correction fails the comparison; both are
planted below.
"""
import dataclasses
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

TRAIN_DIR = os.path.join(os.path.dirname(__file__), "golden", "train")
F = np.float32


def adamw(params, grads, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.01, plant=""):
    """One AdamWOptimizer::step over float32 arrays, in the reference's
    operation order (every operation rounded to float32)."""
    lr, b1, b2, eps, wd = F(lr), F(b1), F(b2), F(eps), F(wd)
    # 1 / (1 - powf(beta, t)): powf of these arguments is the correctly
    # rounded power, which float64 gives exactly here
    ms = F(1) / (F(1) - F(np.float64(b1) ** t))
    vs = F(1) / (F(1) - F(np.float64(b2) ** t))
    if plant == "no_bias_correction":
        ms = vs = F(1)
    out = []
    for p, g, mi, vi in zip(params, grads, m, v):
        mi[:] = b1 * mi + (F(1) - b1) * g
        vi[:] = b2 * vi + ((F(1) - b2) * g) * g
        m_hat = mi * ms
        v_hat = vi * vs
        q = p.copy()
        if plant != "no_weight_decay":
            q = q - (lr * wd) * q
        q = q - (lr * m_hat) / (np.sqrt(v_hat) + eps)
        out.append(q.astype(np.float32))
    return out


def flat_params(inp):
    return [np.ascontiguousarray(p, np.float32).reshape(-1).copy() for p in inp.params()]


def with_params(inp, flat):
    cfg = inp.cfg
    Cc, H, E = cfg.C, cfg.H, cfg.E
    Wg = np.stack([flat[2 + 6 * e].reshape(Cc, H) for e in range(E)])
    bg = np.stack([flat[3 + 6 * e] for e in range(E)])
    Wu = np.stack([flat[4 + 6 * e].reshape(Cc, H) for e in range(E)])
    bu = np.stack([flat[5 + 6 * e] for e in range(E)])
    Wd = np.stack([flat[6 + 6 * e].reshape(H, Cc) for e in range(E)])
    bd = np.stack([flat[7 + 6 * e] for e in range(E)])
    return dataclasses.replace(inp, Wr=flat[0].reshape(Cc, E), br=flat[1].copy(), Wg=Wg, bg=bg,
                               Wu=Wu, bu=bu, Wd=Wd, bd=bd, raw=None)


def grads_flat(g, E):
    out = [g["dWr"].reshape(-1), g["dbr"].reshape(-1)]
    for e in range(E):
        for n in ("dWg", "dbg", "dWu", "dbu", "dWd", "dbd"):
            out.append(g[n][e].reshape(-1))
    return [np.ascontiguousarray(a, np.float32) for a in out]


def replay(case, plant=""):
    """(y of every forward, params after every step) by oracle + AdamW."""
    inp = C.build_inputs(case)
    dy = C.build_dy(case)
    params = flat_params(inp)
    m = [np.zeros_like(p) for p in params]
    v = [np.zeros_like(p) for p in params]
    ys, after = [], []
    cur = inp
    for s in range(C.TRAIN_STEPS + 1):
        if plant == "stale" and s > 0:
            ys.append(O.forward(inp)["y"])
        else:
            ys.append(O.forward(cur)["y"])
        if s == C.TRAIN_STEPS:
            break
        g = grads_flat(O.backward(cur, dy), case.cfg.E)
        params = adamw(params, g, m, v, s + 1, C.TRAIN_LR, plant=plant)
        after.append(params)
        cur = with_params(inp, params)
    return ys, after


def fixture(name):
    path = os.path.join(TRAIN_DIR, name + ".npz")
    if not os.path.exists(path):
        pytest.skip(f"no fixture {name}")
    return np.load(path, allow_pickle=False)


def matches(fx, ys, after):
    if not all(np.array_equal(a.view(np.uint32), b.view(np.uint32))
               for a, b in zip(ys, fx["y"])):
        return False
    for s, step in enumerate(after):
        for i, p in enumerate(step):
            if wl.digest(p) != str(fx[f"p{s}_{i}_sha"]):
                return False
            if not np.array_equal(p[C.sample_flat(p.size, 64)].view(np.uint32),
                                  fx[f"p{s}_{i}_val"].view(np.uint32)):
                return False
    return True


@pytest.mark.parametrize("name", C.TRAIN_CASES)
def test_training_fixture_is_oracle_plus_adamw(name):
    fx = fixture(name)
    assert int(fx["steps"]) == C.TRAIN_STEPS and float(fx["lr"]) == np.float32(C.TRAIN_LR)
    ys, after = replay(C.ALL_CASES[name])
    assert matches(fx, ys, after)
    # the steps move the weights far more than the forward's 1e-5 bar
    y0, yS = fx["y"][0].astype(np.float64), fx["y"][-1].astype(np.float64)
    assert np.linalg.norm(yS - y0) > 1e-3 * np.linalg.norm(y0)


@pytest.mark.parametrize("plant", ["stale", "no_weight_decay", "no_bias_correction"])
def test_planted_training_mistakes_fail(plant):
    name = "small_f32"
    ys, after = replay(C.ALL_CASES[name], plant=plant)
    assert not matches(fixture(name), ys, after)
