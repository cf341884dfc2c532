"""GPU parity of the fused block's backward (mgpt_moe_forward_block_train +
mgpt_moe_backward_block through the C ABI): the MoE half of the reference's
TransformerBlock::backward_into (layers/TransformerBlock.cpp:81-85) -- the
MoE backward, ln2's RMSNorm backward (utils/Tensor.cpp:1665-1689) and the
residual add.

Expected values are the CPU oracle's block backward
(oracle_moe_block_backward), which reproduces the reference's own CPU path
bit for bit on every fixture in tests/golden/block_backward/
(tests/test_oracle_block.py).  dx, dgamma and each of the 2 + 6E MoE
gradients must satisfy, per tensor,
    ||g - g_ref||_2 / ||g_ref||_2 <= tol  and  max|g - g_ref| <= tol * max|g_ref|
with tol = 1e-5 for fp32 handles and 2e-2 for bf16 (the backward's bars).
A second call adds its contribution again (dgamma and the router gradients
exactly, the expert gradients to within one rounding), zero_grad + the same
call repeats bit for bit, and a plain backward after a block forward is
refused.
"""
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = {"f32": 1e-5, "bf16": 2e-2}
BBK = os.path.join(os.path.dirname(__file__), "golden", "block_backward")
GRADS = ("dWr", "dbr", "dWg", "dbg", "dWu", "dbu", "dWd", "dbd")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()   # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)


def _dt(act):
    return torch.float32 if act == "f32" else torch.bfloat16


def make_layer(inp):
    from mgpt_amd.moe import MoELayer
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    return layer


def grads_of(layer, E):
    g = [t.cpu().numpy() for t in layer.get_gradients()]
    out = {"dWr": g[0], "dbr": g[1].reshape(-1)}
    for i, n in enumerate(GRADS[2:]):
        arr = np.stack([g[2 + 6 * e + i] for e in range(E)])
        out[n] = arr.reshape(E, -1) if n.startswith("db") else arr
    return out


def run_block_backward(layer, inp, x1, gamma, dout, zeros=(True,)):
    """One training forward + block backward per entry of `zeros` (True:
    zero_grad and a fresh dgamma first, False: add into the previous ones)."""
    cfg = inp.cfg
    dt = _dt(cfg.act)
    x = torch.from_numpy(np.ascontiguousarray(x1)).to("cuda").to(dt)
    g = torch.from_numpy(np.ascontiguousarray(gamma)).to("cuda")
    d = torch.from_numpy(np.ascontiguousarray(dout)).to("cuda").to(dt)
    outs = []
    for zero in zeros:
        if zero:
            layer.zero_grad()
            dgamma = torch.zeros(cfg.C, dtype=torch.float32, device="cuda")
        layer.forward_block_into(x, g, C.BLOCK_EPS, torch.empty_like(x), train=True)
        dx, _ = layer.backward_block(d, dgamma)
        torch.cuda.synchronize()
        out = {"dx": dx.float().cpu().numpy(), "dgamma": dgamma.cpu().numpy().copy()}
        out.update(grads_of(layer, cfg.E))
        outs.append(out)
    return outs


def rel_errors(got, ref):
    d = (np.asarray(got, np.float64) - np.asarray(ref, np.float64)).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    rel = np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)
    mx = np.max(np.abs(d)) / max(np.max(np.abs(r)), 1e-30) if d.size else 0.0
    return rel, mx


def check_all(out, ref, tol, name):
    for n in ("dx", "dgamma") + GRADS:
        rel, mx = rel_errors(out[n], ref[n])
        print(f"{name} {n}: normwise {rel:.3e}  max/max {mx:.3e}  (tol {tol})", flush=True)
        assert rel <= tol, f"{name} {n}: normwise error {rel} > {tol}"
        assert mx <= tol, f"{name} {n}: elementwise error {mx} > {tol}"


GPU_CASES = [n for n in C.BLOCK_BACKWARD_CASES if C.ALL_CASES[n].gpu]


@pytest.mark.parametrize("name", GPU_CASES)
def test_block_backward_parity(name):
    case = C.ALL_CASES[name]
    print(f"case {name}: {case.cfg}", flush=True)
    inp, x1, gamma = C.build_block_inputs(case)
    dout = C.build_dy(case)
    out = run_block_backward(make_layer(inp), inp, x1, gamma, dout)[0]
    ref = O.block_backward(inp, x1, gamma, dout, C.BLOCK_EPS)
    check_all(out, ref, TOL[case.cfg.act], name)
    # and the reference's own values where the fixture holds them
    fx = np.load(os.path.join(BBK, name + ".npz"), allow_pickle=False)
    rel, mx = rel_errors(out["dgamma"], fx["dgamma"])
    assert rel <= TOL[case.cfg.act] and mx <= TOL[case.cfg.act], ("fixture dgamma", rel, mx)
    rel, mx = rel_errors(out["dx"][fx["rows"]], fx["dx_rows"])
    assert rel <= TOL[case.cfg.act] and mx <= TOL[case.cfg.act], ("fixture dx rows", rel, mx)


# (N, C, E, k, H, act): padded widths (the RMSNorm backward runs at the
# caller's width), one not a multiple of the 16-byte piece (the scalar
# path: 10 fp32, 100 bf16), a large-M bf16 shape on the 256 x 256 GEMMs
# with the weight gradients on the second stream, and 128 experts (the wide
# router, token and weight gradients).
SHAPES = [
    (40, 10, 3, 2, 24, "f32"),
    (90, 96, 5, 2, 72, "f32"),
    (77, 100, 6, 2, 64, "bf16"),
    (64, 200, 8, 2, 136, "bf16"),
    (2048, 256, 8, 2, 384, "bf16"),
    (150, 128, 128, 4, 64, "bf16"),
]


def shaped_case(N, Cm, E, k, H, act):
    cfg = wl.MoEConfig(f"bb{Cm}", N, Cm, E, k, H, act, act, "normal")
    inp = wl.make_inputs(cfg, C.SEED + 53 * Cm + E, bias_std=0.05)
    rng = np.random.default_rng(Cm + N)
    x1 = (inp.x * rng.uniform(0.25, 4.0, (N, 1)) + np.float32(0.05)).astype(np.float32)
    gamma = (np.float32(1.0) + wl.normal_f32(C.SEED, 4013, Cm, std=0.2)).astype(np.float32)
    dout = rng.standard_normal((N, Cm)).astype(np.float32)
    if act == "bf16":
        x1, dout = wl.bf16_round(x1), wl.bf16_round(dout)
        inp.Wr[:] = wl.bf16_round(inp.Wr)
    return inp, x1, gamma, dout


@pytest.mark.parametrize("N,Cm,E,k,H,act", SHAPES)
def test_block_backward_shapes(N, Cm, E, k, H, act):
    inp, x1, gamma, dout = shaped_case(N, Cm, E, k, H, act)
    print(f"case {inp.cfg}", flush=True)
    out = run_block_backward(make_layer(inp), inp, x1, gamma, dout)[0]
    ref = O.block_backward(inp, x1, gamma, dout, C.BLOCK_EPS)
    check_all(out, ref, TOL[act], f"N={N} C={Cm} {act}")


def test_block_backward_accumulates_and_repeats():
    """A second forward/backward without zero_grad adds the same values
    again: dgamma and the router gradients double bit for bit, the expert
    gradients to within one rounding of the sum per element (their row
    chunks add into the gradient one after the other); zero_grad + the same
    call repeats the first result bit for bit; dx repeats."""
    inp, x1, gamma, dout = shaped_case(2048, 256, 8, 2, 384, "bf16")
    a, b, c = run_block_backward(make_layer(inp), inp, x1, gamma, dout,
                                 zeros=(True, False, True))
    assert np.array_equal(a["dx"], b["dx"]) and np.array_equal(a["dx"], c["dx"])
    for n in ("dgamma",) + GRADS:
        assert np.array_equal(c[n], a[n]), n
        if n in ("dgamma", "dWr", "dbr"):
            assert np.array_equal(b[n], a[n] * np.float32(2.0)), n
        two = 2.0 * a[n].astype(np.float64)
        err = np.max(np.abs(b[n] - two)) / max(np.max(np.abs(two)), 1e-30)
        assert err <= 1e-6, (n, err)


def test_plain_backward_after_block_forward_is_refused():
    inp, x1, gamma, dout = shaped_case(40, 10, 3, 2, 24, "f32")
    layer = make_layer(inp)
    x = torch.from_numpy(x1).cuda()
    layer.forward_block_into(x, torch.from_numpy(gamma).cuda(), C.BLOCK_EPS,
                             torch.empty_like(x), train=True)
    with pytest.raises(RuntimeError, match="backward_block"):
        layer.backward(torch.from_numpy(dout).cuda())
