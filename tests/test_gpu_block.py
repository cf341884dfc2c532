"""GPU parity of the fused block mgpt_moe_forward_block:
out = x1 + MoE(RMSNorm(x1) * gamma), the MoE half of the engine's
TransformerBlock::forward_into (layers/TransformerBlock.cpp:42-46).

Against the committed fixtures of the reference's own ln2 RMSNormLayer ->
MoELayer -> Tensor::add_into (tests/golden/block/, pinned to the oracle in
tests/test_oracle_block.py):
  * the per-token 1/rms, the routing (ids, probabilities, permutation) and
    the counts bit for bit -- the router normalises while it reads x with
    the reference's operation order;
  * out normwise and elementwise against the reference at the forward's bars
    (1e-5 fp32, 2e-2 bf16, 6e-2 fp8), on sampled rows for cfg3 and in full
    (oracle) elsewhere; for fp32 the MoE part out - x1 is checked at 1e-5 of
    its own size too, plus the ulp of the final rounding of x1 + MoE.
The unfused composition (normalise on the host, mgpt_moe_forward, add) must
route identically.
"""
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

BLK = os.path.join(os.path.dirname(__file__), "golden", "block")
TOL = {"f32": 1e-5, "bf16": 2e-2, "fp8": 6e-2}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()
    return torch.device("cuda", 0)


def errors(got, ref):
    d = np.asarray(got, np.float64) - np.asarray(ref, np.float64)
    r = np.asarray(ref, np.float64)
    return (np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30),
            np.abs(d).max() / max(np.abs(r).max(), 1e-30))


def run_block(inp, x1, gamma):
    from mgpt_amd.moe import MoELayer
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    dt = torch.float32 if cfg.act == "f32" else torch.bfloat16
    x = torch.from_numpy(np.ascontiguousarray(x1)).to("cuda").to(dt)
    g = torch.from_numpy(gamma).to("cuda")
    out = layer.forward_block(x, g, C.BLOCK_EPS)
    torch.cuda.synchronize()
    r = {k: v.cpu().numpy() for k, v in layer.routing().items()}
    return layer, out.float().cpu().numpy(), layer.rstd().cpu().numpy(), r


@pytest.mark.parametrize("name", C.BLOCK_CASES)
def test_block_parity(name):
    case = C.ALL_CASES[name]
    print(f"case {name}: {case.cfg}", flush=True)
    fx = np.load(os.path.join(BLK, name + ".npz"), allow_pickle=False)
    inp, x1, gamma = C.build_block_inputs(case)
    layer, out, rstd, r = run_block(inp, x1, gamma)
    bad = np.nonzero(rstd.view(np.uint32) != fx["rstd"].view(np.uint32))[0]
    if bad.size:
        ulps = rstd.view(np.int32)[bad].astype(np.int64) - fx["rstd"].view(np.int32)[bad]
        print(f"rstd: {bad.size} of {rstd.size} differ, first {bad[:8]}, ulps {ulps[:8]}")
    assert bad.size == 0, "rstd"
    assert np.array_equal(r["counts"], fx["counts"]), "counts"
    for n, a in (("idx", r["topk_idx"]), ("topp", r["topk_p"]), ("perm", r["perm"])):
        assert wl.digest(a) == str(fx["sha_" + n]), n
    tol = TOL[case.cfg.weights]
    if name == "cfg3":
        rows = fx["rows"]
        rel, mx = errors(out[rows], fx["out_rows"])
    else:
        ref = O.block(inp, x1, gamma, C.BLOCK_EPS)
        rel, mx = errors(out, ref["out"])
        if case.cfg.act == "f32":
            # the MoE part m = out - x1 at the forward's bar on m's own
            # size, plus the one rounding of x1 + m both sides make
            m = (ref["out"].astype(np.float64) - x1)
            d = np.abs(out.astype(np.float64) - ref["out"])
            ulp = np.spacing(np.abs(ref["out"]))
            mrel = np.linalg.norm(d) / (tol * np.linalg.norm(m) + np.linalg.norm(ulp))
            mmx = np.max(d / (tol * np.abs(m).max() + ulp))
            print(f"{name} MoE part: normwise {mrel:.3f} elementwise {mmx:.3f} of the allowance")
            assert mrel <= 1.0 and mmx <= 1.0
    print(f"{name} out: normwise {rel:.3e} max/max {mx:.3e} (tol {tol})")
    assert rel <= tol and mx <= tol


@pytest.mark.parametrize("name", ["small_f32", "k8_bf16"])
def test_block_routes_like_the_unfused_composition(name):
    case = C.ALL_CASES[name]
    inp, x1, gamma = C.build_block_inputs(case)
    layer, out, _, r = run_block(inp, x1, gamma)
    xn, _ = O.rmsnorm_scaled(x1, gamma, C.BLOCK_EPS)
    dt = torch.float32 if case.cfg.act == "f32" else torch.bfloat16
    xt = torch.from_numpy(xn).to("cuda").to(dt)
    y = layer.forward(xt)
    torch.cuda.synchronize()
    r2 = {k: v.cpu().numpy() for k, v in layer.routing().items()}
    if case.cfg.act == "f32":   # bf16 would round xn before routing
        assert np.array_equal(r["topk_idx"], r2["topk_idx"])
        assert np.array_equal(r["perm"], r2["perm"])
        rel, mx = errors(out, x1 + y.float().cpu().numpy())
        assert rel <= 1e-6


def test_block_edge_cases_and_errors():
    """Empty input is a no-op; a null gamma, a negative eps and an output
    that overlaps x are rejected with a status (nothing runs)."""
    import ctypes
    from mgpt_amd import capi
    case = C.ALL_CASES["small_f32"]
    inp, x1, gamma = C.build_block_inputs(case)
    from mgpt_amd.moe import MoELayer
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act="f32")
    layer.load_parameters(inp.params(raw=True))
    x = torch.from_numpy(x1).to("cuda")
    g = torch.from_numpy(gamma).to("cuda")
    empty = layer.forward_block(x[:0], g, C.BLOCK_EPS)
    assert empty.shape == (0, cfg.C)
    layer.reserve(cfg.N)
    ws = layer._ws
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    L = capi.lib()

    def call(gp, eps, o):
        return L.mgpt_moe_forward_block(layer._h, x.data_ptr(), gp, ctypes.c_float(eps), o,
                                        cfg.N, ws.data_ptr(), ws.numel(), stream)

    assert call(None, 1e-5, out.data_ptr()) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert call(g.data_ptr(), -1.0, out.data_ptr()) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert call(g.data_ptr(), 1e-5, x.data_ptr()) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert call(g.data_ptr(), 1e-5, out.data_ptr()) == capi.MGPT_OK
    torch.cuda.synchronize()
    ref = O.block(inp, x1, gamma, C.BLOCK_EPS)
    rel, mx = errors(out.cpu().numpy(), ref["out"])
    assert rel <= 1e-5 and mx <= 1e-5
