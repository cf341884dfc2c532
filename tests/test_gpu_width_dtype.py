"""GPU parity of embed widths that are not a multiple of 64 and of fp32
tensors over bf16 / fp8 expert products.

The reference layer runs any embed_dim (layers/MoELayer.cpp:4-12); its own
test uses C = 16 (tests/networkTest/moeTests.cpp:6-39).  The library runs
such widths through zero-padded rows of width round_up(C, 64): the padded
columns of x, gamma, the router and expert weights are zero, so every sum
gains +0 terms only and routing stays bit-exact.  The engine's tensors are
fp32; with bf16 or fp8 weights the library routes on the fp32 rows
(bit-exact with the reference on the same fp32 inputs), gathers them as bf16
and returns fp32 outputs of bf16 expert products.

Expected values come from the CPU oracle on the same inputs (pinned to the
reference bit for bit by tests/test_oracle.py): routing bit for bit, outputs
and gradients normwise and elementwise within 1e-5 (fp32), 2e-2 (bf16
products), 6e-2 (fp8 weights).
"""
import dataclasses

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = {"f32": 1e-5, "bf16": 2e-2, "fp8": 6e-2}
GRADS = ("dWr", "dbr", "dWg", "dbg", "dWu", "dbu", "dWd", "dbd")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()   # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)


def _torch_dt(act):
    return torch.float32 if act == "f32" else torch.bfloat16


def make_case(name, N, Cm, E, k, H, act, weights, rb="normal", seed_off=0, bias_std=0.05):
    cfg = wl.MoEConfig(name, N, Cm, E, k, H, act, weights, rb)
    inp = wl.make_inputs(cfg, C.SEED + 31 * Cm + E + seed_off, bias_std=bias_std)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
        inp.Wr[:] = wl.bf16_round(inp.Wr)
    return inp


def layer_for(inp):
    from mgpt_amd.moe import MoELayer
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    return layer


def check_close(y, ref, tol, what):
    fin = np.isfinite(ref).all(axis=1)
    d = (y[fin] - ref[fin]).astype(np.float64)
    r = ref[fin].astype(np.float64)
    rel = np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)
    mx = np.max(np.abs(d)) / max(np.max(np.abs(r)), 1e-30) if d.size else 0.0
    print(f"{what}: normwise {rel:.3e}  max/max {mx:.3e}  (tol {tol})", flush=True)
    assert rel <= tol, f"{what}: normwise error {rel} > {tol}"
    assert mx <= tol, f"{what}: elementwise error {mx} > {tol}"


def check_routing(r, ref):
    assert np.array_equal(r["counts"], ref["counts"]), "counts"
    assert np.array_equal(r["topk_idx"], ref["idx"]), "topk_idx"
    assert np.array_equal(r["topk_p"].view(np.uint32), ref["topp"].view(np.uint32)), "topk_p"
    assert np.array_equal(r["perm"], ref["perm"]), "perm"


def forward(layer, inp):
    x = torch.from_numpy(np.ascontiguousarray(inp.x)).to("cuda").to(_torch_dt(inp.cfg.act))
    y = layer.forward(x)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), {k: v.cpu().numpy() for k, v in layer.routing().items()}


# (N, C, E, k, H, act, weights): widths below, between and above multiples of
# 64, one that is not a multiple of 4 (rows not 16-byte aligned), the fp32
# and bf16 paths, the large-M bf16 GEMM and the small-M decode path.
WIDTHS = [
    (8, 16, 4, 2, 64, "f32", "f32"),
    (40, 10, 3, 2, 24, "f32", "f32"),
    (70, 96, 6, 3, 80, "f32", "f32"),
    (50, 200, 16, 4, 96, "f32", "f32"),
    (64, 72, 8, 2, 136, "bf16", "bf16"),
    (1300, 200, 4, 2, 320, "bf16", "bf16"),
    (60, 328, 64, 8, 192, "bf16", "bf16"),
    (48, 200, 8, 4, 192, "bf16", "fp8"),
]


@pytest.mark.parametrize("N,Cm,E,k,H,act,weights", WIDTHS)
def test_width_not_multiple_of_64(N, Cm, E, k, H, act, weights):
    inp = make_case(f"w{Cm}", N, Cm, E, k, H, act, weights)
    print(f"case {inp.cfg}", flush=True)
    y, r = forward(layer_for(inp), inp)
    ref = O.forward(inp)
    check_routing(r, ref)
    check_close(y, ref["y"], TOL[weights], f"C={Cm} {act}/{weights}")


@pytest.mark.parametrize("Cm,act", [(16, "f32"), (96, "f32"), (200, "bf16")])
def test_width_backward(Cm, act):
    """Training at a padded width: dx and every gradient in the caller's
    layouts (the padded columns are dropped) against the oracle's backward."""
    inp = make_case(f"wb{Cm}", 90, Cm, 5, 2, 72, act, act)
    dy = np.random.default_rng(Cm).standard_normal((90, Cm)).astype(np.float32)
    if act == "bf16":
        dy = wl.bf16_round(dy)
    layer = layer_for(inp)
    dt = _torch_dt(act)
    x = torch.from_numpy(inp.x).to("cuda").to(dt)
    layer.zero_grad()
    layer.forward(x, train=True)
    dx = layer.backward(torch.from_numpy(dy).to("cuda").to(dt))
    torch.cuda.synchronize()
    g = [t.cpu().numpy() for t in layer.get_gradients()]
    E = inp.cfg.E
    out = {"dx": dx.float().cpu().numpy(), "dWr": g[0], "dbr": g[1].reshape(-1)}
    for i, n in enumerate(GRADS[2:]):
        arr = np.stack([g[2 + 6 * e + i] for e in range(E)])
        out[n] = arr.reshape(E, -1) if n.startswith("db") else arr
    ref = O.backward(inp, dy)
    for n in ("dx",) + GRADS:
        check_close(np.asarray(out[n], np.float32).reshape(-1, 1).T,
                    np.asarray(ref[n], np.float32).reshape(-1, 1).T, TOL[act], f"C={Cm} {n}")


@pytest.mark.parametrize("Cm,act,weights", [(96, "f32", "f32"), (200, "bf16", "bf16"),
                                            (200, "f32", "bf16")])
def test_width_fused_block(Cm, act, weights):
    """out = x + MoE(RMSNorm(x) * gamma) at a padded width: the mean's divisor
    is the caller's width, so 1/rms is bit-exact with the reference's."""
    inp = make_case(f"wblk{Cm}", 77, Cm, 6, 2, 64, act, weights)
    N = inp.cfg.N
    t = np.arange(N)
    x1 = (inp.x * (np.float32(1.0) + (t % 4).astype(np.float32))[:, None]).astype(np.float32)
    gamma = (np.float32(1.0) + wl.normal_f32(C.SEED, 4013, Cm, std=0.2)).astype(np.float32)
    if act == "bf16":
        x1 = wl.bf16_round(x1)
    layer = layer_for(inp)
    xd = torch.from_numpy(x1).to("cuda").to(_torch_dt(act))
    out = layer.forward_block(xd, torch.from_numpy(gamma).cuda(), C.BLOCK_EPS)
    torch.cuda.synchronize()
    r = {k: v.cpu().numpy() for k, v in layer.routing().items()}
    ref = O.block(inp, x1, gamma, C.BLOCK_EPS)
    assert np.array_equal(layer.rstd().cpu().numpy().view(np.uint32), ref["rstd"].view(np.uint32))
    check_routing(r, ref)
    check_close(out.float().cpu().numpy(), ref["out"], TOL[weights], f"block C={Cm}")


# fp32 tensors over bf16 / fp8 expert weights (the engine's Tensors are fp32):
# the benchmark shapes cfg2 (bf16) and cfg5 (fp8 decode), a large-M bf16
# shape with skewed load, and fp8 decode widths with C % 128 == 64 (the
# register-staged fp8 path instead of the tiled weight stream).
MIXED = [
    ("cfg2", None),
    ("cfg5", None),
    ("large_m", (3000, 320, 6, 2, 448, "f32", "bf16", "zipf")),
    ("fp8_c192", (40, 192, 16, 4, 256, "f32", "fp8", "normal")),
    ("fp8_c1088", (24, 1088, 32, 8, 384, "f32", "fp8", "normal")),
]


@pytest.mark.parametrize("name,shape", MIXED)
def test_f32_tensors_low_precision_weights(name, shape):
    """Routing on the fp32 rows is bit-exact with the reference on those
    rows; outputs within the weight dtype's bar of the fp32 reference."""
    if shape is None:
        base = wl.CONFIGS[name]
        cfg = wl.MoEConfig(f"{name}_f32io", base.N, base.C, base.E, base.k, base.H, "f32",
                           base.weights, base.router_bias)
        inp = wl.make_inputs(cfg, C.SEED)
    else:
        N, Cm, E, k, H, act, weights, rb = shape
        inp = make_case(name, N, Cm, E, k, H, act, weights, rb)
    cfg = inp.cfg
    print(f"case {cfg}", flush=True)
    y, r = forward(layer_for(inp), inp)
    ref = O.forward(inp, with_y=cfg.N <= 4096)
    check_routing(r, ref)
    rows = C.sample_rows(cfg.N, 256) if cfg.N > 4096 else np.arange(cfg.N)
    yref = ref["y"] if ref["y"] is not None else O.tokens(inp, ref["idx"], ref["topp"], rows)
    check_close(y[rows], yref if ref["y"] is None else yref[rows], TOL[cfg.weights], name)


# fp8 decode steps whose gate/up GEMM reads the caller's rows itself (no
# permute): the cfg5 shape at the 512-id limit, a ragged one, one with
# C = 2048 (several K stages) and one whose rows are zero-padded from C = 200
# to 256 before the GEMM reads them.
GATHERED = [
    (64, 1024, 64, 8, 256),
    (37, 512, 40, 4, 320),
    (16, 2048, 32, 2, 128),
    (24, 200, 16, 4, 192),
]


@pytest.mark.parametrize("shape", GATHERED)
def test_f32_rows_gathered_like_bf16_rows(shape):
    """The same bf16-representable rows as fp32 and as bf16 tensors: the
    fp32 step routes identically and its outputs, rounded to bf16, equal the
    bf16 step's bit for bit (the gathered fp32 rows are rounded to the same
    bf16 products the bf16 rows hold); both within the fp8 bar of the
    oracle."""
    N, Cm, E, k, H = shape
    inp = make_case("gath", N, Cm, E, k, H, "bf16", "fp8")
    print(f"case {inp.cfg}", flush=True)
    y16, r16 = forward(layer_for(inp), inp)
    cfg32 = dataclasses.replace(inp.cfg, name="gath_f32io", act="f32")
    inp32 = dataclasses.replace(inp, cfg=cfg32)
    y32, r32 = forward(layer_for(inp32), inp32)
    for key in r16:
        np.testing.assert_array_equal(r32[key], r16[key], err_msg=key)
    y32b = torch.from_numpy(y32).bfloat16().float().numpy()
    np.testing.assert_array_equal(y32b, y16)
    ref = O.forward(inp32, with_y=True)
    check_routing(r32, ref)
    check_close(y32, ref["y"], TOL["fp8"], "gath_f32io")


def test_f32_rows_gathered_nonfinite_stay_in_their_token():
    """A NaN and an infinity in two fp32 rows of a permute-free decode step:
    the fp32 step still matches the bf16 step on the same rows bit for bit
    (NaN where the bf16 step has NaN), and every other token's output is
    finite, so the gathered rows (and the padding rows of a tile, which
    re-read a segment's last token) reach no other token's output."""
    N, Cm, E, k, H = 64, 1024, 64, 8, 256
    inp = make_case("nonfin", N, Cm, E, k, H, "bf16", "fp8")
    inp.x[5, 17] = np.nan
    inp.x[9, 3] = np.inf
    print(f"case {inp.cfg}", flush=True)
    y16, r16 = forward(layer_for(inp), inp)
    inp32 = dataclasses.replace(inp, cfg=dataclasses.replace(inp.cfg, name="nonfin_f32io",
                                                              act="f32"))
    y32, r32 = forward(layer_for(inp32), inp32)
    for key in r16:
        np.testing.assert_array_equal(r32[key], r16[key], err_msg=key)
    np.testing.assert_array_equal(torch.from_numpy(y32).bfloat16().float().numpy(), y16)
    others = np.setdiff1d(np.arange(N), [5, 9])
    assert np.isfinite(y32[others]).all()


def test_f32_rows_rounded_to_nearest_even():
    """Every fp32 element sits a quarter, half or three quarters of a bf16
    step above a bf16 value (or one unit either side of the half).  With a
    zero router weight both steps route on the bias alone, so the fp32 step
    and the bf16 step on the host's nearest-even rounding of the rows
    (ties to even) agree bit for bit only if the decode GEMM rounds the
    gathered fp32 rows the same way; truncation or ties away from zero
    would move about half of the elements by one step."""
    N, Cm, E, k, H = 64, 1024, 64, 8, 256
    inp = make_case("rne", N, Cm, E, k, H, "f32", "fp8")
    inp.Wr[:] = 0.0
    rng = np.random.default_rng(11)
    hi = wl.bf16_round(inp.x).view(np.uint32) & np.uint32(0xFFFF0000)
    lo = rng.choice(np.array([0x4000, 0x8000, 0x8000, 0xC000, 0x7FFF, 0x8001], np.uint32),
                    size=hi.shape)
    inp.x[:] = (hi | lo).view(np.float32)
    print(f"case {inp.cfg}", flush=True)
    y32, r32 = forward(layer_for(inp), inp)
    cfg16 = dataclasses.replace(inp.cfg, name="rne_bf16", act="bf16")
    inp16 = dataclasses.replace(inp, cfg=cfg16, x=wl.bf16_round(inp.x))
    y16, r16 = forward(layer_for(inp16), inp16)
    for key in r16:
        np.testing.assert_array_equal(r32[key], r16[key], err_msg=key)
    y32b = torch.from_numpy(y32).bfloat16().float().numpy()
    np.testing.assert_array_equal(y32b, y16)


def test_f32_tensors_low_precision_weights_do_not_train():
    """Training with fp32 tensors needs fp32 weights; the bf16-product
    option is an inference format and says so."""
    from mgpt_amd import capi
    inp = make_case("mixbwd", 64, 128, 4, 2, 64, "f32", "bf16")
    layer = layer_for(inp)
    with pytest.raises(capi.MoEError) as ei:
        layer.forward(torch.from_numpy(inp.x).cuda(), train=True)
    assert ei.value.status == capi.MGPT_ERR_UNSUPPORTED


def test_workspace_grows_with_tokens():
    """The workspace size never decreases as N grows (a reserve() for the
    largest N covers every smaller one), across the split router's range
    (E > 16, N < 4096) and the large-M GEMM's partial tiles."""
    from mgpt_amd.moe import MoELayer
    for act, w in (("bf16", "bf16"), ("bf16", "fp8"), ("f32", "f32"), ("f32", "bf16")):
        layer = MoELayer(200, 256, 64, 8, act=act, weights=w)
        prev = prev_t = 0
        for n in list(range(1, 64)) + list(range(3900, 4300, 7)) + [8192, 20000]:
            b = layer.workspace_bytes(n)
            assert b >= prev, (act, w, n, b, prev)
            prev = b
            if w == act:
                b = layer.train_workspace_bytes(n)
                assert b >= prev_t, (act, w, n, b, prev_t)
                prev_t = b
