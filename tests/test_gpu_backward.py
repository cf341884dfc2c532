"""GPU parity of the MoE block backward (mgpt_moe_forward_train +
mgpt_moe_backward through the C ABI) against the reference.

Expected values are the CPU oracle's backward (oracle_moe_backward), which
reproduces the reference's own CPU backward bit for bit
(tests/test_oracle_backward.py), on the same inputs and upstream gradient;
cfg2 is compared with the committed reference fixture's sampled rows and
entries.  dx and each of the 2+6E gradients must satisfy, per tensor,
    ||g - g_ref||_2 / ||g_ref||_2 <= tol  and  max|g - g_ref| <= tol * max|g_ref|
with tol = 1e-5 for fp32 handles and 2e-2 for bf16 (the forward's bars).
Gradients of experts no token chose must stay exactly zero, accumulation
across calls must add, and repeated runs must give identical bits.
"""
import os

import numpy as np
import pytest

import cases as C
import oracle_lib as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = {"f32": 1e-5, "bf16": 2e-2}
BWD_DIR = os.path.join(os.path.dirname(__file__), "golden", "backward")
NAMES = ("dWr", "dbr", "dWg", "dbg", "dWu", "dbu", "dWd", "dbd")

# NaN inputs (nan_rows) are left out: the reference propagates NaN through
# whole gradient matrices, which says nothing about the kernels.
GPU_BWD = [n for n in C.BACKWARD_CASES
           if C.ALL_CASES[n].gpu and C.ALL_CASES[n].cfg.weights != "fp8"
           and C.ALL_CASES[n].tweak != "nan_rows" and n != "cfg2"]


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()   # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)


def _dt(cfg):
    return torch.float32 if cfg.act == "f32" else torch.bfloat16


def make_layer(inp):
    from mgpt_amd.moe import MoELayer
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    return layer


def run_backward(layer, inp, dy, zero=True):
    cfg = inp.cfg
    x = torch.from_numpy(np.ascontiguousarray(inp.x)).to("cuda").to(_dt(cfg))
    d = torch.from_numpy(np.ascontiguousarray(dy)).to("cuda").to(_dt(cfg))
    if zero:
        layer.zero_grad()
    layer.forward(x, train=True)
    dx = layer.backward(d)
    torch.cuda.synchronize()
    g = [t.cpu().numpy() for t in layer.get_gradients()]
    E = cfg.E
    out = {"dx": dx.float().cpu().numpy(), "dWr": g[0], "dbr": g[1].reshape(-1)}
    for i, n in enumerate(NAMES[2:]):
        arr = np.stack([g[2 + 6 * e + i] for e in range(E)])
        out[n] = arr.reshape(E, -1) if n.startswith("db") else arr
    return out


def rel_errors(got, ref):
    d = (np.asarray(got, np.float64) - np.asarray(ref, np.float64)).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    rel = np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)
    mx = np.max(np.abs(d)) / max(np.max(np.abs(r)), 1e-30) if d.size else 0.0
    return rel, mx


def check_all(out, ref, tol, name):
    for n in ("dx",) + NAMES:
        rel, mx = rel_errors(out[n], ref[n])
        print(f"{name} {n}: normwise {rel:.3e}  max/max {mx:.3e}  (tol {tol})", flush=True)
        assert rel <= tol, f"{name} {n}: normwise error {rel} > {tol}"
        assert mx <= tol, f"{name} {n}: elementwise error {mx} > {tol}"


@pytest.mark.parametrize("name", GPU_BWD)
def test_backward_parity(name):
    case = C.ALL_CASES[name]
    print(f"case {name}: {case.cfg}", flush=True)
    inp = C.build_inputs(case)
    dy = C.build_dy(case)
    out = run_backward(make_layer(inp), inp, dy)
    ref = O.backward(inp, dy)
    check_all(out, ref, TOL[case.cfg.act], name)


@pytest.mark.parametrize("name,k", [("exact_tiles_k2", 2), ("one_expert", 1)])
def test_backward_forced_routing(name, k):
    """The backward on routing forced as in the forward's tile-boundary test
    (tests/test_gpu_parity.py): expert segments that end on 256-row tile
    boundaries, or every row in one expert, which the weight gradients then
    cut into several row chunks alone.  Against the oracle's backward."""
    from mgpt_amd import workload as wl
    N, Cm, H, E = 4096, 256, 256, 8
    cfg = wl.MoEConfig(f"forced_bwd_{name}", N, Cm, E, k, H, "bf16", "bf16", "zero")
    inp = wl.make_inputs(cfg, C.SEED + 7, bias_std=0.02)
    inp.x[:] = wl.bf16_round(inp.x)
    inp.Wr[:] = 0.0
    inp.br[:] = 0.0
    if name == "one_expert":
        inp.br[5] = 5.0
    else:
        t = np.arange(N)
        inp.x[:, :E] = 0.0
        inp.x[t, t % E] = 1.0
        inp.Wr[np.arange(E), np.arange(E)] = 10.0
    dy = wl.bf16_round(np.random.default_rng(9).standard_normal((N, Cm)).astype(np.float32))
    out = run_backward(make_layer(inp), inp, dy)
    ref = O.backward(inp, dy)
    check_all(out, ref, TOL["bf16"], cfg.name)


def test_backward_cfg2_against_reference_fixture():
    """cfg2 (bf16, 8192 tokens, 8 experts, H = 1376): sampled dx rows and
    gradient entries against the reference's own backward."""
    case = C.ALL_CASES["cfg2"]
    print(f"case cfg2: {case.cfg}", flush=True)
    fx = np.load(os.path.join(BWD_DIR, "cfg2.npz"), allow_pickle=False)
    inp = C.build_inputs(case)
    out = run_backward(make_layer(inp), inp, C.build_dy(case))
    tol = TOL["bf16"]
    rel, mx = rel_errors(out["dx"][fx["rows"]], fx["dx_rows"])
    print(f"cfg2 dx rows: normwise {rel:.3e}  max/max {mx:.3e}", flush=True)
    assert rel <= tol and mx <= tol
    for n in NAMES:
        got = out[n].reshape(-1)[fx[n + "_at"]]
        rel, mx = rel_errors(got, fx[n + "_val"])
        print(f"cfg2 {n} samples: normwise {rel:.3e}  max/max {mx:.3e}", flush=True)
        assert rel <= tol and mx <= tol, n


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_backward_accumulates_and_is_deterministic(act):
    """Two calls without zero_grad add exactly (the kernels are
    deterministic, so the second contribution equals the first);
    zero_grad resets; dx repeats bit for bit."""
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("acc", 300, 128, 6, 2, 192, act, act, "normal")
    inp = wl.make_inputs(cfg, seed=11, bias_std=0.05)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    dy = np.random.default_rng(5).standard_normal((cfg.N, cfg.C)).astype(np.float32)
    if act == "bf16":
        dy = wl.bf16_round(dy)
    layer = make_layer(inp)
    a = run_backward(layer, inp, dy)
    b = run_backward(layer, inp, dy, zero=False)
    c = run_backward(layer, inp, dy)
    assert np.array_equal(a["dx"], b["dx"]) and np.array_equal(a["dx"], c["dx"])
    for n in NAMES:
        assert np.array_equal(b[n], 2 * a[n]), n
        assert np.array_equal(c[n], a[n]), n


def test_two_stream_backward_repeats_and_matches_serial():
    """At cfg3's shape the bf16 backward runs part of its work on a second
    stream (the weight gradients beside the d(act) and dX products, which run
    on part of the CUs).  Twenty steps must repeat every gradient and dx bit
    for bit (a missing fork or join dependency would show as a difference),
    and a step with stage timing (every launch serial on one stream, all CUs)
    must give the same weight gradients; dx may differ within bf16 rounding,
    since dX on fewer CUs splits a different last round along K."""
    from mgpt_amd import workload as wl
    cfg = wl.CONFIGS["cfg3"]
    inp = wl.make_inputs(cfg, seed=7)
    dy = wl.bf16_round(np.random.default_rng(3).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    layer = make_layer(inp)
    x = torch.from_numpy(np.ascontiguousarray(inp.x)).to("cuda").to(torch.bfloat16)
    d = torch.from_numpy(dy).to("cuda").to(torch.bfloat16)

    def step():
        layer.zero_grad()
        layer.forward(x, train=True)
        dx = layer.backward(d)
        torch.cuda.synchronize()
        return dx.clone(), [t.clone() for t in layer.get_gradients()]

    dx0, g0 = step()
    for i in range(20):
        dx, g = step()
        assert torch.equal(dx, dx0), i
        assert all(torch.equal(a, b) for a, b in zip(g, g0)), i
    layer.set_profiling(True)
    dxs, gs = step()
    layer.set_profiling(False)
    assert all(torch.equal(a, b) for a, b in zip(gs, g0))
    rel, mx = rel_errors(dxs.float().cpu().numpy(), dx0.float().cpu().numpy())
    assert rel <= 4e-3 and mx <= 4e-3, (rel, mx)


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_backward_after_zero_grad_overwrites_stale_gradients(act):
    """zero_grad only marks the gradients zero; the next backward writes
    them.  After a backward that gave every expert a gradient, zero_grad and
    a backward routed to experts 0 and 1 only must equal a fresh layer's
    gradients bit for bit (the other experts exactly zero), and
    get_gradients right after zero_grad must read zeros."""
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("stale", 256, 64, 6, 2, 96, act, act, "zero")   # every expert chosen
    inp = wl.make_inputs(cfg, seed=4, bias_std=0.05)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    dy = wl.bf16_round(np.random.default_rng(2).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    layer = make_layer(inp)
    first = run_backward(layer, inp, dy)
    for n in ("dWg", "dWd", "dbd"):
        assert np.all(np.any(first[n].reshape(cfg.E, -1) != 0, axis=1)), n
    inp.br[:] = np.array([9, 8, -9, -9, -9, -9], np.float32)   # experts 0, 1 always win
    layer.load_parameters(inp.params(raw=True))
    again = run_backward(layer, inp, dy)
    fresh = run_backward(make_layer(inp), inp, dy)
    assert np.array_equal(again["dx"], fresh["dx"])
    for n in NAMES:
        assert np.array_equal(again[n], fresh[n]), n
    for n in ("dWg", "dbg", "dWu", "dbu", "dWd", "dbd"):
        assert np.all(again[n][2:] == 0) and np.any(again[n][:2] != 0), n
    layer.zero_grad()
    assert all(not torch.any(t != 0) for t in layer.get_gradients())


def test_accumulation_with_row_chunks():
    """bf16 large-M shape whose weight-gradient contraction is cut into row
    chunks (experts of 3943, 2410, 1837 and 2 rows against 1024-row
    chunks): a second backward without zero_grad adds the same contribution
    again (to within one rounding of the sum per element), and zero_grad +
    backward repeats the first result bit for bit."""
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("chunks", 4096, 256, 4, 2, 256, "bf16", "bf16", "normal")
    inp = wl.make_inputs(cfg, seed=21, bias_std=0.05)
    inp.x[:] = wl.bf16_round(inp.x)
    dy = wl.bf16_round(np.random.default_rng(8).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    layer = make_layer(inp)
    a = run_backward(layer, inp, dy)
    b = run_backward(layer, inp, dy, zero=False)
    c = run_backward(layer, inp, dy)
    ref = O.backward(inp, dy)
    check_all(a, ref, TOL["bf16"], "chunks")
    for n in NAMES:
        assert np.array_equal(c[n], a[n]), n
        two = 2.0 * a[n].astype(np.float64)
        err = np.max(np.abs(b[n] - two)) / max(np.max(np.abs(two)), 1e-30)
        assert err <= 1e-6, (n, err)


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_unchosen_experts_get_no_gradient(act):
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("unchosen", 128, 64, 6, 2, 96, act, act, "zero")
    inp = wl.make_inputs(cfg, seed=3, bias_std=0.05)
    inp.br[:] = np.array([9, 8, -9, -9, -9, -9], np.float32)   # experts 0, 1 always win
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    dy = wl.bf16_round(np.random.default_rng(9).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    out = run_backward(make_layer(inp), inp, dy)
    for n in ("dWg", "dbg", "dWu", "dbu", "dWd", "dbd"):
        assert np.all(out[n][2:] == 0) and np.any(out[n][:2] != 0), n
    ref = O.backward(inp, dy)
    check_all(out, ref, TOL[act], f"unchosen-{act}")


def test_backward_profiling_modes():
    """Profiling mode 1 times every backward stage; mode 2 (events only
    around the forward's gate/up GEMM) records no backward events, so the
    backward stage times report no profiled backward; profiled backwards
    give the same bits as unprofiled ones."""
    from mgpt_amd import capi
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("prof", 512, 128, 4, 2, 256, "bf16", "bf16", "zero")
    inp = wl.make_inputs(cfg, seed=6, bias_std=0.05)
    inp.x[:] = wl.bf16_round(inp.x)
    dy = wl.bf16_round(np.random.default_rng(4).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    layer = make_layer(inp)
    ref = run_backward(layer, inp, dy)
    layer.set_profiling(True)
    out = run_backward(layer, inp, dy)
    st = layer.backward_stage_times()
    assert st["backwards"] == 1 and all(v > 0.0 for k, v in st.items() if k != "backwards"), st
    layer.set_profiling(True, gemm_only=True)
    out2 = run_backward(layer, inp, dy)
    with pytest.raises(capi.MoEError) as ei:
        layer.backward_stage_times()
    assert ei.value.status == capi.MGPT_ERR_NOT_READY
    layer.set_profiling(False)
    for n in ("dx",) + NAMES:
        assert np.array_equal(out[n], ref[n]) and np.array_equal(out2[n], ref[n]), n


def test_fp8_handle_has_no_backward():
    from mgpt_amd import capi
    from mgpt_amd import workload as wl
    from mgpt_amd.moe import MoELayer
    cfg = wl.MoEConfig("fp8bwd", 64, 128, 4, 2, 128, "bf16", "fp8", "zero")
    inp = wl.make_inputs(cfg, seed=1)
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act="bf16", weights="fp8")
    layer.load_parameters(inp.params(raw=True))
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16)
    with pytest.raises(capi.MoEError) as ei:
        layer.forward(x, train=True)
    assert ei.value.status == capi.MGPT_ERR_UNSUPPORTED


def _collect(layer, cfg, dx):
    g = [t.cpu().numpy() for t in layer.get_gradients()]
    out = {"dx": dx.float().cpu().numpy(), "dWr": g[0], "dbr": g[1].reshape(-1)}
    for i, n in enumerate(NAMES[2:]):
        arr = np.stack([g[2 + 6 * e + i] for e in range(cfg.E)])
        out[n] = arr.reshape(cfg.E, -1) if n.startswith("db") else arr
    return out


@pytest.mark.parametrize("act,E,k", [("f32", 6, 2), ("bf16", 6, 2), ("bf16", 128, 4)])
def test_graph_captured_training_step(act, E, k):
    """forward_train + backward captured into one HIP graph.  A captured
    backward always adds.  Captured right after zero_grad, the pending zeros
    are part of the graph: every replay equals an eager zero_grad + step, bit
    for bit.  Captured with nothing pending, replays accumulate (2x after two),
    and zero_grad between replays (now a fill on the stream) restarts the
    sum.  Eager steps between replays leave the replays unchanged.  E = 128
    runs the wide router, token and weight gradients."""
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("cap", 300, 128, E, k, 192, act, act, "normal")
    inp = wl.make_inputs(cfg, seed=11, bias_std=0.05)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    dy = np.random.default_rng(5).standard_normal((cfg.N, cfg.C)).astype(np.float32)
    if act == "bf16":
        dy = wl.bf16_round(dy)
    layer = make_layer(inp)
    eager = run_backward(layer, inp, dy)          # allocates the workspace and gradients
    dt = _dt(cfg)
    x = torch.from_numpy(np.ascontiguousarray(inp.x)).to("cuda").to(dt)
    d = torch.from_numpy(np.ascontiguousarray(dy)).to("cuda").to(dt)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                 # warm-up off the capture
        layer.forward_into(x, y, train=True)
        layer.backward_into(d, dx)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    def same(got, ref, mult=1):
        for n in ("dx",) + NAMES:
            want = ref[n] if n == "dx" else mult * ref[n]
            assert np.array_equal(got[n], want), (n, mult)

    layer.zero_grad()                             # eager: zeros pending at capture
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        layer.forward_into(x, y, train=True)
        layer.backward_into(d, dx)
    torch.cuda.synchronize()
    for r in range(2):
        g1.replay()
        torch.cuda.synchronize()
        same(_collect(layer, cfg, dx), eager)
        run_backward(layer, inp, dy)              # eager work between replays
        print(f"{act}: graph with the pending zeros, replay {r} equals the eager step",
              flush=True)

    layer.zero_grad()                             # a fill now: nothing pending at capture
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        layer.forward_into(x, y, train=True)
        layer.backward_into(d, dx)
    torch.cuda.synchronize()
    layer.zero_grad()
    g2.replay()
    torch.cuda.synchronize()
    same(_collect(layer, cfg, dx), eager, 1)
    g2.replay()
    torch.cuda.synchronize()
    same(_collect(layer, cfg, dx), eager, 2)
    layer.zero_grad()
    g2.replay()
    torch.cuda.synchronize()
    same(_collect(layer, cfg, dx), eager, 1)
    print(f"{act}: adding graph accumulates 1x, 2x, then 1x after zero_grad", flush=True)


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_accumulate_gradients_host_and_device(act):
    """mgpt_moe_accumulate_gradients adds the handle's gradients into
    caller buffers (Tensor::add_grad, utils/Tensor.cpp:638-650): host
    destinations (copied in windows of whole pieces) and device
    destinations must both give dest + gradient, one rounded add per
    element, equal to get_gradients' values added on the host."""
    from mgpt_amd import capi
    from mgpt_amd import workload as wl
    import ctypes
    cfg = wl.MoEConfig("accum", 200, 64, 5, 2, 96, act, act, "normal")
    inp = wl.make_inputs(cfg, seed=17, bias_std=0.05)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    dy = wl.bf16_round(np.random.default_rng(9).standard_normal((cfg.N, cfg.C)).astype(np.float32))
    layer = make_layer(inp)
    out = run_backward(layer, inp, dy)
    grads = [t.cpu().numpy() for t in layer.get_gradients()]
    rng = np.random.default_rng(3)
    base = [rng.standard_normal(g.shape).astype(np.float32) for g in grads]
    # host destinations
    host = [np.ascontiguousarray(b.copy()) for b in base]
    ptrs = (ctypes.c_void_p * len(host))(*[h.ctypes.data for h in host])
    st = torch.cuda.current_stream().cuda_stream
    capi.check(capi.lib().mgpt_moe_accumulate_gradients(layer._h, ptrs, len(host), 0, st))
    # device destinations
    dev = [torch.from_numpy(b.copy()).cuda() for b in base]
    dptrs = (ctypes.c_void_p * len(dev))(*[t.data_ptr() for t in dev])
    capi.check(capi.lib().mgpt_moe_accumulate_gradients(layer._h, dptrs, len(dev), 1, st))
    torch.cuda.synchronize()
    for i, (b, g) in enumerate(zip(base, grads)):
        want = (b + g).astype(np.float32)
        assert np.array_equal(host[i], want), f"host piece {i}"
        assert np.array_equal(dev[i].cpu().numpy(), want), f"device piece {i}"
    assert out["dx"].shape == (cfg.N, cfg.C)
