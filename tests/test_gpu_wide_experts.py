"""GPU parity of the forward with more experts than a wave has lanes
(64 < E <= 512), and of its training, against the reference.

The reference's layer takes any expert count (pipeline/CLIConfig.h:177-178).
Here such handles run the split router (logits per expert or per group of
64 experts, then a block softmax / top-k over rows of up to 512 experts),
the permute's offsets scan in wave-sized chunks with eight or nine ballots
on the expert ids, the 256 x 256 GEMMs once per group of 64 experts, and
the generic grouped GEMMs whose tile lookup scans the counts 64 experts at
a time.
Routing must be bit-exact with the committed fixtures of the compiled
reference (full arrays for the small cases, digests for the large one);
outputs are compared with the oracle's fp32 forward at 1e-5 (fp32), 2e-2
(bf16), 6e-2 (fp8 weights), normwise and elementwise, as in
tests/test_gpu_parity.py.  The fused block runs the same wide router with
normalisation.  Training runs too: the small wide cases are in
tests/test_gpu_backward.py against the reference's fixtures, a large-M one
here against the oracle.
"""
import numpy as np
import pytest

import cases as C
import oracle_lib as O
from test_gpu_parity import TOL, check_close, check_routing, fixture, run_gpu

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

WIDE = [c.name for c in C.WIDE_CASES]


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()   # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)


@pytest.mark.parametrize("name", WIDE)
def test_wide_forward_parity(name):
    case = C.ALL_CASES[name]
    print(f"case {name}: {case.cfg}", flush=True)
    fx = fixture(name)
    inp = C.build_inputs(case)
    layer, y, r, counts_host, _ = run_gpu(inp)
    check_routing(r, fx, full=case.full_arrays)
    assert counts_host == [float(c) for c in fx["counts"]]
    ref = O.forward(inp)   # every token (a few seconds at most)
    check_close(y, ref["y"], TOL[case.cfg.weights], name)
    if "rows" in fx.files:
        check_close(y[fx["rows"]], fx["y_rows"], TOL[case.cfg.weights], name + " reference rows")


@pytest.mark.parametrize("N,E,rb", [(150, 128, "normal"), (4096, 256, "zero")])
def test_wide_fused_block(N, E, rb):
    """out = x + MoE(RMSNorm(x) * gamma) with E = 128 and 256: the wide
    router normalises the rows (1/rms bit-exact; at 4096 tokens x 256
    experts in the 64-expert-group logits kernel), routing bit-exact with the
    oracle's block, out at the bf16 bar."""
    from mgpt_amd import workload as wl
    cfg = wl.MoEConfig("wide_blk", N, 128, E, 4, 64, "bf16", "bf16", rb)
    inp = wl.make_inputs(cfg, C.SEED + 77, bias_std=0.02)
    N = cfg.N
    t = np.arange(N)
    x1 = wl.bf16_round((inp.x * (np.float32(1.0) + (t % 4).astype(np.float32))[:, None])
                       .astype(np.float32))
    gamma = (np.float32(1.0) + wl.normal_f32(C.SEED, 4013, cfg.C, std=0.2)).astype(np.float32)
    inp.Wr[:] = wl.bf16_round(inp.Wr)
    from mgpt_amd.moe import MoELayer
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act="bf16", weights="bf16")
    layer.load_parameters(inp.params(raw=True))
    xd = torch.from_numpy(x1).cuda().to(torch.bfloat16)
    out = layer.forward_block(xd, torch.from_numpy(gamma).cuda(), C.BLOCK_EPS)
    torch.cuda.synchronize()
    r = {k: v.cpu().numpy() for k, v in layer.routing().items()}
    ref = O.block(inp, x1, gamma, C.BLOCK_EPS)
    assert np.array_equal(layer.rstd().cpu().numpy().view(np.uint32), ref["rstd"].view(np.uint32))
    assert np.array_equal(r["counts"], ref["counts"])
    assert np.array_equal(r["topk_idx"], ref["idx"])
    assert np.array_equal(r["topk_p"].view(np.uint32), ref["topp"].view(np.uint32))
    assert np.array_equal(r["perm"], ref["perm"])
    check_close(out.float().cpu().numpy(), ref["out"], TOL["bf16"], "wide block")


def test_wide_repeats_and_graph_replay():
    """Two eager forwards and a captured graph's replays give the same bits
    (no state carried between calls; the histogram is rewritten each time)."""
    case = C.ALL_CASES["wide_e128_k8"]
    inp = C.build_inputs(case)
    layer, y, r, _, ys = run_gpu(inp, repeat=2)
    assert np.array_equal(ys[0], ys[1])
    x = torch.from_numpy(np.ascontiguousarray(inp.x)).cuda().to(torch.bfloat16)
    out = torch.empty_like(x)
    layer.forward_into(x, out)   # workspace at this N before capture
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        layer.forward_into(x, out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.float().cpu().numpy(), y)


def test_wide_training_large_m():
    """Training at E = 96 on bf16 rows with enough tokens per expert for the
    128 x 128 grouped GEMMs, the tokens spread over every expert (zero router
    bias): dx and the 2 + 6E gradients against the
    oracle's backward at the bf16 bar (the small wide cases run in
    tests/test_gpu_backward.py with the reference's fixtures)."""
    from mgpt_amd import workload as wl
    from test_gpu_backward import check_all, make_layer, run_backward
    cfg = wl.MoEConfig("wide_train", 2048, 128, 96, 4, 96, "bf16", "bf16", "zero")
    inp = wl.make_inputs(cfg, C.SEED + 91, bias_std=0.02)
    inp.x[:] = wl.bf16_round(inp.x)
    inp.Wr[:] = wl.bf16_round(inp.Wr)
    dy = wl.bf16_round(np.random.default_rng(96).standard_normal((cfg.N, cfg.C))
                       .astype(np.float32))
    out = run_backward(make_layer(inp), inp, dy)
    ref = O.backward(inp, dy)
    check_all(out, ref, TOL["bf16"], "wide train")


# (N, C, E, k, H, act, router bias): one decode token over 65 experts, an odd
# expert count over a width that is not a multiple of 64 (fp32), top-1 of 256,
# a bf16 shape with 97 experts on the small-row tiles, and 4096 tokens over
# 256 experts (the router's logits in 64-expert groups).  With a zero router
# bias the tokens spread over (nearly) every expert, so more than 64 experts
# hold rows (the weight gradients' and the permute's scans past one wave).
EDGE = [
    (1, 64, 65, 8, 64, "bf16", "normal"),
    (33, 100, 255, 8, 40, "f32", "zero"),
    (64, 128, 256, 1, 64, "f32", "zero"),
    (700, 192, 97, 3, 96, "bf16", "zero"),
    # enough (64 tokens, 64 experts) blocks for the grouped logits kernel
    (4096, 128, 256, 8, 64, "bf16", "zero"),
    # past 256 experts (nine id bits, the 512-wide softmax row and token
    # gradients), prefill-sized with the grouped kernels and decode-sized
    (8192, 64, 384, 8, 64, "bf16", "zero"),
    (64, 128, 512, 4, 64, "f32", "zero"),
]


@pytest.mark.parametrize("N,Cm,E,k,H,act,rb", EDGE)
def test_wide_edge_shapes_forward_and_backward(N, Cm, E, k, H, act, rb):
    """Routing bit-exact with the oracle's forward (counts, ids, weights,
    permutation), y at the forward's bar, dx and every gradient at the
    backward's."""
    from mgpt_amd import workload as wl
    from test_gpu_backward import check_all, make_layer, run_backward
    cfg = wl.MoEConfig(f"wide_edge_{E}", N, Cm, E, k, H, act, act, rb)
    inp = wl.make_inputs(cfg, C.SEED + E + N, bias_std=0.02)
    dy = np.random.default_rng(E).standard_normal((N, Cm)).astype(np.float32)
    if act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
        inp.Wr[:] = wl.bf16_round(inp.Wr)
        dy = wl.bf16_round(dy)
    print(f"case {cfg}", flush=True)
    ref = O.forward(inp)
    _, y, _, _, _ = run_gpu(inp)
    check_close(y, ref["y"], TOL[act], cfg.name)
    layer = make_layer(inp)
    out = run_backward(layer, inp, dy)
    r = {n: v.cpu().numpy() for n, v in layer.routing().items()}
    assert np.array_equal(r["counts"], ref["counts"])
    assert np.array_equal(r["topk_idx"], ref["idx"])
    assert np.array_equal(r["topk_p"].view(np.uint32), ref["topp"].view(np.uint32))
    assert np.array_equal(r["perm"], ref["perm"])
    print(f"{cfg.name}: {int((ref['counts'] > 0).sum())} experts with rows", flush=True)
    check_all(out, O.backward(inp, dy), TOL[act], cfg.name)


def test_more_than_512_experts_is_refused():
    from mgpt_amd import capi
    from mgpt_amd.moe import MoELayer
    with pytest.raises(capi.MoEError) as err:
        MoELayer(64, 64, 513, 2, act="f32")
    assert err.value.status == capi.MGPT_ERR_UNSUPPORTED
