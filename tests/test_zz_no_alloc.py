"""mgpt_moe_forward_noalloc (the forward whose workspace is the library's
built-in per-device scratch array) against mgpt_moe_forward with a caller
workspace, through the C ABI: the same kernels on the same inputs, so the
outputs and the routing must be identical bit for bit, on two calls in a row
with the second one smaller (the array keeps the first call's contents), for
fp32, bf16, fp8-weight and padded-width handles; a token count whose
workspace exceeds the array is refused with a clear error.
"""
import ctypes

import numpy as np
import pytest

import cases as C
from mgpt_amd import workload as wl

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SCRATCH_BYTES = 64 << 20   # MGPT_MOE_NOALLOC_SCRATCH_BYTES in include/mgpt_moe.h


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    capi.lib()   # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)


def _layer(cfg, seed):
    from mgpt_amd.moe import MoELayer
    inp = wl.make_inputs(cfg, seed, bias_std=0.05)
    if cfg.act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    dt = torch.float32 if cfg.act == "f32" else torch.bfloat16
    return layer, torch.from_numpy(inp.x).to("cuda").to(dt)


def _noalloc(layer, x):
    from mgpt_amd import capi
    y = torch.empty_like(x)
    n = x.shape[0]
    st = torch.cuda.current_stream().cuda_stream
    capi.check(capi.lib().mgpt_moe_forward_noalloc(layer._h, x.data_ptr(), y.data_ptr(), n, st))
    torch.cuda.synchronize()
    counts = layer_counts(layer)
    return y, counts


def layer_counts(layer):
    from mgpt_amd import capi
    c = np.zeros(layer.E, np.int32)
    capi.check(capi.lib().mgpt_moe_expert_counts(layer._h, c.ctypes.data, layer.E))
    return c


SHAPES = [
    # (N, C, E, k, H, act, weights): decode-shaped fp8 and bf16 (the callers
    # this is for; bf16 prefill shapes on the large-tile GEMM need more than
    # the array: its split-K partials alone take 256 KB per CU), fp32, and a
    # width that is not a multiple of 64 (padded rows inside the workspace)
    (64, 2048, 64, 8, 1408, "bf16", "fp8"),
    (200, 256, 16, 2, 384, "bf16", "bf16"),
    (300, 128, 6, 3, 192, "f32", "f32"),
    (90, 96, 5, 2, 72, "f32", "f32"),
    # more experts than a wave has lanes (the split router and generic GEMMs)
    (48, 512, 256, 8, 256, "bf16", "fp8"),
    (64, 256, 128, 4, 384, "bf16", "bf16"),
]


@pytest.mark.parametrize("N,Cm,E,k,H,act,weights", SHAPES)
def test_noalloc_matches_caller_workspace(N, Cm, E, k, H, act, weights):
    cfg = wl.MoEConfig(f"noalloc_{Cm}", N, Cm, E, k, H, act, weights, "normal")
    layer, x = _layer(cfg, C.SEED + N)
    print(f"noalloc case {cfg}", flush=True)
    assert layer.workspace_bytes(N) <= SCRATCH_BYTES
    for n in (N, max(1, N // 3)):   # the second call smaller than the first
        xs = x[:n].contiguous()
        y_ref = layer.forward(xs)
        torch.cuda.synchronize()
        c_ref = layer_counts(layer)
        y, c = _noalloc(layer, xs)
        assert torch.equal(y.view(torch.int16) if y.dtype == torch.bfloat16 else y.view(torch.int32),
                           y_ref.view(torch.int16) if y.dtype == torch.bfloat16
                           else y_ref.view(torch.int32)), f"output differs at N={n}"
        assert np.array_equal(c, c_ref), f"counts differ at N={n}"


def test_noalloc_refuses_beyond_its_scratch():
    from mgpt_amd import capi
    cfg = wl.MoEConfig("noalloc_big", 64, 1024, 16, 2, 2816, "bf16", "bf16", "normal")
    layer, x = _layer(cfg, C.SEED)
    n = 1
    while layer.workspace_bytes(n) <= SCRATCH_BYTES:
        n *= 2
    big = torch.zeros((n, cfg.C), dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(big)
    st = capi.lib().mgpt_moe_forward_noalloc(layer._h, big.data_ptr(), y.data_ptr(), n, None)
    assert st == capi.MGPT_ERR_WORKSPACE_TOO_SMALL
    assert "scratch" in capi.lib().mgpt_moe_last_error().decode()
    # the handle still works afterwards, with and without the scratch array
    y_ref = layer.forward(x)
    y2, _ = _noalloc(layer, x)
    assert torch.equal(y2.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("N,Cm,E,k,H,act,weights", SHAPES[:2])
def test_noalloc_captured_graph_replays(N, Cm, E, k, H, act, weights):
    """The use the entry point is for: mgpt_moe_forward_noalloc captured into
    a HIP graph (its scratch address was looked up at handle creation, so
    the capture records only kernels).  Each replay on new inputs equals an
    eager noalloc forward of the same inputs bit for bit, with eager work
    between the replays."""
    from mgpt_amd import capi
    cfg = wl.MoEConfig(f"noalloc_graph_{Cm}", N, Cm, E, k, H, act, weights, "normal")
    layer, x = _layer(cfg, C.SEED + 7 * N)
    print(f"noalloc graph case {cfg}", flush=True)
    static_x = x.clone()
    static_y = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                 # warm-up off the capture
        capi.check(capi.lib().mgpt_moe_forward_noalloc(layer._h, static_x.data_ptr(),
                                                       static_y.data_ptr(), N,
                                                       side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        capi.check(capi.lib().mgpt_moe_forward_noalloc(
            layer._h, static_x.data_ptr(), static_y.data_ptr(), N,
            torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    iv = torch.int16 if x.dtype == torch.bfloat16 else torch.int32
    for r in range(3):
        ctx = torch.roll(x, shifts=-5 * r, dims=0).contiguous()
        static_x.copy_(ctx)
        g.replay()
        torch.cuda.synchronize()
        got = static_y.clone()
        want, _ = _noalloc(layer, ctx)            # eager work between replays
        assert torch.equal(got.view(iv), want.view(iv)), f"replay {r} differs"
    print(f"3 replays at N = {N} equal the eager noalloc forward", flush=True)
