"""GPU: the MoE layer inside the engine's sampling loop (decode integration).

The engine's Generator (pipeline/Generator.cpp:13-36) has no KV cache: every
step re-runs the whole context, cropped to max_seq_len, with B = 1, so the
MoE sees N = 1, 2, ..., S tokens while the context grows and N = S from then
on.  At cfg5's shape (S = 64, C = 2048, E = 64, k = 8, H = 1408, fp8
weights) these tests check that

  * every step of the growing loop routes its N tokens exactly as the
    reference routes the first N rows of the full context (routing is per
    token), and its output matches those rows of the reference output
    (fixture digests pin the oracle at N = 64) at the fp8 bar, 6e-2;
  * the loop never waits for the device: 64 steps enqueued behind a long
    device-side sleep return to the host long before the sleep ends (no
    device-to-host or pageable host-to-device copy, no synchronisation);
  * the steady-state step (N = S), captured once into a HIP graph, gives on
    every replay the same bits as the eager forward on the same context,
    with eager work and synchronisation between the replays.
"""
import os
import time

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from mgpt_amd import workload as wl

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 6e-2


@pytest.fixture(scope="module")
def cfg5():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mgpt_amd import capi
    from mgpt_amd.moe import MoELayer
    capi.lib()
    case = C.ALL_CASES["cfg5"]
    inp = C.build_inputs(case)
    cfg = inp.cfg
    layer = MoELayer(cfg.C, cfg.H, cfg.E, cfg.k, act=cfg.act, weights=cfg.weights)
    layer.load_parameters(inp.params(raw=True))
    layer.reserve(cfg.N)
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16)
    return inp, layer, x


def errors(got, ref):
    d = np.asarray(got, np.float64) - np.asarray(ref, np.float64)
    r = np.asarray(ref, np.float64)
    return (np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30),
            np.abs(d).max() / max(np.abs(r).max(), 1e-30))


def test_growing_context_matches_reference_rows(cfg5):
    inp, layer, x = cfg5
    S, k = inp.cfg.N, inp.cfg.k
    ref = O.forward(inp)
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg5.npz"),
                 allow_pickle=False)
    assert wl.digest(ref["idx"]) == str(fx["sha_idx"])
    ys = torch.empty((S, S, inp.cfg.C), dtype=torch.bfloat16, device="cuda")
    idx = torch.empty((S, S, k), dtype=torch.int32, device="cuda")
    print(f"decode loop N = 1..{S}", flush=True)
    for n in range(1, S + 1):
        layer.forward_into(x[:n], ys[n - 1, :n])
        idx[n - 1, :n].copy_(layer.routing()["topk_idx"])   # device to device
    torch.cuda.synchronize()
    ys, idx = ys.float().cpu().numpy(), idx.cpu().numpy()
    worst = 0.0
    for n in range(1, S + 1):
        assert np.array_equal(idx[n - 1, :n], ref["idx"][:n]), n
        rel, mx = errors(ys[n - 1, :n], ref["y"][:n])
        worst = max(worst, rel, mx)
        assert rel <= TOL and mx <= TOL, (n, rel, mx)
    print(f"worst error over the loop {worst:.3e} (tol {TOL})", flush=True)


def test_loop_never_waits_for_the_device(cfg5):
    inp, layer, x = cfg5
    S = inp.cfg.N
    y = torch.empty_like(x)
    for n in (1, S):                 # warm: kernels loaded, workspace reserved
        layer.forward_into(x[:n], y[:n])
    torch.cuda.synchronize()
    cycles = 400_000_000
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    torch.cuda._sleep(cycles)
    b.record()
    torch.cuda.synchronize()
    sleep_s = a.elapsed_time(b) / 1e3
    t0 = time.perf_counter()
    torch.cuda._sleep(cycles)
    for n in range(1, S + 1):
        layer.forward_into(x[:n], y[:n])
    host_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    print(f"device sleep {sleep_s * 1e3:.1f} ms; host enqueue of {S} steps behind it "
          f"{host_s * 1e3:.1f} ms", flush=True)
    assert sleep_s > 0.05
    assert host_s < 0.5 * sleep_s


def test_steady_state_step_graph_matches_eager(cfg5):
    inp, layer, x = cfg5
    S = inp.cfg.N
    static_x = x.clone()
    static_y = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.forward_into(static_x, static_y)    # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.forward_into(static_x, static_y)
    torch.cuda.synchronize()
    eager_y = torch.empty_like(x)
    for r in range(4):
        # a new context each step: the window slides by one token
        ctx = torch.roll(x, shifts=-r, dims=0).contiguous()
        static_x.copy_(ctx)
        g.replay()
        torch.cuda.synchronize()
        got = static_y.clone()
        layer.forward_into(ctx, eager_y)          # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager_y.view(torch.int16)), r
    print(f"{4} replays at N = {S} equal the eager forward", flush=True)
