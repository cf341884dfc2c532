"""The C++ drop-in (mgpt_amd/host/MoELayer.{h,cpp}) inside the engine.

CPU: the drop-in compiles against the engine's own headers (Layer.h,
Tensor.h, LinearLayer.h, SwiGLU.h under /root/reference) and keeps the
engine's public MoELayer interface (layers/MoELayer.h:36-51).
GPU: tests/engine/_build/dropin_main -- the engine's unmodified Tensor,
LinearLayer and SwiGLU sources with the drop-in in place of MoELayer.cpp,
host tensors -- and tests/engine/_build/dropin_dev -- the same with the
engine's device-memory primitives over HIP, so parameters, inputs, the
optimizer state and a Scratchpad live on the device -- each run the engine's
own MoE test at its shape (C = 16), full forwards whose outputs are compared
with the oracle (fp32: 1e-5) and whose expert counts must equal the reference
fixture's, full backwards whose din and parameter gradients are compared
with the oracle's backward (fp32: 1e-5), and the Trainer's step sequence with
the engine's own AdamWOptimizer, whose every forward must use the parameters
as the optimizer left them.  dropin_dev also runs the Generator's loop with
fp8 expert weights behind the fp32 tensors, with no host wait per step.
tests/engine/_build/gpt_main -- the engine's whole GPT with the drop-in as
every block's MoE -- loads a reference-written checkpoint with the engine's
own GPT::load_weights_bin and must reproduce the reference GPT's logits.
"""
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import cases as C
import oracle_lib as O
from make_golden import write_input

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ENGINE = "/root/reference/src/main"
BIN = os.path.join(HERE, "engine", "_build", "dropin_main")
DEV_BIN = os.path.join(HERE, "engine", "_build", "dropin_dev")
BINS = [pytest.param(BIN, id="host"), pytest.param(DEV_BIN, id="device")]
HOST = os.path.join(ROOT, "mgpt_amd", "host")


def public_methods(header_text):
    body = header_text.split("public:", 1)[1]
    return set(re.findall(r"\b(\w+)\s*\(", body))


@pytest.mark.skipif(not os.path.isdir(ENGINE), reason="engine sources not present")
def test_dropin_compiles_against_engine_headers():
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-include", "cstring",
           f"-I{HOST}", f"-I{ROOT}/include", f"-I{ENGINE}/utils",
           f"-I{ENGINE}/neuralnetwork/layers", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__",
           os.path.join(HOST, "MoELayer.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.isdir(ENGINE), reason="engine sources not present")
def test_dropin_keeps_engine_interface():
    ref = public_methods(open(os.path.join(ENGINE, "neuralnetwork/layers/MoELayer.h")).read())
    ours = public_methods(open(os.path.join(HOST, "MoELayer.h")).read())
    missing = ref - ours
    assert not missing, f"drop-in lacks {missing}"


def _run(args, binary=BIN):
    if not os.path.exists(binary):
        pytest.skip(f"{binary} not built")
    print(os.path.basename(binary), *args, flush=True)
    return subprocess.run([binary, *args], capture_output=True, text=True, timeout=300)


@pytest.mark.gpu
@pytest.mark.parametrize("binary", BINS)
def test_engine_moe_shapes(binary):
    """The engine's own MoE test (tests/networkTest/moeTests.cpp:6-76) at its
    shape C = 16, E = 4, k = 2, all-ones input and dout."""
    r = _run(["shapes"], binary)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("binary", BINS)
@pytest.mark.parametrize("name", ["moetests_shape", "small_f32", "ragged_k3", "cfg1"])
def test_engine_forward_matches_reference(name, binary):
    case = C.ALL_CASES[name]
    inp = C.build_inputs(case)
    fx = np.load(os.path.join(HERE, "golden", name + ".npz"))
    with tempfile.TemporaryDirectory() as d:
        ip, op = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        write_input(ip, inp)
        r = _run(["run", ip, op], binary)
        assert r.returncode == 0, r.stdout + r.stderr
        raw = open(op, "rb").read()
    assert raw[:8] == b"MGPTDRP1"
    N, Cc, E = np.frombuffer(raw, np.int32, 3, 8)
    y = np.frombuffer(raw, np.float32, N * Cc, 20).reshape(N, Cc)
    counts = np.frombuffer(raw, np.float32, E, 20 + 4 * N * Cc)
    assert np.array_equal(counts, fx["counts"].astype(np.float32))
    ref = O.forward(inp)["y"]
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    mx = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"{name}: normwise {rel:.3e} max/max {mx:.3e}")
    assert rel <= 1e-5 and mx <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("binary", BINS)
@pytest.mark.parametrize("name", ["moetests_shape", "small_f32", "ragged_k3", "cfg1"])
def test_engine_backward_matches_reference(name, binary):
    """The drop-in's backward_into inside the engine: din and every
    parameter's Tensor::grad (added with the engine's own add_grad) against
    the oracle backward, which matches the reference's bit for bit; fp32
    handle, tolerance 1e-5 normwise and elementwise per tensor."""
    case = C.ALL_CASES[name]
    inp = C.build_inputs(case)
    dy = C.build_dy(case)
    with tempfile.TemporaryDirectory() as d:
        ip, dp, op = (os.path.join(d, n) for n in ("in.bin", "dy.bin", "grad.bin"))
        write_input(ip, inp)
        np.ascontiguousarray(dy, np.float32).tofile(dp)
        r = _run(["backward", ip, dp, op], binary)
        assert r.returncode == 0, r.stdout + r.stderr
        raw = open(op, "rb").read()
    assert raw[:8] == b"MGPTGRD1"
    cfg = inp.cfg
    N, Cc, H, E = cfg.N, cfg.C, cfg.H, cfg.E
    off = 28
    got = []
    for n in [N * Cc, Cc * E, E] + [Cc * H, H, Cc * H, H, H * Cc, Cc] * E:
        got.append(np.frombuffer(raw, np.float32, n, off))
        off += 4 * n
    assert off == len(raw)
    ref = O.backward(inp, dy)
    want = [ref["dx"], ref["dWr"], ref["dbr"]]
    for e in range(E):
        want += [ref["dWg"][e], ref["dbg"][e], ref["dWu"][e], ref["dbu"][e], ref["dWd"][e],
                 ref["dbd"][e]]
    worst = 0.0
    for g, w in zip(got, want):
        w = np.asarray(w, np.float64).reshape(-1)
        dd = g.astype(np.float64) - w
        scale = max(np.abs(w).max(), 1e-30)
        rel = np.linalg.norm(dd) / max(np.linalg.norm(w), 1e-30)
        worst = max(worst, rel, np.abs(dd).max() / scale)
    print(f"{name}: worst per-tensor error {worst:.3e}")
    assert worst <= 1e-5


def _rel(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    d = got - want
    return (np.linalg.norm(d) / max(np.linalg.norm(want), 1e-30),
            np.abs(d).max() / max(np.abs(want).max(), 1e-30))


@pytest.mark.gpu
@pytest.mark.parametrize("binary", BINS)
@pytest.mark.parametrize("name", C.TRAIN_CASES)
def test_engine_training_steps_use_updated_weights(name, binary):
    """The Trainer's step (zero grads, forward_into, backward_into,
    AdamWOptimizer::step; pipeline/Trainer.cpp:303-386) twice, then a
    forward, through the drop-in with the engine's own optimizer.
      * Every forward after a step equals the oracle's forward on the
        parameters as the optimizer left them (dumped by the driver), at the
        fp32 bar 1e-5: the layer reads the updated weights.
      * The first forward equals the reference's (tests/golden/train/).
      * The steps move the output far beyond 1e-5, so stale weights fail.
      * The whole sequence tracks the reference's own (same fixture): the
        parameters after each step entrywise within 1e-3 of the step's median
        size, and the outputs at the fp32 bar 1e-5.  (AdamW's first steps
        normalise each gradient entry, g / (|g| + eps), so an entry whose
        gradient is near zero could move differently for a 1e-6 difference
        in the gradients; on these cases the largest deviation is below 1e-5
        of the median step, and the kernels are deterministic.)
    """
    from test_oracle_train import flat_params, with_params, fixture as train_fixture
    case = C.ALL_CASES[name]
    inp = C.build_inputs(case)
    dy = C.build_dy(case)
    fx = train_fixture(name)
    cfg = inp.cfg
    N, Cc, H, E = cfg.N, cfg.C, cfg.H, cfg.E
    with tempfile.TemporaryDirectory() as d:
        ip, dp, op = (os.path.join(d, n) for n in ("in.bin", "dy.bin", "out.bin"))
        write_input(ip, inp)
        np.ascontiguousarray(dy, np.float32).tofile(dp)
        r = _run(["train", ip, dp, op, str(C.TRAIN_STEPS), repr(C.TRAIN_LR)], binary)
        assert r.returncode == 0, r.stdout + r.stderr
        from make_golden import read_train
        got = read_train(open(op, "rb").read(), cfg)
    S = C.TRAIN_STEPS
    rel, mx = _rel(got["y"][0], fx["y"][0])
    print(f"{name} y0 vs reference: {rel:.2e} {mx:.2e}", flush=True)
    assert rel <= 1e-5 and mx <= 1e-5
    for s in range(1, S + 1):
        ref = O.forward(with_params(inp, got["params"][s - 1]))["y"]
        rel, mx = _rel(got["y"][s], ref)
        print(f"{name} y{s} vs oracle on the stepped parameters: {rel:.2e} {mx:.2e}", flush=True)
        assert rel <= 1e-5 and mx <= 1e-5
    moved, _ = _rel(got["y"][S], got["y"][0])
    assert moved > 100 * 1e-5, f"the steps moved the output by only {moved}"
    p0 = flat_params(inp)
    for s in range(S):
        worst = 0.0
        for i, p in enumerate(got["params"][s]):
            at = C.sample_flat(p.size, 64)
            step = np.abs(fx[f"p{s}_{i}_val"].astype(np.float64) - p0[i][at])
            scale = max(np.median(step), 1e-30)
            dev_ = np.abs(p[at].astype(np.float64) - fx[f"p{s}_{i}_val"]).max() / scale
            worst = max(worst, dev_)
        print(f"{name} step {s + 1}: parameters vs reference, worst |diff| / median step "
              f"{worst:.2e}", flush=True)
        assert worst <= 1e-3
    for s in range(1, S + 1):
        rel, mx = _rel(got["y"][s], fx["y"][s])
        print(f"{name} y{s} vs reference: {rel:.2e} {mx:.2e}", flush=True)
        assert rel <= 1e-5 and mx <= 1e-5


@pytest.mark.gpu
def test_engine_decode_loop_fp8_device_tensors(tmp_path):
    """The Generator's sampling loop (pipeline/Generator.cpp:24-36) at cfg5's
    shape (N = 64, C = 2048, E = 64, k = 8, H = 1408) through the drop-in:
    the engine's fp32 device tensors, fp8 e4m3 expert weights
    (set_expert_dtype) and inference forwards (set_inference).  64 steps
    are enqueued behind a 300 ms device spin and must return to the host
    long before it ends (no host wait and no synchronous copy inside a
    step); the output must match the reference's cfg5 rows (the fixture) at
    the fp8 bar 6e-2."""
    case = C.ALL_CASES["cfg5"]
    cfg = case.cfg
    inp = C.build_inputs(case)
    fx = np.load(os.path.join(HERE, "golden", "cfg5.npz"))
    xp, rp, op = (str(tmp_path / n) for n in ("x.bin", "router.bin", "out.bin"))
    np.ascontiguousarray(inp.x, np.float32).tofile(xp)
    with open(rp, "wb") as f:
        f.write(np.ascontiguousarray(inp.Wr, np.float32).tobytes())
        f.write(np.ascontiguousarray(inp.br, np.float32).tobytes())
    spin_ms = 300.0
    r = _run(["decode", xp, rp, str(C.SEED), str(cfg.C), str(cfg.H), str(cfg.E), str(cfg.k),
              "64", str(spin_ms), op], DEV_BIN)
    assert r.returncode == 0, r.stdout + r.stderr
    print(r.stdout.strip(), flush=True)
    raw = open(op, "rb").read()
    assert raw[:8] == b"MGPTDEC1"
    N, Cc = np.frombuffer(raw, np.int32, 2, 8)
    enqueue_ms = float(np.frombuffer(raw, np.float32, 1, 16)[0])
    y = np.frombuffer(raw, np.float32, N * Cc, 20).reshape(N, Cc)
    assert enqueue_ms < 0.5 * spin_ms, f"64 steps took {enqueue_ms} ms to enqueue"
    rows = fx["rows"]
    rel, mx = _rel(y[rows], fx["y_rows"])
    print(f"cfg5 fp8 through the drop-in: {rel:.2e} {mx:.2e}", flush=True)
    assert rel <= 6e-2 and mx <= 6e-2


GPT_BIN = os.path.join(HERE, "engine", "_build", "gpt_main")


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(GPT_BIN), reason="engine GPT test binary not built")
def test_engine_gpt_loads_checkpoint_and_matches_reference_logits(tmp_path):
    """The engine's whole GPT (its own sources: embedding, attention, norms,
    LM head) with the drop-in as every block's MoE: GPT::load_weights_bin
    fills the drop-in's tensors from a checkpoint the reference wrote, and
    GPT::forward gives the reference's logits (its own GPT with its own
    MoELayer on the same file and tokens, tests/golden/gptbin/small.npz)
    to 1e-5 normwise and elementwise (fp32 handles)."""
    import gptbin_case as G
    g = C.GPTBIN
    fx = G.fixture()
    path = G.write_bin(tmp_path)
    ids = os.path.join(str(tmp_path), "ids.bin")
    out = os.path.join(str(tmp_path), "logits.bin")
    C.gptbin_ids().tofile(ids)
    print("gpt_main logits", flush=True)
    r = subprocess.run([GPT_BIN, "logits", path] + [str(g[n]) for n in ("heads", "E", "k", "H")]
                       + [ids, out], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(out, np.float32).reshape(fx["logits"].shape)
    ref = fx["logits"]
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    mx = np.abs(got - ref).max() / np.abs(ref).max()
    print(f"GPT logits: normwise {rel:.3e} max/max {mx:.3e}")
    assert rel <= 1e-5 and mx <= 1e-5
