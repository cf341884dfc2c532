"""The C++ drop-in (mgpt_amd/host/MoELayer.{h,cpp}) inside the engine.

CPU: the drop-in compiles against the engine's own headers (Layer.h,
Tensor.h, LinearLayer.h, SwiGLU.h under /root/reference) and keeps the
engine's public MoELayer interface (layers/MoELayer.h:36-51).
GPU: tests/engine/_build/dropin_main -- the engine's unmodified Tensor,
LinearLayer and SwiGLU sources with the drop-in in place of MoELayer.cpp --
runs the engine's MoE shape and backward test, full forwards whose outputs
are compared with the oracle (fp32: 1e-5) and whose expert counts must equal
the reference fixture's, and full backwards whose din and parameter
gradients are compared with the oracle's backward (fp32: 1e-5).
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


def _run(args):
    print("dropin_main", *args, flush=True)
    return subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(BIN), reason="engine test binary not built")
def test_engine_moe_shapes():
    r = _run(["shapes"])
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(BIN), reason="engine test binary not built")
@pytest.mark.parametrize("name", ["small_f32", "ragged_k3", "cfg1"])
def test_engine_forward_matches_reference(name):
    case = C.ALL_CASES[name]
    inp = C.build_inputs(case)
    fx = np.load(os.path.join(HERE, "golden", name + ".npz"))
    with tempfile.TemporaryDirectory() as d:
        ip, op = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        write_input(ip, inp)
        r = _run(["run", ip, op])
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
@pytest.mark.skipif(not os.path.exists(BIN), reason="engine test binary not built")
@pytest.mark.parametrize("name", ["small_f32", "ragged_k3", "cfg1"])
def test_engine_backward_matches_reference(name):
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
        r = _run(["backward", ip, dp, op])
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
