"""Writes the golden fixtures from the reference's own CPU MoE forward.

Runs oracle/_ref/ref_driver (the unmodified reference sources compiled by
`make -C oracle ref`) on every case of cases.py and stores, per case,
tests/golden/<case>.npz with the reference's outputs:

  counts [E] int32, offsets [E] int32          always, verbatim
  idx [N,k], topp [N,k], perm [N*k],           verbatim for small cases
  logits [N,E], probs [N,E]
  sha256 digests of idx/topp/perm/logits/probs/y   always
  rows [r], y_rows [r,C]                       outputs of sampled tokens

Inputs are not stored: they are rebuilt from the case definition and seed.
Usage: python tests/golden/make_golden.py [case ...]   (default: all cases)
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import cases as C  # noqa: E402
from mgpt_amd import workload as wl  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "ref_driver")


def write_input(path: str, inp: wl.MoEInputs) -> None:
    cfg = inp.cfg
    with open(path, "wb") as f:
        f.write(b"MGPTMOE1")
        f.write(np.array([cfg.N, cfg.C, cfg.H, cfg.E, cfg.k], dtype=np.int32).tobytes())
        f.write(np.ascontiguousarray(inp.x, dtype=np.float32).tobytes())
        for p in inp.params():
            f.write(np.ascontiguousarray(p, dtype=np.float32).tobytes())


def read_output(path: str):
    raw = open(path, "rb").read()
    assert raw[:8] == b"MGPTOUT1", "bad reference output"
    N, Cc, E, k = np.frombuffer(raw, dtype=np.int32, count=4, offset=8)
    off = 24
    out = {}

    def take(name, dtype, n):
        nonlocal off
        out[name] = np.frombuffer(raw, dtype=dtype, count=n, offset=off).copy()
        off += n * 4

    A = N * k
    take("y", np.float32, N * Cc)
    take("idx", np.int32, A)
    take("topp", np.float32, A)
    take("counts", np.int32, E)
    take("offsets", np.int32, E)
    take("perm", np.int32, A)
    take("logits", np.float32, N * E)
    take("probs", np.float32, N * E)
    out["y"] = out["y"].reshape(N, Cc)
    out["idx"] = out["idx"].reshape(N, k)
    out["topp"] = out["topp"].reshape(N, k)
    out["logits"] = out["logits"].reshape(N, E)
    out["probs"] = out["probs"].reshape(N, E)
    return out


def run_reference(inp: wl.MoEInputs):
    with tempfile.TemporaryDirectory() as d:
        ip, op = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        write_input(ip, inp)
        subprocess.run([REF, "run", ip, op], check=True)
        return read_output(op)


def make_case(case: C.Case) -> None:
    t0 = time.time()
    inp = C.build_inputs(case)
    ref = run_reference(inp)
    rows = C.sample_rows(case.cfg.N)
    fx = {
        "counts": ref["counts"], "offsets": ref["offsets"],
        "rows": rows, "y_rows": ref["y"][rows],
    }
    for name in ("idx", "topp", "perm", "logits", "probs", "y"):
        fx["sha_" + name] = np.array(wl.digest(ref[name]))
    if case.full_arrays:
        for name in ("idx", "topp", "perm", "logits", "probs"):
            fx[name] = ref[name]
    np.savez_compressed(os.path.join(HERE, case.name + ".npz"), **fx)
    cnt = ref["counts"]
    print(f"{case.name}: N={case.cfg.N} E={case.cfg.E} k={case.cfg.k} "
          f"counts max/mean={cnt.max() / max(cnt.mean(), 1e-9):.2f} min={cnt.min()} "
          f"({time.time() - t0:.1f}s)", flush=True)


def main(argv):
    if not os.path.exists(REF):
        sys.exit("oracle/_ref/ref_driver missing: run `make -C oracle ref` first")
    names = argv or list(C.ALL_CASES)
    for n in names:
        make_case(C.ALL_CASES[n])


if __name__ == "__main__":
    main(sys.argv[1:])
