"""The committed reference checkpoint (tests/golden/gptbin/small.npz) as
files on disk, and MoEInputs built from one of its blocks."""
from __future__ import annotations

import os

import numpy as np

import cases as C
from mgpt_amd import workload as wl

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "gptbin", "small.npz")


def fixture():
    return np.load(FIXTURE, allow_pickle=False)


def write_bin(tmp_path, legacy: bool = False, cut: int = 0) -> str:
    """The reference's checkpoint bytes; legacy drops completed_steps (the
    4-int header of older files), cut removes that many trailing bytes."""
    blob = fixture()["bin"].tobytes()
    if legacy:
        blob = blob[:16] + blob[20:]
    if cut:
        blob = blob[:-cut]
    p = os.path.join(str(tmp_path), "legacy.bin" if legacy else "model.bin")
    with open(p, "wb") as f:
        f.write(blob)
    return p


def block_inputs(params, N: int, act: str, seed: int = 5) -> wl.MoEInputs:
    """MoEInputs of the checkpoint block whose get_parameters() list is
    `params`, with N unit-RMS tokens from the portable generator."""
    g = C.GPTBIN
    Cc, E, H, k = g["C"], g["E"], g["H"], g["k"]
    cfg = wl.MoEConfig("gptbin", N, Cc, E, k, H, act, act, "normal")
    x = wl.normal_f32(seed, 1, N * Cc).reshape(N, Cc)
    if act == "bf16":
        x = wl.bf16_round(x)
    ex = [params[2 + 6 * e: 8 + 6 * e] for e in range(E)]
    stack = lambda i: np.stack([p[i] for p in ex])   # noqa: E731
    return wl.MoEInputs(cfg, x, params[0], params[1].reshape(-1), stack(0),
                        stack(1).reshape(E, H), stack(2), stack(3).reshape(E, H), stack(4),
                        stack(5).reshape(E, Cc), None)
