"""ctypes binding of the CPU oracle (oracle/libmoe_oracle.so).

Test infrastructure: the checker the HIP path is compared with.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "libmoe_oracle.so")
REF_DRIVER = os.path.join(ORACLE_DIR, "_ref", "ref_driver")

_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-C", ORACLE_DIR, "libmoe_oracle.so"], check=True,
                           capture_output=True)
        L = ctypes.CDLL(LIB_PATH)
        vp, i = ctypes.c_void_p, ctypes.c_int
        L.oracle_expf.argtypes = [ctypes.c_float]
        L.oracle_expf.restype = ctypes.c_float
        L.oracle_expf_array.argtypes = [vp, vp, ctypes.c_int64]
        L.oracle_router_logits.argtypes = [i, i, i, vp, vp, vp, vp]
        L.oracle_softmax.argtypes = [i, i, vp, vp]
        L.oracle_topk.argtypes = [i, i, i, vp, vp, vp]
        L.oracle_dispatch.argtypes = [i, i, i, vp, vp, vp, vp]
        L.oracle_moe_forward.argtypes = [i] * 5 + [vp] * 17
        L.oracle_moe_forward.restype = i
        L.oracle_moe_tokens.argtypes = [i] * 5 + [vp] * 11
        L.oracle_moe_tokens.restype = i
        L.oracle_rmsnorm.argtypes = [i, i, ctypes.c_float, vp, vp]
        L.oracle_moe_backward.argtypes = [i] * 5 + [vp] * 19
        L.oracle_moe_backward.restype = i
        L.oracle_rmsnorm_scaled.argtypes = [i, i, ctypes.c_float, vp, vp, vp, vp]
        L.oracle_moe_block.argtypes = [i] * 5 + [ctypes.c_float] + [vp] * 17
        L.oracle_moe_block.restype = i
        L.oracle_rmsnorm_backward.argtypes = [i, i] + [vp] * 6
        L.oracle_moe_block_backward.argtypes = [i] * 5 + [ctypes.c_float] + [vp] * 21
        L.oracle_moe_block_backward.restype = i
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def expf(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().oracle_expf_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def router_logits(x, Wr, br):
    x, Wr, br = _f32(x), _f32(Wr), _f32(br)
    N, C = x.shape
    E = Wr.shape[1]
    out = np.empty((N, E), np.float32)
    lib().oracle_router_logits(N, C, E, _p(x), _p(Wr), _p(br), _p(out))
    return out


def softmax(logits):
    logits = _f32(logits)
    out = np.empty_like(logits)
    lib().oracle_softmax(logits.shape[0], logits.shape[1], _p(logits), _p(out))
    return out


def topk(probs, k):
    probs = _f32(probs)
    N, E = probs.shape
    idx = np.empty((N, k), np.int32)
    p = np.empty((N, k), np.float32)
    lib().oracle_topk(N, E, k, _p(probs), _p(idx), _p(p))
    return idx, p


def dispatch(idx, E):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    N, k = idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E, np.int32)
    perm = np.empty(N * k, np.int32)
    lib().oracle_dispatch(N, E, k, _p(idx), _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm


def forward(inp, with_y: bool = True) -> dict:
    """Full reference-order forward of a workload.MoEInputs."""
    cfg = inp.cfg
    N, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    arrs = [_f32(a) for a in (inp.x, inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu,
                              inp.Wd, inp.bd)]
    out = {
        "y": np.empty((N, C), np.float32) if with_y else None,
        "logits": np.empty((N, E), np.float32), "probs": np.empty((N, E), np.float32),
        "idx": np.empty((N, k), np.int32), "topp": np.empty((N, k), np.float32),
        "counts": np.empty(E, np.int32), "offsets": np.empty(E, np.int32),
        "perm": np.empty(N * k, np.int32),
    }
    rc = lib().oracle_moe_forward(N, C, H, E, k, *[_p(a) for a in arrs],
                                  _p(out["y"]), _p(out["logits"]), _p(out["probs"]),
                                  _p(out["idx"]), _p(out["topp"]), _p(out["counts"]),
                                  _p(out["offsets"]), _p(out["perm"]))
    assert rc == 0
    return out


def tokens(inp, idx, topp, rows) -> np.ndarray:
    """Output rows of the given tokens under the given routing."""
    cfg = inp.cfg
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    topp = _f32(topp)
    arrs = [_f32(a) for a in (inp.x, inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd, inp.bd)]
    y = np.empty((rows.size, cfg.C), np.float32)
    rc = lib().oracle_moe_tokens(cfg.C, cfg.H, cfg.E, cfg.k, rows.size, _p(rows), _p(arrs[0]),
                                 _p(idx), _p(topp), *[_p(a) for a in arrs[1:]], _p(y))
    assert rc == 0
    return y


def tokens_parallel(inp, idx, topp, rows, threads: int | None = None) -> np.ndarray:
    """tokens() over chunks of rows on several host threads (the oracle is
    reentrant and ctypes releases the GIL during the call); every output row
    is an independent computation, so the result equals one call's."""
    import concurrent.futures as cf
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    threads = threads or max(1, min(16, os.cpu_count() or 1))
    chunks = [c for c in np.array_split(rows, threads * 4) if c.size]
    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        parts = list(ex.map(lambda c: tokens(inp, idx, topp, c), chunks))
    return np.concatenate(parts) if parts else np.empty((0, inp.cfg.C), np.float32)


GRAD_NAMES = ("dWr", "dbr", "dWg", "dbg", "dWu", "dbu", "dWd", "dbd")


def load_variant(path: str) -> ctypes.CDLL:
    """Binds a separately built copy of the oracle (planted-mistake builds)."""
    L = ctypes.CDLL(path)
    L.oracle_moe_backward.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p] * 19
    L.oracle_moe_backward.restype = ctypes.c_int
    L.oracle_moe_block_backward.argtypes = ([ctypes.c_int] * 5 + [ctypes.c_float] +
                                            [ctypes.c_void_p] * 21)
    L.oracle_moe_block_backward.restype = ctypes.c_int
    return L


def backward(inp, dy, library=None) -> dict:
    """Reference-order backward of a workload.MoEInputs for upstream dy:
    dx [N,C] and the parameter gradients of one call (zero-started), with
    expert gradients stacked over experts like the weights."""
    cfg = inp.cfg
    N, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    arrs = [_f32(a) for a in (inp.x, inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu,
                              inp.Wd, inp.bd)]
    dy = _f32(dy)
    assert dy.shape == (N, C)
    out = {"dx": np.empty((N, C), np.float32)}
    for name, a in zip(GRAD_NAMES, arrs[1:]):
        out[name] = np.zeros(a.shape, np.float32)
    rc = (library or lib()).oracle_moe_backward(N, C, H, E, k, *[_p(a) for a in arrs], _p(dy),
                                   _p(out["dx"]), *[_p(out[n]) for n in GRAD_NAMES])
    assert rc == 0
    return out


def rmsnorm_scaled(x, gamma, eps=1e-5):
    """(RMSNorm(x) * gamma, rstd) as the engine's RMSNormLayer computes them."""
    x, gamma = _f32(x), _f32(gamma)
    out = np.empty_like(x)
    rstd = np.empty(x.shape[0], np.float32)
    lib().oracle_rmsnorm_scaled(x.shape[0], x.shape[1], eps, _p(x), _p(gamma), _p(out), _p(rstd))
    return out, rstd


def block(inp, x1, gamma, eps=1e-5) -> dict:
    """The fused block out = x1 + MoE(RMSNorm(x1) * gamma) with its routing."""
    cfg = inp.cfg
    N, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    x1, gamma = _f32(x1), _f32(gamma)
    arrs = [_f32(a) for a in (inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd, inp.bd)]
    out = {"out": np.empty((N, C), np.float32), "xn": np.empty((N, C), np.float32),
           "rstd": np.empty(N, np.float32), "idx": np.empty((N, k), np.int32),
           "topp": np.empty((N, k), np.float32), "counts": np.empty(E, np.int32),
           "perm": np.empty(N * k, np.int32)}
    rc = lib().oracle_moe_block(N, C, H, E, k, eps, _p(x1), _p(gamma), *[_p(a) for a in arrs],
                                *[_p(out[n]) for n in ("out", "xn", "rstd", "idx", "topp",
                                                       "counts", "perm")])
    assert rc == 0
    return out


def rmsnorm_backward(dout, x_hat, gamma, rstd):
    """(dx, dgamma) of the engine's RMSNormLayer backward (dgamma from zero)."""
    dout, x_hat, gamma, rstd = _f32(dout), _f32(x_hat), _f32(gamma), _f32(rstd)
    N, C = dout.shape
    dx = np.empty_like(dout)
    dgamma = np.zeros(C, np.float32)
    lib().oracle_rmsnorm_backward(N, C, _p(dout), _p(x_hat), _p(gamma), _p(rstd), _p(dx),
                                  _p(dgamma))
    return dx, dgamma


def block_backward(inp, x1, gamma, dout, eps=1e-5, library=None) -> dict:
    """Backward of the fused block for upstream dout: dx [N,C] (= dx1),
    dgamma [C] and the MoE parameter gradients of one call (zero-started)."""
    cfg = inp.cfg
    N, C, H, E, k = cfg.N, cfg.C, cfg.H, cfg.E, cfg.k
    x1, gamma, dout = _f32(x1), _f32(gamma), _f32(dout)
    arrs = [_f32(a) for a in (inp.Wr, inp.br, inp.Wg, inp.bg, inp.Wu, inp.bu, inp.Wd, inp.bd)]
    out = {"dx": np.empty((N, C), np.float32), "dgamma": np.zeros(C, np.float32)}
    for name, a in zip(GRAD_NAMES, arrs):
        out[name] = np.zeros(a.shape, np.float32)
    rc = (library or lib()).oracle_moe_block_backward(
        N, C, H, E, k, eps, _p(x1), _p(gamma), *[_p(a) for a in arrs], _p(dout), _p(out["dx"]),
        _p(out["dgamma"]), *[_p(out[n]) for n in GRAD_NAMES])
    assert rc == 0
    return out


def rmsnorm(x, eps=1e-5):
    x = _f32(x)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(x.shape[0], x.shape[1], eps, _p(x), _p(out))
    return out
