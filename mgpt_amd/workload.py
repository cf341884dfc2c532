"""Seeded synthetic workloads for the MoE block (the five benchmark shapes).

The generator is counter-based (element i of stream s is a pure function of
(seed, s, i)) and uses only integer arithmetic and IEEE-754 correctly-rounded
float64 +, -, *, / and sqrt.  Logarithm and cosine are evaluated with fixed
polynomials below instead of libm or numpy's SIMD transcendental kernels,
whose last bits can differ between host CPUs; the same seed therefore gives
the same float32 arrays on this build host and on any GPU box, which is what
lets committed golden fixtures be checked against freshly generated inputs.

Normal variates: Box-Muller, z = sqrt(-2 ln u1) cos(2 pi u2), with u1 in
(0, 1] and u2 in [0, 1) taken from the top 53 bits of SplitMix64 outputs.

Input preparation follows the benchmark definition: x ~ N(0, 1), then RMSNorm
with gamma = 1 and eps = 1e-5 in the reference's float32 arithmetic
(/root/reference/src/main/utils/Tensor.cpp:769-802: sequential sum of
squares, r = 1/sqrt(ms/C + eps), out = (x*r)*1); weights ~ N(0, 0.02^2);
expert biases 0.  For bf16 configurations, activations and weights are
rounded to bfloat16 (round-to-nearest-even) and carried as float32 values,
so the reference CPU path and the bf16 kernels see the same numbers.
"""
from __future__ import annotations

import dataclasses
import hashlib
import math

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_seed(seed: int, stream: int) -> int:
    """Seed of an independent stream: SplitMix64 of (seed, stream)."""
    with np.errstate(over="ignore"):
        z = np.array([(seed * 0x100000001B3 + stream * 0x2545F4914F6CDD1D)
                      & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
        return int(_mix(z + _GAMMA)[0])


def uniform_bits(seed: int, start: int, count: int) -> np.ndarray:
    """SplitMix64 outputs number start .. start+count-1 of a stream."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        return _mix(np.uint64(seed) + i * _GAMMA)


_LN2 = 0.6931471805599453
_SQRT_HALF = 0.7071067811865476
_LOG_COEF = [1.0 / (2 * j + 1) for j in range(12)]          # atanh series
_COS_COEF = [(-1.0) ** n / math.factorial(2 * n) for n in range(12)]
_SIN_COEF = [(-1.0) ** n / math.factorial(2 * n + 1) for n in range(12)]
_HALF_PI = 1.5707963267948966


def _log(u: np.ndarray) -> np.ndarray:
    """ln(u) for u in (0, 1]: u = m 2^e, m in [sqrt(1/2), sqrt 2), ln m via
    the atanh series 2 s (1 + s^2/3 + s^4/5 + ...), s = (m-1)/(m+1)."""
    m, e = np.frexp(u)
    small = m < _SQRT_HALF
    m = np.where(small, m * 2.0, m)
    e = np.where(small, e - 1, e).astype(np.float64)
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    p = np.full_like(s, _LOG_COEF[-1])
    for c in reversed(_LOG_COEF[:-1]):
        p = p * s2 + c
    return e * _LN2 + 2.0 * s * p


def _cos_2pi(v: np.ndarray) -> np.ndarray:
    """cos(2 pi v) for v in [0, 1): quarter-turn reduction, then Taylor
    series of cos/sin on [0, pi/2)."""
    w = v * 4.0
    q = np.floor(w)
    f = w - q
    x = f * _HALF_PI
    x2 = x * x
    c = np.full_like(x, _COS_COEF[-1])
    for a in reversed(_COS_COEF[:-1]):
        c = c * x2 + a
    s = np.full_like(x, _SIN_COEF[-1])
    for a in reversed(_SIN_COEF[:-1]):
        s = s * x2 + a
    s = s * x
    q = q.astype(np.int64)
    return np.select([q == 0, q == 1, q == 2], [c, -s, -c], default=s)


def normal(seed: int, stream: int, count: int, start: int = 0) -> np.ndarray:
    """float64 N(0,1) variates start .. start+count-1 of a stream."""
    s = stream_seed(seed, stream)
    b = uniform_bits(s, 2 * start, 2 * count).reshape(count, 2)
    u1 = ((b[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (b[:, 1] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return np.sqrt(-2.0 * _log(u1)) * _cos_2pi(u2)


_CLIB = None


def _clib():
    """The C twin of this generator (mgpt_amd/csrc/workload_gen.c), if it has
    been built; it is ~50x faster and bit-identical."""
    global _CLIB
    if _CLIB is None:
        import ctypes
        import os
        path = os.path.join(os.path.dirname(__file__), "lib", "libmgpt_workload.so")
        if not os.path.exists(path):
            _CLIB = False
        else:
            lib = ctypes.CDLL(path)
            lib.mgpt_wl_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                               ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_double, ctypes.c_void_p]
            lib.mgpt_wl_normal_f32.restype = None
            lib.mgpt_wl_quantize_e4m3.argtypes = [ctypes.c_void_p, ctypes.c_int64,
                                                  ctypes.c_int64, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_void_p]
            lib.mgpt_wl_quantize_e4m3.restype = None
            _CLIB = lib
    return _CLIB or None


def normal_f32(seed: int, stream: int, count: int, std: float = 1.0,
               chunk: int = 1 << 22, use_c: bool = True) -> np.ndarray:
    """float32 values of std * N(0,1) variates 0 .. count-1 of a stream."""
    out = np.empty(count, dtype=np.float32)
    lib = _clib() if use_c else None
    if lib is not None:
        lib.mgpt_wl_normal_f32(seed, stream, 0, count, float(std),
                               out.ctypes.data)
        return out
    for a in range(0, count, chunk):
        n = min(chunk, count - a)
        out[a:a + n] = (normal(seed, stream, n, start=a) * std).astype(np.float32)
    return out


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest-even), returned as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))
         & np.uint32(0xFFFF0000))
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r)
    return r.astype(np.uint32).view(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values already on the bf16
    grid (as returned by bf16_round)."""
    return (np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
            >> np.uint32(16)).astype(np.uint16)


def rmsnorm_f32(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """RMSNorm with gamma = 1 in the reference's float32 order
    (utils/Tensor.cpp:769-802): sequential sum over channels."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, c = x.shape
    ms = np.zeros(n, dtype=np.float32)
    for j in range(c):
        col = x[:, j]
        ms = ms + col * col
    r = np.float32(1.0) / np.sqrt(ms / np.float32(c) + np.float32(eps))
    return (x * r[:, None]) * np.float32(1.0)


# ---------------------------------------------------------------- e4m3 (OCP)
def e4m3_decode_table() -> np.ndarray:
    """float32 value of every OCP FP8 E4M3FN byte (0x7F/0xFF are NaN)."""
    vals = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            vals[b] = np.nan
        elif e == 0:
            vals[b] = s * m * 2.0 ** -9
        else:
            vals[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Round float32 values to OCP E4M3FN bytes, nearest-even, saturating to
    +-448 (the largest finite value)."""
    v = np.asarray(v, dtype=np.float32)
    table = e4m3_decode_table()
    pos = table[:0x7F].astype(np.float64)           # bytes 0x00..0x7E, ascending
    a = np.minimum(np.abs(v).astype(np.float64), 448.0)
    hi = np.searchsorted(pos, a, side="left")       # first code >= a
    hi = np.minimum(hi, 0x7E)
    lo = np.maximum(hi - 1, 0)
    dlo = a - pos[lo]
    dhi = pos[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pos[hi] == a, hi, np.where(pick_hi, hi, lo)).astype(np.uint8)
    sign = (np.signbit(v) & (code != 0)).astype(np.uint8) << 7
    return code | sign


def quantize_e4m3_per_out_channel(w: np.ndarray, use_c: bool = True):
    """Per-output-channel scaling of a reference-layout weight W[in, out]:
    scale[o] = amax_o / 448 (1 if the column is all zero), q = e4m3(w/scale).
    Returns (q uint8 [in,out], scale float32 [out], dequantised float32).
    Uses the C twin (mgpt_wl_quantize_e4m3) when built; both agree bit for
    bit (tests/test_workload.py)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib = _clib() if use_c else None
    if lib is not None and w.ndim == 2:
        q = np.empty(w.shape, np.uint8)
        scale = np.empty(w.shape[1], np.float32)
        deq = np.empty(w.shape, np.float32)
        lib.mgpt_wl_quantize_e4m3(w.ctypes.data, w.shape[0], w.shape[1], q.ctypes.data,
                                  scale.ctypes.data, deq.ctypes.data)
        return q, scale, deq
    amax = np.max(np.abs(w), axis=0)
    scale = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    q = e4m3_encode(w / scale[None, :])
    deq = e4m3_decode_table()[q] * scale[None, :]
    return q, scale, deq.astype(np.float32)


# ------------------------------------------------------------------ configs
@dataclasses.dataclass(frozen=True)
class MoEConfig:
    name: str
    N: int
    C: int
    E: int
    k: int
    H: int
    act: str            # "f32" | "bf16"
    weights: str        # "f32" | "bf16" | "fp8"
    router_bias: str    # "zero" | "normal" | "zipf"
    B: int = 1
    T: int = 0

    @property
    def A(self) -> int:
        return self.N * self.k


# BASELINE.json configs[0..4]
CONFIGS = {
    "cfg1": MoEConfig("cfg1", 1024, 128, 8, 2, 512, "f32", "f32", "zero", 16, 64),
    "cfg2": MoEConfig("cfg2", 8192, 512, 8, 2, 1376, "bf16", "bf16", "zero", 32, 256),
    "cfg3": MoEConfig("cfg3", 16384, 1024, 16, 2, 2816, "bf16", "bf16", "normal", 64, 256),
    "cfg4": MoEConfig("cfg4", 32768, 2048, 64, 6, 1408, "bf16", "bf16", "zipf", 64, 512),
    "cfg5": MoEConfig("cfg5", 64, 2048, 64, 8, 1408, "bf16", "fp8", "zero", 1, 64),
    # Beyond the benchmark: cfg3's tokens and width over 128 fine-grained
    # experts, top-8 of H = 704 (the same expert FLOPs per token as cfg3),
    # with a zero router bias so the tokens spread over every expert.
    "wide128": MoEConfig("wide128", 16384, 1024, 128, 8, 704, "bf16", "bf16", "zero", 64, 256),
}

ZIPF_S = 1.1
ZIPF_BETA = 1.0

# stream ids
_S_X, _S_WR, _S_BR, _S_PERM = 1, 2, 3, 4
_S_EXPERT = 100          # + 8*e + {0: W_g, 1: W_u, 2: W_d, 3: b_g, 4: b_u, 5: b_d}


def router_bias(cfg: MoEConfig, seed: int) -> np.ndarray:
    E = cfg.E
    if cfg.router_bias == "zero":
        return np.zeros(E, dtype=np.float32)
    if cfg.router_bias == "normal":
        return normal_f32(seed, _S_BR, E)
    if cfg.router_bias == "zipf":
        # rank = seeded permutation of 1..E (argsort of uniform keys)
        keys = uniform_bits(stream_seed(seed, _S_PERM), 0, E)
        rank = np.empty(E, dtype=np.int64)
        rank[np.argsort(keys, kind="stable")] = np.arange(1, E + 1)
        w = rank.astype(np.float64) ** (-ZIPF_S)
        return (ZIPF_BETA * np.log(w / w.sum())).astype(np.float32)
    raise ValueError(cfg.router_bias)


def make_x(cfg: MoEConfig, seed: int, N: int | None = None) -> np.ndarray:
    N = cfg.N if N is None else N
    x = normal_f32(seed, _S_X, N * cfg.C).reshape(N, cfg.C)
    x = rmsnorm_f32(x)
    return bf16_round(x) if cfg.act == "bf16" else x


def make_router(cfg: MoEConfig, seed: int):
    Wr = normal_f32(seed, _S_WR, cfg.C * cfg.E, std=0.02).reshape(cfg.C, cfg.E)
    if cfg.act == "bf16":
        Wr = bf16_round(Wr)
    return Wr, router_bias(cfg, seed)


def make_expert(cfg: MoEConfig, seed: int, e: int, bias_std: float = 0.0):
    """Reference-layout fp32 parameters of expert e (values already on the
    bf16 grid for bf16 weights; fp8 quantisation is applied by the caller)."""
    C, H = cfg.C, cfg.H
    base = _S_EXPERT + 8 * e
    Wg = normal_f32(seed, base + 0, C * H, std=0.02).reshape(C, H)
    Wu = normal_f32(seed, base + 1, C * H, std=0.02).reshape(C, H)
    Wd = normal_f32(seed, base + 2, H * C, std=0.02).reshape(H, C)
    if bias_std > 0:
        bg = normal_f32(seed, base + 3, H, std=bias_std)
        bu = normal_f32(seed, base + 4, H, std=bias_std)
        bd = normal_f32(seed, base + 5, C, std=bias_std)
    else:
        bg = np.zeros(H, np.float32)
        bu = np.zeros(H, np.float32)
        bd = np.zeros(C, np.float32)
    if cfg.weights == "bf16":
        Wg, Wu, Wd = bf16_round(Wg), bf16_round(Wu), bf16_round(Wd)
        bg, bu, bd = bf16_round(bg), bf16_round(bu), bf16_round(bd)
    return Wg, bg, Wu, bu, Wd, bd


@dataclasses.dataclass
class MoEInputs:
    cfg: MoEConfig
    x: np.ndarray            # [N, C] float32
    Wr: np.ndarray           # [C, E]
    br: np.ndarray           # [E]
    Wg: np.ndarray           # [E, C, H] (dequantised values for fp8)
    bg: np.ndarray           # [E, H]
    Wu: np.ndarray
    bu: np.ndarray
    Wd: np.ndarray           # [E, H, C]
    bd: np.ndarray           # [E, C]
    # fp8 only: the unquantised fp32 weights the library is given (it
    # quantises them itself; Wg/Wu/Wd above hold the dequantised values)
    raw: tuple | None = None

    def params(self, raw: bool = False):
        """The 2+6E fp32 parameters in MoELayer::get_parameters() order
        (layers/MoELayer.cpp:225-236); raw=True gives the unquantised expert
        weights of an fp8 configuration."""
        Wg, Wu, Wd = self.raw if (raw and self.raw is not None) else (self.Wg, self.Wu, self.Wd)
        out = [self.Wr, self.br.reshape(1, -1)]
        for e in range(self.cfg.E):
            out += [Wg[e], self.bg[e].reshape(1, -1), Wu[e],
                    self.bu[e].reshape(1, -1), Wd[e], self.bd[e].reshape(1, -1)]
        return out


def make_inputs(cfg: MoEConfig, seed: int = 1234, N: int | None = None,
                bias_std: float = 0.0) -> MoEInputs:
    """Full inputs of a configuration (optionally with N tokens instead of
    cfg.N, and with nonzero expert biases for the unit tests).  For fp8
    weights the returned expert weights are the dequantised e4m3 values
    (q * per-output-channel scale), which is what the fp8 kernels compute
    with and what the reference CPU path is fed."""
    if N is not None:
        cfg = dataclasses.replace(cfg, N=N)
    x = make_x(cfg, seed)
    Wr, br = make_router(cfg, seed)
    E, C, H = cfg.E, cfg.C, cfg.H
    Wg = np.empty((E, C, H), np.float32)
    Wu = np.empty((E, C, H), np.float32)
    Wd = np.empty((E, H, C), np.float32)
    bg = np.empty((E, H), np.float32)
    bu = np.empty((E, H), np.float32)
    bd = np.empty((E, C), np.float32)
    raw = None
    if cfg.weights == "fp8":
        raw = (np.empty((E, C, H), np.float32), np.empty((E, C, H), np.float32),
               np.empty((E, H, C), np.float32))
    for e in range(E):
        g, bgv, u, buv, d, bdv = make_expert(cfg, seed, e, bias_std)
        if cfg.weights == "fp8":
            raw[0][e], raw[1][e], raw[2][e] = g, u, d
            g = quantize_e4m3_per_out_channel(g)[2]
            u = quantize_e4m3_per_out_channel(u)[2]
            d = quantize_e4m3_per_out_channel(d)[2]
        Wg[e], Wu[e], Wd[e], bg[e], bu[e], bd[e] = g, u, d, bgv, buv, bdv
    return MoEInputs(cfg, x, Wr, br, Wg, bg, Wu, bu, Wd, bd, raw)


def small_config(name: str, N: int, C: int, E: int, k: int, H: int,
                 act: str = "f32", weights: str | None = None,
                 router_bias_kind: str = "zero") -> MoEConfig:
    return MoEConfig(name, N, C, E, k, H, act, weights or act, router_bias_kind)


def digest(a: np.ndarray) -> str:
    """SHA-256 (first 16 hex digits) of an array's little-endian bytes."""
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]
