"""The router's correctly rounded square root (router.hip: sqrt_rn), pinned on
the CPU.

sqrt_rn takes the hardware estimate s (within an ulp of sqrt(y), not always
the nearest float) and moves it to a neighbour when the exact residual
y - s_-*s (or y - s_+*s) says the nearest float lies there; each residual
is one fused multiply-add on the GPU, so only its sign is used.  Here the
same decision is restated with float64 arithmetic, where s_-*s is exact (two
24-bit significands) and y - s_-*s keeps its sign, and fed every estimate the
hardware may return (the nearest float and both neighbours) for inputs
across the normalisation's range; the result must be the host's correctly
rounded sqrtf in every case.  A planted mistake (testing against s instead of
its neighbour) must fail.
"""
import numpy as np


def _neighbours(s):
    b = s.view(np.uint32)
    return (b - 1).view(np.float32), (b + 1).view(np.float32)


def sqrt_rn(y, s, plant=False):
    """Restatement of sqrt_rn's correction for float32 arrays y > 0 and
    estimates s."""
    sd, su = _neighbours(s)
    y64, s64 = y.astype(np.float64), s.astype(np.float64)
    lo = sd.astype(np.float64) if not plant else s64
    down = (y64 - lo * s64) <= 0.0
    up = (y64 - su.astype(np.float64) * s64) > 0.0
    return np.where(down, sd, np.where(up, su, s))


def _inputs():
    rng = np.random.default_rng(7)
    # the range 1/rms meets: eps = 1e-5 up to large mean squares, plus
    # powers of two and their neighbours (binade edges) and exact squares
    y = np.exp2(rng.uniform(-17.0, 40.0, 400_000)).astype(np.float32)
    p2 = np.exp2(np.arange(-17, 41, dtype=np.float32))
    b = p2.view(np.uint32)
    edges = np.concatenate([p2, (b - 1).view(np.float32), (b + 1).view(np.float32)])
    squares = (np.arange(1, 4097, dtype=np.float32) ** 2).astype(np.float32)
    return np.concatenate([y, edges, squares, squares / np.float32(1024.0)])


def test_every_estimate_is_corrected_to_the_nearest():
    y = _inputs()
    ref = np.sqrt(y)                       # correctly rounded (IEEE)
    rd, ru = _neighbours(ref)
    for est in (ref, rd, ru):
        got = sqrt_rn(y, est)
        bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))[0]
        assert bad.size == 0, (bad[:5], y[bad[:5]])


def test_planted_mistake_is_detected():
    y = _inputs()
    ref = np.sqrt(y)
    got = sqrt_rn(y, ref, plant=True)
    assert np.any(got.view(np.uint32) != ref.view(np.uint32))
