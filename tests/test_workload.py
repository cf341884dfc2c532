"""The seeded workload generator and the fp8/bf16 helpers.

The C twin of the generator must produce the same bits as the numpy version
(fixtures are regenerated from seeds on other hosts); the e4m3 quantiser of
the workload (used to feed the reference) must follow the OCP E4M3FN rounding
rule that the library's load-time quantiser implements (the GPU test
compares the two)."""
import numpy as np
import pytest

import oracle_lib as O
from mgpt_amd import workload as wl


@pytest.mark.parametrize("seed,stream,n,std", [(1234, 1, 100003, 1.0), (7, 105, 4096, 0.02),
                                               (2 ** 63 + 5, 3, 999, 1.0), (0, 0, 1, 1.0)])
def test_c_and_numpy_generators_agree(seed, stream, n, std):
    a = wl.normal_f32(seed, stream, n, std, use_c=False)
    b = wl.normal_f32(seed, stream, n, std)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_generator_is_counter_based_and_normal():
    z = wl.normal(99, 4, 20000)
    tail = wl.normal(99, 4, 5000, start=15000)
    assert np.array_equal(z[15000:], tail)
    big = wl.normal_f32(5, 5, 1 << 20)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01
    assert wl.stream_seed(1, 2) != wl.stream_seed(2, 1)


def test_polynomial_log_and_cos_accuracy():
    u = np.linspace(1e-300, 1, 200001)[1:]
    assert np.max(np.abs(wl._log(u) - np.log(u))) < 1e-13
    v = np.linspace(0, 1, 200001)[:-1]
    assert np.max(np.abs(wl._cos_2pi(v) - np.cos(2 * np.pi * v))) < 1e-14


def test_bf16_round_nearest_even():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -0.0,
                     np.inf, -np.inf, 3.3e38], np.float32)
    r = wl.bf16_round(vals)
    assert r[0] == 1.0 and r[1] == 1.0                    # tie -> even
    assert r[2] == np.float32(1.0 + 2 ** -6)               # tie -> even (up)
    assert r[3] == np.float32(1.0 + 2 ** -7)               # above the tie -> up
    assert np.signbit(r[4]) and np.isinf(r[5]) and np.isinf(r[6])
    assert np.isnan(wl.bf16_round(np.array([np.nan], np.float32)))[0]


def test_e4m3_table_and_round_trip():
    t = wl.e4m3_decode_table()
    assert t[0x7E] == 448 and t[0x08] == 2 ** -6 and t[0x01] == 2 ** -9
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    finite = [b for b in range(256) if not np.isnan(t[b]) and b != 0x80]
    codes = wl.e4m3_encode(t[finite])
    assert list(codes) == finite
    # midpoints between neighbours round to the even code; saturation at 448
    pos = t[:0x7F].astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    exact = mids.astype(np.float64) == (pos[:-1] + pos[1:]) / 2
    c = wl.e4m3_encode(mids)
    lo = np.arange(0x7E)
    expect = np.where(lo % 2 == 0, lo, lo + 1)
    assert np.array_equal(c[exact], expect[exact])
    assert list(wl.e4m3_encode(np.array([1000.0, -1000.0, 460.0], np.float32))) == [0x7E, 0xFE, 0x7E]


def test_c_and_numpy_quantisers_agree():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((300, 77)) * 0.02).astype(np.float32)
    w[:, 5] = 0.0
    w[7, 9] = 1e-12
    a = wl.quantize_e4m3_per_out_channel(w, use_c=False)
    b = wl.quantize_e4m3_per_out_channel(w)
    for x, y in zip(a, b):
        assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
    assert np.all(a[1][5] == 1.0)


def test_rmsnorm_matches_oracle_restatement():
    x = wl.normal_f32(11, 1, 257 * 192).reshape(257, 192)
    assert np.array_equal(wl.rmsnorm_f32(x).view(np.uint32), O.rmsnorm(x).view(np.uint32))


def test_config_shapes_match_the_benchmark_definition():
    c = wl.CONFIGS
    assert (c["cfg1"].N, c["cfg1"].C, c["cfg1"].E, c["cfg1"].k, c["cfg1"].H) == (1024, 128, 8, 2, 512)
    assert (c["cfg3"].N, c["cfg3"].C, c["cfg3"].E, c["cfg3"].k, c["cfg3"].H) == (16384, 1024, 16, 2, 2816)
    assert (c["cfg4"].N, c["cfg4"].C, c["cfg4"].E, c["cfg4"].k, c["cfg4"].H) == (32768, 2048, 64, 6, 1408)
    assert (c["cfg5"].N, c["cfg5"].C, c["cfg5"].E, c["cfg5"].k, c["cfg5"].H) == (64, 2048, 64, 8, 1408)
    assert c["cfg5"].weights == "fp8" and c["cfg1"].act == "f32"
