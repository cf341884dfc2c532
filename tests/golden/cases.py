"""Input cases shared by the golden-fixture generator and the tests.

Each case is rebuilt from (config, seed, tweaks) with the seeded generator in
mgpt_amd.workload, so a committed fixture holds only the reference's
outputs.  The unit cases cover the edge cases of the routing rules in
/root/reference/src/main/utils/Tensor.cpp: exact ties (:1296-1334, lower
expert id first), clamped probabilities (:879), NaN/Inf inputs (F16: every
p = 1e-7 so experts 0..k-1 win), ragged token counts, k = 1 and k = E, one
expert, and nonzero biases everywhere (the benchmark configurations use zero
expert biases, which would hide a dropped bias term).
"""
from __future__ import annotations

import dataclasses

import numpy as np

from mgpt_amd import workload as wl

SEED = 20261201


@dataclasses.dataclass(frozen=True)
class Case:
    name: str
    cfg: wl.MoEConfig
    bias_std: float = 0.0
    tweak: str = ""           # "ones", "tie_router", "nan_rows", "wide_router"
    gpu: bool = True          # run on the HIP path too (every case is)
    full_arrays: bool = True  # store full routing arrays (small cases)


def _c(name, N, C, E, k, H, act="f32", weights=None, rb="zero"):
    return wl.MoEConfig(name, N, C, E, k, H, act, weights or act, rb)


UNIT_CASES = [
    # the shape of the reference's own MoE test (tests/networkTest/moeTests.cpp:6-19):
    # B=2, T=4, C=16, E=4, k=2, hidden 4C, input all ones -> every token ties;
    # on the GPU C = 16 runs through the library's zero-padded width
    Case("moetests_shape", _c("moetests_shape", 8, 16, 4, 2, 64), 0.0, "ones"),
    Case("ties_ones", _c("ties_ones", 16, 64, 4, 2, 64), 0.1, "tie_router"),
    Case("small_f32", _c("small_f32", 64, 64, 4, 2, 96, rb="normal"), 0.1),
    Case("ragged_k3", _c("ragged_k3", 37, 64, 6, 3, 80, rb="normal"), 0.05),
    Case("k8_bf16", _c("k8_bf16", 50, 128, 16, 8, 64, "bf16", rb="zipf"), 0.02),
    Case("nan_rows", _c("nan_rows", 16, 64, 8, 2, 64), 0.05, "nan_rows"),
    Case("clamp_ties", _c("clamp_ties", 32, 64, 8, 3, 64), 0.05, "wide_router"),
    Case("single_expert", _c("single_expert", 20, 64, 1, 1, 64), 0.05),
    Case("k_equals_e", _c("k_equals_e", 24, 64, 4, 4, 64, rb="normal"), 0.05),
    Case("bf16_e64_k6", _c("bf16_e64_k6", 96, 128, 64, 6, 128, "bf16", rb="zipf"), 0.02),
    Case("fp8_small", _c("fp8_small", 48, 128, 8, 4, 192, "bf16", "fp8", rb="normal"), 0.02),
    # enough rows per expert for the large-M (256/128-row tile) GEMM path,
    # with a ragged last tile in every expert
    Case("bf16_large_m", _c("bf16_large_m", 1100, 192, 4, 2, 320, "bf16", rb="zipf"), 0.02),
    Case("fp8_large_m", _c("fp8_large_m", 900, 256, 4, 2, 256, "bf16", "fp8", rb="normal"), 0.02),
]

# More experts than a wave has lanes (E > 64): the wide paths (split router
# with the wide softmax, wave-chunked permute scan, generic grouped GEMMs,
# the backward's wide token and router gradients, one weight-gradient item
# per expert).
WIDE_CASES = [
    Case("wide_e128_k8", _c("wide_e128_k8", 96, 128, 128, 8, 64, "bf16", rb="zipf"), 0.02),
    Case("wide_e256_f32", _c("wide_e256_f32", 80, 64, 256, 4, 48, rb="normal"), 0.05),
    Case("wide_e96_large", _c("wide_e96_large", 3000, 128, 96, 6, 96, "bf16"), 0.02,
         full_arrays=False),
    Case("wide_e200_fp8", _c("wide_e200_fp8", 40, 128, 200, 8, 128, "bf16", "fp8", rb="normal"),
         0.02),
    Case("wide_e384_k8", _c("wide_e384_k8", 128, 64, 384, 8, 32, "bf16", rb="zero"), 0.02),
]

CONFIG_CASES = [
    Case("cfg1", wl.CONFIGS["cfg1"], full_arrays=True),
    Case("cfg2", wl.CONFIGS["cfg2"], full_arrays=False),
    Case("cfg3", wl.CONFIGS["cfg3"], full_arrays=False),
    Case("cfg4", wl.CONFIGS["cfg4"], full_arrays=False),
    Case("cfg5", wl.CONFIGS["cfg5"], full_arrays=True),
]

ALL_CASES = {c.name: c for c in UNIT_CASES + WIDE_CASES + CONFIG_CASES}


def build_inputs(case: Case) -> wl.MoEInputs:
    inp = wl.make_inputs(case.cfg, SEED, bias_std=case.bias_std)
    if case.tweak == "ones":
        inp.x[:] = 1.0
    elif case.tweak == "tie_router":
        # identical router columns: every logit of a token ties exactly
        inp.Wr[:] = inp.Wr[:, :1]
        inp.br[:] = 0.0
    elif case.tweak == "nan_rows":
        inp.x[3, :] = np.nan
        inp.x[5, 2] = np.nan
        inp.x[9, 0] = np.inf
        inp.x[11, 7] = -np.inf
    elif case.tweak == "wide_router":
        # large logit gaps: most probabilities clamp to exactly 1e-7 (and the
        # winner to 1), so lower-index tie-breaks among the losers decide
        # the second and third choices
        inp.Wr[:] = inp.Wr * np.float32(100.0)
    if case.cfg.act == "bf16":
        inp.x[:] = wl.bf16_round(inp.x)
        inp.Wr[:] = wl.bf16_round(inp.Wr)
    return inp


# Cases whose backward the reference is run on (tests/golden/backward/):
# every unit case plus two benchmark shapes whose expert gradients still
# fit a CPU run of a few seconds.
BACKWARD_CASES = [c.name for c in UNIT_CASES] + ["wide_e128_k8", "wide_e256_f32", "wide_e384_k8",
                                                  "cfg1", "cfg2"]


def build_dy(case: Case) -> np.ndarray:
    """Upstream gradient dy [N,C] of a case (standard normal, seeded; bf16
    values for bf16 cases so the HIP path reads it exactly).  The all-ones
    case takes dout = 1 like the reference's own backward test
    (tests/networkTest/moeTests.cpp:22-39)."""
    if case.tweak == "ones":
        return np.ones((case.cfg.N, case.cfg.C), np.float32)
    rng = np.random.default_rng([SEED, 11])
    dy = rng.standard_normal((case.cfg.N, case.cfg.C)).astype(np.float32)
    if case.cfg.act == "bf16":
        dy = wl.bf16_round(dy)
    return dy


# Cases of the training sequence (tests/golden/train/): the Trainer's step
# (zero grads, forward, backward with dy = build_dy(case), AdamW step,
# pipeline/Trainer.cpp:303-386) TRAIN_STEPS times, then a forward, with the
# engine's AdamWOptimizer at learning rate TRAIN_LR (other hyper-parameters
# at their defaults, optimisers/AdamWOptimiser.h:20-22).
TRAIN_CASES = ["moetests_shape", "small_f32", "ragged_k3"]
TRAIN_STEPS = 2
TRAIN_LR = 1e-3


# Cases of the fused block (tests/golden/block/): out = x1 + MoE(RMSNorm(x1)*gamma).
BLOCK_CASES = ["small_f32", "ragged_k3", "k8_bf16", "bf16_large_m", "fp8_small", "cfg1", "cfg3",
               "cfg5"]
BLOCK_EPS = 1e-5   # the engine's RMSNormLayer default (layers/RMSNormLayer.h:23)
# Cases of the fused block's backward (tests/golden/block_backward/): the
# trainable block cases (weights in the activation dtype), dout = build_dy.
BLOCK_BACKWARD_CASES = ["small_f32", "ragged_k3", "k8_bf16", "bf16_large_m", "cfg1"]


def build_block_inputs(case: Case):
    """(x1, gamma) of a fused-block case: the case's unit-RMS rows scaled per
    token by 2^(t%5 - 2) * (1 + (t%3)/4), i.e. 0.25 .. 6 (so the
    normalisation matters), plus a small offset, and gamma = 1 + 0.2 N(0,1)
    from the portable generator.  Only float32 arithmetic on exactly
    generated values, so every host builds the same bits (no libm)."""
    inp = build_inputs(case)
    N, Cc = inp.x.shape
    t = np.arange(N)
    scale = (np.exp2((t % 5 - 2).astype(np.float32)) *
             (np.float32(1.0) + (t % 3).astype(np.float32) / np.float32(4.0)))
    x1 = (inp.x * scale[:, None].astype(np.float32) + np.float32(0.05)).astype(np.float32)
    gamma = (np.float32(1.0) + wl.normal_f32(SEED, 4013, Cc, std=0.2)).astype(np.float32)
    if case.cfg.act == "bf16":
        x1 = wl.bf16_round(x1)
    return inp, x1, gamma


def sample_flat(n: int, m: int = 256) -> np.ndarray:
    """Deterministic sample of flat indices of an n-element gradient."""
    if n <= m:
        return np.arange(n, dtype=np.int64)
    return np.unique(np.linspace(0, n - 1, m).round().astype(np.int64))


def sample_rows(N: int, n: int = 32) -> np.ndarray:
    """Deterministic sample of token rows whose outputs fixtures store."""
    if N <= n:
        return np.arange(N, dtype=np.int32)
    return np.unique(np.linspace(0, N - 1, n).round().astype(np.int32))


# A small MoE GPT checkpoint written by the reference's GPT::save_weights_bin
# (tests/golden/gptbin/small.npz): vocab V, max_seq_len S, embed_dim C,
# L blocks, heads, E experts, top-k, hidden H, completed_steps, seed.
GPTBIN = {"V": 16, "S": 32, "C": 64, "L": 2, "heads": 2, "E": 4, "k": 2, "H": 64,
          "steps": 7, "seed": 20261202}


def gptbin_ids() -> np.ndarray:
    """Token ids of the checkpoint's GPT forward: 24 tokens < V."""
    return ((7 * np.arange(24) + 3) % GPTBIN["V"]).astype(np.int32)

