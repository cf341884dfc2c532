"""The GPT checkpoint (.bin) weight path on the host: mgpt_gpt_bin_inspect and
mgpt_gpt_bin_read_block against a checkpoint written by the reference's own
GPT::save_weights_bin (nn/GPT.cpp:128-155; tests/golden/gptbin/small.npz).

The fixture's digests were taken from the reference's live layers
(blocks[l]->ln2 and blocks[l]->mlp.get_parameters()), not from file offsets,
so matching them pins the block location computed from the header.  The
4-int header of older files follows GPT::load_weights_bin's rule
(nn/GPT.cpp:187-190); files of any other size, a wrong expert count or
hidden size, and layers out of range are rejected.  Host code only.
"""
import numpy as np
import pytest

import cases as C
import gptbin_case as G
from mgpt_amd import capi, checkpoint
from mgpt_amd import workload as wl

g = C.GPTBIN


def test_header_and_sizes(tmp_path):
    info = checkpoint.inspect(G.write_bin(tmp_path), g["E"], g["H"])
    assert (info["vocab_size"], info["max_seq_len"], info["embed_dim"], info["num_layers"]) == \
        (g["V"], g["S"], g["C"], g["L"])
    assert info["header_ints"] == 5 and info["completed_steps"] == g["steps"]
    assert info["file_bytes"] == 20 + 4 * info["param_floats"]
    Cc, V, E, H = g["C"], g["V"], g["E"], g["H"]
    moe = Cc * E + E + E * (2 * (Cc * H + H) + H * Cc + Cc)
    assert info["moe_floats"] == moe
    assert info["block_floats"] == 2 * Cc + 4 * Cc * Cc + 4 * Cc + moe
    assert info["param_floats"] == V * Cc + g["L"] * info["block_floats"] + 2 * Cc + Cc * V + V


@pytest.mark.parametrize("legacy", [False, True])
def test_blocks_match_the_reference_layers(tmp_path, legacy):
    fx = G.fixture()
    path = G.write_bin(tmp_path, legacy=legacy)
    info = checkpoint.inspect(path, g["E"], g["H"])
    assert info["header_ints"] == (4 if legacy else 5)
    assert info["completed_steps"] == (0 if legacy else g["steps"])
    for layer in range(g["L"]):
        gamma, params = checkpoint.read_block(path, g["E"], g["H"], layer)
        assert wl.digest(gamma) == str(fx[f"sha_ln2_{layer}"]), layer
        flat = np.concatenate([p.reshape(-1) for p in params])
        assert wl.digest(flat) == str(fx[f"sha_moe_{layer}"]), layer
        # ln2 scales are 1 + small values, MoE parameters centred on 0
        assert abs(float(gamma.mean()) - 1.0) < 0.1
        assert abs(float(params[0].mean())) < 0.1


def test_blocks_differ(tmp_path):
    path = G.write_bin(tmp_path)
    _, p0 = checkpoint.read_block(path, g["E"], g["H"], 0)
    _, p1 = checkpoint.read_block(path, g["E"], g["H"], 1)
    assert not np.array_equal(p0[0], p1[0])


def _status(fn):
    with pytest.raises(capi.MoEError) as ei:
        fn()
    return ei.value.status


def test_rejects_wrong_sizes_and_layers(tmp_path):
    path = G.write_bin(tmp_path)
    bad = capi.MGPT_ERR_INVALID_ARGUMENT
    assert _status(lambda: checkpoint.inspect(path, g["E"] + 1, g["H"])) == bad
    assert _status(lambda: checkpoint.inspect(path, g["E"] - 1, g["H"])) == bad
    assert _status(lambda: checkpoint.inspect(path, g["E"], -1)) == bad   # 4C != H
    assert _status(lambda: checkpoint.read_block(path, g["E"], g["H"], g["L"])) == bad
    assert _status(lambda: checkpoint.read_block(path, g["E"], g["H"], -1)) == bad
    cut = G.write_bin(tmp_path, cut=4)   # one float short of a 5-int file: read as 4-int
    assert checkpoint.inspect(cut, g["E"], g["H"])["header_ints"] == 4
    short = G.write_bin(tmp_path, cut=8)
    assert _status(lambda: checkpoint.inspect(short, g["E"], g["H"])) == bad
    assert _status(lambda: checkpoint.inspect(str(tmp_path / "missing.bin"), 4, 64)) == bad
    assert "missing.bin" in capi.lib().mgpt_moe_last_error().decode()
