"""GPU: a MoE block loaded straight from a GPT checkpoint written by the
reference's GPT::save_weights_bin (mgpt_moe_load_gpt_bin) computes what the
reference computes with that block's parameters.

Expected values are the CPU oracle's forward / fused block (pinned to the
reference in test_oracle.py and test_oracle_block.py) on the parameters
that mgpt_gpt_bin_read_block returns, which test_gptbin.py pins to the
reference's live layers.  Routing bit for bit; outputs at the forward's bars
(1e-5 fp32, 2e-2 bf16).
"""
import numpy as np
import pytest

import cases as C
import gptbin_case as G
import oracle_lib as O
from mgpt_amd import capi, checkpoint

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

g = C.GPTBIN
TOL = {"f32": 1e-5, "bf16": 2e-2}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    capi.lib()
    return torch.device("cuda", 0)


def errors(got, ref):
    d = np.asarray(got, np.float64) - np.asarray(ref, np.float64)
    r = np.asarray(ref, np.float64)
    return (np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30),
            np.abs(d).max() / max(np.abs(r).max(), 1e-30))


def layer_from_bin(path, layer, act):
    from mgpt_amd.moe import MoELayer
    m = MoELayer(g["C"], g["H"], g["E"], g["k"], act=act)
    gamma = m.load_gpt_bin(path, layer)
    return m, gamma


@pytest.mark.parametrize("act", ["f32", "bf16"])
@pytest.mark.parametrize("layer", [0, 1])
def test_forward_from_checkpoint(tmp_path, layer, act):
    print(f"checkpoint block {layer}, act {act}", flush=True)
    path = G.write_bin(tmp_path)
    m, gamma = layer_from_bin(path, layer, act)
    gamma_ref, params = checkpoint.read_block(path, g["E"], g["H"], layer)
    assert np.array_equal(gamma.numpy(), gamma_ref)
    inp = G.block_inputs(params, 300, act)
    dt = torch.float32 if act == "f32" else torch.bfloat16
    y = m.forward(torch.from_numpy(inp.x).to("cuda").to(dt))
    torch.cuda.synchronize()
    r = {k: v.cpu().numpy() for k, v in m.routing().items()}
    ref = O.forward(inp)
    assert np.array_equal(r["topk_idx"], ref["idx"])
    assert np.array_equal(r["counts"], ref["counts"])
    rel, mx = errors(y.float().cpu().numpy(), ref["y"])
    print(f"block {layer} {act}: normwise {rel:.3e} max/max {mx:.3e}", flush=True)
    assert rel <= TOL[act] and mx <= TOL[act]


def test_fused_block_from_checkpoint(tmp_path):
    """The block's ln2 scale from the file feeds mgpt_moe_forward_block."""
    path = G.write_bin(tmp_path, legacy=True)
    m, gamma = layer_from_bin(path, 1, "f32")
    _, params = checkpoint.read_block(path, g["E"], g["H"], 1)
    inp = G.block_inputs(params, 200, "f32", seed=9)
    x1 = (inp.x * np.float32(1.5) + np.float32(0.25)).astype(np.float32)
    out = m.forward_block(torch.from_numpy(x1).to("cuda"), gamma.to("cuda"), 1e-5)
    torch.cuda.synchronize()
    ref = O.block(inp, x1, gamma.numpy(), 1e-5)
    r = {k: v.cpu().numpy() for k, v in m.routing().items()}
    assert np.array_equal(r["topk_idx"], ref["idx"])
    assert np.array_equal(m.rstd().cpu().numpy().view(np.uint32), ref["rstd"].view(np.uint32))
    rel, mx = errors(out.cpu().numpy(), ref["out"])
    assert rel <= 1e-5 and mx <= 1e-5


def test_checkpoint_of_another_width_is_rejected(tmp_path):
    from mgpt_amd.moe import MoELayer
    path = G.write_bin(tmp_path)
    m = MoELayer(2 * g["C"], g["H"], g["E"], g["k"], act="f32")
    with pytest.raises(capi.MoEError) as ei:
        m.load_gpt_bin(path, 0)
    assert ei.value.status == capi.MGPT_ERR_INVALID_ARGUMENT
