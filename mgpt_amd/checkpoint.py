"""GPT checkpoint (.bin) reader over the C ABI, host only.

The engine's checkpoint is GPT::save_weights_bin's file
(/root/reference/src/main/neuralnetwork/GPT.cpp:128-155): an int32 header
(vocab_size, max_seq_len, embed_dim, num_layers[, completed_steps]) and
every parameter as float32 in GPT::get_parameters() order.  inspect() and
read_block() call mgpt_gpt_bin_inspect / mgpt_gpt_bin_read_block, which
locate one transformer block's ln2 scale and MoE parameters and read only
those bytes; MoELayer.load_gpt_bin loads them onto the GPU.  No device call.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import capi


def inspect(path: str, num_experts: int, hidden_dim: int) -> dict:
    """Header and size layout of a checkpoint for a GPT with num_experts
    experts of hidden size hidden_dim (-1: 4 * embed_dim)."""
    info = capi.GptBinInfo()
    capi.check(capi.lib().mgpt_gpt_bin_inspect(os.fsencode(path), int(num_experts),
                                               int(hidden_dim), ctypes.byref(info)))
    return {name: getattr(info, name) for name, _ in capi.GptBinInfo._fields_}


def read_block(path: str, num_experts: int, hidden_dim: int, layer: int):
    """(ln2 scale [C], the 2 + 6E MoE parameters in get_parameters() order
    and reference shapes: W_r [C,E], b_r [1,E], then per expert W_gate [C,H],
    b_gate [1,H], W_up [C,H], b_up [1,H], W_down [H,C], b_down [1,C])."""
    info = inspect(path, num_experts, hidden_dim)
    C, E = info["embed_dim"], int(num_experts)
    H = hidden_dim if hidden_dim > 0 else 4 * C
    gamma = np.empty(C, np.float32)
    flat = np.empty(info["moe_floats"], np.float32)
    capi.check(capi.lib().mgpt_gpt_bin_read_block(os.fsencode(path), E, int(hidden_dim),
                                                  int(layer), gamma.ctypes.data,
                                                  flat.ctypes.data, flat.size))
    shapes = [(C, E), (1, E)] + [(C, H), (1, H), (C, H), (1, H), (H, C), (1, C)] * E
    params, at = [], 0
    for shp in shapes:
        n = shp[0] * shp[1]
        params.append(flat[at:at + n].reshape(shp))
        at += n
    assert at == flat.size
    return gamma, params
