"""ctypes binding of the C ABI in include/mgpt_moe.h (libmgpt_moe.so).

This is the binding a host program in Python would add; the C++ engine
links the same library directly (mgpt_amd/host/MoELayer.cpp).  Loading fails
loudly if the HIP library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# MGPT_MOE_LIB: another build of the same library (e.g. one compiled with
# different tile constants, for measurement)
LIB_PATH = os.environ.get("MGPT_MOE_LIB") or os.path.join(HERE, "lib", "libmgpt_moe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "mgpt_moe.h")

MGPT_OK = 0
MGPT_ERR_INVALID_ARGUMENT = 1
MGPT_ERR_UNSUPPORTED = 2
MGPT_ERR_WORKSPACE_TOO_SMALL = 3
MGPT_ERR_NOT_READY = 4
MGPT_ERR_HIP = 5
MGPT_ERR_OUT_OF_MEMORY = 6

DTYPE_F32, DTYPE_BF16, DTYPE_FP8_E4M3 = 0, 1, 2
NUM_STAGES = 5
STAGE_NAMES = ["router_topk", "permute", "gemm_gateup", "gemm_down", "combine"]
NUM_BWD_STAGES = 7
BWD_STAGE_NAMES = ["scatter_bwd", "gemm_dact_swiglu_bwd", "gemm_dx", "wgrad_down",
                   "wgrad_gateup", "token_bwd", "router_wgrad"]


class Config(ctypes.Structure):
    _fields_ = [("embed_dim", ctypes.c_int), ("hidden_dim", ctypes.c_int),
                ("num_experts", ctypes.c_int), ("top_k", ctypes.c_int),
                ("act_dtype", ctypes.c_int), ("weight_dtype", ctypes.c_int)]


class Routing(ctypes.Structure):
    _fields_ = [("topk_idx", ctypes.c_void_p), ("topk_p", ctypes.c_void_p),
                ("counts", ctypes.c_void_p), ("perm", ctypes.c_void_p),
                ("slot_of", ctypes.c_void_p)]


class GptBinInfo(ctypes.Structure):
    _fields_ = [("vocab_size", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
                ("embed_dim", ctypes.c_int32), ("num_layers", ctypes.c_int32),
                ("completed_steps", ctypes.c_int32), ("header_ints", ctypes.c_int32),
                ("file_bytes", ctypes.c_int64), ("param_floats", ctypes.c_int64),
                ("block_floats", ctypes.c_int64), ("moe_floats", ctypes.c_int64)]


class MoEError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"mgpt_moe status {status}: {message}")
        self.status = status


_LIB = None


def declared_functions() -> list[str]:
    """Names of the functions declared in include/mgpt_moe.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(mgpt_\w+)\s*\(", text, re.M)))


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mgpt_amd.build` "
                           "(the MoE forward has no non-HIP implementation)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sig = {
        "mgpt_moe_create": [ctypes.POINTER(Config), ctypes.POINTER(vp)],
        "mgpt_moe_destroy": [vp],
        "mgpt_moe_load_parameters": [vp, ctypes.POINTER(vp), i, i, vp],
        "mgpt_moe_workspace_bytes": [vp, i, ctypes.POINTER(sz)],
        "mgpt_moe_forward": [vp, vp, vp, i, vp, sz, vp],
        "mgpt_moe_forward_noalloc": [vp, vp, vp, i, vp],
        "mgpt_moe_get_routing": [vp, i, vp, ctypes.POINTER(Routing)],
        "mgpt_moe_expert_counts": [vp, vp, i],
        "mgpt_moe_set_profiling": [vp, i],
        "mgpt_moe_stage_times": [vp, vp, i],
        "mgpt_moe_export_fp8": [vp, i, i, vp, vp],
        "mgpt_moe_device_expf": [vp, vp, i, vp],
        "mgpt_moe_train_workspace_bytes": [vp, i, ctypes.POINTER(sz)],
        "mgpt_moe_forward_train": [vp, vp, vp, i, vp, sz, vp],
        "mgpt_moe_backward": [vp, vp, vp, vp, i, vp, sz, vp],
        "mgpt_moe_zero_grad": [vp, vp],
        "mgpt_moe_get_gradients": [vp, ctypes.POINTER(vp), i, i, vp],
        "mgpt_moe_accumulate_gradients": [vp, ctypes.POINTER(vp), i, i, vp],
        "mgpt_moe_backward_stage_times": [vp, vp, i],
        "mgpt_moe_forward_block": [vp, vp, vp, ctypes.c_float, vp, i, vp, sz, vp],
        "mgpt_moe_get_rstd": [vp, i, vp, ctypes.POINTER(vp)],
        "mgpt_moe_forward_block_train": [vp, vp, vp, ctypes.c_float, vp, i, vp, sz, vp],
        "mgpt_moe_backward_block": [vp, vp, vp, vp, vp, vp, i, vp, sz, vp],
        "mgpt_gpt_bin_inspect": [ctypes.c_char_p, i, i, ctypes.POINTER(GptBinInfo)],
        "mgpt_gpt_bin_read_block": [ctypes.c_char_p, i, i, i, vp, vp, sz],
        "mgpt_moe_load_gpt_bin": [vp, ctypes.c_char_p, i, vp, vp],
    }
    for name, args in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = ctypes.c_int
    L.mgpt_moe_last_error.argtypes = []
    L.mgpt_moe_last_error.restype = ctypes.c_char_p
    _LIB = L
    return L


def check(status: int) -> None:
    if status != MGPT_OK:
        raise MoEError(status, lib().mgpt_moe_last_error().decode())
