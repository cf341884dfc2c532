"""CPU checks of the C ABI library: it loads, exports every function
include/mgpt_moe.h declares, and rejects bad configurations before touching
a GPU.  No compute call is made here (there is no GPU in this container)."""
import ctypes
import os
import subprocess

import pytest

from mgpt_amd import capi


def test_header_declares_the_boundary():
    names = capi.declared_functions()
    for required in ("mgpt_moe_create", "mgpt_moe_destroy", "mgpt_moe_load_parameters",
                     "mgpt_moe_workspace_bytes", "mgpt_moe_forward", "mgpt_moe_get_routing",
                     "mgpt_moe_expert_counts", "mgpt_moe_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    L = capi.lib()
    for name in capi.declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(capi.declared_functions()) <= exported
    # only the C ABI (plus runtime glue) is exported with C names
    assert not [s for s in exported if s.startswith("mgpt_") and s not in
                set(capi.declared_functions())]


def test_library_targets_gfx950():
    # the embedded device code object is built for gfx950 (and only for it)
    blob = open(capi.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"amdgcn-amd-amdhsa--gfx942" not in blob


def _create(C, H, E, k, act=capi.DTYPE_F32, w=capi.DTYPE_F32):
    cfg = capi.Config(C, H, E, k, act, w)
    h = ctypes.c_void_p()
    st = capi.lib().mgpt_moe_create(ctypes.byref(cfg), ctypes.byref(h))
    return st, h


@pytest.mark.parametrize("shape,expect", [
    ((64, 64, 4, 5), capi.MGPT_ERR_INVALID_ARGUMENT),    # k > E
    ((64, 64, 513, 2), capi.MGPT_ERR_UNSUPPORTED),       # E > 512
    ((64, 64, 16, 9), capi.MGPT_ERR_UNSUPPORTED),        # k > 8
    ((0, 64, 4, 2), capi.MGPT_ERR_INVALID_ARGUMENT),
    ((64, -2, 4, 2), capi.MGPT_ERR_INVALID_ARGUMENT),
])
def test_bad_configs_rejected_without_gpu(shape, expect):
    st, h = _create(*shape)
    assert st == expect
    assert h.value is None
    assert capi.lib().mgpt_moe_last_error().decode()


def test_bad_dtype_pairs_rejected():
    # bf16 activations over fp32 weights is not a supported pair (fp32
    # activations over bf16 / fp8 weights are: the expert products then run
    # in bf16 behind fp32 tensors)
    st, _ = _create(64, 64, 4, 2, capi.DTYPE_BF16, capi.DTYPE_F32)
    assert st == capi.MGPT_ERR_UNSUPPORTED
    st, _ = _create(64, 64, 4, 2, capi.DTYPE_F32, 7)
    assert st == capi.MGPT_ERR_UNSUPPORTED


def test_null_arguments_rejected():
    L = capi.lib()
    n = ctypes.c_size_t()
    assert L.mgpt_moe_workspace_bytes(None, 10, ctypes.byref(n)) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert L.mgpt_moe_forward(None, None, None, 1, None, 0, None) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert L.mgpt_moe_create(None, None) == capi.MGPT_ERR_INVALID_ARGUMENT
    assert L.mgpt_moe_destroy(None) == capi.MGPT_OK
