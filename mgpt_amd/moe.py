"""MoELayer: Python mirror of the reference's C++ layer API over the C ABI.

Mirrors /root/reference/src/main/neuralnetwork/layers/MoELayer.h:9-51 --
constructor (embed_dim, hidden_dim (-1 -> 4C), num_experts, top_k),
forward / forward_into on [B, T, C] activations, get_parameters() order for
loading, get_expert_counts(), get_footprint() -- for Python callers, tests
and the benchmark.  Activations are torch tensors on the GPU (torch supplies
device memory and the stream, nothing else); all compute runs in
libmgpt_moe.so.  There is no CPU path: a CPU tensor is rejected.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import capi

_ACT = {"f32": capi.DTYPE_F32, "bf16": capi.DTYPE_BF16}
_W = {"f32": capi.DTYPE_F32, "bf16": capi.DTYPE_BF16, "fp8": capi.DTYPE_FP8_E4M3}
_TORCH = {"f32": torch.float32, "bf16": torch.bfloat16}


class MoELayer:
    def __init__(self, embed_dim: int, hidden_dim: int, num_experts: int, top_k: int,
                 act: str = "bf16", weights: str | None = None):
        weights = weights or act
        self.C = embed_dim
        self.H = 4 * embed_dim if hidden_dim == -1 else hidden_dim
        self.E = num_experts
        self.k = top_k
        self.act = act
        self.weights = weights
        self.dtype = _TORCH[act]
        cfg = capi.Config(embed_dim, hidden_dim, num_experts, top_k, _ACT[act], _W[weights])
        h = ctypes.c_void_p()
        capi.check(capi.lib().mgpt_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self._ws = None
        self._last_n = None
        self._loaded = False

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            capi.lib().mgpt_moe_destroy(h)
            self._h = None

    # ---------------------------------------------------------------- params
    def load_parameters(self, params) -> None:
        """params: the 2+6E fp32 tensors in MoELayer::get_parameters() order
        (numpy arrays -> host pointers; CUDA tensors -> device pointers)."""
        if len(params) != 2 + 6 * self.E:
            raise ValueError(f"expected {2 + 6 * self.E} parameters, got {len(params)}")
        keep = []
        on_device = None
        for p in params:
            if isinstance(p, torch.Tensor):
                p = p.detach().to(torch.float32).contiguous()
                dev = p.is_cuda
            else:
                p = np.ascontiguousarray(p, dtype=np.float32)
                dev = False
            if on_device is None:
                on_device = dev
            elif on_device != dev:
                raise ValueError("parameters must be all host or all device")
            keep.append(p)
        ptrs = (ctypes.c_void_p * len(keep))(
            *[(p.data_ptr() if isinstance(p, torch.Tensor) else p.ctypes.data) for p in keep])
        stream = torch.cuda.current_stream().cuda_stream
        capi.check(capi.lib().mgpt_moe_load_parameters(self._h, ptrs, len(keep),
                                                        int(bool(on_device)), stream))
        self._loaded = True

    # --------------------------------------------------------------- forward
    def workspace_bytes(self, num_tokens: int) -> int:
        n = ctypes.c_size_t()
        capi.check(capi.lib().mgpt_moe_workspace_bytes(self._h, num_tokens, ctypes.byref(n)))
        return n.value

    def get_footprint(self, B: int, T: int) -> int:
        """Forward workspace in bytes for a [B, T, C] input (the C ABI's
        replacement for MoELayer::get_footprint, layers/MoELayer.cpp:238-251)."""
        return self.workspace_bytes(B * T)

    def _workspace(self, n: int, device) -> torch.Tensor:
        need = self.workspace_bytes(n)
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = torch.empty(max(need, 256), dtype=torch.uint8, device=device)
        return self._ws

    def forward_into(self, x: torch.Tensor, out: torch.Tensor) -> None:
        if not x.is_cuda or not out.is_cuda:
            raise ValueError("MoELayer runs on the GPU only: x and out must be device tensors")
        if x.dtype != self.dtype or out.dtype != self.dtype:
            raise TypeError(f"expected {self.dtype} activations")
        if x.shape[-1] != self.C or out.shape != x.shape:
            raise ValueError("shape mismatch")
        if not x.is_contiguous() or not out.is_contiguous():
            raise ValueError("x and out must be contiguous")
        n = x.numel() // self.C
        ws = self._workspace(n, x.device)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        capi.check(capi.lib().mgpt_moe_forward(self._h, x.data_ptr(), out.data_ptr(), n,
                                               ws.data_ptr(), ws.numel(), stream))
        self._last_n = n

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(x)
        self.forward_into(x, out)
        return out

    # --------------------------------------------------------------- routing
    def routing(self) -> dict:
        """Device views (torch tensors) of the last forward's routing:
        topk_idx [N,k] int32, topk_p [N,k] f32, counts [E], perm [N*k],
        slot_of [N*k]."""
        if self._last_n is None:
            raise RuntimeError("no forward has been run")
        n = self._last_n
        r = capi.Routing()
        capi.check(capi.lib().mgpt_moe_get_routing(self._h, n, self._ws.data_ptr(),
                                                   ctypes.byref(r)))
        base = self._ws.data_ptr()

        def view(ptr, count, dtype):
            off = ptr - base
            nbytes = count * 4
            return self._ws[off:off + nbytes].view(dtype)

        A = n * self.k
        return {
            "topk_idx": view(r.topk_idx, A, torch.int32).view(n, self.k),
            "topk_p": view(r.topk_p, A, torch.float32).view(n, self.k),
            "counts": view(r.counts, self.E, torch.int32),
            "perm": view(r.perm, A, torch.int32),
            "slot_of": view(r.slot_of, A, torch.int32),
        }

    def get_expert_counts(self) -> list:
        """Per-expert token counts of the last forward, as floats like the
        reference's get_expert_counts() (layers/MoELayer.h:39)."""
        c = np.zeros(self.E, dtype=np.int32)
        capi.check(capi.lib().mgpt_moe_expert_counts(self._h, c.ctypes.data, self.E))
        return [float(v) for v in c]

    # ----------------------------------------------------------- measurement
    def set_profiling(self, on: bool) -> None:
        capi.check(capi.lib().mgpt_moe_set_profiling(self._h, int(on)))

    def stage_times(self) -> dict:
        """Mean stage durations (ms) over the profiled forwards since
        set_profiling(True) (at most the last 64), plus their count."""
        ms = np.zeros(capi.NUM_STAGES + 1, dtype=np.float32)
        capi.check(capi.lib().mgpt_moe_stage_times(self._h, ms.ctypes.data, capi.NUM_STAGES + 1))
        out = dict(zip(capi.STAGE_NAMES, ms[:capi.NUM_STAGES].tolist()))
        out["forwards"] = int(ms[capi.NUM_STAGES])
        return out

    def export_fp8(self, expert: int, which: int):
        rows, cols = (self.C, self.H) if which < 2 else (self.H, self.C)
        q = np.zeros((rows, cols), np.uint8)
        s = np.zeros(cols, np.float32)
        capi.check(capi.lib().mgpt_moe_export_fp8(self._h, expert, which, q.ctypes.data,
                                                  s.ctypes.data))
        return q, s
