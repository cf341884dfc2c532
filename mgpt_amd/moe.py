"""MoELayer: Python mirror of the reference's C++ layer API over the C ABI.

Mirrors /root/reference/src/main/neuralnetwork/layers/MoELayer.h:9-51 --
constructor (embed_dim, hidden_dim (-1 -> 4C), num_experts, top_k),
forward / forward_into on [B, T, C] activations, backward / backward_into
(with the parameter gradients accumulated like Tensor::add_grad and read
back in get_parameters() order), get_parameters() order for loading,
get_expert_counts(), get_footprint() -- for Python callers, tests and the
benchmark.  Activations are torch tensors on the GPU (torch supplies
device memory and the stream, nothing else); all compute runs in
libmgpt_moe.so.  There is no CPU path: a CPU tensor is rejected.
"""
from __future__ import annotations

import ctypes
import os

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
        self._train_x = None   # input of the last training forward (cached_input)
        self._train_block = None   # (x, gamma) of the last training forward_block

    def __del__(self):
        h = getattr(self, "_h", None)
        # at interpreter exit the module's globals may already be gone; the
        # process then releases the device memory itself
        lib = getattr(capi, "lib", None) if capi is not None else None
        if h is not None and h.value and lib is not None:
            lib().mgpt_moe_destroy(h)
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

    def load_gpt_bin(self, path: str, layer: int) -> torch.Tensor:
        """Loads block `layer`'s MoE parameters from a GPT checkpoint written
        by GPT::save_weights_bin (nn/GPT.cpp:128-155), reading only that
        block's bytes, and packs them as load_parameters does.  Returns the
        block's ln2 scale (float32 [C], host) for forward_block."""
        gamma = np.empty(self.C, np.float32)
        stream = torch.cuda.current_stream().cuda_stream
        capi.check(capi.lib().mgpt_moe_load_gpt_bin(self._h, os.fsencode(path), int(layer),
                                                     gamma.ctypes.data, stream))
        self._loaded = True
        return torch.from_numpy(gamma)

    # --------------------------------------------------------------- forward
    def workspace_bytes(self, num_tokens: int) -> int:
        n = ctypes.c_size_t()
        capi.check(capi.lib().mgpt_moe_workspace_bytes(self._h, num_tokens, ctypes.byref(n)))
        return n.value

    def get_footprint(self, B: int, T: int) -> int:
        """Forward workspace in bytes for a [B, T, C] input (the C ABI's
        replacement for MoELayer::get_footprint, layers/MoELayer.cpp:238-251)."""
        return self.workspace_bytes(B * T)

    def train_workspace_bytes(self, num_tokens: int) -> int:
        n = ctypes.c_size_t()
        capi.check(capi.lib().mgpt_moe_train_workspace_bytes(self._h, num_tokens,
                                                             ctypes.byref(n)))
        return n.value

    def reserve(self, max_tokens: int, train: bool = False, device=None) -> None:
        """Allocates the workspace for up to max_tokens tokens now, so that
        forwards of any N <= max_tokens allocate nothing: a sampling loop
        whose context grows to max_seq_len (pipeline/Generator.cpp:13-36
        re-runs the whole cropped context every step), or a decode step
        captured into a HIP graph."""
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._workspace(max_tokens, dev, train)

    def _workspace(self, n: int, device, train: bool = False) -> torch.Tensor:
        need = self.train_workspace_bytes(n) if train else self.workspace_bytes(n)
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = torch.empty(max(need, 256), dtype=torch.uint8, device=device)
        return self._ws

    def forward_into(self, x: torch.Tensor, out: torch.Tensor, train: bool = False) -> None:
        """out = MoE(x).  train=True also keeps what backward() needs (the
        reference's forward always does: layers/MoELayer.cpp:28-128)."""
        if not x.is_cuda or not out.is_cuda:
            raise ValueError("MoELayer runs on the GPU only: x and out must be device tensors")
        if x.dtype != self.dtype or out.dtype != self.dtype:
            raise TypeError(f"expected {self.dtype} activations")
        if x.shape[-1] != self.C or out.shape != x.shape:
            raise ValueError("shape mismatch")
        if not x.is_contiguous() or not out.is_contiguous():
            raise ValueError("x and out must be contiguous")
        n = x.numel() // self.C
        ws = self._workspace(n, x.device, train)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        fn = capi.lib().mgpt_moe_forward_train if train else capi.lib().mgpt_moe_forward
        capi.check(fn(self._h, x.data_ptr(), out.data_ptr(), n, ws.data_ptr(), ws.numel(), stream))
        self._last_n = n
        self._train_x = x if train else None
        self._train_block = None

    def forward(self, x: torch.Tensor, train: bool = False) -> torch.Tensor:
        out = torch.empty_like(x)
        self.forward_into(x, out, train)
        return out

    def forward_block(self, x: torch.Tensor, gamma: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
        """out = x + MoE(RMSNorm(x) * gamma): the MoE half of a transformer
        block (ln2, mlp and the residual add of
        layers/TransformerBlock.cpp:42-46) in one fused pass."""
        out = torch.empty_like(x)
        self.forward_block_into(x, gamma, eps, out)
        return out

    def forward_block_into(self, x: torch.Tensor, gamma: torch.Tensor, eps: float,
                           out: torch.Tensor, train: bool = False) -> None:
        """forward_block writing into a caller-provided `out` (same shape and
        dtype as x); gamma is a float32 device tensor of C elements.
        train=True also keeps what backward_block_into needs."""
        if not x.is_cuda or x.dtype != self.dtype or x.shape[-1] != self.C or not x.is_contiguous():
            raise ValueError("x must be a contiguous device tensor [..., C] of the layer's dtype")
        if not out.is_cuda or out.dtype != self.dtype or out.shape != x.shape or not out.is_contiguous():
            raise ValueError("out must be a contiguous device tensor shaped like x")
        g = gamma.detach().to(device=x.device, dtype=torch.float32).contiguous()
        if g.numel() != self.C:
            raise ValueError("gamma must have C elements")
        n = x.numel() // self.C
        ws = self._workspace(n, x.device, train)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        fn = (capi.lib().mgpt_moe_forward_block_train if train
              else capi.lib().mgpt_moe_forward_block)
        capi.check(fn(self._h, x.data_ptr(), g.data_ptr(), float(eps), out.data_ptr(), n,
                      ws.data_ptr(), ws.numel(), stream))
        self._last_n = n
        self._train_x = None
        self._train_block = (x, g) if train else None

    def rstd(self) -> torch.Tensor:
        """Device view [N] of the per-token 1/rms of the last forward_block."""
        n = self._last_n
        p = ctypes.c_void_p()
        capi.check(capi.lib().mgpt_moe_get_rstd(self._h, n, self._ws.data_ptr(), ctypes.byref(p)))
        off = p.value - self._ws.data_ptr()
        return self._ws[off:off + 4 * n].view(torch.float32)

    # -------------------------------------------------------------- backward
    def backward_into(self, dout: torch.Tensor, din: torch.Tensor) -> None:
        """din = dL/dx for upstream gradient dout after forward(x, train=True);
        adds the parameter gradients to the layer's gradient buffers
        (MoELayer::backward_into, layers/MoELayer.cpp:130-223)."""
        x = self._train_x
        if x is None:
            if self._train_block is not None:
                raise RuntimeError("after forward_block(..., train=True) use backward_block_into")
            raise RuntimeError("backward needs a preceding forward(x, train=True)")
        if dout.shape != x.shape or din.shape != x.shape:
            raise ValueError("dout and din must have the input's shape")
        if dout.dtype != self.dtype or din.dtype != self.dtype:
            raise TypeError(f"expected {self.dtype} gradients")
        if not (dout.is_cuda and din.is_cuda and dout.is_contiguous() and din.is_contiguous()):
            raise ValueError("dout and din must be contiguous device tensors")
        n = x.numel() // self.C
        stream = torch.cuda.current_stream(x.device).cuda_stream
        capi.check(capi.lib().mgpt_moe_backward(self._h, x.data_ptr(), dout.data_ptr(),
                                                din.data_ptr(), n, self._ws.data_ptr(),
                                                self._ws.numel(), stream))

    def backward(self, dout: torch.Tensor) -> torch.Tensor:
        din = torch.empty_like(dout)
        self.backward_into(dout, din)
        return din

    def backward_block_into(self, dout: torch.Tensor, din: torch.Tensor,
                            dgamma: torch.Tensor) -> None:
        """Backward of forward_block(x, gamma, train=True) for the upstream
        gradient dout of its output: din = dL/dx (the residual path plus the
        ln2 RMSNorm's backward of the MoE input gradient), dgamma (float32
        device [C]) += the ln2 scale's gradient, and the MoE parameter
        gradients added to the layer's buffers (layers/TransformerBlock.cpp:
        81-85 with layers/RMSNormLayer.cpp:30-33)."""
        blk = self._train_block
        if blk is None:
            raise RuntimeError("backward_block needs a preceding forward_block(..., train=True)")
        x, g = blk
        if dout.shape != x.shape or din.shape != x.shape:
            raise ValueError("dout and din must have the input's shape")
        if dout.dtype != self.dtype or din.dtype != self.dtype:
            raise TypeError(f"expected {self.dtype} gradients")
        if not (dout.is_cuda and din.is_cuda and dout.is_contiguous() and din.is_contiguous()):
            raise ValueError("dout and din must be contiguous device tensors")
        if (not dgamma.is_cuda or dgamma.dtype != torch.float32 or dgamma.numel() != self.C
                or not dgamma.is_contiguous()):
            raise ValueError("dgamma must be a contiguous float32 device tensor of C elements")
        n = x.numel() // self.C
        stream = torch.cuda.current_stream(x.device).cuda_stream
        capi.check(capi.lib().mgpt_moe_backward_block(self._h, x.data_ptr(), g.data_ptr(),
                                                      dout.data_ptr(), din.data_ptr(),
                                                      dgamma.data_ptr(), n, self._ws.data_ptr(),
                                                      self._ws.numel(), stream))

    def backward_block(self, dout: torch.Tensor, dgamma: torch.Tensor | None = None):
        """(din, dgamma) of backward_block_into; dgamma starts from zero
        unless one is passed to add into."""
        din = torch.empty_like(dout)
        if dgamma is None:
            dgamma = torch.zeros(self.C, dtype=torch.float32, device=dout.device)
        self.backward_block_into(dout, din, dgamma)
        return din, dgamma

    def zero_grad(self) -> None:
        stream = torch.cuda.current_stream().cuda_stream
        capi.check(capi.lib().mgpt_moe_zero_grad(self._h, stream))

    def get_gradients(self) -> list:
        """The 2+6E fp32 gradients (device tensors) in get_parameters() order
        and reference layout: W_r [C,E], b_r [1,E], then per expert
        W_gate [C,H], b_gate [1,H], W_up [C,H], b_up [1,H], W_down [H,C],
        b_down [1,C]."""
        C, H, E = self.C, self.H, self.E
        shapes = [(C, E), (1, E)] + [(C, H), (1, H), (C, H), (1, H), (H, C), (1, C)] * E
        dev = self._ws.device if self._ws is not None else torch.device("cuda")
        out = [torch.empty(s, dtype=torch.float32, device=dev) for s in shapes]
        ptrs = (ctypes.c_void_p * len(out))(*[t.data_ptr() for t in out])
        stream = torch.cuda.current_stream(dev).cuda_stream
        capi.check(capi.lib().mgpt_moe_get_gradients(self._h, ptrs, len(out), 1, stream))
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
    def set_profiling(self, on: bool, gemm_only: bool = False) -> None:
        """Record HIP events at the forward's stage boundaries (gemm_only:
        only around the gate/up GEMM, leaving the other launches' spacing
        as it is unprofiled)."""
        mode = 0 if not on else (2 if gemm_only else 1)
        capi.check(capi.lib().mgpt_moe_set_profiling(self._h, mode))

    def stage_times(self) -> dict:
        """Mean stage durations (ms) over the profiled forwards since
        set_profiling(True) (at most the last 64), plus their count."""
        ms = np.zeros(capi.NUM_STAGES + 1, dtype=np.float32)
        capi.check(capi.lib().mgpt_moe_stage_times(self._h, ms.ctypes.data, capi.NUM_STAGES + 1))
        out = dict(zip(capi.STAGE_NAMES, ms[:capi.NUM_STAGES].tolist()))
        out["forwards"] = int(ms[capi.NUM_STAGES])
        return out

    def backward_stage_times(self) -> dict:
        """Mean backward stage durations (ms) over the profiled backwards
        since set_profiling(True), plus their count."""
        n = capi.NUM_BWD_STAGES
        ms = np.zeros(n + 1, dtype=np.float32)
        capi.check(capi.lib().mgpt_moe_backward_stage_times(self._h, ms.ctypes.data, n + 1))
        out = dict(zip(capi.BWD_STAGE_NAMES, ms[:n].tolist()))
        out["backwards"] = int(ms[n])
        return out

    def export_fp8(self, expert: int, which: int):
        rows, cols = (self.C, self.H) if which < 2 else (self.H, self.C)
        q = np.zeros((rows, cols), np.uint8)
        s = np.zeros(cols, np.float32)
        capi.check(capi.lib().mgpt_moe_export_fp8(self._h, expert, which, q.ctypes.data,
                                                  s.ctypes.data))
        return q, s
