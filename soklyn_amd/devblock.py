"""Device-side DenseBlock state for driving the C ABI from Python.

`DeviceBlock` owns one block's device buffers (torch tensors used purely as
device memory) laid out exactly as `skl_dense_desc` expects, initialised the
way src/mlp.rs:45-110 / 377-421 initialises a block: W from the caller, bias
and norm bias 0, norm weight 1, moments 0, caches 0, mask 1, and for fp16
blocks fp32 masters.  Every hot-path step is one C-ABI call.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import abi

T_FIELDS = ("w", "b", "norm_w", "norm_b", "out", "predrop", "preact", "centered", "prenorm", "norm_rstd", "mask")
F32_FIELDS = ("master_w", "master_b", "master_norm_w", "master_norm_b",
              "dv_w", "dv_b", "dm_w", "dm_b", "dv_norm_w", "dv_norm_b", "dm_norm_w", "dm_norm_b",
              "grad", "d_prenorm", "d_norm_w", "d_norm_b")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class DeviceBlock:
    def __init__(self, ctx: abi.Context, inputs: int, outputs: int, max_batch: int, w: np.ndarray, *,
                 half: bool = False, norm: int = 0, act: int = 0, leaky: float = 0.0, mask_coeff: float = 0.0,
                 regularisation: int = 0, regu_coeff: float = 0.0, is_training: bool = True,
                 master_w: np.ndarray | None = None, b: np.ndarray | None = None, device: str = "cuda"):
        self.ctx = ctx
        self.half = half
        self.inputs, self.outputs, self.max_batch = inputs, outputs, max_batch
        self.norm, self.act, self.leaky, self.mask_coeff = norm, act, leaky, mask_coeff
        self.regularisation, self.regu_coeff = regularisation, regu_coeff
        self.is_training = is_training
        K, N, M = inputs, outputs, max_batch
        T = torch.float16 if half else torch.float32
        self.tdtype = T
        dev = torch.device(device)

        def up(a, dt):
            return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device=dev, dtype=dt).contiguous()

        def zeros(shape, dt):
            return torch.zeros(shape, device=dev, dtype=dt)

        w = np.asarray(w, np.float32).reshape(K, N)
        self.w = up(w, T)
        self.b = zeros((1, N), T) if b is None else up(np.asarray(b, np.float32).reshape(1, N), T)
        self.norm_w = torch.ones((1, N), device=dev, dtype=T)
        self.norm_b = zeros((1, N), T)
        if half:
            self.master_w = up(master_w.reshape(K, N) if master_w is not None else self.w.float().cpu().numpy(),
                               torch.float32)
            self.master_b = self.b.float().clone()
            self.master_norm_w = torch.ones((1, N), device=dev, dtype=torch.float32)
            self.master_norm_b = zeros((1, N), torch.float32)
        else:
            self.master_w = self.master_b = self.master_norm_w = self.master_norm_b = None
        for n, shape in (("dv_w", (K, N)), ("dm_w", (K, N)), ("dv_b", (1, N)), ("dm_b", (1, N)),
                         ("dv_norm_w", (1, N)), ("dv_norm_b", (1, N)), ("dm_norm_w", (1, N)),
                         ("dm_norm_b", (1, N))):
            setattr(self, n, zeros(shape, torch.float32) if is_training else None)
        for n in ("out", "predrop", "preact", "centered", "prenorm"):
            setattr(self, n, zeros((M, N), T))
        self.norm_rstd = zeros((max(M, N),), T)
        self.mask = torch.ones((M, N), device=dev, dtype=T)
        for n in ("grad", "d_prenorm", "d_norm_w", "d_norm_b"):
            setattr(self, n, zeros((M, N), torch.float32) if is_training else None)
        self.d_prenorm_h = zeros((M, N), torch.float16) if (half and is_training) else None
        self._desc = None

    # -- descriptor -----------------------------------------------------------------
    def desc(self) -> abi.SklDenseDesc:
        d = abi.SklDenseDesc()
        d.dtype = abi.F16 if self.half else abi.F32
        d.inputs, d.outputs, d.max_batch = self.inputs, self.outputs, self.max_batch
        d.norm, d.act, d.leaky, d.mask_coeff = self.norm, self.act, self.leaky, self.mask_coeff
        d.regularisation, d.regu_coeff = self.regularisation, self.regu_coeff
        d.is_training = int(self.is_training)
        for n in T_FIELDS + F32_FIELDS + ("d_prenorm_h",):
            setattr(d, n, _ptr(getattr(self, n)))
        self._desc = d
        return d

    # -- hot-path steps ------------------------------------------------------------------
    def forward(self, x: torch.Tensor, batch: int, use_dropout: bool = False, seed: int = 0):
        abi.call("skl_dense_forward", self.ctx.h, C.byref(self.desc()), C.c_void_p(x.data_ptr()),
                 x.shape[0], x.shape[1], batch, int(use_dropout), seed & 0xFFFFFFFF)
        return self.out

    def output_error(self, target: torch.Tensor, loss: int, act: int, leaky: float = 0.0):
        abi.call("skl_dense_output_error", self.ctx.h, C.byref(self.desc()), C.c_void_p(target.data_ptr()),
                 target.shape[0], target.shape[1], loss, act, leaky)

    def hidden_error(self, nxt: "DeviceBlock", batch: int):
        abi.call("skl_dense_hidden_error", self.ctx.h, C.byref(self.desc()), C.byref(nxt.desc()), batch)

    def backward(self, x: torch.Tensor, tc: abi.SklTrainCtx, step: int):
        abi.call("skl_dense_backward", self.ctx.h, C.byref(self.desc()), C.c_void_p(x.data_ptr()),
                 x.shape[0], x.shape[1], C.byref(tc), step)

    def backward_hidden(self, nxt: "DeviceBlock", x: torch.Tensor, tc: abi.SklTrainCtx, step: int):
        abi.call("skl_dense_backward_hidden", self.ctx.h, C.byref(self.desc()), C.byref(nxt.desc()),
                 C.c_void_p(x.data_ptr()), x.shape[0], x.shape[1], C.byref(tc), step)

    def error_from_sum(self, s: torch.Tensor, batch: int):
        assert s.dtype == torch.float32 and s.is_contiguous()
        abi.call("skl_dense_error_from_sum", self.ctx.h, C.byref(self.desc()), C.c_void_p(s.data_ptr()), batch)

    def error_from_sum_noalloc(self, s: torch.Tensor, batch: int):
        assert s.dtype == torch.float32 and s.is_contiguous()
        abi.call("skl_dense_error_from_sum_noalloc", self.ctx.h, C.byref(self.desc()), C.c_void_p(s.data_ptr()),
                 batch)

    def input_grad(self, batch: int, out: torch.Tensor | None = None) -> torch.Tensor:
        if out is None:
            out = torch.empty((batch, self.inputs), device=self.w.device, dtype=torch.float32)
        abi.call("skl_dense_input_grad", self.ctx.h, C.byref(self.desc()), batch, C.c_void_p(out.data_ptr()))
        return out

    # -- host views ----------------------------------------------------------------------
    def get(self, name: str) -> np.ndarray | None:
        t = getattr(self, name)
        return None if t is None else t.float().cpu().numpy()

    def snapshot(self) -> dict:
        return {n: self.get(n) for n in T_FIELDS + F32_FIELDS}
