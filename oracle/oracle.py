"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the soklyn_amd product path.

`OracleBlock` holds one DenseBlock's state as numpy float32 arrays with the
same field names as the reference's DenseBlock getters (src/mlp.rs:422-465)
and calls the C restatement for each hot-path step.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_FP = C.POINTER(C.c_float)


class _OrcBlock(C.Structure):
    _fields_ = [
        ("half", C.c_int32), ("inputs", C.c_uint32), ("outputs", C.c_uint32),
        ("max_batch", C.c_uint32), ("norm", C.c_uint32), ("act", C.c_uint32),
        ("leaky", C.c_float), ("mask_coeff", C.c_float),
        ("regularisation", C.c_uint32), ("regu_coeff", C.c_float),
    ] + [(n, _FP) for n in (
        "w", "b", "norm_w", "norm_b",
        "master_w", "master_b", "master_norm_w", "master_norm_b",
        "dv_w", "dv_b", "dm_w", "dm_b", "dv_norm_w", "dv_norm_b", "dm_norm_w", "dm_norm_b",
        "out", "predrop", "preact", "centered", "prenorm", "norm_rstd", "mask",
        "grad", "d_prenorm", "d_norm_w", "d_norm_b")]


class _OrcOptimiser(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("nesterov", C.c_uint32)]


class _OrcTrain(C.Structure):
    _fields_ = [("optimiser", _OrcOptimiser), ("norm_optimiser", _OrcOptimiser),
                ("batch_size", C.c_uint32), ("learn_rate", C.c_float), ("grad_clamp", C.c_float)]


def build() -> str:
    """Compile liboracle.so from oracle/soklyn_oracle.c (make)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_f32_to_f16_bits.restype = C.c_uint16
        L.orc_f32_to_f16_bits.argtypes = [C.c_float]
        L.orc_f16_bits_to_f32.restype = C.c_float
        L.orc_f16_bits_to_f32.argtypes = [C.c_uint16]
        L.orc_round_f16.restype = C.c_float
        L.orc_round_f16.argtypes = [C.c_float]
        L.orc_round_f16_array.argtypes = [_FP, C.c_size_t]
        L.orc_scramble_seed.restype = C.c_uint32
        L.orc_scramble_seed.argtypes = [C.c_uint32, C.c_uint32]
        L.orc_dropout_u.restype = C.c_float
        L.orc_dropout_u.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_activation.restype = C.c_float
        L.orc_activation.argtypes = [C.c_uint32, C.c_float, C.c_float]
        L.orc_activation_derivative.restype = C.c_float
        L.orc_activation_derivative.argtypes = [C.c_uint32, C.c_float, C.c_float, C.c_float, C.c_float]
        B = C.POINTER(_OrcBlock)
        L.orc_forward.argtypes = [B, _FP, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_softmax.argtypes = [B]
        L.orc_output_error.argtypes = [B, _FP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float]
        L.orc_hidden_error.argtypes = [B, B, C.c_uint32]
        L.orc_error_from_sum.argtypes = [B, _FP, C.c_uint32]
        L.orc_input_grad.argtypes = [B, C.c_uint32, _FP]
        L.orc_backward.argtypes = [B, _FP, C.POINTER(_OrcTrain), C.c_uint32]
        L.orc_gemm_nn.argtypes = [_FP, _FP, _FP, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_num_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


def round_f16(x) -> np.ndarray:
    """Oracle binary16 RNE rounding (kept as float32)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).copy()
    lib().orc_round_f16_array(_p(a), a.size)
    return a


def scramble_seed(step: int, layer_id: int) -> int:
    return int(lib().orc_scramble_seed(step & 0xFFFFFFFF, layer_id & 0xFFFFFFFF))


def dropout_u(col: int, row: int, seed: int) -> float:
    return float(lib().orc_dropout_u(col & 0xFFFFFFFF, row & 0xFFFFFFFF, seed & 0xFFFFFFFF))


def activation(act: int, x: float, leaky: float = 0.0) -> float:
    return float(lib().orc_activation(act, x, leaky))


def activation_derivative(act: int, err: float, out_v: float, in_x: float, leaky: float = 0.0) -> float:
    return float(lib().orc_activation_derivative(act, err, out_v, in_x, leaky))


def gemm_nn(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().orc_gemm_nn(_p(a), _p(b), _p(c), m, k, n)
    return c


def num_threads() -> int:
    return int(lib().orc_num_threads())


class Optimiser:
    """Mirror of util/function.rs:77-117 (SGD {v_coeff, nesterov}, Adam {m, v, eps})."""

    def __init__(self, kind: int, beta1: float = 0.0, beta2: float = 0.0, epsilon: float = 0.0,
                 nesterov: bool = False):
        self.kind, self.beta1, self.beta2, self.epsilon, self.nesterov = kind, beta1, beta2, epsilon, nesterov

    @staticmethod
    def sgd(v_coeff: float = 0.0, nesterov: bool = False) -> "Optimiser":
        return Optimiser(0, v_coeff, 0.0, 0.0, nesterov)

    @staticmethod
    def adam(m_coeff: float = 0.9, v_coeff: float = 0.999, epsilon: float = 1e-8) -> "Optimiser":
        return Optimiser(1, m_coeff, v_coeff, epsilon, False)

    def _c(self) -> _OrcOptimiser:
        return _OrcOptimiser(self.kind, self.beta1, self.beta2, self.epsilon, int(self.nesterov))


BLOCK_FIELDS_T = ("w", "b", "norm_w", "norm_b", "out", "predrop", "preact", "centered",
                  "prenorm", "norm_rstd", "mask")
BLOCK_FIELDS_F32 = ("master_w", "master_b", "master_norm_w", "master_norm_b",
                    "dv_w", "dv_b", "dm_w", "dm_b", "dv_norm_w", "dv_norm_b", "dm_norm_w", "dm_norm_b",
                    "grad", "d_prenorm", "d_norm_w", "d_norm_b")


class OracleBlock:
    """One DenseBlock's state on the host (src/mlp.rs:265-288, 341-421)."""

    def __init__(self, inputs: int, outputs: int, max_batch: int, w: np.ndarray, *, half: bool = False,
                 norm: int = 0, act: int = 0, leaky: float = 0.0, mask_coeff: float = 0.0,
                 regularisation: int = 0, regu_coeff: float = 0.0, master_w: np.ndarray | None = None,
                 b: np.ndarray | None = None):
        K, N, M = inputs, outputs, max_batch
        self.half = half
        self.inputs, self.outputs, self.max_batch = K, N, M
        self.norm, self.act, self.leaky, self.mask_coeff = norm, act, leaky, mask_coeff
        self.regularisation, self.regu_coeff = regularisation, regu_coeff
        f = np.float32
        w = np.ascontiguousarray(w, f).reshape(K, N)
        self.w = round_f16(w) if half else w.copy()
        self.b = np.zeros((1, N), f) if b is None else np.ascontiguousarray(b, f).reshape(1, N).copy()
        if half:
            self.b = round_f16(self.b)
        self.norm_w = np.ones((1, N), f)
        self.norm_b = np.zeros((1, N), f)
        if half:
            # fp16 masters: f32 of the rounded values (mlp.rs:27-43) unless given (convert_f16 route)
            self.master_w = (np.ascontiguousarray(master_w, f).reshape(K, N).copy()
                             if master_w is not None else self.w.copy())
            self.master_b = self.b.copy()
            self.master_norm_w = np.ones((1, N), f)
            self.master_norm_b = np.zeros((1, N), f)
        else:
            self.master_w = self.master_b = self.master_norm_w = self.master_norm_b = None
        for n, shape in (("dv_w", (K, N)), ("dm_w", (K, N)), ("dv_b", (1, N)), ("dm_b", (1, N)),
                         ("dv_norm_w", (1, N)), ("dv_norm_b", (1, N)), ("dm_norm_w", (1, N)),
                         ("dm_norm_b", (1, N))):
            setattr(self, n, np.zeros(shape, f))
        for n in ("out", "predrop", "preact", "centered", "prenorm"):
            setattr(self, n, np.zeros((M, N), f))
        self.norm_rstd = np.zeros((max(M, N),), f)
        self.mask = np.ones((M, N), f)
        for n in ("grad", "d_prenorm", "d_norm_w", "d_norm_b"):
            setattr(self, n, np.zeros((M, N), f))

    def _c(self) -> _OrcBlock:
        s = _OrcBlock()
        s.half = int(self.half)
        s.inputs, s.outputs, s.max_batch = self.inputs, self.outputs, self.max_batch
        s.norm, s.act, s.leaky, s.mask_coeff = self.norm, self.act, self.leaky, self.mask_coeff
        s.regularisation, s.regu_coeff = self.regularisation, self.regu_coeff
        for n in BLOCK_FIELDS_T + BLOCK_FIELDS_F32:
            setattr(s, n, _p(getattr(self, n)))
        self._keep = s
        return s

    # -- hot-path steps ---------------------------------------------------------
    def forward(self, x: np.ndarray, m: int, use_dropout: bool = False, seed: int = 0):
        x = np.ascontiguousarray(x, np.float32)
        assert x.shape[1] == self.inputs
        rc = lib().orc_forward(C.byref(self._c()), _p(x), m, int(use_dropout), seed & 0xFFFFFFFF)
        assert rc == 0, rc
        return self.out

    def output_error(self, target: np.ndarray, loss: int, act: int, leaky: float = 0.0):
        t = np.ascontiguousarray(target, np.float32)
        rc = lib().orc_output_error(C.byref(self._c()), _p(t), t.shape[0], loss, act, leaky)
        assert rc == 0, rc

    def hidden_error(self, nxt: "OracleBlock", m: int):
        rc = lib().orc_hidden_error(C.byref(self._c()), C.byref(nxt._c()), m)
        assert rc == 0, rc

    def error_from_sum(self, s: np.ndarray, m: int):
        s = np.ascontiguousarray(s, np.float32)
        rc = lib().orc_error_from_sum(C.byref(self._c()), _p(s), m)
        assert rc == 0, rc

    def input_grad(self, m: int) -> np.ndarray:
        dx = np.empty((m, self.inputs), np.float32)
        rc = lib().orc_input_grad(C.byref(self._c()), m, _p(dx))
        assert rc == 0, rc
        return dx

    def backward(self, x: np.ndarray, optimiser: Optimiser, norm_optimiser: Optimiser, batch_size: int,
                 learn_rate: float, grad_clamp: float, step: int):
        x = np.ascontiguousarray(x, np.float32)
        tc = _OrcTrain(optimiser._c(), norm_optimiser._c(), batch_size, learn_rate, grad_clamp)
        rc = lib().orc_backward(C.byref(self._c()), _p(x), C.byref(tc), step)
        assert rc == 0, rc

    def snapshot(self) -> dict:
        return {n: (None if getattr(self, n) is None else getattr(self, n).copy())
                for n in BLOCK_FIELDS_T + BLOCK_FIELDS_F32}
