"""ctypes binding of include/soklyn_hip.h (libsoklyn_hip.so).

This is the same binding a Python caller of the drop-in boundary would write;
tests, bench.py and __graft_entry__ drive the HIP path through it.  Loading
fails loudly when the library has not been built: there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsoklyn_hip.so")

SKL_OK = 0
STATUS = {
    -1: "InvalidConfiguration", -2: "TrainingModeRequired", -3: "AllocationLimitExceeded",
    -4: "MismatchedDimensions", -5: "InvalidBatchSize", -6: "HardwareConstraintViolation",
    -7: "TryFromIntError", -8: "NullPointer", -9: "UnsupportedTypeCast", -10: "NoDevice",
}
F32, F16 = 0, 1
NORM_DISABLED, NORM_RMS, NORM_LAYER, NORM_BATCH = 0, 1, 2, 3
ACT_IDENTITY, ACT_SIGMOID, ACT_RELU, ACT_LEAKY, ACT_TANH, ACT_SOFTMAX, ACT_SILU, ACT_MISH = range(8)
OPT_SGD, OPT_ADAM = 0, 1
LOSS_MSE, LOSS_CE, LOSS_BCE = 0, 1, 2

_VP = C.c_void_p
_FP = C.c_void_p   # float* passed as raw addresses


class SklDenseDesc(C.Structure):
    _fields_ = [
        ("dtype", C.c_uint32), ("inputs", C.c_uint32), ("outputs", C.c_uint32), ("max_batch", C.c_uint32),
        ("norm", C.c_uint32), ("act", C.c_uint32), ("leaky", C.c_float), ("mask_coeff", C.c_float),
        ("regularisation", C.c_uint32), ("regu_coeff", C.c_float), ("is_training", C.c_uint32),
        ("reserved0", C.c_uint32),
    ] + [(n, _VP) for n in (
        "w", "b", "norm_w", "norm_b",
        "master_w", "master_b", "master_norm_w", "master_norm_b",
        "dv_w", "dv_b", "dm_w", "dm_b", "dv_norm_w", "dv_norm_b", "dm_norm_w", "dm_norm_b",
        "out", "predrop", "preact", "centered", "prenorm", "norm_rstd", "mask",
        "grad", "d_prenorm", "d_norm_w", "d_norm_b", "d_prenorm_h")]


DESC_POINTERS = [n for n, _ in SklDenseDesc._fields_[12:]]


class SklOptimiser(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("nesterov", C.c_uint32)]


class SklTrainCtx(C.Structure):
    _fields_ = [("optimiser", SklOptimiser), ("norm_optimiser", SklOptimiser),
                ("batch_size", C.c_uint32), ("learn_rate", C.c_float), ("grad_clamp", C.c_float)]


# name -> (restype, argtypes)
_SIGS = {
    "skl_ctx_create": (C.c_int32, [C.c_int32, C.c_uint32, C.POINTER(C.c_void_p)]),
    "skl_ctx_destroy": (C.c_int32, [_VP]),
    "skl_ctx_set_sync": (C.c_int32, [_VP, C.c_uint32]),
    "skl_ctx_set_stream": (C.c_int32, [_VP, _VP]),
    "skl_ctx_stream": (_VP, [_VP]),
    "skl_synchronize": (C.c_int32, [_VP]),
    "skl_status_string": (C.c_char_p, [C.c_int32]),
    "skl_malloc": (C.c_int32, [_VP, C.POINTER(C.c_void_p), C.c_size_t]),
    "skl_free": (C.c_int32, [_VP, _VP]),
    "skl_memcpy_h2d": (C.c_int32, [_VP, _VP, _VP, C.c_size_t]),
    "skl_memcpy_d2h": (C.c_int32, [_VP, _VP, _VP, C.c_size_t]),
    "skl_memcpy_d2d": (C.c_int32, [_VP, _VP, _VP, C.c_size_t]),
    "skl_fill": (C.c_int32, [_VP, _VP, C.c_uint32, C.c_float, C.c_size_t]),
    "skl_cast": (C.c_int32, [_VP, _VP, C.c_uint32, _VP, C.c_uint32, C.c_size_t]),
    "skl_scramble_seed": (C.c_uint32, [C.c_uint32, C.c_uint32]),
    "skl_ctx_time_next_gemm": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "skl_dense_forward": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), _VP, C.c_uint32, C.c_uint32, C.c_uint32,
                                      C.c_uint32, C.c_uint32]),
    "skl_dense_output_error": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), _VP, C.c_uint32, C.c_uint32,
                                           C.c_uint32, C.c_uint32, C.c_float]),
    "skl_dense_hidden_error": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), C.POINTER(SklDenseDesc), C.c_uint32]),
    "skl_dense_backward": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), _VP, C.c_uint32, C.c_uint32,
                                       C.POINTER(SklTrainCtx), C.c_uint32]),
    "skl_dense_backward_hidden": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), C.POINTER(SklDenseDesc), _VP,
                                              C.c_uint32, C.c_uint32, C.POINTER(SklTrainCtx), C.c_uint32]),
    "skl_dense_error_from_sum": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), _VP, C.c_uint32]),
    "skl_dense_error_from_sum_noalloc": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), _VP, C.c_uint32]),
    "skl_dense_input_grad": (C.c_int32, [_VP, C.POINTER(SklDenseDesc), C.c_uint32, _VP]),
}

EXPORTED = tuple(_SIGS)
_lib = None


class SklError(RuntimeError):
    def __init__(self, fn: str, code: int):
        self.code = code
        name = STATUS.get(code, f"hipError {code}" if code > 0 else f"status {code}")
        super().__init__(f"{fn} failed: {name} ({code})")


def load(path: str = LIB_PATH):
    """Load libsoklyn_hip.so; raises if it has not been built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run soklyn_amd.build.build() (hipcc, gfx950) first")
        L = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def call(name: str, *args) -> int:
    rc = getattr(load(), name)(*args)
    if rc != SKL_OK:
        raise SklError(name, rc)
    return rc


def status(name: str, *args) -> int:
    """Call and return the raw status (for tests of the validation paths)."""
    return int(getattr(load(), name)(*args))


def optimiser(kind: int, beta1: float = 0.0, beta2: float = 0.0, epsilon: float = 0.0,
              nesterov: bool = False) -> SklOptimiser:
    return SklOptimiser(kind, beta1, beta2, epsilon, int(nesterov))


def sgd(v_coeff: float = 0.0, nesterov: bool = False) -> SklOptimiser:
    return optimiser(OPT_SGD, v_coeff, 0.0, 0.0, nesterov)


def adam(m_coeff: float = 0.9, v_coeff: float = 0.999, epsilon: float = 1e-8) -> SklOptimiser:
    return optimiser(OPT_ADAM, m_coeff, v_coeff, epsilon)


def train_ctx(opt: SklOptimiser, norm_opt: SklOptimiser, batch_size: int, learn_rate: float,
              grad_clamp: float = 3.4028234663852886e38) -> SklTrainCtx:
    return SklTrainCtx(opt, norm_opt, batch_size, learn_rate, grad_clamp)


class Context:
    """GpuContext (src/io/device.rs:22-183) over the C ABI."""

    def __init__(self, ordinal: int = 0, tile_dim: int = 16, stream=None):
        h = C.c_void_p()
        call("skl_ctx_create", ordinal, tile_dim, C.byref(h))
        self.h = h
        if stream is not None:
            call("skl_ctx_set_stream", self.h, C.c_void_p(stream))

    def set_stream(self, stream_ptr: int | None):
        call("skl_ctx_set_stream", self.h, C.c_void_p(stream_ptr) if stream_ptr else None)

    def time_next_gemm(self, start, stop):
        """Record two torch.cuda.Event objects at the start and end of the GEMM kernel of the next
        hot-path call (torch creates an event's HIP object on its first record(), so record each
        once beforehand)."""
        call("skl_ctx_time_next_gemm", self.h, C.c_void_p(start.cuda_event), C.c_void_p(stop.cuda_event))

    def set_sync(self, sync: bool):
        call("skl_ctx_set_sync", self.h, int(sync))

    def synchronize(self):
        call("skl_synchronize", self.h)

    def close(self):
        if self.h:
            load().skl_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
