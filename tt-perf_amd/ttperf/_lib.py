"""ctypes binding of libttperf_hip (include/ttperf/ttperf.h).

The HIP library is the only compute path: if it is not built, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("TTPERF_LIB", os.path.join(_PKG, "lib", "libttperf_hip.so"))

OK = 0
ERR_INVALID, ERR_NO_DEVICE, ERR_HIP, ERR_OOM, ERR_STATE, ERR_RANGE = -1, -2, -3, -4, -5, -6
MODE_FP32, MODE_MIXED, MODE_BF16 = 0, 1, 2
STORE_SGD = 0x100
ABI_VERSION = 3
BUF_PARAM, BUF_GRAD, BUF_MASTER, BUF_EXP_AVG, BUF_EXP_AVG_SQ, BUF_MOMENTUM = range(6)
ALL_TENSORS = 0xFFFFFFFF
TENSOR_DECAY = 1
HOST, DEVICE = 0, 1
DTYPE_F32, DTYPE_BF16 = 0, 1
ACCUM_SUMSQ = 0x100
ACCUM_MULTI_MAX = 64  # tensors per ttp_accumulate_grad_multi call
ZERO_NO_FILL = 0x100  # OR'd into zero_grad's set_to_none: flags only
STEP_TENSOR_SUMS = 1
STEP_DEFER_SCALE = 2
KERNEL_NORM, KERNEL_UPDATE = 0, 1


class TensorDesc(C.Structure):
    _fields_ = [("numel", C.c_uint64), ("flags", C.c_uint32), ("reserved", C.c_uint32)]


class AdamHParams(C.Structure):
    _fields_ = [("lr", C.c_double), ("beta1", C.c_double), ("beta2", C.c_double),
                ("eps", C.c_double), ("weight_decay", C.c_double), ("decoupled", C.c_int32),
                ("flags", C.c_int32), ("max_grad_norm", C.c_double)]


class SgdHParams(C.Structure):
    _fields_ = [("lr", C.c_double), ("momentum", C.c_double), ("dampening", C.c_double),
                ("weight_decay", C.c_double), ("nesterov", C.c_int32), ("flags", C.c_int32),
                ("max_grad_norm", C.c_double)]


class ScalerConfig(C.Structure):
    _fields_ = [("enabled", C.c_int32), ("growth_interval", C.c_int32),
                ("init_scale", C.c_double), ("growth_factor", C.c_double),
                ("backoff_factor", C.c_double)]


class StepReport(C.Structure):
    _fields_ = [("found_inf", C.c_int32), ("skipped", C.c_int32), ("grad_norm", C.c_double),
                ("clip_coef", C.c_float), ("scale", C.c_float), ("growth_tracker", C.c_int32),
                ("reserved", C.c_int32), ("step", C.c_uint64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_ if k != "reserved"}


# name -> (restype, argtypes); the ABI surface the header declares
_P = C.c_void_p
SIGNATURES = {
    "ttp_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "ttp_create": (C.c_int, [C.c_int, C.POINTER(TensorDesc), C.c_uint32, C.c_int, C.POINTER(_P)]),
    "ttp_destroy": (C.c_int, [_P]),
    "ttp_set_stream": (C.c_int, [_P, _P]),
    "ttp_reset_stream": (C.c_int, [_P]),
    "ttp_sync": (C.c_int, [_P]),
    "ttp_num_tensors": (C.c_int, [_P, C.POINTER(C.c_uint32)]),
    "ttp_mode": (C.c_int, [_P, C.POINTER(C.c_int)]),
    "ttp_flat_numel": (C.c_int, [_P, C.POINTER(C.c_uint64)]),
    "ttp_tensor_info": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_uint32)]),
    "ttp_buffer_ptr": (C.c_int, [_P, C.c_int, C.c_uint32, C.POINTER(_P)]),
    "ttp_buffer_layout": (C.c_int, [_P, C.c_int, C.POINTER(_P), C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint32)]),
    "ttp_upload": (C.c_int, [_P, C.c_int, C.c_uint32, _P, C.c_uint64, C.c_int]),
    "ttp_download": (C.c_int, [_P, C.c_int, C.c_uint32, _P, C.c_uint64, C.c_int]),
    "ttp_set_has_grad": (C.c_int, [_P, C.c_uint32, C.c_int]),
    "ttp_get_has_grad": (C.c_int, [_P, C.c_uint32, C.POINTER(C.c_int)]),
    "ttp_zero_grad": (C.c_int, [_P, C.c_int]),
    "ttp_zero_grad_subset": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_uint32, C.c_int]),
    "ttp_accumulate_grad": (C.c_int, [_P, C.c_uint32, _P, C.c_uint64, C.c_int, C.c_int]),
    "ttp_accumulate_grad_multi": (C.c_int, [_P, C.POINTER(C.c_uint32), C.POINTER(_P), C.c_uint32,
                                            C.c_int]),
    "ttp_adam_step": (C.c_int, [_P, C.POINTER(AdamHParams), C.POINTER(StepReport)]),
    "ttp_sgd_step": (C.c_int, [_P, C.POINTER(SgdHParams), C.POINTER(StepReport)]),
    "ttp_adam_step_subset": (C.c_int, [_P, C.POINTER(AdamHParams), C.POINTER(C.c_uint32),
                                       C.c_uint32, C.POINTER(StepReport)]),
    "ttp_sgd_step_subset": (C.c_int, [_P, C.POINTER(SgdHParams), C.POINTER(C.c_uint32),
                                      C.c_uint32, C.POINTER(StepReport)]),
    "ttp_adam_step_noalloc": (C.c_int, [_P, C.POINTER(AdamHParams), C.POINTER(C.c_uint32),
                                        C.c_uint32]),
    "ttp_grad_norm": (C.c_int, [_P, C.POINTER(C.c_double)]),
    "ttp_grad_sumsq_tensors": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_uint32]),
    "ttp_get_step": (C.c_int, [_P, C.POINTER(C.c_uint64)]),
    "ttp_set_step": (C.c_int, [_P, C.c_uint64]),
    "ttp_scaler_configure": (C.c_int, [_P, C.POINTER(ScalerConfig)]),
    "ttp_scaler_get": (C.c_int, [_P, C.POINTER(C.c_float), C.POINTER(C.c_int32)]),
    "ttp_scaler_set": (C.c_int, [_P, C.c_float, C.c_int32]),
    "ttp_scaler_update": (C.c_int, [_P]),
    "ttp_save_state": (C.c_int, [_P, C.c_char_p]),
    "ttp_load_state": (C.c_int, [_P, C.c_char_p]),
    "ttp_capture_begin": (C.c_int, [_P]),
    "ttp_capture_end": (C.c_int, [_P, C.POINTER(_P)]),
    "ttp_graph_launch": (C.c_int, [_P]),
    "ttp_graph_destroy": (C.c_int, [_P]),
    "ttp_timing_enable": (C.c_int, [_P, C.c_int]),
    "ttp_timing_collect": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "ttp_last_error": (C.c_char_p, []),
    "ttp_abi_version": (C.c_int, []),
}


class TTPError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libttperf_hip error {code}: {msg}")
        self.code = code


class TTPValueError(TTPError, ValueError):
    """Argument errors: the cases py/optim.py raises ValueError for."""


class TTPMemoryError(TTPError, MemoryError):
    """A device or pinned-host allocation did not fit (TTP_ERR_OOM)."""


def _bind_one_hip_runtime():
    """Load torch (when installed) before libttperf_hip.

    torch ships its own HIP/HSA runtimes (SONAMEs libamdhip64.so.7, libhsa-runtime64.so.1)
    and loads them by file name from its own lib directory.  The dynamic loader satisfies
    this library's DT_NEEDED entries with an already-loaded object of the same SONAME, so
    loading torch first gives one HIP runtime per process, shared by torch and this engine
    (one device context, one set of streams, tensors and hipStream_t handles valid in both).
    Loading this library first would instead map /opt/rocm's runtime and let torch map a
    second copy, with two independent device contexts in one process."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def _load():
    _bind_one_hip_runtime()
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libttperf_hip.so not found at {LIB_PATH}; build it with `make -C tt-perf_amd` "
            "(or __graft_entry__.build()). There is no CPU fallback.")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
if lib.ttp_abi_version() != ABI_VERSION:
    raise ImportError(f"{LIB_PATH} implements ABI version {lib.ttp_abi_version()}; this binding "
                      f"is written against version {ABI_VERSION}: rebuild the library")


def check(rc):
    if rc != OK:
        msg = lib.ttp_last_error().decode(errors="replace")
        if rc in (ERR_INVALID, ERR_RANGE):
            raise TTPValueError(rc, msg)
        if rc == ERR_OOM:
            raise TTPMemoryError(rc, msg)
        raise TTPError(rc, msg)
    return rc


def device_count():
    n = C.c_int(0)
    check(lib.ttp_device_count(C.byref(n)))
    return n.value
