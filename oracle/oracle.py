"""ctypes front end of the CPU oracle (oracle/ttp_oracle.c).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker.  Nothing in the product (tt-perf_amd/) imports it.

`OracleStore` holds the same flat layout as a libttperf_hip context (numpy arrays instead
of HBM buffers) and steps it with the C restatement of the reference optimizer
(py/optim.py:49-87 for Adam, autograd/dynamic/optim.hpp:21-27 for SGD).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libttp_oracle.so")

MODE_FP32 = 0
MODE_MIXED = 1
MODE_BF16 = 2  # bf16 weights (param) and grads only: plain SGD with bf16 roundings
DECAY = 1
DEFER_SCALE = 2  # ORC_STEP_DEFER_SCALE
ALIGN = 64  # elements; the engine's tensor alignment


class Tensor(C.Structure):
    _fields_ = [("offset", C.c_uint64), ("numel", C.c_uint64), ("flags", C.c_uint32),
                ("has_grad", C.c_int32)]


class Store(C.Structure):
    _fields_ = [("mode", C.c_int32), ("n_tensors", C.c_uint32), ("tensors", C.POINTER(Tensor)),
                ("total", C.c_uint64), ("param", C.c_void_p), ("grad", C.c_void_p),
                ("master", C.POINTER(C.c_float)), ("exp_avg", C.POINTER(C.c_float)),
                ("exp_avg_sq", C.POINTER(C.c_float)), ("momentum", C.POINTER(C.c_float)),
                ("mom_init", C.POINTER(C.c_uint8)), ("scaler_enabled", C.c_int32),
                ("growth_interval", C.c_int32), ("growth_factor", C.c_double),
                ("backoff_factor", C.c_double), ("scale", C.c_float),
                ("growth_tracker", C.c_int32), ("t", C.c_uint64), ("nthreads", C.c_int32),
                ("pending", C.c_int32)]


class AdamHP(C.Structure):
    _fields_ = [("lr", C.c_double), ("beta1", C.c_double), ("beta2", C.c_double),
                ("eps", C.c_double), ("weight_decay", C.c_double), ("decoupled", C.c_int32),
                ("flags", C.c_int32), ("max_grad_norm", C.c_double)]


class SgdHP(C.Structure):
    _fields_ = [("lr", C.c_double), ("momentum", C.c_double), ("dampening", C.c_double),
                ("weight_decay", C.c_double), ("nesterov", C.c_int32), ("flags", C.c_int32),
                ("max_grad_norm", C.c_double)]


class Report(C.Structure):
    _fields_ = [("found_inf", C.c_int32), ("skipped", C.c_int32), ("grad_norm", C.c_double),
                ("clip_coef", C.c_float), ("scale", C.c_float), ("growth_tracker", C.c_int32),
                ("reserved", C.c_int32), ("step", C.c_uint64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_ if k != "reserved"}


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_bf16_rne.restype = C.c_uint16
        L.orc_bf16_rne.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16_array.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.orc_bf16_to_f32_array.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.orc_bf16_check_range.restype = C.c_uint64
        L.orc_bf16_check_range.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
        L.orc_bias_correction.restype = C.c_float
        L.orc_bias_correction.argtypes = [C.c_double, C.c_uint64]
        L.orc_clip_coef.restype = C.c_float
        L.orc_clip_coef.argtypes = [C.c_double, C.c_double]
        L.orc_scaler_update.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_int32), C.c_int,
                                        C.c_double, C.c_double, C.c_int32]
        L.orc_scaler_update_pending.argtypes = [C.POINTER(Store)]
        L.orc_layout.restype = C.c_uint64
        L.orc_layout.argtypes = [C.c_void_p, C.c_uint32, C.c_uint64, C.c_void_p]
        L.orc_accumulate_grad.argtypes = [C.POINTER(Store), C.c_uint32, C.c_void_p, C.c_int]
        L.orc_grad_sumsq.restype = C.c_double
        L.orc_grad_sumsq.argtypes = [C.POINTER(Store), C.c_float, C.POINTER(C.c_int32)]
        for name, hp in (("orc_adam_step", AdamHP), ("orc_adam_step_opbyop", AdamHP),
                         ("orc_sgd_step", SgdHP)):
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = [C.POINTER(Store), C.POINTER(hp), C.POINTER(Report)]
        _lib = L
    return _lib


def _ptr(a, ctype=None):
    if a is None:
        return None
    p = a.ctypes.data_as(C.c_void_p)
    return C.cast(p, C.POINTER(ctype)) if ctype is not None else p


def bf16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def layout(numels, align=ALIGN):
    n = len(numels)
    nums = np.ascontiguousarray(numels, dtype=np.uint64)
    offs = np.zeros(max(n, 1), dtype=np.uint64)
    total = lib().orc_layout(_ptr(nums), n, align, _ptr(offs))
    return offs[:n].copy(), int(total)


class OracleStore:
    """Flat parameter store on the host, stepped by the C oracle."""

    def __init__(self, numels, flags=None, mode=MODE_FP32, nthreads=None):
        self.numels = [int(n) for n in numels]
        self.n = len(self.numels)
        self.flags = [int(f) for f in (flags if flags is not None else [0] * self.n)]
        self.mode = mode
        self.offsets, self.total = layout(self.numels)
        tot = max(self.total, 1)
        self._tensors = (Tensor * max(self.n, 1))()
        for i in range(self.n):
            self._tensors[i].offset = int(self.offsets[i])
            self._tensors[i].numel = self.numels[i]
            self._tensors[i].flags = self.flags[i]
            self._tensors[i].has_grad = 0
        self.master = np.zeros(tot, np.float32)  # unused by a BF16 store
        if mode in (MODE_MIXED, MODE_BF16):
            self.param = np.zeros(tot, np.uint16)
            self.grad = np.zeros(tot, np.uint16)
        else:
            self.param = self.master
            self.grad = np.zeros(tot, np.float32)
        self.exp_avg = np.zeros(tot, np.float32)
        self.exp_avg_sq = np.zeros(tot, np.float32)
        self.momentum = np.zeros(tot, np.float32)
        self.mom_init = np.zeros(max(self.n, 1), np.uint8)
        s = Store()
        s.mode = mode
        s.n_tensors = self.n
        s.tensors = C.cast(self._tensors, C.POINTER(Tensor))
        s.total = self.total
        s.param = _ptr(self.param)
        s.grad = _ptr(self.grad)
        s.master = _ptr(self.master, C.c_float)
        s.exp_avg = _ptr(self.exp_avg, C.c_float)
        s.exp_avg_sq = _ptr(self.exp_avg_sq, C.c_float)
        s.momentum = _ptr(self.momentum, C.c_float)
        s.mom_init = _ptr(self.mom_init, C.c_uint8)
        s.scaler_enabled = 0
        s.growth_interval = 2000
        s.growth_factor = 2.0
        s.backoff_factor = 0.5
        s.scale = 65536.0
        s.growth_tracker = 0
        s.t = 0
        s.nthreads = nthreads or (os.cpu_count() or 1)
        self.s = s

    # ---- views -------------------------------------------------------------------------
    def view(self, which, i):
        o, n = int(self.offsets[i]), self.numels[i]
        return getattr(self, which)[o:o + n]

    def set_master(self, i, x):
        self.view("master", i)[:] = np.asarray(x, np.float32).ravel()
        if self.mode == MODE_MIXED:
            self.view("param", i)[:] = bf16_rne(self.view("master", i))

    def set_grad(self, i, g):
        """g: float32 values (FP32) or uint16 bf16 bits (MIXED, BF16)."""
        dst = self.view("grad", i)
        dst[:] = np.asarray(g).ravel().astype(dst.dtype, copy=False)
        self._tensors[i].has_grad = 1

    def accumulate_grad(self, i, g):
        """g: float32 values or uint16 bf16 bits (any mode)."""
        a = np.ascontiguousarray(g).ravel()
        if a.dtype != np.uint16:
            a = a.astype(np.float32)
        assert a.size == self.numels[i]
        lib().orc_accumulate_grad(C.byref(self.s), i, _ptr(a), 1 if a.dtype == np.uint16 else 0)

    def set_has_grad(self, i, has):
        self._tensors[i].has_grad = 1 if has else 0

    def has_grad(self, i):
        return bool(self._tensors[i].has_grad)

    def zero_grad(self, set_to_none=True, fill=True):
        """fill=False (with set_to_none): the flags only, the values stay."""
        if fill:
            self.grad[:] = 0
        if set_to_none:
            for i in range(self.n):
                self._tensors[i].has_grad = 0

    # ---- scaler / counters -----------------------------------------------------------------
    def configure_scaler(self, enabled=True, init_scale=65536.0, growth_factor=2.0,
                         backoff_factor=0.5, growth_interval=2000):
        self.s.scaler_enabled = 1 if enabled else 0
        self.s.scale = init_scale
        self.s.growth_factor = growth_factor
        self.s.backoff_factor = backoff_factor
        self.s.growth_interval = growth_interval
        self.s.growth_tracker = 0
        self.s.pending = 0

    @property
    def t(self):
        return int(self.s.t)

    @t.setter
    def t(self, v):
        self.s.t = int(v)

    @property
    def scale(self):
        return float(self.s.scale)

    @property
    def growth_tracker(self):
        return int(self.s.growth_tracker)

    def set_scaler_state(self, scale, tracker):
        self.s.scale = scale
        self.s.growth_tracker = tracker
        self.s.pending = 0

    def scaler_update(self):
        """The scale update after steps that all deferred it (update_scale=False); nothing
        if no step deferred it since the last update."""
        lib().orc_scaler_update_pending(C.byref(self.s))

    # ---- steps -----------------------------------------------------------------------------
    def adam_step(self, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                  decoupled=True, max_grad_norm=0.0, opbyop=False, update_scale=True):
        hp = AdamHP(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=weight_decay,
                    decoupled=1 if decoupled else 0, flags=0 if update_scale else DEFER_SCALE,
                    max_grad_norm=max_grad_norm)
        rep = Report()
        fn = lib().orc_adam_step_opbyop if opbyop else lib().orc_adam_step
        rc = fn(C.byref(self.s), C.byref(hp), C.byref(rep))
        if rc != 0:
            raise ValueError(f"oracle adam_step rejected arguments (rc={rc})")
        return rep.as_dict()

    def sgd_step(self, lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False,
                 max_grad_norm=0.0, update_scale=True):
        hp = SgdHP(lr=lr, momentum=momentum, dampening=dampening, weight_decay=weight_decay,
                   nesterov=1 if nesterov else 0, flags=0 if update_scale else DEFER_SCALE,
                   max_grad_norm=max_grad_norm)
        rep = Report()
        rc = lib().orc_sgd_step(C.byref(self.s), C.byref(hp), C.byref(rep))
        if rc != 0:
            raise ValueError(f"oracle sgd_step rejected arguments (rc={rc})")
        return rep.as_dict()

    def grad_sumsq(self, inv_scale=1.0):
        fi = C.c_int32(0)
        v = lib().orc_grad_sumsq(C.byref(self.s), inv_scale, C.byref(fi))
        return v, bool(fi.value)
