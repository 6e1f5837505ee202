"""ttperf — MI355X (gfx950) optimizer-step engine for csirak/tt-perf's autograd.

Python host side of libttperf_hip: a flat parameter store (`ParamStore`, `Tensor`) and the
optimizers of the reference's py/optim.py (`SGD`, `Adam`) plus `AdamW`, each step a single
multi-tensor HIP launch.  Importing fails if the HIP library is not built.
"""
from . import _lib
from ._lib import (ALL_TENSORS, BUF_EXP_AVG, BUF_EXP_AVG_SQ, BUF_GRAD, BUF_MASTER,
                   BUF_MOMENTUM, BUF_PARAM, TTPError, TTPMemoryError, TTPValueError,
                   device_count)
from .optim import SGD, Adam, AdamW
from .store import GradView, Parameter, ParamStore, StepGraph, Tensor, TraceContext

__all__ = ["SGD", "Adam", "AdamW", "ParamStore", "Tensor", "Parameter", "GradView",
           "StepGraph", "TraceContext",
           "TTPError", "TTPValueError", "TTPMemoryError", "device_count", "_lib",
           "BUF_PARAM", "BUF_GRAD", "BUF_MASTER", "BUF_EXP_AVG", "BUF_EXP_AVG_SQ",
           "BUF_MOMENTUM", "ALL_TENSORS"]
