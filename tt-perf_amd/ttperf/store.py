"""Flat parameter store: the host-side owner of one libttperf_hip context.

Replaces the per-parameter tensors the reference's optimizers walk (py/engine.py:74-156
`Tensor.tt` / `Tensor.grad`; autograd/dynamic/autograd.hpp:38-84 `Value::data` / `grad`) with
views into flat HBM buffers: each `Tensor` here is (store, index) and its data lives at
`offset` of the store's param and grad buffers.  The fp32 optimizer state (master, m, v in
mixed precision; m, v in fp32 mode) is interleaved in records of 64-element slots;
upload/download convert it to and from contiguous arrays, and ParamStore.layout() gives its
device addressing.
"""
from __future__ import annotations

import ctypes as C
import gc
import math
import weakref

import numpy as np

from . import _lib as L


def _is_torch(x):
    return type(x).__module__.startswith("torch")


def _bf16_bits_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_value(x):
    """The float x rounded to bf16 (nearest even), as a Python float."""
    return float(_bf16_bits_to_f32(_f32_to_bf16_bits(np.float32(x)))[0])


def _f32_to_bf16_bits(x):
    """float32 values -> bf16 bit patterns, rounded to nearest even (NaN -> 0x7FC0)."""
    u = np.ascontiguousarray(x, np.float32).ravel().view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(np.asarray(x, np.float32).ravel()), np.uint16(0x7FC0), r)


class Tensor:
    """A parameter: a view of one tensor of a ParamStore.

    `grad` is None (py/engine.py:141 `grad = None`) until a gradient is written; assigning an
    array uploads it, assigning None is the reference's `zero_grad` for this parameter.
    """

    def __init__(self, store: "ParamStore", index: int, shape, name: str = ""):
        self.store = store
        self.index = index
        self.shape = tuple(int(s) for s in shape)
        self.numel = int(math.prod(self.shape)) if self.shape else 1
        self.name = name
        self.requires_grad = True

    def __repr__(self):
        return f"Tensor(shape={self.shape}, requires_grad=True, index={self.index})"

    @property
    def decay(self) -> bool:
        return bool(self.store.flags[self.index] & L.TENSOR_DECAY)

    # ---- gradient ------------------------------------------------------------------------
    @property
    def grad(self):
        return GradView(self) if self.store.has_grad(self.index) else None

    @grad.setter
    def grad(self, value):
        if value is None:
            self.store.set_has_grad(self.index, False)
        else:
            self.store.upload(L.BUF_GRAD, self.index, value)

    def zero_grad(self):
        self.grad = None

    def accumulate_grad(self, value, sums=False):
        """py/engine.py:149-156 `_add_grad`: grad = value if grad is None else grad + value,
        summed in fp32 and rounded once to the grad buffer's type (bf16 in MIXED mode).
        sums=True also stores this tensor's gradient sum of squares for a tensor_sums step
        (TTP_ACCUM_SUMSQ)."""
        self.store.accumulate_grad(self.index, value, sums=sums)

    # ---- data ----------------------------------------------------------------------------
    def numpy(self):
        """Model-facing weights as float32 (bf16 widened in MIXED and BF16 mode)."""
        x = self.store.download(L.BUF_PARAM, self.index)
        if self.store.mode != L.MODE_FP32:
            x = _bf16_bits_to_f32(x)
        return x.reshape(self.shape)

    def master(self):
        return self.store.download(L.BUF_MASTER, self.index).reshape(self.shape)

    def set_data(self, value):
        """fp32 values -> master (and the bf16 copy in MIXED mode); in BF16 mode, the bf16
        weights (rounded to nearest even)."""
        if self.store.mode == L.MODE_BF16:
            self.store.upload(L.BUF_PARAM, self.index, _f32_to_bf16_bits(value))
            return
        self.store.upload(L.BUF_MASTER, self.index, value)

    def data_ptr(self, which=L.BUF_PARAM):
        return self.store.ptr(which, self.index)

    def torch_view(self, which=L.BUF_PARAM):
        """A torch tensor of this tensor's shape aliasing its slice of the store's buffer
        `which` (no copy): the weights a torch forward reads (BUF_PARAM), or the gradients a
        torch backward accumulates into (BUF_GRAD).  See ParamStore.torch_view."""
        return self.store.torch_view(which, self.index).view(self.shape)


Parameter = Tensor


class GradView:
    def __init__(self, p: Tensor):
        self.p = p

    def numpy(self):
        x = self.p.store.download(L.BUF_GRAD, self.p.index)
        if self.p.store.mode != L.MODE_FP32:
            x = _bf16_bits_to_f32(x)
        return x.reshape(self.p.shape)

    def data_ptr(self):
        return self.p.store.ptr(L.BUF_GRAD, self.p.index)


# Stream capture forbids HIP calls that free memory or synchronise on the capturing thread
# (they invalidate the capture).  Python may run a finalizer at any allocation (cyclic GC), so
# while any store is capturing, stores and graphs that get closed are destroyed only after
# the capture ends, and the cyclic collector is paused.
_capturing = 0
_gc_was_enabled = True
_deferred = []


def _capture_started():
    global _capturing, _gc_was_enabled
    if _capturing == 0:
        _gc_was_enabled = gc.isenabled()
        gc.disable()
    _capturing += 1


def _capture_ended():
    global _capturing
    _capturing -= 1
    if _capturing == 0:
        if _gc_was_enabled:
            gc.enable()
        while _deferred:
            _deferred.pop().close()


class StepGraph:
    """A captured hipGraph of a store's work (ttp_capture_begin .. ttp_capture_end).

    It remembers which optimizer held the store's step count at capture and hands the count
    back to it before each replay (a no-op unless another optimizer stepped the store since),
    so the replayed steps use that optimizer's own count."""

    def __init__(self, store: "ParamStore", handle):
        self.store = store
        self._g = handle
        self._owner = store._t_owner

    def replay(self):
        owner = self._owner() if self._owner is not None else None
        if owner is not None:
            owner._claim(self.store)
        L.check(L.lib.ttp_graph_launch(self._g))

    def close(self):
        if getattr(self, "_g", None):
            if _capturing:
                _deferred.append(self)
                return
            L.lib.ttp_graph_destroy(self._g)
            self._g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TraceContext:
    """autograd/traced/trace.hpp:21-88 over a store: the first run(fn) captures what fn
    queues on the store's stream (its optimizer steps, zero_grad, device transfers) and
    executes it once; later calls replay the graph."""

    def __init__(self, store: "ParamStore"):
        self.store = store
        self.graph = None

    def run(self, fn):
        if self.graph is None:
            self.store.begin_capture()
            try:
                fn()
            except BaseException:
                self.store.end_capture(discard=True)
                raise
            self.graph = self.store.end_capture()
        self.graph.replay()

    def is_captured(self):
        return self.graph is not None

    def release(self):
        if self.graph is not None:
            self.graph.close()
            self.graph = None

    reset = release


class ParamStore:
    """One context: tensors laid out 64-element aligned in caller order.

    shapes : list of shapes (tuples) or element counts
    mode   : "fp32" (fp32 params/grads, params are the master copy),
             "mixed" (bf16 params/grads + fp32 master, m, v) or
             "bf16" (bf16 params/grads only, the reference C++ autograd's tensors: plain SGD
             with each op rounded to bf16; Adam and SGD with momentum or decay refuse)
    decay  : per-tensor bools (weight decay applies), default: tensors with >= 2 dims
    layout : "default", or "sgd": a mixed store for SGD, with a contiguous fp32 master and no
             m / v (TTP_STORE_SGD; the first Adam step converts it to the default layout)
    """

    def __init__(self, shapes, *, mode="fp32", decay=None, names=None, device=0,
                 layout="default"):
        shapes = [tuple(s) if isinstance(s, (tuple, list)) else (int(s),) for s in shapes]
        if mode not in ("fp32", "mixed", "bf16"):
            raise ValueError("mode must be 'fp32', 'mixed' or 'bf16'")
        if layout not in ("default", "sgd"):
            raise ValueError("layout must be 'default' or 'sgd'")
        self.mode = {"fp32": L.MODE_FP32, "mixed": L.MODE_MIXED, "bf16": L.MODE_BF16}[mode]
        if decay is None:
            decay = [len(s) >= 2 for s in shapes]
        self.flags = [L.TENSOR_DECAY if d else 0 for d in decay]
        n = len(shapes)
        descs = (L.TensorDesc * max(n, 1))()
        for i, s in enumerate(shapes):
            descs[i].numel = int(math.prod(s)) if s else 1
            descs[i].flags = self.flags[i]
        h = C.c_void_p()
        create_mode = self.mode | (L.STORE_SGD if layout == "sgd" else 0)
        L.check(L.lib.ttp_create(device, descs, n, create_mode, C.byref(h)))
        self._h = h
        self.device = device
        names = names or [f"p{i}" for i in range(n)]
        self.tensors = [Tensor(self, i, s, names[i]) for i, s in enumerate(shapes)]
        self.offsets = []
        for i in range(n):
            off = C.c_uint64()
            L.check(L.lib.ttp_tensor_info(self._h, i, C.byref(off), None, None))
            self.offsets.append(off.value)
        tot = C.c_uint64()
        L.check(L.lib.ttp_flat_numel(self._h, C.byref(tot)))
        self.total = tot.value
        self._graphs = weakref.WeakSet()
        self._in_capture = False
        self._t_owner = None  # weakref to the optimizer whose step count the store holds
        self._stream_obj = None  # the adopted stream (set_stream), kept alive while in use

    # ---- lifetime --------------------------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            if getattr(self, "_in_capture", False):
                # closing a capturing store discards its capture first, which also resumes
                # the collector and the deferred closes the capture paused
                self.end_capture(discard=True)
            if _capturing:
                _deferred.append(self)  # another store is capturing: destroyed when it ends
                return
            for g in list(getattr(self, "_graphs", ())):
                g.close()  # a context's graphs go before the context
            L.lib.ttp_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def parameters(self):
        return list(self.tensors)

    def set_stream(self, stream):
        """Queue all work on a torch.cuda.Stream or a raw hipStream_t (int; 0 is the legacy
        default stream); None returns to the context's own stream."""
        if stream is None:
            L.check(L.lib.ttp_reset_stream(self._h))
            self._stream_obj = None
            return
        handle = stream.cuda_stream if hasattr(stream, "cuda_stream") else stream
        L.check(L.lib.ttp_set_stream(self._h, C.c_void_p(int(handle))))
        # the store queues work on this stream until it moves or closes: keep the object
        # (a torch.cuda.Stream, say) alive as long
        self._stream_obj = stream

    def sync(self):
        L.check(L.lib.ttp_sync(self._h))

    # ---- buffers -----------------------------------------------------------------------------
    def ptr(self, which, index=L.ALL_TENSORS):
        """Device address of a contiguously stored buffer (PARAM, GRAD, MOMENTUM; MASTER in
        FP32 mode and in the SGD layout); the interleaved optimizer state raises (see
        layout())."""
        p = C.c_void_p()
        L.check(L.lib.ttp_buffer_ptr(self._h, which, index, C.byref(p)))
        return p.value

    @property
    def sgd_layout(self):
        """Whether the master is contiguous because of the SGD layout (a mixed store created
        with layout="sgd" that no Adam step has converted yet)."""
        if self.mode != L.MODE_MIXED:
            return False
        return self.layout(L.BUF_MASTER)[2] == 64

    def layout(self, which):
        """(base, group, stride): flat element e of `which` sits at
        base + (e // group * stride + e % group) * element_size."""
        p, g, s = C.c_void_p(), C.c_uint32(), C.c_uint32()
        L.check(L.lib.ttp_buffer_layout(self._h, which, C.byref(p), C.byref(g), C.byref(s)))
        return p.value, g.value, s.value

    def _esize(self, which):
        if which in (L.BUF_PARAM, L.BUF_GRAD) and self.mode != L.MODE_FP32:
            return 2
        return 4

    def _numel(self, index):
        return self.total if index == L.ALL_TENSORS else self.tensors[index].numel

    def _host_dtype(self, which):
        return np.uint16 if self._esize(which) == 2 else np.float32

    def upload(self, which, index, value):
        """numpy (host) or torch (host or device) data.  For 2-byte buffers pass bf16 as
        uint16 bits (numpy) or torch.bfloat16; float32 values are rounded by torch/numpy
        callers, never here."""
        n = self._numel(index)
        if _is_torch(value):
            if value.is_cuda and self._in_capture:
                self._check_captured_tensor(value, n, which)
                # a captured copy, ordered on the store's stream: nothing synchronises here
                L.check(L.lib.ttp_upload(self._h, which, index, C.c_void_p(value.data_ptr()), n,
                                         L.DEVICE))
                return
            t = value.detach().contiguous()
            if t.numel() != n:
                raise ValueError(f"expected {n} elements, got {t.numel()}")
            if t.element_size() != self._esize(which):
                raise ValueError("element size does not match the buffer's type")
            kind = L.DEVICE if t.is_cuda else L.HOST
            if t.is_cuda:
                import torch
                torch.cuda.current_stream(t.device).synchronize()
            L.check(L.lib.ttp_upload(self._h, which, index, C.c_void_p(t.data_ptr()), n, kind))
            if t.is_cuda:
                self.sync()  # `t` may be freed and reused by torch as soon as we return
            return
        a = np.asarray(value)
        want = self._host_dtype(which)
        if a.dtype != want:
            if want == np.uint16:
                raise ValueError("bf16 buffers take uint16 bit patterns from numpy")
            a = a.astype(np.float32)
        a = np.ascontiguousarray(a).ravel()
        if a.size != n:
            raise ValueError(f"expected {n} elements, got {a.size}")
        L.check(L.lib.ttp_upload(self._h, which, index, a.ctypes.data_as(C.c_void_p), n, L.HOST))

    def _check_captured_tensor(self, t, n, which):
        """While capturing, a device transfer becomes a copy node that reads or writes `t`'s
        memory at every launch of the graph: `t` itself must be contiguous, of the buffer's
        element count and size, and kept alive (and ordered on the store's stream) by the
        caller for as long as the graph is launched."""
        if t.numel() != n or t.element_size() != self._esize(which) or not t.is_contiguous():
            raise ValueError(f"a captured transfer needs a contiguous device tensor of {n} "
                             f"elements of {self._esize(which)} bytes, used in place")

    def download(self, which, index=L.ALL_TENSORS, out=None):
        """The buffer's elements (bf16 as uint16 bits), into a new numpy array or into `out`:
        a contiguous, writable numpy array or torch tensor (host or device) of exactly the
        element count and element size, which the ABI fills in place."""
        n = self._numel(index)
        if out is not None and _is_torch(out) and out.is_cuda and self._in_capture:
            self._check_captured_tensor(out, n, which)
            L.check(L.lib.ttp_download(self._h, which, index, C.c_void_p(out.data_ptr()), n,
                                       L.DEVICE))
            return out
        if out is not None and _is_torch(out):
            if out.numel() != n or out.element_size() != self._esize(which) or \
                    not out.is_contiguous():
                raise ValueError(f"out must be a contiguous tensor of {n} elements of "
                                 f"{self._esize(which)} bytes")
            kind = L.DEVICE if out.is_cuda else L.HOST
            if out.is_cuda:
                import torch
                torch.cuda.current_stream(out.device).synchronize()
            L.check(L.lib.ttp_download(self._h, which, index, C.c_void_p(out.data_ptr()), n, kind))
            if kind == L.DEVICE:
                self.sync()
            return out
        if out is None:
            a = np.empty(n, self._host_dtype(which))
        else:
            a = out
            if not isinstance(a, np.ndarray) or a.dtype != self._host_dtype(which) or \
                    a.size != n or not a.flags.c_contiguous or not a.flags.writeable:
                dt = self._host_dtype(which).__name__
                raise ValueError(f"out must be a contiguous, writable {dt} array of {n} elements")
        L.check(L.lib.ttp_download(self._h, which, index, a.ctypes.data_as(C.c_void_p), n, L.HOST))
        return a

    # ---- grads ---------------------------------------------------------------------------------
    def has_grad(self, index):
        h = C.c_int()
        L.check(L.lib.ttp_get_has_grad(self._h, index, C.byref(h)))
        return bool(h.value)

    def set_has_grad(self, index, has):
        L.check(L.lib.ttp_set_has_grad(self._h, index, 1 if has else 0))

    def mark_grads(self, indices=None):
        """Record that grads were written outside the ABI (through torch_view(BUF_GRAD) or a
        device pointer): the listed tensors, or all, now have a grad."""
        for i in range(len(self.tensors)) if indices is None else indices:
            self.set_has_grad(i, True)

    def torch_view(self, which=L.BUF_PARAM, index=L.ALL_TENSORS):
        """Zero-copy torch tensor over a contiguously stored buffer (PARAM, GRAD, MOMENTUM;
        MASTER in fp32 mode): the whole flat buffer, or one tensor's slice as a 1-D tensor.
        bf16 buffers come back as torch.bfloat16.  The view aliases the store's memory for the
        store's lifetime.  Torch work on it is ordered on torch's current stream and the
        store's on its own: share one stream (set_stream(torch.cuda.current_stream())) or
        synchronise between them.  Writes to BUF_GRAD through a view need mark_grads()."""
        import torch
        ptr = self.ptr(which, index)
        n = self._numel(index)
        two = self._esize(which) == 2
        if n == 0:
            return torch.empty(0, dtype=torch.bfloat16 if two else torch.float32,
                               device=f"cuda:{self.device}")

        class _Device:  # the CUDA array interface torch wraps without copying
            __cuda_array_interface__ = {"data": (ptr, False), "shape": (n,),
                                        "typestr": "<u2" if two else "<f4", "strides": None,
                                        "version": 3}

        t = torch.as_tensor(_Device(), device=f"cuda:{self.device}")
        if t.data_ptr() != ptr:
            raise RuntimeError("torch copied the buffer instead of wrapping it")
        return t.view(torch.bfloat16) if two else t

    def zero_grad(self, set_to_none=True, indices=None, fill=True):
        """Zero every grad (one fill), or only the listed tensors' grads (one launch);
        set_to_none also marks them as having no grad.  set_to_none=False leaves the has-grad
        flags alone, as torch's zero_grad(set_to_none=False) does: a tensor without a grad
        stays without one (mark_grads() marks zeroed grads present).  fill=False (with
        set_to_none): the flags only, as the reference's `grad = None` touches no memory; the
        gradients keep their old contents until written (TTP_ZERO_NO_FILL)."""
        mode = (1 if set_to_none else 0) | (0 if fill else L.ZERO_NO_FILL)
        if indices is None:
            L.check(L.lib.ttp_zero_grad(self._h, mode))
            return
        idx, n = self._index_array(indices)
        L.check(L.lib.ttp_zero_grad_subset(self._h, idx, n, mode))

    def accumulate_grad(self, index, value, sums=False):
        """Add an incoming gradient (numpy float32 / uint16 bf16 bits, or a torch float32 /
        bfloat16 tensor on the host or the GPU) into tensor `index`'s grad.  sums=True: the
        same launch also stores the sum of squares of the tensor's resulting (unscaled)
        gradients, as grad_sumsq_tensors([index]) would, bit for bit, so that a step with
        tensor_sums=True needs no pass over them (TTP_ACCUM_SUMSQ)."""
        n = self.tensors[index].numel
        flag = L.ACCUM_SUMSQ if sums else 0
        if _is_torch(value):
            import torch
            if value.dtype not in (torch.float32, torch.bfloat16):
                raise ValueError("incoming gradients must be float32 or bfloat16")
            dtype = L.DTYPE_BF16 if value.dtype == torch.bfloat16 else L.DTYPE_F32
            if value.is_cuda and self._in_capture:
                # captured: the graph reads `value` in place at every launch (see
                # _check_captured_tensor); nothing synchronises here
                if value.numel() != n or not value.is_contiguous():
                    raise ValueError(f"a captured accumulate needs a contiguous device tensor "
                                     f"of {n} elements, used in place")
                L.check(L.lib.ttp_accumulate_grad(self._h, index, C.c_void_p(value.data_ptr()),
                                                  n, dtype | flag, L.DEVICE))
                return
            t = value.detach().contiguous()
            if t.numel() != n:
                raise ValueError(f"expected {n} elements, got {t.numel()}")
            if t.is_cuda:
                torch.cuda.current_stream(t.device).synchronize()
            L.check(L.lib.ttp_accumulate_grad(self._h, index, C.c_void_p(t.data_ptr()), n,
                                              dtype | flag, L.DEVICE if t.is_cuda else L.HOST))
            if t.is_cuda:
                self.sync()  # `t` may be freed and reused by torch as soon as we return
            return
        a = np.asarray(value)
        if a.dtype == np.uint16:
            dtype = L.DTYPE_BF16
        else:
            a = a.astype(np.float32, copy=False)
            dtype = L.DTYPE_F32
        a = np.ascontiguousarray(a).ravel()
        if a.size != n:
            raise ValueError(f"expected {n} elements, got {a.size}")
        L.check(L.lib.ttp_accumulate_grad(self._h, index, a.ctypes.data_as(C.c_void_p), n,
                                          dtype | flag, L.HOST))

    def accumulate_grads(self, indices, values, sums=False):
        """Several tensors' incoming gradients in one launch (ttp_accumulate_grad_multi), as a
        backward hands over a bucket: tensor indices[k] receives values[k], a contiguous
        float32 or bfloat16 torch tensor on the GPU (one dtype for the call), exactly as
        accumulate_grad(indices[k], values[k], sums) would.  At most ACCUM_MULTI_MAX tensors
        per call.  While capturing, the graph reads each value in place at every launch."""
        import torch
        indices = [int(i) for i in indices]
        if len(values) != len(indices):
            raise ValueError("one value per index")
        dtypes = {v.dtype for v in values}
        if not dtypes <= {torch.float32, torch.bfloat16} or len(dtypes) > 1:
            raise ValueError("incoming gradients must be all float32 or all bfloat16")
        dtype = L.DTYPE_BF16 if dtypes == {torch.bfloat16} else L.DTYPE_F32
        for i, v in zip(indices, values):
            # an index out of range is the library's to refuse (TTP_ERR_RANGE), as for a list
            # that names a tensor twice
            if 0 <= i < len(self.tensors) and not (
                    _is_torch(v) and v.is_cuda and v.is_contiguous()
                    and v.numel() == self.tensors[i].numel):
                raise ValueError(f"tensor {i}: a contiguous device tensor of "
                                 f"{self.tensors[i].numel} elements is needed")
        if not self._in_capture and values:
            torch.cuda.current_stream(values[0].device).synchronize()
        n = len(indices)
        idx = (C.c_uint32 * max(n, 1))(*indices)
        ptrs = (C.c_void_p * max(n, 1))(*[v.data_ptr() for v in values])
        L.check(L.lib.ttp_accumulate_grad_multi(self._h, idx, ptrs, n,
                                                dtype | (L.ACCUM_SUMSQ if sums else 0)))
        if not self._in_capture:
            self.sync()  # the values may be freed and reused by torch as soon as we return

    # ---- steps -----------------------------------------------------------------------------------
    @staticmethod
    def _index_array(indices):
        if indices is None:
            return None, 0
        idx = (C.c_uint32 * max(len(indices), 1))(*[int(i) for i in indices])
        return idx, len(indices)

    @staticmethod
    def _step_flags(tensor_sums, update_scale):
        return ((L.STEP_TENSOR_SUMS if tensor_sums else 0)
                | (0 if update_scale else L.STEP_DEFER_SCALE))

    def adam_step(self, lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, decoupled=True,
                  max_grad_norm=None, report=False, indices=None, tensor_sums=False,
                  update_scale=True):
        """One Adam/AdamW step over every tensor with a grad, or only over `indices`.
        tensor_sums: take the norm from grad_sumsq_tensors() instead of a norm pass.
        update_scale=False (loss scaling on): leave the loss scale to the iteration's last
        step or to scaler_update(), as GradScaler.step does for one of several optimizers."""
        hp = L.AdamHParams(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
                           weight_decay=weight_decay, decoupled=1 if decoupled else 0,
                           flags=self._step_flags(tensor_sums, update_scale),
                           max_grad_norm=max_grad_norm or 0.0)
        rep = L.StepReport() if report else None
        rp = C.byref(rep) if report else None
        idx, n = self._index_array(indices)
        if idx is None:
            L.check(L.lib.ttp_adam_step(self._h, C.byref(hp), rp))
        else:
            L.check(L.lib.ttp_adam_step_subset(self._h, C.byref(hp), idx, n, rp))
        return rep.as_dict() if report else None

    def sgd_step(self, lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False,
                 max_grad_norm=None, report=False, indices=None, tensor_sums=False,
                 update_scale=True):
        """One SGD step over every tensor with a grad, or only over `indices`.
        tensor_sums and update_scale as in adam_step."""
        hp = L.SgdHParams(lr=lr, momentum=momentum, dampening=dampening,
                          weight_decay=weight_decay, nesterov=1 if nesterov else 0,
                          flags=self._step_flags(tensor_sums, update_scale),
                          max_grad_norm=max_grad_norm or 0.0)
        rep = L.StepReport() if report else None
        rp = C.byref(rep) if report else None
        idx, n = self._index_array(indices)
        if idx is None:
            L.check(L.lib.ttp_sgd_step(self._h, C.byref(hp), rp))
        else:
            L.check(L.lib.ttp_sgd_step_subset(self._h, C.byref(hp), idx, n, rp))
        return rep.as_dict() if report else None

    def grad_sumsq_tensors(self, indices=None):
        """Per-tensor sums of squares of the listed tensors' grads (all when None), kept on the
        device for the next step with tensor_sums=True: a bucket's norm work, done once its
        grads are final, so the step itself runs no norm pass."""
        if indices is None:
            indices = range(len(self.tensors))
        idx, n = self._index_array(list(indices))
        L.check(L.lib.ttp_grad_sumsq_tensors(self._h, idx, n))

    def grad_norm(self):
        v = C.c_double()
        L.check(L.lib.ttp_grad_norm(self._h, C.byref(v)))
        return v.value

    # ---- step count / loss scaler ---------------------------------------------------------------
    @property
    def step_count(self):
        v = C.c_uint64()
        L.check(L.lib.ttp_get_step(self._h, C.byref(v)))
        return v.value

    @step_count.setter
    def step_count(self, t):
        L.check(L.lib.ttp_set_step(self._h, int(t)))

    def configure_scaler(self, enabled=True, init_scale=2.0 ** 16, growth_factor=2.0,
                         backoff_factor=0.5, growth_interval=2000):
        cfg = L.ScalerConfig(enabled=1 if enabled else 0, growth_interval=growth_interval,
                             init_scale=init_scale, growth_factor=growth_factor,
                             backoff_factor=backoff_factor)
        L.check(L.lib.ttp_scaler_configure(self._h, C.byref(cfg)))

    def scaler_state(self):
        s, t = C.c_float(), C.c_int32()
        L.check(L.lib.ttp_scaler_get(self._h, C.byref(s), C.byref(t)))
        return s.value, t.value

    def set_scaler_state(self, scale, growth_tracker):
        L.check(L.lib.ttp_scaler_set(self._h, scale, growth_tracker))

    def scaler_update(self):
        """GradScaler.update() for an iteration whose steps all passed update_scale=False:
        back off if any of them saw an overflow, else count a clean step toward growth.
        Nothing happens when no step deferred the update since the last one."""
        L.check(L.lib.ttp_scaler_update(self._h))

    # ---- optimizer-state checkpoint ---------------------------------------------------------
    def save_state(self, path):
        """Write master weights, moments, momentum, step count and scaler state to `path`."""
        L.check(L.lib.ttp_save_state(self._h, str(path).encode()))

    def load_state(self, path):
        """Restore a save_state() file written for the same tensor table and mode."""
        L.check(L.lib.ttp_load_state(self._h, str(path).encode()))

    # ---- graph capture ------------------------------------------------------------------------
    def begin_capture(self):
        """Capture the store's work until end_capture() (the store must use its own stream
        or a created stream, not the legacy default stream)."""
        L.check(L.lib.ttp_capture_begin(self._h))
        self._in_capture = True
        _capture_started()

    def end_capture(self, discard=False):
        g = C.c_void_p()
        try:
            rc = L.lib.ttp_capture_end(self._h, None if discard else C.byref(g))
        finally:
            if self._in_capture:
                self._in_capture = False
                _capture_ended()
        L.check(rc)
        if discard:
            return None
        graph = StepGraph(self, g)
        self._graphs.add(graph)
        return graph

    # ---- timing -----------------------------------------------------------------------------------
    def timing(self, on=True):
        L.check(L.lib.ttp_timing_enable(self._h, 1 if on else 0))

    def timing_collect(self, kernel):
        ms, n = C.c_double(), C.c_uint64()
        L.check(L.lib.ttp_timing_collect(self._h, kernel, C.byref(ms), C.byref(n)))
        return ms.value, n.value
