"""Optimizers with the interface of the reference's py/optim.py, stepping flat stores.

SGD   — py/optim.py:6-27 (`SGD(params, *, lr)`, ValueError on lr <= 0 and on non-Tensor
        params, skips params whose grad is None, `zero_grad` sets grads to None), extended
        with momentum / dampening / nesterov / weight_decay (torch.optim.SGD semantics).  On a
        BF16 store (the reference's bf16 tensors) lr is rounded to bf16 first, as
        py/optim.py:19's full_like fill of the gradient's dtype rounds it.
Adam  — py/optim.py:30-92 (`Adam(params, *, lr=1e-3, betas=(0.9, 0.999), eps=1e-8)`, the
        same validation, a step count that advances on every step() call, bias corrections
        in host double), extended with weight_decay (L2) and max_grad_norm.
AdamW — Adam with decoupled weight decay (p *= 1 - lr*wd before the update), applied only
        to the store's decay-flagged tensors.

Each optimizer counts its own steps, as py/optim.py:46,50 keeps `_step` per Adam, although
the count the kernels read lives in the store: when a different live optimizer stepped a
store last, its count is saved and this optimizer's restored (one synchronising read and
one write, on a change of owner only), so two optimizers over two parameter groups of one
store see the bias corrections of their own step counts.

Every step is one libttperf_hip call per store: one multi-tensor launch (plus the norm pass
when clipping or loss scaling), instead of ~15 elementwise programs per tensor.
"""
from __future__ import annotations

import weakref

from . import _lib as L
from .store import Tensor, bf16_value


def _group_by_store(params, what):
    groups = {}
    for p in params:
        if not isinstance(p, Tensor):
            raise ValueError(f"{what} expects Tensor parameters")
        groups.setdefault(id(p.store), (p.store, []))[1].append(p)
    return list(groups.values())


class _Optimizer:
    _name = "Optimizer"

    def __init__(self, params):
        self.params = list(params)
        self._saved_t = weakref.WeakKeyDictionary()  # store -> this optimizer's step count

    def _stores(self):
        return _group_by_store(self.params, self._name)

    def _claim(self, store):
        """Make the store's step count this optimizer's before it steps the store.

        A store that no live optimizer stepped last keeps its count (a loaded checkpoint's,
        say) for the optimizer that steps it next; one that a different live optimizer
        stepped last has that optimizer's count saved, and this optimizer's restored (0 if
        it never stepped the store)."""
        prev = store._t_owner() if store._t_owner is not None else None
        if prev is self:
            return
        if prev is not None or store in self._saved_t:
            if store._in_capture:
                raise RuntimeError(
                    "a second optimizer steps this store inside a graph capture; the step "
                    "count hand-over reads the device and cannot be captured")
            if prev is not None:
                prev._saved_t[store] = store.step_count
            store.step_count = self._saved_t.pop(store, 0)
        store._t_owner = weakref.ref(self)

    def zero_grad(self):
        # py/optim.py:89-92 -> Tensor.zero_grad (py/engine.py:141-142): grad = None, and
        # non-Tensor entries are skipped (step() is where they raise).  A store fully owned
        # by this optimizer is cleared with one fill (zeros + no grads).
        tensors = [p for p in self.params if isinstance(p, Tensor)]
        for store, members in _group_by_store(tensors, self._name):
            if len(members) == len(store.tensors):
                store.zero_grad(set_to_none=True)
            else:
                for p in members:
                    p.zero_grad()

    def step(self, tensor_sums=False, update_scale=True):
        """py/optim.py's step().  Extensions: tensor_sums=True takes the gradient norm from
        the sums ParamStore.grad_sumsq_tensors() took for these tensors, bucket by bucket
        during the backward, instead of a norm pass.  update_scale=False, for all but the last
        of several optimizers stepping one loss-scaled store in an iteration, leaves the loss
        scale to that last step (or to ParamStore.scaler_update()), as torch's
        GradScaler.step(opt) per optimizer followed by one GradScaler.update() does."""
        for store, members in self._stores():
            self._claim(store)
            whole = len(members) == len(store.tensors)
            self._step_store(store, None if whole else sorted({p.index for p in members}),
                             tensor_sums, update_scale)

    def _step_store(self, store, indices, tensor_sums, update_scale):  # pragma: no cover
        raise NotImplementedError


class SGD(_Optimizer):
    _name = "SGD"

    def __init__(self, params, *, lr: float, momentum: float = 0.0, dampening: float = 0.0,
                 weight_decay: float = 0.0, nesterov: bool = False, max_grad_norm=None):
        super().__init__(params)
        if lr <= 0:
            raise ValueError("lr must be > 0")
        if momentum < 0:
            raise ValueError("momentum must be >= 0")
        if weight_decay < 0:
            raise ValueError("weight_decay must be >= 0")
        if nesterov and (momentum <= 0 or dampening != 0):
            raise ValueError("nesterov requires momentum > 0 and zero dampening")
        self.lr = float(lr)
        self.momentum = float(momentum)
        self.dampening = float(dampening)
        self.weight_decay = float(weight_decay)
        self.nesterov = bool(nesterov)
        self.max_grad_norm = max_grad_norm

    def _step_store(self, store, indices, tensor_sums, update_scale):
        lr = self.lr
        if store.mode == L.MODE_BF16:
            # py/optim.py:19 fills lr into a tensor of the gradient's dtype (ttnn.full_like):
            # on the reference's bf16 tensors the product uses lr rounded to bf16
            lr = bf16_value(lr)
        store.sgd_step(lr, self.momentum, self.dampening, self.weight_decay,
                       self.nesterov, self.max_grad_norm, indices=indices,
                       tensor_sums=tensor_sums, update_scale=update_scale)


class Adam(_Optimizer):
    _name = "Adam"
    _decoupled = False

    def __init__(self, params, *, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, max_grad_norm=None):
        super().__init__(params)
        # py/optim.py:33-41
        if lr <= 0:
            raise ValueError("lr must be > 0")
        if eps <= 0:
            raise ValueError("eps must be > 0")
        if not isinstance(betas, (tuple, list)) or len(betas) != 2:
            raise ValueError("betas must be a tuple of (beta1, beta2)")
        beta1, beta2 = float(betas[0]), float(betas[1])
        if not (0.0 < beta1 < 1.0 and 0.0 < beta2 < 1.0):
            raise ValueError("betas must be in (0, 1)")
        if weight_decay < 0:
            raise ValueError("weight_decay must be >= 0")
        self.lr = float(lr)
        self.beta1 = beta1
        self.beta2 = beta2
        self.eps = float(eps)
        self.weight_decay = float(weight_decay)
        self.max_grad_norm = max_grad_norm

    def _step_store(self, store, indices, tensor_sums, update_scale):
        store.adam_step(self.lr, (self.beta1, self.beta2), self.eps, self.weight_decay,
                        self._decoupled, self.max_grad_norm, indices=indices,
                        tensor_sums=tensor_sums, update_scale=update_scale)


class AdamW(Adam):
    _name = "AdamW"
    _decoupled = True

    def __init__(self, params, *, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, max_grad_norm=None):
        super().__init__(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                         max_grad_norm=max_grad_norm)
