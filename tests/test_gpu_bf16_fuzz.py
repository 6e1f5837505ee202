"""Stateful differential fuzzing of a BF16 store (TTP_MODE_BF16: bf16 weights and gradients, no
fp32 state) against the CPU oracle, with the operations of tests/test_gpu_fuzz.py that such a
store takes, and the ones it refuses:

  gradients written flat or per tensor, from host or device memory (an occasional +inf while
  loss scaling is on); gradients accumulated from fp32 or bf16 sources, host or device, per
  tensor or in bucket calls, with or without their sums; `grad = None`; zero_grad of all or of
  a subset, to zeros or to None (with or without the fill); bf16 weight uploads; the
  reference's plain SGD over everything or a subset, with or without clipping and reports,
  deferring the scale update or not; steps from bucket sums and from a producer's sums (and
  their refusals after a gradient write); the loss scaler switched on or off; the step count
  set; the gradient norm probed; checkpoints saved and loaded; SGD steps, zero_grad calls and
  whole producer iterations (zero_grad, accumulates with sums, the SGD step from them)
  captured into graphs and replayed later with new sources; and the calls that need fp32 state (Adam through
  every entry point, SGD with momentum or weight decay), which must be refused with
  TTP_ERR_INVALID and change nothing.

After every operation the bf16 weights and the gradients are compared bit for bit, and the
has-grad flags, the step count and the loss-scaler state exactly; step reports must agree.
Every operation is printed before it runs.
"""
import os

import numpy as np
import pytest

import oracle as O
from test_gpu_fuzz import Case

pytestmark = pytest.mark.gpu

# 300 seeded cases of 50 operations by default; TTP_BF16_FUZZ_CASES=N runs N, from seed
# TTP_BF16_FUZZ_FIRST (5000)
_FIRST = int(os.environ.get("TTP_BF16_FUZZ_FIRST", "5000"))
SEEDS = list(range(_FIRST, _FIRST + int(os.environ.get("TTP_BF16_FUZZ_CASES", "300"))))
N_OPS = int(os.environ.get("TTP_FUZZ_OPS", "50"))


class Bf16Case(Case):
    def __init__(self, seed, tmp_path):
        super().__init__(seed, tmp_path, bf16=True)
        self.last_sgd = None  # (hp, indices, active set) of the last eager SGD step

    def _adam_ok(self, adam):
        return False

    def _sums_sgd_hp(self, lr, clip):
        return dict(lr=lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False,
                    max_grad_norm=clip)

    # a captured producer iteration ends with the reference's SGD from the producer's sums
    PRODUCER_KIND = "sgd"

    def _producer_hp(self, rng):
        return dict(lr=float(10 ** rng.uniform(-3, -1)), max_grad_norm=float(10 ** rng.uniform(-2, 1)))

    def _producer_step(self, indices, hp, report):
        return self.store.sgd_step(report=report, indices=indices, tensor_sums=True, **hp)

    def _plain_hp(self):
        rng = self.rng
        return dict(lr=float(10 ** rng.uniform(-3, -1)), momentum=0.0, dampening=0.0,
                    weight_decay=0.0, nesterov=False,
                    max_grad_norm=None if rng.random() < 0.5 else float(10 ** rng.uniform(-2, 1)))

    def op_upload_weights(self):
        from ttperf import _lib as L
        i = int(self.rng.integers(0, self.n))
        bits = O.bf16_rne((self.rng.standard_normal(self.numels[i]) * 0.05).astype(np.float32))
        print(f"  bf16 weights of tensor {i}", flush=True)
        self.store.upload(L.BUF_PARAM, i, bits)
        self.ref.view("param", i)[:] = bits

    def op_adam(self):
        """Adam through one of its entry points: refused, nothing changed."""
        import ctypes as C
        import ttperf
        from ttperf import _lib as L
        which = int(self.rng.integers(0, 4))
        print(f"  adam through entry point {which}: refused", flush=True)
        hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, decoupled=True)
        if which == 3:
            h = L.AdamHParams(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8)
            rc = L.lib.ttp_adam_step_noalloc(self.store.handle, C.byref(h), None, 0)
            assert rc == L.ERR_INVALID
            return
        with pytest.raises(ttperf.TTPValueError) as e:
            if which == 0:
                self.store.adam_step(**hp)
            elif which == 1:
                self.store.adam_step(indices=self.pick_subset(), report=True, **hp)
            else:
                self.store.adam_step(tensor_sums=True, max_grad_norm=1.0, **hp)
        assert e.value.code == L.ERR_INVALID

    def op_sgd(self):
        import ttperf
        from ttperf import _lib as L
        rng = self.rng
        hp = self._plain_hp()
        indices = None if rng.random() < 0.6 else self.pick_subset()
        report = rng.random() < 0.5
        defer = self.scaler_on and rng.random() < 0.3
        if rng.random() < 0.15:
            extra = [dict(momentum=0.9), dict(weight_decay=0.01),
                     dict(momentum=0.9, nesterov=True)][int(rng.integers(0, 3))]
            print(f"  sgd {dict(hp, **extra)}: refused", flush=True)
            with pytest.raises(ttperf.TTPValueError) as e:
                self.store.sgd_step(indices=indices, **dict(hp, **extra))
            assert e.value.code == L.ERR_INVALID
            return
        active = self._active(indices)
        print(f"  sgd {hp} indices={indices} active={active}"
              f"{' deferring the scale update' if defer else ''}", flush=True)
        r = self.store.sgd_step(report=report, indices=indices, update_scale=not defer, **hp)
        e = self._ref_step("sgd", hp, active, update_scale=not defer)
        if report:
            self._check_report(r, e)
        self.last_sgd = (hp, indices, active)

    def op_capture(self):
        """Capture the last eager SGD step's call (a set never stepped eagerly has no work
        table, which a capture cannot build), half of them with the bucket sums it takes its
        norm from."""
        if self.last_sgd is None or len(self.graphs) >= 3:
            return self.op_sgd()
        hp, indices, eager_active = self.last_sgd
        active = self._active(indices)
        if active != eager_active:
            return self.op_sgd()
        sums = bool(self.rng.random() < 0.5) and bool(hp["max_grad_norm"] or self.scaler_on)
        print(f"  capture sgd{' from captured bucket sums' if sums else ''} {hp} "
              f"indices={indices} active={active}", flush=True)
        bucket = list(range(self.n)) if indices is None else indices
        if sums:
            self.store.grad_sumsq_tensors(bucket)
        self.store.begin_capture()
        if sums:
            self.store.grad_sumsq_tensors(bucket)
        self.store.sgd_step(indices=indices, tensor_sums=sums, **hp)
        self.graphs.append((self.store.end_capture(), hp, active))

    def op_replay(self):
        if not self.graphs:
            return self.op_capture()
        g, hp, active = self.graphs[int(self.rng.integers(0, len(self.graphs)))]
        print(f"  replay sgd {hp} active={active}", flush=True)
        g.replay()
        self._ref_step("sgd", hp, active)

    OPS = [("grads_flat", 6), ("grad_one", 3), ("accumulate", 3), ("drop_grad", 2),
           ("zero_grad", 2), ("upload_weights", 1), ("adam", 2), ("sgd", 8), ("scaler", 1),
           ("set_step", 1), ("grad_norm", 1), ("save", 1), ("load", 1), ("capture", 2),
           ("replay", 3), ("sums_step", 4), ("zero_graph", 2), ("scaler_update", 1),
           ("producer_step", 3), ("producer_graph", 1), ("producer_replay", 2)]

    def compare(self):
        from ttperf import _lib as L
        mask = np.zeros(self.store.total, bool)
        for i, t in enumerate(self.store.tensors):
            mask[self.store.offsets[i]:self.store.offsets[i] + t.numel] = True
        got = self.store.download(L.BUF_PARAM)
        bad = int(np.count_nonzero((got != self.ref.param[:self.store.total]) & mask))
        assert bad == 0, f"{bad} bf16 weights differ"
        got = self.store.download(L.BUF_GRAD)
        want = self.ref.grad[:self.store.total]
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), "gradients differ"
        assert [self.store.has_grad(i) for i in range(self.n)] == \
            [self.ref.has_grad(i) for i in range(self.n)], "has-grad flags differ"
        assert self.store.step_count == self.ref.t
        if self.scaler_on:
            scale, tracker = self.store.scaler_state()
            assert (scale, tracker) == (np.float32(self.ref.scale), self.ref.growth_tracker)


@pytest.mark.parametrize("seed", SEEDS)
def test_bf16_store_random_operation_sequence(seed, tmp_path):
    c = Bf16Case(seed, tmp_path)
    print(f"case {seed}: bf16 shapes={c.shapes}", flush=True)
    names = [n for n, _ in Bf16Case.OPS]
    weights = np.array([w for _, w in Bf16Case.OPS], np.float64)
    weights /= weights.sum()
    try:
        for k in range(N_OPS):
            op = names[int(c.rng.choice(len(names), p=weights))]
            print(f" op {k}: {op}", flush=True)
            getattr(c, "op_" + op)()
            c.compare()
    finally:
        c.close()
