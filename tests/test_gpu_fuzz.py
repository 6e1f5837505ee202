"""Stateful differential fuzzing of libttperf_hip against the CPU oracle.

Each seeded case builds a small ragged store (empty, 1-element, odd, 2-D tensors; decay
flags; fp32 or mixed precision, half the mixed stores in the SGD layout, which the first Adam
step converts and live graphs keep it from converting) and runs a random sequence of
operations drawn from the whole host interface, mirrored on the oracle:

  gradients written flat or per tensor, from host or device memory (an occasional +inf while
  loss scaling is on); gradients accumulated from fp32 or bf16 sources, host or device;
  `grad = None`; zero_grad of all or of a subset, to zeros or to None (with or without the
  fill); master or bf16 weight
  uploads; Adam / AdamW / L2 and SGD (momentum, dampening, nesterov, L2) steps over everything
  or over a subset, with or without clipping, with step reports; steps that take their norm
  from bucket sums (ttp_grad_sumsq_tensors), and their refusal after a gradient write; a
  backward's gradient producer (accumulates in reverse order whose last one per tensor also
  stores that tensor's gradient sum, TTP_ACCUM_SUMSQ, some tensors with bucket sums instead)
  followed by a step from those sums, and its refusal after an accumulate without sums; such
  a producer iteration (from device buffers read in place) and its Adam step captured as one
  graph and launched later with new buffer contents; both producers with their gradients in
  bucket calls (ttp_accumulate_grad_multi) half of the time; the
  loss scaler switched on or off; the step count set; the gradient norm probed; a checkpoint
  saved and later loaded; an Adam step captured into a graph (half of them together with
  the bucket sums it takes its norm from), and a zero_grad captured into one, replayed
  later, between other operations; with loss scaling on, steps that defer the scale update
  to a later step or to ttp_scaler_update; Adam steps through the no-allocation entry point
  (ttp_adam_step_noalloc), and its refusals when a tensor set or betas were never stepped.

After every operation the whole state is compared: master, m, v and momentum within the
2-ulp bar of the other parity tests (in practice 0), bf16 weights and the gradients bit for
bit, the has-grad flags, the step count and the loss-scaler state; step reports must agree
on skip, found_inf, step count and scale.  Every operation is printed before it runs.
"""
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, make_pair, torch_mod

pytestmark = pytest.mark.gpu

# 1000 seeded cases of 50 operations by default; TTP_FUZZ_CASES=N runs N (the same first 1000,
# then more), from seed TTP_FUZZ_FIRST on (2000), TTP_FUZZ_OPS operations each; and 100 longer
# cases of 250 operations (TTP_FUZZ_LONG_CASES), which reach deeper states: more live graphs,
# checkpoints and scale changes per store
_FIRST = int(os.environ.get("TTP_FUZZ_FIRST", "2000"))
SEEDS = list(range(_FIRST, _FIRST + int(os.environ.get("TTP_FUZZ_CASES", "1000"))))
N_OPS = int(os.environ.get("TTP_FUZZ_OPS", "50"))  # operations per case
LONG_SEEDS = list(range(90000, 90000 + int(os.environ.get("TTP_FUZZ_LONG_CASES", "100"))))
LONG_OPS = 250
BETAS = [(0.9, 0.999), (0.9, 0.95), (0.8, 0.99)]


def _shapes(rng):
    out = []
    for _ in range(int(rng.integers(2, 9))):
        k = int(rng.integers(0, 8))
        if k == 0:
            out.append((0,))
        elif k == 1:
            out.append((1,))
        elif k <= 4:
            out.append((int(rng.integers(2, 3000)),))
        else:
            out.append((int(rng.integers(1, 90)), int(rng.integers(1, 90))))
    return out


class Case:
    def __init__(self, seed, tmp_path, bf16=False):
        """bf16: a BF16 store (bf16 weights and gradients only) instead of a drawn mode."""
        self.torch = torch_mod()
        self.rng = np.random.default_rng(seed)
        rng = self.rng
        self.shapes = _shapes(rng)
        self.n = len(self.shapes)
        self.decay = [len(s) == 2 for s in self.shapes]
        if bf16:
            self.mixed = True  # bf16 gradients, as a mixed store's
            mode = O.MODE_BF16
            self.sgd_layout = False
        else:
            self.mixed = bool(rng.integers(0, 2))
            mode = O.MODE_MIXED if self.mixed else O.MODE_FP32
            # half the mixed cases start in the SGD layout (a generator of its own keeps the
            # other draws of a seed as they were); the first Adam step converts the store
            self.sgd_layout = self.mixed and np.random.default_rng(seed + 7777).random() < 0.5
        self.store, self.ref = make_pair(self.shapes, self.decay, mode, seed=seed,
                                         layout="sgd" if self.sgd_layout else "default")
        self.store.set_stream(None)  # the store's own stream: capturable
        self.numels = [t.numel for t in self.store.tensors]
        self.graphs = []      # (graph, hp, captured active set)
        self.zero_graphs = []  # (graph, set_to_none, indices, fill) of captured zero_grad calls
        # (graph, hp, indices, targets, device sources) of captured producer iterations
        self.prod_graphs = []
        self.last_adam = None  # (hp, indices, active set) of the last eager Adam step
        self.saved = None     # oracle snapshot of the last checkpoint
        self.path = tmp_path / f"state_{seed}.bin"
        self.scaler_on = False
        self.adam_seen = False
        self.mom_seen = False

    # ---- helpers ------------------------------------------------------------------------
    def grad_values(self, n, std=None):
        std = float(10 ** self.rng.uniform(-4, -1)) if std is None else std
        g = (self.rng.standard_normal(n) * std).astype(np.float32)
        if self.scaler_on:
            g *= np.float32(self.ref.scale)
        return O.bf16_rne(g) if self.mixed else g

    def to_device(self, a):
        torch = self.torch
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
        return torch.from_numpy(a.copy()).cuda()

    def pick_subset(self):
        k = int(self.rng.integers(1, self.n + 1))
        return sorted(int(i) for i in self.rng.choice(self.n, size=k, replace=False))

    def nonempty(self):
        return [i for i in range(self.n) if self.numels[i]]

    # ---- operations -----------------------------------------------------------------------
    def op_grads_flat(self):
        from ttperf import _lib as L
        g = self.grad_values(self.store.total)
        inf = self.scaler_on and self.rng.random() < 0.25 and self.nonempty()
        if inf:
            i = int(self.rng.choice(self.nonempty()))
            j = self.store.offsets[i] + int(self.rng.integers(0, self.numels[i]))
            g[j] = 0x7F80 if self.mixed else np.float32(np.inf)
        dev = self.rng.random() < 0.5
        print(f"  grads flat ({'device' if dev else 'host'}, inf={bool(inf)})", flush=True)
        self.store.upload(L.BUF_GRAD, L.ALL_TENSORS, self.to_device(g) if dev else g)
        self.ref.grad[:self.store.total] = g
        for i in range(self.n):
            self.ref.set_has_grad(i, True)

    def op_grad_one(self):
        i = int(self.rng.integers(0, self.n))
        g = self.grad_values(self.numels[i])
        print(f"  grad of tensor {i} (host)", flush=True)
        self.store.tensors[i].grad = g
        self.ref.set_grad(i, g)

    def op_accumulate(self):
        i = int(self.rng.integers(0, self.n))
        bf16 = self.rng.random() < 0.5
        dev = self.rng.random() < 0.5
        g = (self.rng.standard_normal(self.numels[i]) * 1e-2).astype(np.float32)
        if self.scaler_on:
            g *= np.float32(self.ref.scale)
        src = O.bf16_rne(g) if bf16 else g
        print(f"  accumulate into tensor {i} ({'bf16' if bf16 else 'fp32'}, "
              f"{'device' if dev else 'host'}, had grad {self.ref.has_grad(i)})", flush=True)
        self.store.accumulate_grad(i, self.to_device(src) if dev else src)
        self.ref.accumulate_grad(i, src)

    def op_drop_grad(self):
        i = int(self.rng.integers(0, self.n))
        print(f"  grad of tensor {i} = None", flush=True)
        self.store.set_has_grad(i, False)
        self.ref.set_has_grad(i, False)

    def op_zero_grad(self):
        none = bool(self.rng.integers(0, 2))
        # to None, half of the time without the fill (TTP_ZERO_NO_FILL: the flags only)
        fill = not none or bool(self.rng.random() < 0.5)
        if self.rng.random() < 0.5:
            print(f"  zero_grad(set_to_none={none}, fill={fill})", flush=True)
            self.store.zero_grad(set_to_none=none, fill=fill)
            self.ref.zero_grad(set_to_none=none, fill=fill)
        else:
            idx = self.pick_subset()
            print(f"  zero_grad(set_to_none={none}, indices={idx}, fill={fill})", flush=True)
            self.store.zero_grad(set_to_none=none, indices=idx, fill=fill)
            for i in idx:
                if fill:
                    self.ref.view("grad", i)[:] = 0
                if none:  # set_to_none=False leaves the has-grad flags as they are
                    self.ref.set_has_grad(i, False)

    def op_upload_weights(self):
        i = int(self.rng.integers(0, self.n))
        x = (self.rng.standard_normal(self.numels[i]) * 0.05).astype(np.float32)
        if self.mixed and self.rng.random() < 0.5:
            from ttperf import _lib as L
            bits = O.bf16_rne(x)
            print(f"  bf16 weights of tensor {i}", flush=True)
            self.store.upload(L.BUF_PARAM, i, bits)
            self.ref.view("param", i)[:] = bits
            self.ref.view("master", i)[:] = O.bf16_to_f32(bits)
        else:
            print(f"  master weights of tensor {i}", flush=True)
            self.store.tensors[i].set_data(x)
            self.ref.set_master(i, x)

    def _live(self):
        return len(self.graphs) + len(self.zero_graphs) + len(self.prod_graphs)

    def _active(self, indices):
        cand = range(self.n) if indices is None else indices
        return [i for i in cand if self.ref.has_grad(i) and self.numels[i]]

    def _ref_step(self, kind, hp, active, update_scale=True):
        """The oracle steps exactly `active` (has-grad flags narrowed, then restored)."""
        flags = [self.ref.has_grad(i) for i in range(self.n)]
        for i in range(self.n):
            self.ref.set_has_grad(i, i in active)
        if kind == "adam":
            e = self.ref.adam_step(max_grad_norm=hp["max_grad_norm"] or 0.0,
                                   update_scale=update_scale,
                                   **{k: v for k, v in hp.items() if k != "max_grad_norm"})
        else:
            e = self.ref.sgd_step(max_grad_norm=hp["max_grad_norm"] or 0.0,
                                  update_scale=update_scale,
                                  **{k: v for k, v in hp.items() if k != "max_grad_norm"})
        for i in range(self.n):
            self.ref.set_has_grad(i, flags[i])
        return e

    def _check_report(self, r, e):
        assert r["skipped"] == e["skipped"] and r["found_inf"] == e["found_inf"], (r, e)
        assert r["step"] == e["step"], (r, e)
        if self.scaler_on:
            assert r["scale"] == e["scale"] and r["growth_tracker"] == e["growth_tracker"]
        if np.isfinite(e["grad_norm"]) and e["grad_norm"] > 0 and np.isfinite(r["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]

    def _conversion_refused(self, step):
        """An Adam step on a store still in the SGD layout converts it, which is refused while
        graphs live (they hold the master's address): checks that the refusal changed nothing.
        True when the step was refused."""
        import ttperf
        from ttperf import _lib as L
        live = self._live()
        if not (self.store.sgd_layout and live):
            return False
        t0 = self.store.step_count
        with pytest.raises(ttperf.TTPError) as e:
            step()
        assert e.value.code == L.ERR_STATE and "SGD layout" in str(e.value)
        assert self.store.step_count == t0 and self.store.sgd_layout
        print(f"   refused: converting the SGD layout with {live} live graph(s)", flush=True)
        return True

    def op_adam(self):
        rng = self.rng
        wd = 0.0 if rng.random() < 0.3 else float(rng.uniform(0.01, 0.2))
        hp = dict(lr=float(10 ** rng.uniform(-4, -1.5)), betas=BETAS[int(rng.integers(0, 3))],
                  eps=[1e-8, 1e-6][int(rng.integers(0, 2))], weight_decay=wd,
                  decoupled=bool(rng.integers(0, 2)),
                  max_grad_norm=None if rng.random() < 0.5 else float(10 ** rng.uniform(-2, 1)))
        indices = None if rng.random() < 0.6 else self.pick_subset()
        report = rng.random() < 0.5
        defer = self.scaler_on and rng.random() < 0.3
        noalloc = not report and rng.random() < 0.3
        active = self._active(indices)
        print(f"  adam {hp} indices={indices} active={active}"
              f"{' deferring the scale update' if defer else ''}"
              f"{' (no-allocation entry point)' if noalloc else ''}", flush=True)
        r = None
        if noalloc and not self._noalloc_adam(hp, indices, defer):
            noalloc = False  # refused, nothing changed: the allocating step instead
        if not noalloc and self._conversion_refused(
                lambda: self.store.adam_step(report=report, indices=indices,
                                             update_scale=not defer, **hp)):
            return
        if not noalloc:
            r = self.store.adam_step(report=report, indices=indices, update_scale=not defer,
                                     **hp)
        e = self._ref_step("adam", hp, active, update_scale=not defer)
        if report:
            self._check_report(r, e)
        if not noalloc:
            # a capture repeats the last allocating step: the no-allocation step builds no
            # bias table in host-count mode, which a capture could then not build either
            self.last_adam = (hp, indices, active)
        self.adam_seen = True

    def _noalloc_adam(self, hp, indices, defer):
        """ttp_adam_step_noalloc; False when it refuses (a tensor set, betas or FP32 moments
        that would need an allocation), after checking that the refusal changed nothing."""
        import ctypes as C
        from ttperf import _lib as L
        h = L.AdamHParams(lr=hp["lr"], beta1=hp["betas"][0], beta2=hp["betas"][1],
                          eps=hp["eps"], weight_decay=hp["weight_decay"],
                          decoupled=1 if hp["decoupled"] else 0,
                          flags=L.STEP_DEFER_SCALE if defer else 0,
                          max_grad_norm=hp["max_grad_norm"] or 0.0)
        t0 = self.store.step_count
        if indices is None:
            rc = L.lib.ttp_adam_step_noalloc(self.store.handle, C.byref(h), None, 0)
        else:
            idx = (C.c_uint32 * len(indices))(*indices)
            rc = L.lib.ttp_adam_step_noalloc(self.store.handle, C.byref(h), idx, len(indices))
        if rc == L.OK:
            return True
        msg = L.lib.ttp_last_error().decode()
        assert rc == L.ERR_STATE and "no-allocation" in msg and "first" in msg, (rc, msg)
        assert self.store.step_count == t0
        print(f"   refused: {msg}", flush=True)
        return False

    def op_sgd(self):
        rng = self.rng
        kind = int(rng.integers(0, 4))
        hp = dict(lr=float(10 ** rng.uniform(-3, -1)), momentum=0.0, dampening=0.0,
                  weight_decay=0.0, nesterov=False,
                  max_grad_norm=None if rng.random() < 0.5 else float(10 ** rng.uniform(-2, 1)))
        if kind == 1:
            hp.update(momentum=0.9)
        elif kind == 2:
            hp.update(momentum=0.9, nesterov=True, weight_decay=0.01)
        elif kind == 3:
            hp.update(momentum=0.8, dampening=0.1, weight_decay=0.05)
        indices = None if rng.random() < 0.6 else self.pick_subset()
        report = rng.random() < 0.5
        defer = self.scaler_on and rng.random() < 0.3
        active = self._active(indices)
        print(f"  sgd {hp} indices={indices} active={active}"
              f"{' deferring the scale update' if defer else ''}", flush=True)
        r = self.store.sgd_step(report=report, indices=indices, update_scale=not defer, **hp)
        e = self._ref_step("sgd", hp, active, update_scale=not defer)
        if report:
            self._check_report(r, e)
        self.last_adam = None
        self.mom_seen = self.mom_seen or hp["momentum"] > 0

    def _adam_ok(self, adam):
        """Whether a step drawn as Adam stays Adam (a store without fp32 state steps SGD)."""
        return adam

    # the step a captured producer iteration ends with: AdamW from the producer's sums
    PRODUCER_KIND = "adam"

    def _producer_hp(self, rng):
        return dict(lr=float(10 ** rng.uniform(-4, -1.5)), betas=BETAS[int(rng.integers(0, 3))],
                    eps=1e-8, weight_decay=0.05, decoupled=True,
                    max_grad_norm=float(10 ** rng.uniform(-2, 1)))

    def _producer_step(self, indices, hp, report):
        return self.store.adam_step(report=report, indices=indices, tensor_sums=True, **hp)

    def _sums_sgd_hp(self, lr, clip):
        """The SGD step that follows bucket sums or a producer: momentum 0.9."""
        return dict(lr=lr, momentum=0.9, dampening=0.0, weight_decay=0.0, nesterov=False,
                    max_grad_norm=clip)

    def op_sums_step(self):
        """Bucket sums over a random partition of the tensors, then a step that takes its norm
        from them; sometimes a gradient write in between, after which the step is refused
        with nothing changed."""
        import ttperf
        from ttperf import _lib as L
        rng = self.rng
        perm = [int(i) for i in rng.permutation(self.n)]
        cuts = sorted(set(int(c) for c in rng.integers(1, self.n + 1, size=2)))
        buckets = [sorted(perm[a:b]) for a, b in zip([0] + cuts, cuts + [self.n]) if b > a]
        for b in buckets:
            self.store.grad_sumsq_tensors(b)
        adam = self._adam_ok(rng.random() < 0.6)
        clip = None if rng.random() < 0.3 else float(10 ** rng.uniform(-2, 1))
        indices = None if rng.random() < 0.6 else self.pick_subset()
        if adam:
            kind, hp = "adam", dict(lr=float(10 ** rng.uniform(-4, -1.5)),
                                    betas=BETAS[int(rng.integers(0, 3))], eps=1e-8,
                                    weight_decay=0.05, decoupled=True, max_grad_norm=clip)
        else:
            kind, hp = "sgd", self._sums_sgd_hp(float(10 ** rng.uniform(-3, -1)), clip)
        cand = [i for i in (range(self.n) if indices is None else indices) if self.numels[i]]
        stale = (clip or self.scaler_on) and cand and rng.random() < 0.3
        print(f"  sums over {buckets} then {kind} {hp} indices={indices}"
              f"{' after a gradient write' if stale else ''}", flush=True)
        if stale:
            i = int(rng.choice(cand))
            g = self.grad_values(self.numels[i])
            self.store.tensors[i].grad = g
            self.ref.set_grad(i, g)
            t0 = self.store.step_count
            with pytest.raises(ttperf.TTPError) as e:
                step = self.store.adam_step if adam else self.store.sgd_step
                step(indices=indices, tensor_sums=True, **hp)
            assert e.value.code == L.ERR_STATE and self.store.step_count == t0
            return
        active = self._active(indices)
        step = self.store.adam_step if adam else self.store.sgd_step
        if adam and self._conversion_refused(
                lambda: step(report=True, indices=indices, tensor_sums=True, **hp)):
            return
        r = step(report=True, indices=indices, tensor_sums=True, **hp)
        e = self._ref_step(kind, hp, active)
        self._check_report(r, e)
        if adam:
            self.last_adam = (hp, indices, active)
            self.adam_seen = True
        else:
            self.last_adam = None
            self.mom_seen = True

    def op_producer_step(self):
        """A backward's gradient producer: one or two accumulates into each tensor of a random
        set, in reverse order as a backward delivers them, the last one of each with
        TTP_ACCUM_SUMSQ so that the launch also stores the tensor's gradient sum; a few of the
        tensors take bucket sums instead; then a step over them from those sums (no norm
        pass).  Sometimes an accumulate without sums comes last into one of them, which makes
        its sum stale: the step is refused and changes nothing."""
        import ttperf
        from ttperf import _lib as L
        rng = self.rng
        if rng.random() < 0.5:
            fill = bool(rng.random() < 0.5)
            print(f"  zero_grad(set_to_none=True, fill={fill}) before the producer", flush=True)
            self.store.zero_grad(set_to_none=True, fill=fill)
            self.ref.zero_grad(set_to_none=True, fill=fill)
        indices = None if rng.random() < 0.5 else self.pick_subset()
        targets = list(range(self.n)) if indices is None else list(indices)
        bucket = [i for i in targets if rng.random() < 0.2]
        adam = self._adam_ok(rng.random() < 0.6)
        clip = None if (self.scaler_on and rng.random() < 0.3) else float(10 ** rng.uniform(-2, 1))
        if adam:
            kind, hp = "adam", dict(lr=float(10 ** rng.uniform(-4, -1.5)),
                                    betas=BETAS[int(rng.integers(0, 3))], eps=1e-8,
                                    weight_decay=0.05, decoupled=True, max_grad_norm=clip)
        else:
            kind, hp = "sgd", self._sums_sgd_hp(float(10 ** rng.uniform(-3, -1)), clip)
        log = []
        multi = rng.random() < 0.5  # the tensors in bucket calls (ttp_accumulate_grad_multi)
        if multi:
            # two rounds over the reverse order cut into buckets of 1..4 tensors (one source
            # dtype per call): an add (or assign) round, then a round with sums except for the
            # tensors that take bucket sums, which get no second round
            for rnd in range(2):
                order = [i for i in reversed(targets) if rnd == 0 or i not in bucket]
                k = 0
                while k < len(order):
                    part = order[k:k + int(rng.integers(1, 5))]
                    k += len(part)
                    bf16 = rng.random() < 0.5
                    hosts, devs = [], []
                    for i in part:
                        g = (rng.standard_normal(self.numels[i])
                             * float(10 ** rng.uniform(-4, -1))).astype(np.float32)
                        if self.scaler_on:
                            g *= np.float32(self.ref.scale)
                        hosts.append(O.bf16_rne(g) if bf16 else g)
                        devs.append(self.to_device(hosts[-1]))
                    self.store.accumulate_grads(part, devs, sums=rnd == 1)
                    for i, h in zip(part, hosts):
                        self.ref.accumulate_grad(i, h)
                    log.append("[" + " ".join(f"{i}{'s' if rnd == 1 else ''}" for i in part) + "]")
        for i in ([] if multi else reversed(targets)):
            reps = int(rng.integers(1, 3))
            for rep in range(reps):
                sums = rep == reps - 1 and i not in bucket
                bf16 = rng.random() < 0.5
                dev = rng.random() < 0.5
                g = (rng.standard_normal(self.numels[i]) * float(10 ** rng.uniform(-4, -1)))
                g = g.astype(np.float32)
                if self.scaler_on:
                    g *= np.float32(self.ref.scale)
                src = O.bf16_rne(g) if bf16 else g
                self.store.accumulate_grad(i, self.to_device(src) if dev else src, sums=sums)
                self.ref.accumulate_grad(i, src)
                log.append(f"{i}{'s' if sums else ''}")
        if bucket:
            self.store.grad_sumsq_tensors(bucket)
        nonempty = [i for i in targets if self.numels[i]]
        stale = (clip is not None or self.scaler_on) and nonempty and rng.random() < 0.2
        print(f"  producer {' '.join(log)}, bucket sums {bucket}, then {kind} {hp} "
              f"indices={indices}{' after an accumulate without sums' if stale else ''}",
              flush=True)
        step = self.store.adam_step if adam else self.store.sgd_step
        if stale:
            i = int(rng.choice(nonempty))
            g = self.grad_values(self.numels[i])
            self.store.accumulate_grad(i, g)
            self.ref.accumulate_grad(i, g)
            t0, layout = self.store.step_count, self.store.sgd_layout
            with pytest.raises(ttperf.TTPError) as e:
                step(indices=indices, tensor_sums=True, **hp)
            assert e.value.code == L.ERR_STATE and self.store.step_count == t0
            assert self.store.sgd_layout == layout
            return
        active = self._active(indices)
        if adam and self._conversion_refused(
                lambda: step(report=True, indices=indices, tensor_sums=True, **hp)):
            return
        r = step(report=True, indices=indices, tensor_sums=True, **hp)
        e = self._ref_step(kind, hp, active)
        self._check_report(r, e)
        if adam:
            self.last_adam = (hp, indices, active)
            self.adam_seen = True
        else:
            self.last_adam = None
            self.mom_seen = True

    def op_scaler(self):
        on = not self.scaler_on
        init = float(2.0 ** int(self.rng.integers(4, 14)))
        interval = int(self.rng.integers(2, 5))
        live = self._live()  # every graph holds the settings
        print(f"  scaler {'on' if on else 'off'} (init {init:g}, interval {interval}), "
              f"{live} live graph(s)", flush=True)
        if live:
            import ttperf
            with pytest.raises(ttperf.TTPError):
                self.store.configure_scaler(on, init_scale=init, growth_interval=interval)
            return
        self.store.configure_scaler(on, init_scale=init, growth_interval=interval)
        if on:
            self.ref.configure_scaler(True, init, growth_interval=interval)
        else:
            self.ref.s.scaler_enabled = 0
            self.ref.s.pending = 0  # a configure drops a pending overflow
        self.scaler_on = on

    def op_scaler_update(self):
        """GradScaler.update() after deferred steps (a no-op while loss scaling is off)."""
        print(f"  scaler_update (scaler {'on' if self.scaler_on else 'off'}, pending overflow "
              f"{self.ref.s.pending})", flush=True)
        self.store.scaler_update()
        self.ref.scaler_update()

    def op_set_step(self):
        t = int(self.rng.integers(0, 50))
        print(f"  step count = {t}", flush=True)
        self.store.step_count = t
        self.ref.t = t

    def op_grad_norm(self):
        print("  grad_norm()", flush=True)
        got = self.store.grad_norm()
        inv = 1.0 / self.ref.scale if self.scaler_on else 1.0
        sumsq, _ = self.ref.grad_sumsq(inv)
        want = float(np.sqrt(sumsq))
        if np.isfinite(want) and want > 0:
            assert abs(got - want) <= 1e-5 * want, (got, want)

    def _snapshot(self):
        r, s = self.ref, self.ref.s
        return dict(master=r.master.copy(), param=r.param.copy(), exp_avg=r.exp_avg.copy(),
                    exp_avg_sq=r.exp_avg_sq.copy(), momentum=r.momentum.copy(),
                    mom_init=r.mom_init.copy(), t=r.t, scale=s.scale,
                    tracker=s.growth_tracker, enabled=s.scaler_enabled,
                    interval=s.growth_interval, growth=s.growth_factor,
                    backoff=s.backoff_factor)

    def op_save(self):
        print(f"  save_state -> {self.path.name}", flush=True)
        self.store.save_state(self.path)
        self.saved = self._snapshot()

    def op_load(self):
        if self.saved is None:
            return self.op_save()
        snap = self.saved
        differs = bool(snap["enabled"]) != self.scaler_on or (
            self.scaler_on and snap["interval"] != self.ref.s.growth_interval)
        live = self._live()
        print(f"  load_state <- {self.path.name} ({live} live graph(s), "
              f"scaler settings differ: {differs})", flush=True)
        if live and differs:
            import ttperf
            with pytest.raises(ttperf.TTPError):
                self.store.load_state(self.path)
            return
        self.store.load_state(self.path)
        r, s = self.ref, self.ref.s
        for k in ("master", "param", "exp_avg", "exp_avg_sq", "momentum", "mom_init"):
            getattr(r, k)[:] = snap[k]
        r.t = snap["t"]
        s.scale, s.growth_tracker = snap["scale"], snap["tracker"]
        s.scaler_enabled, s.growth_interval = snap["enabled"], snap["interval"]
        s.growth_factor, s.backoff_factor = snap["growth"], snap["backoff"]
        s.pending = 0  # a loaded state has no pending overflow
        self.scaler_on = bool(snap["enabled"])

    def op_capture(self):
        """Capture the last eager Adam step's call (same hyperparameters, same tensor set: a
        set never stepped eagerly has no work table, which a capture cannot build)."""
        if self.last_adam is None or len(self.graphs) >= 3:
            return self.op_adam()
        hp, indices, eager_active = self.last_adam
        active = self._active(indices)
        if active != eager_active:
            return self.op_adam()
        # half the graphs take their norm from bucket sums captured with the step (an eager
        # sums call first gives the tile buffer its size: a capture cannot allocate)
        sums = bool(self.rng.random() < 0.5)
        print(f"  capture adam{' from captured bucket sums' if sums else ''} {hp} "
              f"indices={indices} active={active}", flush=True)
        bucket = list(range(self.n)) if indices is None else indices
        if sums:
            self.store.grad_sumsq_tensors(bucket)
        self.store.begin_capture()
        if sums:
            self.store.grad_sumsq_tensors(bucket)
        self.store.adam_step(indices=indices, tensor_sums=sums, **hp)
        self.graphs.append((self.store.end_capture(), hp, active))

    def op_replay(self):
        if not self.graphs:
            return self.op_capture()
        g, hp, active = self.graphs[int(self.rng.integers(0, len(self.graphs)))]
        print(f"  replay adam {hp} active={active}", flush=True)
        g.replay()
        self._ref_step("adam", hp, active)

    def _producer_calls(self, targets, srcs):
        """zero_grad to None, then the targets' gradients with sums in reverse order: one
        accumulate per tensor, or bucket calls of up to three tensors when the sources were
        made for them (srcs["multi"])."""
        self.store.zero_grad(set_to_none=True, fill=srcs.get("fill", True))
        order = list(reversed(targets))
        if srcs.get("multi"):
            for k in range(0, len(order), 3):
                part = order[k:k + 3]
                self.store.accumulate_grads(part, [srcs[i] for i in part], sums=True)
            return
        for i in order:
            self.store.accumulate_grad(i, srcs[i], sums=True)

    def _producer_iteration(self, hp, indices, targets, srcs, graph=None):
        """New contents for the producer's device sources, then either its eager calls
        (zero_grad to None, one accumulate with TTP_ACCUM_SUMSQ per tensor in reverse order,
        the Adam step from those sums) or a launch of their captured graph; the oracle does
        the same iteration.  Returns the store's step report (eager) or None."""
        torch = self.torch
        host = {}
        for i in reversed(targets):
            g = (self.rng.standard_normal(self.numels[i]) * float(10 ** self.rng.uniform(-4, -1)))
            g = g.astype(np.float32)
            if self.scaler_on:
                g *= np.float32(self.ref.scale)
            if srcs[i].dtype == torch.bfloat16:
                host[i] = O.bf16_rne(g)
                srcs[i].copy_(torch.from_numpy(host[i].view(np.int16)).view(torch.bfloat16))
            else:
                host[i] = g
                srcs[i].copy_(torch.from_numpy(g))
        torch.cuda.synchronize()
        r = None
        if graph is None:
            self._producer_calls(targets, srcs)
            r = self._producer_step(indices, hp, True)
        else:
            graph.replay()
            self.store.sync()
        self.ref.zero_grad(set_to_none=True, fill=srcs.get("fill", True))
        for i in reversed(targets):
            self.ref.accumulate_grad(i, host[i])
        e = self._ref_step(self.PRODUCER_KIND, hp, self._active(indices))
        if r is not None:
            self._check_report(r, e)
        self.last_adam = None
        self.adam_seen = self.adam_seen or self.PRODUCER_KIND == "adam"
        return r

    def op_producer_graph(self):
        """A backward's producer and its step captured as one graph: zero_grad to None, one
        accumulate with TTP_ACCUM_SUMSQ per tensor of a set (reverse order) from device
        buffers that the graph reads in place, then the AdamW step from those sums.  One eager
        run of the same calls comes first (it builds the step's tables, which a capture cannot
        build); each later launch rewrites the buffers first (op_producer_replay)."""
        torch = self.torch
        if len(self.prod_graphs) >= 2:
            return self.op_producer_replay()
        rng = self.rng
        indices = None if rng.random() < 0.5 else self.pick_subset()
        targets = [i for i in (range(self.n) if indices is None else indices) if self.numels[i]]
        if not targets:
            return self.op_adam()
        hp = self._producer_hp(rng)
        dt = torch.bfloat16 if rng.random() < 0.5 else torch.float32
        srcs = {i: torch.zeros(self.numels[i], device="cuda", dtype=dt) for i in targets}
        srcs["multi"] = bool(rng.random() < 0.5)
        srcs["fill"] = bool(rng.random() < 0.5)  # zero_grad with or without the fill
        print(f"  capture producer + {self.PRODUCER_KIND} from its sums {hp} indices={indices} "
              f"targets={targets} sources {dt}{' in bucket calls' if srcs['multi'] else ''}"
              f"{'' if srcs['fill'] else ', zero_grad(fill=False)'}",
              flush=True)
        if self._conversion_refused(lambda: self.store.adam_step(indices=indices, **hp)):
            return
        self._producer_iteration(hp, indices, targets, srcs)
        self.compare()
        self.store.begin_capture()
        self._producer_calls(targets, srcs)
        self._producer_step(indices, hp, False)
        self.prod_graphs.append((self.store.end_capture(), hp, indices, targets, srcs))

    def op_producer_replay(self):
        if not self.prod_graphs:
            return self.op_producer_graph()
        g, hp, indices, targets, srcs = self.prod_graphs[int(self.rng.integers(0, len(self.prod_graphs)))]
        print(f"  replay producer + {self.PRODUCER_KIND} {hp} indices={indices} "
              f"targets={targets}", flush=True)
        self._producer_iteration(hp, indices, targets, srcs, graph=g)

    def _zero_ref(self, none, idx, fill=True):
        if idx is None:
            self.ref.zero_grad(set_to_none=none, fill=fill)
            return
        for i in idx:
            if fill:
                self.ref.view("grad", i)[:] = 0
            if none:
                self.ref.set_has_grad(i, False)

    def op_zero_graph(self):
        """A captured zero_grad (all tensors or a subset, to zeros or to None, to None with or
        without the fill).  Capturing it changes nothing, neither the gradients nor the
        has-grad flags; each launch does what the eager call does.  A subset is zeroed eagerly
        once first, since a capture cannot build its work table."""
        if self.zero_graphs and (len(self.zero_graphs) >= 2 or self.rng.random() < 0.7):
            g, none, idx, fill = self.zero_graphs[int(self.rng.integers(0, len(self.zero_graphs)))]
            print(f"  replay zero_grad(set_to_none={none}, indices={idx}, fill={fill})", flush=True)
            g.replay()
            self._zero_ref(none, idx, fill)
            return
        none = bool(self.rng.integers(0, 2))
        fill = not none or bool(self.rng.random() < 0.5)
        idx = None if self.rng.random() < 0.5 else self.pick_subset()
        print(f"  capture zero_grad(set_to_none={none}, indices={idx}, fill={fill})", flush=True)
        if idx is not None:
            self.store.zero_grad(set_to_none=none, indices=idx, fill=fill)
            self._zero_ref(none, idx, fill)
        self.store.begin_capture()
        self.store.zero_grad(set_to_none=none, indices=idx, fill=fill)
        self.zero_graphs.append((self.store.end_capture(), none, idx, fill))

    OPS = [("grads_flat", 6), ("grad_one", 3), ("accumulate", 3), ("drop_grad", 2),
           ("zero_grad", 2), ("upload_weights", 1), ("adam", 6), ("sgd", 4), ("scaler", 1),
           ("set_step", 1), ("grad_norm", 1), ("save", 1), ("load", 1), ("capture", 2),
           ("replay", 3), ("sums_step", 4), ("zero_graph", 2), ("scaler_update", 1),
           ("producer_step", 3), ("producer_graph", 1), ("producer_replay", 2)]

    def compare(self):
        from ttperf import _lib as L
        which = ["master", "param"]
        if self.adam_seen:
            which += ["exp_avg", "exp_avg_sq"]
        if self.mom_seen:
            which += ["momentum"]
        compare_state(self.store, self.ref, which=tuple(which), max_ulp=2)
        # the SGD layout lasts until the first Adam step
        assert self.store.sgd_layout == (self.sgd_layout and not self.adam_seen)
        got = self.store.download(L.BUF_GRAD)
        want = self.ref.grad[:self.store.total]
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), "gradients differ"
        assert [self.store.has_grad(i) for i in range(self.n)] == \
            [self.ref.has_grad(i) for i in range(self.n)], "has-grad flags differ"
        assert self.store.step_count == self.ref.t
        if self.scaler_on:
            scale, tracker = self.store.scaler_state()
            assert (scale, tracker) == (np.float32(self.ref.scale), self.ref.growth_tracker)

    def close(self):
        for g in [x[0] for x in self.graphs + self.zero_graphs + self.prod_graphs]:
            g.close()
        self.graphs.clear()
        self.zero_graphs.clear()
        self.prod_graphs.clear()
        self.store.close()


def _run_case(seed, tmp_path, n_ops):
    c = Case(seed, tmp_path)
    print(f"case {seed}: {'mixed' if c.mixed else 'fp32'}"
          f"{' (SGD layout)' if c.sgd_layout else ''} shapes={c.shapes}", flush=True)
    names = [n for n, _ in Case.OPS]
    weights = np.array([w for _, w in Case.OPS], np.float64)
    weights /= weights.sum()
    try:
        for k in range(n_ops):
            op = names[int(c.rng.choice(len(names), p=weights))]
            print(f" op {k}: {op}", flush=True)
            getattr(c, "op_" + op)()
            c.compare()
    finally:
        c.close()


@pytest.mark.parametrize("seed", SEEDS)
def test_random_operation_sequence(seed, tmp_path):
    _run_case(seed, tmp_path, N_OPS)


@pytest.mark.parametrize("seed", LONG_SEEDS)
def test_long_random_operation_sequence(seed, tmp_path):
    _run_case(seed, tmp_path, LONG_OPS)
