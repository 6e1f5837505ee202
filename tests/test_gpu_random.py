"""Randomized differential parity: libttperf_hip against the CPU oracle on seeded random
configurations, each printed before it runs.

Every case draws a ragged tensor table (empty, 1-element, odd and 2-D tensors, decay flags),
a precision mode (a mixed store in its default or its SGD layout), an optimizer (Adam with
decoupled, L2 or no weight decay; SGD plain, with momentum, dampening, nesterov, L2),
clipping on or off, and in mixed precision loss scaling with a short growth interval and an
injected +inf on some steps.  Three steps run, each with
fresh gradients, a random active set (a subset step, None grads, or every tensor), and the
full state and step report are compared after every step: bf16 bit-exact, fp32 within the
2-ulp bar of the other parity tests, identical skip / scale / step-count decisions.
"""
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

# 1000 seeded cases by default; TTP_RANDOM_CASES=N runs N (the same first 1000, then more)
SEEDS = list(range(1000, 1000 + int(os.environ.get("TTP_RANDOM_CASES", "1000"))))


def _shape(rng):
    kind = rng.integers(0, 10)
    if kind == 0:
        return (0,)
    if kind == 1:
        return (1,)
    if kind <= 4:
        return (int(rng.integers(2, 200)),)
    if kind <= 7:
        return (int(rng.integers(1, 300)), int(rng.integers(1, 300)))
    return (int(rng.integers(1000, 70000)),)


def _draw(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 13))
    shapes = [_shape(rng) for _ in range(n)]
    decay = [bool(rng.integers(0, 2)) for _ in range(n)]
    mixed = bool(rng.integers(0, 2))
    opt = ["adamw", "adam_l2", "adam", "sgd", "sgd_mom", "sgd_nesterov", "sgd_damp_l2"][
        int(rng.integers(0, 7))]
    clip = None if rng.random() < 0.4 else float(10 ** rng.uniform(-2, 1))
    scaler = mixed and rng.random() < 0.6
    init_scale = float(2.0 ** int(rng.integers(4, 17))) if rng.random() < 0.7 else 1000.0
    # half the mixed cases in the SGD layout (drawn from a generator of its own, so the
    # other draws of a seed stay as they were); an Adam step converts such a store
    sgd_layout = mixed and np.random.default_rng(seed + 7777).random() < 0.5
    return dict(rng=rng, shapes=shapes, decay=decay, mixed=mixed, opt=opt, clip=clip,
                scaler=scaler, init_scale=init_scale, sgd_layout=sgd_layout)


def _hp(opt, rng):
    lr = float(10 ** rng.uniform(-4, -1))
    if opt.startswith("adam"):
        b2 = [0.95, 0.999][int(rng.integers(0, 2))]
        wd = 0.0 if opt == "adam" else float(rng.uniform(0.01, 0.2))
        return "adam", dict(lr=lr, betas=(0.9, b2), eps=1e-8, weight_decay=wd,
                            decoupled=(opt == "adamw"))
    kw = dict(lr=lr)
    if opt == "sgd_mom":
        kw.update(momentum=0.9)
    elif opt == "sgd_nesterov":
        kw.update(momentum=0.9, nesterov=True)
    elif opt == "sgd_damp_l2":
        kw.update(momentum=0.8, dampening=0.1, weight_decay=0.01)
    return "sgd", kw


@pytest.mark.parametrize("seed", SEEDS)
def test_random_configuration(seed):
    torch = torch_mod()
    c = _draw(seed)
    rng = c["rng"]
    kind, hp = _hp(c["opt"], rng)
    print(f"case {seed}: {'mixed' if c['mixed'] else 'fp32'}"
          f"{' (SGD layout)' if c['sgd_layout'] else ''} {c['opt']} clip={c['clip']} "
          f"scaler={c['scaler']}({c['init_scale']:g}) hp={hp} shapes={c['shapes']}", flush=True)
    mode = O.MODE_MIXED if c["mixed"] else O.MODE_FP32
    store, ref = make_pair(c["shapes"], c["decay"], mode, seed=seed,
                           layout="sgd" if c["sgd_layout"] else "default")
    assert store.sgd_layout == c["sgd_layout"]
    if c["scaler"]:
        store.configure_scaler(True, init_scale=c["init_scale"], growth_interval=2)
        ref.configure_scaler(True, c["init_scale"], growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    numels = [t.numel for t in store.tensors]
    n = len(numels)
    which = ["master", "param"]
    if kind == "adam":
        which += ["exp_avg", "exp_avg_sq"]
    elif hp.get("momentum"):
        which += ["momentum"]
    for step in range(3):
        scale = ref.scale if c["scaler"] else 1.0
        inf_at = None
        if c["scaler"] and rng.random() < 0.3 and store.total:
            nonempty = [i for i in range(n) if numels[i]]
            if nonempty:
                i = nonempty[int(rng.integers(0, len(nonempty)))]
                inf_at = store.offsets[i] + int(rng.integers(0, numels[i]))
        host = device_grads(store, gen, float(10 ** rng.uniform(-4, -1)), scale=scale,
                            inf_at=inf_at)
        ref.grad[:store.total] = host
        # the active set: every tensor, a subset step, or some grads set to None
        pick = rng.integers(0, 3)
        active = list(range(n))
        indices = None
        if pick == 1:
            active = sorted(set(int(x) for x in rng.integers(0, n, size=max(1, n // 2))))
            indices = active
        elif pick == 2:
            active = [i for i in range(n) if rng.random() < 0.7]
            for i in range(n):
                if i not in active:
                    store.set_has_grad(i, False)
        for i in range(n):
            ref.set_has_grad(i, i in active)
        if kind == "adam":
            r = store.adam_step(report=True, indices=indices, max_grad_norm=c["clip"], **hp)
            e = ref.adam_step(max_grad_norm=c["clip"] or 0.0, **hp)
        else:
            r = store.sgd_step(report=True, indices=indices, max_grad_norm=c["clip"], **hp)
            e = ref.sgd_step(max_grad_norm=c["clip"] or 0.0, **hp)
        print(f"  step {step}: active {len(active)}/{n}, inf_at {inf_at}, norm {e['grad_norm']:.6g}, "
              f"skipped {e['skipped']}, scale {e['scale']:g}", flush=True)
        assert r["skipped"] == e["skipped"] and r["found_inf"] == e["found_inf"]
        assert r["step"] == e["step"]
        if c["scaler"]:
            assert r["scale"] == e["scale"] and r["growth_tracker"] == e["growth_tracker"]
        if (c["clip"] or c["scaler"]) and np.isfinite(e["grad_norm"]) and e["grad_norm"] > 0:
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        compare_state(store, ref, which=tuple(which), max_ulp=2)
        # an SGD-layout store keeps its layout through SGD steps; an Adam step converts it
        assert store.sgd_layout == (c["sgd_layout"] and kind == "sgd")
    store.close()
