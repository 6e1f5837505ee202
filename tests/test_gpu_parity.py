"""GPU parity: libttperf_hip (through its C ABI) against the CPU oracle on identical seeded
inputs, at the benchmark configurations' real shapes.

Bar (from the north star): bf16 params bit-exact (RNE of the fp32 master); fp32 master, m, v
within 2 ulp — the engine evaluates the reference's op order with IEEE fp32 ops and no
contraction, so without clipping the expected difference is 0 ulp, and the tests require it;
with clipping the coefficient comes from an fp64 norm whose last bits depend on summation
order, so they allow the 2 ulp; grad norm within 1e-5 relative; identical found_inf / skip /
loss-scale / step-count decisions.
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu


def _table(name):
    from ttperf import configs
    return configs.table(name)


def _set_ref_grads(ref, host):
    """host: device_grads' copy, taken straight into ref.grad (into=ref.grad)."""
    assert np.shares_memory(host, ref.grad)
    for i in range(ref.n):
        ref.set_has_grad(i, True)


def _check_report(r, e, norm_rtol=1e-5):
    assert r["found_inf"] == e["found_inf"]
    assert r["skipped"] == e["skipped"]
    assert r["step"] == e["step"]
    assert r["scale"] == e["scale"] and r["growth_tracker"] == e["growth_tracker"]
    if np.isfinite(e["grad_norm"]):
        assert abs(r["grad_norm"] - e["grad_norm"]) <= norm_rtol * e["grad_norm"]
    else:
        assert not np.isfinite(r["grad_norm"]) or np.isnan(e["grad_norm"])


def test_cfg1_mlp_fp32_adam_bit_exact():
    """Config 1: Adam on the 2-layer MLP, all fp32, 100 steps with fresh seeded grads."""
    torch = torch_mod()
    names, shapes, decay, _ = _table("mlp")
    store, ref = make_pair(shapes, [False] * 4, O.MODE_FP32, init="uniform", seed=1)
    gen = torch.Generator(device="cuda").manual_seed(2)
    hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    for step in range(100):
        host = device_grads(store, gen, 1e-2, into=ref.grad)
        _set_ref_grads(ref, host)
        r = store.adam_step(report=(step % 25 == 24), **hp)
        e = ref.adam_step(**hp)
        if r is not None:
            _check_report(r, e)
            compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=0)
    assert store.step_count == 100 == ref.t
    compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=0)


def test_cfg2_nanogpt_mixed_adamw_clip():
    """Config 2: 76 ragged tensors, bf16 params/grads, fp32 master/m/v, AdamW, clip 1.0."""
    torch = torch_mod()
    names, shapes, decay, _ = _table("nanogpt_char")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=3)
    gen = torch.Generator(device="cuda").manual_seed(4)
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    steps = 50
    for step in range(steps):
        host = device_grads(store, gen, 1e-3, into=ref.grad)
        _set_ref_grads(ref, host)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        _check_report(r, e)
        assert r["clip_coef"] < 1.0  # the clip path is exercised
        print(f"cfg2 step {step}: norm {r['grad_norm']:.6f}", flush=True)
        if step in (0, steps - 1):
            compare_state(store, ref, max_ulp=2)


def test_cfg3_gpt2_small_scaler_inf_skip():
    """Config 3: GPT-2 124M, mixed precision, dynamic loss scaling with a seeded +inf every
    50th step (skip, t unchanged, scale backoff), AdamW, clip 1.0; all 200 steps, so all four
    overflows happen (scale 65536 -> 4096).  Every step's report is checked; the whole state
    after steps 1, 50 (the first skip), 51 and 200."""
    torch = torch_mod()
    names, shapes, decay, _ = _table("gpt2_124m")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=5)
    store.configure_scaler(True, init_scale=2.0 ** 16)
    ref.configure_scaler(True, 2.0 ** 16)
    gen = torch.Generator(device="cuda").manual_seed(6)
    rng = np.random.default_rng(7)
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    steps = 200
    check_at = {1, 50, 51, 200}
    for step in range(1, steps + 1):
        scale = ref.scale
        inf_at = None
        if step % 50 == 0:
            t = int(rng.integers(0, len(shapes)))
            inf_at = store.offsets[t] + int(rng.integers(0, store.tensors[t].numel))
        host = device_grads(store, gen, 1e-3, scale=scale, inf_at=inf_at, into=ref.grad)
        _set_ref_grads(ref, host)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        _check_report(r, e)
        assert r["skipped"] == (step % 50 == 0)
        if step % 10 == 0:
            print(f"cfg3 step {step}: scale {r['scale']} skipped {r['skipped']}", flush=True)
        if step in check_at:
            compare_state(store, ref, max_ulp=2)
    expected_scale = 65536.0 / 2 ** (steps // 50)
    assert expected_scale == 4096.0
    assert ref.scale == expected_scale and store.scaler_state()[0] == expected_scale
    assert store.step_count == steps - steps // 50


def test_cfg4_gpt2_large_scaler_clip_inf_skip():
    """Config 4: GPT-2 774M's 436 ragged tensors (1,280 .. 64.3M elements), mixed-precision
    AdamW with dynamic loss scaling from 2^16, clip 1.0 and a +inf at a seeded position on
    steps 3 and 13 (skip, step count unchanged, scale backoff), as config 3 but over the
    large table: the configuration's 20 steps.  Every step's report is checked against the
    oracle, and the whole state after the first overflow and at the end."""
    torch = torch_mod()
    names, shapes, decay, _ = _table("gpt2_774m")
    assert len(shapes) == 436
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=8)
    store.configure_scaler(True, init_scale=2.0 ** 16)
    ref.configure_scaler(True, 2.0 ** 16)
    gen = torch.Generator(device="cuda").manual_seed(9)
    rng = np.random.default_rng(10)
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    steps = 20
    inf_steps = {3, 13}
    for step in range(1, steps + 1):
        inf_at = None
        if step in inf_steps:
            t = int(rng.integers(0, len(shapes)))
            inf_at = store.offsets[t] + int(rng.integers(0, store.tensors[t].numel))
        host = device_grads(store, gen, 1e-3, scale=ref.scale, inf_at=inf_at, into=ref.grad)
        _set_ref_grads(ref, host)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        _check_report(r, e)
        assert r["skipped"] == (step in inf_steps)
        assert r["clip_coef"] < 1.0 or r["skipped"]  # the clip path is exercised
        print(f"cfg4 step {step}: norm {r['grad_norm']:.6f} scale {r['scale']} "
              f"skipped {r['skipped']} t {r['step']}", flush=True)
        if step == 3:
            compare_state(store, ref, max_ulp=2)
    n_inf = len(inf_steps)
    assert store.step_count == ref.t == steps - n_inf
    assert store.scaler_state()[0] == ref.scale == 65536.0 / 2 ** n_inf
    compare_state(store, ref, max_ulp=2)
