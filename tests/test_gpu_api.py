"""GPU tests of the optimizer API and of the edge cases, through the C ABI (libttperf_hip),
against the CPU oracle on identical inputs.

The first group restates the reference's own optimizer tests on this engine:
tests/adam_optimizer.py:25-123 (seeds 31-34: one and two Adam steps of a 32x32 Linear against
the closed form `_adam_step_ref`, zero_grad clears, None grads are skipped) and
tests/sgd_optimizer.py:15-110 (seeds 21-24, bf16).  The reference compares with atol/rtol
1e-1 / 5e-2 because TTNN runs in bf16; here the closed form is met to fp32 rounding (the
closed form's own op order differs from py/optim.py's in the last bits) and the oracle
bit for bit.
"""
import numpy as np
import pytest

import oracle as O
from conftest import f32_ulp_diff
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu


def _linear_store(seed, mode):
    """A 32x32 Linear of py/nn.py:28-37: weight [in, out] ~ randn * 1/sqrt(in)."""
    import ttperf
    torch = torch_mod()
    torch.manual_seed(seed)
    x = torch.randn(32, 32)
    w0 = torch.randn(32, 32) * (1.0 / np.sqrt(32.0))
    store = ttperf.ParamStore([(32, 32)], mode=mode)
    if mode == "mixed":
        w0 = w0.to(torch.bfloat16).float()  # the reference holds bf16 weights
    store.tensors[0].set_data(w0.numpy())
    return store, store.tensors[0], x, w0


def _adam_step_ref(weight, grad, lr, betas, eps, step, m, v):
    # the closed form of tests/adam_optimizer.py:15-22
    beta1, beta2 = betas
    m = beta1 * m + (1.0 - beta1) * grad
    v = beta2 * v + (1.0 - beta2) * (grad * grad)
    m_hat = m / (1.0 - (beta1 ** step))
    v_hat = v / (1.0 - (beta2 ** step))
    weight = weight - lr * m_hat / (v_hat.sqrt() + eps)
    return weight, m, v


def _oracle_for(store, mode_mixed=False):
    ref = O.OracleStore([t.numel for t in store.tensors],
                        flags=[int(t.decay) for t in store.tensors],
                        mode=O.MODE_MIXED if mode_mixed else O.MODE_FP32, nthreads=4)
    ref.master[:] = store.download(2)  # BUF_MASTER
    if mode_mixed:
        ref.param[:] = O.bf16_rne(ref.master)
    return ref


def test_adam_step_matches_closed_form():
    import ttperf
    torch = torch_mod()
    store, w, x, w0 = _linear_store(31, "fp32")
    ref = _oracle_for(store)
    grad = x.t() @ torch.ones(32, 32)  # dW of y = x @ W with dY = ones
    w.grad = grad.numpy()
    ref.set_grad(0, grad.numpy())
    opt = ttperf.Adam(store.parameters(), lr=0.1, betas=(0.9, 0.999), eps=1e-8)
    opt.step()
    ref.adam_step(lr=0.1, betas=(0.9, 0.999), eps=1e-8, decoupled=False)
    w1 = w.numpy()
    w_ref, _, _ = _adam_step_ref(w0, grad, 0.1, (0.9, 0.999), 1e-8, 1, torch.zeros(32, 32),
                                 torch.zeros(32, 32))
    assert np.allclose(w1, w_ref.numpy(), atol=1e-6, rtol=1e-6)  # reference: 1e-1
    assert f32_ulp_diff(w1.ravel(), ref.master[:1024]).max() == 0


def test_adam_two_steps_match_closed_form():
    import ttperf
    torch = torch_mod()
    store, w, x, w0 = _linear_store(32, "fp32")
    ref = _oracle_for(store)
    opt = ttperf.Adam(store.parameters(), lr=0.1, betas=(0.9, 0.999), eps=1e-8)

    def grad_at(weight):  # y = tanh(x @ W), dY = ones (tests/adam_optimizer.py:61-69)
        z = torch.tanh(x @ weight)
        return x.t() @ (1 - z * z)

    m = torch.zeros(32, 32)
    v = torch.zeros(32, 32)
    wt = w0.clone()
    for step in (1, 2):
        g = grad_at(torch.from_numpy(w.numpy().copy()))
        w.grad = g.numpy()
        ref.set_grad(0, g.numpy())
        opt.step()
        opt.zero_grad()
        ref.adam_step(lr=0.1, betas=(0.9, 0.999), eps=1e-8, decoupled=False)
        wt, m, v = _adam_step_ref(wt, g, 0.1, (0.9, 0.999), 1e-8, step, m, v)
    assert np.allclose(w.numpy(), wt.numpy(), atol=1e-5, rtol=1e-5)
    assert f32_ulp_diff(w.numpy().ravel(), ref.master[:1024]).max() == 0
    assert store.step_count == 2


@pytest.mark.parametrize("cls", ["SGD", "Adam", "AdamW"])
def test_zero_grad_clears(cls):
    import ttperf
    store, w, x, _ = _linear_store(33, "fp32")
    w.grad = np.ones((32, 32), np.float32)
    assert w.grad is not None
    kw = dict(lr=0.1)
    getattr(ttperf, cls)(store.parameters(), **kw).zero_grad()
    assert w.grad is None


@pytest.mark.parametrize("cls", ["SGD", "Adam", "AdamW"])
def test_skips_none_grad(cls):
    import ttperf
    store, w, x, _ = _linear_store(34, "mixed")
    before = store.download(0).copy()  # bf16 bits of the weight
    master = w.master().copy()
    w.grad = np.full((32, 32), 0x3F80, np.uint16)  # a grad exists ...
    w.grad = None                                   # ... and is dropped
    getattr(ttperf, cls)(store.parameters(), lr=0.1).step()
    assert np.array_equal(store.download(0), before)
    assert np.array_equal(w.master().view(np.uint32), master.view(np.uint32))


def test_sgd_step_bf16_matches_closed_form():
    """tests/sgd_optimizer.py:15-40: bf16 weights, w1 = w0 - 0.1 * (x^T @ ones)."""
    import ttperf
    torch = torch_mod()
    store, w, x, w0 = _linear_store(21, "mixed")
    ref = _oracle_for(store, mode_mixed=True)
    gb = x.to(torch.bfloat16).t() @ torch.ones(32, 32, dtype=torch.bfloat16)
    bits = gb.contiguous().view(torch.int16).numpy().view(np.uint16)
    w.grad = bits
    ref.set_grad(0, bits)
    ttperf.SGD(store.parameters(), lr=0.1).step()
    ref.sgd_step(lr=0.1)
    w_ref = w0 - 0.1 * gb.float()
    assert np.allclose(w.numpy(), w_ref.numpy(), atol=5e-2, rtol=5e-2)  # the reference's bar
    assert np.array_equal(store.download(0), ref.param[:1024])        # bit-exact bf16


def test_sgd_two_steps_bf16():
    """tests/sgd_optimizer.py:43-78: two steps with tanh-derived grads, bf16."""
    import ttperf
    torch = torch_mod()
    store, w, x, w0 = _linear_store(22, "mixed")
    ref = _oracle_for(store, mode_mixed=True)
    opt = ttperf.SGD(store.parameters(), lr=0.1)
    wt = w0.to(torch.bfloat16)
    xb = x.to(torch.bfloat16)
    for _ in range(2):
        z = torch.tanh(xb @ torch.from_numpy(w.numpy().copy()).to(torch.bfloat16))
        g = xb.t() @ (1 - z * z)
        bits = g.contiguous().view(torch.int16).numpy().view(np.uint16)
        w.grad = bits
        ref.set_grad(0, bits)
        opt.step()
        ref.sgd_step(lr=0.1)
        wt = wt - 0.1 * g
    assert np.allclose(w.numpy(), wt.float().numpy(), atol=5e-2, rtol=5e-2)
    assert np.array_equal(store.download(0), ref.param[:1024])


# ---- SGD family at config 2's shapes, both precision modes -------------------------------

SGD_CASES = {
    "plain": dict(lr=1e-2),
    "momentum": dict(lr=1e-2, momentum=0.9),
    "nesterov": dict(lr=1e-2, momentum=0.9, nesterov=True),
    "damp_wd_clip": dict(lr=1e-2, momentum=0.9, dampening=0.1, weight_decay=0.01,
                         max_grad_norm=1.0),
}


# (precision mode, store layout): the mixed store in its default layout ([master|m|v]
# records) and in the SGD layout (contiguous master), and the fp32 store
STORE_KINDS = {"mixed": (O.MODE_MIXED, "default"), "mixed_sgd": (O.MODE_MIXED, "sgd"),
               "fp32": (O.MODE_FP32, "default")}


@pytest.mark.parametrize("kind", list(STORE_KINDS))
@pytest.mark.parametrize("case", list(SGD_CASES))
def test_sgd_family_parity(case, kind):
    from ttperf import configs
    torch = torch_mod()
    mode, layout = STORE_KINDS[kind]
    _, shapes, decay, _ = configs.table("nanogpt_char")
    store, ref = make_pair(shapes, decay, mode, seed=40, layout=layout)
    gen = torch.Generator(device="cuda").manual_seed(41)
    hp = SGD_CASES[case]
    for step in range(3):
        host = device_grads(store, gen, 1e-1 if hp.get("max_grad_norm") else 1e-3, into=ref.grad)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        r = store.sgd_step(report=True, **hp)
        e = ref.sgd_step(**{k: v for k, v in hp.items()})
        assert r["step"] == e["step"] == step + 1
        if hp.get("max_grad_norm"):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
            assert r["clip_coef"] < 1.0
    which = ["master"] + (["param"] if mode == O.MODE_MIXED else [])
    if hp.get("momentum"):
        which.append("momentum")
    compare_state(store, ref, which=tuple(which), max_ulp=2 if hp.get("max_grad_norm") else 0)
    assert store.sgd_layout == (layout == "sgd")


# ---- subsets, missing grads, loss-scale growth, ragged and empty tables --------------------

def test_subset_step_touches_only_listed_tensors():
    """A module's sgd_step / an optimizer over some of a store's tensors: one launch over
    the listed tensors; the clip norm covers the listed tensors only."""
    torch = torch_mod()
    shapes = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049)]
    decay = [True, False, True, False, False, True]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=50)
    gen = torch.Generator(device="cuda").manual_seed(51)
    host = device_grads(store, gen, 1e-2, into=ref.grad)
    listed = [0, 3, 5]
    for i in range(ref.n):
        ref.set_has_grad(i, i in listed)  # the oracle sees only the listed tensors
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.05)
    r = store.adam_step(report=True, indices=listed, **hp)
    e = ref.adam_step(**hp)
    assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-9 * e["grad_norm"]
    compare_state(store, ref, max_ulp=2)
    r = store.sgd_step(report=True, indices=[1, 4], lr=0.5)
    for i in range(ref.n):
        ref.set_has_grad(i, i in (1, 4))
    ref.sgd_step(lr=0.5)
    compare_state(store, ref, which=("master", "param"), max_ulp=2)


def test_none_grad_tensors_untouched_and_out_of_the_norm():
    torch = torch_mod()
    shapes = [(1000,), (64, 64), (77,), (3, 3)]
    store, ref = make_pair(shapes, [False, True, False, True], O.MODE_FP32, seed=52)
    gen = torch.Generator(device="cuda").manual_seed(53)
    host = device_grads(store, gen, 1.0, into=ref.grad)
    for i in range(ref.n):
        ref.set_has_grad(i, True)
    store.tensors[1].grad = None
    ref.set_has_grad(1, False)
    before = store.tensors[1].master().copy()
    hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    r = store.adam_step(report=True, **hp)
    e = ref.adam_step(**hp)
    assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-9 * e["grad_norm"]
    assert np.array_equal(store.tensors[1].master(), before)
    compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=2)
    assert abs(store.grad_norm() - e["grad_norm"]) <= 1e-9 * e["grad_norm"]


def test_scaler_growth_and_backoff_sequence():
    """Tracker forced to growth_interval - 1 through the ABI setter: the next clean step
    doubles the scale; an overflow step halves it, skips, and keeps t."""
    torch = torch_mod()
    shapes = [(4096,), (33, 65)]
    store, ref = make_pair(shapes, [False, True], O.MODE_MIXED, seed=54)
    store.configure_scaler(True, init_scale=1024.0, growth_interval=2000)
    ref.configure_scaler(True, 1024.0, growth_interval=2000)
    store.set_scaler_state(1024.0, 1999)
    ref.set_scaler_state(1024.0, 1999)
    gen = torch.Generator(device="cuda").manual_seed(55)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    expect = [(2048.0, 0, 1, 0), (2048.0, 1, 2, 0), (1024.0, 0, 2, 1), (1024.0, 1, 3, 0)]
    for k, (scale, tracker, t, skipped) in enumerate(expect):
        host = device_grads(store, gen, 1e-3, scale=ref.scale,
                            inf_at=store.offsets[1] + 7 if k == 2 else None, into=ref.grad)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        assert (r["scale"], r["growth_tracker"], r["step"], r["skipped"]) == \
               (scale, tracker, t, skipped) == \
               (e["scale"], e["growth_tracker"], e["step"], e["skipped"])
    compare_state(store, ref, max_ulp=0)


def test_ragged_sizes_and_empty_tensors():
    """Partial vectors (sizes not a multiple of 4/8), chunk boundaries (2047..2049, 4097),
    single elements and zero-element tensors, with loss scaling + clipping."""
    torch = torch_mod()
    sizes = [1, 3, 0, 63, 64, 65, 127, 2047, 2048, 2049, 4097, 0, 5, 10007]
    shapes = [(n,) for n in sizes]
    decay = [i % 2 == 0 for i in range(len(sizes))]
    for mode in (O.MODE_MIXED, O.MODE_FP32):
        store, ref = make_pair(shapes, decay, mode, seed=56)
        store.configure_scaler(True, init_scale=256.0)
        ref.configure_scaler(True, 256.0)
        gen = torch.Generator(device="cuda").manual_seed(57)
        hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.1)
        for _ in range(3):
            host = device_grads(store, gen, 1e-2, scale=ref.scale, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, True)
            r = store.adam_step(report=True, **hp)
            e = ref.adam_step(**hp)
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-9 * e["grad_norm"]
        compare_state(store, ref, max_ulp=2)


def test_empty_store_and_no_grads():
    """No tensors at all, and tensors none of which has a grad: a step launches no update,
    touches nothing, and still advances t (py/optim.py:50 increments before the loop)."""
    import ttperf
    empty = ttperf.ParamStore([], mode="mixed")
    r = empty.adam_step(report=True, lr=1e-3, max_grad_norm=1.0)
    assert r["step"] == 1 and r["grad_norm"] == 0.0
    store = ttperf.ParamStore([(10,), (20,)], mode="fp32")
    store.tensors[0].set_data(np.arange(10, dtype=np.float32))
    r = store.sgd_step(report=True, lr=0.1)
    assert r["step"] == 1
    assert np.array_equal(store.tensors[0].numpy(), np.arange(10, dtype=np.float32))


def test_nan_grad_without_scaler_propagates_like_the_oracle():
    torch = torch_mod()
    store, ref = make_pair([(100,), (50,)], [False, False], O.MODE_MIXED, seed=58)
    gen = torch.Generator(device="cuda").manual_seed(59)
    host = device_grads(store, gen, 1e-2)
    host[store.offsets[1] + 3] = 0x7FC0  # one NaN gradient
    store.upload(1, 0xFFFFFFFF, host)
    ref.grad[:] = host
    for i in range(ref.n):
        ref.set_has_grad(i, True)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, max_grad_norm=1.0)
    r = store.adam_step(report=True, **hp)
    e = ref.adam_step(**hp)
    assert r["found_inf"] == e["found_inf"] == 1 and r["skipped"] == e["skipped"] == 0
    assert np.isnan(r["grad_norm"]) and np.isnan(e["grad_norm"])
    compare_state(store, ref, max_ulp=0)


def test_context_stream_and_timing():
    """Steps on a torch side stream and on the context's own stream agree bit for bit; the
    timing API counts one norm pass and one update per step."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(5000,), (64, 128)]
    outs = []
    for use_side in (False, True):
        store, ref = make_pair(shapes, [False, True], O.MODE_MIXED, seed=60)
        if use_side:
            s = torch.cuda.Stream()
            store.set_stream(s)
        else:
            store.set_stream(None)
        gen = torch.Generator(device="cuda").manual_seed(61)
        device_grads(store, gen, 1e-2)
        store.timing(True)
        for _ in range(4):
            store.adam_step(lr=1e-3, betas=(0.9, 0.95), max_grad_norm=0.5, weight_decay=0.1)
        ms, n = store.timing_collect(L.KERNEL_UPDATE)
        ms2, n2 = store.timing_collect(L.KERNEL_NORM)
        assert n == 4 and n2 == 4 and ms > 0 and ms2 > 0
        outs.append(store.download(L.BUF_MASTER))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


# ---- config 5: GPT-2 XL shapes, full fp32, AdamW + clip then SGD-momentum ------------------

def test_cfg5_gpt2_xl_fp32_adamw_then_sgd_momentum():
    """Config 5: 580 tensors, 1.56B fp32 params (~25 GB resident with m and v, ~31 GB with
    the momentum buffer).  Grads N(0, 1e-3) with 1% drawn from N(0, 1) (clip path active).
    AdamW lr 1.5e-4 betas (0.9, 0.95) wd 0.1 clip 1.0, then SGD momentum 0.9 on the same
    buffers: the configuration's 10 + 10 steps."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, numels = configs.table("gpt2_1558m")
    assert len(shapes) == 580 and sum(numels) == 1557611200
    store, ref = make_pair(shapes, decay, O.MODE_FP32, seed=70)
    gen = torch.Generator(device="cuda").manual_seed(71)
    steps = 10
    hp = dict(lr=1.5e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    for step in range(steps):
        host = device_grads(store, gen, 1e-3, heavy_frac=0.01, heavy_std=1.0, into=ref.grad)
        del host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        assert r["clip_coef"] < 1.0
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        print(f"cfg5 adamw step {step}: norm {r['grad_norm']:.6f}", flush=True)
    compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=2)
    sgd = dict(lr=1e-3, momentum=0.9, max_grad_norm=1.0)
    for step in range(steps):
        host = device_grads(store, gen, 1e-3, heavy_frac=0.01, heavy_std=1.0, into=ref.grad)
        del host
        r = store.sgd_step(report=True, **sgd)
        e = ref.sgd_step(**sgd)
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        print(f"cfg5 sgd-m step {step}: norm {r['grad_norm']:.6f}", flush=True)
    compare_state(store, ref, which=("master", "momentum"), max_ulp=2)


@pytest.mark.parametrize("mode", ["mixed", "mixed_sgd", "fp32"])
def test_update_forms_on_both_sides_of_the_cached_gradient_bound(mode):
    """Mixed-precision updates take their form from the stepped set's gradient bytes: up to
    256 MiB the four-element kernel (SGD momentum) or Adam's 128-lane form, beyond that the
    256-lane lane forms; plain SGD (no momentum) runs its two-element 256-lane form on both
    sides; FP32 updates run the same lane forms (one or two elements per lane) on both sides.
    SGD with momentum and dampening, plain SGD with weight decay, then AdamW, on a store just
    over the bound, each against the oracle: the whole store and a subset that stays over it
    (lane forms with inactive tensors between and after the active ones), then a subset under
    it.  Both stores hold tensors of odd element count, so two-element lanes end on a lone
    element.  "mixed_sgd": the mixed store in the SGD layout (contiguous master, four- and
    two-element SGD lanes, which then end on one to three elements); its first AdamW step
    converts it to the records, from the master the SGD steps left."""
    torch = torch_mod()
    if mode != "fp32":
        shapes = [(50257, 768), (8192, 8192), (7000, 5000), (768,), (3,)]  # 140.7M params
        decay = [True, True, True, False, False]
        subsets = (None, [0, 1, 2], [0, 3, 4])
        store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=80,
                               layout="sgd" if mode == "mixed_sgd" else "default")
        gbytes = 2
    else:
        shapes = [(8193, 8191), (77,), (3,)]  # 67.1M params
        decay = [True, False, False]
        subsets = (None, [0, 2], [1, 2])
        store, ref = make_pair(shapes, decay, O.MODE_FP32, seed=82)
        gbytes = 4
    sizes = [int(np.prod(sh)) for sh in shapes]
    bound = 256 << 20
    assert sum(sizes) * gbytes > bound
    assert sum(sizes[i] for i in subsets[1]) * gbytes > bound
    assert sum(sizes[i] for i in subsets[2]) * gbytes <= bound
    gen = torch.Generator(device="cuda").manual_seed(81)
    sgd = dict(lr=1e-2, momentum=0.9, dampening=0.1, max_grad_norm=1.0)
    plain = dict(lr=1e-2, weight_decay=0.01, max_grad_norm=1.0)
    adam = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    slots = ("master", "param", "momentum") if mode != "fp32" else ("master", "momentum")
    adam_slots = ("master", "exp_avg", "exp_avg_sq") + (("param",) if mode != "fp32" else ())
    for label, subset in zip(("whole store", "lane-form subset", "cached-gradient subset"),
                             subsets):
        for step in range(2):
            host = device_grads(store, gen, 1e-3, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, subset is None or i in subset)
            r = store.sgd_step(report=True, indices=subset, **sgd)
            e = ref.sgd_step(**sgd)
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
            print(f"{mode} {label} sgd-m step {step}: norm {r['grad_norm']:.6f}", flush=True)
        compare_state(store, ref, which=slots, max_ulp=2)
        host = device_grads(store, gen, 1e-3, into=ref.grad)
        for i in range(ref.n):
            ref.set_has_grad(i, subset is None or i in subset)
        r = store.sgd_step(report=True, indices=subset, **plain)
        e = ref.sgd_step(**plain)
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        print(f"{mode} {label} sgd step: norm {r['grad_norm']:.6f}", flush=True)
        compare_state(store, ref, which=slots, max_ulp=2)
        for step in range(2):
            host = device_grads(store, gen, 1e-3, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, subset is None or i in subset)
            r = store.adam_step(report=True, indices=subset, **adam)
            e = ref.adam_step(**adam)
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
            print(f"{mode} {label} adamw step {step}: norm {r['grad_norm']:.6f}", flush=True)
        compare_state(store, ref, which=adam_slots, max_ulp=2)
    store.close()


@pytest.mark.parametrize("mode", ["mixed", "mixed_sgd", "fp32"])
def test_lane_form_update_split_into_several_launches(mode, monkeypatch):
    """A lane-form update over more blocks than one launch may hold runs as several launches
    at increasing part offsets.  TTP_LANE_LAUNCH_BLOCKS (read at ttp_create) lowers that limit
    to 4099 blocks, so that a store just over the 256 MiB bound takes dozens of launches, whose
    boundaries fall inside chunks and tensors; SGD with momentum, plain SGD and AdamW on the
    whole store and on a subset, against the oracle.  In mixed precision also a subset under the bound,
    which MIXED Adam steps in its 128-lane form (37 launches).  "mixed_sgd": the SGD layout's
    SGD forms split the same way, then the AdamW step converts the store."""
    torch = torch_mod()
    monkeypatch.setenv("TTP_LANE_LAUNCH_BLOCKS", "4099")
    if mode != "fp32":
        shapes = [(50257, 768), (8192, 8192), (7000, 5000), (768,), (3,)]
        decay = [True, True, True, False, False]
        subset = [0, 1, 2]
        store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=84,
                               layout="sgd" if mode == "mixed_sgd" else "default")
    else:
        shapes = [(8193, 8191), (77,), (3,)]
        decay = [True, False, False]
        subset = [0, 2]
        store, ref = make_pair(shapes, decay, O.MODE_FP32, seed=85)
    gen = torch.Generator(device="cuda").manual_seed(86)
    sgd = dict(lr=1e-2, momentum=0.9, dampening=0.1, max_grad_norm=1.0)
    plain = dict(lr=1e-2, weight_decay=0.01, max_grad_norm=1.0)
    adam = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    slots = ("master", "param", "momentum") if mode != "fp32" else ("master", "momentum")
    adam_slots = ("master", "exp_avg", "exp_avg_sq") + (("param",) if mode != "fp32" else ())
    legs = [("whole store", None), ("subset", subset)]
    if mode != "fp32":
        legs.append(("cached-gradient subset", [0, 3, 4]))
    for label, sub in legs:
        for name, hp in (("sgd-m", sgd), ("sgd", plain), ("adamw", adam)):
            host = device_grads(store, gen, 1e-3, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, sub is None or i in sub)
            sgd_like = name.startswith("sgd")
            step = store.sgd_step if sgd_like else store.adam_step
            r = step(report=True, indices=sub, **hp)
            e = (ref.sgd_step if sgd_like else ref.adam_step)(**hp)
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
            print(f"{mode} {label} {name}: norm {r['grad_norm']:.6f}", flush=True)
        compare_state(store, ref, which=slots, max_ulp=2)
        compare_state(store, ref, which=adam_slots, max_ulp=2)
    store.close()


@pytest.mark.parametrize("mode", ["mixed", "mixed_sgd", "fp32"])
def test_lane_form_with_many_small_tensors(mode):
    """A store just over the 256 MiB bound made of one large tensor of odd length and 1500
    small ones of 1..200 elements (most chunks hold less than one lane-form piece, many
    blocks have nothing to do): AdamW with loss scaling and clipping, then SGD with Nesterov
    momentum, then plain SGD with weight decay, against the oracle; the second Adam step on a
    subset of every third tensor.  "mixed_sgd": a store created in the SGD layout takes the
    SGD legs first (the layout's own four- and two-element forms over the small tensors), and
    the first AdamW step then converts it."""
    torch = torch_mod()
    rng = np.random.default_rng(87)
    big = (1 << 27) + 3 if mode != "fp32" else (1 << 26) + 5
    small = [int(x) for x in rng.integers(1, 201, size=1500)]
    shapes = [(big,)] + [(n,) for n in small]
    decay = [True] + [bool(x) for x in rng.integers(0, 2, size=len(small))]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED if mode != "fp32" else O.MODE_FP32,
                           seed=88, layout="sgd" if mode == "mixed_sgd" else "default")
    store.configure_scaler(True, init_scale=4096.0)
    ref.configure_scaler(True, 4096.0)
    gen = torch.Generator(device="cuda").manual_seed(89)
    param = ("param",) if mode != "fp32" else ()

    def adam_legs():
        adam = dict(lr=1e-3, betas=(0.9, 0.99), eps=1e-8, weight_decay=0.05, max_grad_norm=0.5)
        subset = list(range(0, len(shapes), 3))
        for step, sub in enumerate((None, subset)):
            device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, sub is None or i in sub)
            r = store.adam_step(report=True, indices=sub, **adam)
            e = ref.adam_step(**adam)
            assert r["skipped"] == e["skipped"] and r["step"] == e["step"]
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
            print(f"{mode} adamw step {step}: norm {r['grad_norm']:.6f}", flush=True)
        compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq") + param, max_ulp=2)

    def sgd_legs():
        sgd = dict(lr=1e-2, momentum=0.9, nesterov=True, max_grad_norm=0.5)
        for step in range(2):
            device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
            for i in range(ref.n):
                ref.set_has_grad(i, True)
            r = store.sgd_step(report=True, **sgd)
            e = ref.sgd_step(**sgd)
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        compare_state(store, ref, which=("master", "momentum") + param, max_ulp=2)
        plain = dict(lr=1e-2, weight_decay=0.01, max_grad_norm=0.5)
        device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
        r = store.sgd_step(report=True, **plain)
        e = ref.sgd_step(**plain)
        assert r["skipped"] == e["skipped"]
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        compare_state(store, ref, which=("master",) + param, max_ulp=2)

    if mode == "mixed_sgd":
        sgd_legs()
        assert store.sgd_layout
        adam_legs()
        assert not store.sgd_layout
    else:
        adam_legs()
        sgd_legs()
    store.close()


def test_zero1_shard_step_matches_oracle():
    """One GPU's ZeRO-1 shard of GPT-2 124M (the last of 8: 28 pieces of tensors, 15.6M
    params) stepped with config 3's mixed AdamW, loss scaling and clipping; against the oracle.
    With sharding, the norm of each shard would be all-reduced; here the shard is its own
    store, so the clip uses the shard's norm on both sides."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, numels = configs.table("gpt2_124m_shard8")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=90)
    store.configure_scaler(True, init_scale=65536.0)
    ref.configure_scaler(True, 65536.0)
    gen = torch.Generator(device="cuda").manual_seed(91)
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    for step in range(3):
        host = device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        r = store.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        assert r["skipped"] == e["skipped"] == 0 and r["step"] == e["step"]
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
    compare_state(store, ref, max_ulp=2)
    store.close()


def test_two_adam_parameter_groups_keep_their_own_step_counts():
    """Two optimizers over two parameter groups of one store, stepped in an uneven order:
    each group's bias corrections use its own optimizer's step count, as two py/optim.py Adam
    instances (:46,50, `_step` per optimizer) would.  The oracle steps one group at a time with
    that group's count; the moments of the other group stay untouched."""
    import ttperf
    torch = torch_mod()
    shapes = [(64, 48), (48,), (48, 32), (32,), (300,)]
    decay = [True, False, True, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=95)
    groups = {"a": [0, 1, 4], "b": [2, 3]}
    hps = {"a": dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1),
           "b": dict(lr=1e-2, betas=(0.8, 0.999), eps=1e-6, weight_decay=0.0)}
    opts = {"a": ttperf.AdamW([store.tensors[i] for i in groups["a"]], **hps["a"]),
            "b": ttperf.Adam([store.tensors[i] for i in groups["b"]],
                             **{k: v for k, v in hps["b"].items() if k != "weight_decay"})}
    counts = {"a": 0, "b": 0}
    gen = torch.Generator(device="cuda").manual_seed(96)
    for k, g in enumerate("aabbbaba"):
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        for i in range(ref.n):
            ref.set_has_grad(i, i in groups[g])
        opts[g].step()
        ref.t = counts[g]
        ref.adam_step(decoupled=(g == "a"), **hps[g])
        counts[g] = ref.t
        print(f"step {k}: group {g}, its count {counts[g]}", flush=True)
        assert store.step_count == counts[g]
    assert counts == {"a": 4, "b": 4}
    compare_state(store, ref, max_ulp=0)
    store.close()


@pytest.mark.parametrize("how", ["defer_first", "defer_all_then_update"])
def test_two_optimizers_share_one_scale_update_per_iteration(how):
    """Loss scaling with two optimizers over two groups of one store, as torch's
    GradScaler.step(opt_a), GradScaler.step(opt_b), GradScaler.update(): each optimizer skips
    on an overflow in its own gradients only, the scale moves once per iteration (backing off
    if either group overflowed, growing after `interval` clean iterations), and each group's
    step count is its own.  Either the first step defers the update to the second, or both
    defer and ParamStore.scaler_update() runs.  Checked against the oracle after every
    iteration (reports, scale, tracker) and in the final state."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(64, 48), (48,), (48, 32), (32,), (300,)]
    decay = [True, False, True, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=97)
    store.configure_scaler(True, init_scale=2.0 ** 12, growth_interval=3)
    ref.configure_scaler(True, 2.0 ** 12, growth_interval=3)
    groups = {"a": [0, 1, 4], "b": [2, 3]}
    hp = dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    opts = {g: ttperf.AdamW([store.tensors[i] for i in groups[g]], **hp) for g in groups}
    counts = {"a": 0, "b": 0}
    inf_in = {3: "a", 5: "b", 8: "ab", 12: "a"}
    gen = torch.Generator(device="cuda").manual_seed(98)
    rng = np.random.default_rng(99)
    scales = []
    for it in range(1, 15):
        inf_at = []
        for g in inf_in.get(it, ""):
            t = groups[g][int(rng.integers(0, len(groups[g])))]
            inf_at.append(store.offsets[t] + int(rng.integers(0, store.tensors[t].numel)))
        host = device_grads(store, gen, 1e-2, scale=ref.scale)
        if inf_at:  # +inf in the chosen groups, on the device and in the oracle's copy
            g16 = store.download(L.BUF_GRAD)
            for k in inf_at:
                g16[k] = 0x7F80  # bf16 +inf
            store.upload(L.BUF_GRAD, L.ALL_TENSORS, g16)
            host = g16
        ref.grad[:store.total] = host
        for g in "ab":
            last = g == "b" and how == "defer_first"
            for i in range(ref.n):
                ref.set_has_grad(i, i in groups[g])
            opts[g].step(update_scale=last)
            ref.t = counts[g]
            e = ref.adam_step(update_scale=last, **hp)
            assert e["skipped"] == (g in inf_in.get(it, "")), (it, g)
            assert e["step"] == counts[g] + (0 if e["skipped"] else 1)
            counts[g] = ref.t
            # the store holds the stepping optimizer's count: a skip leaves it unchanged
            assert store.step_count == e["step"], (it, g)
            assert store.scaler_state() == (e["scale"], e["growth_tracker"]), (it, g)
        if how == "defer_all_then_update":
            store.scaler_update()
            ref.scaler_update()
        scale, tracker = store.scaler_state()
        assert (scale, tracker) == (ref.scale, ref.growth_tracker), it
        scales.append(scale)
        print(f"iteration {it}: overflow in {inf_in.get(it, '-')!r}, scale {scale}, "
              f"tracker {tracker}, counts {counts}", flush=True)
    # an update after the iteration's updating step changes nothing
    store.scaler_update()
    ref.scaler_update()
    assert store.scaler_state() == (ref.scale, ref.growth_tracker) == (scales[-1], tracker)
    # one move per iteration: a backoff at iterations 3, 5, 8 (both groups: once) and 12,
    # growth after the three clean iterations 9-11
    assert scales == [4096.0, 4096.0, 2048.0, 2048.0, 1024.0, 1024.0, 1024.0, 512.0, 512.0,
                      512.0, 1024.0, 512.0, 512.0, 512.0]
    compare_state(store, ref, max_ulp=2)
    store.close()


def test_out_of_memory_is_reported_and_stale_hip_errors_are_not_misattributed():
    """A store larger than the device fails with TTP_ERR_OOM (TTPMemoryError) and leaves no
    trace: HIP keeps a failed call's error as the thread's "last error", which the engine's
    post-launch checks read.  After that failure, and after a failing HIP call of the caller's
    own (hipSetDevice to a device that does not exist), the next store steps normally and
    matches the oracle."""
    import ctypes

    import ttperf
    from ttperf import _lib as L
    with pytest.raises(ttperf.TTPMemoryError) as e:
        ttperf.ParamStore([(1 << 38,)], mode="mixed")  # 3.3 TB of fp32 state records
    assert e.value.code == L.ERR_OOM and "hipMalloc" in str(e.value)
    hip = ctypes.CDLL("libamdhip64.so.7")
    assert hip.hipSetDevice(ctypes.c_int(99)) != 0  # leaves an error in HIP's last-error slot
    store, ref = make_pair([(300, 7), (64,)], [True, False], O.MODE_MIXED, seed=101)
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(102)
    ref.grad[:store.total] = device_grads(store, gen, 1e-2)
    for i in range(ref.n):
        ref.set_has_grad(i, True)
    assert hip.hipSetDevice(ctypes.c_int(99)) != 0
    store.adam_step(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True)
    ref.adam_step(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True)
    compare_state(store, ref, max_ulp=0)
    store.close()


def test_device_transfers_refuse_host_pointers_and_short_buffers():
    """TTP_DEVICE uploads and downloads and device gradient sources are read or written by the
    GPU directly.  A host pointer, or a device buffer shorter than the elements requested, is
    refused on the host (TTP_ERR_INVALID / TTP_ERR_RANGE) before anything is launched, and the
    store is left as it was.  Before each refused call the test checks, through the HIP
    runtime itself, the fact the library's check relies on (the pointer is not device memory;
    the allocation is shorter than the request)."""
    import ctypes

    import ttperf
    from ttperf import _lib as L
    hip = ctypes.CDLL("libamdhip64.so.7")
    store = ttperf.ParamStore([(1 << 20,), (64,)], mode="mixed")
    before = [store.download(b).tobytes() for b in (L.BUF_MASTER, L.BUF_GRAD, L.BUF_PARAM)]
    n = 1 << 20
    host = np.zeros(n, np.float32)
    attr = (ctypes.c_int * 16)()
    if hip.hipPointerGetAttributes(attr, ctypes.c_void_p(host.ctypes.data)) == 0:
        assert attr[0] not in (2, 3), "the runtime calls a numpy buffer device memory"
    hip.hipGetLastError()
    cases = [
        lambda: L.lib.ttp_accumulate_grad(store.handle, 0, host.ctypes.data, n, L.DTYPE_F32,
                                          L.DEVICE),
        lambda: L.lib.ttp_upload(store.handle, L.BUF_MASTER, 0, host.ctypes.data, n, L.DEVICE),
        lambda: L.lib.ttp_download(store.handle, L.BUF_MASTER, 0, host.ctypes.data, n, L.DEVICE),
        lambda: L.lib.ttp_upload(store.handle, L.BUF_GRAD, 0, host.ctypes.data, n, L.DEVICE),
    ]
    for k, call in enumerate(cases):
        assert call() == L.ERR_INVALID, k
        assert "is not device memory" in L.lib.ttp_last_error().decode()
    # a 1 MiB device allocation offered as the 4 MiB fp32 source of tensor 0
    dev = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(dev), ctypes.c_size_t(1 << 20)) == 0
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    assert hip.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), dev) == 0
    assert base.value == dev.value and size.value < 4 * n, size.value
    try:
        for call in (
            lambda: L.lib.ttp_accumulate_grad(store.handle, 0, dev.value, n, L.DTYPE_F32,
                                              L.DEVICE),
            lambda: L.lib.ttp_upload(store.handle, L.BUF_MASTER, 0, dev.value, n, L.DEVICE),
            lambda: L.lib.ttp_download(store.handle, L.BUF_MASTER, 0, dev.value, n, L.DEVICE),
        ):
            assert call() == L.ERR_RANGE
            assert "do not fit its allocation" in L.lib.ttp_last_error().decode()
        # the same buffer is accepted for what fits in it: the 64-element tensor 1
        assert L.lib.ttp_download(store.handle, L.BUF_MASTER, 1, dev.value, 64, L.DEVICE) == 0
        store.sync()
    finally:
        assert hip.hipFree(dev) == 0
    assert [store.download(b).tobytes() for b in (L.BUF_MASTER, L.BUF_GRAD, L.BUF_PARAM)] == before
    assert not store.has_grad(0)
    store.close()


def test_download_into_out_checks_the_buffer():
    """download(..., out=...) fills the caller's buffer in place; one of the wrong size, type
    or layout is refused before anything is written."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    store.tensors[1].set_data(np.arange(512, dtype=np.float32))
    bad = [np.empty(511, np.float32), np.empty(512, np.float64), np.empty(1024, np.float32)[::2],
           torch.empty(511, device="cuda"), torch.empty(1024, device="cuda")[::2],
           torch.empty(512, dtype=torch.bfloat16, device="cuda")]
    for out in bad:
        with pytest.raises(ValueError):
            store.download(L.BUF_MASTER, 1, out=out)
    ro = np.empty(512, np.float32)
    ro.flags.writeable = False
    with pytest.raises(ValueError):
        store.download(L.BUF_MASTER, 1, out=ro)
    good = np.empty(512, np.float32)
    assert store.download(L.BUF_MASTER, 1, out=good) is good
    assert np.array_equal(good, np.arange(512, dtype=np.float32))
    dev = torch.empty(512, device="cuda")
    store.download(L.BUF_MASTER, 1, out=dev)
    assert np.array_equal(dev.cpu().numpy(), good)
    store.close()


def test_store_beyond_2_to_the_32_elements():
    """Offsets past 2^32 elements (64-bit indexing in every kernel and host path): an fp32
    store of one 4.3G-element tensor and one more tensor behind it (69 GB of HBM).  The big
    tensor's first and last 2048 weights and grads are set through zero-copy views, its
    middle stays zero (zero grads leave zero weights and moments unchanged and add nothing to
    the norm), and the second tensor goes through the API's upload, download and accumulate
    paths.  Two clipped AdamW steps over the whole store must match an oracle holding just the
    head, the tail and the second tensor; the moments are read through ttp_buffer_layout's
    addressing."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    big, k = (1 << 32) + 1000, 2048
    store = ttperf.ParamStore([(big,), (4096,)], mode="fp32", decay=[True, False])
    assert store.offsets[1] > (1 << 32)
    ref = O.OracleStore([k, k, 4096], flags=[1, 1, 0], mode=O.MODE_FP32, nthreads=4)
    rng = np.random.default_rng(110)
    master = store.torch_view(L.BUF_MASTER, 0)
    grad = store.torch_view(L.BUF_GRAD, 0)
    head_w, tail_w = [rng.normal(0, 0.02, k).astype(np.float32) for _ in range(2)]
    w1 = rng.normal(0, 0.02, 4096).astype(np.float32)
    master[:k] = torch.from_numpy(head_w).cuda()
    master[-k:] = torch.from_numpy(tail_w).cuda()
    torch.cuda.synchronize()
    store.tensors[1].set_data(w1)
    for i, w in enumerate((head_w, tail_w, w1)):
        ref.set_master(i, w)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True)
    for step in range(2):
        gh, gt, g1 = [(rng.standard_normal(n) * 3e-2).astype(np.float32) for n in (k, k, 4096)]
        grad[:k] = torch.from_numpy(gh).cuda()
        grad[-k:] = torch.from_numpy(gt).cuda()
        torch.cuda.synchronize()
        store.mark_grads([0])
        store.set_has_grad(1, False)
        store.tensors[1].accumulate_grad(g1)  # the accumulate path at an offset past 2^32
        for i, g in enumerate((gh, gt, g1)):
            ref.set_grad(i, g)
        r = store.adam_step(report=True, max_grad_norm=1.0, **hp)
        e = ref.adam_step(max_grad_norm=1.0, **hp)
        print(f"step {step}: norm {r['grad_norm']:.6f} (oracle {e['grad_norm']:.6f})", flush=True)
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
        assert e["clip_coef"] < 1.0  # the clip is active
    torch.cuda.synchronize()

    def check(got, want, what):
        d = f32_ulp_diff(np.ascontiguousarray(got), want)
        assert d.max() <= 2, f"{what}: {d.max()} ulp"

    check(master[:k].cpu().numpy(), ref.view("master", 0), "head master")
    check(master[-k:].cpu().numpy(), ref.view("master", 1), "tail master")
    check(store.download(L.BUF_MASTER, 1), ref.view("master", 2), "tensor 1 master")
    mid = master[k:-k]  # the untouched middle: min and max on the device, no temporaries
    assert float(mid.min()) == 0.0 and float(mid.max()) == 0.0
    for which, name in ((L.BUF_EXP_AVG, "exp_avg"), (L.BUF_EXP_AVG_SQ, "exp_avg_sq")):
        base, group, stride = store.layout(which)
        assert (group, stride) == (64, 128)
        for (lo, hi), i in (((0, k), 0), ((big - k, big), 1)):
            r0, r1 = lo // group, (hi + group - 1) // group
            addr = base + r0 * stride * 4

            class _Records:  # records r0..r1-1 of the slot, as (records, stride) fp32
                __cuda_array_interface__ = {"data": (addr, False),
                                            "shape": (r1 - r0, stride), "typestr": "<f4",
                                            "strides": None, "version": 3}

            recs = torch.as_tensor(_Records(), device="cuda")[:, :group].reshape(-1)
            vals = recs[lo - r0 * group: hi - r0 * group].cpu().numpy()
            check(vals, ref.view(name, i), f"{name} {'head' if i == 0 else 'tail'}")
        check(store.download(which, 1), ref.view(name, 2), f"{name} tensor 1")
    del master, grad, mid
    store.close()
