"""GPU tests of the BF16 store (TTP_MODE_BF16): the reference C++ autograd's own storage, bf16
weights and gradients with no fp32 state, stepped by its plain SGD with each ttnn op's bf16
rounding, `data = RNE(data - RNE(grad * lr))` (autograd/dynamic/optim.hpp:21-27,
autograd/traced/ops.hpp:132-134 on BFLOAT16 tensors, autograd/dynamic/autograd.hpp:72).

Checked against the oracle bit for bit: the reference's own test formulas
(tests/sgd_optimizer.py, whose expected weights torch computes in bf16), GPT-2 124M's and
774M's tables with loss scaling, an overflow, clipping and a module-sized subset step, accumulation per
tensor and in buckets with the step's norm from their sums, a captured step replayed between
eager ones, and a checkpoint round trip; the calls that would need fp32 state are refused
with nothing changed.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from conftest import golden
from gpu_util import device_grads, make_pair, pad_mask, torch_mod

pytestmark = pytest.mark.gpu


def _set_all(ref, active=None):
    for i in range(ref.n):
        ref.set_has_grad(i, active is None or i in active)


def _check(r, e, scaler):
    assert (r["skipped"], r["found_inf"], r["step"]) == (e["skipped"], e["found_inf"], e["step"])
    if scaler:
        assert (r["scale"], r["growth_tracker"]) == (e["scale"], e["growth_tracker"])
    assert np.float32(r["clip_coef"]) == np.float32(e["clip_coef"])
    if np.isfinite(e["grad_norm"]) and e["grad_norm"] > 0:
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]


def _same_weights(store, ref, what):
    from ttperf import _lib as L
    mask = pad_mask(store)
    got = store.download(L.BUF_PARAM)[mask]
    want = ref.param[:store.total][mask]
    bad = int(np.count_nonzero(got != want))
    print(f"  {what}: {bad} of {got.size} bf16 weights differ", flush=True)
    assert bad == 0, f"{what}: {bad} bf16 weights differ"


def test_reference_sgd_test_formulas_bit_for_bit():
    """tests/sgd_optimizer.py:15-39 and :42-78: the expected weights the reference's tests
    compute with torch in bf16 (`w - 0.1 * grad`), from the fixtures' own weights and
    gradients, one step and two steps, equal bit for bit; and the drop-in SGD of py/optim.py
    equal to torch's run of that file's own three ops on bf16 tensors."""
    import ttperf
    from ttperf import _lib as L
    d = golden("reference_known_answers.npz")
    store = ttperf.ParamStore([(32, 32)], mode="bf16")
    store.upload(L.BUF_PARAM, 0, d["sgd1_w0"].ravel())
    store.upload(L.BUF_GRAD, 0, d["sgd1_grad"].ravel())
    store.sgd_step(lr=0.1)
    assert np.array_equal(store.download(L.BUF_PARAM, 0), d["sgd1_w1"].ravel())
    store.upload(L.BUF_PARAM, 0, d["sgd2_w0"].ravel())
    for g, w in (("sgd2_g1", "sgd2_w1"), ("sgd2_g2", "sgd2_w2")):
        store.upload(L.BUF_GRAD, 0, d[g].ravel())
        store.sgd_step(lr=0.1)
        assert np.array_equal(store.download(L.BUF_PARAM, 0), d[w].ravel()), w
    # the drop-in py/optim.py SGD (ttperf.SGD) on the same weights: py/optim.py:19 fills lr
    # into a bf16 tensor, so the step equals torch's run of full_like / mul / sub on bf16
    # tensors (lr 0.1 rounded to 0.10009765625)
    store.upload(L.BUF_PARAM, 0, d["sgd1_w0"].ravel())
    store.upload(L.BUF_GRAD, 0, d["sgd1_grad"].ravel())
    ttperf.SGD(store.parameters(), lr=0.1).step()
    assert np.array_equal(store.download(L.BUF_PARAM, 0), d["sgd_pyopt_w1"].ravel())
    store.close()


def test_gpt2_124m_plain_sgd_matches_the_oracle():
    """Config 3's 148 tensors in a BF16 store: plain SGD with loss scaling (2^16, growth every
    3 clean steps) and clipping at 1.0, a +inf on step 3 (skipped, scale halved); then one
    block's 12 tensors stepped alone (a module's sgd_step), and steps without scaling or
    clipping.  Every bf16 weight equal to the oracle's after every step."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, _ = configs.table("gpt2_124m")
    store, ref = make_pair(shapes, decay, O.MODE_BF16, seed=400)
    store.configure_scaler(True, init_scale=65536.0, growth_interval=3)
    ref.configure_scaler(True, 65536.0, growth_interval=3)
    gen = torch.Generator(device="cuda").manual_seed(401)
    hp = dict(lr=1e-2, max_grad_norm=1.0)
    for step in range(6):
        inf_at = store.offsets[40] + 17 if step == 3 else None
        device_grads(store, gen, 1e-3, scale=ref.scale, inf_at=inf_at, into=ref.grad)
        _set_all(ref)
        r = store.sgd_step(report=True, **hp)
        e = ref.sgd_step(**hp)
        print(f"  step {step}: skipped {e['skipped']} scale {e['scale']:g} "
              f"norm {e['grad_norm']:.6g}", flush=True)
        _check(r, e, True)
        assert e["skipped"] == (step == 3)
        _same_weights(store, ref, f"step {step}")
    block = list(range(2, 14))
    device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
    _set_all(ref, block)
    _check(store.sgd_step(report=True, indices=block, **hp), ref.sgd_step(**hp), True)
    _same_weights(store, ref, "module subset")
    store.configure_scaler(False)
    ref.configure_scaler(False)
    for step in range(2):
        device_grads(store, gen, 1e-1, into=ref.grad)
        _set_all(ref)
        store.sgd_step(lr=0.05)
        ref.sgd_step(lr=0.05)
        _same_weights(store, ref, f"unscaled step {step}")
    store.close()


def test_gpt2_774m_plain_sgd_at_full_size():
    """Config 4's table (436 tensors, 774,030,080 params) in a BF16 store, the reference's own
    storage at the largest model its configurations hold that a BF16 store takes: plain SGD
    with loss scaling and clipping at 1.0 for five steps, a +inf on step 2 (skipped, scale
    halved), then a step without either.  Every bf16 weight equal to the oracle's after every
    step, the reports equal."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, _ = configs.table("gpt2_774m")
    store, ref = make_pair(shapes, decay, O.MODE_BF16, seed=410)
    print(f"  {store.total} elements in {len(shapes)} tensors", flush=True)
    store.configure_scaler(True, init_scale=65536.0, growth_interval=2)
    ref.configure_scaler(True, 65536.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(411)
    hp = dict(lr=1e-2, max_grad_norm=1.0)
    for step in range(5):
        inf_at = store.offsets[300] + 1234 if step == 2 else None
        device_grads(store, gen, 1e-3, scale=ref.scale, inf_at=inf_at, into=ref.grad)
        _set_all(ref)
        r = store.sgd_step(report=True, **hp)
        e = ref.sgd_step(**hp)
        print(f"  step {step}: skipped {e['skipped']} scale {e['scale']:g} "
              f"norm {e['grad_norm']:.6g} clip {e['clip_coef']:.6g}", flush=True)
        _check(r, e, True)
        assert e["skipped"] == (step == 2)
        _same_weights(store, ref, f"step {step}")
    store.configure_scaler(False)
    ref.configure_scaler(False)
    device_grads(store, gen, 1e-1, into=ref.grad)
    _set_all(ref)
    store.sgd_step(lr=0.05)
    ref.sgd_step(lr=0.05)
    _same_weights(store, ref, "unscaled step")
    store.close()


@pytest.mark.parametrize("multi", [False, True])
@pytest.mark.parametrize("src", ["bf16", "f32"])
def test_accumulate_then_step_from_sums(multi, src):
    """Gradients accumulated into a BF16 store (assign, then add: rounded once to bf16), one
    call per tensor or one bucket call, with their sums; then a step with clipping and loss
    scaling that takes its norm from those sums, against the oracle."""
    torch = torch_mod()
    shapes = [(300, 7), (64,), (129, 33), (5,), (4097,), (1,)]
    decay = [True, False, True, False, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_BF16, seed=410)
    store.configure_scaler(True, init_scale=1024.0, growth_interval=2)
    ref.configure_scaler(True, 1024.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(411)
    dt = torch.bfloat16 if src == "bf16" else torch.float32
    hp = dict(lr=0.02, max_grad_norm=0.5)
    for it in range(3):
        store.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)
        for _ in range(2):
            vals = [(torch.randn(t.numel, generator=gen, device="cuda") * 1e-2 * ref.scale).to(dt)
                    for t in store.tensors]
            for i, v in enumerate(vals):
                ref.accumulate_grad(i, v.view(torch.int16).cpu().numpy().view(np.uint16)
                                    if src == "bf16" else v.cpu().numpy())
            if multi:
                store.accumulate_grads(list(range(len(vals))), vals, sums=True)
            else:
                for i, v in enumerate(vals):
                    store.accumulate_grad(i, v, sums=True)
        from ttperf import _lib as L
        mask = pad_mask(store)
        assert np.array_equal(store.download(L.BUF_GRAD)[mask], ref.grad[:store.total][mask])
        r = store.sgd_step(report=True, tensor_sums=True, **hp)
        e = ref.sgd_step(**hp)
        _check(r, e, True)
        _same_weights(store, ref, f"iteration {it}")
    store.close()


def test_captured_step_replays_between_eager_steps(tmp_path):
    """A clipped, loss-scaled SGD step captured on a BF16 store, replayed with new gradients
    (one holding +inf) and eager steps in between, each against the oracle; then a checkpoint
    of the store loads into a fresh store byte for byte and both continue equal to the
    oracle."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(300, 7), (64,), (129, 33), (5,), (4097,)]
    decay = [True, False, True, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_BF16, seed=420)
    store.set_stream(None)  # the store's own stream: capturable
    store.configure_scaler(True, init_scale=256.0, growth_interval=2)
    ref.configure_scaler(True, 256.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(421)
    hp = dict(lr=0.02, max_grad_norm=0.5)
    device_grads(store, gen, 1e-2, scale=ref.scale, into=ref.grad)
    _set_all(ref)
    _check(store.sgd_step(report=True, **hp), ref.sgd_step(**hp), True)  # builds the tables
    store.begin_capture()
    store.sgd_step(**hp)
    graph = store.end_capture()
    for k in range(3):
        device_grads(store, gen, 1e-2, scale=ref.scale,
                     inf_at=store.offsets[2] + 9 if k == 1 else None, into=ref.grad)
        _set_all(ref)
        graph.replay()
        e = ref.sgd_step(**hp)
        store.sync()
        assert store.step_count == e["step"]
        assert store.scaler_state() == (np.float32(e["scale"]), e["growth_tracker"])
        _same_weights(store, ref, f"replay {k}")
        device_grads(store, gen, 1e-2, scale=ref.scale, into=ref.grad)
        _set_all(ref)
        _check(store.sgd_step(report=True, lr=0.01), ref.sgd_step(lr=0.01), True)
        _same_weights(store, ref, f"eager step after replay {k}")
    graph.close()
    path = tmp_path / "bf16.ttp"
    store.save_state(path)
    fresh = ttperf.ParamStore(shapes, mode="bf16", decay=decay)
    fresh.load_state(path)
    assert np.array_equal(fresh.download(L.BUF_PARAM), store.download(L.BUF_PARAM))
    assert fresh.step_count == store.step_count
    assert fresh.scaler_state() == store.scaler_state()
    for s in (store, fresh):
        s.upload(L.BUF_GRAD, L.ALL_TENSORS, ref.grad[:store.total])
    _set_all(ref)
    e = ref.sgd_step(**hp)
    for s, name in ((store, "resumed-from store"), (fresh, "loaded store")):
        _check(s.sgd_step(report=True, **hp), e, True)
        _same_weights(s, ref, name)
    store.close()
    fresh.close()


def test_refusals_change_nothing():
    """What needs fp32 state is refused with TTP_ERR_INVALID and changes nothing: Adam (both
    entry points and the no-allocation step), SGD with momentum or weight decay, the master,
    moment and momentum buffers in every transfer and address call, and TTP_STORE_SGD at
    create.  The weights and gradients themselves are contiguous and addressable, and torch
    views alias them."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(64, 3), (10,)]
    store, ref = make_pair(shapes, [True, False], O.MODE_BF16, seed=430)
    gen = torch.Generator(device="cuda").manual_seed(431)
    device_grads(store, gen, 1e-2, into=ref.grad)
    before = store.download(L.BUF_PARAM).copy()
    t0 = store.step_count
    for call in (lambda: store.adam_step(lr=1e-3),
                 lambda: store.adam_step(lr=1e-3, indices=[0]),
                 lambda: store.sgd_step(lr=0.1, momentum=0.9),
                 lambda: store.sgd_step(lr=0.1, weight_decay=0.01),
                 lambda: store.sgd_step(lr=0.1, momentum=0.9, nesterov=True),
                 lambda: store.download(L.BUF_MASTER),
                 lambda: store.download(L.BUF_EXP_AVG),
                 lambda: store.upload(L.BUF_MASTER, L.ALL_TENSORS,
                                      np.zeros(store.total, np.float32)),
                 lambda: store.upload(L.BUF_MOMENTUM, 0, np.zeros(192, np.float32)),
                 lambda: store.ptr(L.BUF_MASTER, 0),
                 lambda: store.ptr(L.BUF_MOMENTUM, 0),
                 lambda: store.layout(L.BUF_EXP_AVG_SQ)):
        with pytest.raises(ttperf.TTPValueError) as e:
            call()
        assert e.value.code == L.ERR_INVALID
    hp = L.AdamHParams(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8)
    assert L.lib.ttp_adam_step_noalloc(store._h, C.byref(hp), None, 0) == L.ERR_INVALID
    assert store.step_count == t0
    assert np.array_equal(store.download(L.BUF_PARAM), before)
    h = C.c_void_p()
    desc = (L.TensorDesc * 1)()
    desc[0].numel = 8
    assert L.lib.ttp_create(0, desc, 1, L.MODE_BF16 | L.STORE_SGD, C.byref(h)) == L.ERR_INVALID
    # the weights and gradients: contiguous bf16, aliased by torch views
    base, group, stride = store.layout(L.BUF_PARAM)
    assert (group, stride) == (64, 64) and store.ptr(L.BUF_PARAM, 1) == base + store.offsets[1] * 2
    view = store.torch_view(L.BUF_PARAM)
    assert view.dtype == torch.bfloat16 and view.data_ptr() == base
    assert np.array_equal(view.view(torch.int16).cpu().numpy().view(np.uint16), before)
    gview = store.torch_view(L.BUF_GRAD)
    assert gview.dtype == torch.bfloat16
    _set_all(ref)
    store.sgd_step(lr=0.1)
    ref.sgd_step(lr=0.1)
    _same_weights(store, ref, "after the refusals")
    store.close()


def test_split_launches_and_many_small_tensors(monkeypatch):
    """The BF16 update over more blocks than one launch may hold runs as several launches at
    increasing part offsets: TTP_LANE_LAUNCH_BLOCKS (read at ttp_create) lowers that limit to
    4099 blocks, so the store below takes dozens of launches whose boundaries fall inside
    chunks and tensors.  The store mixes two large tensors of odd sizes with 600 tensors of
    1..200 elements (most chunks hold less than one piece of 512 elements, and many lanes end
    inside a tensor's last word).  Plain SGD with loss scaling and clipping over the whole
    store and over a subset of every third tensor, against the oracle."""
    torch = torch_mod()
    monkeypatch.setenv("TTP_LANE_LAUNCH_BLOCKS", "4099")
    rng = np.random.default_rng(440)
    small = [(int(n),) for n in rng.integers(1, 201, size=600)]
    shapes = [(50257, 768), (7001, 4999)] + small + [(3,)]
    decay = [True, True] + [False] * (len(small) + 1)
    store, ref = make_pair(shapes, decay, O.MODE_BF16, seed=441)
    store.configure_scaler(True, init_scale=4096.0, growth_interval=2)
    ref.configure_scaler(True, 4096.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(442)
    hp = dict(lr=1e-2, max_grad_norm=1.0)
    subset = list(range(0, len(shapes), 3))
    for label, sub in (("whole store", None), ("subset", subset), ("whole store", None)):
        device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
        _set_all(ref, sub)
        _check(store.sgd_step(report=True, indices=sub, **hp), ref.sgd_step(**hp), True)
        _same_weights(store, ref, label)
    store.close()
