"""GPU tests of the SGD layout of a mixed store (TTP_STORE_SGD): a contiguous fp32 master and
no m / v, which the update of the reference's own optimizer (autograd::SGD, TracedSGD, every
module's sgd_step: `w - lr*g`, autograd/dynamic/optim.hpp:21-27) and SGD with momentum stream
like a copy.

Checked against the oracle at GPT-2 124M (config 3's table) and at GPT-2 774M (config 4's):
plain SGD (the reference's) and SGD with momentum, with loss scaling, an overflow step and
clipping, whole-store steps and module-sized subset steps; the raw device memory of the
master against ttp_buffer_layout's addressing; a captured SGD step replayed between eager
steps; and the conversion to the default layout by the first Adam step.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu


def _set_all(ref, active=None):
    for i in range(ref.n):
        ref.set_has_grad(i, active is None or i in active)


def _check(r, e, scaler):
    assert (r["skipped"], r["found_inf"], r["step"]) == (e["skipped"], e["found_inf"], e["step"])
    if scaler:
        assert (r["scale"], r["growth_tracker"]) == (e["scale"], e["growth_tracker"])
    if np.isfinite(e["grad_norm"]) and e["grad_norm"] > 0:
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]


def test_gpt2_124m_plain_and_momentum_sgd_match_the_oracle():
    """Config 3's 148 tensors in the SGD layout: the reference's plain SGD with loss scaling
    (2^16, growth every 3 clean steps) and clipping at 1.0, a +inf on step 3 (skipped, scale
    halved); then one block's 12 tensors stepped alone (a module's sgd_step); then SGD with
    momentum 0.9 over everything.  bf16 weights bit-exact, master and momentum within 2 ulp,
    identical skip / scale / step decisions, norm within 1e-5."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, _ = configs.table("gpt2_124m")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=300, layout="sgd")
    assert store.sgd_layout
    store.configure_scaler(True, init_scale=65536.0, growth_interval=3)
    ref.configure_scaler(True, 65536.0, growth_interval=3)
    gen = torch.Generator(device="cuda").manual_seed(301)
    plain = dict(lr=1e-2, max_grad_norm=1.0)
    for step in range(6):
        inf_at = store.offsets[40] + 17 if step == 3 else None
        device_grads(store, gen, 1e-3, scale=ref.scale, inf_at=inf_at, into=ref.grad)
        _set_all(ref)
        r = store.sgd_step(report=True, **plain)
        e = ref.sgd_step(**plain)
        print(f"  plain step {step}: skipped {e['skipped']} scale {e['scale']:g} "
              f"norm {e['grad_norm']:.6g}", flush=True)
        _check(r, e, True)
        assert e["skipped"] == (step == 3)
    compare_state(store, ref, which=("master", "param"), max_ulp=2)
    block = list(range(2 + 12 * 5, 2 + 12 * 6))  # h.5's tensors
    device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
    _set_all(ref, block)
    r = store.sgd_step(report=True, indices=block, lr=0.05)
    e = ref.sgd_step(lr=0.05)
    _check(r, e, True)
    compare_state(store, ref, which=("master", "param"), max_ulp=2)
    mom = dict(lr=1e-2, momentum=0.9, max_grad_norm=1.0)
    for step in range(3):
        device_grads(store, gen, 1e-3, scale=ref.scale, into=ref.grad)
        _set_all(ref)
        r = store.sgd_step(report=True, **mom)
        e = ref.sgd_step(**mom)
        _check(r, e, True)
    compare_state(store, ref, which=("master", "param", "momentum"), max_ulp=2)
    assert store.sgd_layout
    store.close()


def test_gpt2_774m_sgd_layout_matches_the_oracle():
    """Config 4's 436 ragged tensors (1,280 to 64.3M elements) in the SGD layout: plain SGD
    with clipping, then SGD with momentum and dampening; the norm pass takes its two launches
    (non-temporal, then cached) above 256 MiB of gradients."""
    from ttperf import configs
    torch = torch_mod()
    _, shapes, decay, _ = configs.table("gpt2_774m")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=310, layout="sgd")
    gen = torch.Generator(device="cuda").manual_seed(311)
    legs = [dict(lr=1e-2, max_grad_norm=1.0)] * 2 + \
        [dict(lr=1e-2, momentum=0.9, dampening=0.1, max_grad_norm=1.0)] * 2
    for k, hp in enumerate(legs):
        device_grads(store, gen, 1e-3, into=ref.grad)
        _set_all(ref)
        r = store.sgd_step(report=True, **hp)
        e = ref.sgd_step(**hp)
        print(f"  step {k} {hp}: norm {e['grad_norm']:.6g}", flush=True)
        _check(r, e, False)
    compare_state(store, ref, which=("master", "param", "momentum"), max_ulp=2)
    store.close()


def test_sgd_layout_matches_raw_device_memory():
    """ttp_buffer_layout reports the master as contiguous (group = stride = 64), and the raw
    device memory at that base, read with hipMemcpy, equals the master download; the pointer
    of each tensor is base + offset * 4."""
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(1,), (63,), (65,), (7, 9), (130,), (64, 64), (3,)]
    decay = [False, False, False, True, False, True, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=320, layout="sgd")
    gen = torch.Generator(device="cuda").manual_seed(321)
    for _ in range(2):
        device_grads(store, gen, 1e-2, into=ref.grad)
        _set_all(ref)
        store.sgd_step(lr=0.1, momentum=0.5)
        ref.sgd_step(lr=0.1, momentum=0.5)
    compare_state(store, ref, which=("master", "param", "momentum"), max_ulp=0)
    base, group, stride = store.layout(L.BUF_MASTER)
    assert (group, stride) == (64, 64)
    for i in range(len(shapes)):
        assert store.ptr(L.BUF_MASTER, i) == base + store.offsets[i] * 4
    torch.cuda.synchronize()
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.restype = C.c_int
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    raw = np.empty(store.total, np.float32)
    assert hip.hipMemcpy(raw.ctypes.data, base, store.total * 4, 2) == 0
    assert np.array_equal(raw.view(np.uint32), store.download(L.BUF_MASTER).view(np.uint32))
    store.close()


def test_captured_sgd_step_replays_between_eager_steps():
    """A plain SGD step with loss scaling captured on an SGD-layout store, replayed three
    times with new gradients (one holding +inf) and eager momentum-free steps in between, each
    against the oracle; the store keeps its layout, and the first Adam step's conversion waits
    until the graph is gone."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(300, 7), (64,), (129, 33), (5,), (4097,)]
    decay = [True, False, True, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=330, layout="sgd")
    store.set_stream(None)  # the store's own stream: capturable
    store.configure_scaler(True, init_scale=256.0, growth_interval=2)
    ref.configure_scaler(True, 256.0, growth_interval=2)
    gen = torch.Generator(device="cuda").manual_seed(331)
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
        compare_state(store, ref, which=("master", "param"), max_ulp=2)
        device_grads(store, gen, 1e-2, scale=ref.scale, into=ref.grad)
        _set_all(ref)
        _check(store.sgd_step(report=True, lr=0.01), ref.sgd_step(lr=0.01), True)
        compare_state(store, ref, which=("master", "param"), max_ulp=2)
    assert store.sgd_layout
    with pytest.raises(ttperf.TTPError) as e:
        store.adam_step(lr=1e-3)
    assert e.value.code == L.ERR_STATE and store.sgd_layout
    graph.close()
    adam = dict(lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1)
    device_grads(store, gen, 1e-2, scale=ref.scale, into=ref.grad)
    _set_all(ref)
    _check(store.adam_step(report=True, **adam), ref.adam_step(**adam), True)
    assert not store.sgd_layout
    compare_state(store, ref, max_ulp=2)
    store.close()


def test_refused_calls_leave_the_sgd_layout():
    """A call that is refused changes nothing, the layout included: the conversion to the
    record layout (which moves the master, so that a master pointer taken before is no longer
    valid) comes after every check that can refuse the call.  Refused here: Adam steps (from
    tensor sums made stale by a later gradient write, over an unknown tensor index, with bad
    hyperparameters) and the buffer calls that would otherwise convert for m or v; each
    leaves the layout, the master pointer and the state as they were.  A valid step then
    converts the store and matches the oracle."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(52, 58), (54, 61), (913,)]
    decay = [True, True, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=340, layout="sgd")
    gen = torch.Generator(device="cuda").manual_seed(341)
    device_grads(store, gen, 1e-2, into=ref.grad)
    _set_all(ref)
    master_ptr = store.ptr(L.BUF_MASTER)
    hp = dict(lr=5e-4, betas=(0.9, 0.999), weight_decay=0.05, max_grad_norm=0.5)
    store.grad_sumsq_tensors([0])
    store.grad_sumsq_tensors([1, 2])
    g = torch.randn(store.tensors[1].numel, generator=gen, device="cuda") * 1e-2
    store.accumulate_grad(1, g)  # tensor 1's sum is now stale
    ref.accumulate_grad(1, g.cpu().numpy())
    refusals = [(dict(hp, tensor_sums=True), None, L.ERR_STATE),
                (hp, [0, 7], L.ERR_RANGE),
                (dict(hp, lr=0.0), None, L.ERR_INVALID)]
    for kw, idx, code in refusals:
        with pytest.raises(ttperf.TTPError) as err:
            store.adam_step(indices=idx, **kw)
        assert err.value.code == code, (kw, idx, err.value)
        assert store.sgd_layout and store.ptr(L.BUF_MASTER) == master_ptr
        assert store.step_count == 0
        compare_state(store, ref, which=("master", "param"), max_ulp=0)
    # the buffer calls that would convert for m or v, refused for something else first (raw
    # C ABI calls, so that the library's own checks answer): m has no plain pointer in either
    # layout; a transfer of the wrong size, of an unknown tensor, or with a host pointer where
    # device memory is declared
    h = store.handle
    buf = np.zeros(store.total + 1, np.float32)
    out = C.c_void_p()
    calls = [(L.lib.ttp_buffer_ptr(h, L.BUF_EXP_AVG, L.ALL_TENSORS, C.byref(out)), L.ERR_STATE),
             (L.lib.ttp_buffer_ptr(h, L.BUF_EXP_AVG_SQ, 0, C.byref(out)), L.ERR_STATE),
             (L.lib.ttp_upload(h, L.BUF_EXP_AVG, L.ALL_TENSORS, buf.ctypes.data, store.total + 1,
                               L.HOST), L.ERR_RANGE),
             (L.lib.ttp_download(h, L.BUF_EXP_AVG_SQ, 7, buf.ctypes.data, 3, L.HOST), L.ERR_RANGE),
             (L.lib.ttp_upload(h, L.BUF_EXP_AVG, 2, buf.ctypes.data, 913, L.DEVICE),
              L.ERR_INVALID)]
    for k, (rc, code) in enumerate(calls):
        assert rc == code, (k, rc, code)
        assert store.sgd_layout and store.ptr(L.BUF_MASTER) == master_ptr, k
    _check(store.adam_step(report=True, **hp), ref.adam_step(**hp), True)
    assert not store.sgd_layout
    compare_state(store, ref, max_ulp=2)
    store.close()


def test_refused_momentum_steps_allocate_nothing(tmp_path):
    """The SGD side of the same rule: a momentum step refused for stale tensor sums leaves
    the store without a momentum buffer, so a checkpoint taken after it holds the master only
    (buffer mask 1 at byte 20 of the state file's header); the valid step that follows
    allocates it, and the next checkpoint holds it (mask 1 | 8)."""
    import struct
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    shapes = [(52, 58), (54, 61), (913,)]
    decay = [True, True, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=350, layout="sgd")
    gen = torch.Generator(device="cuda").manual_seed(351)
    device_grads(store, gen, 1e-2, into=ref.grad)
    _set_all(ref)
    hp = dict(lr=0.01, momentum=0.9, max_grad_norm=0.5)
    store.grad_sumsq_tensors()
    store.zero_grad(set_to_none=False, indices=[2])  # tensor 2's sum is now stale
    ref.grad[store.offsets[2]:store.offsets[2] + store.tensors[2].numel] = 0
    with pytest.raises(ttperf.TTPError) as err:
        store.sgd_step(tensor_sums=True, **hp)
    assert err.value.code == L.ERR_STATE
    mask = lambda p: struct.unpack_from("<I", p.read_bytes(), 20)[0]
    store.save_state(tmp_path / "a.bin")
    assert mask(tmp_path / "a.bin") == 1 and store.step_count == 0
    _check(store.sgd_step(report=True, **hp), ref.sgd_step(**hp), False)
    store.save_state(tmp_path / "b.bin")
    assert mask(tmp_path / "b.bin") == 1 | 8
    compare_state(store, ref, which=("master", "param", "momentum"), max_ulp=2)
    store.close()
