"""GPU test of ttp_adam_step_noalloc, the Adam step that allocates nothing: its norm pass
keeps its partials in the library's fixed per-device scratch array instead of the context's
buffer.  Called through the C ABI, it must give what ttp_adam_step / ttp_adam_step_subset give
on twin stores (bit for bit: the same kernels and the same summation order), on calls in a row
of which a later one is smaller, so that partials a larger call left in the shared array are
never read; and it must refuse, before queuing any work, whatever would need an allocation."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

HP = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)


def _hp(L, update_scale=True):
    return L.AdamHParams(lr=HP["lr"], beta1=HP["betas"][0], beta2=HP["betas"][1],
                         eps=HP["eps"], weight_decay=HP["weight_decay"], decoupled=1,
                         flags=0 if update_scale else L.STEP_DEFER_SCALE,
                         max_grad_norm=HP["max_grad_norm"])


def _noalloc(store, indices=None):
    from ttperf import _lib as L
    hp = _hp(L)
    if indices is None:
        return L.lib.ttp_adam_step_noalloc(store.handle, C.byref(hp), None, 0)
    idx = (C.c_uint32 * max(len(indices), 1))(*indices)
    return L.lib.ttp_adam_step_noalloc(store.handle, C.byref(hp), idx, len(indices))


def _pair_of_twins(shapes, decay, seed):
    """Two identical loss-scaled mixed-precision stores (the allocating and the no-allocation
    entry point's) plus the oracle's."""
    a, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=seed)
    b, _ = make_pair(shapes, decay, O.MODE_MIXED, seed=seed)
    for s in (a, b):
        s.configure_scaler(True, init_scale=2.0 ** 16)
    ref.configure_scaler(True, 2.0 ** 16)
    return a, b, ref


def _same_grads(a, b, ref, gen, indices=None):
    from ttperf import _lib as L
    host = device_grads(a, gen, 1e-3, scale=ref.scale)
    b.upload(L.BUF_GRAD, L.ALL_TENSORS, host)
    ref.grad[:a.total] = host
    for i in range(ref.n):
        ref.set_has_grad(i, indices is None or i in indices)


def _identical(a, b, what):
    from ttperf import _lib as L
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM):
        assert a.download(which).tobytes() == b.download(which).tobytes(), (what, which)
    assert a.scaler_state() == b.scaler_state(), what
    assert a.step_count == b.step_count, what
    print(f"{what}: bit-identical to the allocating step (scale {a.scaler_state()[0]}, "
          f"t {a.step_count})", flush=True)


def test_noalloc_step_equals_the_allocating_step_on_calls_in_a_row():
    from ttperf import _lib as L
    from ttperf import configs
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(150)
    _, big_shapes, big_decay, _ = configs.table("nanogpt_char")  # ~1300 norm-pass partials
    small_shapes = [(300, 7), (64,), (129, 33), (4097,)]          # a handful
    small_decay = [True, False, True, False]
    A, A2, refA = _pair_of_twins(big_shapes, big_decay, 151)
    B, B2, refB = _pair_of_twins(small_shapes, small_decay, 152)
    sub = [1, 2, 5, 30, 75]
    # set-up with the allocating entry point: the bias table of these betas, and the work
    # tables of the whole stores and of the subset
    for x, x2, r in ((A, A2, refA), (B, B2, refB)):
        _same_grads(x, x2, r, gen)
        x.adam_step(**HP)
        x2.adam_step(**HP)
        r.adam_step(**HP)
    _same_grads(A, A2, refA, gen, indices=sub)
    A.adam_step(indices=sub, **HP)
    A2.adam_step(indices=sub, **HP)
    refA.adam_step(**HP)
    torch.cuda.synchronize()
    _identical(A, A2, "set-up")

    # two no-allocation calls in a row, the second over a smaller store: its norm pass writes
    # a few partials where the first left ~1300
    _same_grads(A, A2, refA, gen)
    _same_grads(B, B2, refB, gen)
    A.adam_step(**HP)
    B.adam_step(**HP)
    assert _noalloc(A2) == L.OK, L.lib.ttp_last_error()
    assert _noalloc(B2) == L.OK, L.lib.ttp_last_error()
    refA.adam_step(**HP)
    refB.adam_step(**HP)
    torch.cuda.synchronize()
    _identical(A, A2, "call 1 (whole nanoGPT store)")
    _identical(B, B2, "call 2 (smaller store)")
    compare_state(A2, refA, max_ulp=2)
    compare_state(B2, refB, max_ulp=2)

    # then a subset call (smaller than the whole store) and an overflow step (skipped, scale
    # backed off) on the big store again
    _same_grads(A, A2, refA, gen, indices=sub)
    A.adam_step(indices=sub, **HP)
    assert _noalloc(A2, sub) == L.OK, L.lib.ttp_last_error()
    refA.adam_step(**HP)
    torch.cuda.synchronize()
    _identical(A, A2, "call 3 (subset of the nanoGPT store)")
    host = device_grads(A, gen, 1e-3, scale=refA.scale, inf_at=int(A.offsets[7]) + 3)
    A2.upload(L.BUF_GRAD, L.ALL_TENSORS, host)
    A.adam_step(**HP)
    assert _noalloc(A2) == L.OK, L.lib.ttp_last_error()
    torch.cuda.synchronize()
    _identical(A, A2, "call 4 (overflow: skipped)")
    assert A2.scaler_state()[0] == refA.scale / 2
    for s in (A, A2, B, B2):
        s.close()


def test_noalloc_step_over_the_infinity_cache_bound():
    """Above 256 MiB of gradients the norm pass runs as two launches (non-temporal, then
    cached loads: about 2850 partials) and the update takes its lane form.  The no-allocation
    step equals the allocating one there too, on a whole-store call followed by a smaller
    subset call that stays over the bound and by one under it."""
    from ttperf import _lib as L
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(170)
    shapes = [(50257, 768), (8192, 8192), (7000, 5000), (768,), (3,)]  # 281 MB of bf16 grads
    decay = [True, True, True, False, False]
    A, A2, refA = _pair_of_twins(shapes, decay, 171)
    del refA  # the allocating entry point is the reference here
    over, under = [0, 1, 2], [0, 3, 4]
    for sub in (None, over, under):  # set-up: bias table and work tables
        _same_grads_no_oracle(A, A2, gen)
        A.adam_step(indices=sub, **HP)
        A2.adam_step(indices=sub, **HP)
    torch.cuda.synchronize()
    _identical(A, A2, "set-up")
    for label, sub in (("whole store", None), ("subset over the bound", over),
                       ("subset under the bound", under)):
        _same_grads_no_oracle(A, A2, gen)
        A.adam_step(indices=sub, **HP)
        assert _noalloc(A2, sub) == L.OK, L.lib.ttp_last_error()
        torch.cuda.synchronize()
        _identical(A, A2, label)
    A.close()
    A2.close()


def _same_grads_no_oracle(a, b, gen):
    from ttperf import _lib as L
    host = device_grads(a, gen, 1e-3, scale=a.scaler_state()[0])
    b.upload(L.BUF_GRAD, L.ALL_TENSORS, host)


def test_noalloc_step_refuses_what_it_would_have_to_allocate():
    """Each refusal comes before any work is queued and leaves the store as it was."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(160)
    shapes, decay = [(300, 7), (64,), (129, 33)], [True, False, True]

    def refused(store, code, words, indices=None):
        t0 = store.step_count
        master = store.download(L.BUF_MASTER).tobytes()
        assert _noalloc(store, indices) == code
        msg = L.lib.ttp_last_error().decode()
        assert all(w in msg for w in words), msg
        assert store.step_count == t0 and store.download(L.BUF_MASTER).tobytes() == master
        print(f"refused as expected: {msg}", flush=True)

    store, _ = make_pair(shapes, decay, O.MODE_MIXED, seed=161)
    store.configure_scaler(True, init_scale=1024.0)
    device_grads(store, gen, 1e-3, scale=1024.0)
    refused(store, L.ERR_STATE, ["bias-correction table"])   # betas never stepped
    store.adam_step(**HP)
    refused(store, L.ERR_STATE, ["work table"], indices=[0, 2])  # a set never stepped
    assert _noalloc(store) == L.OK, L.lib.ttp_last_error()
    store.close()

    fp32, _ = make_pair(shapes, decay, O.MODE_FP32, seed=162)
    device_grads(fp32, gen, 1e-3)
    refused(fp32, L.ERR_STATE, ["allocates m and v"])  # FP32 m and v do not exist yet
    fp32.close()

    old = os.environ.get("TTP_NORM_GRID")
    os.environ["TTP_NORM_GRID"] = "16384"  # read at ttp_create
    try:
        # 2^26 + 2^24 bf16 gradients: 10240 norm tiles of 16 KiB
        big = ttperf.ParamStore([(1 << 26,), (1 << 24,)], mode="mixed", decay=[True, True])
    finally:
        if old is None:
            del os.environ["TTP_NORM_GRID"]
        else:
            os.environ["TTP_NORM_GRID"] = old
    device_grads(big, gen, 1e-3)
    big.adam_step(**HP)
    refused(big, L.ERR_RANGE, ["10240 partials", "8192"])
    big.close()


def test_captured_noalloc_step_replays_like_the_eager_step():
    """The entry point's first callers: code under HIP graph capture.  A no-allocation step
    with loss scaling and clipping over a store just above the 256 MiB bound (so the
    two-launch norm pass writes its ~2850 partials into the scratch array) is captured, then
    replayed four times with new gradients, one holding +inf (skipped, scale halved); each
    replay is bit-compared with an eager ttp_adam_step on a twin store, with eager work of the
    program (gradient uploads and synchronisations) between the replays.  Around an eager
    no-allocation call the device's free memory does not change."""
    from ttperf import _lib as L
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(180)
    shapes = [(50257, 768), (8192, 8192), (7000, 5000), (768,), (3,)]  # 281 MB of bf16 grads
    decay = [True, True, True, False, False]
    A, A2, refA = _pair_of_twins(shapes, decay, 181)
    del refA
    A2.set_stream(None)  # the store's own stream: capturable
    for _ in range(2):  # set-up with the allocating entry point: bias and work tables
        _same_grads_no_oracle(A, A2, gen)
        A.adam_step(**HP)
        A2.adam_step(**HP)
    torch.cuda.synchronize()
    _identical(A, A2, "set-up")
    # an eager no-allocation call allocates nothing on the device
    _same_grads_no_oracle(A, A2, gen)
    A.adam_step(**HP)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    assert _noalloc(A2) == L.OK, L.lib.ttp_last_error()
    A2.sync()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
    _identical(A, A2, "eager no-allocation step")
    A2.begin_capture()
    assert _noalloc(A2) == L.OK, L.lib.ttp_last_error()
    graph = A2.end_capture()
    for k in range(4):
        inf_at = int(A.offsets[1]) + 4321 if k == 2 else None
        host = device_grads(A, gen, 1e-3, scale=A.scaler_state()[0], inf_at=inf_at)
        A2.upload(L.BUF_GRAD, L.ALL_TENSORS, host)
        A2.sync()
        r = A.adam_step(report=True, **HP)
        graph.replay()
        A2.sync()
        assert r["skipped"] == (k == 2)
        _identical(A, A2, f"replay {k}")
    graph.close()
    A.close()
    A2.close()


def test_noalloc_steps_of_two_stores_on_two_streams():
    """Two stores on two torch streams take eager no-allocation steps in turn, without any
    synchronisation between the calls: the library orders each call after the previous one
    on the shared scratch array, so each store ends bit-identical to its allocating twin."""
    from ttperf import _lib as L
    from ttperf import configs
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(190)
    _, shapes, decay, _ = configs.table("nanogpt_char")
    A, A2, _ = _pair_of_twins(shapes, decay, 191)
    B, B2, _ = _pair_of_twins(shapes, decay, 192)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    A2.set_stream(s1)
    B2.set_stream(s2)
    for x, x2 in ((A, A2), (B, B2)):
        _same_grads_no_oracle(x, x2, gen)
        x.adam_step(**HP)
        x2.adam_step(**HP)
    torch.cuda.synchronize()
    for k in range(6):
        for x, x2 in ((A, A2), (B, B2)):
            _same_grads_no_oracle(x, x2, gen)
        torch.cuda.synchronize()
        A.adam_step(**HP)
        B.adam_step(**HP)
        assert _noalloc(A2) == L.OK, L.lib.ttp_last_error()
        assert _noalloc(B2) == L.OK, L.lib.ttp_last_error()
    torch.cuda.synchronize()
    _identical(A, A2, "store on stream 1")
    _identical(B, B2, "store on stream 2")
    for s in (A, A2, B, B2):
        s.close()


def test_noalloc_step_refuses_to_convert_the_sgd_layout():
    """A mixed store in the SGD layout has no m and v until its first Adam step converts it;
    the no-allocation step refuses that step, with the store unchanged."""
    from ttperf import _lib as L
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(195)
    store, _ = make_pair([(300, 7), (64,)], [True, False], O.MODE_MIXED, seed=196, layout="sgd")
    device_grads(store, gen, 1e-3)
    master = store.download(L.BUF_MASTER).tobytes()
    assert _noalloc(store) == L.ERR_STATE
    msg = L.lib.ttp_last_error().decode()
    assert "SGD layout" in msg and "allocates m and v" in msg, msg
    assert store.sgd_layout and store.download(L.BUF_MASTER).tobytes() == master
    store.close()
