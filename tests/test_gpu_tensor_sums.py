"""GPU tests of bucketed gradient sums (ttp_grad_sumsq_tensors) and steps that take their norm
from them (TTP_STEP_TENSOR_SUMS) instead of running a norm pass.

The per-tensor sums add the same squares as the norm pass in another order, so the norm may
differ in its last bits and the clip coefficient, rarely, by one rounding: the state is held
to the oracle within the 2-ulp bar of the other parity tests, and to an eager twin that runs
the norm pass.  Skip / found_inf / scale / step-count decisions must be identical."""
import numpy as np
import pytest

import oracle as O
from conftest import f32_ulp_diff
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

SHAPES = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049), (4097,), (96, 64), (0,),
          (40000,), (3,), (8192, 3)]
DECAY = [len(s) == 2 for s in SHAPES]


def _buckets(n, size=4):
    """Reverse tensor order in buckets, as a backward produces them."""
    order = list(range(n))[::-1]
    return [sorted(order[k:k + size]) for k in range(0, n, size)]


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_step_from_bucket_sums_matches_oracle_and_norm_pass(mode):
    import ttperf
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, mode, seed=120)
    twin, _ = make_pair(SHAPES, DECAY, mode, seed=120)  # the same step with its norm pass
    scaler = mode == O.MODE_MIXED
    if scaler:
        for s in (store, twin):
            s.configure_scaler(True, init_scale=1024.0, growth_interval=2)
        ref.configure_scaler(True, 1024.0, growth_interval=2)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(121)
    from ttperf import _lib as L
    for step in range(6):
        inf_at = store.offsets[9] + 77 if (scaler and step == 3) else None
        host = device_grads(store, gen, 1e-2, scale=ref.scale if scaler else 1.0, inf_at=inf_at)
        twin.upload(L.BUF_GRAD, L.ALL_TENSORS, store.download(L.BUF_GRAD))
        ref.grad[:store.total] = host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        for b in _buckets(len(SHAPES)):
            store.grad_sumsq_tensors(b)
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        rt = twin.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        print(f"step {step}: norm {r['grad_norm']!r} (norm pass {rt['grad_norm']!r}, oracle "
              f"{e['grad_norm']!r}), skipped {r['skipped']}", flush=True)
        for k in ("skipped", "found_inf", "step", "scale", "growth_tracker"):
            assert r[k] == rt[k] == e[k], (k, r, rt, e)
        if np.isfinite(e["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
        compare_state(store, ref, max_ulp=2)
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ):
        a, b = store.download(which), twin.download(which)
        assert f32_ulp_diff(a, b).max() <= 2
    store.close()
    twin.close()


@pytest.mark.parametrize("config,ntensors,nparams", [("gpt2_124m", 148, 124439808),
                                                     ("gpt2_774m", 436, 774030080)])
def test_bucket_sums_at_full_size(config, ntensors, nparams):
    """Configs 3 and 4 at their real shapes (bf16 gradients; at 774M the update takes its lane
    form): loss scaling, clipping and AdamW, the norm taken from bench.py's buckets (25 MB of
    gradients each, in reverse tensor order), with an overflow at a seeded index on the second
    step.  Against the oracle: the same skip / scale / step decisions, the norm within 1e-10
    relative, the state within 2 ulp."""
    from ttperf import configs
    from ttperf import _lib as L
    torch = torch_mod()
    _, shapes, decay, numels = configs.table(config)
    assert len(shapes) == ntensors and sum(numels) == nparams
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=132)
    store.configure_scaler(True, init_scale=65536.0)
    ref.configure_scaler(True, 65536.0)
    buckets, cur, cur_bytes = [], [], 0
    for i in reversed(range(len(numels))):
        cur.append(i)
        cur_bytes += numels[i] * 2
        if cur_bytes >= 25 << 20:
            buckets.append(sorted(cur))
            cur, cur_bytes = [], 0
    if cur:
        buckets.append(sorted(cur))
    assert sorted(i for b in buckets for i in b) == list(range(len(numels)))
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    gen = torch.Generator(device="cuda").manual_seed(133)
    for step in range(3):
        # a weight matrix in the middle of the table (GPT-2 124M: h.6 attn.c_attn.weight)
        inf_at = store.offsets[ntensors // 2 + 2] + 12345 if step == 1 else None
        device_grads(store, gen, 1e-3, scale=ref.scale, inf_at=inf_at, into=ref.grad)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        for b in buckets:
            store.grad_sumsq_tensors(b)
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        e = ref.adam_step(**hp)
        print(f"step {step}: {len(buckets)} buckets, norm {r['grad_norm']!r} (oracle "
              f"{e['grad_norm']!r}), skipped {r['skipped']}, scale {r['scale']}", flush=True)
        for k in ("skipped", "found_inf", "step", "scale", "growth_tracker"):
            assert r[k] == e[k], (k, r, e)
        assert r["skipped"] == (step == 1)
        if np.isfinite(e["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
    compare_state(store, ref, max_ulp=2)
    store.close()


def test_sgd_momentum_subset_step_from_sums():
    """SGD with momentum over a subset: only the subset's tensors need sums."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=122)
    gen = torch.Generator(device="cuda").manual_seed(123)
    subset = [0, 2, 4, 9, 11]
    hp = dict(lr=1e-2, momentum=0.9, max_grad_norm=0.3)
    for step in range(4):
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        store.grad_sumsq_tensors(subset)
        for i in range(ref.n):
            ref.set_has_grad(i, i in subset)
        r = store.sgd_step(report=True, indices=subset, tensor_sums=True, **hp)
        e = ref.sgd_step(**hp)
        assert r["step"] == e["step"]
        assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
        compare_state(store, ref, which=("master", "momentum"), max_ulp=2)
    store.close()


def test_stale_or_missing_sums_are_refused():
    """A step with tensor_sums fails (TTP_ERR_STATE, nothing queued, nothing changed) unless
    every tensor it updates has a sum taken after its last gradient write and after the
    previous step."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=124)
    gen = torch.Generator(device="cuda").manual_seed(125)
    device_grads(store, gen, 1e-2)
    hp = dict(lr=1e-3, max_grad_norm=1.0, tensor_sums=True)

    def refused(why):
        t0 = store.step_count
        master = store.download(L.BUF_MASTER).tobytes()
        with pytest.raises(ttperf.TTPError) as e:
            store.adam_step(**hp)
        assert e.value.code == L.ERR_STATE and "no current gradient sum" in str(e.value), why
        assert store.step_count == t0 and store.download(L.BUF_MASTER).tobytes() == master, why

    refused("no sums taken")
    store.grad_sumsq_tensors(range(6))
    refused("sums of some tensors only")
    store.grad_sumsq_tensors()
    store.adam_step(**hp)  # current sums: accepted
    refused("a step consumed the sums")
    # a step consumes the sums of the tensors it updates only: without a scale update the
    # others stay current, for the iteration's other optimizers
    store.grad_sumsq_tensors()
    store.adam_step(indices=[0, 1, 2], **hp)
    refused("the first group's sums were consumed")
    store.adam_step(indices=[3, 4, 5, 6, 7], **hp)
    for write in (lambda: store.tensors[2].__setattr__("grad", np.zeros(129 * 33, np.uint16)),
                  lambda: store.tensors[3].accumulate_grad(np.ones(5, np.float32)),
                  lambda: store.mark_grads([4]),
                  lambda: store.zero_grad(set_to_none=False, indices=[7]),
                  lambda: store.configure_scaler(True, init_scale=512.0)):
        store.grad_sumsq_tensors()
        write()
        refused("a gradient write or scale change after the sums")
    store.grad_sumsq_tensors()
    store.adam_step(**hp)
    # without clipping or loss scaling there is no norm to take: the flag is accepted
    store.configure_scaler(False)
    store.adam_step(lr=1e-3, tensor_sums=True)
    bad = L.AdamHParams(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, flags=4)
    assert L.lib.ttp_adam_step(store.handle, bad, None) == L.ERR_INVALID
    store.close()


def test_graph_of_bucket_sums_and_step_replays():
    """The bucket sums and the step captured together: each replay (new gradients copied in
    between, outside the graph) matches an eager twin that runs the norm pass, and the oracle."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=126)
    twin, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=126)
    for s in (store, twin):
        s.set_stream(None)
        s.configure_scaler(True, init_scale=4096.0, growth_interval=3)
    ref.configure_scaler(True, 4096.0, growth_interval=3)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.5)
    buckets = _buckets(len(SHAPES))
    gen = torch.Generator(device="cuda").manual_seed(127)
    graph = None
    for it in range(5):
        host = device_grads(store, gen, 1e-2, scale=ref.scale)
        twin.upload(L.BUF_GRAD, L.ALL_TENSORS, store.download(L.BUF_GRAD))
        ref.grad[:store.total] = host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        if it == 0:  # eager once: work tables, tile buffer and bias table exist
            for b in buckets:
                store.grad_sumsq_tensors(b)
            store.adam_step(tensor_sums=True, **hp)
        else:
            if graph is None:
                store.begin_capture()
                for b in buckets:
                    store.grad_sumsq_tensors(b)
                store.adam_step(tensor_sums=True, **hp)
                graph = store.end_capture()
            graph.replay()
        twin.adam_step(**hp)
        ref.adam_step(**hp)
        store.sync()
        print(f"iteration {it}: step {store.step_count}, scale {store.scaler_state()[0]}",
              flush=True)
        assert store.step_count == twin.step_count == ref.t
        assert store.scaler_state() == twin.scaler_state()
        compare_state(store, ref, max_ulp=2)
        for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ):
            assert f32_ulp_diff(store.download(which), twin.download(which)).max() <= 2
    graph.close()
    store.close()
    twin.close()


def test_sums_freshness_follows_graph_launches():
    """Captured calls change which sums are current when their graph is launched, not when
    they are captured: captured sums make nothing current until a launch, a launched step
    consumes sums, and a graph whose step reads sums taken before its capture is refused at
    launch (nothing queued, nothing changed) unless they are current.  Every accepted step
    matches the oracle."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=130)
    store.set_stream(None)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.05)
    gen = torch.Generator(device="cuda").manual_seed(131)

    def grads():
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        for i in range(ref.n):
            ref.set_has_grad(i, True)

    def refused(fn, why):
        t0 = store.step_count
        master = store.download(L.BUF_MASTER).tobytes()
        with pytest.raises(ttperf.TTPError) as e:
            fn()
        assert e.value.code == L.ERR_STATE and "no current gradient sum" in str(e.value), why
        assert store.step_count == t0, why
        assert store.download(L.BUF_MASTER).tobytes() == master, why
        print(f"refused as expected: {why}", flush=True)

    def eager_step():
        store.adam_step(tensor_sums=True, **hp)
        ref.adam_step(**hp)
        compare_state(store, ref, max_ulp=2)

    grads()
    store.grad_sumsq_tensors()
    eager_step()  # eager once: work tables, tile buffer and bias table exist
    # a graph of sums alone: its capture makes nothing current, its launch does
    grads()
    store.begin_capture()
    store.grad_sumsq_tensors()
    sums_graph = store.end_capture()
    refused(lambda: store.adam_step(tensor_sums=True, **hp), "the captured sums have not run")
    sums_graph.replay()
    eager_step()
    # a graph of a step reading sums taken before its capture
    grads()
    store.grad_sumsq_tensors()
    store.begin_capture()
    store.adam_step(tensor_sums=True, **hp)
    step_graph = store.end_capture()
    eager_step()  # the capture ran nothing: the eager sums are still current
    refused(step_graph.replay, "the eager step consumed the sums the graph reads")
    grads()
    sums_graph.replay()  # current sums of the new gradients
    step_graph.replay()
    ref.adam_step(**hp)
    store.sync()
    assert store.step_count == ref.t
    compare_state(store, ref, max_ulp=2)
    refused(lambda: store.adam_step(tensor_sums=True, **hp), "the launched step consumed them")
    refused(step_graph.replay, "the launched step consumed them")
    sums_graph.close()
    step_graph.close()
    store.close()


def test_growing_the_tile_buffer_keeps_captured_graphs_valid():
    """A captured bucket-sum call writes the tile buffer it was captured with.  An eager call
    over a larger bucket grows that buffer while the graph is alive; the old one is kept until
    the store closes, so the graph's replays stay correct (against the oracle), and so does
    the eager step that uses the new buffer."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=128)
    store.set_stream(None)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.05)
    small = [0, 1]  # one 16 KiB tile each: the smallest tile buffer
    gen = torch.Generator(device="cuda").manual_seed(129)

    def grads(active):
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        for i in range(ref.n):
            ref.set_has_grad(i, i in active)

    grads(small)
    store.grad_sumsq_tensors(small)
    store.adam_step(indices=small, tensor_sums=True, **hp)
    ref.adam_step(**hp)
    store.begin_capture()
    store.grad_sumsq_tensors(small)
    store.adam_step(indices=small, tensor_sums=True, **hp)
    graph = store.end_capture()
    for it in range(3):
        grads(list(range(len(SHAPES))))
        store.grad_sumsq_tensors()  # every tensor: a larger tile buffer while the graph lives
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        e = ref.adam_step(**hp)
        assert r["step"] == e["step"]
        compare_state(store, ref, max_ulp=2)
        grads(small)
        graph.replay()
        store.sync()
        ref.adam_step(**hp)
        print(f"round {it}: replay after growth, step {store.step_count}", flush=True)
        assert store.step_count == ref.t
        compare_state(store, ref, max_ulp=2)
    graph.close()
    store.close()


def test_optimizer_step_with_tensor_sums():
    """The drop-in AdamW's step(tensor_sums=True) after bucket sums matches the same optimizer
    stepping with its norm pass, within 2 ulp, and is refused without current sums."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    a, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=130)
    b, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=130)
    oa = ttperf.AdamW(a.parameters(), lr=1e-3, weight_decay=0.1, max_grad_norm=0.2)
    ob = ttperf.AdamW(b.parameters(), lr=1e-3, weight_decay=0.1, max_grad_norm=0.2)
    gen = torch.Generator(device="cuda").manual_seed(131)
    for _ in range(3):
        device_grads(a, gen, 1e-2)
        b.upload(L.BUF_GRAD, L.ALL_TENSORS, a.download(L.BUF_GRAD))
        for bucket in _buckets(len(SHAPES)):
            a.grad_sumsq_tensors(bucket)
        oa.step(tensor_sums=True)
        ob.step()
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ):
        assert f32_ulp_diff(a.download(which), b.download(which)).max() <= 2
    with pytest.raises(ttperf.TTPError):
        oa.step(tensor_sums=True)  # the last step consumed the sums
    a.close()
    b.close()


def test_bucket_sums_on_a_side_stream_wait_for_the_backward():
    """The documented side-stream pattern: the backward writes each bucket's gradients on its
    own stream (through the zero-copy grad views, after a long GEMM standing in for its
    compute) and records an event; the bucket sums run on a side stream, each after its
    bucket's event; the step follows on the side stream once the whole backward is done.  A
    sum that ran before its event would see the zeroed gradients, and the clip would differ
    from the twin's."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=132)
    twin, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=132)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.05)
    main, side = torch.cuda.Stream(), torch.cuda.Stream()
    gen = torch.Generator(device="cuda").manual_seed(133)
    a = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
    views = [store.torch_view(L.BUF_GRAD, i) for i in range(len(SHAPES))]  # 1-D views
    buckets = _buckets(len(SHAPES))
    for it in range(3):
        src = [(torch.randn(t.numel, generator=gen, device="cuda") * 1e-2).to(torch.bfloat16)
               for t in store.tensors]
        torch.cuda.synchronize()
        store.set_stream(side)
        store.zero_grad(set_to_none=False)  # the previous iteration's grads are gone
        store.mark_grads()  # the grads about to be written: marked before their sums
        store.sync()
        events = []
        with torch.cuda.stream(main):
            for b in buckets:
                for _ in range(3):
                    torch.mm(a, a)  # the backward's compute before this bucket is ready
                for i in b:
                    views[i].copy_(src[i])
                ev = torch.cuda.Event()
                ev.record(main)
                events.append(ev)
        for b, ev in zip(buckets, events):
            side.wait_event(ev)
            store.grad_sumsq_tensors(b)
        side.wait_stream(main)
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        torch.cuda.synchronize()
        for i, t in enumerate(twin.tensors):
            twin.upload(L.BUF_GRAD, i, src[i])
        rt = twin.adam_step(report=True, **hp)
        print(f"iteration {it}: norm {r['grad_norm']!r} (twin {rt['grad_norm']!r})", flush=True)
        assert abs(r["grad_norm"] - rt["grad_norm"]) <= 1e-12 * rt["grad_norm"]
        assert r["clip_coef"] == rt["clip_coef"] < 1.0
        for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ):
            assert f32_ulp_diff(store.download(which), twin.download(which)).max() <= 2
    del views
    store.close()
    twin.close()


def test_step_from_sums_of_more_tensors_than_one_finalize_round():
    """The finalize sums at most 8 x 256 partials per round; a step over 3000 tensors takes its
    norm from 3000 per-tensor sums, read through the tensor list in two rounds, with loss
    scaling and clipping (and an overflow on one step), against the oracle and a twin that
    runs the norm pass."""
    torch = torch_mod()
    rng = np.random.default_rng(130)
    shapes = [(int(n),) for n in rng.integers(1, 300, size=3000)]
    decay = [bool(x) for x in rng.integers(0, 2, size=len(shapes))]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=131)
    twin, _ = make_pair(shapes, decay, O.MODE_MIXED, seed=131)
    for s in (store, twin):
        s.configure_scaler(True, init_scale=256.0, growth_interval=2)
    ref.configure_scaler(True, 256.0, growth_interval=2)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(132)
    from ttperf import _lib as L
    for step in range(4):
        inf_at = store.offsets[2500] if step == 2 else None
        host = device_grads(store, gen, 1e-2, scale=ref.scale, inf_at=inf_at)
        twin.upload(L.BUF_GRAD, L.ALL_TENSORS, store.download(L.BUF_GRAD))
        ref.grad[:store.total] = host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        for b in _buckets(len(shapes), size=700):
            store.grad_sumsq_tensors(b)
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        rt = twin.adam_step(report=True, **hp)
        e = ref.adam_step(**hp)
        print(f"step {step}: norm {r['grad_norm']!r} (norm pass {rt['grad_norm']!r}, oracle "
              f"{e['grad_norm']!r}), skipped {r['skipped']}", flush=True)
        for k in ("skipped", "found_inf", "step", "scale", "growth_tracker"):
            assert r[k] == rt[k] == e[k], (k, r, rt, e)
        if np.isfinite(e["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
        compare_state(store, ref, max_ulp=2)
    store.close()
    twin.close()


def _bits(t):
    """A torch tensor's host copy in the oracle's types (bf16 bits or float32)."""
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_accumulate_with_sums_feeds_a_tensor_sums_step(mode):
    """The gradient producer's side of the bucketed norm: a backward accumulates two
    gradients into every tensor (assign, then add), the second with TTP_ACCUM_SUMSQ, which
    stores the tensor's sum of squares of its resulting gradients in the same launch; the
    step then takes its norm from those sums (no norm pass, no bucket call).  Sources vary:
    device bf16 / fp32, host fp32 / bf16 bits, and a device source that is not 16-byte aligned.
    Against the oracle (orc_accumulate_grad, then its own norm): gradients bit-exact, the
    same skip / found_inf / scale / step decisions, the norm within 1e-10, the state within
    2 ulp; against a twin store given the same accumulates without sums and a bucket-sums
    call over every tensor: the norm and the whole state bit-identical (the sums are the same
    tile for tile).  With loss scaling (mixed), an incoming +inf on step 2 makes the sum
    non-finite and the step skip.  An accumulate without sums after one with them leaves the
    tensor's sum stale, and the step is refused."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, mode, seed=140)
    twin, _ = make_pair(SHAPES, DECAY, mode, seed=140)
    mixed = mode == O.MODE_MIXED
    if mixed:
        for s in (store, twin):
            s.configure_scaler(True, init_scale=512.0, growth_interval=2)
        ref.configure_scaler(True, 512.0, growth_interval=2)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(141)
    n = len(SHAPES)
    for step in range(5):
        scale = ref.scale if mixed else 1.0
        for s in (store, twin):
            s.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)
        for i in reversed(range(n)):  # the order a backward produces them
            numel = store.tensors[i].numel
            g1 = torch.randn(numel, generator=gen, device="cuda") * 1e-2 * scale
            g1 = g1.to(torch.bfloat16) if mixed else g1
            g2 = (torch.randn(numel, generator=gen, device="cuda") * 1e-2 * scale)
            if mixed and step == 2 and i == 9:
                g2[77] = float("inf")
            if i == 5:  # a device source at an odd address: element-wise loads
                buf = torch.zeros(numel + 1, device="cuda", dtype=torch.float32)
                buf[1:] = g2
                src2 = buf[1:]
                assert src2.data_ptr() % 16
                host2 = _bits(src2)
            elif mixed:
                src2 = host2 = g2.cpu().numpy()  # host fp32 into bf16 gradients
            else:
                src2 = host2 = _bits(g2.to(torch.bfloat16))  # host bf16 bits into fp32
            for s in (store, twin):
                s.accumulate_grad(i, g1)
            store.accumulate_grad(i, src2, sums=True)
            twin.accumulate_grad(i, src2)
            ref.accumulate_grad(i, _bits(g1))
            ref.accumulate_grad(i, host2)
        twin.grad_sumsq_tensors(list(range(n)))
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        rt = twin.adam_step(report=True, tensor_sums=True, **hp)
        e = ref.adam_step(**hp)
        print(f"step {step}: norm {r['grad_norm']!r} (bucket sums {rt['grad_norm']!r}, oracle "
              f"{e['grad_norm']!r}), skipped {r['skipped']}", flush=True)
        for k in ("skipped", "found_inf", "step", "scale", "growth_tracker"):
            assert r[k] == rt[k] == e[k], (k, r, rt, e)
        assert r["skipped"] == (mixed and step == 2)
        assert np.array_equal(np.float64(r["grad_norm"]), np.float64(rt["grad_norm"])) or \
            not np.isfinite(rt["grad_norm"])
        if np.isfinite(e["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
        got = store.download(L.BUF_GRAD)
        assert np.array_equal(got.view(np.uint8), ref.grad[:store.total].view(np.uint8))
        compare_state(store, ref, max_ulp=2)
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM):
        assert np.array_equal(store.download(which).view(np.uint8),
                              twin.download(which).view(np.uint8)), which
    # a later accumulate without sums makes that tensor's sum stale: refused, nothing changed
    store.accumulate_grad(3, np.ones(store.tensors[3].numel, np.float32), sums=True)
    store.accumulate_grad(3, np.ones(store.tensors[3].numel, np.float32))
    t0 = store.step_count
    with pytest.raises(ttperf.TTPError) as err:
        store.adam_step(tensor_sums=True, indices=[3], **hp)
    assert err.value.code == L.ERR_STATE and store.step_count == t0
    store.close()
    twin.close()


def test_captured_accumulates_with_sums_and_step_replay():
    """A backward's accumulates with their sums and the step from those sums captured as one
    graph (zero_grad to None, one accumulate per tensor from device memory, the AdamW step
    with loss scaling and clipping), replayed four times with new source gradients (one with
    +inf), each against the oracle; eager steps from bucket sums between the replays, and the
    first replay before any eager accumulate with sums (the captured step combines the pending
    tile sums whatever the eager history)."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=150)
    store.set_stream(None)  # the store's own stream: capturable
    store.configure_scaler(True, init_scale=256.0, growth_interval=3)
    ref.configure_scaler(True, 256.0, growth_interval=3)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(151)
    n = len(SHAPES)
    srcs = [torch.zeros(store.tensors[i].numel, device="cuda", dtype=torch.bfloat16)
            for i in range(n)]

    def refill(inf=False):
        for i in range(n):
            srcs[i].copy_((torch.randn(srcs[i].numel(), generator=gen, device="cuda") * 1e-2
                           * ref.scale).to(torch.bfloat16))
        if inf:
            srcs[6][11] = float("inf")
        torch.cuda.synchronize()

    def ref_iteration():
        ref.zero_grad(set_to_none=True)
        for i in reversed(range(n)):
            ref.accumulate_grad(i, _bits(srcs[i]))
        return ref.adam_step(**hp)

    # one eager Adam step builds the work and bias tables a capture cannot build
    ref.grad[:store.total] = device_grads(store, gen, 1e-2, scale=ref.scale)
    for i in range(n):
        ref.set_has_grad(i, True)
    store.adam_step(**hp)
    ref.adam_step(**hp)
    store.begin_capture()
    store.zero_grad(set_to_none=True)
    for i in reversed(range(n)):
        store.accumulate_grad(i, srcs[i], sums=True)
    store.adam_step(tensor_sums=True, **hp)
    graph = store.end_capture()
    for k in range(4):
        refill(inf=(k == 2))
        graph.replay()
        e = ref_iteration()
        store.sync()
        print(f"replay {k}: oracle norm {e['grad_norm']!r}, skipped {e['skipped']}", flush=True)
        assert store.step_count == e["step"]
        assert store.scaler_state() == (np.float32(e["scale"]), e["growth_tracker"])
        assert e["skipped"] == (k == 2)
        compare_state(store, ref, max_ulp=2)
        # an eager step from bucket sums in between
        ref.grad[:store.total] = device_grads(store, gen, 1e-2, scale=ref.scale)
        for i in range(n):
            ref.set_has_grad(i, True)
        store.grad_sumsq_tensors(list(range(n)))
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        e = ref.adam_step(**hp)
        assert (r["skipped"], r["step"], r["scale"]) == (e["skipped"], e["step"], e["scale"])
        compare_state(store, ref, max_ulp=2)
    graph.close()
    store.close()
