"""GPU tests of graph capture/replay (the counterpart of traced::TraceContext,
autograd/traced/trace.hpp:21-88) and of gradient accumulation into the flat grad buffer
(Value::accumulate_grad, autograd/dynamic/autograd.hpp:78-83), through the C ABI, against
eager steps of the same engine and the CPU oracle.

Every replay is followed by the program's own eager work (new gradients copied in, host
synchronisation) and is checked on its own, not only after the last one.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

SHAPES = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049), (4097,)]
DECAY = [True, False, True, False, False, True, False]


def _bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


def _same_grads(stores, gen, std, scale=1.0, inf_at=None, mixed=True):
    """One seeded gradient tensor on the device, copied into every store's grad buffer."""
    import torch
    from ttperf import _lib as L
    total = stores[0].total
    g = torch.randn(total, generator=gen, device="cuda") * std * scale
    if inf_at is not None:
        g[inf_at] = float("inf")
    g = g.to(torch.bfloat16) if mixed else g
    for s in stores:
        s.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
    host = g.cpu()
    return host.view(torch.int16).numpy().view(np.uint16) if mixed else host.numpy()


@pytest.mark.parametrize("scaler", [False, True])
@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_adam_graph_replays_match_eager_and_oracle(mode, scaler):
    from ttperf import _lib as L
    torch = torch_mod()
    mixed = mode == O.MODE_MIXED
    eager, ref = make_pair(SHAPES, DECAY, mode, seed=90)
    graphed, _ = make_pair(SHAPES, DECAY, mode, seed=90)
    graphed.set_stream(None)  # the context's own stream (the legacy stream cannot be captured)
    if scaler:
        for s in (eager, graphed):
            s.configure_scaler(True, init_scale=1024.0)
        ref.configure_scaler(True, 1024.0)
    gen = torch.Generator(device="cuda").manual_seed(91)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.05)

    def oracle_step(host):
        ref.grad[:] = host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        return ref.adam_step(**hp)

    # one eager step on both (allocates m/v, builds tables and the bias table)
    host = _same_grads([eager, graphed], gen, 1e-2, scale=ref.scale, mixed=mixed)
    eager.adam_step(**hp)
    graphed.adam_step(**hp)
    oracle_step(host)

    graphed.begin_capture()
    graphed.adam_step(**hp)
    graph = graphed.end_capture()
    for k in range(5):
        inf_at = graphed.offsets[2] + 11 if (scaler and k == 2) else None
        host = _same_grads([eager, graphed], gen, 1e-2, scale=ref.scale, inf_at=inf_at,
                           mixed=mixed)
        eager.adam_step(**hp)
        graph.replay()
        graphed.sync()
        e = oracle_step(host)
        for buf in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM):
            assert _bits_equal(graphed.download(buf), eager.download(buf)), (k, buf)
        assert graphed.step_count == eager.step_count == ref.t
        if scaler:
            assert graphed.scaler_state() == eager.scaler_state() == (ref.scale, ref.growth_tracker)
            assert e["skipped"] == (k == 2)
    compare_state(graphed, ref, max_ulp=2)
    graph.close()
    graphed.close()


@pytest.mark.parametrize("mode,opt", [(O.MODE_MIXED, "adamw"), (O.MODE_FP32, "adamw"),
                                      (O.MODE_FP32, "sgdm")])
def test_graph_replays_over_the_cache_bound(mode, opt):
    """A captured step over a store just above 256 MiB of gradients: a two-launch norm pass
    and a lane-form update (split into several launches by TTP_LANE_LAUNCH_BLOCKS in the
    graphed store).  Replays with new gradients, one of them with an overflow, match an eager
    twin bit for bit."""
    import os
    from ttperf import _lib as L
    torch = torch_mod()
    mixed = mode == O.MODE_MIXED
    if mixed:
        shapes = [(50257, 768), (8192, 8192), (7000, 5000), (768,), (3,)]
        decay = [True, True, True, False, False]
    else:
        shapes = [(8193, 8191), (77,), (3,)]
        decay = [True, False, False]
    eager, _ = make_pair(shapes, decay, mode, seed=95)
    os.environ["TTP_LANE_LAUNCH_BLOCKS"] = "70001"
    try:
        graphed, _ = make_pair(shapes, decay, mode, seed=95)
    finally:
        del os.environ["TTP_LANE_LAUNCH_BLOCKS"]
    graphed.set_stream(None)
    for s in (eager, graphed):
        s.configure_scaler(True, init_scale=1024.0)
    gen = torch.Generator(device="cuda").manual_seed(96)
    if opt == "adamw":
        hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
        step = lambda s: s.adam_step(**hp)
        bufs = (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM)
    else:
        hp = dict(lr=1e-2, momentum=0.9, max_grad_norm=1.0)
        step = lambda s: s.sgd_step(**hp)
        bufs = (L.BUF_MASTER, L.BUF_MOMENTUM, L.BUF_PARAM)
    _same_grads([eager, graphed], gen, 1e-3, scale=1024.0, mixed=mixed)
    step(eager)
    step(graphed)
    graphed.begin_capture()
    step(graphed)
    graph = graphed.end_capture()
    for k in range(3):
        scale = eager.scaler_state()[0]
        inf_at = int(graphed.offsets[1]) + 5 if k == 1 else None
        _same_grads([eager, graphed], gen, 1e-3, scale=scale, inf_at=inf_at, mixed=mixed)
        step(eager)
        graph.replay()
        graphed.sync()
        for buf in bufs:
            assert _bits_equal(graphed.download(buf), eager.download(buf)), (k, buf)
        assert graphed.scaler_state() == eager.scaler_state(), k
        assert graphed.step_count == eager.step_count, k
        print(f"replay {k}: identical to the eager step (scale {eager.scaler_state()[0]})",
              flush=True)
    graph.close()
    graphed.close()
    eager.close()


def test_captured_train_step_zero_accumulate_sgd_momentum():
    """The whole optimizer side of a training step in one graph: zero_grad, gradients
    accumulated from a device buffer the program rewrites between replays, SGD momentum
    with clipping.  The first replay initialises the momentum buffers."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=92)
    store.set_stream(None)
    src = torch.zeros(store.total, dtype=torch.bfloat16, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(93)
    hp = dict(lr=1e-2, momentum=0.9, weight_decay=0.01, max_grad_norm=0.5)

    def accumulate_all():
        for i, t in enumerate(store.tensors):
            ptr = src.data_ptr() + 2 * store.offsets[i]
            L.check(L.lib.ttp_accumulate_grad(store.handle, i, C.c_void_p(ptr), t.numel,
                                              L.DTYPE_BF16, L.DEVICE))

    # eager warm-up of the same sequence (tables, momentum buffer)
    store.zero_grad(set_to_none=True)
    accumulate_all()
    store.sgd_step(**hp)
    store.sync()
    ref.zero_grad()
    for i in range(ref.n):
        ref.accumulate_grad(i, np.zeros(ref.numels[i], np.uint16))
    ref.sgd_step(**hp)

    store.begin_capture()
    store.zero_grad(set_to_none=True)
    accumulate_all()
    store.sgd_step(**hp)
    graph = store.end_capture()
    for k in range(4):
        src.copy_((torch.randn(store.total, generator=gen, device="cuda") * 0.1)
                  .to(torch.bfloat16))
        torch.cuda.synchronize()
        host = src.cpu().view(torch.int16).numpy().view(np.uint16)
        graph.replay()
        store.sync()
        ref.zero_grad()
        for i in range(ref.n):
            o = int(ref.offsets[i])
            ref.accumulate_grad(i, host[o:o + ref.numels[i]])
        ref.sgd_step(**hp)
        compare_state(store, ref, which=("master", "param", "momentum"), max_ulp=2)
        assert store.step_count == ref.t == k + 2
    graph.close()
    store.close()


def test_captured_zero_grad_clears_grad_flags_at_launch():
    """Capturing runs nothing, so it changes no has-grad flag: after capturing
    zero_grad(set_to_none=True) every gradient is still present, and an eager step updates
    every tensor, as in the oracle.  Each launch clears the flags (and the gradients) as the
    eager call does, after which an eager step updates nothing."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=94)
    store.set_stream(None)
    gen = torch.Generator(device="cuda").manual_seed(95)
    hp = dict(lr=1e-2, momentum=0.9)

    def grads():
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        for i in range(ref.n):
            ref.set_has_grad(i, True)

    def flags():
        return [store.has_grad(i) for i in range(len(SHAPES))]

    grads()
    store.sgd_step(**hp)  # eager once: tables and the momentum buffer exist
    ref.sgd_step(**hp)
    store.begin_capture()
    store.zero_grad(set_to_none=True)
    graph = store.end_capture()
    assert flags() == [True] * len(SHAPES), "a capture changed the has-grad flags"
    store.sgd_step(**hp)
    ref.sgd_step(**hp)
    compare_state(store, ref, which=("master", "momentum"), max_ulp=2)
    for k in range(2):
        graph.replay()
        store.sync()
        ref.zero_grad(set_to_none=True)
        assert flags() == [False] * len(SHAPES), f"launch {k} left has-grad flags set"
        assert not store.download(L.BUF_GRAD).any()
        store.sgd_step(**hp)  # no gradients: nothing changes
        ref.sgd_step(**hp)
        compare_state(store, ref, which=("master", "momentum"), max_ulp=2)
        grads()
        assert flags() == [True] * len(SHAPES)
        store.sgd_step(**hp)
        ref.sgd_step(**hp)
        compare_state(store, ref, which=("master", "momentum"), max_ulp=2)
        print(f"launch {k}: flags cleared, then set by new gradients", flush=True)
    graph.close()
    store.close()


def test_captured_python_device_transfers_use_the_callers_tensors():
    """Through the Python layer, device transfers inside a capture become copy nodes over the
    caller's own tensors, with no synchronisation and no temporary copy.  A gradient upload
    from one torch tensor, an accumulate from another and a download of the bf16 weights into
    a third are replayed with new contents each time and match the oracle.  A non-contiguous
    tensor is refused."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=96)
    store.set_stream(None)
    gen = torch.Generator(device="cuda").manual_seed(97)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decoupled=True,
              max_grad_norm=0.5)
    g_all = torch.zeros(store.total, dtype=torch.bfloat16, device="cuda")
    extra = torch.zeros(store.tensors[2].numel, dtype=torch.float32, device="cuda")
    out = torch.zeros(store.total, dtype=torch.bfloat16, device="cuda")

    def sequence():
        store.upload(L.BUF_GRAD, L.ALL_TENSORS, g_all)
        store.accumulate_grad(2, extra)
        store.adam_step(**hp)
        store.download(L.BUF_PARAM, out=out)

    def new_inputs():
        g_all.copy_((torch.randn(store.total, generator=gen, device="cuda") * 1e-2)
                    .to(torch.bfloat16))
        extra.copy_(torch.randn(extra.numel(), generator=gen, device="cuda") * 1e-2)
        torch.cuda.synchronize()
        ref.grad[:store.total] = g_all.cpu().view(torch.int16).numpy().view(np.uint16)
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        ref.accumulate_grad(2, extra.cpu().numpy())
        ref.adam_step(**hp)

    new_inputs()
    sequence()  # eager once: tables and the bias table exist
    store.sync()
    compare_state(store, ref, max_ulp=2)
    store.begin_capture()
    with pytest.raises(ValueError):
        store.upload(L.BUF_GRAD, L.ALL_TENSORS, g_all.view(2, -1).t())  # not contiguous
    sequence()
    graph = store.end_capture()
    for k in range(3):
        new_inputs()
        graph.replay()
        store.sync()
        print(f"replay {k}: step {store.step_count}", flush=True)
        assert store.step_count == ref.t
        compare_state(store, ref, max_ulp=2)
        want = store.download(L.BUF_PARAM)
        assert (out.cpu().view(torch.int16).numpy().view(np.uint16) == want).all()
    graph.close()
    store.close()


def test_per_launch_timing_skips_captured_work():
    """With per-kernel timing on, eager steps record one event pair per kernel launch; a
    capture records none (an event recorded into it would become part of the graph), and
    launches of the graph are not timed.  The replayed steps still run (the step count)."""
    import ttperf
    from ttperf import _lib as L
    store = ttperf.ParamStore([(300, 7), (64,)], mode="mixed")
    store.set_stream(None)
    store.configure_scaler(True, init_scale=1024.0)
    for t in store.tensors:
        t.grad = np.zeros(t.numel, np.uint16)
    store.adam_step(lr=1e-3, max_grad_norm=1.0)  # eager once: tables and bias table
    store.timing(True)
    store.adam_step(lr=1e-3, max_grad_norm=1.0)
    store.sync()
    for k in (L.KERNEL_NORM, L.KERNEL_UPDATE):
        ms, n = store.timing_collect(k)
        assert n == 1 and ms > 0, (k, n, ms)
    store.begin_capture()
    store.adam_step(lr=1e-3, max_grad_norm=1.0)
    graph = store.end_capture()
    t0 = store.step_count
    for _ in range(3):
        graph.replay()
    store.sync()
    assert store.step_count == t0 + 3
    for k in (L.KERNEL_NORM, L.KERNEL_UPDATE):
        assert store.timing_collect(k) == (0.0, 0), k
    store.adam_step(lr=1e-3, max_grad_norm=1.0)
    store.sync()
    assert store.timing_collect(L.KERNEL_UPDATE)[1] == 1
    store.timing(False)
    graph.close()
    store.close()


def test_capture_rejects_what_cannot_be_captured(tmp_path):
    import ttperf
    from ttperf import _lib as L
    store = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    store.tensors[0].grad = np.zeros(100, np.uint16)
    store.tensors[1].grad = np.zeros(512, np.uint16)
    store.adam_step(lr=1e-3)
    # a report synchronises
    store.begin_capture()
    with pytest.raises(ttperf.TTPError) as e:
        store.adam_step(lr=1e-3, report=True)
    assert e.value.code == L.ERR_STATE
    # a tensor set never stepped before would build tables
    with pytest.raises(ttperf.TTPError) as e:
        store.adam_step(lr=1e-3, indices=[1])
    assert e.value.code == L.ERR_STATE
    # host transfers synchronise
    with pytest.raises(ttperf.TTPError) as e:
        store.tensors[0].grad = np.zeros(100, np.uint16)
    assert e.value.code == L.ERR_STATE
    assert store.end_capture(discard=True) is None
    # the capture was discarded cleanly: eager work continues
    r = store.adam_step(lr=1e-3, report=True)
    assert r["step"] == 2
    # a context with live graphs cannot be destroyed; its graphs go first
    store.begin_capture()
    store.adam_step(lr=1e-3)
    g = store.end_capture()
    assert L.lib.ttp_destroy(store.handle) == L.ERR_STATE
    # the graph holds the loss-scaler settings (here: off): changing them is refused, also
    # through a state file, and leaves the store as it was; the same settings are accepted
    with pytest.raises(ttperf.TTPError) as e:
        store.configure_scaler(True)
    assert e.value.code == L.ERR_STATE
    store.configure_scaler(False)
    other = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    other.configure_scaler(True, init_scale=1024.0)
    other.save_state(tmp_path / "scaled.bin")
    other.close()
    master = store.download(L.BUF_MASTER).tobytes()
    with pytest.raises(ttperf.TTPError) as e:
        store.load_state(tmp_path / "scaled.bin")
    assert e.value.code == L.ERR_STATE
    assert store.download(L.BUF_MASTER).tobytes() == master
    g.replay()
    assert store.step_count == 3
    g.close()
    store.configure_scaler(True)  # no graph holds the settings any more
    store.configure_scaler(False)
    # the legacy default stream cannot be captured
    store.set_stream(0)
    with pytest.raises(ttperf.TTPError) as e:
        store.begin_capture()
    assert e.value.code == L.ERR_STATE
    store.close()


def test_trace_context_run_captures_once_then_replays():
    import ttperf
    torch = torch_mod()
    store, ref = make_pair([(1000,), (32, 32)], [False, True], O.MODE_FP32, seed=94)
    store.set_stream(None)
    opt = ttperf.AdamW(store.parameters(), lr=1e-3, weight_decay=0.1)
    gen = torch.Generator(device="cuda").manual_seed(95)
    trace = ttperf.TraceContext(store)
    for k in range(4):
        host = _same_grads([store], gen, 1e-2, mixed=False)
        ref.grad[:] = host
        for i in range(ref.n):
            ref.set_has_grad(i, True)
        if k == 0:
            opt.step()          # eager once: allocates m, v
        else:
            trace.run(opt.step)  # k == 1 captures and runs, later calls replay
        store.sync()
        ref.adam_step(lr=1e-3, weight_decay=0.1, decoupled=True)
        compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=0)
        assert trace.is_captured() == (k >= 1)
    trace.release()
    store.close()


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_accumulate_grad_host_and_device_sources(mode):
    """First call assigns, later calls add (fp32 add, one rounding to the grad type), from
    host or device memory, fp32 or bf16 sources; then a step uses the result."""
    torch = torch_mod()
    from ttperf import _lib as L
    store, ref = make_pair(SHAPES, DECAY, mode, seed=96)
    rng = np.random.default_rng(97)
    for i, t in enumerate(store.tensors):
        for kind in ("host_f32", "host_bf16", "dev_f32", "dev_bf16"):
            x = (rng.standard_normal(t.numel) * 0.3).astype(np.float32)
            if kind.endswith("bf16"):
                bits = O.bf16_rne(x)
                ref.accumulate_grad(i, bits)
                if kind.startswith("host"):
                    store.accumulate_grad(i, bits)
                else:
                    dt = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
                    store.accumulate_grad(i, dt)
            else:
                ref.accumulate_grad(i, x)
                store.accumulate_grad(i, x if kind.startswith("host")
                                      else torch.from_numpy(x).cuda())
    got = store.download(L.BUF_GRAD)
    mask = np.zeros(store.total, bool)
    for i, t in enumerate(store.tensors):
        mask[store.offsets[i]:store.offsets[i] + t.numel] = True
        assert t.grad is not None
    assert _bits_equal(got[mask], ref.grad[mask])
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    r = store.adam_step(report=True, **hp)
    e = ref.adam_step(**hp)
    assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-9 * e["grad_norm"]
    compare_state(store, ref, max_ulp=2)


# ragged sizes: empty, one vector or less, partial last vectors, several tiles with a partial
# last tile (8192 bf16 / 4096 fp32 elements per tile), and an exact number of tiles
BACKWARD_SHAPES = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049), (4097,), (96, 64),
                   (0,), (40000,), (3,), (8192, 3)]


@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_accumulates_in_backward_order_leave_other_tensors_untouched(mode):
    """A backward delivers gradients in reverse tensor order, so the tensor after each one
    already holds its gradient when that one's accumulate runs.  Assigns, then adds with and
    without sums, from host and device memory in both source types (one device source at an
    odd address), in that order; after every call the whole gradient buffer, padding
    included, equals the oracle's bit for bit.  A kernel that wrote past a tensor's end (a
    last tile taken whole) fails here at the first call; in forward order the next tensor's
    own assign would overwrite the damage."""
    torch = torch_mod()
    from ttperf import _lib as L
    decay = [len(sh) == 2 for sh in BACKWARD_SHAPES]
    store, ref = make_pair(BACKWARD_SHAPES, decay, mode, seed=150)
    gen = torch.Generator(device="cuda").manual_seed(151)
    store.zero_grad(set_to_none=True)
    ref.zero_grad(set_to_none=True)
    kinds = ["dev_bf16", "host_f32", "dev_f32_odd", "host_bf16", "dev_f32"]
    calls = 0
    for rnd, sums in enumerate((False, False, True)):  # assign, add, add with sums
        for i in reversed(range(len(BACKWARD_SHAPES))):
            numel = store.tensors[i].numel
            kind = kinds[(i + rnd) % len(kinds)]
            x = torch.randn(numel, generator=gen, device="cuda") * 1e-2
            if kind.endswith("bf16"):
                x = x.to(torch.bfloat16)
                host = x.cpu().view(torch.int16).numpy().view(np.uint16)
            else:
                host = x.cpu().numpy()
            if kind == "dev_f32_odd":
                buf = torch.zeros(numel + 1, device="cuda")
                buf[1:] = x
                src = buf[1:]
                assert numel == 0 or src.data_ptr() % 16
            elif kind.startswith("host"):
                src = host
            else:
                src = x
            store.accumulate_grad(i, src, sums=sums)
            ref.accumulate_grad(i, host)
            calls += 1
            got = store.download(L.BUF_GRAD)
            bad = np.nonzero(got.view(np.uint8) != ref.grad[:store.total].view(np.uint8))[0]
            assert bad.size == 0, (f"call {calls} (tensor {i}, {kind}, round {rnd}): bytes "
                                   f"{bad[:4].tolist()}.. of the gradient buffer differ "
                                   f"(tensor offsets {list(store.offsets)})")
    assert calls == 3 * len(BACKWARD_SHAPES)
    store.close()


def test_closing_other_stores_during_capture_is_deferred():
    """A store (or graph) closed while another store is capturing would free device memory on
    the capturing thread, which invalidates the capture: the close waits for the capture to
    end.  This is what an unrelated store's finalizer does when Python collects it."""
    import gc
    import ttperf
    other = ttperf.ParamStore([(4096,)], mode="fp32")
    store = ttperf.ParamStore([(1000,)], mode="mixed")
    store.tensors[0].grad = np.zeros(1000, np.uint16)
    store.sgd_step(lr=0.1)
    store.begin_capture()
    assert not gc.isenabled()
    other.close()                      # deferred, not destroyed inside the capture
    assert other.handle is not None
    store.sgd_step(lr=0.1)
    graph = store.end_capture()        # the capture is intact
    assert other.handle is None        # destroyed once the capture ended
    assert gc.isenabled()
    graph.replay()
    assert store.step_count == 2
    graph.close()
    store.close()


def test_graph_replay_hands_the_step_count_back_to_its_optimizer():
    """Optimizers a and b over two groups of one store, with different betas.  a's step is
    captured once, and its replays interleave with b's eager steps.  Each replay uses a's own
    step count (the graph hands it back to a), b keeps its own, and each betas pair keeps its
    own bias-correction table.  Checked against the oracle stepping each group with its own
    count, after every step."""
    import ttperf
    torch = torch_mod()
    shapes = [(64, 48), (48,), (48, 32), (32,), (300,)]
    decay = [True, False, True, False, False]
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=98)
    store.set_stream(None)
    groups = {"a": [0, 1, 4], "b": [2, 3]}
    hps = {"a": dict(lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1),
           "b": dict(lr=1e-2, betas=(0.8, 0.999), eps=1e-6, weight_decay=0.0)}
    opts = {"a": ttperf.AdamW([store.tensors[i] for i in groups["a"]], **hps["a"]),
            "b": ttperf.Adam([store.tensors[i] for i in groups["b"]], **hps["b"])}
    counts = {"a": 0, "b": 0}
    gen = torch.Generator(device="cuda").manual_seed(99)
    graph = None
    # lower case: an eager step; "C": capture a's step (runs nothing); "A": replay it
    for k, what in enumerate("abaCbAAbbA"):
        if what == "C":
            store.begin_capture()
            opts["a"].step()
            graph = store.end_capture()
            continue
        g = what.lower()
        ref.grad[:store.total] = device_grads(store, gen, 1e-2)
        for i in range(ref.n):
            ref.set_has_grad(i, i in groups[g])
        if what == "A":
            graph.replay()
        else:
            opts[g].step()
        ref.t = counts[g]
        ref.adam_step(decoupled=(g == "a"), **hps[g])
        counts[g] = ref.t
        print(f"step {k}: {what}, count of {g}: {counts[g]}", flush=True)
        assert store.step_count == counts[g]
        compare_state(store, ref, max_ulp=0)
    assert counts == {"a": 5, "b": 4}
    graph.close()
    store.close()


def test_closing_a_capturing_store_ends_its_capture():
    """Closing a store in the middle of its own capture discards the capture, resumes the
    cyclic collector the capture paused, and destroys the store; other stores work after."""
    import gc

    import ttperf
    from ttperf import store as S
    was = gc.isenabled()
    store = ttperf.ParamStore([(100,), (64, 8)], mode="mixed")
    store.tensors[0].grad = np.zeros(100, np.uint16)
    store.adam_step(lr=1e-3)
    store.begin_capture()
    store.adam_step(lr=1e-3)
    assert not gc.isenabled() and S._capturing == 1
    store.close()
    assert S._capturing == 0 and gc.isenabled() == was
    assert store.handle is None
    other = ttperf.ParamStore([(10,)], mode="fp32")
    other.tensors[0].grad = np.ones(10, np.float32)
    r = other.adam_step(lr=1e-3, report=True)
    assert r["step"] == 1
    other.close()


def test_captured_accumulate_needs_its_flag_set_in_the_same_capture():
    """Whether an accumulate assigns (no grad yet) or adds is fixed when it is captured, so a
    captured accumulate is refused (TTP_ERR_STATE, nothing queued, the capture still valid)
    unless an earlier call of the same capture set that tensor's has-grad flag: an
    accumulate-only graph would otherwise overwrite on every launch when captured without a
    grad, or add onto stale values after an eager set_has_grad(0).  Zeroing to zeros leaves
    the flag as a launch finds it, so it does not count.  A graph that sets the flag itself
    (set_has_grad(0), then two accumulates: assign, then add) replays as the eager calls do,
    whatever the flag is at launch: launched twice in a row, and after an eager
    set_has_grad(1) and an eager set_has_grad(0), each time equal to the oracle."""
    import ttperf
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=140)
    store.set_stream(None)
    i = 2
    n = store.tensors[i].numel
    a = torch.zeros(n, dtype=torch.float32, device="cuda")
    b = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(141)
    store.tensors[i].accumulate_grad(a)  # eager once: staging, and the one-tensor table
    store.zero_grad(set_to_none=False, indices=[i])

    def refused(calls, why):
        store.begin_capture()
        try:
            calls()
            with pytest.raises(ttperf.TTPError) as e:
                store.accumulate_grad(i, a)
            assert e.value.code == L.ERR_STATE and "fixed when it is captured" in str(e.value)
        finally:
            store.end_capture(discard=True)
        print(f"refused as expected: {why}", flush=True)

    refused(lambda: None, "an accumulate-only capture")
    refused(lambda: store.zero_grad(set_to_none=False, indices=[i]),
            "zeroing to zeros does not set the flag")
    refused(lambda: store.zero_grad(set_to_none=False), "nor does the whole-store zero_grad")
    refused(lambda: store.set_has_grad(1, False), "a flag set for another tensor")

    store.begin_capture()
    store.set_has_grad(i, False)
    store.accumulate_grad(i, a)  # assigns
    store.accumulate_grad(i, b)  # adds
    graph = store.end_capture()
    for k, before in enumerate([None, None, True, False]):
        a.copy_(torch.randn(n, generator=gen, device="cuda") * 0.1)
        b.copy_((torch.randn(n, generator=gen, device="cuda") * 0.1).to(torch.bfloat16))
        torch.cuda.synchronize()
        if before is not None:  # an eager flag change between launches
            store.set_has_grad(i, before)
        graph.replay()
        store.sync()
        ref.set_has_grad(i, False)
        ref.accumulate_grad(i, a.cpu().numpy())
        ref.accumulate_grad(i, b.cpu().view(torch.int16).numpy().view(np.uint16))
        got = store.download(L.BUF_GRAD, i)
        assert np.array_equal(got, ref.view("grad", i)), f"launch {k}"
        assert store.has_grad(i)
        print(f"launch {k} (flag before: {before}): grad equals the oracle's", flush=True)
    graph.close()
    store.close()


def test_zero_grad_subset_to_zeros_keeps_the_has_grad_flags():
    """zero_grad(set_to_none=False) over some tensors zeroes their grads and leaves their
    has-grad flags as they were, as the whole-store call and torch's
    zero_grad(set_to_none=False) do: a tensor without a grad is still skipped by the next
    step (py/optim.py:56-57), one with a grad is stepped with a zero gradient."""
    from ttperf import _lib as L
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_FP32, seed=142)
    gen = torch.Generator(device="cuda").manual_seed(143)
    ref.grad[:store.total] = device_grads(store, gen, 1e-2)
    for k in range(ref.n):
        ref.set_has_grad(k, True)
    store.tensors[1].grad = None
    ref.set_has_grad(1, False)
    store.zero_grad(set_to_none=False, indices=[1, 3])
    for k in (1, 3):
        ref.view("grad", k)[:] = 0
    assert [store.has_grad(k) for k in range(len(SHAPES))] == \
        [ref.has_grad(k) for k in range(len(SHAPES))] == [k != 1 for k in range(len(SHAPES))]
    assert not store.download(L.BUF_GRAD, 3).any()
    before = store.tensors[1].master().copy()
    hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    store.adam_step(**hp)
    ref.adam_step(**hp)
    assert np.array_equal(store.tensors[1].master(), before)
    compare_state(store, ref, which=("master", "exp_avg", "exp_avg_sq"), max_ulp=2)
    store.close()
