"""GPU tests of ttp_accumulate_grad_multi: several tensors' incoming gradients in one launch, as a
backward hands over a bucket of them.

Each call must leave exactly what the same tensors' ttp_accumulate_grad calls leave, bit for bit:
the gradients (assign into a tensor without a grad, fp32 add and one rounding into one with a
grad), the has-grad flags and, with TTP_ACCUM_SUMSQ, the tensor sums a step from sums takes its
norm from (compared through the steps' norms and states).  Both are checked against the oracle
too (orc_accumulate_grad, then its own norm).  Refused calls change nothing.  A captured bucket
of accumulates with sums and the step from them replays against the oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, device_grads, make_pair, torch_mod

pytestmark = pytest.mark.gpu

# ragged sizes: empty, one vector or less, partial last vectors, several tiles with a partial
# last tile (8192 bf16 / 4096 fp32 elements per tile), and an exact number of tiles
SHAPES = [(300, 7), (64,), (129, 33), (5,), (2048,), (1, 2049), (4097,), (96, 64), (0,),
          (40000,), (3,), (8192, 3)]
DECAY = [len(s) == 2 for s in SHAPES]


def _bits(t):
    """A torch tensor's host copy in the oracle's types (bf16 bits or float32)."""
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _buckets(order, rng, max_size):
    """`order` cut into consecutive buckets of 1..max_size tensors."""
    out, k = [], 0
    while k < len(order):
        m = int(rng.integers(1, max_size + 1))
        out.append(order[k:k + m])
        k += m
    return out


def _grads_equal(a, b):
    from ttperf import _lib as L
    ga, gb = a.download(L.BUF_GRAD), b.download(L.BUF_GRAD)
    assert np.array_equal(ga.view(np.uint8), gb.view(np.uint8))
    assert [a.has_grad(i) for i in range(len(a.tensors))] == \
        [b.has_grad(i) for i in range(len(b.tensors))]


@pytest.mark.parametrize("src", ["bf16", "f32"])
@pytest.mark.parametrize("mode", [O.MODE_MIXED, O.MODE_FP32])
def test_multi_accumulates_equal_per_tensor_calls(mode, src):
    """Five iterations of a backward's producer in reverse tensor order over random buckets:
    zero_grad to None, then every tensor's gradient in a bucket call (one source of each
    bucket at an odd address in the second round, which takes the element-wise source path),
    then a second round of adds, the last round with sums; the twin store takes the same
    values one tensor per call.  After each round the gradients and flags are identical; the
    AdamW step from the sums then reports the same norm as the twin's, bit for bit, and the
    same state, and both match the oracle.  With loss scaling (mixed), iteration 3 carries a
    +inf and skips."""
    from ttperf import _lib as L
    torch = torch_mod()
    mixed = mode == O.MODE_MIXED
    store, ref = make_pair(SHAPES, DECAY, mode, seed=160)
    twin, _ = make_pair(SHAPES, DECAY, mode, seed=160)
    if mixed:
        for s in (store, twin):
            s.configure_scaler(True, init_scale=512.0, growth_interval=2)
        ref.configure_scaler(True, 512.0, growth_interval=2)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(161)
    rng = np.random.default_rng(162)
    dt = torch.bfloat16 if src == "bf16" else torch.float32
    n = len(SHAPES)
    for it in range(5):
        scale = ref.scale if mixed else 1.0
        for s in (store, twin):
            s.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)
        for rnd in range(2):
            sums = rnd == 1
            for bucket in _buckets(list(reversed(range(n))), rng, 5):
                vals, keep = [], []
                for i in bucket:
                    x = (torch.randn(store.tensors[i].numel, generator=gen, device="cuda")
                         * 1e-2 * scale).to(dt)
                    if mixed and it == 3 and rnd == 1 and i == 9:
                        x[77] = float("inf")
                    if rnd == 1 and i == bucket[0] and x.numel():
                        buf = torch.zeros(x.numel() + 1, device="cuda", dtype=dt)
                        buf[1:] = x
                        keep.append(buf)
                        x = buf[1:]
                        assert x.data_ptr() % 16
                    vals.append(x)
                store.accumulate_grads(bucket, vals, sums=sums)
                for i, x in zip(bucket, vals):
                    twin.accumulate_grad(i, x, sums=sums)
                    ref.accumulate_grad(i, _bits(x))
            _grads_equal(store, twin)
        got = store.download(L.BUF_GRAD)
        assert np.array_equal(got.view(np.uint8), ref.grad[:store.total].view(np.uint8))
        r = store.adam_step(report=True, tensor_sums=True, **hp)
        rt = twin.adam_step(report=True, tensor_sums=True, **hp)
        e = ref.adam_step(**hp)
        print(f"iteration {it}: norm {r['grad_norm']!r} (twin {rt['grad_norm']!r}, oracle "
              f"{e['grad_norm']!r}), skipped {r['skipped']}", flush=True)
        for k in ("skipped", "found_inf", "step", "scale", "growth_tracker"):
            assert r[k] == rt[k] == e[k], (k, r, rt, e)
        assert r["skipped"] == (mixed and it == 3)
        assert np.array_equal(np.float64(r["grad_norm"]), np.float64(rt["grad_norm"])) or \
            not np.isfinite(r["grad_norm"])
        if np.isfinite(e["grad_norm"]):
            assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
        compare_state(store, ref, max_ulp=2)
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM):
        assert np.array_equal(store.download(which).view(np.uint8),
                              twin.download(which).view(np.uint8)), which
    store.close()
    twin.close()


def test_refused_multi_accumulates_change_nothing():
    """Raw C ABI calls the library refuses, each leaving the gradients and flags as they were:
    more than 64 tensors, an index listed twice, an unknown index, a host pointer, a null
    source for a tensor with elements, an unknown dtype; a call of none is a no-op.  The
    refusal reasons come from the library's own checks, not from the binding.  Through the
    Python binding, an unknown index is the library's TTP_ERR_RANGE too, and a value of the
    wrong size a ValueError before any call."""
    torch = torch_mod()
    from ttperf import _lib as L
    shapes = [(7,)] * 70
    store, _ = make_pair(shapes, [False] * 70, O.MODE_MIXED, seed=170)
    store.zero_grad(set_to_none=True)
    srcs = [torch.randn(7, device="cuda").to(torch.bfloat16) for _ in range(70)]
    store.accumulate_grads([0, 1, 2], srcs[:3])
    torch.cuda.synchronize()
    before = store.download(L.BUF_GRAD).copy()
    flags = [store.has_grad(i) for i in range(70)]
    host = np.zeros(7, np.uint16)

    def call(idx, ptrs, dtype=L.DTYPE_BF16):
        ia = (C.c_uint32 * max(len(idx), 1))(*idx)
        pa = (C.c_void_p * max(len(ptrs), 1))(*ptrs)
        return L.lib.ttp_accumulate_grad_multi(store.handle, ia, pa, len(idx), dtype)

    dev = [s.data_ptr() for s in srcs]
    cases = [(list(range(65)), dev[:65], L.DTYPE_BF16, L.ERR_RANGE),
             ([3, 4, 3], dev[3:6], L.DTYPE_BF16, L.ERR_INVALID),
             ([3, 70], dev[3:5], L.DTYPE_BF16, L.ERR_RANGE),
             ([3, 4], [dev[3], host.ctypes.data], L.DTYPE_BF16, L.ERR_INVALID),
             ([3, 4], [dev[3], None], L.DTYPE_BF16, L.ERR_INVALID),
             ([3, 4], dev[3:5], 7, L.ERR_INVALID)]
    for k, (idx, ptrs, dtype, code) in enumerate(cases):
        rc = call(idx, ptrs, dtype)
        assert rc == code, (k, rc, code)
        assert np.array_equal(store.download(L.BUF_GRAD), before), k
        assert [store.has_grad(i) for i in range(70)] == flags, k
    assert call([], []) == L.OK
    # through the Python binding: an index out of range is the library's refusal
    with pytest.raises(L.TTPError) as e:
        store.accumulate_grads([3, 70], [srcs[3], srcs[4]])
    assert e.value.code == L.ERR_RANGE
    with pytest.raises(ValueError):  # a value of the wrong size
        store.accumulate_grads([3, 4], [srcs[3], torch.zeros(8, device="cuda",
                                                             dtype=torch.bfloat16)])
    assert np.array_equal(store.download(L.BUF_GRAD), before)
    assert [store.has_grad(i) for i in range(70)] == flags
    # 64 tensors is the limit, not an error
    store.accumulate_grads(list(range(64)), srcs[:64])
    assert all(store.has_grad(i) for i in range(64)) and not store.has_grad(64)
    store.close()


def test_captured_multi_accumulates_and_step_replay():
    """zero_grad to None, the tensors' gradients in three bucket calls with sums from device
    buffers read in place, and the AdamW step from those sums (loss scaling, clipping),
    captured as one graph after one eager run; replayed four times with new buffer contents
    (one holding +inf), each against the oracle."""
    torch = torch_mod()
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=180)
    store.set_stream(None)  # the store's own stream: capturable
    store.configure_scaler(True, init_scale=256.0, growth_interval=3)
    ref.configure_scaler(True, 256.0, growth_interval=3)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(181)
    n = len(SHAPES)
    srcs = [torch.zeros(store.tensors[i].numel, device="cuda", dtype=torch.bfloat16)
            for i in range(n)]
    order = list(reversed(range(n)))
    buckets = [order[:4], order[4:9], order[9:]]

    def refill(inf=False):
        for i in range(n):
            srcs[i].copy_((torch.randn(srcs[i].numel(), generator=gen, device="cuda") * 1e-2
                           * ref.scale).to(torch.bfloat16))
        if inf:
            srcs[6][11] = float("inf")
        torch.cuda.synchronize()

    def iteration():
        store.zero_grad(set_to_none=True)
        for b in buckets:
            store.accumulate_grads(b, [srcs[i] for i in b], sums=True)
        return store.adam_step(tensor_sums=True, **hp)

    def ref_iteration():
        ref.zero_grad(set_to_none=True)
        for b in buckets:
            for i in b:
                ref.accumulate_grad(i, _bits(srcs[i]))
        return ref.adam_step(**hp)

    refill()
    iteration()  # eagerly once: the step's work and bias tables
    ref_iteration()
    store.sync()
    compare_state(store, ref, max_ulp=2)
    store.begin_capture()
    iteration()
    graph = store.end_capture()
    for k in range(4):
        refill(inf=(k == 2))
        graph.replay()
        e = ref_iteration()
        store.sync()
        assert store.step_count == e["step"]
        assert store.scaler_state() == (np.float32(e["scale"]), e["growth_tracker"])
        assert e["skipped"] == (k == 2)
        compare_state(store, ref, max_ulp=2)
    graph.close()
    store.close()


def test_gpt2_124m_buckets_equal_per_tensor_calls():
    """GPT-2 124M's 148 tensors in reverse order as buckets of up to 25 MB of gradients (and at
    most 64 tensors), accumulated with sums into one store and one tensor per call into its
    twin: the gradients, and the AdamW step from the sums (loss scaling, clipping), identical
    bit for bit, and the step matches a norm-pass step of a third store within the oracle's
    2-ulp bar."""
    from ttperf import configs
    from ttperf import _lib as L
    torch = torch_mod()
    _, shapes, decay, numels = configs.table("gpt2_124m")
    store, ref = make_pair(shapes, decay, O.MODE_MIXED, seed=190)
    twin, _ = make_pair(shapes, decay, O.MODE_MIXED, seed=190)
    for s in (store, twin):
        s.configure_scaler(True, init_scale=65536.0)
    ref.configure_scaler(True, 65536.0)
    hp = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    flat = device_grads(store, torch.Generator(device="cuda").manual_seed(191), 1e-3,
                        scale=65536.0, into=ref.grad)
    del flat
    g = store.torch_view(L.BUF_GRAD).clone()  # the incoming gradients, in the store's layout
    for s in (store, twin):
        s.zero_grad(set_to_none=True)
    order = [i for i in reversed(range(len(shapes))) if numels[i]]
    buckets, cur, size = [], [], 0
    for i in order:
        cur.append(i)
        size += 2 * numels[i]
        if size >= 25 << 20 or len(cur) == L.ACCUM_MULTI_MAX:
            buckets.append(cur)
            cur, size = [], 0
    if cur:
        buckets.append(cur)
    print(f"{len(buckets)} buckets of {[len(b) for b in buckets]} tensors", flush=True)
    views = {i: g[store.offsets[i]:store.offsets[i] + numels[i]] for i in order}
    for b in buckets:
        store.accumulate_grads(b, [views[i] for i in b], sums=True)
        for i in b:
            twin.accumulate_grad(i, views[i], sums=True)
    _grads_equal(store, twin)
    for i in range(len(shapes)):
        ref.set_has_grad(i, True)
    r = store.adam_step(report=True, tensor_sums=True, **hp)
    rt = twin.adam_step(report=True, tensor_sums=True, **hp)
    e = ref.adam_step(**hp)
    assert np.float64(r["grad_norm"]) == np.float64(rt["grad_norm"])
    assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-5 * e["grad_norm"]
    assert (r["skipped"], r["step"], r["scale"]) == (e["skipped"], e["step"], e["scale"])
    for which in (L.BUF_MASTER, L.BUF_PARAM):
        assert np.array_equal(store.download(which).view(np.uint8),
                              twin.download(which).view(np.uint8)), which
    compare_state(store, ref, max_ulp=2)
    store.close()
    twin.close()


def test_zero_grad_without_fill():
    """zero_grad(set_to_none=True, fill=False) (TTP_ZERO_NO_FILL) clears the has-grad flags and
    leaves the gradient memory as it was, for all tensors or a list; without set_to_none it is
    refused, as is a listed index twice.  A producer iteration after it (bucket calls that
    assign every gradient, with sums, then the AdamW step from them) gives the state of a twin
    whose zero_grad filled the buffer, bit for bit, and the oracle's; captured as one graph
    (the flags-only zero_grad included) it replays against the oracle."""
    torch = torch_mod()
    from ttperf import _lib as L
    store, ref = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=200)
    twin, _ = make_pair(SHAPES, DECAY, O.MODE_MIXED, seed=200)
    store.set_stream(None)  # the store's own stream: capturable
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=0.5)
    gen = torch.Generator(device="cuda").manual_seed(201)
    n = len(SHAPES)
    device_grads(store, gen, 1e-2, into=ref.grad)
    before = store.download(L.BUF_GRAD).copy()
    store.mark_grads()
    store.zero_grad(set_to_none=True, indices=[1, 3], fill=False)
    assert [store.has_grad(i) for i in range(n)] == [i not in (1, 3) for i in range(n)]
    store.zero_grad(set_to_none=True, fill=False)
    assert not any(store.has_grad(i) for i in range(n))
    assert np.array_equal(store.download(L.BUF_GRAD), before)
    h = store.handle
    assert L.lib.ttp_zero_grad(h, L.ZERO_NO_FILL) == L.ERR_INVALID
    idx = (C.c_uint32 * 2)(2, 2)
    assert L.lib.ttp_zero_grad_subset(h, idx, 2, 1 | L.ZERO_NO_FILL) == L.ERR_INVALID
    assert L.lib.ttp_zero_grad_subset(h, idx, 1, L.ZERO_NO_FILL) == L.ERR_INVALID
    srcs = [torch.zeros(store.tensors[i].numel, device="cuda", dtype=torch.bfloat16)
            for i in range(n)]
    order = list(reversed(range(n)))
    buckets = [order[:5], order[5:]]

    def refill():
        for i in range(n):
            srcs[i].copy_((torch.randn(srcs[i].numel(), generator=gen, device="cuda") * 1e-2)
                          .to(torch.bfloat16))
        torch.cuda.synchronize()

    def iteration(s, fill):
        s.zero_grad(set_to_none=True, fill=fill)
        for b in buckets:
            s.accumulate_grads(b, [srcs[i] for i in b], sums=True)
        return s.adam_step(report=True, tensor_sums=True, **hp) if not s._in_capture else \
            s.adam_step(tensor_sums=True, **hp)

    def ref_iteration():
        ref.zero_grad(set_to_none=True, fill=False)
        for b in buckets:
            for i in b:
                ref.accumulate_grad(i, _bits(srcs[i]))
        return ref.adam_step(**hp)

    refill()
    r, rt, e = iteration(store, False), iteration(twin, True), ref_iteration()
    assert np.float64(r["grad_norm"]) == np.float64(rt["grad_norm"])
    assert abs(r["grad_norm"] - e["grad_norm"]) <= 1e-10 * e["grad_norm"]
    for which in (L.BUF_MASTER, L.BUF_EXP_AVG, L.BUF_EXP_AVG_SQ, L.BUF_PARAM):
        assert np.array_equal(store.download(which).view(np.uint8),
                              twin.download(which).view(np.uint8)), which
    compare_state(store, ref, max_ulp=2)
    store.begin_capture()
    iteration(store, False)
    graph = store.end_capture()
    for _ in range(2):
        refill()
        graph.replay()
        e = ref_iteration()
        store.sync()
        assert store.step_count == e["step"]
        compare_state(store, ref, max_ulp=2)
    graph.close()
    store.close()
    twin.close()
