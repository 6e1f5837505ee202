"""Several host threads, each driving its own store, at the same time.

The C ABI allows one host thread per context (include/ttperf/ttperf.h) and ctypes releases
the GIL during each call, so these threads' calls interleave inside libttperf_hip.  Each
thread runs its own mix of uploads, steps with reports and argument errors, and its store
must end bit-identical to its own oracle; the error message each thread reads back
(ttp_last_error, thread-local) is the one its own call left."""
import threading

import numpy as np
import pytest

import oracle as O
from gpu_util import compare_state, make_pair

pytestmark = pytest.mark.gpu


def _worker(k, out):
    import ttperf
    from ttperf import _lib as L
    try:
        rng = np.random.default_rng(300 + k)
        mixed = k % 2 == 0
        shapes = [(int(rng.integers(1, 200)), int(rng.integers(1, 200))), (int(rng.integers(1, 5000)),),
                  (3,), (64, 65)]
        decay = [True, False, False, True]
        store, ref = make_pair(shapes, decay, O.MODE_MIXED if mixed else O.MODE_FP32,
                               seed=300 + k)
        store.set_stream(None)  # this thread's store on its own stream
        if mixed:
            store.configure_scaler(True, init_scale=1024.0, growth_interval=3)
            ref.configure_scaler(True, 1024.0, growth_interval=3)
        hp = dict(lr=1e-3 * (k + 1), betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                  decoupled=True)
        for step in range(12):
            g = (rng.standard_normal(store.total) * 1e-2 * (ref.scale if mixed else 1.0))
            g = O.bf16_rne(g.astype(np.float32)) if mixed else g.astype(np.float32)
            store.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
            ref.grad[:store.total] = g
            for i in range(ref.n):
                ref.set_has_grad(i, True)
            r = store.adam_step(report=True, max_grad_norm=1.0, **hp)
            e = ref.adam_step(max_grad_norm=1.0, **hp)
            assert r["step"] == e["step"] and r["skipped"] == e["skipped"]
            # an argument error of this thread's own: its message is the one read back
            with pytest.raises(ttperf.TTPValueError) as err:
                store.adam_step(lr=-1.0 - k)
            assert "lr must be > 0" in str(err.value)
            # straight through the C ABI: a size error, then this thread's message
            wrong = store.tensors[1].numel + 1 + k + 100 * step
            buf = np.zeros(wrong, np.uint16 if mixed else np.float32)
            rc = L.lib.ttp_upload(store.handle, L.BUF_GRAD, 1, buf.ctypes.data, wrong, L.HOST)
            assert rc == L.ERR_RANGE
            msg = L.lib.ttp_last_error().decode()
            assert msg.endswith(f"got {wrong}"), msg
        compare_state(store, ref, max_ulp=0)
        store.close()
        out[k] = "ok"
    except BaseException as exc:  # reported by the main thread
        out[k] = exc


def test_threads_with_their_own_stores():
    n = 6
    out = [None] * n
    threads = [threading.Thread(target=_worker, args=(k, out)) for k in range(n)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    for k, r in enumerate(out):
        if r != "ok":
            raise AssertionError(f"thread {k}: {r!r}") from (r if isinstance(r, BaseException)
                                                            else None)
