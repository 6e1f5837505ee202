"""Benchmark of the fused optimizer step: `python bench.py [--gpus 1] [--steps K] [--warmup W]`.

Workload (BASELINE.json metric, configs[2]): GPT-2 124M mixed precision — 148 tensors,
124,439,808 params, bf16 params/grads, fp32 master/m/v, dynamic loss scaling (2^16),
global-norm clip 1.0, AdamW lr 6e-4 betas (0.9, 0.95) wd 0.1 on the 2-D tensors.
One step = the norm/inf-check/scaler pass + the fused multi-tensor AdamW pass over
synthetic N(0, 1e-3) x scale bf16 gradients already resident in HBM.

Prints ONE JSON line: Gparams/s and ms/step of the timed region (K steps between one event
pair, after --settle-ms of untimed steps and then W warmup steps), the roofline of the
dominant (update) kernel from HIP events recorded around each of its launches on the
kernel's stream during a second pass of K steps, and the CPU oracle baseline timed on this
host's cores on a bounded sample.  Beside the headline: the same steps timed right after the
set-up (before the settle steps), the step with a cold Infinity Cache (512 MB of unrelated
reads before each step, outside its event pair), the step right after a rewrite of its
gradients, the mean skipped (overflow) step, the step with its norm from bucketed sums, and
the other configurations' steps (the MLP, nanoGPT-char, GPT-2 774M mixed AdamW, GPT-2 XL
fp32 AdamW and SGD momentum; the reference's plain SGD and SGD momentum in mixed precision at
GPT-2 124M and 774M on stores in the SGD layout, and SGD momentum at 774M in the default
layout; the reference's plain SGD on its own bf16-only storage at GPT-2 124M and 774M), each
in a store of its own, and the step of the reference's GPT benchmark model
through the C++ drop-in surface (tests/cpp/bench_gpt2_step).  `--optimizer sgd|sgdm` and
`--layout sgd` time those steps as the main leg instead (for profiling).
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tt-perf_amd"))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
# gradient bytes up to which libttperf_hip counts a store's gradients as Infinity-Cache resident
# and picks its update form accordingly (kCachedGradBytes in tt-perf_amd/csrc/ttperf.hip):
# names the kernel in the roofline
CACHED_GRAD_BYTES = 256 << 20
# algorithmic bytes per parameter of one update-kernel pass (and of the norm pass)
UPDATE_BYTES = {("adamw", "mixed"): 28, ("adamw", "fp32"): 28, ("sgdm", "fp32"): 20,
                ("sgdm", "mixed"): 20, ("sgd", "mixed"): 12, ("sgd", "fp32"): 12,
                # a BF16 store: bf16 gradient and weight read, weight written
                ("sgd", "bf16"): 6}
# update legs below this many algorithmic bytes are launch-bound or Infinity-Cache resident:
# an event pair around each launch then measures mostly its own overhead, and a copy of their
# bytes no ceiling, so neither is reported for them
MIN_TIMED_UPDATE_BYTES = 1 << 30
NORM_BYTES = {"mixed": 2, "fp32": 4, "bf16": 2}

# The step of each BASELINE.json configuration: optimizer hyperparameters, loss scaling, and
# the synthetic gradient distribution (N(0, std), a fraction `heavy` drawn from N(0, 1)).
BENCH = {
    "mlp": dict(hp=dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                        max_grad_norm=None), decoupled=False, scaler=None, std=1e-2, heavy=0.0),
    "nanogpt_char": dict(hp=dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                                 max_grad_norm=1.0), decoupled=True, scaler=None, std=1e-3,
                         heavy=0.0),
    "gpt2_124m": dict(hp=dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                              max_grad_norm=1.0), decoupled=True, scaler=65536.0, std=1e-3,
                      heavy=0.0),
    "gpt2_774m": dict(hp=dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                              max_grad_norm=1.0), decoupled=True, scaler=65536.0, std=1e-3,
                      heavy=0.0),
    "gpt2_1558m": dict(hp=dict(lr=1.5e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                               max_grad_norm=1.0), decoupled=True, scaler=None, std=1e-3,
                       heavy=0.01),
}
# one GPU's shard of GPT-2 124M under ZeRO-1 over 8 GPUs (the per-GPU kernel of the design)
BENCH["gpt2_124m_shard8"] = BENCH["gpt2_124m"]
HEADLINE = "fused AdamW step Gparams/s + % of HBM peak, GPT-2 124M mixed precision"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="gpt2_124m", choices=sorted(BENCH),
                    help="a BASELINE.json configuration (gpt2_124m is the headline metric's), "
                         "or gpt2_124m_shard8: one GPU's ZeRO-1 shard of it")
    ap.add_argument("--optimizer", default="adamw", choices=["adamw", "sgdm", "sgd"],
                    help="adamw (the headline); sgdm: SGD with momentum 0.9 and the "
                         "configuration's clipping; sgd: the reference's plain SGD, w - lr*g")
    ap.add_argument("--mode", default="config", choices=["config", "bf16"],
                    help="the store's precision mode: the configuration's, or bf16 (the "
                         "reference's bf16-only storage, TTP_MODE_BF16; with --optimizer sgd)")
    ap.add_argument("--layout", default="default", choices=["default", "sgd"],
                    help="store layout of a mixed store (sgd: TTP_STORE_SGD, a contiguous "
                         "master and no m / v)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--overlap", action="store_true",
                    help="also time the bucket sums beside a bf16 GEMM on another stream (the "
                         "backward's compute stand-in) against each alone")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of the step captured as a hipGraph (measured equal to "
                         "eager launches on MI355X, so eager is the default)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the GPT-2 774M and XL steps timed after the headline")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="run the step back to back for this long before the W warmup steps "
                         "(0: not at all); see settle() ")
    return ap.parse_args()


def settle(step, ms):
    """Run `step` back to back, in batches of 20 with a synchronisation after each, for at
    least `ms` milliseconds; returns (steps, ms).  After an idle phase (process start, store
    set-up) MI355X runs its first tens of milliseconds of work at lower clocks: the busy-cycle
    counter of the GPT-2 124M update read 17 cycles/ns at first and 19 after about 15 ms, and
    20 steps timed after 5 warmup steps ran 0.571 ms (four-element update) and 0.59-0.61 ms
    (lane form) against 0.560 and 0.553-0.557 ms after 50 ms or more of steps.  A training
    loop keeps the GPU busy between its steps, so the step is timed at those clocks.  The
    settle steps are not timed and precede the W warmup steps."""
    import torch

    n, t0 = 0, time.perf_counter()
    while ms > 0:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
        n += 20
        if (time.perf_counter() - t0) * 1e3 >= ms:
            break
    return n, round((time.perf_counter() - t0) * 1e3, 1)


def traffic_from_profiles(config, optimizer):
    """HBM bytes per update launch from the committed rocprofv3 --pmc summary of the AdamW
    update, if any (none is committed for the SGD updates)."""
    if optimizer != "adamw":
        return None
    path = os.path.join(REPO, "profiles", f"adam_lane_kernel_{config}_pmc.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo) with its family, model and stepping
    numbers (a virtual machine may shorten the name to the vendor's brand), or None."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break  # the first processor's block
            key, _, val = line.partition(":")
            fields.setdefault(key.strip(), val.strip())
    except OSError:
        return None
    name = fields.get("model name")
    if name is None:
        return None
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_baseline(numels, flags, mode_mixed, grads_host, hp, seconds, scaler):
    """The CPU oracle (C restatement of the reference's optimizer) on this host's cores:
    the fused step on all threads (the reported value), the same on 1 thread, and the
    op-by-op restatement of py/optim.py (one full pass per ttnn op) on all threads.  Each leg
    runs for about `seconds`."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import oracle as O
    nthreads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    st = O.OracleStore(numels, flags=flags, mode=O.MODE_MIXED if mode_mixed else O.MODE_FP32,
                       nthreads=nthreads)
    if scaler:
        st.configure_scaler(True, scaler)
    hp = dict(hp, max_grad_norm=hp["max_grad_norm"] or 0.0)
    rng = np.random.default_rng(0)
    st.master[:] = rng.normal(0, 0.02, st.total).astype(np.float32)
    st.grad[:] = grads_host
    for i in range(st.n):
        st.set_has_grad(i, True)
    res = {}
    for label, kw, nt in (("fused", {}, nthreads), ("fused_1", {}, 1),
                          ("opbyop", {"opbyop": True}, nthreads)):
        st.s.nthreads = nt
        st.adam_step(**hp, **kw)  # warm
        t0 = time.perf_counter()
        n = 0
        while True:
            st.adam_step(**hp, **kw)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 200:
                break
        res[label] = (n, el)
        log(f"bench: cpu {label} on {nt} thread(s): {el / n * 1e3:.1f} ms/step")
    total = sum(numels)
    n, el = res["fused"]
    out = {"value": round(total * n / el / 1e9, 4), "unit": "Gparams/s", "cores": nthreads,
           "cpu_model": cpu_model(), "kind": "port",
           "sample": f"full {len(numels)}-tensor table ({total} params), {n} fused steps "
                     f"(the same step as the GPU's) in {el:.1f} s on {nthreads} threads",
           "ms_per_step": round(el / n * 1e3, 3)}
    n1, el1 = res["fused_1"]
    out["single_core_value"] = round(total * n1 / el1 / 1e9, 4)
    out["single_core_sample"] = f"{n1} fused steps in {el1:.1f} s on 1 thread"
    n2, el2 = res["opbyop"]
    out["opbyop_value"] = round(total * n2 / el2 / 1e9, 4)
    out["opbyop_sample"] = (f"{n2} steps executing py/optim.py's ops as separate full passes, "
                            f"{el2:.1f} s on {nthreads} threads")
    return out


def bucketed_norm(store, stream, args, hp, mode, numels):
    """The step when its norm comes from per-tensor sums taken bucket by bucket (in reverse
    tensor order, as a backward produces them; 25 MB of gradients each, or a sixteenth of them
    for large models), which can run beside the backward's compute; the step then runs the
    finalize and the update only.  With --overlap, also the share of the bucket sums' time
    hidden beside a GEMM on another stream.  Returns the JSON object."""
    import numpy as np
    import torch

    dev = torch.device("cuda:0")
    esz = 2 if mode == "mixed" else 4
    bucket_bytes = max(25 << 20, sum(numels) * esz // 16)
    buckets, cur, cur_bytes = [], [], 0
    for i in reversed(range(len(numels))):
        cur.append(i)
        cur_bytes += numels[i] * esz
        if cur_bytes >= bucket_bytes:
            buckets.append(sorted(cur))
            cur, cur_bytes = [], 0
    if cur:
        buckets.append(sorted(cur))

    def bucket_sums():
        for b in buckets:
            store.grad_sumsq_tensors(b)

    def step_after_sums():
        if args.optimizer == "adamw":
            store.adam_step(tensor_sums=True, **hp)
        else:
            store.sgd_step(lr=hp["lr"], momentum=0.9, max_grad_norm=hp["max_grad_norm"],
                           tensor_sums=True)

    for _ in range(3):
        bucket_sums()
        step_after_sums()
    torch.cuda.synchronize()
    # an event pair around the bucket calls and one around the step, per iteration, on the
    # store's stream: the GPU time of each (subtracting loop totals would mislead where
    # hundreds of small bucket launches make the bucket loop host-bound)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for k in range(args.steps):
        evs[k][0].record(stream)
        bucket_sums()
        evs[k][1].record(stream)
        step_after_sums()
        evs[k][2].record(stream)
    torch.cuda.synchronize()
    sums_ms = sum(a.elapsed_time(b) for a, b, _ in evs) / args.steps
    after_ms = sum(b.elapsed_time(c) for _, b, c in evs) / args.steps
    overlap = None
    if args.overlap:
        # a bf16 GEMM on its own stream stands in for the backward's compute; the bucket
        # sums run on the store's stream at the same time
        comp = torch.cuda.Stream()
        a = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
        b = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
        c_out = torch.empty(8192, 8192, device=dev, dtype=torch.bfloat16)

        def gemm():
            with torch.cuda.stream(comp):
                torch.mm(a, b, out=c_out)

        def both():
            gemm()
            bucket_sums()

        # interleaved rounds, each launch synchronised and host-timed; medians
        runs = {"gemm": [], "sums": [], "both": []}
        fns = {"gemm": gemm, "sums": bucket_sums, "both": both}
        for _ in range(3):
            for fn in fns.values():
                fn()
        torch.cuda.synchronize()
        for _ in range(30):
            for name, fn in fns.items():
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                runs[name].append((time.perf_counter() - t0) * 1e3)
        gemm_ms, sums_alone_ms, both_ms = (float(np.median(runs[k]))
                                           for k in ("gemm", "sums", "both"))
        overlap = {"gemm_ms": round(gemm_ms, 4), "bucket_sums_ms": round(sums_alone_ms, 4),
                   "together_ms": round(both_ms, 4),
                   "sums_hidden_frac": round((gemm_ms + sums_alone_ms - both_ms)
                                             / sums_alone_ms, 3),
                   "note": "bf16 8192^3 torch.mm on one stream, the bucket sums on the "
                           "store's stream; medians of 30 interleaved rounds, each launch "
                           "synchronised and host-timed"}
        del a, b, c_out
    return {"buckets": len(buckets), "bucket_sums_ms": round(sums_ms, 4),
            "step_after_sums_ms": round(after_ms, 4),
            "note": "ttp_grad_sumsq_tensors per bucket, then the step with "
                    "TTP_STEP_TENSOR_SUMS; in training the bucket sums overlap the "
                    "backward, leaving step_after_sums_ms on the step's own path",
            "overlap": overlap}


def producer_step(store, stream, args, hp, mode, numels):
    """The step fed by a backward's gradient producer: zero_grad(set_to_none), then one
    ttp_accumulate_grad per tensor from device memory (in reverse tensor order, as a backward
    produces them; the gradients are a device copy of the store's own), then the step.  Each
    variant is captured once as a hipGraph (so the host's 100+ calls per iteration do not pace
    the GPU) and replayed K times between one event pair:
      norm_pass:   plain accumulates, then the step with its norm pass;
      fused_sums:  accumulates that also store each tensor's sum (TTP_ACCUM_SUMSQ), then the
                   step from those sums (TTP_STEP_TENSOR_SUMS: no norm pass);
    and the producer alone (zero_grad + accumulates) with and without the sums.  Returns the
    JSON object."""
    import torch
    from ttperf import _lib as L

    src = store.torch_view(L.BUF_GRAD).clone()  # the store's layout, so tensor i at offsets[i]
    base, esz = src.data_ptr(), src.element_size()
    dtype = L.DTYPE_BF16 if mode == "mixed" else L.DTYPE_F32
    order = [i for i in reversed(range(len(numels))) if numels[i]]

    # buckets for the multi-tensor calls: consecutive tensors of the backward order, up to
    # 25 MB of gradients and ACCUM_MULTI_MAX tensors each
    buckets, cur, size = [], [], 0
    for i in order:
        cur.append(i)
        size += numels[i] * esz
        if size >= 25 << 20 or len(cur) == L.ACCUM_MULTI_MAX:
            buckets.append(cur)
            cur, size = [], 0
    if cur:
        buckets.append(cur)
    tables = [((ctypes.c_uint32 * len(b))(*b),
               (ctypes.c_void_p * len(b))(*[base + store.offsets[i] * esz for i in b]))
              for b in buckets]

    def produce(sums, multi=False, fill=True):
        store.zero_grad(set_to_none=True, fill=fill)
        flag = L.ACCUM_SUMSQ if sums else 0
        if multi:
            for b, (idx, ptrs) in zip(buckets, tables):
                L.check(L.lib.ttp_accumulate_grad_multi(store.handle, idx, ptrs, len(b),
                                                        dtype | flag))
            return
        for i in order:
            L.check(L.lib.ttp_accumulate_grad(store.handle, i,
                                              ctypes.c_void_p(base + store.offsets[i] * esz),
                                              numels[i], dtype | flag, L.DEVICE))

    def iteration(sums, step=True, multi=False, fill=True):
        produce(sums, multi, fill)
        if step:
            store.adam_step(tensor_sums=sums, **hp)

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {}
    for key, sums, step, multi, fill in (
            ("norm_pass_ms", False, True, False, True), ("fused_sums_ms", True, True, False, True),
            ("producer_ms", False, False, False, True),
            ("producer_with_sums_ms", True, False, False, True),
            ("multi_norm_pass_ms", False, True, True, True),
            ("multi_fused_sums_ms", True, True, True, True),
            ("multi_producer_ms", False, False, True, True),
            ("multi_producer_with_sums_ms", True, False, True, True),
            ("multi_fused_sums_nofill_ms", True, True, True, False),
            ("multi_producer_with_sums_nofill_ms", True, False, True, False)):
        iteration(sums, step, multi, fill)  # eagerly once: work tables and the tile-sum buffer
        torch.cuda.synchronize()
        store.begin_capture()
        iteration(sums, step, multi, fill)
        graph = store.end_capture()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        out[key] = round(e0.elapsed_time(e1) / args.steps, 4)
        graph.close()
    del src
    out["step_saved_ms"] = round(out["norm_pass_ms"] - out["fused_sums_ms"], 4)
    out["multi_step_saved_ms"] = round(out["multi_norm_pass_ms"] - out["multi_fused_sums_ms"], 4)
    out["tensors"] = len(order)
    out["buckets"] = len(buckets)
    out["note"] = ("zero_grad(set_to_none) + one ttp_accumulate_grad per tensor from device "
                   "memory + the AdamW step, captured as one hipGraph and replayed K times "
                   "between one event pair; fused_sums: the accumulates also store each "
                   "tensor's gradient sum and the step runs no norm pass; producer_*: the "
                   "zero_grad and accumulates alone; multi_*: the same with one "
                   "ttp_accumulate_grad_multi call per bucket of up to 25 MB of gradients; "
                   "*_nofill: zero_grad(set_to_none) clears the has-grad flags only "
                   "(TTP_ZERO_NO_FILL), the first accumulate assigns each gradient")
    log(f"bench: producer + step: {out['norm_pass_ms']} ms with the norm pass, "
        f"{out['fused_sums_ms']} ms with fused sums; in {len(buckets)} bucket calls "
        f"{out['multi_norm_pass_ms']} / {out['multi_fused_sums_ms']} ms, "
        f"{out['multi_fused_sums_nofill_ms']} ms without the zero_grad fill")
    return out


def ceilings(stream, update_bytes):
    """The practical ceilings of the update's traffic on this GPU, over its byte count
    `update_bytes`: torch's device copy (a blit kernel), and libttperf_ceiling's non-temporal
    16-byte copies (the update's 50/50 read/write mix; 256-lane blocks of 4 KiB and 64-lane
    blocks of 1 KiB, the fastest copy measured) and read-only pass, each timed over 10
    launches between one event pair on `stream`.  Returns (torch copy GB/s, NT copy GB/s,
    NT read GB/s, bytes each way, 64-lane NT copy GB/s)."""
    import torch

    dev = torch.device("cuda:0")
    copy_bytes = update_bytes // 2 // 16 * 16
    src = torch.empty(copy_bytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    src.normal_()
    ceil = ctypes.CDLL(os.path.join(REPO, "tt-perf_amd", "lib", "libttperf_ceiling.so"))
    ceil.ttpc_copy_nt.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                  ctypes.c_int, ctypes.c_void_p]
    ceil.ttpc_read_nt.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                  ctypes.c_void_p, ctypes.c_void_p]
    ceil.ttpc_copy_nt64.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                    ctypes.c_void_p]
    # the fastest forms measured (see tt-perf_amd/csrc/ceiling.hip): a straight-line copy,
    # one block per 4 KB tile, and a read over 8 blocks per CU
    read_grid = torch.cuda.get_device_properties(dev).multi_processor_count * 8
    n16 = copy_bytes // 16
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def nt_copy():
        rc = ceil.ttpc_copy_nt(src.data_ptr(), dst.data_ptr(), n16, 0, stream.cuda_stream)
        assert rc == 0, f"ttpc_copy_nt: hipError {rc}"

    def nt_copy64():
        rc = ceil.ttpc_copy_nt64(src.data_ptr(), dst.data_ptr(), n16, stream.cuda_stream)
        assert rc == 0, f"ttpc_copy_nt64: hipError {rc}"

    def nt_read():
        rc = ceil.ttpc_read_nt(src.data_ptr(), n16, read_grid, stream.cuda_stream,
                               sink.data_ptr())
        assert rc == 0, f"ttpc_read_nt: hipError {rc}"

    with torch.cuda.stream(stream):
        copy_gbps = 2 * copy_bytes / (timed(lambda: dst.copy_(src)) / 1e3) / 1e9
    nt_copy_gbps = 2 * copy_bytes / (timed(nt_copy) / 1e3) / 1e9
    nt_copy64_gbps = 2 * copy_bytes / (timed(nt_copy64) / 1e3) / 1e9
    nt_read_gbps = copy_bytes / (timed(nt_read) / 1e3) / 1e9
    del src, dst, sink
    return copy_gbps, nt_copy_gbps, nt_read_gbps, copy_bytes, nt_copy64_gbps


def make_store(config, seed=1234, layout="default", scaler=True, mode=None):
    """A store of `config`'s table on cuda:0 (in `layout`) with N(0, 0.02) master weights and
    the configuration's synthetic gradients resident in HBM, on a created stream; loss scaling
    as the configuration has it, unless `scaler` is False.  mode: the store's precision mode
    instead of the configuration's ("bf16": the same values as bf16 weights, no master).
    Returns (store, stream, grads as a device tensor)."""
    import torch
    import ttperf
    from ttperf import _lib as L
    from ttperf import configs

    names, shapes, decay, numels = configs.table(config)
    mode = mode or configs.mode(config)
    dev = torch.device("cuda:0")
    store = ttperf.ParamStore(shapes, mode=mode, decay=decay, names=names, layout=layout)
    # a created stream (the legacy default stream cannot be captured); torch's events and
    # synchronisation see it
    stream = torch.cuda.Stream()
    store.set_stream(stream)
    cfg = BENCH[config]
    scale = (cfg["scaler"] or 1.0) if scaler else 1.0
    gen = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn(store.total, generator=gen, device=dev) * 0.02
    if mode == "bf16":
        store.upload(L.BUF_PARAM, L.ALL_TENSORS, w.to(torch.bfloat16))
    else:
        store.upload(L.BUF_MASTER, L.ALL_TENSORS, w)
    del w
    if cfg["scaler"] and scaler:
        store.configure_scaler(True, init_scale=scale)
    g = torch.randn(store.total, generator=gen, device=dev) * cfg["std"]
    if cfg["heavy"]:
        pick = torch.rand(store.total, generator=gen, device=dev) < cfg["heavy"]
        g = torch.where(pick, torch.randn(store.total, generator=gen, device=dev), g)
        del pick
    g = g * scale
    g = g.to(torch.bfloat16) if mode != "fp32" else g
    store.upload(L.BUF_GRAD, L.ALL_TENSORS, g)
    return store, stream, g


# the reference's SGD (autograd/dynamic/optim.hpp:21-27, every traced sgd_step): w - lr*g, no
# clipping or loss scaling (bench/autograd/bench_gpt2_full.cpp:110 trains at lr 0.01)
SGD_LR = 0.01


def step_fn(store, optimizer, hp):
    if optimizer == "adamw":
        return lambda: store.adam_step(**hp)
    if optimizer == "sgd":
        return lambda: store.sgd_step(lr=SGD_LR)
    return lambda: store.sgd_step(lr=hp["lr"], momentum=0.9, max_grad_norm=hp["max_grad_norm"])


def update_kernel_name(optimizer, mode, total_elems, layout="default"):
    """The update instantiation libttperf_hip launches for a store (its rocprof name): the lane
    form with its elements per lane, lanes per block and pieces per block (kLaneAdamMixed ...
    in tt-perf_amd/csrc/ttperf.hip; the SGD forms also with their master's record stride, 64
    for a contiguous master), except while the gradients fit the Infinity Cache: MIXED Adam
    then takes the kLaneAdamMixedCached shape, and MIXED SGD momentum in the default layout the
    four-element kernel; a BF16 store's plain SGD its own kernel (kLaneSgdBf16)."""
    if mode == "bf16":
        return "sgd_bf16_lane_kernel<8, 64, 1>"
    grad_t, mixed_t = ("unsigned short", "true") if mode == "mixed" else ("float", "false")
    if optimizer == "adamw":
        if mode == "mixed" and total_elems * 2 <= CACHED_GRAD_BYTES:
            return f"adam_lane_kernel<{grad_t}, {mixed_t}, 1, 128, 2>"
        e, ln, it = (1, 256, 2) if mode == "mixed" else (1, 128, 2)
        return f"adam_lane_kernel<{grad_t}, {mixed_t}, {e}, {ln}, {it}>"
    contiguous = mode == "fp32" or layout == "sgd"
    stride = "64u" if contiguous else "192u"
    if optimizer == "sgdm" and not contiguous and total_elems * 2 <= CACHED_GRAD_BYTES:
        return f"sgd_kernel<{grad_t}, {mixed_t}, {stride}>"
    shape = {("sgdm", "mixed", False): (1, 256, 2), ("sgd", "mixed", False): (2, 256, 1),
             ("sgdm", "mixed", True): (2, 128, 1), ("sgd", "mixed", True): (4, 64, 1),
             ("sgdm", "fp32", True): (2, 64, 1), ("sgd", "fp32", True): (2, 256, 2)}[
        (optimizer, mode, contiguous)]
    return f"sgd_lane_kernel<{grad_t}, {mixed_t}, {stride}, {shape[0]}, {shape[1]}, {shape[2]}>"


def other_config(config, optimizer, steps, warmup, settle_ms, layout="default", mode=None):
    """One more configuration's step in a store of its own (created, timed, closed): settle
    steps and W warmup steps, K steps between one event pair, then K more with an event pair
    around every launch for the update kernel's own time.  The SGD legs step without loss
    scaling (plain SGD: the reference's w - lr*g, no norm pass; SGD momentum: the
    configuration's clipping).  mode: the store's precision mode instead of the
    configuration's ("bf16": the reference's own bf16-only storage).  Returns the JSON
    object."""
    import torch
    from ttperf import _lib as L
    from ttperf import configs

    _, _, _, numels = configs.table(config)
    mode = mode or configs.mode(config)
    n_params = sum(numels)
    cfg = BENCH[config]
    hp = dict(cfg["hp"], decoupled=cfg["decoupled"])
    scaler = bool(cfg["scaler"]) and optimizer == "adamw"
    store, stream, g = make_store(config, layout=layout, scaler=scaler, mode=mode)
    del g
    torch.cuda.empty_cache()
    step = step_fn(store, optimizer, hp)
    settle_n, _ = settle(step, settle_ms)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    store.timing(True)
    store.timing_collect(L.KERNEL_NORM)
    store.timing_collect(L.KERNEL_UPDATE)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    upd_ms, upd_n = store.timing_collect(L.KERNEL_UPDATE)
    nrm_ms, nrm_n = store.timing_collect(L.KERNEL_NORM)
    store.timing(False)
    upd_kernel = update_kernel_name(optimizer, mode, store.total, layout)
    sgd_layout = store.sgd_layout
    # with loss scaling: 20 overflow steps between one event pair (a +inf planted in the
    # first tensor's gradients), as for the headline configuration
    skip_ms = None
    if scaler:
        store.upload(L.BUF_GRAD, 0, torch.full((numels[0],), float("inf"), device="cuda",
                                               dtype=torch.bfloat16 if mode != "fp32"
                                               else torch.float32))
        rs = store.adam_step(report=True, **hp)
        assert rs["skipped"], rs
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(20):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        skip_ms = e0.elapsed_time(e1) / 20
    store.close()
    torch.cuda.empty_cache()
    ub = UPDATE_BYTES[(optimizer, mode)]
    # the norm pass runs only with clipping or loss scaling (plain SGD has neither)
    norm_runs = optimizer != "sgd" and bool(cfg["hp"]["max_grad_norm"] or scaler)
    nb = NORM_BYTES[mode] if norm_runs else 0
    upd_avg = upd_ms / max(upd_n, 1)
    step_gbps = n_params * (ub + nb) / (ms / 1e3) / 1e9
    upd_gbps = n_params * ub / (upd_avg / 1e3) / 1e9
    # the plain non-temporal copies of the update's bytes on this GPU, in the same run; the
    # update's own time and rate only where they mean something (MIN_TIMED_UPDATE_BYTES)
    timed = n_params * ub >= MIN_TIMED_UPDATE_BYTES
    nt_copy_gbps = nt_copy64_gbps = None
    if timed:
        _, nt_copy_gbps, _, _, nt_copy64_gbps = ceilings(stream, n_params * ub)
    log(f"bench: {config} {optimizer} ({layout} layout): {ms:.4f} ms/step, "
        f"update {upd_avg:.4f} ms")
    return {"ms_per_step": round(ms, 4),
            "Gparams_per_s": round(n_params / (ms / 1e3) / 1e9, 3),
            "step_bytes_per_param": ub + nb,
            "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
            "update_ms": round(upd_avg, 4) if timed else None,
            "update_frac": round(upd_gbps / HBM_PEAK_GBPS, 4) if timed else None,
            "update_vs_nt_copy": round(upd_gbps / nt_copy_gbps, 4) if nt_copy_gbps else None,
            "nt_copy_GBps": round(nt_copy_gbps, 1) if nt_copy_gbps else None,
            "update_vs_nt_copy64": round(upd_gbps / nt_copy64_gbps, 4) if nt_copy64_gbps else None,
            "nt_copy64_GBps": round(nt_copy64_gbps, 1) if nt_copy64_gbps else None,
            "norm_pass_ms": round(nrm_ms / max(nrm_n, 1), 4) if (timed and norm_runs) else None,
            "skipped_step_ms": round(skip_ms, 4) if skip_ms is not None else None,
            "update_kernel": upd_kernel,
            "optimizer": {"adamw": "AdamW", "sgdm": "SGD momentum 0.9",
                          "sgd": f"SGD (w - lr*g, lr {SGD_LR})"}[optimizer]
                         + (", clip 1.0" if optimizer != "sgd" and cfg["hp"]["max_grad_norm"]
                            else "")
                         + (f", loss scaling {cfg['scaler']:g}" if scaler else ""),
            "layout": "sgd" if sgd_layout else "default",
            "params": n_params, "tensors": len(numels), "mode": mode,
            "steps": steps, "warmup": warmup, "settle_steps": settle_n}


def cpp_dropin(steps, warmup, settle_ms):
    """The optimizer step of the reference's GPT benchmark model (traced::
    TracedTransformerWithEmbedding<12> at GPT-2 small dimensions, bench/autograd/
    bench_gpt2_full.cpp:74-100), timed by the C++ drop-in program tests/cpp/bench_gpt2_step
    through autograd::AdamW and the model's sgd_step(), in a process of its own.  Returns its
    JSON line, and whether its checks passed."""
    import subprocess
    exe = os.path.join(REPO, "tests", "cpp", "build", "bench_gpt2_step")
    if not os.access(exe, os.X_OK):
        return {"error": f"{exe} is not built (make -C tests/cpp)"}
    env = dict(os.environ, BENCH_ITERS=str(steps), BENCH_WARMUP=str(warmup),
               BENCH_SETTLE_MS=str(int(settle_ms)))
    try:
        p = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    except subprocess.TimeoutExpired:
        return {"error": f"{exe} did not finish within 300 s"}
    line = next((ln for ln in p.stdout.splitlines() if ln.startswith('{"bench"')), None)
    if p.returncode != 0 or line is None:
        return {"error": f"exit {p.returncode}: {(p.stdout + p.stderr)[-500:]}"}
    res = json.loads(line)
    res["checks_passed"] = "bench_gpt2_step: PASS" in p.stdout
    res["note"] = ("C++ drop-in surface, mixed precision, 200 ms of settle steps then W warmup "
                   "and K steps between two synchronisations (std::chrono, as the reference's "
                   "bench); AdamW with loss scaling 2^16 and clip 1.0 at 30 B/param, the "
                   "model's sgd_step at 12 B/param (SGD layout), and the same sgd_step on the "
                   "reference's bf16-only storage (sgd_bf16_*, a Bf16 arena, 6 B/param); no "
                   "tied embedding, so 163M params")
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this engine runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import ttperf
    from ttperf import _lib as L
    from ttperf import configs

    names, shapes, decay, numels = configs.table(args.config)
    mode = configs.mode(args.config) if args.mode == "config" else args.mode
    if mode == "bf16" and args.optimizer != "sgd":
        sys.exit("bench.py: a bf16 store steps plain SGD only (--optimizer sgd)")
    n_params = sum(numels)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = BENCH[args.config]
    hp = dict(cfg["hp"], decoupled=cfg["decoupled"])
    # the SGD steps run without loss scaling (see other_config)
    scaler = bool(cfg["scaler"]) and args.optimizer == "adamw"
    scale = cfg["scaler"] if scaler else 1.0
    norm_runs = args.optimizer != "sgd" and bool(cfg["hp"]["max_grad_norm"] or scaler)
    store, stream, g = make_store(args.config, layout=args.layout, scaler=scaler, mode=mode)
    store_total = store.total
    grads_host = None
    if not args.no_cpu_baseline and args.optimizer == "adamw":
        grads_host = (g.cpu().view(torch.int16).numpy().view(np.uint16) if mode == "mixed"
                      else g.cpu().numpy())
    del g
    torch.cuda.empty_cache()

    step = step_fn(store, args.optimizer, hp)

    r = store.adam_step(report=True, **hp) if args.optimizer == "adamw" else None
    if r is not None:
        assert not r["skipped"], r
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # for comparison, the same W warmup + K timed steps right after the set-up, before the
    # settle phase: they fall in the clocks' ramp after the idle set-up
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    unsettled_ms = e0.elapsed_time(e1) / args.steps
    settle_n, settle_ms = settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # the step as a hipGraph (the reference's trace capture/replay): one capture, K replays
    run = step
    if args.graph:
        store.begin_capture()
        step()
        graph = store.end_capture()
        run = graph.replay
        for _ in range(2):
            run()
        torch.cuda.synchronize()

    # timed region: exactly K steps between one event pair (an event per launch would put
    # a marker packet between the kernels and lengthen the step)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    total_ms = e0.elapsed_time(e1)
    ms_step = total_ms / args.steps

    # per-kernel durations for the roofline: the same K steps again, with a HIP event pair
    # recorded around every launch on the stream the kernels run on
    store.timing(True)
    store.timing_collect(L.KERNEL_NORM)
    store.timing_collect(L.KERNEL_UPDATE)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    upd_ms, upd_n = store.timing_collect(L.KERNEL_UPDATE)
    nrm_ms, nrm_n = store.timing_collect(L.KERNEL_NORM)
    store.timing(False)
    upd_avg = upd_ms / max(upd_n, 1)
    nrm_avg = nrm_ms / max(nrm_n, 1)

    if args.graph:
        graph.close()

    # the step with a cold Infinity Cache: before each step, a read of 512 MB of unrelated
    # data (twice the 256 MB cache) on the same stream, outside the step's event pair
    flush = torch.ones(128 << 20, dtype=torch.float32, device=dev)
    sink = torch.zeros((), dtype=torch.float32, device=dev)
    cold = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(args.steps)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for a, b in cold:
            torch.sum(flush, dim=0, out=sink)
            a.record(stream)
            step()
            b.record(stream)
    torch.cuda.synchronize()
    cold_ms = sum(a.elapsed_time(b) for a, b in cold) / args.steps
    del flush, sink

    # the step right after its gradients were rewritten, as a backward leaves them: K times a
    # device copy of the gradients from a second buffer, then the step, between one event pair;
    # then the K copies alone
    gview = store.torch_view(L.BUF_GRAD)
    backup = gview.clone()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(args.steps):
            gview.copy_(backup)
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        pair_ms = e0.elapsed_time(e1) / args.steps
        e0.record(stream)
        for _ in range(args.steps):
            gview.copy_(backup)
        e1.record(stream)
        torch.cuda.synchronize()
        gcopy_ms = e0.elapsed_time(e1) / args.steps
    del gview, backup

    # skipped (overflow) steps: only the norm pass and the finalize do work; min(K, 20) of
    # them between one event pair (each backs the loss scale off; it is reset afterwards)
    skip_ms, n_skip = None, 0
    if scaler:
        store.upload(L.BUF_GRAD, 0, torch.full((store.tensors[0].numel,), float("inf"),
                                               device=dev, dtype=torch.bfloat16 if mode != "fp32"
                                               else torch.float32))
        rs = store.adam_step(report=True, **hp)
        assert rs["skipped"], rs
        n_skip = min(args.steps, 20)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n_skip):
            store.adam_step(**hp)
        e1.record(stream)
        torch.cuda.synchronize()
        skip_ms = e0.elapsed_time(e1) / n_skip
        store.configure_scaler(True, init_scale=scale)

    # context: the step with its norm from bucketed per-tensor sums (first undoing the overflow
    # planted above), and the practical ceilings of the update's traffic on this GPU
    sums = None
    if norm_runs:
        store.upload(L.BUF_GRAD, 0, torch.zeros(store.tensors[0].numel, device=dev,
                                                dtype=torch.bfloat16 if mode != "fp32"
                                                else torch.float32))
        sums = bucketed_norm(store, stream, args, hp, mode, numels)
    producer = None
    if norm_runs and args.optimizer == "adamw":
        producer = producer_step(store, stream, args, hp, mode, numels)
    ub = UPDATE_BYTES[(args.optimizer, mode)]
    nb = NORM_BYTES[mode] if norm_runs else 0
    copy_gbps, nt_copy_gbps, nt_read_gbps, copy_bytes, nt_copy64_gbps = \
        ceilings(stream, n_params * ub)

    achieved = n_params * ub / (upd_avg / 1e3) / 1e9
    upd_kernel = update_kernel_name(args.optimizer, mode, store_total, args.layout)
    step_gbps = n_params * (ub + nb) / (ms_step / 1e3) / 1e9
    out = {
        "metric": HEADLINE if args.config == "gpt2_124m" and args.optimizer == "adamw" else
                  f"fused {args.optimizer} step Gparams/s + % of HBM peak, {args.config} {mode}"
                  + (" (SGD layout)" if args.layout == "sgd" else ""),
        "value": round(n_params / (ms_step / 1e3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if mode == "bf16" else "fp32",
        "launch": "hipGraph replay of the captured step" if args.graph else "eager launches",
        "data": f"synthetic (seeded N(0,{cfg['std']:g})"
                + (f", {cfg['heavy']:g} of them N(0,1)" if cfg["heavy"] else "")
                + (f" x loss scale {scale:g}" if scaler else "")
                + (" bf16" if mode != "fp32" else " fp32") + " grads, N(0,0.02) "
                + ("bf16 weights)" if mode == "bf16" else "fp32 master)"),
        "config": {"workload": f"{args.config} {args.optimizer} step: {len(numels)} tensors, "
                               f"{n_params} params, {mode} precision, "
                               + (f"loss scaling {scale:g}, " if scaler else "")
                               + (f"clip {hp['max_grad_norm']}, "
                                  if hp["max_grad_norm"] and args.optimizer != "sgd" else "")
                               + (f"lr {hp['lr']:g}, betas {hp['betas']}, "
                                  f"wd {hp['weight_decay']:g} on 2-D tensors"
                                  if args.optimizer == "adamw" else
                                  f"lr {hp['lr']:g}, momentum 0.9" if args.optimizer == "sgdm"
                                  else f"lr {SGD_LR:g} (w - lr*g)")
                               + (", SGD layout" if args.layout == "sgd" else ""),
                   "params": n_params, "tensors": len(numels), "mode": mode,
                   "bytes_per_param": ub + nb},
        "step_hbm_GBps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "kernels_ms": {"norm_pass": round(nrm_avg, 4), "update": round(upd_avg, 4),
                       "source": "second pass of K steps with an event pair per launch"},
        "settle": {"steps": settle_n, "ms": settle_ms,
                   "unsettled_ms_per_step": round(unsettled_ms, 4),
                   "note": "untimed steps run back to back before the W warmup steps, so that "
                           "the timed steps see the clocks of a busy GPU, as in a training loop "
                           "(the first tens of ms after an idle phase run at lower clocks); "
                           "unsettled_ms_per_step: W warmup + K timed steps right after the "
                           "set-up, before the settle steps"},
        "cold_ms_per_step": round(cold_ms, 4),
        "cold_Gparams_per_s": round(n_params / (cold_ms / 1e3) / 1e9, 3),
        "cold_note": "each step after a 512 MB read of unrelated data on its stream (outside "
                     "its event pair), so no gradient is left in the 256 MB Infinity Cache",
        "after_grad_write": {
            "pair_ms": round(pair_ms, 4), "grad_copy_ms": round(gcopy_ms, 4),
            "step_ms": round(pair_ms - gcopy_ms, 4),
            "Gparams_per_s": round(n_params / ((pair_ms - gcopy_ms) / 1e3) / 1e9, 3),
            "note": "K times a device copy of the gradients from a second buffer (as a backward "
                    "writes them) then the step, between one event pair (pair_ms); the copies "
                    "alone (grad_copy_ms); step_ms is the difference"},
        "skipped_step_ms": round(skip_ms, 4) if skip_ms is not None else None,
        "skipped_step_note": f"mean of {n_skip} overflow steps between one event pair",
        "bucketed_norm": sums,
        "producer_step": producer,
        "torch_copy_GBps": round(copy_gbps, 1),
        "ceilings": {"nt_copy_GBps": round(nt_copy_gbps, 1),
                     "nt_copy_frac": round(nt_copy_gbps / HBM_PEAK_GBPS, 4),
                     "nt_read_GBps": round(nt_read_gbps, 1),
                     "bytes_each_way": copy_bytes,
                     "update_vs_nt_copy": round(achieved / nt_copy_gbps, 4),
                     "nt_copy64_GBps": round(nt_copy64_gbps, 1),
                     "update_vs_nt_copy64": round(achieved / nt_copy64_gbps, 4),
                     "source": "libttperf_ceiling: 16-byte non-temporal straight-line copies "
                               "(reads + writes counted; 256-lane blocks, and 64-lane blocks, "
                               "the fastest copy measured) and read-only pass over the "
                               "update's byte count; 10 launches between one event pair"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_from_profiles(args.config, args.optimizer),
                     "kernel": upd_kernel,
                     "algorithmic_bytes_per_launch": n_params * ub},
        "cpu_baseline": None,
        "other_configs": None,
        "cpp_dropin": None,
    }
    store.close()
    del store
    torch.cuda.empty_cache()
    if not args.no_other_configs and args.config == "gpt2_124m" and args.optimizer == "adamw":
        # the other large configurations, one store at a time (GPT-2 XL fp32 holds 31 GB)
        legs = (("mlp_fp32_adam", "mlp", "adamw", "default"),
                ("nanogpt_char_mixed_adamw", "nanogpt_char", "adamw", "default"),
                ("gpt2_774m_mixed_adamw", "gpt2_774m", "adamw", "default"),
                ("gpt2_1558m_fp32_adamw", "gpt2_1558m", "adamw", "default"),
                ("gpt2_1558m_fp32_sgdm", "gpt2_1558m", "sgdm", "default"),
                # the reference's own optimizer (plain SGD) and SGD momentum in mixed
                # precision, on stores in the SGD layout; SGD momentum also in the default
                # layout ([master|m|v] records), which a store that Adam also steps keeps
                ("gpt2_124m_mixed_sgd", "gpt2_124m", "sgd", "sgd"),
                ("gpt2_774m_mixed_sgd", "gpt2_774m", "sgd", "sgd"),
                ("gpt2_124m_mixed_sgdm", "gpt2_124m", "sgdm", "sgd"),
                ("gpt2_774m_mixed_sgdm", "gpt2_774m", "sgdm", "sgd"),
                ("gpt2_774m_mixed_sgdm_default_layout", "gpt2_774m", "sgdm", "default"),
                # the reference's own storage and arithmetic: bf16 weights and gradients only,
                # plain SGD with each op rounded to bf16 (TTP_MODE_BF16)
                ("gpt2_124m_bf16_sgd", "gpt2_124m", "sgd", "default", "bf16"),
                ("gpt2_774m_bf16_sgd", "gpt2_774m", "sgd", "default", "bf16"))
        out["other_configs"] = {
            leg[0]: other_config(leg[1], leg[2], args.steps, args.warmup, args.settle_ms,
                                 *leg[3:])
            for leg in legs}
        out["other_configs"]["note"] = (
            "each in a store of its own, created, timed (settle steps and W warmup steps, then "
            "K steps between one event pair; the update alone from a second pass with an event "
            "pair per launch) and closed before the next; no CPU leg; the update's own time, "
            "the copy ceilings and the norm pass's time only where the update moves at least "
            "1 GiB (the MLP's 269 KB step is launch-bound and the char model's 301 MB update "
            "mostly Infinity-Cache resident: an event pair around each of their launches "
            "measures mostly its own overhead; see profiles/ for their kernels' durations)")
        log("bench: the C++ drop-in program (tests/cpp/bench_gpt2_step) ...")
        out["cpp_dropin"] = cpp_dropin(args.steps, args.warmup, args.settle_ms)
    if grads_host is not None:
        log("bench: timing the CPU oracle baseline ...")
        out["cpu_baseline"] = cpu_baseline(numels, [1 if d else 0 for d in decay],
                                           mode == "mixed", grads_host, hp, args.cpu_seconds,
                                           cfg["scaler"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
