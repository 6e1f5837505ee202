"""Host-side checks that need no GPU: the C ABI library loads and exports every entry point
include/ttperf/ttperf.h declares, the ctypes and C struct layouts agree, argument errors are
reported as the reference reports them (ValueError in py/optim.py), and the C++ drop-in
headers compile against the library."""
import ctypes as C
import os
import re
import subprocess
import sys

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "ttperf", "ttperf.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ttp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from ttperf import _lib as L
    declared = _declared_functions()
    assert len(declared) >= 30
    missing = [n for n in declared if not hasattr(L.lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ttp_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared) <= exported
    # and the ctypes binding describes each of them
    assert set(declared) == set(L.SIGNATURES)


def test_ceiling_probe_library_exports_its_entry_points():
    """bench.py's HBM ceilings come from libttperf_ceiling (built with the engine)."""
    path = os.path.join(REPO, "tt-perf_amd", "lib", "libttperf_ceiling.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    names = set(re.findall(r"\b(ttpc_\w+)", out))
    assert {"ttpc_copy_nt", "ttpc_copy_nt64", "ttpc_read_nt"} <= names


def test_abi_version():
    """The library, the header and the ctypes binding agree on the ABI version (3: the BF16
    store mode; 2: the SGD layout flag, and the has-grad behaviour of zero_grad_subset /
    captured accumulates), and on the mode and flag values."""
    from ttperf import _lib as L
    text = open(HEADER).read()
    header = int(re.search(r"#define TTP_ABI_VERSION (\d+)", text).group(1))
    assert L.lib.ttp_abi_version() == header == L.ABI_VERSION == 3
    for name in ("FP32", "MIXED", "BF16"):
        assert int(re.search(r"#define TTP_MODE_%s (\d+)" % name, text).group(1)) == \
            getattr(L, "MODE_" + name)
    assert int(re.search(r"#define TTP_STORE_SGD (0x[0-9a-fA-F]+)", text).group(1), 16) == \
        L.STORE_SGD
    assert int(re.search(r"#define TTP_ACCUM_SUMSQ (0x[0-9a-fA-F]+)", text).group(1), 16) == \
        L.ACCUM_SUMSQ
    # the C++ wrapper refuses a library of another version
    hpp = open(os.path.join(REPO, "include", "ttperf", "ttperf.hpp")).read()
    assert "ttp_abi_version() != TTP_ABI_VERSION" in hpp


def test_struct_layouts_match_the_header(tmp_path):
    """Compiles a C probe against the header and compares sizeof/offsetof with ctypes."""
    from ttperf import _lib as L
    structs = {"ttp_tensor_desc": L.TensorDesc, "ttp_adam_hparams": L.AdamHParams,
               "ttp_sgd_hparams": L.SgdHParams, "ttp_scaler_config": L.ScalerConfig,
               "ttp_step_report": L.StepReport}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ttperf/ttperf.h"',
             "int main(void) {"]
    for cname, ct in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in ct._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), "-o", str(exe),
                    str(src)], check=True)
    got = dict(line.rsplit(" ", 1) for line in
               subprocess.run([str(exe)], capture_output=True, text=True,
                              check=True).stdout.splitlines())
    for cname, ct in structs.items():
        assert int(got[f"{cname} size"]) == C.sizeof(ct), cname
        for f, _ in ct._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(ct, f).offset, f"{cname}.{f}"


def test_c_abi_argument_errors_without_a_device():
    from ttperf import _lib as L
    lib = L.lib
    h = C.c_void_p()
    d = (L.TensorDesc * 1)()
    d[0].numel = 10
    assert lib.ttp_create(0, d, 1, 7, C.byref(h)) == L.ERR_INVALID  # unknown mode
    assert b"mode" in lib.ttp_last_error()
    d[0].flags = 0x80
    assert lib.ttp_create(0, d, 1, L.MODE_FP32, C.byref(h)) == L.ERR_INVALID  # unknown flag
    d[0].flags = 0
    d[0].reserved = 1
    assert lib.ttp_create(0, d, 1, L.MODE_FP32, C.byref(h)) == L.ERR_INVALID  # reserved != 0
    assert b"reserved" in lib.ttp_last_error()
    d[0].reserved = 0
    # a table whose padded sizes would wrap 64 bits (or exceed 2^40 elements) is rejected
    # before any device work: a wrapped footprint would let kernels index past the buffers
    d[0].flags = 0
    d[0].numel = 2**64 - 1
    assert lib.ttp_create(0, d, 1, L.MODE_FP32, C.byref(h)) == L.ERR_INVALID
    assert b"2^40" in lib.ttp_last_error()
    d2 = (L.TensorDesc * 3)()
    for k in range(3):
        d2[k].numel = 2**39 + 1
    assert lib.ttp_create(0, d2, 3, L.MODE_FP32, C.byref(h)) == L.ERR_INVALID
    assert b"total" in lib.ttp_last_error()
    d[0].numel = 10
    assert lib.ttp_create(0, d, 1, L.MODE_FP32, None) == L.ERR_INVALID
    hp = L.AdamHParams(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8)
    assert lib.ttp_adam_step(None, C.byref(hp), None) == L.ERR_INVALID
    assert b"null context" in lib.ttp_last_error()
    assert lib.ttp_sync(None) == L.ERR_INVALID
    assert lib.ttp_destroy(None) == L.OK
    n = C.c_int(-1)
    assert lib.ttp_device_count(C.byref(n)) == L.OK and n.value >= 0


def test_store_without_a_device_fails_loudly():
    import ttperf
    from ttperf import _lib as L
    if ttperf.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(ttperf.TTPError) as e:
        ttperf.ParamStore([(4, 4)])
    assert e.value.code == L.ERR_NO_DEVICE


# ---- the reference's validation cases (tests/adam_optimizer.py:126-151,
#      tests/sgd_optimizer.py:112-122, py/optim.py:9-16,33-41) -----------------------------

@pytest.mark.parametrize("kw", [dict(lr=0.0), dict(lr=-1.0), dict(eps=0.0), dict(betas=(0.9,)),
                                dict(betas=(1.1, 0.9)), dict(betas=(0.9, 1.0)),
                                dict(betas=0.9), dict(weight_decay=-0.1)])
def test_adam_validation(kw):
    import ttperf
    for cls in (ttperf.Adam, ttperf.AdamW):
        with pytest.raises(ValueError):
            cls([], **kw)


@pytest.mark.parametrize("kw", [dict(lr=0.0), dict(lr=-1.0), dict(lr=0.1, momentum=-0.5),
                                dict(lr=0.1, weight_decay=-1.0), dict(lr=0.1, nesterov=True),
                                dict(lr=0.1, momentum=0.9, dampening=0.1, nesterov=True)])
def test_sgd_validation(kw):
    import ttperf
    with pytest.raises(ValueError):
        ttperf.SGD([], **kw)


def test_sgd_lr_is_keyword_only():
    import ttperf
    with pytest.raises(TypeError):
        ttperf.SGD([], 0.1)  # py/optim.py:7 `SGD(params, *, lr)`


def test_adam_defaults_match_reference():
    import ttperf
    a = ttperf.Adam([])
    assert (a.lr, a.beta1, a.beta2, a.eps) == (1e-3, 0.9, 0.999, 1e-8)  # py/optim.py:31


def test_non_tensor_params_raise_at_step_and_are_skipped_by_zero_grad():
    import ttperf
    for cls, kw in ((ttperf.SGD, dict(lr=0.1)), (ttperf.Adam, {})):
        opt = cls([object()], **kw)  # construction accepts anything (py/optim.py:8,32)
        opt.zero_grad()              # skips non-Tensors (py/optim.py:24-27,89-92)
        with pytest.raises(ValueError, match="expects Tensor parameters"):
            opt.step()


class _CountingStore:
    """Stands in for a ParamStore: a step count that every step advances, and a count of the
    synchronising reads and writes of it."""

    def __init__(self, n):
        import ttperf
        self.mode = ttperf._lib.MODE_MIXED
        self._t = 0
        self.reads = self.writes = 0
        self._t_owner = None
        self._in_capture = False
        self.tensors = [ttperf.Tensor(self, i, (4,)) for i in range(n)]
        self.log = []

    @property
    def step_count(self):
        self.reads += 1
        return self._t

    @step_count.setter
    def step_count(self, t):
        self.writes += 1
        self._t = t

    def adam_step(self, lr, betas, eps, weight_decay, decoupled, max_grad_norm, indices=None,
                  tensor_sums=False, update_scale=True):
        self._t += 1
        self.log.append((lr, self._t))

    def sgd_step(self, lr, momentum, dampening, weight_decay, nesterov, max_grad_norm,
                 indices=None, tensor_sums=False, update_scale=True):
        self._t += 1
        self.log.append((lr, self._t))


def test_each_optimizer_keeps_its_own_step_count():
    """py/optim.py:46,50: `_step` belongs to the optimizer.  Two optimizers over two groups
    of one store each see their own count; one optimizer alone never reads the device."""
    import gc
    import ttperf
    s = _CountingStore(4)
    a = ttperf.Adam(s.tensors[:2], lr=1.0)
    b = ttperf.Adam(s.tensors[2:], lr=2.0)
    for opt in (a, a, a):
        opt.step()
    assert (s.reads, s.writes) == (0, 0)
    for opt in (b, a, b, b, a):
        opt.step()
    assert [t for _, t in s.log] == [1, 2, 3, 1, 4, 2, 3, 5]
    assert [lr for lr, _ in s.log] == [1.0] * 3 + [2.0, 1.0, 2.0, 2.0, 1.0]
    assert s.step_count == 5  # the count of the optimizer that stepped last
    # an SGD over a third group hands the count over too, so Adam's bias corrections hold
    c = ttperf.SGD(s.tensors[1:2], lr=3.0)
    c.step()
    b.step()
    a.step()
    assert s.log[-3:] == [(3.0, 1), (2.0, 4), (1.0, 6)]
    # a store whose last optimizer is gone keeps its count for the next one (a checkpoint's)
    del a, c, opt
    gc.collect()
    s._t = 41
    s.log.clear()
    d = ttperf.AdamW(s.tensors[:2], lr=4.0)
    d.step()
    assert s.log == [(4.0, 42)]
    b.step()
    assert s.log[-1] == (2.0, 5)
    # a hand-over reads the device, which a graph capture cannot hold
    s._in_capture = True
    with pytest.raises(RuntimeError, match="capture"):
        d.step()
    b.step()  # no hand-over: fine while capturing
    assert s.log[-1] == (2.0, 6)


def test_cpp_dropin_headers_compile():
    """The C++ drop-in tests and bench program (tests/cpp) build against include/ and the
    library."""
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "tests", "cpp")], check=True)
    for t in ("test_sgd", "test_traced", "test_adam", "test_modules", "train_mlp", "test_store",
              "bench_gpt2_step"):
        assert os.access(os.path.join(REPO, "tests", "cpp", "build", t), os.X_OK)


def test_product_code_never_touches_the_oracle():
    """Only tests/, smoke() and bench.py's cpu_baseline may load oracle/."""
    pkg = os.path.join(REPO, "tt-perf_amd")
    hits = []
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")) or f == "Makefile":
                text = open(os.path.join(root, f), errors="replace").read()
                if re.search(r"import oracle|from oracle|ttp_oracle|\borc_[a-z]|oracle/", text):
                    hits.append(os.path.join(root, f))
    for root, _, files in os.walk(os.path.join(REPO, "include")):
        for f in files:
            if re.search(r"ttp_oracle|orc_", open(os.path.join(root, f)).read()):
                hits.append(os.path.join(root, f))
    assert not hits, hits


@pytest.mark.parametrize("args, env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})])
def test_bench_refuses_more_than_one_gpu(args, env):
    """This build measures one GPU: bench.py with --gpus above 1 (or under a multi-rank
    launcher) exits with status 2 and says so, before it touches a GPU."""
    e = dict(os.environ, **env)
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py")] + args, env=e,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stderr)
    assert "one GPU" in r.stderr and not r.stdout.strip()


def test_one_hip_runtime_is_mapped():
    """ttperf loads torch's HIP runtime (when torch is installed) before libttperf_hip, so
    the process maps a single libamdhip64 / libhsa-runtime64."""
    import ttperf  # noqa: F401
    maps = open("/proc/self/maps").read().splitlines()
    for lib in ("libamdhip64", "libhsa-runtime64"):
        paths = {line.split()[-1] for line in maps if lib in line}
        assert len(paths) == 1, paths


def test_shard_tables_partition_the_flat_store():
    """configs.shard_table: the 8 shards of GPT-2 124M cover every element exactly once, each
    piece starts and ends on 64-element boundaries of the flat layout (whole state records)
    unless it ends its tensor, and keeps its tensor's decay flag."""
    from ttperf import configs
    names, _, decay, numels = configs.table("gpt2_124m")
    flags = dict(zip(names, decay))
    covered = {n: 0 for n in names}
    for k in range(8):
        pn, ps, pd, pe = configs.shard_table("gpt2_124m", 8, k)
        for nm, shape, d, e in zip(pn, ps, pd, pe):
            base, rng = nm.split("[")
            a, b = (int(x) for x in rng.rstrip("]").split(":"))
            assert shape == (e,) and b - a == e and d == flags[base]
            assert a % 64 == 0
            assert b % 64 == 0 or b == numels[names.index(base)]
            covered[base] += e
    assert covered == dict(zip(names, numels))
    assert configs.table("gpt2_124m_shard8") == configs.shard_table("gpt2_124m", 8, 7)
    assert configs.mode("gpt2_124m_shard8") == "mixed"


def test_bench_calls_match_its_function_signatures():
    """Every call in bench.py of one of its own functions passes as many positional arguments
    as the function takes without defaults, at most as many as it takes in all, and only
    keywords it names (a mismatch would surface only on the GPU box, after minutes of
    timing)."""
    import ast
    tree = ast.parse(open(os.path.join(REPO, "bench.py")).read())
    defs = {f.name: f for f in tree.body if isinstance(f, ast.FunctionDef)}
    calls = 0
    for node in ast.walk(tree):
        if not (isinstance(node, ast.Call) and isinstance(node.func, ast.Name)
                and node.func.id in defs):
            continue
        a = defs[node.func.id].args
        names = [x.arg for x in a.args]
        required = len(names) - len(a.defaults)
        given = len(node.args) + sum(1 for k in node.keywords if k.arg in names[len(node.args):])
        assert given >= required, (node.func.id, node.lineno)
        assert len(node.args) <= len(names) or a.vararg, (node.func.id, node.lineno)
        assert all(k.arg in names or a.kwarg for k in node.keywords), (node.func.id, node.lineno)
        calls += 1
    assert calls >= 10


def test_bench_names_the_update_shapes_the_library_launches():
    """bench.py reports the update instantiation it timed (its rocprof name); the shapes it
    assumes for the lane forms must be the library's (ttperf.hip's kLane* constants) and its
    Infinity Cache bound the library's kCachedGradBytes."""
    src = open(os.path.join(REPO, "tt-perf_amd", "csrc", "ttperf.hip")).read()

    def shape(name):
        m = re.search(r"constexpr int kLane%s = (\d+), kLanes%s = (\d+), kIt%s = (\d+);"
                      % (name, name, name), src)
        assert m, name
        return tuple(int(x) for x in m.groups())

    m = re.search(r"constexpr uint64_t kCachedGradBytes = (\d+)ull << (\d+);", src)
    assert m
    bound = int(m.group(1)) << int(m.group(2))
    sys.path.insert(0, REPO)
    import bench
    assert bench.CACHED_GRAD_BYTES == bound
    big = 1 << 30
    # (optimizer, mode, layout, shape constant, master stride of an SGD form)
    for (opt, mode, layout, name, stride) in (
            ("adamw", "mixed", "default", "AdamMixed", None),
            ("adamw", "fp32", "default", "AdamFp32", None),
            ("sgdm", "mixed", "default", "SgdMixed", "192u"),
            ("sgd", "mixed", "default", "SgdPlainMixed", "192u"),
            ("sgdm", "mixed", "sgd", "SgdMomContig", "64u"),
            ("sgd", "mixed", "sgd", "SgdPlainContig", "64u"),
            ("sgdm", "fp32", "default", "SgdFp32", "64u"),
            ("sgd", "fp32", "default", "SgdPlainFp32", "64u")):
        grad_t, mixed_t = ("unsigned short", "true") if mode == "mixed" else ("float", "false")
        e, lanes, it = shape(name)
        kname = "adam" if opt == "adamw" else "sgd"
        tmpl = f"{grad_t}, {mixed_t}, " + (f"{stride}, " if stride else "")
        want = f"{kname}_lane_kernel<{tmpl}{e}, {lanes}, {it}>"
        assert bench.update_kernel_name(opt, mode, big, layout) == want, (opt, mode, layout)
        # below the bound: MIXED Adam its cached-gradient lane shape, MIXED SGD momentum in
        # the default layout the four-element kernel, every other update the same lane form
        if name == "AdamMixed":
            e, lanes, it = shape("AdamMixedCached")
            want = f"adam_lane_kernel<{tmpl}{e}, {lanes}, {it}>"
        if name == "SgdMixed":
            want = f"sgd_kernel<{grad_t}, {mixed_t}, {stride}>"
        assert bench.update_kernel_name(opt, mode, 1 << 20, layout) == want, (opt, mode, layout)
        # and the library launches that instantiation
        kern = re.sub(r"<.*", "", want)
        assert kern in src
    # the library launches no four-element Adam kernel, and the four-element SGD kernel only
    # in mixed precision
    assert "adam_kernel<" not in src
    assert "sgd_kernel<float" not in src
