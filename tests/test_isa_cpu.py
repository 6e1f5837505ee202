"""Checks of the library's own gfx950 assembly (hipcc -S of tt-perf_amd/csrc, the same flags
as the build; no GPU needed).

SCC live into a basic block.  The scalar condition code (SCC) is set by most scalar ALU
instructions and read by s_cselect, s_cbranch_scc0/1 and s_cmov.  hipcc (ROCm 7.2, gfx950)
once built accumulate_grad_tiles_kernel's min(n - t0, 8192) as an `s_cselect_b32` at the top
of the branch that takes the partial tile, reading an SCC last written by the compare of
another argument (`first`) in the block before: an assign into a tensor's last tile then
took the whole tile and wrote past the tensor's end.  None of this library's code reads SCC
before writing it in the same block, so any such read is reported here as a failure to be
looked at in the assembly before the build is trusted."""
import os
import re
import subprocess

import pytest

from conftest import REPO

PKG = os.path.join(REPO, "tt-perf_amd")
HIPCC = "/opt/rocm/bin/hipcc"

# instructions that read SCC (s_addc_u32 / s_subb_u32 read it as the carry of the add or
# subtract just before them, which the scan requires in the same block too)
_READS = re.compile(r"^\s*(s_cselect_b(32|64)|s_cbranch_scc[01]|s_cmov_b(32|64)|s_addc_u32|"
                    r"s_subb_u32)\b")
# scalar instructions that leave SCC alone
_KEEPS = re.compile(r"^\s*(s_mov|s_movk|s_cmov|s_cselect|s_load|s_store|s_buffer|s_waitcnt|"
                    r"s_nop|s_getpc|s_setpc|s_swappc|s_branch|s_cbranch|s_endpgm|s_barrier|"
                    r"s_sleep|s_setprio|s_sendmsg|s_dcache|s_memtime|s_memrealtime|s_getreg|"
                    r"s_setreg|s_trap|s_icache|s_inst_prefetch|s_set_gpr|s_delay|s_clause|"
                    r"s_mul_i32|s_mul_hi|s_sext|s_movrel|s_bitset|s_brev|s_ff|s_flbit|"
                    r"s_quadmask|s_wqm|s_version|s_cvt|s_pack|s_sched)")


def scc_reads_live_into_a_block(asm_lines):
    """(line number, function, block, instruction) of every SCC read with no SCC write before
    it in its basic block (a label, or a fall-through block the compiler marks `; %bb.N:`)."""
    out, fn, block, written = [], None, None, False
    for ln, line in enumerate(asm_lines, 1):
        if re.match(r"^_Z\S+:", line):
            fn, block, written = line.split(":")[0], "entry", False
            continue
        if re.match(r"^\.LBB\S+:", line) or line.startswith("; %bb."):
            block, written = line.strip(), False
            continue
        if fn is None or not line.startswith("\t") or line.lstrip().startswith(";"):
            continue
        if _READS.match(line) and not written:
            out.append((ln, fn, block, line.strip()))
        if re.match(r"^\s*s_\w+", line) and (not _KEEPS.match(line) or
                                              re.match(r"^\s*(s_addc_u32|s_subb_u32)", line)):
            written = True
    return out


@pytest.fixture(scope="module")
def isa(tmp_path_factory):
    if not os.access(HIPCC, os.X_OK):
        pytest.skip("hipcc absent")
    d = tmp_path_factory.mktemp("isa")
    subprocess.run(["make", "-s", "-C", PKG, "isa", f"ISA_DIR={d}"], check=True,
                   capture_output=True, timeout=600)
    return {name: open(os.path.join(d, name)).read().splitlines()
            for name in ("ttperf.s", "ceiling.s")}


@pytest.mark.parametrize("name", ["ttperf.s", "ceiling.s"])
def test_no_scc_read_is_live_into_a_block(isa, name):
    bad = scc_reads_live_into_a_block(isa[name])
    assert not bad, "SCC read before any write in its block:\n" + "\n".join(
        f"  {name}:{ln} {fn[:80]} {blk}: {ins}" for ln, fn, blk, ins in bad[:20])


def test_the_scan_finds_the_miscompiled_form():
    """The scan on the shape of the miscompiled block: the select reads the SCC of an earlier
    block's compare (found), and the same select after its own compare (not found)."""
    bad = ["_Zkernel:", "\ts_cmp_eq_u32 s12, 0", "\ts_cselect_b64 s[0:1], -1, 0",
           "\ts_cbranch_vccnz .LBB15_3", ".LBB15_3:", "\ts_cselect_b32 s16, s2, 0x2000",
           "\ts_endpgm"]
    good = bad[:5] + ["\ts_and_b64 s[8:9], vcc, exec"] + bad[5:]
    found = scc_reads_live_into_a_block(bad)
    assert [(f[2], f[3]) for f in found] == [(".LBB15_3:", "s_cselect_b32 s16, s2, 0x2000")]
    assert scc_reads_live_into_a_block(good) == []


def test_every_kernel_is_in_the_assembly(isa):
    """The scan read the real device code: each kernel family of the library is there."""
    text = "\n".join(isa["ttperf.s"])
    for k in ("adam_lane_kernel", "sgd_lane_kernel", "norm_partials_kernel",
              "norm_finalize_kernel", "accumulate_grad_tiles_kernel",
              "combine_pending_sums_kernel", "tensor_sums_kernel"):
        assert re.search(r"^_ZN3ttp\d+" + k, text, re.M), k
