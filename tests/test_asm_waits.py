"""The fragment reads of the MFMA tiles are inline assembly whose results the
compiler believes ready at once; only later `s_waitcnt lgkmcnt` blocks tied
to the fragment registers order them.  These tests scan the gfx950 assembly
that hipcc writes for the kernels using them (tests/asm_waits.py) for any
instruction touching such a register before its wait, after pinning the
scan on small listings with planted mistakes."""
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

from tests.asm_waits import check

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "burn_dragon_amd", "csrc")
# Translation units with assembly LDS reads (bdh_mfma.h: mma_64x128_dsasm,
# mma_64x64_dsasm, frag_64x128_read; bdh_gemm_f32.h: dread_kc, dread_rc).
UNITS = ["snap_wide.hip", "carry_prefill.hip", "layer_bf16.hip", "mfma_prefill.hip", "prefill_f32.hip", "vjp.hip",
         "roles_prefill.hip", "wide_gram.hip"]

_HEAD = "kern:\n"


def _listing(body):
    return _HEAD + "\n".join("\t" + l if not l.endswith(":") else l for l in body) + "\n\ts_endpgm\n"


def test_scan_accepts_a_waited_read():
    asm = _listing(["ds_read_b128 v[4:7], v1 offset:0", "s_waitcnt lgkmcnt(0)",
                    "v_mov_b32_e32 v8, v4"])
    assert check(asm) == []


def test_scan_flags_a_copy_before_the_wait():
    asm = _listing(["ds_read_b128 v[4:7], v1 offset:0", "v_mov_b32_e32 v8, v5",
                    "s_waitcnt lgkmcnt(0)"])
    assert len(check(asm)) == 1


def test_scan_flags_an_overwrite_before_the_wait():
    asm = _listing(["ds_read_b128 v[4:7], v1 offset:0", "v_add_u32_e32 v6, s5, v2",
                    "s_waitcnt lgkmcnt(0)"])
    assert len(check(asm)) == 1


def test_scan_counts_later_lds_operations():
    # lgkmcnt(1) with one later LDS read retires the first, not the second.
    first_ok = _listing(["ds_read_b128 v[4:7], v1", "ds_read_b128 v[8:11], v1 offset:16",
                         "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v20, v4"])
    second_early = _listing(["ds_read_b128 v[4:7], v1", "ds_read_b128 v[8:11], v1 offset:16",
                             "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v20, v9"])
    assert check(first_ok) == []
    assert len(check(second_early)) == 1


def test_scan_does_not_let_scalar_loads_stand_for_lds_reads():
    # A scalar load may return before an older LDS read: lgkmcnt(1) then
    # proves nothing about the read.
    asm = _listing(["ds_read_b128 v[4:7], v1", "s_load_dwordx2 s[4:5], s[0:1], 0x0",
                    "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v20, v4"])
    assert len(check(asm)) == 1


def test_scan_follows_branches():
    # The read is waited on the fall-through path only; the branch target
    # uses it unwaited.
    asm = _listing(["ds_read_b128 v[4:7], v1", "s_cbranch_scc1 .LBB0_2", "s_waitcnt lgkmcnt(0)",
                    "v_mov_b32_e32 v20, v4", "s_endpgm", ".LBB0_2:", "v_mov_b32_e32 v21, v4"])
    assert len(check(asm)) == 1
    # A loop that waits at its head for the reads issued at its tail.
    loop = _listing(["ds_read_b128 v[4:7], v1", ".LBB0_1:", "s_waitcnt lgkmcnt(0)",
                     "v_mov_b32_e32 v20, v4", "ds_read_b128 v[4:7], v1 offset:64",
                     "s_cbranch_scc1 .LBB0_1", "s_waitcnt lgkmcnt(0)"])
    assert check(loop) == []
    # The same loop reading the registers before the wait at its head.
    bad_loop = _listing(["ds_read_b128 v[4:7], v1", ".LBB0_1:", "v_mov_b32_e32 v20, v4",
                         "s_waitcnt lgkmcnt(0)", "ds_read_b128 v[4:7], v1 offset:64",
                         "s_cbranch_scc1 .LBB0_1", "s_waitcnt lgkmcnt(0)"])
    assert len(check(bad_loop)) >= 1


def test_scan_flags_a_write_on_every_path_only():
    # Read in flight on both paths into the merge, then overwritten: flagged.
    both = _listing(["ds_read_b128 v[4:7], v1", "s_cbranch_scc1 .LBB0_2", "v_mov_b32_e32 v20, v2",
                     ".LBB0_2:", "v_mov_b32_e32 v5, 0", "s_waitcnt lgkmcnt(0)"])
    assert len(check(both)) == 1
    # Waited on one path only: a write after the merge is not reported (the
    # step loops' loop-invariant branches make such paths, never taken).
    one = _listing(["ds_read_b128 v[4:7], v1", "s_cbranch_scc1 .LBB0_2", "s_waitcnt lgkmcnt(0)",
                    ".LBB0_2:", "v_mov_b32_e32 v5, 0", "s_waitcnt lgkmcnt(0)"])
    assert check(one) == []


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


def test_kernels_wait_for_their_lds_reads():
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    from burn_dragon_amd import build
    flags = [f for f in build.common_flags() if f not in ("-fPIC",)]
    out = tempfile.mkdtemp(prefix="bdh_asm_")

    def compile_one(unit):
        dst = os.path.join(out, unit + ".s")
        cmd = [hipcc] + flags + ["--cuda-device-only", "-S", os.path.join(CSRC, unit), "-o", dst]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return unit, open(dst).read()

    try:
        with ThreadPoolExecutor(max_workers=len(UNITS)) as ex:
            listings = list(ex.map(compile_one, UNITS))
    finally:
        shutil.rmtree(out, ignore_errors=True)
    problems = []
    for unit, text in listings:
        assert text.count("ds_read_b128") > 0, unit  # the scan sees the fragment reads
        problems += check(text, unit)
    assert problems == [], "\n".join(problems[:20])
