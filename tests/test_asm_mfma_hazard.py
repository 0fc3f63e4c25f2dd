"""The 4-wave gram tiles (burn_dragon_amd/csrc/wide_gram.hip) issue their MFMAs
as inline assembly with the accumulators tied in place, so the compiler does
not know that those instructions write the accumulator registers and inserts
no wait states before later instructions read them.  The kernel covers the
hazard by hand (s_nop after the step loop; without them the schedule of this
build still leaves 28 wait states, with them 52).  This test scans the gfx950
assembly that hipcc writes for it: every instruction that names an
accumulator register (a0..a255) after an MFMA, other than another MFMA, must
come at least 19 wait states later (the most that any MFMA result read needs
on gfx950: s_nop N counts N + 1, any other instruction 1).  The scan is
followed along the control flow and pinned first on small listings with
planted mistakes."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "burn_dragon_amd", "csrc")
NEED = 19
_AGPR = re.compile(r"\ba(\d+|\[\d+:\d+\])")


def scan(text, need=NEED):
    """From every MFMA, walk the control flow (fall-through, branch targets)
    until `need` wait states have passed or another MFMA comes; return
    (line, instruction, wait states) for each accumulator access met sooner,
    with the fewest wait states over the paths."""
    ins, labels = [], {}
    for n, raw in enumerate(text.splitlines(), 1):
        t = raw.split(";")[0].strip()
        if not t or t.startswith("."):
            if t.endswith(":"):
                labels[t[:-1]] = len(ins)
            continue
        if t.endswith(":"):
            labels[t[:-1]] = len(ins)
            continue
        ins.append((n, t))
    worst = {}
    for i, (_, t) in enumerate(ins):
        if not t.startswith("v_mfma"):
            continue
        stack, seen = [(i + 1, 0)], set()
        while stack:
            j, w = stack.pop()
            if w >= need or j >= len(ins) or (j, w) in seen:
                continue
            seen.add((j, w))
            n, u = ins[j]
            op = u.split()[0]
            if op.startswith("v_mfma"):
                continue  # its own walk covers what follows it
            if _AGPR.search(u[len(op):]):
                worst[(n, u)] = min(w, worst.get((n, u), need))
            if op == "s_endpgm":
                continue
            m = re.match(r"s_nop\s+(\d+)", u)
            w2 = w + (int(m.group(1)) + 1 if m else 1)
            target = u.split()[1] if op.startswith(("s_branch", "s_cbranch")) and len(u.split()) > 1 else None
            if target in labels:
                stack.append((labels[target], w2))
            if op != "s_branch":
                stack.append((j + 1, w2))
    return sorted((n, u, w) for (n, u), w in worst.items())


def test_scan_accepts_enough_wait_states():
    body = "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]\n" + "\ts_nop 7\n" * 3 + \
           "\tds_write_b32 v8, a0\n"
    assert scan(body) == []


def test_scan_flags_a_read_too_soon():
    body = "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]\n\ts_nop 7\n\tv_accvgpr_read_b32 v9, a2\n"
    assert [p[2] for p in scan(body)] == [8]


def test_scan_lets_mfma_chains_and_other_registers_pass():
    body = ("\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]\n"
            "\tv_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[8:11], a[4:7]\n"
            "\tds_read_b128 v[12:15], v16 offset:64 ; a comment naming a0\n"
            "\tv_add_u32_e32 v1, 4, v1\n")
    assert scan(body) == []


def test_scan_follows_branches():
    body = ("\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]\n"
            "\ts_branch .LBB0_2\n"
            ".LBB0_1:\n"
            "\tv_accvgpr_write_b32 a1, 0\n"      # not reached from the MFMA
            ".LBB0_2:\n"
            "\ts_cbranch_scc1 .LBB0_3\n"
            "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
            ".LBB0_3:\n"
            "\tds_write_b32 v8, a0\n")            # 2 wait states on the taken path
    assert [(p[1], p[2]) for p in scan(body)] == [("ds_write_b32 v8, a0", 2)]


def test_wide_gram_covers_its_mfma_hazards():
    hipcc = next((c for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc"))
                  if c and os.path.exists(c)), None)
    if hipcc is None:
        pytest.skip("hipcc not available")
    from burn_dragon_amd import build
    flags = [f for f in build.common_flags() if f != "-fPIC"]
    out = tempfile.mkdtemp(prefix="bdh_mfma_")
    try:
        dst = os.path.join(out, "wide_gram.s")
        r = subprocess.run([hipcc] + flags + ["--cuda-device-only", "-S", os.path.join(CSRC, "wide_gram.hip"),
                            "-o", dst], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        text = open(dst).read()
    finally:
        shutil.rmtree(out, ignore_errors=True)
    assert text.count("v_mfma_f32_16x16x32_bf16") >= 128  # the scan sees the step loops
    assert any(_AGPR.search(l) and "ds_write" in l for l in text.splitlines())  # and the epilogue's reads
    problems = scan(text)
    assert problems == [], "\n".join(f"line {n}: '{i}' after {w} wait states" for n, i, w in problems[:20])
