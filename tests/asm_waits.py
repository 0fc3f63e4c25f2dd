"""Checks the gfx950 assembly that hipcc writes for this package's kernels:
no instruction touches the destination registers of an LDS read before an
`s_waitcnt lgkmcnt` has covered that read.

The MFMA tiles issue their fragment reads (`ds_read_b128`) in inline
assembly and wait for them with `s_waitcnt lgkmcnt(N)` in later assembly
blocks tied to the fragment registers.  The compiler treats an assembly
output as ready at once, so a register copy it might place between the read
and the wait (a `v_mov`, an AGPR move) would read stale data.  This scan
reads each kernel's instructions and reports any instruction that reads a
register of an LDS read still in flight, or writes one (the read would land
over the new value later).

Model of the counter: LDS operations (`ds_*`) complete in issue order;
scalar memory operations (`s_load*`, `s_buffer_load*`, `s_memtime`, ...)
may complete in any order, so only `lgkmcnt(0)` retires them.  After
`s_waitcnt lgkmcnt(N)` an LDS read is complete when at least N LDS
operations were issued after it (on every path: the scan is a forward
dataflow over each kernel's basic blocks).

Used by tests/test_asm_waits.py; run directly as
`python tests/asm_waits.py file.s ...`.
"""
import re
import sys

_REG = re.compile(r"\b([va])(?:(\d+)\b|\[(\d+):(\d+)\])")
_WAIT = re.compile(r"lgkmcnt\((\d+)\)")
_FUNC = re.compile(r"^([A-Za-z_.][\w.$]*):")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        kind = m.group(1)
        if m.group(2) is not None:
            out.add((kind, int(m.group(2))))
        else:
            for r in range(int(m.group(3)), int(m.group(4)) + 1):
                out.add((kind, r))
    return out


def _is_smem(op):
    return op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_sendmsg",
                          "s_scratch_load", "s_dcache"))


def _parse(asm_text):
    """Functions as lists of (line no, label or None, op, operands, text)."""
    funcs, cur = {}, None
    for no, raw in enumerate(asm_text.splitlines(), 1):
        fm = _FUNC.match(raw)
        if fm:
            lab = fm.group(1)
            if not lab.startswith("."):
                cur = funcs.setdefault(lab, [])
                continue
            if cur is not None:
                cur.append((no, lab, None, "", ""))
            continue
        line = raw.split(";", 1)[0].strip()
        if cur is None or not line or line.startswith("."):
            continue
        op, _, operands = line.partition(" ")
        cur.append((no, None, op, operands.strip(), line))
    return funcs


def _blocks(insts):
    """Basic blocks: list of (label, [instructions], [successor indices])."""
    blocks, cur_label, body = [], None, []
    for it in insts:
        no, lab, op, operands, text = it
        if lab is not None:
            if body or cur_label is not None:
                blocks.append([cur_label, body])
            cur_label, body = lab, []
            continue
        body.append(it)
        if op.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc", "s_trap")):
            blocks.append([cur_label, body])
            cur_label, body = None, []
    if body or cur_label is not None:
        blocks.append([cur_label, body])
    index = {b[0]: i for i, b in enumerate(blocks) if b[0]}
    out = []
    for i, (lab, body) in enumerate(blocks):
        succ = []
        last = body[-1] if body else None
        op = last[2] if last else ""
        if op.startswith(("s_branch", "s_cbranch")):
            tgt = last[3].split(",")[0].strip()
            if tgt in index:
                succ.append(index[tgt])
        if not op.startswith(("s_branch", "s_endpgm", "s_setpc", "s_trap")) and i + 1 < len(blocks):
            succ.append(i + 1)
        out.append((lab, body, succ))
    return out


_CAP = 64


def _operands(op, operands):
    """(source registers, destination registers) of one instruction."""
    parts = [x.strip() for x in operands.split(",")] if operands else []
    all_src = ("store" in op or op.startswith("ds_write") or "_lds" in op
               or (op.startswith("ds_") and not op.startswith(("ds_read", "ds_load")) and "rtn" not in op))
    if all_src or not parts:
        return _regs(operands), set()
    return _regs(",".join(parts[1:])), _regs(parts[0])


def _transfer(state, body, report, writes):
    """state: {entry: [is_lds, dest regs, newer LDS ops (lower bound), line, text]}.
    Reports instructions that read (writes=False) or write (writes=True) a
    register of a read still in flight."""
    st = {k: list(v) for k, v in state.items()}
    for no, _, op, operands, text in body:
        if op == "s_waitcnt" or op.startswith("s_waitcnt_lgkmcnt"):
            if op.startswith("s_waitcnt_lgkmcnt"):
                n = int(operands.split(",")[-1].strip(), 0)
            else:
                m = _WAIT.search(text)
                if m is None:
                    continue
                n = int(m.group(1))
            st = {k: v for k, v in st.items() if not ((v[2] >= n) if v[0] else n == 0)}
            continue
        if report is not None:
            srcs, dsts = _operands(op, operands)
            regs = dsts if writes else srcs
            for v in st.values():
                if v[0] and v[1] & regs:
                    report.add((no, text, v[3], v[4]))
        if op.startswith(("ds_", "flat_")):
            for v in st.values():
                if v[0]:
                    v[2] = min(_CAP, v[2] + 1)
            dest = set()
            if op.startswith(("ds_read", "ds_load")) and "addtid" not in op:
                dest = _regs(operands.split(",")[0])
            st[no] = [True, dest, 0, no, text]
        elif _is_smem(op):
            st[no] = [False, set(), 0, no, text]
    return st


def _merge(a, b, must):
    """Union (a read in flight on some path) or, with must, intersection (in
    flight on every path); either keeps the fewest later LDS operations."""
    if must:
        return {k: [*v[:2], min(v[2], b[k][2]), *v[3:]] for k, v in a.items() if k in b}
    out = {k: list(v) for k, v in a.items()}
    for k, v in b.items():
        if k in out:
            out[k][2] = min(out[k][2], v[2])
        else:
            out[k] = list(v)
    return out


def _solve(blocks, must):
    ins = [None] * len(blocks)
    ins[0] = {}
    work = [0]
    while work:
        i = work.pop()
        out = _transfer(ins[i], blocks[i][1], None, False)
        for j in blocks[i][2]:
            new = out if ins[j] is None else _merge(ins[j], out, must)
            if ins[j] is None or _key(new) != _key(ins[j]):
                ins[j] = new
                work.append(j)
    return ins


def check(asm_text, name="<asm>"):
    """Returns a list of violation strings for one assembly file.  A forward
    dataflow over each function's blocks: an instruction that reads a
    register of an LDS read in flight on some path into it, or writes one in
    flight on every path (a write on some path only is what a loop-invariant
    branch taken one way in one half-step and the other way in the next
    produces in the step loops: infeasible, and common)."""
    problems = []
    for func, insts in _parse(asm_text).items():
        blocks = _blocks(insts)
        if not blocks:
            continue
        report = set()
        for must in (False, True):
            ins = _solve(blocks, must)
            for i, blk in enumerate(blocks):
                if ins[i] is not None:
                    _transfer(ins[i], blk[1], report, must)
        for no, text, rno, rtext in sorted(report):
            problems.append(f"{name}:{no}: {func}: '{text}' touches a register of the LDS read at "
                            f"line {rno} ('{rtext}') before its wait")
    return problems


def _key(state):
    return sorted((k, v[2]) for k, v in state.items())


if __name__ == "__main__":
    bad = []
    for path in sys.argv[1:]:
        bad += check(open(path).read(), path)
    print("\n".join(bad) if bad else "no LDS read used before its wait")
    sys.exit(1 if bad else 0)
