"""CPU model of the hand-over protocol of layer_x_roles_kernel (the C5 GEMM X
in wave roles, burn_dragon_amd/csrc/layer_bf16.hip): 4 MFMA waves, 4 DMA
waves and 8 store waves of one workgroup, a 3-slot LDS ring of K steps, per
wave progress counters (steps landed per DMA wave, steps read per MFMA
wave) and two workgroup barriers per tile.  Random interleavings of the
waves' operations must always finish (no deadlock, no barrier mismatch) and
never let an MFMA wave read a slot that a DMA wave has refilled with a
later step.  A planted mistake (one shared counter per group instead of
per-wave counters, which lets fast waves stand in for slow ones) must be
caught."""
import random

import pytest

MW, DW, SW, RING = 4, 4, 8, 3


def _programs(ntile, nk, shared_counters=False):
    J = ntile * nk
    progs = []
    for w in range(MW):
        ops = []
        for j in range(J):
            ops.append(("wait", "landed", j + 1))
            ops.append(("read", j % RING, j))
            ops.append(("done", "consumed", w, j + 1))
            if (j + 1) % nk == 0:
                ops += [("bar",), ("bar",)]  # G, then the staging writes, F
        progs.append(ops)
    for d in range(DW):
        ops, met = [], 0
        for j in range(J):
            if j >= RING:
                ops.append(("wait", "consumed", j - RING + 1))
            if met < ntile and j == (met + 1) * nk + 2:
                ops += [("bar",), ("bar",)]
                met += 1
            ops.append(("write", j % RING, j, d))
            if j > 0:
                ops.append(("done", "landed", d, j))  # vmcnt(2): step j - 1 landed
        ops.append(("done", "landed", d, J))
        while met < ntile:
            ops += [("bar",), ("bar",)]
            met += 1
        progs.append(ops)
    for _ in range(SW):
        progs.append([("bar",)] * (2 * ntile))
    return progs


def _run(ntile, nk, seed, shared_counters=False):
    """True if the waves finish with every read fresh; False on a deadlock;
    raises AssertionError on a stale read."""
    rnd = random.Random(seed)
    progs = _programs(ntile, nk)
    n = len(progs)
    pc = [0] * n
    per_wave = {"landed": [0] * DW, "consumed": [0] * MW}
    shared = {"landed": 0, "consumed": 0}
    slots = {}
    at_bar = set()

    def level(name):
        if shared_counters:
            return shared[name] // (DW if name == "landed" else MW)
        return min(per_wave[name])

    while True:
        live = [w for w in range(n) if pc[w] < len(progs[w])]
        if not live:
            return True
        if at_bar and at_bar == set(live):
            for w in at_bar:
                pc[w] += 1
            at_bar.clear()
            continue
        runnable = []
        for w in live:
            if w in at_bar:
                continue
            op = progs[w][pc[w]]
            if op[0] == "wait" and level(op[1]) < op[2]:
                continue
            runnable.append(w)
        if not runnable:
            return False
        w = rnd.choice(runnable)
        op = progs[w][pc[w]]
        if op[0] == "bar":
            at_bar.add(w)
            continue
        if op[0] == "done":
            per_wave[op[1]][op[2]] = op[3]
            shared[op[1]] += 1
        elif op[0] == "write":
            slots[(op[1], op[3])] = op[2]
        elif op[0] == "read":
            for d in range(DW):
                assert slots.get((op[1], d)) == op[2], ("stale slot", op, d)
        pc[w] += 1


@pytest.mark.parametrize("nk", [2, 3, 4, 6, 8])
@pytest.mark.parametrize("ntile", [1, 2, 3, 5])
def test_protocol_finishes_with_fresh_reads(ntile, nk):
    for seed in range(25):
        assert _run(ntile, nk, seed), f"deadlock: {ntile} tiles, {nk} steps, seed {seed}"


def test_model_catches_shared_counters():
    caught = False
    for seed in range(200):
        try:
            _run(3, 8, seed, shared_counters=True)
        except AssertionError:
            caught = True
            break
    assert caught
