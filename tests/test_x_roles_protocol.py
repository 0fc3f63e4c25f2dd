"""CPU model of the hand-over protocol of layer_x_roles_kernel (the C5 GEMM X
in wave roles, burn_dragon_amd/csrc/layer_bf16.hip): 4 MFMA waves, 4 DMA
waves and 8 store waves of one workgroup, a 3-slot LDS ring of K steps, an
f32 staging tile, and per-wave progress counters in LDS (steps landed per
DMA wave, steps read per MFMA wave, tiles staged per MFMA wave, tiles read
from staging per store wave), no workgroup barriers.  Random interleavings
of the waves' operations must always finish (no deadlock) and never let a
wave read a ring slot or a staging part that another wave has already
refilled with later data.  A planted mistake (one shared counter per group
instead of per-wave counters, which lets fast waves stand in for slow ones)
must be caught."""
import random

import pytest

MW, DW, SW, RING = 4, 4, 8, 3


def _programs(ntile, nk):
    J = ntile * nk
    progs = []
    for w in range(MW):
        ops = []
        for j in range(J):
            ops.append(("wait", "landed", j + 1))
            ops.append(("read_slot", j % RING, j))
            ops.append(("done", "consumed", w, j + 1))
            if (j + 1) % nk == 0:
                i = j // nk
                ops.append(("wait", "freed", i))          # store waves have read tile i - 1
                ops.append(("stage", w, i))
                ops.append(("done", "staged", w, i + 1))
        progs.append(ops)
    for d in range(DW):
        ops = []
        for j in range(J):
            if j >= RING:
                ops.append(("wait", "consumed", j - RING + 1))
            ops.append(("write_slot", j % RING, j, d))
            if j > 0:
                ops.append(("done", "landed", d, j))      # vmcnt(2): step j - 1 landed
        ops.append(("done", "landed", d, J))
        progs.append(ops)
    for s in range(SW):
        ops = []
        for i in range(ntile):
            ops.append(("wait", "staged", i + 1))
            ops.append(("read_stage", i))
            ops.append(("done", "freed", s, i + 1))
        progs.append(ops)
    return progs


GROUP = {"landed": DW, "consumed": MW, "staged": MW, "freed": SW}


def _run(ntile, nk, seed, shared_counters=False):
    """True if the waves finish with every read fresh, False on a deadlock;
    AssertionError on a stale read."""
    rnd = random.Random(seed)
    progs = _programs(ntile, nk)
    n = len(progs)
    pc = [0] * n
    per_wave = {k: [0] * v for k, v in GROUP.items()}
    shared = {k: 0 for k in GROUP}
    slots, staging = {}, {}

    def level(name):
        if shared_counters:
            return shared[name] // GROUP[name]
        return min(per_wave[name])

    while True:
        live = [w for w in range(n) if pc[w] < len(progs[w])]
        if not live:
            return True
        runnable = [w for w in live
                    if not (progs[w][pc[w]][0] == "wait" and level(progs[w][pc[w]][1]) < progs[w][pc[w]][2])]
        if not runnable:
            return False
        w = rnd.choice(runnable)
        op = progs[w][pc[w]]
        if op[0] == "done":
            per_wave[op[1]][op[2]] = op[3]
            shared[op[1]] += 1
        elif op[0] == "write_slot":
            slots[(op[1], op[3])] = op[2]
        elif op[0] == "read_slot":
            for d in range(DW):
                assert slots.get((op[1], d)) == op[2], ("stale ring slot", op, d)
        elif op[0] == "stage":
            staging[op[1]] = op[2]
        elif op[0] == "read_stage":
            for m in range(MW):
                assert staging.get(m) == op[1], ("stale staging", op, m)
        pc[w] += 1


@pytest.mark.parametrize("nk", [2, 3, 4, 6, 8])
@pytest.mark.parametrize("ntile", [1, 2, 3, 5])
def test_protocol_finishes_with_fresh_reads(ntile, nk):
    for seed in range(25):
        assert _run(ntile, nk, seed), f"deadlock: {ntile} tiles, {nk} steps, seed {seed}"


def test_model_catches_shared_counters():
    caught = False
    for seed in range(300):
        try:
            _run(3, 8, seed, shared_counters=True)
        except AssertionError:
            caught = True
            break
    assert caught
