"""CPU model of the hand-over protocol of prefill_roles_kernel (the one-interval
RoPE prefill in wave roles, burn_dragon_amd/csrc/roles_prefill.hip): 8 MFMA
waves and 4 producer waves of one workgroup, a 3-stage LDS ring of K steps,
an epilogue whose staging overlaps the ring, and per-wave progress counters
in LDS (steps written per producer, steps read per MFMA wave), no workgroup
barriers.  Gram producers load their raw rows into registers; state
producers fill per-producer raw slots by direct loads two steps ahead
(which land asynchronously, in issue order per wave) and read them one step
ahead.
A diagonal gram tile's MFMA waves 1 and 3 are inactive: they count steps as
read without reading.  Random interleavings must always finish (no deadlock)
and never let a wave read a stage that was already rewritten, nor let the
staging start while a direct load may still land or another wave still reads
the ring.  Planted mistakes (one shared counter per group; an epilogue that
does not wait for the producers' last direct loads) must be caught."""
import random

import pytest

MW, PW, RING = 8, 4, 3


def _programs(J, inactive, wait_tail=True, raw_slots=True):
    progs = []
    for w in range(MW):
        ops = []
        for j in range(J):
            ops.append(("wait", "landed", j + 1))
            if w not in inactive:
                ops.append(("read_slot", j % RING, j))
            ops.append(("done", "consumed", w, j + 1))
        if w not in inactive:
            ops.append(("wait", "consumed", J))
            if wait_tail:
                ops.append(("wait", "landed", J + 1))
            ops.append(("stage", w))
        progs.append(ops)
    for p in range(PW):
        if not raw_slots:
            # registers only: the loads never touch LDS
            ops = []
            for j in range(J):
                if j >= RING:
                    ops.append(("wait", "consumed", j - RING + 1))
                ops.append(("write_slot", j % RING, j, p))
                ops.append(("done", "landed", p, j + 1))
            ops.append(("done", "landed", p, J + 1))
            progs.append(ops)
            continue
        ops = [("dma", p, 0, 0), ("dma", p, 1, min(1, J - 1)),
               ("dma_wait", p, 0), ("read_raw", p, 0, 0)]
        for j in range(J):
            if j >= RING:
                ops.append(("wait", "consumed", j - RING + 1))
            # raw slot j % 2 was read during step j - 1 (or before the loop)
            ops.append(("dma", p, j % 2, min(j + 2, J - 1)))
            ops.append(("write_slot", j % RING, j, p))
            ops.append(("dma_wait", p, j + 1))        # vmcnt: step j + 1's loads landed
            ops.append(("read_raw", p, (j + 1) % 2, min(j + 1, J - 1)))
            ops.append(("done", "landed", p, j + 1))
        ops.append(("dma_wait_all", p))
        ops.append(("done", "landed", p, J + 1))
        progs.append(ops)
    return progs


GROUP = {"landed": PW, "consumed": MW}


def _run(J, inactive, seed, shared_counters=False, wait_tail=True, raw_slots=True):
    """True if the waves finish with every read fresh, False on a deadlock;
    AssertionError on a stale read or a load landing in the staging."""
    rnd = random.Random(seed)
    progs = _programs(J, inactive, wait_tail, raw_slots)
    n = len(progs)
    pc = [0] * n
    per_wave = {k: [0] * v for k, v in GROUP.items()}
    shared = {k: 0 for k in GROUP}
    slots = {}          # (ring slot, producer) -> step written
    raw = {}            # (producer, raw slot) -> step landed
    pending = [[] for _ in range(PW)]   # issued, not landed: (raw slot, step), oldest first
    issued = [0] * PW   # loads issued per producer
    landed_n = [0] * PW
    staged = False
    land_p = rnd.uniform(0.02, 0.5)

    def level(name):
        if shared_counters:
            return shared[name] // GROUP[name]
        return min(per_wave[name])

    def runnable(w):
        op = progs[w][pc[w]]
        if op[0] == "wait":
            return level(op[1]) >= op[2]
        if op[0] == "dma_wait":
            # one load per step, issued in step order: step j's is load j
            return landed_n[op[1]] >= op[2] + 1
        if op[0] == "dma_wait_all":
            return not pending[op[1]]
        return True

    while True:
        live = [w for w in range(n) if pc[w] < len(progs[w])]
        can_land = [p for p in range(PW) if pending[p]]
        if not live and not can_land:
            return True
        ready = [w for w in live if runnable(w)]
        if not ready and not can_land:
            return False
        # Loads land late in some schedules: a landing is picked with a
        # per-run probability from 2 % to 50 %.
        if can_land and (not ready or rnd.random() < land_p):
            kind, who = "land", rnd.choice(can_land)
        else:
            kind, who = "wave", rnd.choice(ready)
        if kind == "land":
            sl, step = pending[who].pop(0)
            assert not staged, ("a direct load landed in the staging", who, step)
            raw[(who, sl)] = step
            landed_n[who] += 1
            continue
        w = who
        op = progs[w][pc[w]]
        if op[0] == "done":
            per_wave[op[1]][op[2]] = op[3]
            shared[op[1]] += 1
        elif op[0] == "dma":
            pending[op[1]].append((op[2], op[3]))
            issued[op[1]] += 1
        elif op[0] == "read_raw":
            assert raw.get((op[1], op[2])) == op[3], ("stale raw slot", op)
        elif op[0] == "write_slot":
            assert not staged, ("stage written after the staging began", op)
            slots[(op[1], op[3])] = op[2]
        elif op[0] == "read_slot":
            assert not staged, ("ring read after the staging began", op)
            for p in range(PW):
                assert slots.get((op[1], p)) == op[2], ("stale ring slot", op, p)
        elif op[0] == "stage":
            staged = True
        pc[w] += 1


@pytest.mark.parametrize("J", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("inactive", [(), (1, 3)])
@pytest.mark.parametrize("raw_slots", [True, False])
def test_protocol_finishes_with_fresh_reads(J, inactive, raw_slots):
    for seed in range(40):
        assert _run(J, inactive, seed, raw_slots=raw_slots), f"deadlock: {J} steps, inactive {inactive}, seed {seed}"


def test_model_catches_shared_counters():
    caught = False
    for seed in range(400):
        try:
            _run(6, (), seed, shared_counters=True)
        except AssertionError:
            caught = True
            break
    assert caught


def test_model_catches_an_epilogue_before_the_last_loads():
    caught = False
    for seed in range(400):
        try:
            _run(4, (1, 3), seed, wait_tail=False)
        except AssertionError:
            caught = True
            break
    assert caught
