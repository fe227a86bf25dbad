"""CPU model of the ring prefill kernel's ping-pong schedule (kv_prefill_ring_kernel with
FDLLM_PREFILL_PIPE, csrc/block_attn.hip): each of the 8 waves' programs is rebuilt from
the kernel's control flow (prologue, the two groups' steps, epilogue) as a list of
vector-memory issues, count waits, workgroup barriers and LDS reads, and the guarantees
the kernel relies on are checked for every tile count from 0 to 13, for the form that
loads the query rows first (no cache write) and for the form with the cache write:

  * both groups pass the same number of barrier instances (no wave waits for ever);
  * a tile's slot is read only after a barrier that every wave passes after its own wait
    covering that tile (its DMA writes into LDS are then complete in every wave's view);
  * a slot is written (a tile, or the zeros of a tile past the range) only after a
    barrier that every wave passes after its last read of the slot's previous contents
    (a tile, or the query rows held in ring slots 2 and 3);
  * a wave reads its query rows only after its own wait covering their loads;
  * nothing is outstanding when the waves leave (the final vmcnt(0)).

Waits follow the hardware rule: s_waitcnt vmcnt(n) returns once at most n of the wave's
vector memory operations (loads, DMA loads and stores alike) are outstanding, and they
complete in issue order. A wave's reads are taken to include every tile in its range
(the kernel skips the math of a tile past the key limits of a wave's rows: fewer reads).
"""
import pytest

WAVES = 8
LOADS_PER_TILE = 4  # K and V, two 1 KB loads each per wave
Q_LOADS = 8         # the query rows: 32 rows of 256 B per wave
OWN_LOADS = 4       # the cache-write form: a thread's new K / V rows (loads, then stores)
OWN_STORES = 4


def wave_program(wave: int, ntiles: int, early_q: bool, fused: bool) -> list:
    """Program of one wave in the kernel's order (the ping-pong form)."""
    grp = wave >> 2
    prog = []

    def issue(tile):
        prog.append(("issue", tile, tile % 4, LOADS_PER_TILE))

    # prologue
    if early_q:
        prog.append(("issue_q", Q_LOADS))
    if fused:
        prog.append(("mem", "own_loads", OWN_LOADS))
    if ntiles > 0:
        issue(0)
        issue(1)
    if early_q:
        prog.append(("wait", 4 if ntiles > 0 else 0))
        prog.append(("barrier",))
        prog.append(("read_q",))
    else:
        prog.append(("mem", "q_loads", 4))  # the query fragments, into registers
        prog.append(("wait", 0))
    if fused:
        prog.append(("mem", "own_stores", OWN_STORES))
    if ntiles == 0:
        prog.append(("wait", 0))
        return prog
    # pipelined loop (prun)
    if grp == 1:
        prog.append(("barrier",))  # instance 0
        issue(2)
    prev_active = False
    steps = (ntiles + 3) // 4 * 4
    for j in range(steps):
        if grp == 0:
            if j >= (1 if early_q else 2):
                prog.append(("wait", 4))
            prog.append(("barrier",))  # instance j
            issue(j + 2)
        if prev_active:
            prog.append(("read", j - 1, (j - 1) % 4, "V"))
        act = j < ntiles
        if act:
            prog.append(("read", j, j % 4, "K"))
        if grp == 1:
            if j >= (0 if early_q else 1):
                prog.append(("wait", 4))
            prog.append(("barrier",))  # instance j + 1
            issue(j + 3)
        prev_active = act
    if grp == 0:
        prog.append(("barrier",))  # the last instance
    if prev_active:
        prog.append(("read", steps - 1, (steps - 1) % 4, "V"))
    prog.append(("wait", 0))
    return prog


def analyse(ntiles: int, early_q: bool, fused: bool):
    """Per wave: the barrier count at each event, when each tile / the query rows were
    covered by a wait, and the reads and writes of each slot."""
    info = []
    for w in range(WAVES):
        prog = wave_program(w, ntiles, early_q, fused)
        nbar = 0
        outstanding = []  # (kind, tile) per vector memory operation, oldest first
        covered = {}      # tile or "q" -> barrier count at the wait that completed it
        reads, writes, q_read_ok = [], [], True
        for ev in prog:
            kind = ev[0]
            if kind == "barrier":
                nbar += 1
            elif kind == "issue":
                _, tile, slot, n = ev
                writes.append((tile, slot, nbar))
                outstanding += [("tile", tile)] * n
            elif kind == "issue_q":
                writes.append(("q", 2, nbar))
                writes.append(("q", 3, nbar))
                outstanding += [("q", None)] * ev[1]
            elif kind == "mem":
                outstanding += [(ev[1], None)] * ev[2]
            elif kind == "wait":
                keep = ev[1]
                done, outstanding = outstanding[:len(outstanding) - keep], outstanding[len(outstanding) - keep:]
                for k, tile in done:
                    key = tile if k == "tile" else ("q" if k == "q" else None)
                    if key is not None and key not in covered:
                        covered[key] = nbar
                # a tile is complete only when none of its loads is still outstanding
                for k, tile in outstanding:
                    key = tile if k == "tile" else ("q" if k == "q" else None)
                    covered.pop(key, None)
            elif kind == "read":
                _, tile, slot, part = ev
                reads.append((tile, slot, part, nbar))
            elif kind == "read_q":
                reads.append(("q", 2, "Q", nbar))
                reads.append(("q", 3, "Q", nbar))
                q_read_ok = "q" in covered
        info.append(dict(nbar=nbar, covered=covered, reads=reads, writes=writes, q_read_ok=q_read_ok,
                         left=len(outstanding)))
    return info


CASES = [(n, eq, fu) for n in range(14) for eq, fu in ((True, False), (False, False), (False, True))]


@pytest.mark.parametrize("ntiles,early_q,fused", CASES)
def test_ring_schedule(ntiles, early_q, fused):
    info = analyse(ntiles, early_q, fused)
    # the same number of barrier instances in every wave
    assert len({i["nbar"] for i in info}) == 1, [i["nbar"] for i in info]
    for i in info:
        assert i["left"] == 0  # nothing outstanding at exit
        assert i["q_read_ok"]  # own query rows waited for before they are read
    # RAW: every read of a tile comes after a barrier every wave passes after its wait
    for w, i in enumerate(info):
        for tile, slot, part, nbar in i["reads"]:
            if tile == "q":
                continue  # a wave reads only its own query rows, covered by its own wait
            for v, j in enumerate(info):
                assert tile in j["covered"], (w, v, tile, "never waited for")
                assert j["covered"][tile] < nbar, (w, v, tile, j["covered"][tile], nbar)
    # WAR: a write into a slot comes after a barrier every wave passes after its last read
    # of the slot's previous contents
    for w, i in enumerate(info):
        for tile, slot, nbar_w in i["writes"]:
            for v, j in enumerate(info):
                for rtile, rslot, part, nbar_r in j["reads"]:
                    if rslot != slot or rtile == tile:
                        continue
                    # previous contents: a read of another tile (or of the query rows) of this
                    # slot that comes earlier in the slot's life than this write
                    earlier = rtile == "q" or (tile != "q" and rtile < tile)
                    if earlier:
                        assert nbar_r < nbar_w, (w, v, slot, tile, rtile, nbar_r, nbar_w)


def test_planted_mistake_is_caught():
    """The model catches a wait moved one step too late: without grp0's wait at step 1 in
    the query-first form, tile 1 could be read before it has landed."""
    global wave_program
    saved = wave_program

    def broken(wave, ntiles, early_q, fused):
        prog = saved(wave, ntiles, early_q, fused)
        # drop the first count wait of group 0 inside the loop
        for k, ev in enumerate(prog):
            if ev == ("wait", 4) and any(e == ("barrier",) for e in prog[:k]) and (wave >> 2) == 0:
                return prog[:k] + prog[k + 1:]
        return prog
    wave_program = broken
    try:
        with pytest.raises(AssertionError):
            test_ring_schedule(5, True, False)
    finally:
        wave_program = saved
