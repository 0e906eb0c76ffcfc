"""Independent Python model of the reference's wave scheduler and linear-scan
planner (B/src/runtime/lancius_scheduler.c:12-59,
B/src/runtime/lancius_memory_planner.c:33-182), used only by tests.

`keep_offsets=False` reproduces the reference exactly, including its active
list storing intervals whose offset field was never written (:140, :167), so
freed blocks re-enter the free list at offset 0; `keep_offsets=True` is the
corrected scan that liblancius_graph implements.
"""
from __future__ import annotations


def levelize(nodes: list[tuple[int, list[int]]]) -> list[list[int]]:
    """nodes: (id, input ids) in graph order -> waves of ids."""
    done: set[int] = set()
    waves = []
    while len(done) < len(nodes):
        wave = [i for i, ins in nodes if i not in done and all(j in done for j in ins)]
        if not wave:
            break
        waves.append(wave)
        done.update(wave)
    return waves


def plan(nodes, ops, nbytes, waves, keep_offsets: bool, input_ops=(1, 2)):
    """nodes: [(id, input ids)] in graph order; ops/nbytes by position."""
    ids = max(i for i, _ in nodes) + 1
    birth = [None] * ids
    death = [0] * ids
    read = [False] * ids
    pos = {i: k for k, (i, _) in enumerate(nodes)}
    for _, ins in nodes:
        for j in ins:
            read[j] = True
    inputs_of = dict(nodes)
    for w, wave in enumerate(waves):
        for i in wave:
            if ops[pos[i]] not in input_ops:
                birth[i] = w
            for j in inputs_of[i]:
                if birth[j] is not None and w > death[j]:
                    death[j] = w
    iv = []
    for i, _ in nodes:
        if birth[i] is None:
            continue
        d = max(death[i], birth[i])
        if not read[i]:
            d = len(waves)
        iv.append({"id": i, "birth": birth[i], "death": d, "size": (nbytes[pos[i]] + 31) // 32 * 32, "offset": 0})
    iv.sort(key=lambda t: t["birth"])  # stable, like the insertion sort
    free = [[0, 1 << 64]]  # front = head of the LIFO list
    active = []
    offsets, peak = {}, 0
    for cur in iv:
        keep = []
        for a in active:
            if a["death"] < cur["birth"]:
                free.insert(0, [a["offset"] if keep_offsets else 0, a["size"]])
            else:
                keep.append(a)
        active = keep
        for k, blk in enumerate(free):
            if blk[1] >= cur["size"]:
                off = blk[0]
                if blk[1] > cur["size"]:
                    blk[0] += cur["size"]
                    blk[1] -= cur["size"]
                else:
                    free.pop(k)
                break
        offsets[cur["id"]] = off
        peak = max(peak, off + cur["size"])
        rec = dict(cur)
        if keep_offsets:
            rec["offset"] = off
        active.append(rec)
    return peak, offsets, iv


def overlaps(iv, offsets) -> list[tuple[int, int]]:
    """Pairs of simultaneously live intervals whose blocks intersect."""
    bad = []
    for a in range(len(iv)):
        for b in range(a + 1, len(iv)):
            x, y = iv[a], iv[b]
            if x["birth"] > y["death"] or y["birth"] > x["death"]:
                continue
            ox, oy = offsets[x["id"]], offsets[y["id"]]
            if ox < oy + y["size"] and oy < ox + x["size"]:
                bad.append((x["id"], y["id"]))
    return bad
