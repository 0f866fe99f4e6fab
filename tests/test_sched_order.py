"""The one-launch schedule's item order (mi355moe_sched_item, the same function the kernel evaluates per ticket),
checked on the host for every shape the GPU schedule tests run and a range of lags: every tile exactly once, in
bounds, nothing past the last item, every down item after all gate/up items of its segment (so a down item waits
only for tickets that running workgroups hold), and an event simulation of 256 workgroups taking tickets in order
that always finishes. The expected order is built independently as a list (lead, rounds, tail:
code/fork/kernels/moe_e4m3.cu:867-872, 931-959). No GPU needed."""
from __future__ import annotations

import heapq
import random

import pytest


def _expected(ns: int, lag: int, ncg: int, ncd: int) -> list[tuple[int, int, int]]:
    L = ns if lag <= 0 or lag > ns else lag
    items = [(0, s, b) for s in range(L) for b in range(ncg)]
    for r in range(ns - L):
        items += [(0, L + r, b) for b in range(ncg)]
        items += [(1, r, b) for b in range(ncd)]
    items += [(1, s, b) for s in range(ns - L, ns) for b in range(ncd)]
    return items


def _library_order(ns, lag, ncg, ncd, extra=300):
    from mi355moe import ops
    return [ops.sched_item(t, ns, lag, ncg, ncd) for t in range(ns * (ncg + ncd) + extra)]


# (segments upper bound, intermediate, hidden) of the GPU schedule tests: S_cap = min(P, n) + ceil(P / 256) for
# n experts, T tokens, top-k min(8, n); and the live segment counts below it that routing can produce
def _gpu_shapes():
    out = []
    for n, K, N, T in [(16, 1024, 512, 700), (64, 1024, 512, 4096), (4, 1024, 256, 20), (16, 1024, 512, 100),
                       (288, 4096, 1024, 8192), (32, 1024, 512, 1500)]:
        P = T * min(8, n)
        S_cap = min(P, n) + (P + 255) // 256
        out.append((S_cap, N // 128, K // 256))
    return out


@pytest.mark.parametrize("S_cap,ncg,ncd", _gpu_shapes())
def test_item_order_matches_independent_construction(S_cap, ncg, ncd):
    rnd = random.Random(S_cap)
    counts = sorted({1, 2, min(3, S_cap), S_cap - 1, S_cap, rnd.randint(1, S_cap)} - {0})
    for ns in counts:
        for lag in sorted({0, 1, 2, 12, 48, ns - 1, ns, ns + 5} - {-1}):
            want = _expected(ns, lag, ncg, ncd)
            got = _library_order(ns, lag, ncg, ncd)
            assert got[:len(want)] == want, (ns, lag)
            assert all(k == -1 for k, _, _ in got[len(want):]), (ns, lag)


@pytest.mark.parametrize("S_cap,ncg,ncd", _gpu_shapes())
def test_every_tile_once_and_down_after_its_gateup(S_cap, ncg, ncd):
    for ns in sorted({1, S_cap // 2, S_cap} - {0}):
        for lag in (0, 1, 12, 48):
            got = _library_order(ns, lag, ncg, ncd, extra=0)
            assert sorted(got) == sorted([(0, s, b) for s in range(ns) for b in range(ncg)] +
                                         [(1, s, b) for s in range(ns) for b in range(ncd)])
            last_gu = {}
            for t, (k, s, b) in enumerate(got):
                assert 0 <= s < ns and 0 <= b < (ncg if k == 0 else ncd)
                if k == 0:
                    last_gu[s] = t
                else:
                    assert s in last_gu and last_gu[s] < t and sum(
                        1 for k2, s2, _ in got[:t] if k2 == 0 and s2 == s) == ncg


def _simulate(ns, lag, ncg, ncd, workers, seed):
    """Workers take tickets in order as they finish; a gate/up item runs 3-4 units, a down item waits for its
    segment's gate/up items, then runs 1 unit. Returns the finish time (fails if a wait could never end)."""
    rnd = random.Random(seed)
    total = ns * (ncg + ncd)
    from mi355moe import ops
    gu_end = [[] for _ in range(ns)]
    ev = [(0.0, w) for w in range(workers)]
    heapq.heapify(ev)
    nxt, end = 0, 0.0
    while ev:
        now, w = heapq.heappop(ev)
        k, s, b = ops.sched_item(nxt, ns, lag, ncg, ncd) if nxt < total + workers else (-1, 0, 0)
        nxt += 1
        if k < 0:
            end = max(end, now)
            continue
        if k == 0:
            fin = now + 3.0 + rnd.random()
            gu_end[s].append(fin)
        else:
            assert len(gu_end[s]) == ncg, "a down item was taken before its segment's gate/up items were"
            fin = max(now, max(gu_end[s])) + 1.0
        heapq.heappush(ev, (fin, w))
    assert nxt >= total
    return end


@pytest.mark.parametrize("lag", [0, 1, 12, 48])
def test_simulated_schedule_finishes(lag):
    for ns, ncg, ncd, workers in [(288, 8, 16, 256), (41, 4, 4, 256), (3, 2, 4, 256), (64, 4, 4, 8)]:
        end = _simulate(ns, lag, ncg, ncd, workers, seed=ns + lag)
        assert end > 0


def test_query_rejects_bad_arguments():
    import ctypes

    from mi355moe import _lib
    L = _lib.lib()
    k, s, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert L.mi355moe_sched_item(0, 4, 0, 0, 4, ctypes.byref(k), ctypes.byref(s), ctypes.byref(b)) != 0
    assert L.mi355moe_sched_item(0, 4, -1, 8, 4, ctypes.byref(k), ctypes.byref(s), ctypes.byref(b)) != 0
    assert L.mi355moe_sched_item(0, 4, 0, 8, 4, None, ctypes.byref(s), ctypes.byref(b)) != 0
    assert L.mi355moe_sched_item(-1, 4, 0, 8, 4, ctypes.byref(k), ctypes.byref(s), ctypes.byref(b)) == 0
    assert k.value == -1
    assert L.mi355moe_sched_item(5, 0, 0, 8, 4, ctypes.byref(k), ctypes.byref(s), ctypes.byref(b)) == 0
    assert k.value == -1


QUEUES, QSTRIDE = 8, 32                       # the kernel's ticket queues and their word stride
HEAD = QUEUES * QSTRIDE + QSTRIDE             # queue counters, the give-up word, then one count per segment


@pytest.mark.parametrize("parts", [1, 2, 4])
@pytest.mark.parametrize("S_cap,ncg,ncd", _gpu_shapes())
def test_queue_and_count_indexing_in_bounds(S_cap, ncg, ncd, parts):
    """The kernel's indexing, emulated on the host for every shape of the GPU tests and every tile kind (1, 2 or 4
    parts per segment): segment s of a call with ns live segments goes to queue s % 8 as its unit s // 8, a queue's
    units are (segment, part) pairs with every first part first; every ticket a queue hands out names a segment below
    ns and a part below `parts`, every word the kernel touches (queue counter, give-up word, the unit's count
    PF_SCHED_HEAD + s * parts + part) lies inside the carved PF_SCHED_HEAD + 4 S_cap words, and every (segment, part,
    tile) is taken exactly once over the eight queues."""
    words = HEAD + 4 * S_cap
    for ns in sorted({1, 2, 7, 8, 9, S_cap // 2, S_cap} - {0}):
        if ns > S_cap:
            continue
        seen = []
        for q in range(QUEUES):
            assert q * QSTRIDE < HEAD - QSTRIDE and QUEUES * QSTRIDE < HEAD     # counter and give-up word
            nq = (ns - q + QUEUES - 1) // QUEUES if ns > q else 0
            if nq == 0:
                continue
            for t in range(nq * parts * (ncg + ncd) + 4):
                k, u, b = _library_order_one(t, nq * parts, ncg, ncd)
                if k < 0:
                    assert t >= nq * parts * (ncg + ncd)
                    continue
                part, j = divmod(u, nq)
                s = q + QUEUES * j
                assert 0 <= s < ns <= S_cap and 0 <= part < parts and HEAD + s * parts + part < words
                seen.append((k, s, part, b))
        assert sorted(seen) == sorted([(0, s, p, b) for s in range(ns) for p in range(parts) for b in range(ncg)] +
                                      [(1, s, p, b) for s in range(ns) for p in range(parts) for b in range(ncd)])


def _library_order_one(t, nq, ncg, ncd):
    from mi355moe import ops
    return ops.sched_item(t, nq, 0, ncg, ncd)
