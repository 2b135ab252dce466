"""Pins of the oracle's chunk-pool policy (pool_assign): an independent brute-force simulation of
the rule on random and adversarial selection streams, and the invariants any correct pool keeps."""
import numpy as np
import pytest

import oracle


class BrutePool:
    """The policy restated over a list of [chunk, last_use] per slot (no tables)."""

    def __init__(self, P, initial):
        self.slots = [[-1, -1] for _ in range(P)]
        for j, c in enumerate(initial):
            self.slots[j] = [int(c), 0]
        self.t = 0

    def step(self, sel):
        self.t += 1
        where = {c: v for v, (c, _) in enumerate(self.slots) if c >= 0}
        hits = {v for c in sel if (v := where.get(int(c))) is not None}
        slot_list = [where.get(int(c), -1) for c in sel]
        for v in hits:
            self.slots[v][1] = self.t
        order = sorted((v for v in range(len(self.slots)) if v not in hits), key=lambda v: (self.slots[v][1], v))
        misses = [j for j, c in enumerate(sel) if int(c) not in where]
        victims = sorted(order[:len(misses)])
        for k, j in enumerate(misses):
            self.slots[victims[k]] = [int(sel[j]), self.t]
            slot_list[j] = victims[k]
        return slot_list, len(sel) - len(misses), [(int(sel[j]), victims[k]) for k, j in enumerate(misses)]


def _tables(rows, chunks, P, initial):
    slot_of = np.full((rows, chunks), -1, np.int32)
    slot_chunk = np.full((rows, P), -1, np.int32)
    slot_used = np.full((rows, P), -1, np.int32)
    S = initial.shape[1]
    for r in range(rows):
        slot_of[r, initial[r]] = np.arange(S)
        slot_chunk[r, :S] = initial[r]
        slot_used[r, :S] = 0
    return slot_of, slot_chunk, slot_used, np.zeros(rows, np.int32)


def _stream(rng, rows, chunks, S, steps, drift):
    """Selections that keep a fraction of the previous step's chunks (drift = fraction replaced)."""
    cur = np.stack([rng.permutation(chunks)[:S] for _ in range(rows)])
    out = [cur.copy()]
    for _ in range(steps):
        nxt = cur.copy()
        for r in range(rows):
            k = max(1, int(drift * S))
            pos = rng.permutation(S)[:k]
            fresh = rng.permutation(np.setdiff1d(np.arange(chunks), nxt[r]))[:k]
            nxt[r, pos] = fresh
            nxt[r] = rng.permutation(nxt[r])
        cur = nxt
        out.append(cur.copy())
    return out


@pytest.mark.parametrize("S,P,drift", [(16, 16, 0.3), (16, 24, 0.3), (16, 64, 0.5), (32, 40, 1.0), (8, 200, 0.2)])
def test_pool_assign_matches_brute_force(S, P, drift):
    rng = np.random.default_rng(S * 1000 + P)
    rows, chunks, steps = 4, 300, 12
    stream = _stream(rng, rows, chunks, S, steps, drift)
    tables = _tables(rows, chunks, P, stream[0])
    brutes = [BrutePool(P, stream[0][r]) for r in range(rows)]
    for t in range(1, steps + 1):
        before = tables[1].copy()
        slot_list, miss_ids, miss_slot, cnts = oracle.pool_assign(stream[t], *tables)
        slot_of, slot_chunk, slot_used, clock = tables
        for r in range(rows):
            want_list, want_hits, want_misses = brutes[r].step(stream[t][r])
            assert slot_list[r].tolist() == want_list, (t, r)
            assert int(cnts[r]) == want_hits
            got_misses = list(zip(miss_ids[r, cnts[r]:].tolist(), miss_slot[r, cnts[r]:].tolist()))
            assert got_misses == want_misses
            # invariants: every selected chunk resident at its listed slot; tables consistent;
            # hits = selected chunks resident before the step
            assert all(slot_chunk[r, slot_list[r, j]] == stream[t][r, j] for j in range(S))
            for v in range(P):
                if slot_chunk[r, v] >= 0:
                    assert slot_of[r, slot_chunk[r, v]] == v
            assert int((slot_of[r] >= 0).sum()) == int((slot_chunk[r] >= 0).sum())
            assert want_hits == len(set(stream[t][r].tolist()) & set(before[r][before[r] >= 0].tolist()))
            assert int(clock[r]) == t
        if P == S:  # the pool holds exactly the selection, as the reference's buffer does
            for r in range(rows):
                assert set(slot_chunk[r].tolist()) == set(stream[t][r].tolist())


def test_pool_evicts_least_recently_used():
    """P = S + 2: chunks selected once and then dropped leave in the order they were last used."""
    S, P, chunks = 4, 6, 50
    init = np.array([[0, 1, 2, 3]])
    tables = _tables(1, chunks, P, init)
    oracle.pool_assign(np.array([[0, 1, 2, 4]]), *tables)   # 3 last used at 0; 4 takes empty slot 4
    oracle.pool_assign(np.array([[0, 1, 5, 6]]), *tables)   # 5 -> empty slot 5; 6 evicts chunk 3 (oldest)
    slot_of, slot_chunk, slot_used, _ = tables
    assert slot_of[0, 3] == -1 and slot_of[0, 2] >= 0 and slot_of[0, 4] >= 0
    oracle.pool_assign(np.array([[0, 1, 7, 8]]), *tables)   # evict 2 (used at 1) and 4 (used at 1): lowest slots
    assert slot_of[0, 2] == -1 and slot_of[0, 4] == -1 and slot_of[0, 5] >= 0 and slot_of[0, 6] >= 0
