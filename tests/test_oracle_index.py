"""Pins for the oracle's index/copy functions (reorder, chunk copies, top-k) on the CPU."""
import numpy as np
import pytest
import torch

import oracle
from tests.golden import make_golden

GOLDEN = make_golden.HERE


def kat():
    return np.load(GOLDEN / "reorder_kat.npz")


def test_kat_inputs_regenerate():
    # The committed inputs are exactly what the reference's seeded generator produces.
    keys, query = make_golden.kat_inputs()
    d = kat()
    assert np.array_equal(keys, d["orig_keys"].astype(np.int64))
    assert np.array_equal(query, d["query_keys"].astype(np.int64))
    assert (d["expected_cnts"] == 154).all()


def test_reorder_matches_reference_kat():
    d = kat()
    ids, offs, cnts = oracle.reorder(d["orig_keys"].astype(np.int64), d["query_keys"].astype(np.int64))
    assert np.array_equal(ids, d["expected_keys"].astype(np.int64))
    assert np.array_equal(offs, d["expected_offsets"].astype(np.int32))
    assert np.array_equal(cnts, d["expected_cnts"].astype(np.int32))


def brute_reorder(old, new):
    """Rule stated from the slots' side: walk old slots in order, keep those whose id is selected."""
    newset = set(int(x) for x in new)
    hit_slots = [j for j in range(len(old)) if old[j] != -1 and int(old[j]) in newset]
    oldset = set(int(x) for x in old if x != -1)
    misses = sorted(x for x in newset if x not in oldset)
    ids = [int(old[j]) for j in hit_slots] + misses
    offs = hit_slots + misses
    return ids, offs, len(hit_slots)


@pytest.mark.parametrize("S", [1, 2, 5, 16, 64])
def test_reorder_brute_force_unsorted(S):
    rng = np.random.default_rng(S)
    rows = 40
    old = np.stack([rng.permutation(3 * S)[:S] for _ in range(rows)]).astype(np.int64)
    old[rng.random(old.shape) < 0.1] = -1  # empty slots never hit
    new = np.stack([rng.permutation(3 * S)[:S] for _ in range(rows)]).astype(np.int64)
    ids, offs, cnts = oracle.reorder(old, new)
    for r in range(rows):
        bi, bo, bc = brute_reorder(old[r], new[r])
        assert cnts[r] == bc
        assert ids[r].tolist() == bi
        assert offs[r].tolist() == bo


def test_reorder_special_cases():
    old = np.array([[5, 3, 9, 1]], dtype=np.int64)
    ids, offs, cnts = oracle.reorder(old, np.array([[9, 1, 5, 3]]))
    assert cnts[0] == 4 and offs[0].tolist() == [0, 1, 2, 3] and ids[0].tolist() == [5, 3, 9, 1]
    ids, offs, cnts = oracle.reorder(old, np.array([[8, 2, 7, 4]]))
    assert cnts[0] == 0 and ids[0].tolist() == [2, 4, 7, 8] and offs[0].tolist() == [2, 4, 7, 8]


def test_reorder_offsets_are_a_forward_compaction():
    # offsets ascending and offsets[i] >= i for the hit part: the in-place copy is safe.
    rng = np.random.default_rng(7)
    old = np.stack([rng.permutation(1000)[:256] for _ in range(32)]).astype(np.int64)
    new = np.stack([rng.permutation(1000)[:256] for _ in range(32)]).astype(np.int64)
    _, offs, cnts = oracle.reorder(old, new)
    for r in range(32):
        h = offs[r, :cnts[r]]
        assert (np.diff(h) > 0).all() and (h >= np.arange(cnts[r])).all()


def coded(rows, n, E, tag):
    """Chunks whose int16 words name (tag, row, chunk, word) so any misplaced copy is visible."""
    r = np.arange(rows)[:, None, None]
    c = np.arange(n)[None, :, None]
    w = np.arange(E)[None, None, :]
    return ((tag * 7919 + r * 1543 + c * 131 + w) % 65521 - 32760).astype(np.int16)


def test_cached_gather_copy_closed_form():
    rows, S, E, nchunks = 6, 32, 64, 200
    rng = np.random.default_rng(3)
    host = coded(rows, nchunks, E, 1)
    old = np.stack([rng.permutation(nchunks)[:S] for _ in range(rows)]).astype(np.int64)
    new = np.stack([rng.permutation(nchunks)[:S] for _ in range(rows)]).astype(np.int64)
    dev = np.stack([host[r, old[r]] for r in range(rows)])  # consistent cache: slot holds its chunk
    ids, offs, cnts = oracle.reorder(old, new)
    out = oracle.cached_gather_copy(host, dev, offs, cnts)
    # After the refresh every slot holds exactly the host chunk of its new id.
    for r in range(rows):
        assert np.array_equal(out[r], host[r, ids[r]])
    comp = oracle.compact_hits(dev, offs, cnts)
    for r in range(rows):
        c = cnts[r]
        assert np.array_equal(comp[r, :c], host[r, ids[r, :c]])
        assert np.array_equal(comp[r, c:], dev[r, c:])
    plain = oracle.gather_copy_plain(host, new)
    for r in range(rows):
        for i in range(S):
            assert np.array_equal(plain[r, i], host[r, new[r, i]])


def test_topk_total_order_vs_torch_tie_aware():
    g = torch.Generator().manual_seed(0)
    x = torch.softmax(torch.randn(64, 3000, generator=g), dim=-1).to(torch.bfloat16)
    k = 256
    ours = oracle.topk_total_order(x, k)
    ref = torch.topk(x.float(), k, dim=-1).indices
    for r in range(x.shape[0]):
        vals = x[r].float()
        kth = vals[ours[r]].min()
        assert torch.equal(vals[ours[r]].sort(descending=True).values, vals[ref[r]].sort(descending=True).values)
        assert set((vals > kth).nonzero().flatten().tolist()) <= set(ours[r].tolist())
        eq_ours = sorted(i for i in ours[r].tolist() if vals[i] == kth)
        eq_all = (vals == kth).nonzero().flatten().tolist()
        assert eq_ours == eq_all[:len(eq_ours)]  # lowest indices win ties


def test_topk_brute_force_small():
    rng = np.random.default_rng(11)
    for _ in range(50):
        n = int(rng.integers(1, 40))
        k = int(rng.integers(1, n + 1))
        v = torch.from_numpy(rng.integers(0, 5, size=(1, n)).astype(np.float32)).to(torch.bfloat16)
        got = oracle.topk_total_order(v, k)[0].tolist()
        want = sorted(range(n), key=lambda i: (-float(v[0, i]), i))[:k]
        assert got == want
