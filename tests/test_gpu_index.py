"""GPU parity of the index/copy kernels (a3 reorder, a4/a5 chunk copies, a2 top-k): bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from shadowkv_amd import _lib
from shadowkv_amd.kernels import shadowkv
from tests.golden import make_golden

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def test_reorder_reference_kat(gpu):
    d = np.load(make_golden.HERE / "reorder_kat.npz")
    rows, S = d["orig_keys"].shape
    _say(f"reorder KAT rows={rows} S={S}")
    cached = torch.from_numpy(d["orig_keys"].astype(np.int64)).to(gpu)
    cur = torch.from_numpy(d["query_keys"].astype(np.int64)).to(gpu)
    offs = torch.zeros(rows * S, dtype=torch.int32, device=gpu)
    cnts = torch.zeros(rows, dtype=torch.int32, device=gpu)
    shadowkv.reorder_keys_and_compute_offsets(cached, cur, offs, cnts, rows // 8, 8, S)
    torch.cuda.synchronize()
    assert np.array_equal(cached.cpu().numpy(), d["expected_keys"].astype(np.int64))
    assert np.array_equal(offs.view(rows, S).cpu().numpy(), d["expected_offsets"].astype(np.int32))
    assert np.array_equal(cnts.cpu().numpy(), d["expected_cnts"].astype(np.int32))


@pytest.mark.parametrize("S", [1, 7, 128, 256, 1000, 2048])
def test_reorder_random_unsorted(gpu, S):
    rng = np.random.default_rng(S)
    B, H = 2, 4
    rows = B * H
    _say(f"reorder random S={S}")
    old = np.stack([rng.permutation(4 * S + 3)[:S] for _ in range(rows)]).astype(np.int64)
    old[rng.random(old.shape) < 0.05] = -1
    new = np.stack([rng.permutation(4 * S + 3)[:S] for _ in range(rows)]).astype(np.int64)
    valid = old[0][old[0] >= 0]  # row 0: every valid old id is selected again
    fresh = np.setdiff1d(np.arange(10 * S + 10), old[0])[:S - len(valid)]
    new[0] = rng.permutation(np.concatenate([valid, fresh]))
    ids, offs, cnts = oracle.reorder(old, new)
    cached = torch.from_numpy(old).to(gpu)
    o = torch.zeros(rows * S, dtype=torch.int32, device=gpu)
    c = torch.zeros(rows, dtype=torch.int32, device=gpu)
    shadowkv.reorder_keys_and_compute_offsets(cached, torch.from_numpy(new).to(gpu), o, c, B, H, S)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), cnts)
    assert np.array_equal(cached.cpu().numpy(), ids)
    assert np.array_equal(o.view(rows, S).cpu().numpy(), offs)


def _setup_cache(gpu, B, H, S, chunk_elems, nchunks, hit_frac, seed, pinned=True):
    rng = np.random.default_rng(seed)
    rows = B * H
    host = torch.from_numpy(oracle_coded(rows, nchunks, chunk_elems, seed)).view(torch.bfloat16)
    host = host.view(B, H, nchunks, chunk_elems)
    if pinned:
        host = host.pin_memory()
    else:
        host = host.to(gpu)
    old = np.stack([rng.permutation(nchunks)[:S] for _ in range(rows)]).astype(np.int64)
    new = np.empty_like(old)
    for r in range(rows):
        nh = int(round(hit_frac * S))
        keep = rng.permutation(old[r])[:nh]
        rest = rng.permutation(np.setdiff1d(np.arange(nchunks), old[r]))[:S - nh]
        new[r] = rng.permutation(np.concatenate([keep, rest]))
    ids, offs, cnts = oracle.reorder(old, new)
    return host, old, new, ids, offs, cnts


def oracle_coded(rows, n, E, tag):
    r = np.arange(rows)[:, None, None]
    c = np.arange(n)[None, :, None]
    w = np.arange(E)[None, None, :]
    return ((tag * 7919 + r * 1543 + c * 131 + w) % 65521 - 32760).astype(np.int16)


@pytest.mark.parametrize("hit_frac,chunk,S,pinned", [(0.6, 8, 256, True), (0.0, 8, 256, True), (1.0, 8, 256, True),
                                                     (0.3, 4, 512, True), (0.6, 8, 2048, True), (0.5, 8, 256, False)])
def test_cached_gather_copy(gpu, hit_frac, chunk, S, pinned):
    B, H, D = 2, 8, 128
    E = chunk * D
    nchunks = 4 * S + 5
    _say(f"gather_copy_with_offsets hit={hit_frac} chunk={chunk} S={S} pinned={pinned}")
    host, old, new, ids, offs, cnts = _setup_cache(gpu, B, H, S, E, nchunks, hit_frac, 17, pinned)
    rows = B * H
    prefix = 3 * chunk  # device slots before the sparse region
    buf_len = prefix + S * chunk + 40
    hostn = host.cpu().view(torch.int16).numpy().reshape(rows, nchunks, E)
    dev = torch.zeros(B, H, buf_len, D, dtype=torch.bfloat16)
    sparse = np.stack([hostn[r, old[r]] for r in range(rows)])  # slot i holds old[i]
    dev[:, :, prefix:prefix + S * chunk] = torch.from_numpy(sparse).view(torch.bfloat16).view(B, H, S * chunk, D)
    dev[:, :, :prefix] = 1.5
    dev_g = dev.to(gpu)
    offs_g = torch.from_numpy(offs.reshape(-1)).to(gpu)
    cnts_g = torch.from_numpy(cnts).to(gpu)
    shadowkv.gather_copy_with_offsets(host, dev_g, None, offs_g, cnts_g, None, B, H, nchunks * E, S * E,
                                      prefix * D, buf_len * D, S)
    torch.cuda.synchronize()
    got = dev_g.cpu()
    want = oracle.cached_gather_copy(hostn, sparse, offs, cnts)
    assert torch.equal(got[:, :, :prefix], dev[:, :, :prefix])
    assert torch.equal(got[:, :, prefix + S * chunk:], dev[:, :, prefix + S * chunk:])
    assert np.array_equal(got[:, :, prefix:prefix + S * chunk].reshape(rows, S, E).view(torch.int16).numpy(), want)
    # key-side compaction on the same layout
    kdev = dev.to(gpu)
    shadowkv.gather_copy_d2d_with_offsets(kdev, offs_g, cnts_g, B, H, S * E, prefix * D, buf_len * D, S)
    torch.cuda.synchronize()
    wantk = oracle.compact_hits(sparse, offs, cnts)
    assert np.array_equal(kdev.cpu()[:, :, prefix:prefix + S * chunk].reshape(rows, S, E).view(torch.int16).numpy(),
                          wantk)
    # the split form the decode handler issues: hit move on one stream, then the miss gather
    # alone on another; same bytes as the combined call
    sdev = dev.to(gpu)
    shadowkv.gather_copy_d2d_with_offsets(sdev, offs_g, cnts_g, B, H, S * E, prefix * D, buf_len * D, S)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        shadowkv.gather_copy_with_offsets(host, sdev, None, offs_g, cnts_g, None, B, H, nchunks * E, S * E,
                                          prefix * D, buf_len * D, S, misses_only=True)
    torch.cuda.synchronize()
    assert torch.equal(sdev.cpu().view(torch.int16), got.view(torch.int16))  # bit patterns (some are NaNs)


@pytest.mark.parametrize("S,chunk,hit_frac", [(2048, 16, 0.9), (9000, 2, 0.95), (300, 8, 1.0)])
def test_compact_hits_many_batches(gpu, S, chunk, hit_frac):
    """The in-place hit compaction over rows whose moving hits span many 64-chunk batches, with
    the offsets held in LDS (map_size <= 8192) and read from global memory (9000)."""
    rows, D = 3, 128
    E = chunk * D
    _say(f"compact_hits S={S} chunk={chunk} hit={hit_frac}")
    rng = np.random.default_rng(S + chunk)
    sparse = rng.integers(-32768, 32767, size=(rows, S, E), dtype=np.int16)
    offs = np.zeros((rows, S), dtype=np.int32)
    cnts = np.zeros(rows, dtype=np.int32)
    for r in range(rows):
        c = int(hit_frac * S) - r  # ragged hit counts
        hit_slots = np.sort(rng.choice(S, size=c, replace=False)).astype(np.int32)
        offs[r, :c] = hit_slots
        offs[r, c:] = rng.integers(0, 4 * S, size=S - c)  # miss ids: not read by the compaction
        cnts[r] = c
    prefix = 2 * chunk
    buf_len = prefix + S * chunk + 8
    dev = torch.zeros(1, rows, buf_len, D, dtype=torch.int16)
    dev[0, :, prefix:prefix + S * chunk] = torch.from_numpy(sparse).view(rows, S * chunk, D)
    kdev = dev.view(torch.bfloat16).to(gpu)
    offs_g, cnts_g = torch.from_numpy(offs.reshape(-1)).to(gpu), torch.from_numpy(cnts).to(gpu)
    # through the C ABI: the Python shim caps map_size at the selection maximum (2048)
    _lib.call("skv_gather_copy_d2d_with_offsets", kdev.data_ptr(), offs_g.data_ptr(), cnts_g.data_ptr(), 1, rows,
              S * E, prefix * D, buf_len * D, S, E, int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    got = kdev.cpu().view(torch.int16)
    assert torch.equal(got[0, :, :prefix], dev[0, :, :prefix])
    assert torch.equal(got[0, :, prefix + S * chunk:], dev[0, :, prefix + S * chunk:])
    want = oracle.compact_hits(sparse, offs, cnts)
    assert np.array_equal(got[0, :, prefix:prefix + S * chunk].reshape(rows, S, E).numpy(), want)


def test_gather_copy_plain(gpu):
    B, H, S, chunk, D = 2, 4, 128, 8, 128
    E = chunk * D
    nchunks = 600
    host, old, new, *_ = _setup_cache(gpu, B, H, S, E, nchunks, 0.0, 5)
    dst = torch.zeros(B * H, S * E, dtype=torch.bfloat16, device=gpu)
    shadowkv.gather_copy(host, dst, torch.from_numpy(new).to(gpu), B, H, nchunks * E, S * E, S)
    torch.cuda.synchronize()
    hostn = host.view(torch.int16).numpy().reshape(B * H, nchunks, E)
    want = oracle.gather_copy_plain(hostn, new)
    assert np.array_equal(dst.cpu().view(torch.int16).numpy().reshape(B * H, S, E), want)


@pytest.mark.parametrize("n,k,ties", [(968, 256, False), (15304, 256, False), (15304, 256, True), (1000, 1000, True),
                                      (130680, 2048, False), (5, 1, True)])
def test_topk_gather_bit_exact(gpu, n, k, ties):
    rows = 8
    g = torch.Generator().manual_seed(n + k)
    _say(f"topk n={n} k={k} ties={ties}")
    x = torch.softmax(torch.randn(rows, n, generator=g) * 3, dim=-1)
    if ties:
        x = (x * 50).round() / 50  # heavy ties, including many zeros
    x = x.to(torch.bfloat16)
    lidx = torch.stack([torch.randperm(10 * n, generator=g)[:n].sort().values for _ in range(rows)])
    want = oracle.topk_gather(x, lidx, k)
    out = torch.empty(rows, k, dtype=torch.int64, device=gpu)
    shadowkv.topk_gather(x.to(gpu), lidx.to(gpu), k, out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("split", ["0", "1", "1ws", "ws"])
@pytest.mark.parametrize("rows,m,n,S", [(64, 4, 15304, 256), (8, 16, 32712, 256), (8, 4, 130680, 2048),
                                        (8, 4, 968, 256), (2, 1, 300, 7)])
def test_select_chunks_fused_equals_unfused(gpu, monkeypatch, rows, m, n, S, split):
    """The fused selection (keys computed per row in the selection kernel; on the split path by
    the many-workgroup softmax + GQA-max kernel first; on the parts path ("ws") also the radix
    passes over many workgroups per row, with a caller workspace) equals the unfused sequence."""
    _fused_equals_unfused(gpu, monkeypatch, rows, m, n, S, split, rows * n + S)


def test_select_chunks_random_shapes(gpu, monkeypatch):
    """The same check on 12 seeded random shapes (rows 1-40, 1-16 queries, landmark counts that are
    not multiples of 8 or of the 256-column tile, selections from 1 to 2048) on every path."""
    rng = np.random.default_rng(2024)
    for case in range(12):
        m = int(rng.choice([1, 2, 3, 4, 5, 8, 9, 12, 16]))
        rows = int(rng.integers(1, 41))
        n = int(rng.integers(100, 40001))
        S = int(min(n // 2, rng.choice([1, 2, 7, 64, 255, 256, 1000, 2048])))  # (half the ids stay unselected)
        for split in ("0", "1", "1ws", "ws"):
            _fused_equals_unfused(gpu, monkeypatch, rows, m, n, S, split, 7919 * case + 11)


def _fused_equals_unfused(gpu, monkeypatch, rows, m, n, S, split, seed):
    monkeypatch.setenv("SKV_SELECT_SPLIT", {"ws": "2", "1ws": "1"}.get(split, split))
    _say(f"select_chunks rows={rows} m={m} n={n} S={S} split={split}")
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(rows, m, 128, generator=g).to(torch.bfloat16).to(gpu)
    L = torch.randn(rows, n, 128, generator=g).to(torch.bfloat16).to(gpu)
    lidx = torch.stack([torch.randperm(n + n // 10, generator=g)[:n].sort().values for _ in range(rows)]).to(gpu)
    tiles = (n + 255) // 256
    D = torch.empty(rows, m, n, dtype=torch.bfloat16, device=gpu)
    norm = torch.empty(rows, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    shadowkv.score_logits(q, L, D, norm, ssum, rows, m, n, 128)
    scores = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    shadowkv.softmax_gqa_max(D, norm, ssum, scores, rows, m, n)
    sel = torch.empty(rows, S, dtype=torch.int64, device=gpu)
    shadowkv.topk_gather(scores, lidx, S, sel)
    torch.cuda.synchronize()
    # previous slots: about half of this step's selection plus other landmark ids, shuffled
    old = []
    for r in range(rows):
        keep = sel[r, :S // 2].cpu()
        pool = lidx[r].cpu()
        others = pool[~torch.isin(pool, sel[r].cpu())]
        others = others[torch.randperm(len(others), generator=g)[:S - len(keep)]]
        old.append(torch.cat([keep, others])[torch.randperm(S, generator=g)])
    old = torch.stack(old).to(gpu)
    pos1, off1, cnt1 = old.clone(), torch.empty(rows * S, dtype=torch.int32, device=gpu), torch.empty(rows, dtype=torch.int32, device=gpu)
    shadowkv.reorder_keys_and_compute_offsets(pos1, sel, off1, cnt1, rows, 1, S)
    pos2, off2, cnt2 = old.clone(), torch.empty_like(off1), torch.empty_like(cnt1)
    scores2 = torch.empty_like(scores)
    sel2 = torch.empty_like(sel)
    nchunks = n + n // 10
    ws = None
    if split in ("ws", "1ws"):  # with the caller's workspace: the key histograms counted by the
        # softmax kernel ("1ws"), or each row's selection over many workgroups ("ws")
        ws = torch.empty(shadowkv.select_workspace_bytes(rows, n, S), dtype=torch.uint8, device=gpu)
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, pos2, off2, cnt2, out_scores=scores2,
                           out_selected=sel2, workspace=ws)
    pos3, off3, cnt3 = old.clone(), torch.empty_like(off1), torch.empty_like(cnt1)
    staging = torch.empty_like(scores) if n > 16384 else None  # scores beyond LDS need global staging
    if split in ("ws", "1ws") and staging is None:
        staging = torch.empty_like(scores)  # the many-workgroup path needs the keys in global memory
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, pos3, off3, cnt3, out_scores=staging,
                           workspace=ws)
    # selection only (no previous slots; a chunk pool's selection): the ids in top-k order
    sel4 = torch.full_like(sel, -7)
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, None, None, None,
                           out_scores=torch.empty_like(scores), out_selected=sel4, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(sel4, sel)
    assert torch.equal(pos3, pos1) and torch.equal(off3, off1) and torch.equal(cnt3, cnt1)
    assert torch.equal(scores2, scores)
    assert torch.equal(sel2, sel)
    assert torch.equal(pos2, pos1) and torch.equal(off2, off1) and torch.equal(cnt2, cnt1)
    # and both against the oracle, from the kernel's own scores
    assert torch.equal(sel.cpu(), oracle.topk_gather(scores.cpu(), lidx.cpu(), S))
    ids, offs, cnts = oracle.reorder(old.cpu().numpy(), sel.cpu().numpy())
    assert np.array_equal(pos2.cpu().numpy(), ids) and np.array_equal(cnt2.cpu().numpy(), cnts)
    assert np.array_equal(off2.view(rows, S).cpu().numpy(), offs)
    assert (cnts >= S // 2).all()


@pytest.mark.parametrize("split", ["0", "1", "1ws", "ws"])
@pytest.mark.parametrize("rows,m,n,S", [(8, 4, 130680, 2048), (8, 16, 32712, 256), (4, 4, 15304, 256)])
def test_select_chunks_all_ties(gpu, monkeypatch, rows, m, n, S, split):
    """Zero queries: every logit 0, every probability 1/n, so all keys tie and the selection is
    the S lowest landmark indices (ties broken by index across every slice of a row)."""
    monkeypatch.setenv("SKV_SELECT_SPLIT", {"ws": "2", "1ws": "1"}.get(split, split))
    _say(f"select_chunks all ties rows={rows} m={m} n={n} S={S} split={split}")
    g = torch.Generator().manual_seed(n + S)
    q = torch.zeros(rows, m, 128, dtype=torch.bfloat16, device=gpu)
    L = torch.randn(rows, n, 128, generator=g).to(torch.bfloat16).to(gpu)
    lidx = torch.stack([torch.randperm(n + n // 10, generator=g)[:n].sort().values for _ in range(rows)]).to(gpu)
    tiles = (n + 255) // 256
    D = torch.empty(rows, m, n, dtype=torch.bfloat16, device=gpu)
    norm = torch.empty(rows, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    shadowkv.score_logits(q, L, D, norm, ssum, rows, m, n, 128)
    nchunks = n + n // 10
    pos = torch.full((rows, S), -1, dtype=torch.int64, device=gpu)
    off = torch.empty(rows * S, dtype=torch.int32, device=gpu)
    cnt = torch.empty(rows, dtype=torch.int32, device=gpu)
    scores = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    sel = torch.empty(rows, S, dtype=torch.int64, device=gpu)
    ws = torch.empty(shadowkv.select_workspace_bytes(rows, n, S), dtype=torch.uint8, device=gpu) if split in ("ws", "1ws") else None
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, pos, off, cnt, out_scores=scores,
                           out_selected=sel, workspace=ws)
    torch.cuda.synchronize()
    assert (scores == scores[0, 0]).all()
    want = lidx[:, :S].cpu()  # lowest indices, ids ascending (previous slots empty: all misses)
    assert torch.equal(sel.cpu(), want)
    assert torch.equal(pos.cpu(), want)
    assert (cnt.cpu() == 0).all()
    assert torch.equal(off.view(rows, S).cpu(), want.to(torch.int32))


@pytest.mark.parametrize("split", ["0", "1", "1ws", "ws"])
@pytest.mark.parametrize("rows,m,n", [(4, 4, 256), (2, 16, 1000), (1, 8, 2048)])
def test_select_chunks_selects_every_landmark(gpu, monkeypatch, rows, m, n, split):
    """select_sets = n: every landmark is selected; with empty previous slots all are misses, so
    the slots hold the landmark ids ascending and the top-k order is the scores' total order."""
    S = n
    monkeypatch.setenv("SKV_SELECT_SPLIT", {"ws": "2", "1ws": "1"}.get(split, split))
    _say(f"select every landmark rows={rows} m={m} n={n} split={split}")
    g = torch.Generator().manual_seed(n + m)
    q = torch.randn(rows, m, 128, generator=g).to(torch.bfloat16).to(gpu)
    L = torch.randn(rows, n, 128, generator=g).to(torch.bfloat16).to(gpu)
    lidx = torch.stack([torch.randperm(2 * n, generator=g)[:n].sort().values for _ in range(rows)]).to(gpu)
    tiles = (n + 255) // 256
    D = torch.empty(rows, m, n, dtype=torch.bfloat16, device=gpu)
    norm = torch.empty(rows, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    shadowkv.score_logits(q, L, D, norm, ssum, rows, m, n, 128)
    pos = torch.full((rows, S), -1, dtype=torch.int64, device=gpu)
    off = torch.empty(rows * S, dtype=torch.int32, device=gpu)
    cnt = torch.empty(rows, dtype=torch.int32, device=gpu)
    scores = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    sel = torch.empty(rows, S, dtype=torch.int64, device=gpu)
    ws = torch.empty(shadowkv.select_workspace_bytes(rows, n, S), dtype=torch.uint8, device=gpu) if split in ("ws", "1ws") else None
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, 2 * n, pos, off, cnt, out_scores=scores,
                           out_selected=sel, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(pos.cpu(), lidx.cpu())
    assert (cnt.cpu() == 0).all()
    assert torch.equal(off.view(rows, S).cpu(), lidx.cpu().to(torch.int32))
    assert torch.equal(sel.cpu(), oracle.topk_gather(scores.cpu(), lidx.cpu(), S))


def _old_slots(sel, lidx, S, mode, g):
    """Previous slots for a folded-move test, per row: "half" about half of this step's selection
    among other ids, shuffled; "shift" the first quarter of the selection in place, one other id,
    then the next quarter (every later hit moves one slot down: each move reads the chunk the next
    move writes); "all" the selection reversed (every slot a hit, no move); "none" no hit."""
    old = []
    for r in range(sel.shape[0]):
        s = sel[r].cpu()
        pool = lidx[r].cpu()
        others = pool[~torch.isin(pool, s)]
        others = others[torch.randperm(len(others), generator=g)]
        if mode == "half":
            keep = s[:S // 2]
            row = torch.cat([keep, others[:S - len(keep)]])[torch.randperm(S, generator=g)]
        elif mode == "shift":
            q = max(S // 4, 1)
            row = torch.cat([s[:q], others[:1], s[q:2 * q]])
            row = torch.cat([row, others[1:1 + S - len(row)]])[:S]
        elif mode == "all":
            row = s.flip(0)
        else:
            row = others[:S]
        old.append(row)
    return torch.stack(old)


@pytest.mark.parametrize("mode", ["half", "shift", "all", "none"])
@pytest.mark.parametrize("split", ["0", "1", "1ws", "ws"])
@pytest.mark.parametrize("rows,m,n,S,chunk_elems", [(64, 4, 15304, 256, 1024), (8, 4, 130680, 2048, 1024),
                                                    (8, 4, 968, 256, 1024), (2, 1, 300, 7, 16)])
def test_select_chunks_folded_hit_moves(gpu, monkeypatch, rows, m, n, S, chunk_elems, split, mode):
    """skv_select_chunks_compact: the selection that also moves each row's hits in both buffers
    (in place, slot i <- slot offsets[i] for i < cnts) leaves the same selection, offsets, counts
    and slot ids as the plain selection, and buffers bit-identical to the plain selection followed
    by the separate compaction kernel on each buffer and to a slot-by-slot compaction on the host;
    also with the value buffer alone."""
    monkeypatch.setenv("SKV_SELECT_SPLIT", {"ws": "2", "1ws": "1"}.get(split, split))
    _say(f"select_chunks folded moves rows={rows} m={m} n={n} S={S} split={split} mode={mode}")
    g = torch.Generator().manual_seed(rows * n + S + len(mode))
    q = torch.randn(rows, m, 128, generator=g).to(torch.bfloat16).to(gpu)
    L = torch.randn(rows, n, 128, generator=g).to(torch.bfloat16).to(gpu)
    lidx = torch.stack([torch.randperm(n + n // 10, generator=g)[:n].sort().values for _ in range(rows)]).to(gpu)
    tiles = (n + 255) // 256
    D = torch.empty(rows, m, n, dtype=torch.bfloat16, device=gpu)
    norm = torch.empty(rows, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    shadowkv.score_logits(q, L, D, norm, ssum, rows, m, n, 128)
    nchunks = n + n // 10
    ws = torch.empty(shadowkv.select_workspace_bytes(rows, n, S), dtype=torch.uint8, device=gpu) if split in ("ws", "1ws") else None
    sel = torch.empty(rows, S, dtype=torch.int64, device=gpu)
    shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, None, None, None,
                           out_scores=torch.empty(rows, n, dtype=torch.bfloat16, device=gpu), out_selected=sel,
                           workspace=ws)
    torch.cuda.synchronize()
    old = _old_slots(sel, lidx, S, mode, g).to(gpu)
    prefix, tail = 40, 24  # elements before and after the selected region of each buffer row
    stride = prefix + S * chunk_elems + tail
    bufs = [torch.randint(-32768, 32768, (rows, stride), generator=g, dtype=torch.int32).to(torch.int16)
            .view(torch.bfloat16).to(gpu) for _ in range(2)]

    def plain():
        pos, off, cnt = old.clone(), torch.empty(rows * S, dtype=torch.int32, device=gpu), \
            torch.empty(rows, dtype=torch.int32, device=gpu)
        sc = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
        shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, pos, off, cnt, out_scores=sc,
                               workspace=ws)
        return pos, off, cnt, sc

    pos1, off1, cnt1, sc1 = plain()
    want = [b.clone() for b in bufs]
    for b in want:
        shadowkv.gather_copy_d2d_with_offsets(b, off1, cnt1, 1, rows, S * chunk_elems, prefix, stride, S)
    for which in ("both", "v"):
        got = [b.clone() for b in bufs]
        pos2, off2, cnt2 = old.clone(), torch.empty_like(off1), torch.empty_like(cnt1)
        sc2 = torch.empty_like(sc1)
        sel2 = torch.empty_like(sel)
        shadowkv.select_chunks(D, norm, ssum, rows, m, n, lidx, S, nchunks, pos2, off2, cnt2, out_scores=sc2,
                               out_selected=sel2, workspace=ws,
                               move=(got[0], got[1] if which == "both" else None, prefix, stride, chunk_elems))
        torch.cuda.synchronize()
        assert torch.equal(sel2, sel) and torch.equal(sc2, sc1)
        assert torch.equal(pos2, pos1) and torch.equal(off2, off1) and torch.equal(cnt2, cnt1)
        # bit patterns compared (random bits include NaNs)
        assert torch.equal(got[0].view(torch.int16), want[0].view(torch.int16)), f"{which}: value buffer"
        assert torch.equal(got[1].view(torch.int16), (want[1] if which == "both" else bufs[1]).view(torch.int16)), \
            f"{which}: key buffer"
    # the host restatement: hits in previous-slot order, slot i <- old slot offsets[i]
    ids, offs, cnts = oracle.reorder(old.cpu().numpy(), sel.cpu().numpy())
    assert np.array_equal(cnt1.cpu().numpy(), cnts) and np.array_equal(off1.view(rows, S).cpu().numpy(), offs)
    host = bufs[0].cpu().view(torch.int16).numpy()
    ref = host.copy()
    for r in range(rows):
        for i in range(int(cnts[r])):
            j = int(offs[r, i])
            ref[r, prefix + i * chunk_elems:prefix + (i + 1) * chunk_elems] = \
                host[r, prefix + j * chunk_elems:prefix + (j + 1) * chunk_elems]
    assert np.array_equal(want[0].cpu().view(torch.int16).numpy(), ref)
    expect = {"all": S, "none": 0}.get(mode)
    if expect is not None:
        assert (cnts == expect).all()
    if mode == "shift" and S >= 4:
        assert (cnts >= 2 * (S // 4)).all() and (offs[:, S // 4] == S // 4 + 1).all()
