"""The HBM read envelope probe (skv_hbm_read_probe): every thread's XOR of the 16-byte vectors it
read equals the XOR of the vectors its access order names, for both orders, for workgroups that
take one or several tiles, the last one partial. The probe's numbers are only meaningful if it
reads every byte of the source once, which this checks."""
import numpy as np
import pytest
import torch

from shadowkv_amd.kernels import shadowkv

pytestmark = pytest.mark.gpu

TILE_VECS = 4096


def _order(pattern: str) -> np.ndarray:
    """[256 threads, 16 loads] -> vector index within a 64 KB tile."""
    t = np.arange(256)[:, None]
    k = np.arange(16)[None, :]
    if pattern == "contiguous":
        return k * 256 + t
    wave, lane = t // 64, t % 64
    li, grp = lane % 16, lane // 16
    kg, ks = k // 4, k % 4
    return (wave * 64 + 16 * kg + li) * 16 + 4 * ks + grp


def _expected(vec: np.ndarray, tiles: int, per_wg: int, pattern: str) -> np.ndarray:
    order = _order(pattern)
    assert sorted(order.ravel().tolist()) == list(range(TILE_VECS))  # each vector of a tile read once
    groups = -(-tiles // per_wg)
    out = np.zeros((groups, 256, 4), dtype=np.uint32)
    for g in range(groups):
        for tile in range(g * per_wg, min(g * per_wg + per_wg, tiles)):
            out[g] ^= np.bitwise_xor.reduce(vec[tile][order], axis=1)
    return out


@pytest.mark.parametrize("nt", [False, True])
@pytest.mark.parametrize("pattern", ["contiguous", "operand"])
@pytest.mark.parametrize("tiles,per_wg", [(1, 1), (7, 1), (7, 3), (9, 4)])
def test_read_probe_reads_every_vector_once(gpu, pattern, tiles, per_wg, nt):
    print(f"hbm_read_probe pattern={pattern} tiles={tiles} per_wg={per_wg} nt={nt}", flush=True)
    g = torch.Generator().manual_seed(tiles * 31 + per_wg)
    src = torch.randint(0, 256, (tiles * 65536,), dtype=torch.uint8, generator=g)
    groups = -(-tiles // per_wg)
    sink = torch.full((groups * 4096 + 64,), 0x5a, dtype=torch.uint8, device=gpu)
    shadowkv.hbm_read_probe(src.to(gpu), per_wg, pattern, sink, nt)
    torch.cuda.synchronize()
    got = sink.cpu().numpy()
    vec = src.numpy().view(np.uint32).reshape(tiles, TILE_VECS, 4)
    exp = _expected(vec, tiles, per_wg, pattern)
    assert np.array_equal(got[: groups * 4096].view(np.uint32).reshape(groups, 256, 4), exp)
    assert (got[groups * 4096:] == 0x5a).all()  # nothing past the workgroups' vectors


def test_read_probe_rejects_bad_arguments(gpu):
    src = torch.zeros(2 * 65536, dtype=torch.uint8, device=gpu)
    sink = torch.zeros(2 * 4096, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="multiple of 65536"):
        shadowkv.hbm_read_probe(src[:1000], 1, "contiguous", sink)
    with pytest.raises(ValueError, match="pattern"):
        shadowkv.hbm_read_probe(src, 1, "strided", sink)
    with pytest.raises(RuntimeError, match="tiles_per_workgroup"):
        shadowkv.hbm_read_probe(src, 0, "contiguous", sink)
    with pytest.raises(RuntimeError, match="sink of"):
        shadowkv.hbm_read_probe(src, 1, "contiguous", sink[:4096])


def test_mfma_probe_flops_and_output(gpu):
    """The MFMA peak probe writes one finite, nonzero float per thread and reports the flops of
    its bf16 32x32x16 instructions (4 chains per wave, 4 waves per workgroup)."""
    sink = torch.full((3 * 256 + 16,), 123.0, dtype=torch.float32, device=gpu)
    flops = shadowkv.mfma_peak_probe(3, 5, sink)
    torch.cuda.synchronize()
    assert flops == 3 * 4 * 5 * 4 * 32 * 32 * 16 * 2
    out = sink.cpu()
    assert torch.isfinite(out[:768]).all() and (out[:768] != 0).all()
    assert (out[768:] == 123.0).all()  # nothing past the workgroups' threads
    with pytest.raises(RuntimeError, match="workgroups"):
        shadowkv.mfma_peak_probe(0, 5, sink)
    with pytest.raises(ValueError, match="are addressed"):  # the shim's bound check
        shadowkv.mfma_peak_probe(4, 5, sink)
    from shadowkv_amd import _lib
    with pytest.raises(RuntimeError, match="sink of"):  # and the library's own
        _lib.call("skv_mfma_peak_probe", 4, 5, sink.data_ptr(), sink.numel() * 4, 0)
    with pytest.raises(RuntimeError, match="product at most"):  # one launch's work is bounded
        _lib.call("skv_mfma_peak_probe", 1 << 13, 1 << 12, sink.data_ptr(), 1 << 40, 0)
