"""Writes the committed golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

reorder_kat.npz — the reference's own known-answer test for the cache-hit reorder
(kernels/test_cached_gather_copy.cu): its input generator is restated here with glibc's
rand() (same libc sequence, srand(12345), :224-280) for 192 rows of 256 slots over 16384
chunks with 154 hits per row, and its host golden procedure (:70-116: std::map of old key ->
slot, hits collected in query order then keys and offsets sorted separately, misses sorted)
is restated as plain loops. This code shares nothing with oracle.reorder, which the fixture
then checks.

decode_small.npz — a small single-layer decode step produced by the oracle (regression
vectors for the GPU tests; see tests/test_gpu_decode.py).
"""
from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BLOCK_NUM = 8 * 24          # test_cached_gather_copy.cu:58
MAP = 256                   # BLOCK_SIZE_MAP
CPU_V_LENGTH = 128 * 1024   # :59
FAKE_HIT_CNT = 154          # :61


def kat_inputs():
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    libc.srand(12345)
    rand = libc.rand
    nkeys = CPU_V_LENGTH // 8
    keys = np.zeros((BLOCK_NUM, MAP), dtype=np.int64)
    query = np.zeros((BLOCK_NUM, MAP), dtype=np.int64)
    for k in range(BLOCK_NUM):
        prev_keys, prev_reorders, prev_hits = set(), set(), set()
        for i in range(MAP):
            while True:
                key = rand() % nkeys
                if key not in prev_keys:
                    break
            prev_keys.add(key)
            keys[k, i] = key
        keys[k].sort()
        for i in range(MAP):
            if i < FAKE_HIT_CNT:
                while True:
                    hr = rand() % MAP
                    if hr not in prev_hits:
                        break
                prev_hits.add(hr)
                query[k, i] = keys[k, hr]
            else:
                while True:
                    r = rand() % nkeys
                    if r not in prev_reorders and r not in prev_keys:
                        break
                query[k, i] = r
            prev_reorders.add(int(query[k, i]))
    return keys, query


def kat_golden(keys, query):
    out_keys = np.zeros_like(keys)
    out_offs = np.zeros_like(keys)
    cnts = np.zeros(keys.shape[0], dtype=np.int64)
    for k in range(keys.shape[0]):
        lut = {}
        for i in range(MAP):
            lut.setdefault(int(keys[k, i]), i)  # std::map::insert keeps the first
        hit_keys, hit_offs, misses = [], [], []
        for i in range(MAP):
            q = int(query[k, i])
            if q in lut:
                hit_keys.append(q)
                hit_offs.append(lut[q])
            else:
                misses.append(q)
        idw = len(hit_keys)
        out_keys[k, :idw] = sorted(hit_keys)
        out_offs[k, :idw] = sorted(hit_offs)
        out_keys[k, idw:] = sorted(misses)
        out_offs[k, idw:] = sorted(misses)
        cnts[k] = idw
    return out_keys, out_offs, cnts


def write_kat():
    keys, query = kat_inputs()
    ek, eo, cnts = kat_golden(keys, query)
    np.savez_compressed(HERE / "reorder_kat.npz", orig_keys=keys.astype(np.int16), query_keys=query.astype(np.int16),
                        expected_keys=ek.astype(np.int16), expected_offsets=eo.astype(np.int16),
                        expected_cnts=cnts.astype(np.int16))


def decode_small_case(chunk=8, glm=False):
    """Seeded inputs of the small decode fixture and the oracle's results (deterministic). The
    committed fixture is the chunk-8 case; other chunk sizes give the same prompt tensors. glm:
    the GLM-4-9B head layout (2 kv heads of 16 query heads) with GLM's interleaved RoPE table."""
    sys.path.insert(0, str(HERE.parents[1]))
    import torch
    import oracle

    g = torch.Generator().manual_seed(1234)
    B, H, G, D, ctx, rank, budget = 1, 2, (16 if glm else 4), 128, 2048, 32, 1024
    A = torch.randn(ctx, rank, generator=g) / rank ** 0.5
    Bm = torch.randn(rank, H * D, generator=g) / rank ** 0.5
    k_pre = (A @ Bm + 0.05 * torch.randn(ctx, H * D, generator=g)).view(1, ctx, H, D).transpose(1, 2)
    k_pre = k_pre.to(torch.bfloat16).contiguous()
    v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
    q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
    cos_sin = oracle.build_glm_cos_sin_cache(ctx + 64, 10000.0) if glm else oracle.build_cos_sin_cache(ctx + 64, 500000.0)
    st = oracle.encode_layer(k_pre, v, q_last, cos_sin, rank=rank, chunk=chunk, budget=budget)
    q = torch.randn(B, H * G, D, generator=g).to(torch.bfloat16)
    k_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    v_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    state_in = dict(U=st.U.clone(), SV=st.SV.clone(), landmarks=st.landmarks.clone(),
                    landmark_idx=st.landmark_idx.clone(), host_v=st.host_v.clone(), kbuf=st.kbuf.clone(),
                    vbuf=st.vbuf.clone(), position_ids=st.position_ids.clone())
    res = oracle.decode_layer_step(st, q, k_new, v_new, cos_sin)
    return dict(state_in=state_in, st=st, res=res, q=q, k_new=k_new, v_new=v_new, cos_sin=cos_sin,
                k_pre=k_pre, v=v, q_last=q_last,
                dims=dict(B=B, H=H, G=G, D=D, ctx=ctx, rank=rank, chunk=chunk, budget=budget))


def single_layer_case(seed: int = 8192):
    """The single-layer decode workload at its own shape: Llama-3-8B heads (8 kv heads x 4 query
    heads, head_dim 128), batch 1, ctx 8192, rank 160, chunk 8, budget 2048 (256 chunks), 48
    outlier chunks and 4 local chunks, hence 968 landmarks; pre-RoPE keys A(8192 x 160).B(160 x 1024)
    + 0.05 N(0,1) with A, B ~ N(0, 1/160) (standard deviation 1/sqrt(160)), values, last prompt query
    and the decode token's q/k/v ~ N(0,1), bf16; RoPE theta 5e5. Encoded by the oracle (full SVD,
    bf16 cosine outliers, torch.topk initial selection); one oracle decode step on top."""
    sys.path.insert(0, str(HERE.parents[1]))
    import torch
    import oracle

    g = torch.Generator().manual_seed(seed)
    B, H, G, D, ctx, rank, budget, chunk = 1, 8, 4, 128, 8192, 160, 2048, 8
    A = torch.randn(ctx, rank, generator=g) / rank ** 0.5
    Bm = torch.randn(rank, H * D, generator=g) / rank ** 0.5
    k_pre = (A @ Bm + 0.05 * torch.randn(ctx, H * D, generator=g)).view(1, ctx, H, D).transpose(1, 2)
    k_pre = k_pre.to(torch.bfloat16).contiguous()
    v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
    q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
    cos_sin = oracle.build_cos_sin_cache(ctx + 64, 500000.0)
    st = oracle.encode_layer(k_pre, v, q_last, cos_sin, rank=rank, chunk=chunk, budget=budget)
    q = torch.randn(B, H * G, D, generator=g).to(torch.bfloat16)
    k_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    v_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    state_in = dict(U=st.U.clone(), SV=st.SV.clone(), landmarks=st.landmarks.clone(),
                    landmark_idx=st.landmark_idx.clone(), host_v=st.host_v.clone(), kbuf=st.kbuf.clone(),
                    vbuf=st.vbuf.clone(), position_ids=st.position_ids.clone())
    res = oracle.decode_layer_step(st, q, k_new, v_new, cos_sin)
    return dict(state_in=state_in, st=st, res=res, q=q, k_new=k_new, v_new=v_new, cos_sin=cos_sin,
                k_pre=k_pre, v=v, q_last=q_last,
                dims=dict(B=B, H=H, G=G, D=D, ctx=ctx, rank=rank, chunk=chunk, budget=budget))


def digest(t) -> str:
    import hashlib
    import torch
    a = t.contiguous().view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.contiguous().numpy()
    return hashlib.sha256(a.tobytes()).hexdigest()


def write_decode_small():
    case = decode_small_case()
    st, res = case["st"], case["res"]
    import torch
    np.savez_compressed(
        HERE / "decode_small.npz",
        meta=np.array([st.prefill_local, st.sparse_start, st.sparse_end, st.buf_len, res["L"]]),
        in_digests=np.array([digest(case["state_in"][k]) for k in sorted(case["state_in"])]),
        out_scores=res["scores"].view(torch.int16).numpy(), out_selected=res["selected"].numpy(),
        out_cnts=res["cnts"], out_offsets=res["offsets"], out_position_ids=st.position_ids.numpy(),
        out_attn=res["out"].view(torch.int16).numpy(),
        out_digests=np.array([digest(st.kbuf), digest(st.vbuf)]))


if __name__ == "__main__":
    write_kat()
    write_decode_small()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
