"""Pins for the prompt geometry and the rotary tables, independent of the formulas that produce them.

* Geometry: the derived sizes the hot-path survey lists for every workload (computed there from
  models/kvcache/shadow.py:329,346,477-482,500-501 by hand), checked against both the oracle's
  prefill_geometry and the product cache's own _set_geometry.
* Rotary tables: float64 closed forms cos/sin(p * base^(-2i/d)) at positions up to 2^18, within
  one bf16 rounding plus the float32 angle error the reference's own float32 table carries
  (models/llama.py:138-142, models/glm.py:132-133 through the model's rotary_pos_emb).
"""
import math
import types

import numpy as np
import pytest
import torch

import oracle
from shadowkv_amd.models.kvcache.shadow import ShadowKVCache_CPU, outlier_chunks
from shadowkv_amd.models.tensor_op import build_cos_sin_cache, build_glm_cos_sin_cache

# ctx, budget -> S, outlier chunks, aligned chunks, prefill_local, landmarks n, sparse_start, sparse_end, buf_len
APPENDIX_A = {
    "single layer, ctx 8192": (8192, 2048, 256, 48, 1016, 64, 968, 448, 2496, 2592),
    "Llama-3.1-8B, ctx 122880": (122880, 2048, 256, 48, 15352, 64, 15304, 448, 2496, 2592),
    "GLM-4-9B, ctx 262144": (262144, 2048, 256, 48, 32760, 64, 32712, 448, 2496, 2592),
    "Llama-3-8B-1M, ctx 1048576": (1048576, 16384, 2048, 384, 131064, 64, 130680, 3136, 19520, 19616),
    "e2e 122k prompt, ctx 124928": (124928, 2048, 256, 48, 15608, 64, 15560, 448, 2496, 2592),
}


@pytest.mark.parametrize("name", list(APPENDIX_A))
def test_oracle_geometry_matches_derived_sizes(name):
    ctx, budget, S, out, chunks, local, n, s0, s1, buf = APPENDIX_A[name]
    g = oracle.prefill_geometry(ctx, budget, 8)
    assert (g["S"], g["outlier_chunk"], g["chunks"], g["prefill_local"], g["n"], g["sparse_start"],
            g["sparse_end"], g["buf_len"]) == (S, out, chunks, local, n, s0, s1, buf)


@pytest.mark.parametrize("name", list(APPENDIX_A))
def test_cache_geometry_matches_derived_sizes(name):
    """The product cache's own geometry code (_set_geometry and the outlier count of its
    constructor), run on a stand-in object with the constructor's attributes (no device)."""
    ctx, budget, S, out, chunks, local, n, s0, s1, buf = APPENDIX_A[name]
    ns = types.SimpleNamespace(chunk_size=8, local_chunk=4, sparse_budget=budget, outlier_chunk=outlier_chunks(budget),
                               head_dim=128, buf_len=buf)
    ShadowKVCache_CPU._set_geometry(ns, ctx)
    assert (ns.outlier_chunk, ns.chunks, ns.prefill_local, ns.chunks - ns.outlier_chunk, ns.sparse_start,
            ns.sparse_end) == (out, chunks, local, n, s0, s1)
    assert ns.max_ctx_chunks_len == ctx and ns.kernel_offset == s0 * 128 and ns.kernel_stride == buf * 128


def _closed_form_check(table: torch.Tensor, inv_freq: np.ndarray, positions, half: int):
    """table rows [cos(half) | sin(half)] against float64 cos/sin(p * inv_freq): one bf16 rounding
    (half an ulp of the value, at most 2^-9) plus the float32 angle error of p * inv_freq (the
    reference builds its table in float32: about 3 float32 roundings of the angle)."""
    for p in positions:
        ang = p * inv_freq
        got = table[p].double().numpy()
        tol = 2.0 ** -9 + ang * 3 * 2.0 ** -24 + 1e-12
        assert np.all(np.abs(got[:half] - np.cos(ang)) <= tol), (p, np.abs(got[:half] - np.cos(ang)).max())
        assert np.all(np.abs(got[half:] - np.sin(ang)) <= tol), (p, np.abs(got[half:] - np.sin(ang)).max())


POSITIONS = [0, 1, 37, 4095, 122879, 262143]


@pytest.mark.parametrize("ratio", [1.0, 500.0])
def test_glm_table_closed_form(ratio):
    """GLM-4's partial rotary table: 32 frequencies (10000*rope_ratio)^(-2i/64) over the first 64 dims,
    rows [cos(32) | sin(32)] (models/glm.py:132-133). Checked for both the oracle's and the product's
    builder; a wrong exponent denominator (128 instead of 64) or frequency count fails at p = 1."""
    base = 10000.0 * ratio
    inv = base ** (-np.arange(0, 64, 2, dtype=np.float64) / 64.0)
    for tab in (oracle.build_glm_cos_sin_cache(262144, base), build_glm_cos_sin_cache(262144, base)):
        assert tab.shape == (262144 + 1024, 64) and tab.dtype == torch.bfloat16
        _closed_form_check(tab, inv, POSITIONS, 32)


@pytest.mark.parametrize("theta", [500000.0, 3.58e6])
def test_llama_table_closed_form(theta):
    """Llama's half-split table: 64 frequencies theta^(-2i/128), rows [cos(64) | sin(64)]
    (models/llama.py:138-142,162-167), for the oracle's and the product's builder."""
    inv = theta ** (-np.arange(0, 128, 2, dtype=np.float64) / 128.0)
    for tab in (oracle.build_cos_sin_cache(262144, theta), build_cos_sin_cache(262144, theta, 128)):
        assert tab.shape == (262144 + 1024, 128) and tab.dtype == torch.bfloat16
        _closed_form_check(tab, inv, POSITIONS, 64)


def test_closed_form_check_catches_a_wrong_denominator():
    """The check fails a table built with the exponent over 128 dims instead of 64 (planted in a
    copy of the oracle's formula, on the CPU)."""
    base = 10000.0
    theta = 1.0 / (base ** (torch.arange(0, 64, 2, dtype=torch.float32) / 128))
    idx = torch.outer(torch.arange(4096 + 1024, dtype=torch.float32), theta)
    wrong = torch.cat((idx.cos(), idx.sin()), dim=-1).to(torch.bfloat16)
    inv = base ** (-np.arange(0, 64, 2, dtype=np.float64) / 64.0)
    with pytest.raises(AssertionError):
        _closed_form_check(wrong, inv, [1, 37], 32)
