"""The skinny decode linear layer (skv_linear) against an fp32 torch reference of the same
product: bf16 inputs, exact products, fp32 sums, one rounding to bf16."""
import pytest
import torch

from shadowkv_amd.kernels import shadowkv
from tests.decode_harness import assert_bf16_close

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _ref(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().t()).to(torch.bfloat16)


# (rows, n, k): the Llama-3-8B projections at 4 and 8 decode rows, GLM-4-9B's down projection
# (k = 13696 is not a multiple of the 512-element block), row counts that are not powers of two,
# n not a multiple of a workgroup's rows, and the smallest k.
CASES = [(4, 6144, 4096), (4, 4096, 4096), (4, 28672, 4096), (8, 4096, 14336), (1, 1000, 4096),
         (2, 520, 1032), (3, 77, 4096), (5, 130, 13696), (8, 64, 8), (13, 333, 2048), (16, 96, 4104)]


@pytest.mark.parametrize("rows,n,k", CASES)
def test_linear(gpu, rows, n, k):
    _say(f"linear rows={rows} n={n} k={k}")
    g = torch.Generator().manual_seed(rows * 7919 + n + k)
    x = torch.randn(rows, 1, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16)
    out = torch.full((rows, 1, n), 7.0, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(x.to(gpu), w.to(gpu), out)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), _ref(x, w), floor=1e-4, what=f"linear {rows}x{n}x{k}")


@pytest.mark.parametrize("rows,n,k", [(4, 4608, 4096), (1, 4608, 4096), (3, 77, 4096), (16, 96, 4104)])
def test_linear_bias(gpu, rows, n, k):
    """The projection with a bias (GLM's query_key_value, models/glm.py:165): the bias added to the
    fp32 sum before the one rounding, against fp32 torch; without a bias the call is skv_linear's."""
    _say(f"linear bias rows={rows} n={n} k={k}")
    g = torch.Generator().manual_seed(rows * 17 + n + k)
    x = torch.randn(rows, 1, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 2).to(torch.bfloat16)
    out = torch.full((rows, 1, n), 7.0, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(x.to(gpu), w.to(gpu), out, bias=b.to(gpu))
    plain = torch.empty_like(out)
    shadowkv.linear(x.to(gpu), w.to(gpu), plain)
    torch.cuda.synchronize()
    want = (x.float() @ w.float().t() + b.float()).to(torch.bfloat16)
    assert_bf16_close(out.cpu(), want, floor=1e-3, what=f"linear bias {rows}x{n}x{k}")
    # the same sums: the biased output is the unbiased fp32 sum plus the bias, rounded once, so it
    # is within one bf16 step of the rounded plain output plus the bias
    near = (plain.cpu().float() + b.float()).to(torch.bfloat16)
    assert ((out.cpu().float() - near.float()).abs() <= near.float().abs() * 2 ** -7 + 1e-2).all()
    with pytest.raises(ValueError, match="bias"):
        shadowkv.linear(x.to(gpu), w.to(gpu), out, bias=b[:-1].to(gpu))


def test_linear_random_shapes(gpu):
    """The skinny linear on 12 seeded random shapes (1-16 rows, n 1-9000, k a multiple of 8 up to
    16000, with and without a bias) against fp32 torch."""
    import numpy as np
    rng = np.random.default_rng(81)
    for case in range(12):
        rows, n, k = int(rng.integers(1, 17)), int(rng.integers(1, 9001)), 8 * int(rng.integers(1, 2001))
        bias = bool(rng.integers(0, 2))
        _say(f"linear random case {case}: rows={rows} n={n} k={k} bias={bias}")
        g = torch.Generator().manual_seed(4000 + case)
        x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
        w = (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16)
        b = torch.randn(n, generator=g).to(torch.bfloat16) if bias else None
        out = torch.full((rows, n), 7.0, dtype=torch.bfloat16, device=gpu)
        shadowkv.linear(x.to(gpu), w.to(gpu), out, bias=None if b is None else b.to(gpu))
        torch.cuda.synchronize()
        want = x.float() @ w.float().t() + (b.float() if bias else 0)
        assert_bf16_close(out.cpu(), want.to(torch.bfloat16), floor=1e-3, what=f"linear random case {case}")


def test_linear_strided_views(gpu):
    """Rows taken from wider buffers (x a column slice, out a slice of a fused output), as the
    decode step passes views of its fused projections."""
    rows, n, k = 4, 512, 4096
    _say("linear strided views")
    g = torch.Generator().manual_seed(3)
    xb = torch.randn(rows, k + 64, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16)
    ob = torch.zeros(rows, 3 * n, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(xb.to(gpu)[:, 64:], w.to(gpu), ob[:, n:2 * n])
    torch.cuda.synchronize()
    o = ob.cpu()
    assert_bf16_close(o[:, n:2 * n], _ref(xb[:, 64:], w), floor=1e-4, what="linear views")
    assert not o[:, :n].any() and not o[:, 2 * n:].any(), "wrote outside the output slice"


def test_linear_rejects(gpu):
    w = torch.zeros(8, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError):  # more rows than the skinny kernel takes
        shadowkv.linear(torch.zeros(17, 64, dtype=torch.bfloat16, device=gpu), w,
                        torch.empty(17, 8, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError):
        shadowkv.linear(torch.zeros(2, 32, dtype=torch.bfloat16, device=gpu), w,
                        torch.empty(2, 8, dtype=torch.bfloat16, device=gpu))


@pytest.mark.parametrize("rows,n,k", [(4, 4096, 14336), (4, 4096, 13696), (1, 4096, 14336), (3, 130, 1032),
                                      (2, 64, 8)])
def test_linear_silu_mul_equals_the_two_kernels(gpu, rows, n, k):
    """The down projection reading the gate/up output through SiLU-and-mul gives, bit for bit,
    silu_and_mul followed by linear (same activation arithmetic and rounding, same sums)."""
    _say(f"linear_silu_mul rows={rows} n={n} k={k}")
    g = torch.Generator().manual_seed(rows * 131 + n + k)
    gu = (torch.randn(rows, 1, 2 * k, generator=g) * 2).to(torch.bfloat16).to(gpu)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(torch.bfloat16).to(gpu)
    act = torch.empty(rows, 1, k, dtype=torch.bfloat16, device=gpu)
    shadowkv.silu_and_mul(gu, act)
    want = torch.empty(rows, 1, n, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(act, w, want)
    got = torch.full((rows, 1, n), 7.0, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear_silu_mul(gu, w, got)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())
    ref = (torch.nn.functional.silu(gu.float()[..., :k]).to(torch.bfloat16).float() * gu.float()[..., k:]).to(
        torch.bfloat16)
    assert_bf16_close(got.cpu(), _ref(ref.cpu(), w.cpu()), floor=1e-3, what=f"linear_silu_mul {rows}x{n}x{k}")


def test_linear_silu_mul_rejects_more_than_four_rows(gpu):
    """The gated form is offered for at most 4 rows: the shim refuses more, and so does the C ABI."""
    from shadowkv_amd import _lib
    k, n = 64, 8
    gu = torch.zeros(5, 2 * k, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(5, n, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        shadowkv.linear_silu_mul(gu, w, out)
    rc = _lib.lib().skv_linear_silu_mul(gu.data_ptr(), 2 * k, w.data_ptr(), k, out.data_ptr(), n, 5, n, k, None)
    assert rc == 2  # SKV_EUNSUPPORTED


@pytest.mark.parametrize("rows,f,k", [(4, 14336, 4096), (4, 13696, 4096), (1, 14336, 4096), (8, 13696, 4096),
                                      (3, 65, 1032), (13, 100, 2048), (16, 7, 8)])
def test_linear_gate_up_silu_equals_the_two_kernels(gpu, rows, f, k):
    """The gate/up projection on the interleaved weight with the SiLU-and-mul in its epilogue gives,
    bit for bit, linear on the reference's [gate | up] weight followed by silu_and_mul, at the
    Llama-3-8B and GLM-4-9B MLP shapes and every row count the kernel takes (1, 3, 4, 8, 13, 16);
    output counts that leave a last workgroup part-full (65, 7 gate/up pairs, which the
    SiLU-and-mul kernel does not take) are checked against torch's SiLU of the projections."""
    _say(f"linear_gate_up_silu rows={rows} f={f} k={k}")
    g = torch.Generator().manual_seed(rows * 977 + f + k)
    x = torch.randn(rows, 1, k, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(2 * f, k, generator=g) / k ** 0.5 * 3).to(torch.bfloat16).to(gpu)
    gu = torch.empty(rows, 1, 2 * f, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(x, w, gu)
    w_il = shadowkv.interleave_gate_up(w)
    assert torch.equal(w_il[0::2], w[:f]) and torch.equal(w_il[1::2], w[f:])
    got = torch.full((rows, 1, f), 7.0, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear_gate_up_silu(x, w_il, got)
    if f % 8 == 0:  # the SiLU-and-mul kernel takes rows of multiples of 8
        want = torch.empty(rows, 1, f, dtype=torch.bfloat16, device=gpu)
        shadowkv.silu_and_mul(gu, want)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want.cpu())
    torch.cuda.synchronize()
    # the projections pinned against fp32 torch (one rounding step), the activation against
    # torch's SiLU of the same bf16 projections
    assert_bf16_close(gu.cpu(), _ref(x.cpu(), w.cpu()), floor=1e-4, what=f"gate/up projection {rows}x{f}x{k}")
    gf, uf = gu.cpu().float()[..., :f], gu.cpu().float()[..., f:]
    ref = (torch.nn.functional.silu(gf).to(torch.bfloat16).float() * uf).to(torch.bfloat16)
    assert_bf16_close(got.cpu(), ref, floor=1e-3, what=f"linear_gate_up_silu {rows}x{f}x{k}")


def test_linear_gate_up_silu_rejects_odd_rows(gpu):
    from shadowkv_amd import _lib
    k, n = 64, 9
    x = torch.zeros(2, k, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(2, 8, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        shadowkv.linear_gate_up_silu(x, w, out)
    rc = _lib.lib().skv_linear_gate_up_silu(x.data_ptr(), k, w.data_ptr(), k, out.data_ptr(), 8, 2, n, k, None)
    assert rc == 1  # SKV_EINVAL
