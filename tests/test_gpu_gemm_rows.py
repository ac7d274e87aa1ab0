"""GPU tests of sdm_rt_gemm_rows (core.linear for a few bfloat16 rows: a decode step's projections, F.linear in the
reference, track4_onesdm_models.py:199-207, :247, :443-455) against the float32 product of the same bfloat16 inputs:
the kernel sums in float32 (in another order than a GEMM library) and rounds once, with the bias, to bfloat16, so
every value is within one bfloat16 unit of the float32 product rounded, and nearly all equal it."""
import pytest
import torch

from sdmchat_amd import core
from tests._gpu_util import say

pytestmark = pytest.mark.gpu


def _ref(x, w, b):
    y = x.float() @ w.float().t()
    if b is not None:
        y = y + b.float()
    return y


@pytest.mark.parametrize("rows,n,k,bias", [(64, 2560, 768, True), (64, 768, 768, False), (1, 768, 768, True),
                                           (37, 4096, 768, False), (100, 768, 2048, False), (256, 32768, 768, False),
                                           (5, 96, 128, True)])
def test_gemm_rows_matches_float32_product(rows, n, k, bias):
    g = torch.Generator(device="cpu").manual_seed(rows * 7 + n + k)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16).cuda()
    b = torch.randn(n, generator=g).to(torch.bfloat16).cuda() if bias else None
    say("gemm_rows", rows, n, k, bias)
    with torch.no_grad():
        got = core.linear(x, w, b)
    want = _ref(x, w, b)
    assert got.dtype == torch.bfloat16 and got.shape == (rows, n)
    diff = (got.float() - want).abs()
    assert bool((diff <= want.abs() * 2.0 ** -7 + 1e-6).all()), float((diff - want.abs() * 2.0 ** -7).max())
    assert float((got == want.to(torch.bfloat16)).float().mean()) > 0.97


def test_gemm_rows_strided_rows_batched_shape_and_determinism():
    g = torch.Generator(device="cpu").manual_seed(3)
    base = torch.randn(8, 3, 1024, generator=g).to(torch.bfloat16).cuda()
    x = base[:, 1, 128:896]                  # rows 3 * 1024 apart, 16-byte aligned
    w = (torch.randn(768, 768, generator=g) * 0.04).to(torch.bfloat16).cuda()
    with torch.no_grad():
        y1 = core.linear(x, w, as_matmul=True)
        y2 = core.linear(x.contiguous()[None], w, as_matmul=True)[0]
    assert torch.equal(y1, y2)
    d = (y1.float() - _ref(x, w, None)).abs()
    assert bool((d <= _ref(x, w, None).abs() * 2.0 ** -7 + 1e-6).all())


def test_gemm_rows_leaves_other_products_to_the_library():
    x = torch.randn(300, 768, device="cuda").to(torch.bfloat16)   # more rows than the kernel takes
    w = torch.randn(64, 768, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        assert torch.equal(core.linear(x, w), torch.nn.functional.linear(x, w))
    wr = w.clone().requires_grad_(True)                            # autograd recording: the library's product
    y = core.linear(x[:8], wr)
    assert y.grad_fn is not None


def _gemm_rows(x, w, b=None):
    """sdm_rt_gemm_rows called directly (any row count: the kernel the launcher picks for the shape)."""
    import ctypes
    from sdmchat_amd import _lib
    lib = _lib.load()
    y = torch.empty(x.shape[0], w.shape[0], dtype=torch.bfloat16, device=x.device)
    p = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)   # noqa: E731
    rc = lib.sdm_rt_gemm_rows(p(x), x.stride(0), p(w), w.stride(0), p(b), p(y), y.stride(0), x.shape[0], w.shape[0],
                              x.shape[1], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, lib)
    return y


def test_gemm_rows_kernels_give_the_same_bits():
    """k = 768: the launcher takes tiles of 16 rows while they fit the compute units at once and of 32 rows past that
    (few column tiles: <= 256 of 64 rows x 32 columns), the walking kernel for wide maps (the tied head) and the
    general 64-row kernel past 256 row tiles; all sum every element in the same order, so a product's bits do not
    depend on which one ran."""
    g = torch.Generator(device="cpu").manual_seed(11)
    x = torch.randn(16448, 768, generator=g).to(torch.bfloat16).cuda()          # 257 tiles of 64 rows
    w = (torch.randn(8224, 768, generator=g) * 0.04).to(torch.bfloat16).cuda()  # 257 column tiles
    b = torch.randn(8224, generator=g).to(torch.bfloat16).cuda()
    say("gemm_rows kernels: 16- and 32-row tiles, wide walk, general")
    with torch.no_grad():
        narrow = _gemm_rows(x[:64], w[:64], b[:64])        # 2 column tiles: 16-row tiles
        narrow32 = _gemm_rows(x[:64], w[:2560], b[:2560])  # 80 column tiles: 32-row tiles
        general = _gemm_rows(x, w[:64], b[:64])            # 257 row tiles: the general kernel
        wide = _gemm_rows(x[:64], w, b)                    # 257 column tiles: the walking kernel, 256 columns
        wide200 = _gemm_rows(x[:200], w, b)                # 4 row tiles: 64 columns, each walking ~4 tiles
        narrow200 = _gemm_rows(x[:200], w[4096:4160], b[4096:4160])
        torch.cuda.synchronize()
    assert torch.equal(general[:64].view(torch.int16), narrow.view(torch.int16))
    assert torch.equal(wide[:, :64].view(torch.int16), narrow.view(torch.int16))
    assert torch.equal(wide[:, :2560].view(torch.int16), narrow32.view(torch.int16))
    assert torch.equal(wide200[:64].view(torch.int16), wide.view(torch.int16))
    assert torch.equal(wide200[:, 4096:4160].view(torch.int16), narrow200.view(torch.int16))
    want = _ref(x[:200], w, b)
    d = (wide200.float() - want).abs()
    assert bool((d <= want.abs() * 2.0 ** -7 + 1e-6).all())


@pytest.mark.parametrize("rows,n,bias", [(64, 2560, True), (1, 2560, True), (5, 768, False), (37, 2560, True),
                                         (100, 768, False), (192, 2560, True)])
def test_gemm_rows_residual_equals_add_norm_then_gemm_rows(rows, n, bias):
    """sdm_rt_gemm_rows_residual (the residual add and the next mixer's input norm folded into its projection map)
    against sdm_rt_add_rms_norm followed by sdm_rt_gemm_rows on the same inputs: the sums and the products bit for
    bit, x and y untouched."""
    g = torch.Generator(device="cpu").manual_seed(rows * 3 + n)
    x = torch.randn(rows, 768, generator=g).to(torch.bfloat16).cuda()
    y = (torch.randn(rows, 768, generator=g) * 0.5).to(torch.bfloat16).cuda()
    nw = (torch.rand(768, generator=g) + 0.5).cuda()
    w = (torch.randn(n, 768, generator=g) * 0.04).to(torch.bfloat16).cuda()
    b = torch.randn(n, generator=g).to(torch.bfloat16).cuda() if bias else None
    x0, y0 = x.clone(), y.clone()
    say("gemm_rows_residual", rows, n, bias)
    with torch.no_grad():
        assert core.linear_residual_fits(x, y, w, b)
        s1, o1 = core.linear_residual(x, y, nw, 1e-6, w, b)
        s0, hx = core.add_rms_norm(x, y, nw, 1e-6, out_dtype=torch.bfloat16, inplace=False)
        o0 = core.linear(hx, w, b)
        torch.cuda.synchronize()
    assert torch.equal(x, x0) and torch.equal(y, y0)
    assert torch.equal(s1.view(torch.int16), s0.view(torch.int16))
    assert torch.equal(o1.view(torch.int16), o0.view(torch.int16))


@pytest.mark.parametrize("rows,n,bias", [(64, 2560, True), (64, 768, False), (1, 2560, True), (37, 768, True),
                                         (192, 2560, False)])
def test_gemm_rows_embed_equals_gather_norm_then_gemm_rows(rows, n, bias):
    """sdm_rt_gemm_rows_embed (the embedding gather and the first mixer's input norm folded into its projection map)
    against the gather, sdm_rt_rms_norm and sdm_rt_gemm_rows on the same tokens: the gathered rows and the products
    bit for bit, with repeated tokens and the table's first and last rows among them."""
    g = torch.Generator(device="cpu").manual_seed(rows * 5 + n)
    vocab = 1000
    table = torch.randn(vocab, 768, generator=g).to(torch.bfloat16).cuda()
    idx = torch.randint(0, vocab, (rows,), generator=g)
    idx[: min(rows, 3)] = torch.tensor([0, vocab - 1, 0])[: min(rows, 3)]
    idx = idx.cuda()
    nw = (torch.rand(768, generator=g) + 0.5).cuda()
    w = (torch.randn(n, 768, generator=g) * 0.04).to(torch.bfloat16).cuda()
    b = torch.randn(n, generator=g).to(torch.bfloat16).cuda() if bias else None
    say("gemm_rows_embed", rows, n, bias)
    with torch.no_grad():
        assert core.linear_embed_fits(idx, table, w, b)
        x1, o1 = core.linear_embed(idx, table, nw, 1e-6, w, b)
        x0 = table[idx]
        hx = core.rms_norm(x0, nw, 1e-6, out_dtype=torch.bfloat16)
        o0 = core.linear(hx, w, b)
        torch.cuda.synchronize()
    assert torch.equal(x1.view(torch.int16), x0.view(torch.int16))
    assert torch.equal(o1.view(torch.int16), o0.view(torch.int16))


def test_gemm_rows_embed_clamps_tokens_outside_the_table():
    """A token below 0 or past the table reads the table's first or last row (the kernel's own bounds check; the host
    never reads the tokens), as the clamped tokens do."""
    g = torch.Generator(device="cpu").manual_seed(12)
    vocab = 50
    table = torch.randn(vocab, 768, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(64, 768, generator=g) * 0.04).to(torch.bfloat16).cuda()
    nw = torch.ones(768).cuda()
    idx = torch.tensor([-3, vocab + 7, 5, vocab - 1, 0], device="cuda")
    with torch.no_grad():
        x1, o1 = core.linear_embed(idx, table, nw, 1e-6, w)
        x0, o0 = core.linear_embed(idx.clamp(0, vocab - 1), table, nw, 1e-6, w)
        torch.cuda.synchronize()
    assert torch.equal(x1, x0) and torch.equal(o1, o0)
    assert torch.equal(x1[0], table[0]) and torch.equal(x1[1], table[vocab - 1])


def test_gemm_rows_residual_declines_large_maps():
    """More than 256 tiles of 64 rows x 32 columns: linear_residual_fits says no, and the entry point returns
    SDM_RT_EUNSUPPORTED without launching."""
    from sdmchat_amd import _lib
    x = torch.zeros(193, 768, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(2560, 768, dtype=torch.bfloat16, device="cuda")
    assert not core.linear_residual_fits(x, x.clone(), w)
    assert core.linear_residual_fits(x[:192], x[:192].clone(), w)
    with pytest.raises(_lib.SdmRtError):
        core.linear_residual(x, x.clone(), torch.ones(768, device="cuda"), 1e-6, w)
