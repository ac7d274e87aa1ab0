"""GPU tests of the fused input norm (sdm_rt_rms_norm, sdm_rt_add_rms_norm) against the torch RMSNorm the module
mirrors (track4_sdmllm_models.py:63-71): x * rsqrt(mean(x^2) + eps), cast to x's dtype, times w, cast to the output
dtype; and of SwiGLU's silu(g) * u kernel (sdm_rt_silu_mul) against torch's ops (track4_sdmllm_models.py:89-97).

The kernel sums the squares in a different order than torch's mean, so the float32 scale can differ in its last
bit; a bfloat16 output may differ by up to two units in its last place (the intermediate cast to the input dtype can
round the other way) with at least 95% of the values identical, and a float32 one within 2e-6 relative."""
import pytest
import torch

from sdmchat_amd import core
from sdmchat_amd.runtime_sdm import RMSNorm
from tests._gpu_util import say

pytestmark = pytest.mark.gpu


def _ref(x, w, eps, out_dtype):
    n = RMSNorm(x.shape[-1], eps).to(x.device)
    with torch.no_grad():
        n.w.copy_(w)
        return n(x).to(out_dtype)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                          (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32)])
def test_rms_norm_matches_module(in_dt, out_dt):
    g = torch.Generator(device="cpu").manual_seed(7)
    x = (torch.randn(3, 37, 768, generator=g) * 3).to(in_dt).cuda()
    w = (1 + 0.1 * torch.randn(768, generator=g)).cuda()
    say("rms_norm", in_dt, out_dt)
    got = core.rms_norm(x, w, 1e-6, out_dtype=out_dt)
    want = _ref(x, w, 1e-6, out_dt)
    assert got.dtype == out_dt and got.shape == x.shape
    if out_dt == torch.bfloat16:
        diff = (got.float() - want.float()).abs()
        bound = want.float().abs() * 2.0 ** -6   # two bf16 ulps: the cast in the middle can round the other way
        assert bool((diff <= bound).all()), f"max excess {float((diff - bound).max())}"
        assert float((got.float() == want.float()).float().mean()) > 0.95
    else:
        torch.testing.assert_close(got.float(), want.float(), rtol=2e-6, atol=1e-7)


def test_rms_norm_strided_rows_and_small_d():
    g = torch.Generator(device="cpu").manual_seed(8)
    base = torch.randn(50, 80, generator=g).cuda()
    x = base[:, 8:72]                     # rows with stride 80
    w = torch.rand(64, generator=g).cuda()
    got = core.rms_norm(x, w, 1e-5)
    want = _ref(x, w, 1e-5, torch.float32)
    torch.testing.assert_close(got, want, rtol=3e-7, atol=1e-7)
    assert core.rms_norm(torch.empty(0, 64, device="cuda"), w).shape == (0, 64)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                          (torch.bfloat16, torch.float32)])
def test_add_rms_norm_matches_add_then_norm(in_dt, out_dt):
    """The residual add and the next norm in one kernel: the sum is x + y exactly as torch rounds it, and the norm
    of that sum is the kernel's own rms_norm of it, bit for bit (one kernel body)."""
    g = torch.Generator(device="cpu").manual_seed(9)
    x = (torch.randn(5, 33, 1024, generator=g) * 2).to(in_dt).cuda()
    y = torch.randn(5, 33, 1024, generator=g).to(in_dt).cuda()
    w = (1 + 0.1 * torch.randn(1024, generator=g)).cuda()
    say("add_rms_norm", in_dt, out_dt)
    want_s = x + y
    want = core.rms_norm(want_s, w, 1e-6, out_dtype=out_dt)
    s, got = core.add_rms_norm(x.clone(), y, w, 1e-6, out_dtype=out_dt)
    assert torch.equal(s, want_s)
    assert torch.equal(got, want)
    x2 = x.clone()
    s2, _ = core.add_rms_norm(x2, y, w, 1e-6, out_dtype=out_dt, inplace=True)
    assert s2.data_ptr() == x2.data_ptr() and torch.equal(x2, want_s)
    s3, _ = core.add_rms_norm(x, y, w, 1e-6, out_dtype=out_dt, inplace=False)
    assert s3.data_ptr() != x.data_ptr() and torch.equal(s3, want_s)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_silu_mul_matches_torch(dt):
    """silu(g) * u on the halves of a fused projection against torch's F.silu(g) * u: the same roundings, so equal
    up to the last bit of exp (at most one unit in the last place, in under 1% of the values)."""
    g = torch.Generator(device="cpu").manual_seed(10)
    gu = (torch.randn(7, 29, 2 * 1536, generator=g) * 3).to(dt).cuda()
    say("silu_mul", dt)
    got = core.silu_mul(gu)
    want = torch.nn.functional.silu(gu[..., :1536]) * gu[..., 1536:]
    assert got.shape == want.shape and got.dtype == dt
    same = got == want
    assert float(same.float().mean()) > 0.99
    ulp = 2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -23
    diff = (got.float() - want.float()).abs()
    assert bool((diff <= want.float().abs() * ulp * 1.01 + 1e-30).all())
    assert core.silu_mul(torch.empty(0, 16, dtype=dt, device="cuda")).shape == (0, 8)
