"""Pins the oracle's memory scan and layer forward (CPU only).

References: RunTimeSdm._chunk / forward / forward_sequential / finish (track4_onesdm_models.py:215-300) and the
reference self-test's chunked = sequential, previous-token head and gate checks (:728-792).
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from oracle import sdm_torch32 as R
from sdmchat_amd import synthetic as S


def _distinct_ids(rng, shape, k, M):
    out = np.empty(shape + (k,), np.int64)
    for idx in np.ndindex(*shape):
        out[idx] = rng.choice(M, size=k, replace=False)
    return out


@pytest.mark.parametrize("lams", [(0.0, 0.5, 1.0), (0.9, 0.99, 0.999)])
def test_recurrence_equals_closed_form_double_sum(lams):
    rng = np.random.Generator(np.random.PCG64(21))
    B, H, T, k, M, dh = 2, 3, 14, 3, 7, 5
    siw = _distinct_ids(rng, (B, H, T), k, M)
    sir = _distinct_ids(rng, (B, H, T), k, M)
    ww, wr = rng.random((B, H, T, k)), rng.random((B, H, T, k))
    V = rng.standard_normal((B, H, T, dh))
    lam = np.array(lams)
    num, den, _, _ = O.scan_recurrence(siw, ww, sir, wr, V, lam,
                                       state=(np.zeros((B, H, M, dh)), np.zeros((B, H, M))))
    cn, cd = O.scan_closed_form(siw, ww, sir, wr, V, lam)
    np.testing.assert_allclose(num, cn, atol=1e-12)
    np.testing.assert_allclose(den, cd, atol=1e-12)
    assert np.all(num[:, :, 0] == 0) and np.all(den[:, :, 0] == 0)


def test_rescaled_recurrence_equals_recurrence():
    """The fade carried as one factor per head (scan_recurrence_rescaled, what the bench-shape GPU test runs over
    all 96 slabs) gives scan_recurrence's values: random picks, repeated slots, fades from 0.5 to 1 over 900 steps
    (0.5^900 = 1e-271: the factor is folded into the memory several times), with and without resets, and a fade of 0
    is refused."""
    rng = np.random.Generator(np.random.PCG64(31))
    B, H, T, k, M, dh = 2, 4, 900, 4, 24, 6
    siw = _distinct_ids(rng, (B, H, T), k, M)
    sir = _distinct_ids(rng, (B, H, T), k, M)
    ww, wr = rng.random((B, H, T, k)), rng.random((B, H, T, k))
    V = rng.standard_normal((B, H, T, dh))
    lam = np.array([0.5, 0.9, 0.999, 1.0])
    num, den, _, _ = O.scan_recurrence(siw, ww, sir, wr, V, lam,
                                       state=(np.zeros((B, H, M, dh)), np.zeros((B, H, M))))
    n2, d2 = O.scan_recurrence_rescaled(siw, ww, sir, wr, V, lam)
    np.testing.assert_allclose(n2, num, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(d2, den, rtol=1e-10, atol=1e-14)
    with pytest.raises(ValueError):
        O.scan_recurrence_rescaled(siw, ww, sir, wr, V, np.array([0.0, 0.9, 0.9, 0.9]))
    reset = np.zeros((B, T), bool)
    reset[0, [0, 17, 18, 400]] = True
    reset[1, [899]] = True
    num, den, _, _ = O.scan_recurrence(siw, ww, sir, wr, V, lam, state=(np.zeros((B, H, M, dh)), np.zeros((B, H, M))),
                                       reset=reset)
    n3, d3 = O.scan_recurrence_rescaled(siw, ww, sir, wr, V, lam, reset=reset)
    np.testing.assert_allclose(n3, num, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(d3, den, rtol=1e-10, atol=1e-14)


def test_recurrence_state_carry_is_the_same_as_one_pass():
    rng = np.random.Generator(np.random.PCG64(22))
    B, H, T, k, M, dh = 1, 2, 20, 2, 9, 4
    siw = _distinct_ids(rng, (B, H, T), k, M)
    sir = _distinct_ids(rng, (B, H, T), k, M)
    ww, wr = rng.random((B, H, T, k)), rng.random((B, H, T, k))
    V = rng.standard_normal((B, H, T, dh))
    lam = np.array([0.7, 1.0])
    z = (np.zeros((B, H, M, dh)), np.zeros((B, H, M)))
    n_all, d_all, m_all, c_all = O.scan_recurrence(siw, ww, sir, wr, V, lam, state=z)
    n1, d1, m1, c1 = O.scan_recurrence(siw[:, :, :8], ww[:, :, :8], sir[:, :, :8], wr[:, :, :8], V[:, :, :8], lam,
                                       state=z)
    n2, d2, m2, c2 = O.scan_recurrence(siw[:, :, 8:], ww[:, :, 8:], sir[:, :, 8:], wr[:, :, 8:], V[:, :, 8:], lam,
                                       state=(m1, c1))
    np.testing.assert_allclose(np.concatenate([n1, n2], 2), n_all, atol=1e-12)
    np.testing.assert_allclose(m2, m_all, atol=1e-12)
    np.testing.assert_allclose(c2, c_all, atol=1e-12)



def test_reset_empties_the_memory_before_the_read():
    """A reset at position t (OM:287-289) equals a fresh recurrence started at t from an empty memory, computed
    independently on the segment; rows without a reset are unaffected."""
    rng = np.random.Generator(np.random.PCG64(24))
    B, H, T, k, M, dh = 3, 2, 30, 3, 10, 4
    siw = _distinct_ids(rng, (B, H, T), k, M)
    sir = _distinct_ids(rng, (B, H, T), k, M)
    ww, wr = rng.random((B, H, T, k)), rng.random((B, H, T, k))
    V = rng.standard_normal((B, H, T, dh))
    lam = np.array([0.8, 1.0])
    z = (np.zeros((B, H, M, dh)), np.zeros((B, H, M)))
    reset = np.zeros((B, T), bool)
    reset[0, 11] = True
    reset[2, 0] = True
    reset[2, 25] = True
    num, den, mem, cnt = O.scan_recurrence(siw, ww, sir, wr, V, lam, state=z, reset=reset)
    n0, d0, _, _ = O.scan_recurrence(siw, ww, sir, wr, V, lam, state=z)
    np.testing.assert_array_equal(num[1], n0[1])                        # no reset in row 1
    np.testing.assert_array_equal(num[0, :, :11], n0[0, :, :11])        # row 0 before its reset
    zr = (np.zeros((1, H, M, dh)), np.zeros((1, H, M)))
    sl = np.s_[0:1, :, 11:]
    ns, ds, ms, cs = O.scan_recurrence(siw[sl], ww[sl], sir[sl], wr[sl], V[sl], lam, state=zr)
    np.testing.assert_allclose(num[0:1, :, 11:], ns, atol=1e-12)
    np.testing.assert_allclose(den[0:1, :, 11:], ds, atol=1e-12)
    np.testing.assert_allclose(mem[0:1], ms, atol=1e-12)
    assert np.all(num[0, :, 11] == 0) and np.all(den[0, :, 11] == 0)   # the reset position reads an empty memory
    sl = np.s_[2:3, :, 25:]
    ns, _, ms, cs = O.scan_recurrence(siw[sl], ww[sl], sir[sl], wr[sl], V[sl], lam, state=zr)
    np.testing.assert_allclose(num[2:3, :, 25:], ns, atol=1e-12)
    np.testing.assert_allclose(cnt[2:3], cs, atol=1e-12)

def _small_layer(seed=3, **over):
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8, **over)
    p = S.layer_params(cfg, seed=seed, decays=(0.0, 0.6, 0.97, 1.0))
    return cfg, p


def _p64(p):
    q = {k: v.astype(np.float64) for k, v in p.items()}
    q["decay"] = q["decays_fixed"]
    return q


@pytest.mark.parametrize("chunk", [1, 5, 7, 23, 64, 128, 77])
def test_torch_chunked_equals_fp64_recurrence(chunk):
    cfg, p = _small_layer()
    x = S.layer_input(2, 77, 64, seed=4)
    pt = {k: torch.from_numpy(v) for k, v in p.items()}
    y32 = R.forward(torch.from_numpy(x), pt, cfg, chunk=chunk).numpy()
    y64 = O.layer_forward(x, _p64(p), cfg)
    np.testing.assert_allclose(y32, y64, atol=1e-5, rtol=1e-4)


def test_torch_sequential_equals_fp64():
    cfg, p = _small_layer(seed=5)
    x = S.layer_input(1, 40, 64, seed=6)
    pt = {k: torch.from_numpy(v) for k, v in p.items()}
    np.testing.assert_allclose(R.forward_sequential(torch.from_numpy(x), pt, cfg).numpy(),
                               O.layer_forward(x, _p64(p), cfg), atol=1e-5, rtol=1e-4)


def test_previous_token_head_closed_form():
    """Fade 0, zero key/query maps: every token addresses the same k locations; position t reads exactly what t-1
    wrote through the mean read: y[t] = V[t-1] * (1/k) / (1/k + eps), y[0] = 0 (reference self-test :773-785)."""
    cfg = S.layer_cfg(d=8, heads=1, n_sub=4, d_a=4, k=4, write_gate=False, out_norm=False)
    p = S.layer_params(cfg, seed=7, decays=(0.0,))
    p["wk.weight"][:] = 0
    p["wq.weight"][:] = 0
    p["wo.weight"] = np.eye(8, dtype=np.float32)
    x = S.layer_input(1, 9, 8, seed=8)
    y = O.layer_forward(x, _p64(p), cfg)
    hx = O.rms_norm(x, np.ones(8))
    V = hx @ p["wv.weight"].T.astype(np.float64)
    want = V[0, :-1] * 0.25 / (0.25 + 1e-3)
    np.testing.assert_allclose(y[0, 1:], want, atol=1e-12)
    assert np.all(y[0, 0] == 0)


def test_never_fading_head_is_a_running_mean():
    """Fade 1 with one shared address: r[t] = (sum_{s<t} V_s / k) / (t / k + eps)."""
    cfg = S.layer_cfg(d=8, heads=1, n_sub=4, d_a=4, k=4, write_gate=False, out_norm=False)
    p = S.layer_params(cfg, seed=9, decays=(1.0,))
    p["wk.weight"][:] = 0
    p["wq.weight"][:] = 0
    p["wo.weight"] = np.eye(8, dtype=np.float32)
    x = S.layer_input(1, 12, 8, seed=10)
    y = O.layer_forward(x, _p64(p), cfg)
    V = O.rms_norm(x, np.ones(8)) @ p["wv.weight"].T.astype(np.float64)
    csum = np.cumsum(V[0], 0)
    t = np.arange(1, 12)[:, None]
    np.testing.assert_allclose(y[0, 1:], (csum[:-1] / 4) / (t / 4 + 1e-3), atol=1e-12)


def test_gate_near_zero_gives_zero_reads():
    cfg, p = _small_layer(seed=11)
    p["wg.weight"][:] = 0
    p["wg.bias"][:] = -30.0
    x = S.layer_input(1, 30, 64, seed=12)
    y = O.layer_forward(x, _p64(p), dict(cfg, out_norm=False))
    assert np.abs(y).max() < 1e-6


def test_zero_output_map_gives_exact_zero():
    cfg, p = _small_layer(seed=13)
    p["wo.weight"][:] = 0
    x = S.layer_input(1, 30, 64, seed=14)
    assert np.all(O.layer_forward(x, _p64(p), cfg) == 0)


def test_finish_closed_form():
    num = np.array([[[[3.0, 4.0]]]])
    den = np.array([[[1.0]]])
    r = O.finish(num, den, "mean", 0.0, True, np.array([[2.0, 2.0]]), 0.0)
    np.testing.assert_allclose(r[0, 0, 0], np.array([3.0, 4.0]) / np.sqrt(12.5) * 2, rtol=1e-15)
    np.testing.assert_allclose(O.finish(num, den, "sum", 1.0, False), num)


def _closed_variant(siw, ww, sir, wr, V, lam, lag, include_self):
    """The closed-form double sum with a fade exponent of t - lag - s, over s < t (or s <= t)."""
    B, H, T, _ = siw.shape
    num = np.zeros(V.shape)
    for b, h, t in np.ndindex(B, H, T):
        for s in range(t + 1 if include_self else t):
            m = (sir[b, h, t][:, None] == siw[b, h, s][None, :]).astype(np.float64)
            c = float(wr[b, h, t] @ m @ ww[b, h, s]) * lam[h] ** (t - lag - s)
            num[b, h, t] += c * V[b, h, s]
    return num


def test_planted_scan_mistakes_fail_the_closed_form():
    """The recurrence agrees with the closed form, and the closed form tells apart the plausible mistakes: a fade
    exponent off by one, and a read that already sees the current position's write."""
    rng = np.random.Generator(np.random.PCG64(23))
    B, H, T, k, M, dh = 1, 2, 12, 3, 5, 3
    siw = _distinct_ids(rng, (B, H, T), k, M)
    sir = _distinct_ids(rng, (B, H, T), k, M)
    ww, wr = rng.random((B, H, T, k)), rng.random((B, H, T, k))
    V = rng.standard_normal((B, H, T, dh))
    lam = np.array([0.6, 0.9])
    num, _, _, _ = O.scan_recurrence(siw, ww, sir, wr, V, lam, state=(np.zeros((B, H, M, dh)), np.zeros((B, H, M))))
    np.testing.assert_allclose(_closed_variant(siw, ww, sir, wr, V, lam, 1, False), num, atol=1e-12)
    assert np.abs(_closed_variant(siw, ww, sir, wr, V, lam, 0, False) - num).max() > 1e-3
    assert np.abs(_closed_variant(siw, ww, sir, wr, V, lam, 1, True) - num).max() > 1e-3


def test_bf16_rounding_equals_torch_cast():
    """oracle.sdm_fp64.bf16 (the casts of the bfloat16 model restatement) equals torch's float32 -> bfloat16 cast on
    random values, exact ties (round half to even, both directions), values one float32 ulp either side of a tie,
    subnormals, zeros and infinities; float64 inputs round through float32."""
    import torch

    from oracle import sdm_fp64 as O
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-30, 30, 10000),
                        [0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39, 3.0e38]]).astype(np.float32)
    u = rng.integers(0, 2 ** 31, 2000, dtype=np.uint64).astype(np.uint32)
    ties = ((u & 0xFFFF0000) | 0x8000).view(np.float32)           # exactly halfway between two bfloat16 values
    near = np.concatenate([ties, np.nextafter(ties, np.inf), np.nextafter(ties, -np.inf)])
    for v in (x, near[np.isfinite(near)]):
        want = torch.from_numpy(v).to(torch.bfloat16).float().numpy().astype(np.float64)
        got = O.bf16(v)
        assert np.array_equal(got, want) or np.allclose(got, want, rtol=0, atol=0, equal_nan=True)
        assert np.array_equal(np.signbit(got), np.signbit(want))
    d = rng.standard_normal(1000)
    assert np.array_equal(O.bf16(d), torch.from_numpy(d.astype(np.float32)).to(torch.bfloat16).double().numpy())
