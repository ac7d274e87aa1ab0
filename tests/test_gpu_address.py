"""GPU parity of the product-key addressing kernel (sdm_rt_address) against the golden vectors and the fp64 oracle.

References: pk_address (track4_onesdm_models.py:134-148), softmax weights and gate (:203-207).  Picks, in order,
must be identical to the reference's (and the oracle's) except where two slots' fp64 scores are within 2.4e-7 (a
float32-level tie; the counts are printed); at exact ties the kernels keep the lowest index.
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from tests._gpu_util import bf16_round, gpu_address, pick_diffs, say, valid_picks

pytestmark = pytest.mark.gpu


def _params(g, H):
    return dict(keys1=g["keys1"], keys2=g["keys2"], addr_b=np.zeros((H, g["z"].shape[-1]), np.float32),
                log_scale=np.full(H, np.log(8.0), np.float32), decay=np.zeros(H, np.float32),
                onorm_w=np.ones((H, 8), np.float32), gate_bias=np.zeros(H, np.float32))


def _as_tokens(a):
    """(B, H, T, kk) -> (B*T, H, kk)."""
    B, H, T, kk = a.shape
    return a.transpose(0, 2, 1, 3).reshape(B * T, H, kk)


@pytest.mark.parametrize("name", ["layer", "default16", "tiny6", "selftest9", "k_gt_nsub", "all_picked", "ties",
                                  "sign_halves"])
def test_golden_vectors(golden, name):
    g = golden[name]
    N, H, d_a = g["z"].shape
    k = int(g["k"])
    say("golden", name, g["z"].shape, "k", k)
    slots, scores, _ = gpu_address(g["z"].reshape(1, N, H * d_a), _params(g, H), k)
    si, sv = _as_tokens(slots), _as_tokens(scores)
    assert si.shape == g["si"].shape
    n = int(pick_diffs(g["z"], g["keys1"].astype(np.float64), g["keys2"].astype(np.float64), g["si"], si).sum())
    say(f"  {n} of {N * H} addresses differ from the reference's picks (all at ties)")
    # near a tie any equally good pick set is valid; where every score is exactly 0 (a zero address) the kernel's
    # lowest-index rule picks slots 0..kk-1
    assert np.all(valid_picks(g["z"], g["keys1"], g["keys2"], k, si))
    zero = np.all(g["z"] == 0, -1)
    if zero.any():
        assert np.all(si[zero] == np.arange(si.shape[-1]))
    np.testing.assert_allclose(sv, g["sv"], atol=3e-7, rtol=0)
    assert np.all(np.diff(sv, axis=-1) <= 0)


def test_bf16_addresses_match_oracle_on_the_same_values():
    rng = np.random.Generator(np.random.PCG64(31))
    H, n_sub, d_a, B, T = 12, 32, 64, 2, 300
    z = bf16_round(rng.standard_normal((B, T, H * d_a)))
    p = dict(keys1=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             keys2=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             addr_b=(rng.standard_normal((H, d_a)) * 0.3).astype(np.float32),
             log_scale=rng.uniform(1.5, 2.5, H).astype(np.float32), decay=np.zeros(H, np.float32),
             onorm_w=np.ones((H, 8), np.float32), gate_bias=rng.uniform(-1, 1, H).astype(np.float32))
    gate = bf16_round(rng.standard_normal((B, T, H)))
    slots, scores, weights = gpu_address(z, p, 8, dtype=torch.bfloat16, gate=gate)
    zz = z.astype(np.float64).reshape(B * T, H, d_a) + p["addr_b"]
    sv, si = O.pk_address(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), 8)
    gsi = _as_tokens(slots)
    same = ~pick_diffs(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), si, gsi)
    say(f"bf16 addresses: {int((~same).sum())} of {same.size} differ from the oracle's picks (all at ties)")
    np.testing.assert_allclose(_as_tokens(scores), sv, atol=3e-7)
    gl = gate.astype(np.float64).reshape(B * T, H) + p["gate_bias"]
    w = O.address_weights(sv, p["log_scale"].astype(np.float64), O.sigmoid(gl))
    np.testing.assert_allclose(_as_tokens(weights)[same], w[same], atol=2e-6, rtol=2e-6)


def test_full_bench_shape_picks():
    """All 2 x 196,608 addresses of the B=8, T=2048, H=12 workload (bf16 inputs) against the fp64 oracle."""
    rng = np.random.Generator(np.random.PCG64(32))
    H, n_sub, d_a, B, T = 12, 32, 64, 8, 2048
    p = dict(keys1=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             keys2=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             addr_b=np.zeros((H, d_a), np.float32), log_scale=np.full(H, np.log(8.0), np.float32),
             decay=np.zeros(H, np.float32), onorm_w=np.ones((H, 8), np.float32), gate_bias=np.zeros(H, np.float32))
    z = bf16_round(rng.standard_normal((B, T, H * d_a)))
    say("bench-shape addressing", z.shape)
    slots, scores, _ = gpu_address(z, p, 8, dtype=torch.bfloat16)
    zz = z.astype(np.float64).reshape(B * T, H, d_a)
    sv, si = O.pk_address(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), 8)
    gsi = _as_tokens(slots)
    diff = pick_diffs(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), si, gsi)
    say("addresses whose picks differ from the oracle's (all at ties):", int(diff.sum()), "of", diff.size)
    np.testing.assert_allclose(_as_tokens(scores), sv, atol=3e-7)


@pytest.mark.parametrize("n_sub,k,H,half", [(64, 16, 1, 16), (64, 8, 2, 16), (48, 12, 2, 16), (40, 16, 3, 8),
                                            (64, 16, 2, 32)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_64_subkey_addressing_matches_oracle(n_sub, k, H, half, dtype):
    """More than 32 sub-keys per half (the TrainedSdm table of the FULL model: 64, k 16) on the matrix cores, two
    sub-key tiles per half: picks in the oracle's order up to ties, scores and weights."""
    rng = np.random.Generator(np.random.PCG64(60 + n_sub + k))
    B, T, d_a = 2, 150, 2 * half
    z = bf16_round(rng.standard_normal((B, T, H * d_a)))
    p = dict(keys1=rng.standard_normal((H, n_sub, half)).astype(np.float32),
             keys2=rng.standard_normal((H, n_sub, half)).astype(np.float32),
             addr_b=(rng.standard_normal((H, d_a)) * 0.3).astype(np.float32),
             log_scale=rng.uniform(1.5, 2.5, H).astype(np.float32), decay=np.zeros(H, np.float32),
             onorm_w=np.ones((H, 8), np.float32), gate_bias=np.zeros(H, np.float32))
    say("64-sub-key addressing", n_sub, k, H, half, dtype)
    slots, scores, weights = gpu_address(z, p, k, dtype=dtype)
    zz = z.astype(np.float64).reshape(B * T, H, d_a) + p["addr_b"]
    k1, k2 = p["keys1"].astype(np.float64), p["keys2"].astype(np.float64)
    sv, si = O.pk_address(zz, k1, k2, k)
    gsi = _as_tokens(slots)
    same = ~pick_diffs(zz, k1, k2, si, gsi)
    say(f"  {int((~same).sum())} of {same.size} addresses differ from the oracle's picks (all at ties)")
    np.testing.assert_allclose(_as_tokens(scores), sv, atol=1e-6)
    w = O.address_weights(sv, p["log_scale"].astype(np.float64))
    np.testing.assert_allclose(_as_tokens(weights)[same], w[same], atol=2e-6, rtol=2e-6)


@pytest.mark.parametrize("n_sub,d_a,k,H,addr_bias,dtype", [(32, 64, 8, 12, 0.0, torch.bfloat16),
                                                           (32, 64, 8, 12, 0.0, torch.float32),
                                                           (64, 32, 16, 1, 0.0, torch.bfloat16),
                                                           (64, 32, 16, 1, 0.0, torch.float32),
                                                           (20, 32, 12, 3, 0.4, torch.bfloat16),
                                                           (48, 16, 8, 2, 0.4, torch.float32)])
def test_few_token_split_path_equals_wave_path(n_sub, d_a, k, H, addr_bias, dtype):
    """Up to 1,024 tokens the addressing splits every address over the block's waves (one per half and sub-key tile,
    then a wave for the grid: a decode step's path); beyond, one wave addresses 64 tokens.  The same tokens give the
    same picks, weights and scores, bit for bit, on both paths (32 and 64 sub-keys per half, full and masked grids,
    gate and address bias), and the picks agree with the oracle."""
    from tests._gpu_util import core_inputs
    kz, _, _, g, p = core_inputs(1, 1100, H, 8, d_a, n_sub, seed=231 + n_sub, addr_bias=addr_bias)
    if dtype == torch.bfloat16:
        kz, g = bf16_round(kz), bf16_round(g)
    say("split vs wave addressing", n_sub, d_a, k, H, dtype)
    s_all, v_all, w_all = gpu_address(kz, p, k, dtype=dtype, gate=g)                           # 1,100: wave path
    s_few, v_few, w_few = gpu_address(kz[:, :500], p, k, dtype=dtype, gate=g[:, :500])         # 500: split path
    assert np.array_equal(s_few, s_all[:, :, :500])
    assert np.array_equal(w_few, w_all[:, :, :500]) and np.array_equal(v_few, v_all[:, :, :500])
    zz = kz[:, :500].astype(np.float64).reshape(500, H, d_a) + p["addr_b"]
    _, osi = O.pk_address(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), k)
    n = int(pick_diffs(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), osi, _as_tokens(s_few)).sum())
    say(f"  {n} of {500 * H} addresses differ from the oracle (ties)")
