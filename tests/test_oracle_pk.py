"""Pins the oracle's product-key addressing (CPU only).

References: pk_address (track4_onesdm_models.py:134-148); its brute-force self-test (:694-702).
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from oracle import sdm_torch32 as R

DELTA = 1e-6   # a pick may differ from another float32 implementation only where the fp64 margin is below this


def test_torch_restatement_is_bit_exact_on_golden(golden):
    torch.set_num_threads(1)
    for name, g in golden.items():
        sv, si = R.pk_address(torch.from_numpy(g["z"]), torch.from_numpy(g["keys1"]), torch.from_numpy(g["keys2"]),
                              int(g["k"]))
        assert np.array_equal(sv.numpy(), g["sv"]), name
        assert np.array_equal(si.numpy(), g["si"].astype(np.int64)), name


def test_fp64_matches_golden_picks_away_from_ties(golden):
    for name, g in golden.items():
        sv, si = O.pk_address(g["z"], g["keys1"], g["keys2"], int(g["k"]))
        margin = O.topk_margin(g["z"], g["keys1"], g["keys2"], int(g["k"]))
        same = np.all(np.sort(si, -1) == np.sort(g["si"], -1), -1)
        assert np.all(same | (margin < DELTA)), name
        np.testing.assert_allclose(sv, g["sv"], atol=3e-7, err_msg=name)


def test_golden_holds_exact_ties_where_reference_order_differs(golden):
    """The reference's topk does not order exactly equal scores by index; the oracle (and the kernels) do."""
    g = golden["ties"]
    sv, si = O.pk_address(g["z"], g["keys1"], g["keys2"], int(g["k"]))
    zero_rows = np.all(g["z"] == 0, -1)          # every score 0: the lowest-index rule picks slots 0..kk-1
    assert zero_rows.any()
    assert np.all(si[zero_rows] == np.arange(8))
    assert not np.all(g["si"][zero_rows] == np.arange(8))


def _rand_case(rng, N, H, half, n_sub):
    return (rng.standard_normal((N, H, 2 * half)), rng.standard_normal((H, n_sub, half)),
            rng.standard_normal((H, n_sub, half)))


@pytest.mark.parametrize("half,n_sub,k", [(32, 32, 8), (16, 32, 16), (4, 6, 5), (6, 9, 5), (4, 4, 8), (3, 2, 8),
                                          (1, 5, 4), (8, 16, 16), (2, 3, 1)])
def test_product_key_equals_bruteforce(half, n_sub, k):
    rng = np.random.Generator(np.random.PCG64(100 + half * 7 + n_sub + k))
    z, k1, k2 = _rand_case(rng, 64, 3, half, n_sub)
    sv, si = O.pk_address(z, k1, k2, k)
    bv, bi = O.pk_address_bruteforce(z, k1, k2, k)
    kk = min(k, min(k, n_sub) ** 2)
    assert si.shape == (64, 3, kk)
    # the picked scores are tie-independent; the picked sets agree wherever no exact tie straddles the cut
    # (with a tie, the product-key form keeps the lowest grid position of the sorted halves, the brute force the
    # lowest slot id: both are "lowest index" rules, at different stages)
    np.testing.assert_allclose(sv, bv, atol=1e-12)
    margin = O.topk_margin(z, k1, k2, k)
    same = np.all(np.sort(si, -1) == np.sort(bi, -1), -1)
    assert np.all(same | (margin == 0))
    if half > 1:
        assert np.all(margin > 0)
    assert np.all(np.diff(sv, axis=-1) <= 0)
    assert np.all((si >= 0) & (si < n_sub * n_sub))
    assert all(len(set(r)) == kk for r in si.reshape(-1, kk).tolist())


def test_bruteforce_catches_swapped_halves():
    """A planted mistake in the oracle (slot id built as i2 * n_sub + i1) must fail the brute-force check."""
    rng = np.random.Generator(np.random.PCG64(5))
    z, k1, k2 = _rand_case(rng, 64, 2, 8, 16)
    _, si = O.pk_address(z, k1, k2, 8)
    swapped = (si % 16) * 16 + si // 16
    _, bi = O.pk_address_bruteforce(z, k1, k2, 8)
    assert not np.array_equal(np.sort(swapped, -1), np.sort(bi, -1))


def test_bruteforce_catches_dropped_half():
    """A planted mistake (score = v1 only) must fail the brute-force check."""
    rng = np.random.Generator(np.random.PCG64(6))
    z, k1, k2 = _rand_case(rng, 64, 2, 8, 16)
    s1, s2 = O.half_scores(z, k1, k2)
    wrong = np.repeat(s1[..., :, None], 16, -1).reshape(64, 2, 256)
    _, wi = O.stable_topk_desc(wrong, 8)
    _, bi = O.pk_address_bruteforce(z, k1, k2, 8)
    assert not np.array_equal(np.sort(wi, -1), np.sort(bi, -1))


def test_weights_closed_form():
    sv = np.array([[[0.5, 0.25, 0.0]]])
    w = O.address_weights(sv, np.array([np.log(8.0)]), gate=np.array([[0.5]]))
    e = np.exp(np.array([4.0, 2.0, 0.0]))
    np.testing.assert_allclose(w[0, 0], 0.5 * e / e.sum(), rtol=1e-15)
    assert abs(O.sigmoid(np.array(0.0)) - 0.5) < 1e-15
    x = np.array([[3.0, 4.0]])
    np.testing.assert_allclose(O.rms_norm(x, np.ones(2), eps=0.0), x / np.sqrt(12.5), rtol=1e-15)
    np.testing.assert_allclose(O.normalize_rows(np.array([3.0, 4.0])), [0.6, 0.8], rtol=1e-15)
    np.testing.assert_allclose(O.normalize_rows(np.zeros(3)), np.zeros(3))


def test_adopt_picks_takes_ties_and_rejects_the_rest():
    """adopt_picks (used when a whole model is compared with the HIP path) swaps in another implementation's picks
    only where the two slots' fp64 scores agree within the tolerance."""
    rng = np.random.Generator(np.random.PCG64(5))
    k1 = rng.standard_normal((1, 6, 3))
    k2 = rng.standard_normal((1, 6, 3))
    k2[0, 3] = k2[0, 2]   # sub-keys 2 and 3 of the second half are equal: slots i*6+2 and i*6+3 tie exactly
    z = rng.standard_normal((4, 1, 6))
    sv, si = O.pk_address(z, k1, k2, 4)
    tied = si.copy()
    for n in range(4):   # swap a 2 <-> 3 partner where the pick list holds exactly one of them
        for j in range(4):
            s = si[n, 0, j]
            if s % 6 in (2, 3) and (s ^ 1) not in si[n, 0]:
                tied[n, 0, j] = s ^ 1
                break
    log = []
    sv2, si2 = O.adopt_picks(z, k1, k2, sv, si, tied, 1e-12, log)
    np.testing.assert_array_equal(si2, tied)
    np.testing.assert_allclose(sv2, sv, atol=1e-15)
    assert log == [int((tied != si).any(-1).sum())]
    wrong = si.copy()
    wrong[0, 0, 0] = int(np.setdiff1d(np.arange(36), si[0, 0])[-1])   # a far worse slot
    with pytest.raises(AssertionError):
        O.adopt_picks(z, k1, k2, sv, si, wrong, 1e-6)


@pytest.mark.parametrize("H,n_sub,half,k", [(3, 32, 16, 8), (2, 64, 16, 16), (2, 6, 4, 5), (1, 2, 3, 8)])
def test_pruned_margin_equals_full_grid_margin(H, n_sub, half, k):
    rng = np.random.Generator(np.random.PCG64(6))
    z = rng.standard_normal((50, H, 2 * half))
    k1 = rng.standard_normal((H, n_sub, half))
    k2 = rng.standard_normal((H, n_sub, half))
    np.testing.assert_array_equal(O.topk_margin_pruned(z, k1, k2, k), O.topk_margin(z, k1, k2, k))
