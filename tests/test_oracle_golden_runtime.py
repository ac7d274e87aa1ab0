"""The oracle against the reference's own outputs (tests/golden/runtime_sdm_golden.npz, written by
tests/golden/make_golden.py from the reference's pk_address, RunTimeSdm and OneSdmLM, track4_onesdm_models.py:134-148,
151-300, 471-555).

- pk_address on the 24,576 addresses of the layer workload: the oracle's picks equal the reference's, in order,
  except where the two candidates' fp64 scores are within 2.4e-7 (a float32-level tie; the count is printed).
- RunTimeSdm.forward at B1 T256 (the float32 validation workload, d768 H12 M1024 k8) and at the edge shape (d32 H4
  n_sub 6 k4, chunk 7, fades 0 and 1): the oracle's y within 2e-5 of the output scale, its picks equal to the
  reference's.
- OneSdmLM logits of both arms (tiny, reset at BOS): the oracle's model_forward within 2e-5 of the logits' scale.
"""
import os

import numpy as np
import pytest

from oracle import sdm_fp64 as O
from tests.golden import golden_inputs as G

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "runtime_sdm_golden.npz"))
TIE = 2.4e-7   # float32 resolution of a cosine score near 1


def compare_picks(si_ref, si, z, keys1, keys2):
    """Rows (token, head) whose picks differ from the reference's, after checking that every difference is a tie:
    at each pick position the fp64 scores of the two slots agree within TIE."""
    g = O.full_grid(z.astype(np.float64), keys1, keys2)
    s_ref = np.take_along_axis(g, si_ref.astype(np.int64), -1)
    s_got = np.take_along_axis(g, si.astype(np.int64), -1)
    diff = si_ref != si
    assert np.all(np.abs(s_ref - s_got)[diff] < TIE), "a pick differs from the reference's away from a tie"
    return int(diff.any(-1).sum())


def test_oracle_picks_equal_reference_on_layer_addresses():
    z, k1, k2 = G.layer_addresses(int(GOLD["addr.seed"]))
    assert G.digest(z) == GOLD["addr.digest"], "regenerated addresses differ from the recorded ones"
    sv, si = O.pk_address(z, k1, k2, int(GOLD["addr.k"]))
    n = compare_picks(GOLD["addr.si"], si, z, k1, k2)
    print(f"oracle vs reference picks: {n} of {si.shape[0] * si.shape[1]} addresses differ, all at fp64 gaps < {TIE}")
    np.testing.assert_allclose(sv, GOLD["addr.sv"], atol=1e-6, rtol=0)


@pytest.mark.parametrize("name", ["b1_t256", "edge"])
def test_oracle_layer_equals_reference(name):
    kw, p, x = G.layer_case(name, int(GOLD[f"{name}.seed"]))
    assert G.digest(x) == GOLD[f"{name}.digest"], "regenerated input differs from the recorded one"
    lp = {n: v.astype(np.float64) for n, v in p.items()}
    lp["decay"] = lp["decays_fixed"]
    cfg = dict(heads=kw["heads"], d_a=kw["d_a"], k=kw["k"], read_mode="mean", read_eps=1e-3, out_norm=True,
               out_norm_eps=1e-2, write_gate=True)
    y = O.layer_forward(x, lp, cfg)
    want = GOLD[f"{name}.y"].astype(np.float64)
    scale = np.abs(want).max()
    np.testing.assert_allclose(y, want, atol=2e-5 * scale, rtol=0)
    # the picks of prepare, as the reference returns them ([B, H, T, kk])
    B, T, d = x.shape
    H, d_a = kw["heads"], kw["d_a"]
    hx = O.rms_norm(x.astype(np.float64), lp["norm.w"])
    for wn, key in (("wk.weight", "siw"), ("wq.weight", "sir")):
        z = (hx @ lp[wn].T).reshape(B * T, H, d_a) + lp["addr_b"]
        _, si = O.pk_address(z, lp["keys1"], lp["keys2"], kw["k"])
        got = si.reshape(B, T, H, -1).transpose(0, 2, 1, 3)
        np.testing.assert_array_equal(got, GOLD[f"{name}.{key}"])


@pytest.mark.parametrize("ffn", ["mlp", "sdm"])
def test_oracle_model_logits_equal_reference(ffn):
    import torch
    from sdmchat_amd import OneSdmLM
    kw = dict(G.MODEL_KW)
    V = kw.pop("V")
    seed = int(GOLD[f"model_{ffn}.seed"])
    m = OneSdmLM(V, ffn=ffn, seed=seed, **kw)
    shapes = {n: tuple(t.shape) for n, t in m.state_dict().items()}
    p = G.model_params(shapes, seed)
    idx = GOLD[f"model_{ffn}.idx"].astype(np.int64)
    np.testing.assert_array_equal(idx, G.model_tokens(seed))
    cfg = dict(layers=kw["layers"], heads=kw["heads"], d_a=kw["d_a"], k=kw["k"], ffn=ffn, reset_at_bos=True,
               bos_id=kw["bos_id"], sdm_heads=kw["sdm_heads"], sdm_d_a=kw["sdm_d_a"], sdm_k=kw["sdm_k"])
    logits = O.model_forward(idx, {n: v.astype(np.float64) for n, v in p.items()}, cfg)
    want = GOLD[f"model_{ffn}.logits"].astype(np.float64)
    np.testing.assert_allclose(logits, want, atol=2e-5 * np.abs(want).max(), rtol=0)
    del torch


BENCH = np.load(os.path.join(os.path.dirname(__file__), "golden", "bench_ties_golden.npz"))


def bench_near_ties():
    """The bench workload's addresses (regenerated, checked against the recorded checksums) and, per address set,
    the flat (token, head) indices of its near-ties with the reference's picks there."""
    zw, zr, k1, k2 = G.bench_addresses()
    assert G.digest(zw) == BENCH["bench.digest_w"] and G.digest(zr) == BENCH["bench.digest_r"], \
        "regenerated bench addresses differ from the recorded ones"
    return {"w": zw, "r": zr}, k1, k2


def spliced_digest(si, s):
    """The checksum of a whole ordered pick array (flat (token, head), 8) with the reference's near-tie rows of set s
    spliced in: the reference's own checksum exactly when every other row equals the reference's."""
    full = np.asarray(si).astype(np.int16).copy()
    full[BENCH[f"bench.near_{s}"]] = BENCH[f"bench.si_{s}"]
    return G.digest(full)


def bench_pick_diffs(z, k1, k2, near, si, ref):
    """Flat near-tie addresses whose ordered picks si differ from the reference's ref (both (n, 8)), after checking
    that every difference is a tie: at each differing position the two slots' fp64 scores agree within TIE."""
    H = z.shape[1]
    diff = si != ref
    rows = np.flatnonzero(diff.any(-1))
    for i in rows:
        tok, h = divmod(int(near[i]), H)
        g = O.full_grid(z[tok:tok + 1, h:h + 1].astype(np.float64), k1[h:h + 1], k2[h:h + 1])[0, 0]
        gap = np.abs(g[ref[i]] - g[si[i]])[diff[i]]
        assert np.all(gap < TIE), f"address {int(near[i])}: a pick differs from the reference's at an fp64 gap of " \
                                  f"{float(gap.max()):.3e}"
    return len(rows)


def test_oracle_picks_equal_reference_at_bench_near_ties():
    """At every address of the bench workload (B=8, T=2048, 12 heads, both sets) where two of its 9 best fp64 scores
    lie within 1e-5 (a near-tie of the pick or of the order), the oracle's ordered picks against the reference's own
    (make_golden.py bench): they differ only where the two slots' fp64 scores are within TIE, and the count is
    printed; at every other address the oracle's ordered picks equal the reference's exactly (the oracle's whole pick
    array with the recorded near-tie rows spliced in has the checksum of the reference's)."""
    zs, k1, k2 = bench_near_ties()
    k1d, k2d = k1.astype(np.float64), k2.astype(np.float64)
    for s in ("w", "r"):
        near = BENCH[f"bench.near_{s}"]
        _, si = O.pk_address(zs[s].astype(np.float64), k1d, k2d, int(BENCH["bench.k"]))
        si = si.reshape(-1, si.shape[-1])
        n = bench_pick_diffs(zs[s], k1d, k2d, near, si[near], BENCH[f"bench.si_{s}"].astype(np.int64))
        assert spliced_digest(si, s) == BENCH[f"bench.all_digest_{s}"], "picks away from the near-ties differ"
        print(f"bench near-ties ({s}): {n} of {len(near)} addresses order or pick differently from the reference, "
              f"all at fp64 gaps < {TIE}")
