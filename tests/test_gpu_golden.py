"""The HIP path against the reference's own outputs (tests/golden/runtime_sdm_golden.npz, written by
tests/golden/make_golden.py from the reference's pk_address, RunTimeSdm and OneSdmLM, track4_onesdm_models.py:134-148,
151-300, 471-555).

- sdm_rt_address on the 24,576 addresses of the layer workload (bf16 values, as bf16 and as float32 input): picks in
  the reference's order; a pick may differ only where the two slots' fp64 scores are within 2.4e-7 (a float32-level
  tie), and the number of such addresses is printed (the tests of the oracle pin it against the same data).
- RunTimeSdm.forward (float32) at B=1, T=256 (the layer's float32 validation workload) and at the edge shape: y within 1e-5 of the output scale.
- OneSdmLM (float32, tiny, both arms, reset at BOS): logits within 1e-5 of their scale.
"""
import os

import numpy as np
import pytest
import torch

from sdmchat_amd import OneSdmLM, RunTimeSdm, core
from tests._gpu_util import say
from tests.golden import golden_inputs as G
from tests.test_oracle_golden_runtime import compare_picks

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "runtime_sdm_golden.npz"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gpu_picks_follow_reference_on_layer_addresses(dtype):
    z, k1, k2 = G.layer_addresses(int(GOLD["addr.seed"]))
    assert G.digest(z) == GOLD["addr.digest"]
    N, H, d_a = z.shape
    say("golden addresses", z.shape, dtype)
    zd = torch.from_numpy(z).cuda().to(dtype).reshape(1, N, H * d_a)
    kt1, kt2 = torch.from_numpy(k1).cuda(), torch.from_numpy(k2).cuda()
    ls = torch.full((H,), float(np.log(8.0)), device="cuda")
    si, sv, _ = core.address(zd, kt1, kt2, int(GOLD["addr.k"]), log_scale=ls)
    torch.cuda.synchronize()
    si = si[0].permute(1, 0, 2).cpu().numpy()   # [N, H, kk]
    sv = sv[0].permute(1, 0, 2).cpu().numpy()
    n = compare_picks(GOLD["addr.si"], si, z, k1, k2)
    print(f"GPU ({dtype}) vs reference picks: {n} of {N * H} addresses differ, all at fp64 gaps < 2.4e-7")
    np.testing.assert_allclose(sv, GOLD["addr.sv"], atol=2e-6, rtol=0)


@pytest.mark.parametrize("name", ["b1_t256", "edge"])
def test_gpu_layer_equals_reference(name):
    kw, p, x = G.layer_case(name, int(GOLD[f"{name}.seed"]))
    assert G.digest(x) == GOLD[f"{name}.digest"]
    say("golden layer", name, x.shape)
    m = RunTimeSdm(kw["d"], heads=kw["heads"], n_sub=kw["n_sub"], d_a=kw["d_a"], k=kw["k"], decays=kw["decays"],
                   chunk=kw["chunk"])
    m.load_state_dict({n: torch.from_numpy(v) for n, v in p.items()}, strict=True)
    m = m.cuda().eval()
    with torch.no_grad():
        y = m(torch.from_numpy(x).cuda()).double().cpu().numpy()
    want = GOLD[f"{name}.y"].astype(np.float64)
    np.testing.assert_allclose(y, want, atol=1e-5 * np.abs(want).max(), rtol=0)


@pytest.mark.parametrize("ffn", ["mlp", "sdm"])
def test_gpu_model_logits_equal_reference(ffn):
    kw = dict(G.MODEL_KW)
    V = kw.pop("V")
    seed = int(GOLD[f"model_{ffn}.seed"])
    m = OneSdmLM(V, ffn=ffn, seed=seed, **kw)
    p = G.model_params({n: tuple(t.shape) for n, t in m.state_dict().items()}, seed)
    m.load_state_dict({n: torch.from_numpy(v) for n, v in p.items()}, strict=True)
    m = m.cuda().eval()
    idx = torch.from_numpy(GOLD[f"model_{ffn}.idx"].astype(np.int64)).cuda()
    say("golden model", ffn)
    with torch.no_grad():
        got = m(idx).double().cpu().numpy()
    want = GOLD[f"model_{ffn}.logits"].astype(np.float64)
    np.testing.assert_allclose(got, want, atol=1e-5 * np.abs(want).max(), rtol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gpu_picks_at_bench_near_ties_follow_reference(dtype):
    """The bench workload's 393,216 addresses (B=8, T=2048, 12 heads, write keys and read queries; bfloat16 values):
    at every address where two of its 9 best fp64 scores lie within 1e-5 (a near-tie of the pick or of the order)
    the kernel's ordered picks against the reference's own (make_golden.py bench), every difference a float32-level
    tie (fp64 gap < 2.4e-7), the exact count printed; at every other address the ordered picks equal the
    reference's (the whole pick array with the recorded near-tie rows spliced in has the checksum of the
    reference's)."""
    from tests.test_oracle_golden_runtime import BENCH, bench_near_ties, bench_pick_diffs, spliced_digest
    zs, k1, k2 = bench_near_ties()
    k1d, k2d = k1.astype(np.float64), k2.astype(np.float64)
    kt1, kt2 = torch.from_numpy(k1).cuda(), torch.from_numpy(k2).cuda()
    ls = torch.full((12,), float(np.log(8.0)), device="cuda")
    say("bench near-ties", dtype)
    total = 0
    for s in ("w", "r"):
        z = zs[s]
        N, H, d_a = z.shape
        si, _, _ = core.address(torch.from_numpy(z).cuda().to(dtype).reshape(8, N // 8, H * d_a), kt1, kt2, 8,
                                log_scale=ls)
        torch.cuda.synchronize()
        si = si.permute(0, 2, 1, 3).reshape(N * H, 8).cpu().numpy().astype(np.int64)   # flat (token, head)
        near = BENCH[f"bench.near_{s}"]
        n = bench_pick_diffs(z, k1d, k2d, near, si[near], BENCH[f"bench.si_{s}"].astype(np.int64))
        total += n
        assert spliced_digest(si, s) == BENCH[f"bench.all_digest_{s}"], \
            "ordered picks away from the near-ties differ from the reference's"
        print(f"GPU ({dtype}) vs reference at the bench near-ties ({s}): {n} of {len(near)} addresses differ "
              f"(fp64 gaps < 2.4e-7); all {N * H - len(near)} other addresses equal the reference's (checksum)")
    print(f"GPU ({dtype}): {total} index mismatches against the reference over the bench workload's near-ties")
