"""GPU parity of TrainedSdm (track4_onesdm_models.py:414-457): the table read (sdm_rt_table_read, the reference's
embedding_bag) and the whole layer against the fp64 oracle.  Picks are checked in order on the kernel's own float32
queries (differences only at float32 score ties, counted and bounded) and as sets against the oracle's float64
queries (differences only where the fp64 top-k margin is within the queries' float32 error); the read-out and the
layer output against the oracle driven by the kernels' own picks (float32 1e-5)."""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import TrainedSdm, core
from tests._gpu_util import DELTA, assert_close, pick_diffs, say

# Against the oracle's own float64 queries the picks may differ where the fp64 top-k margin is within the float32
# error of the kernel's queries: q = wq(hx) is a 768-term float32 dot product (|q| ~ 1, error ~ 2^-24 sqrt(768) ~
# 2e-6 per element), and the score of a unit half is a 16-term cosine of it, so scores move by up to ~1e-6.  On the
# kernel's own float32 queries the ordered picks must equal the oracle's up to float32 score ties (DELTA).
Q_DELTA = 1e-6

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,n_sub,dh,k,vdt,odt", [(1, 64, 768, 16, torch.float32, torch.float32),   # XCD-sliced
                                                   (1, 64, 768, 16, torch.bfloat16, torch.bfloat16),  # XCD-sliced
                                                   (2, 32, 512, 8, torch.bfloat16, torch.float32),    # XCD-sliced
                                                   (4, 8, 64, 8, torch.bfloat16, torch.float32),
                                                   (3, 6, 20, 5, torch.float32, torch.bfloat16)])
def test_table_read_matches_the_weighted_row_sum(H, n_sub, dh, k, vdt, odt):
    rng = np.random.Generator(np.random.PCG64(81))
    B, T, M = 2, 37, n_sub * n_sub
    kk = min(k, min(k, n_sub) ** 2)
    pitch = (kk + 7) // 8 * 8
    si = np.full((B, H, T, pitch), -1, np.int32)
    w = np.zeros((B, H, T, pitch), np.float32)
    for idx in np.ndindex(B, H, T):
        si[idx][:kk] = rng.choice(M, kk, replace=False)
        w[idx][:kk] = rng.random(kk)
    vals = rng.standard_normal((H, M, dh)).astype(np.float32)
    vd = torch.from_numpy(vals).cuda().to(vdt)
    out = core.table_read(torch.from_numpy(si).cuda(), torch.from_numpy(w).cuda(), vd, k, out_dtype=odt)
    torch.cuda.synchronize()
    v64 = vd.float().cpu().numpy().astype(np.float64)
    want = O.table_read(si[..., :kk].transpose(0, 2, 1, 3).reshape(B * T, H, kk),
                        w[..., :kk].transpose(0, 2, 1, 3).reshape(B * T, H, kk), v64).reshape(B, T, H * dh)
    assert_close(out.float().cpu().numpy(), want, 1e-5, bf16_out=odt == torch.bfloat16, msg="table read")


def _layer(d, n_sub, heads, d_a, k, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    m = TrainedSdm(d, n_sub, heads=heads, d_a=d_a, k=k)
    with torch.no_grad():
        m.norm.w.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)))
        m.wq.weight.copy_(torch.from_numpy((rng.standard_normal((heads * d_a, d)) / np.sqrt(d)).astype(np.float32)))
        m.values.copy_(torch.from_numpy(rng.standard_normal(tuple(m.values.shape)).astype(np.float32)))
        m.log_scale.copy_(torch.from_numpy(np.log(8.0) + rng.uniform(-0.3, 0.3, heads).astype(np.float32)))
        m.wo.weight.copy_(torch.from_numpy((rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32)))
    x = rng.standard_normal((2, 48, d)).astype(np.float32)
    return m.cuda().eval(), x


@pytest.mark.parametrize("d,n_sub,heads,d_a,k,BT", [(768, 64, 1, 32, 16, (2, 48)), (64, 8, 4, 16, 8, (2, 48)),
                                                   (96, 12, 3, 32, 12, (2, 48)), (768, 64, 1, 32, 16, (8, 2048))])
def test_trained_sdm_layer_matches_oracle(d, n_sub, heads, d_a, k, BT):
    """The table layer against the oracle: picks (near-ties aside), weights, and the output on the kernel's own
    picks; the FULL model's layer (4,096 slots, k=16) also at the bench's B=8, T=2048."""
    m, x = _layer(d, n_sub, heads, d_a, k, seed=82 + n_sub)
    if BT != (2, 48):
        x = np.random.Generator(np.random.PCG64(83)).standard_normal(BT + (d,)).astype(np.float32)
    say("TrainedSdm", d, n_sub, heads, d_a, k)
    m.keep_picks = True
    with torch.no_grad():
        y = m(torch.from_numpy(x).cuda()).cpu().numpy()
        w_k, si_k = m.address(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    p = {n: v.detach().cpu().numpy().astype(np.float64) for n, v in m.state_dict().items()}
    cfg = dict(heads=heads, d_a=d_a, k=k)
    y64, parts = O.trained_sdm_forward(x, p, cfg, return_parts=True)
    si_k, w_k = si_k.cpu().numpy(), w_k.cpu().numpy()
    B, T = x.shape[:2]
    n_addr = B * T * heads
    # 1. on the kernel's own float32 queries: ordered picks, differences only at float32 score ties
    q_k = m.last_q.float().cpu().numpy().astype(np.float64).reshape(B * T, heads, d_a)
    _, osi_q = O.pk_address(q_k, p["keys1"], p["keys2"], k)
    n_tie = int(pick_diffs(q_k, p["keys1"], p["keys2"], osi_q, si_k).sum())
    # 2. against the oracle's float64 queries: the same pick sets except where the fp64 margin is within Q_DELTA
    same = np.all(np.sort(si_k, -1) == np.sort(parts["si"], -1), -1)
    margin = O.topk_margin(parts["q"], p["keys1"], p["keys2"], k)
    assert np.all(same | (margin < Q_DELTA)), "picks differ away from near-ties"
    n_q = int((~same).sum())
    say(f"TrainedSdm picks: {n_tie} of {n_addr} addresses differ from the oracle on the kernel's queries (ties "
        f"< {DELTA:.1e}); {n_q} differ from the oracle's float64 queries, all at margins < {Q_DELTA:.0e} "
        f"({int((margin < Q_DELTA).sum())} addresses have such a margin)")
    assert n_tie <= max(2, n_addr // 10000) and n_q <= max(4, n_addr // 1000)
    # the layer on the kernel's own picks and weights
    r = O.table_read(si_k, w_k, p["values"]).reshape(B, T, d)
    y_k = r @ p["wo.weight"].T
    assert_close(y, y_k, 1e-5, msg="TrainedSdm output on the kernel's picks")
    np.testing.assert_allclose(w_k[same], parts["w"][same], atol=2e-6, rtol=2e-6)
    if same.all():
        assert_close(y, y64, 1e-5, msg="TrainedSdm output against the independent oracle")
