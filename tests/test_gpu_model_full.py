"""The whole OneSdmLM at the full workload width (d 768, 12 layers, vocabulary 32,768; mixer 12 heads of M=1,024,
k 8) for both arms: the PARTIAL arm (SwiGLU of hidden 2,048, track4_sdmllm_models.py:89-97) and the FULL arm
(TrainedSdm of 4,096 slots, one head, k 16, track4_onesdm_models.py:414-457); forward OM:471-555, decode OM:276-300
and 534-555.

- float32, B=1, T=128: logits against the fp64 oracle (oracle.sdm_fp64.model_forward).  The HIP path's float32
  layer inputs differ from the oracle's float64 ones by rounding, so near ties may resolve the other way; the
  oracle takes the HIP path's picks wherever the two slots' fp64 scores are within 1e-5 (adopt_picks), everywhere
  else its own, and the count of such addresses is printed.
- bfloat16 at the bench shape B=8, T=2048: finite logits; a token changed at position t leaves every logit before
  t bit-identical; reset at BOS makes the logits after a BOS equal those of the suffix run alone.
- decode: prefill + step equals the forward; a HIP graph of steps replays equal to eager steps (the decode of
  config 5 itself is checked stage by stage against the oracle in tests/test_gpu_model_bf16.py).
- a HIP graph of the forward (ForwardGraph, both arms in bfloat16) replays equal to the eager forward, bit for bit,
  on three token batches with eager work between the replays.
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import DecodeGraph, ForwardGraph, decode_state_bytes, synthetic as S
from tests._gpu_util import say

pytestmark = pytest.mark.gpu
ARMS = ["swiglu", "trained_sdm"]


def _cfg(m):
    c = dict(layers=m.n_layers, heads=m.mems[0].h, d_a=m.mems[0].d_a, k=m.mems[0].k, ffn=m.ffn,
             reset_at_bos=m.reset_at_bos, bos_id=m.bos_id)
    if m.ffn == "sdm":
        s = m.sdms[0]
        c.update(sdm_heads=s.h, sdm_d_a=s.d_a, sdm_k=s.k)
    return c


def _picks(m, B, T):
    """The HIP path's picks of the last forward, per layer, as the oracle's (B*T, H, kk)."""
    forced = {}
    for i, mm in enumerate(m.mems):
        kk = min(mm.k, min(mm.k, mm.n_sub) ** 2)
        forced[("mem", i)] = tuple(s[..., :kk].permute(0, 2, 1, 3).reshape(B * T, mm.h, kk).cpu().numpy()
                                   for s in mm.last_picks)
    for i, s in enumerate(getattr(m, "sdms", [])):
        forced[("sdm", i)] = s.last_si.cpu().numpy()
    return forced


@pytest.mark.parametrize("arm", ARMS)
def test_full_model_fp32_logits_match_oracle(arm):
    m = S.full_model(arm)
    p = {n: v.detach().double().numpy() for n, v in m.state_dict().items()}
    idx = S.model_tokens(1, 128, seed=41)
    m = m.cuda().eval()
    for mm in m.mems:
        mm.keep_picks = True
    say("full model fp32", arm)
    with torch.no_grad():
        got = m(torch.from_numpy(idx).cuda()).double().cpu().numpy()
    log = []
    cfg = dict(_cfg(m), adopt_tol=1e-5, adopt_log=log)
    want = O.model_forward(idx, p, cfg, forced=_picks(m, 1, 128))
    scale = np.abs(want).max()
    err = np.abs(got - want).max() / scale
    say(f"  {sum(log)} of the layers' addresses took the HIP picks at ties; max |logit error| / scale {err:.2e}")
    np.testing.assert_allclose(got, want, atol=2e-5 * scale, rtol=0)


@pytest.mark.parametrize("arm", ARMS)
def test_full_model_bf16_properties_at_bench_shape(arm):
    m = S.full_model(arm, reset_at_bos=True, bos_id=7).cuda().to(torch.bfloat16).eval()
    B, T = 8, 2048
    idx = torch.from_numpy(S.model_tokens(B, T, seed=42)).cuda()
    idx[idx == 7] = 8   # no BOS but the planted one below
    say("full model bf16 properties", arm)
    with torch.no_grad():
        base = m(idx)
        assert torch.isfinite(base).all()
        t = 1000   # causality: a token changed at t leaves every earlier logit bit-identical
        alt = idx.clone()
        alt[:, t] = (alt[:, t] + 1) % m.V
        changed = m(alt)
        assert torch.equal(changed[:, :t], base[:, :t]), "a later token changed an earlier logit"
        assert not torch.equal(changed[:, t:], base[:, t:])
        s = 1500   # reset at BOS: with a BOS at s the logits from s on do not depend on the tokens before s
        bos = idx.clone()
        bos[:, s] = 7
        other = bos.clone()
        other[:, :s] = (other[:, :s] * 31 + 5) % m.V
        other[other == 7] = 8
        other[:, s] = 7
        a, b = m(bos), m(other)
        assert not torch.equal(a[:, :s], b[:, :s])
        assert torch.equal(a[:, s:], b[:, s:]), "logits after a BOS depend on the tokens before it"


def _decode_case(T=128, streams=64):
    m = S.full_model("trained_sdm").cuda().eval()
    idx = torch.from_numpy(S.model_tokens(streams, T, seed=43)).cuda()
    return m, idx


def test_full_model_prefill_then_step_equals_forward():
    m, idx = _decode_case(T=96, streams=8)
    with torch.no_grad():
        want = m(idx).float()
        logits, st = m.prefill(idx[:, :64])
        got = torch.stack([m.step(idx[:, t], st) for t in range(64, 96)], 1).float()
    scale = want.abs().max()
    np.testing.assert_allclose(logits.float().cpu().numpy(), want[:, :64].cpu().numpy(), atol=1e-6 * float(scale))
    err = float((got - want[:, 64:]).abs().max() / scale)
    say(f"prefill + step: max |difference| / scale {err:.2e}")
    assert err <= 1e-4


def test_decode_graph_replays_equal_eager_steps():
    m, idx = _decode_case(T=12, streams=16)
    with torch.no_grad():
        eager, graphed = m.decode_state(16), m.decode_state(16)
        g = DecodeGraph(m, graphed, steps=4)
        for rep in range(3):
            toks = idx[:, 4 * rep:4 * rep + 4].t().contiguous()
            out = g.run(toks).clone()
            ref = torch.stack([m.step(toks[t], eager) for t in range(4)])
            torch.randn(1000, device="cuda").sum()   # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep}: logits differ"
            for a, b in zip(graphed.layers, eager.layers):
                assert torch.equal(a.mem, b.mem) and torch.equal(a.scale, b.scale) and torch.equal(a.last, b.last)
        assert graphed.pos == eager.pos == 12


@pytest.mark.parametrize("arm", ARMS)
def test_forward_graph_replays_equal_eager(arm):
    m = S.full_model(arm, layers=3, reset_at_bos=True, bos_id=7).cuda().to(torch.bfloat16).eval()
    B, T = 2, 300
    say("ForwardGraph", arm, B, T)
    with torch.no_grad():
        g = ForwardGraph(m, B, T)
        for rep in range(3):
            idx = torch.from_numpy(S.model_tokens(B, T, seed=40 + rep)).cuda()
            idx[:, 100 + 30 * rep] = 7   # a BOS
            out = g.run(idx).clone()
            torch.randn(1000, device="cuda").sum()   # eager work between replays
            ref = m(idx)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep}: logits differ"


def test_decode_state_bytes():
    m = S.full_model("trained_sdm", layers=2)
    assert decode_state_bytes(m, 10) == 2 * 12 * 1024 * 65 * 4 == decode_state_bytes(m, 10 ** 6)
    st = m.cuda().decode_state(3)
    assert st.nbytes() == 3 * decode_state_bytes(m, 0) + 3 * 2 * 12 * (4 + 8 * 4)   # plus scales and last slots
