"""GPU parity of TrainedSdm's backward: core.TableSdmFunction (sdm_rt_address + sdm_rt_table_read forward,
sdm_rt_table_backward backward) and a OneSdmLM training step of the TrainedSdm arm, against float64 autograd
(oracle/sdm_grad64.py: table_from_picks, pinned by finite differences in tests/test_oracle_grad.py) on the kernels'
own picks.

Reference: TrainedSdm.address / forward (track4_onesdm_models.py:438-455); topk carries no gradient, the scores at the
picks, the softmax weights and the embedding_bag read do.  Bar: within 1e-4 of the largest entry of each gradient
(1e-6 absolute below a scale of 1e-2), float32 arithmetic throughout.
"""
import math

import pytest
import torch

from oracle import sdm_grad64 as G
from sdmchat_amd import core
from tests._gpu_util import say
from tests.test_gpu_grad import _mixer64, _rms64

pytestmark = pytest.mark.gpu


def check_table(name, seed, B, T, H, dh, d_a, n_sub, k, dtype=torch.float32):
    say(f"[table grad] {name}: B={B} T={T} H={H} dh={dh} d_a={d_a} n_sub={n_sub} k={k} {dtype}")
    g = torch.Generator().manual_seed(seed)
    t = dict(q=torch.randn(B, T, H * d_a, generator=g).to(dtype).float(),
             keys1=torch.randn(H, n_sub, d_a // 2, generator=g), keys2=torch.randn(H, n_sub, d_a // 2, generator=g),
             log_scale=math.log(8.0) + 0.3 * torch.randn(H, generator=g),
             values=torch.randn(H, n_sub * n_sub, dh, generator=g))
    wgt = torch.randn(B, T, H * dh, generator=torch.Generator().manual_seed(seed + 7))
    dev = {n: v.to("cuda").to(dtype if n == "q" else torch.float32).requires_grad_(True) for n, v in t.items()}
    cfg = dict(k=k)
    r = core.TableSdmFunction.apply(dev["q"], dev["keys1"], dev["keys2"], dev["log_scale"], dev["values"], cfg)
    (r * wgt.cuda()).sum().backward()
    torch.cuda.synchronize()
    kk = min(k, min(k, n_sub) ** 2)
    si = cfg["slots"][..., :kk].permute(0, 2, 1, 3).long().cpu()
    o = {n: v.double().clone().requires_grad_(True) for n, v in t.items()}
    ref = G.table_from_picks(o["q"].view(B, T, H, d_a), o["keys1"], o["keys2"], o["log_scale"], o["values"], si)
    ref = ref.reshape(B, T, H * dh)
    err = (r.detach().double().cpu() - ref).abs().max().item()
    assert err <= 2e-5 * max(1.0, ref.abs().max().item()), f"read differs by {err}"
    (ref * wgt.double()).sum().backward()
    for n in t:
        gr = o[n].grad
        gg = dev[n].grad.double().cpu()
        scale = gr.abs().max().item()
        rounding = 2.0 ** -8 * gr.abs() if (dtype == torch.bfloat16 and n == "q") else 0.0
        e = ((gg - gr).abs() - rounding).max().item()
        say(f"  d{n}: max err {e:.3e} of scale {scale:.3e}")
        assert e <= 1e-4 * max(scale, 1e-2), f"d{n}: {e:.3e} vs {scale:.3e}"


def test_table_grad_small():
    check_table("small", 1, 2, 100, 2, 32, 16, 16, 16)


def test_table_grad_eight_picks_narrow_rows():
    check_table("k8", 2, 2, 70, 3, 20, 8, 8, 8)


def test_table_grad_trained_sdm_layer_shape():
    """The TrainedSdm of the FULL model (one head of width 768, 4,096 slots, k=16, d_a 32), bf16 queries."""
    check_table("layer", 3, 1, 128, 1, 768, 32, 64, 16, dtype=torch.bfloat16)


def _trained64(P, pre, x, si, H, d_a):
    B, T, d = x.shape
    q = (_rms64(x, P[pre + "norm.w"]) @ P[pre + "wq.weight"].T).view(B, T, H, d_a)
    r = G.table_from_picks(q, P[pre + "keys1"], P[pre + "keys2"], P[pre + "log_scale"], P[pre + "values"], si)
    return r.reshape(B, T, d) @ P[pre + "wo.weight"].T


def test_onesdm_trained_sdm_arm_training_step_matches_the_oracle():
    """Two layers of [x + RunTimeSdm(x); x + TrainedSdm(x)], final norm, tied head: every parameter's gradient of a
    weighted sum of the logits against a float64 autograd model on the same picks."""
    from sdmchat_amd import OneSdmLM
    torch.manual_seed(0)
    Vv, d, L, H, n_sub, d_a, k = 40, 64, 2, 4, 8, 16, 8
    model = OneSdmLM(Vv, d=d, layers=L, mlp_f=96, heads=H, n_sub=n_sub, d_a=d_a, k=k, decays=(0.6, 0.8, 0.95, 0.99),
                     learn_decay=True, addr_bias=0.2, ffn="sdm", sdm_n_sub=12, sdm_heads=2, sdm_d_a=8,
                     sdm_k=16).cuda()
    with torch.no_grad():   # fill the zero-start maps and tables so every path carries gradient
        for m in model.mems:
            torch.nn.init.xavier_uniform_(m.wo.weight)
            torch.nn.init.xavier_uniform_(m.wg.weight)
            m.wq.weight.copy_(0.7 * m.wk.weight + 0.3 * m.wq.weight)
        for s in model.sdms:
            s.values.normal_(0.0, 0.5)
    idx = torch.randint(0, Vv, (2, 90), generator=torch.Generator().manual_seed(1)).cuda()
    ins = {}
    hooks = [m.register_forward_pre_hook(lambda mod, a, i=i: ins.__setitem__(("m", i), a[0].detach()))
             for i, m in enumerate(model.mems)]
    hooks += [s.register_forward_pre_hook(lambda mod, a, i=i: ins.__setitem__(("s", i), a[0].detach()))
              for i, s in enumerate(model.sdms)]
    say(f"[table grad] OneSdmLM TrainedSdm arm: layers={L} d={d} B=2 T=90")
    logits = model(idx)
    for hk in hooks:
        hk.remove()
    wgt = torch.randn(logits.shape, generator=torch.Generator().manual_seed(2)).cuda()
    (logits * wgt).sum().backward()
    torch.cuda.synchronize()
    mp, sp = [], []
    with torch.no_grad():
        for i, m in enumerate(model.mems):
            proj = torch.cat(m._project_train(ins[("m", i)])[:2], -1)
            sw = core.address(proj[..., :H * d_a], m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)[0]
            sr = core.address(proj[..., H * d_a:2 * H * d_a], m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)[0]
            mp.append((sw.permute(0, 2, 1, 3).long().cpu(), sr.permute(0, 2, 1, 3).long().cpu()))
        for i, s in enumerate(model.sdms):
            q = s.wq(s.norm(ins[("s", i)]).float()).float()
            si = core.address(q, s.keys1, s.keys2, s.k, s.log_scale)[0]
            sp.append(si.permute(0, 2, 1, 3).long().cpu())
    P = {n: p.detach().double().cpu().clone().requires_grad_(True) for n, p in model.named_parameters()}
    x = P["emb.weight"][idx.cpu()]
    for i, m in enumerate(model.mems):
        x = x + _mixer64(P, f"mems.{i}.", m, x, None, *mp[i])
        x = x + _trained64(P, f"sdms.{i}.", x, sp[i], model.sdms[i].h, model.sdms[i].d_a)
    ref = _rms64(x, P["nf.w"]) @ P["emb.weight"].T
    err = (logits.detach().double().cpu() - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item(), f"logits differ by {err}"
    (ref * wgt.double().cpu()).sum().backward()
    for n, p in model.named_parameters():
        g, gr = p.grad, P[n].grad
        assert g is not None and gr is not None, n
        scale = gr.abs().max().item()
        e = (g.double().cpu() - gr).abs().max().item()
        say(f"  d{n}: max err {e:.3e} of scale {scale:.3e}")
        assert e <= 1e-4 * max(scale, 1e-2), f"d{n}: {e:.3e} vs {scale:.3e}"


def test_table_backward_is_deterministic():
    """The value-table rows are summed over their picks in pick order (stable sort by slot), the parameter sums in a
    fixed order: two backward calls give identical bits."""
    g = torch.Generator().manual_seed(9)
    B, T, H, dh, d_a, n_sub, k = 2, 150, 2, 32, 16, 8, 16
    q = torch.randn(B, T, H * d_a, generator=g).cuda()
    k1, k2 = (torch.randn(H, n_sub, d_a // 2, generator=g).cuda() for _ in range(2))
    ls = torch.full((H,), math.log(8.0)).cuda()
    vals = torch.randn(H, n_sub * n_sub, dh, generator=g).cuda()
    dy = torch.randn(B, T, H * dh, generator=g).cuda()
    prm = core._params(q.device, k1, k2, None, ls, None, None, None)
    sl, sc, wt = core.address(q, k1, k2, k, ls, padded=True, params=prm)
    g1 = core.table_backward(q, sl, wt, sc, vals, dy, k=k, params=prm)
    g2 = core.table_backward(q, sl, wt, sc, vals, dy, k=k, params=prm)
    torch.cuda.synchronize()
    for n in g1:
        assert torch.equal(g1[n], g2[n]), n
