"""GPU parity of the backward: core.SdmCoreFunction (sdm_rt_forward_train + sdm_rt_backward) and the RunTimeSdm
training path against the float64 autograd oracle (oracle/sdm_grad64.py) for the same picks.

Reference: the reference trains RunTimeSdm by autograd of prepare / _chunk / finish (track4_onesdm_models.py:195-274);
topk carries no gradient, so the picks are taken from the HIP addressing (core.address, the kernel the training
forward runs) and the oracle differentiates the rest in float64.  The oracle is pinned against finite differences of
the fp64 token recurrence (tests/test_oracle_grad.py).

Bar: every gradient within 1e-4 of the oracle's, relative to its largest entry (1e-6 absolute for a gradient whose
largest entry is below 1e-2; float32 arithmetic throughout; the
bfloat16 case feeds the same bf16 values to both sides and its input gradients, returned in bfloat16, get half a
bfloat16 ulp on top); the read-out within 2e-5.  The backward is deterministic:
two runs give identical bits.
"""
import math

import numpy as np
import pytest
import torch

from oracle import sdm_grad64 as G
from sdmchat_amd import RunTimeSdm, core
from tests._gpu_util import say

pytestmark = pytest.mark.gpu

NAMES = ("kz", "qz", "v", "gl", "keys1", "keys2", "addr_b", "log_scale", "decay", "onorm_w", "gate_bias")


def make(seed, B, T, H, dh, d_a, n_sub, dtype=torch.float32, gate=True, decays=None, reset_p=0.0, overlap=0.0,
         learn_decay=True):
    g = torch.Generator().manual_seed(seed)
    kz = torch.randn(B, T, H * d_a, generator=g)
    qz = overlap * kz + torch.randn(B, T, H * d_a, generator=g)   # overlap > 0: reads find this chunk's writes
    t = dict(kz=kz, qz=qz, v=torch.randn(B, T, H * dh, generator=g),
             gl=1.5 * torch.randn(B, T, H, generator=g) if gate else None,
             keys1=torch.randn(H, n_sub, d_a // 2, generator=g), keys2=torch.randn(H, n_sub, d_a // 2, generator=g),
             addr_b=0.3 * torch.randn(H, d_a, generator=g),
             log_scale=math.log(8.0) + 0.3 * torch.randn(H, generator=g),
             decay=torch.tensor(decays, dtype=torch.float32) if decays is not None
             else 0.5 + 0.49 * torch.rand(H, generator=g),
             onorm_w=1.0 + 0.3 * torch.randn(H, dh, generator=g),
             gate_bias=0.4 * torch.randn(H, generator=g) if gate else None)
    for n in ("kz", "qz", "v", "gl"):   # the values a bf16 tensor holds, on both sides
        if t[n] is not None:
            t[n] = t[n].to(dtype).float()
    reset = (torch.rand(B, T, generator=g) < reset_p) if reset_p > 0 else None
    t["decay_grad"] = learn_decay
    return t, reset


def run_hip(t, reset, cfg, dtype, wgt):
    dev = {}
    for n in NAMES:
        x = t[n]
        if x is None:
            dev[n] = None
            continue
        dx = x.to("cuda").to(dtype if n in ("kz", "qz", "v", "gl") else torch.float32)
        dx.requires_grad_(n != "decay" or t["decay_grad"])
        dev[n] = dx
    c = dict(cfg, reset=None if reset is None else reset.to("cuda"), workspace=core.CoreWorkspace())
    r = core.SdmCoreFunction.apply(dev["kz"], dev["qz"], dev["v"], dev["gl"], dev["keys1"], dev["keys2"],
                                   dev["addr_b"], dev["log_scale"], dev["decay"], dev["onorm_w"], dev["gate_bias"], c)
    (r * wgt.to("cuda")).sum().backward()
    torch.cuda.synchronize()
    grads = {n: (None if dev[n] is None or dev[n].grad is None else dev[n].grad.float().cpu()) for n in NAMES}
    return r.detach().cpu(), grads, dev


def picks(dev, k):
    """The HIP picks of both address sets, (B, T, H, kk) int64 (core.address runs the training forward's kernel)."""
    kw = dict(addr_b=dev["addr_b"].detach())
    sw, _, _ = core.address(dev["kz"].detach(), dev["keys1"].detach(), dev["keys2"].detach(), k,
                            dev["log_scale"].detach(), **kw)
    sr, _, _ = core.address(dev["qz"].detach(), dev["keys1"].detach(), dev["keys2"].detach(), k,
                            dev["log_scale"].detach(), **kw)
    return sw.permute(0, 2, 1, 3).long().cpu(), sr.permute(0, 2, 1, 3).long().cpu()


def run_oracle(t, reset, cfg, siw, sir, wgt, H, d_a, dh):
    o = {}
    for n in NAMES:
        o[n] = None if t[n] is None else t[n].double().clone().requires_grad_(n != "decay" or t["decay_grad"])
    B, T = o["kz"].shape[:2]
    r = G.core_from_picks(o["kz"].view(B, T, H, d_a), o["qz"].view(B, T, H, d_a), o["v"].view(B, T, H, dh),
                          o["gl"], o["keys1"], o["keys2"], o["addr_b"], o["log_scale"], o["decay"],
                          o["onorm_w"] if cfg["out_norm"] else None, o["gate_bias"], siw, sir, cfg, reset=reset)
    r = r.reshape(B, T, H * dh)
    (r * wgt.double()).sum().backward()
    return r.detach(), {n: (None if o[n] is None or o[n].grad is None else o[n].grad) for n in NAMES}


def check_case(name, seed, B, T, H, dh, d_a, n_sub, k, dtype=torch.float32, read_mode="mean", out_norm=True,
               gate=True, decays=None, reset_p=0.0, overlap=0.0, learn_decay=True, tol=1e-4):
    say(f"[grad] {name}: B={B} T={T} H={H} dh={dh} d_a={d_a} n_sub={n_sub} k={k} {dtype} {read_mode} "
        f"norm={out_norm} gate={gate} reset_p={reset_p}")
    t, reset = make(seed, B, T, H, dh, d_a, n_sub, dtype, gate, decays, reset_p, overlap, learn_decay)
    cfg = dict(k=k, read_mode=read_mode, out_norm=out_norm, read_eps=1e-3, out_norm_eps=1e-2)
    wgt = torch.randn(B, T, H * dh, generator=torch.Generator().manual_seed(seed + 1000))
    r, grads, dev = run_hip(t, reset, cfg, dtype, wgt)
    siw, sir = picks(dev, k)
    r_ref, ref = run_oracle(t, reset, cfg, siw, sir, wgt, H, d_a, dh)
    err = (r.double() - r_ref).abs().max().item()
    assert err <= 2e-5 * max(1.0, r_ref.abs().max().item()), f"read-out differs by {err}"
    for n in NAMES:
        if ref[n] is None:
            assert grads[n] is None or n == "onorm_w", n
            continue
        scale = ref[n].abs().max().item()
        diff = (grads[n].double() - ref[n]).abs()
        # gradients of bfloat16 inputs are returned in bfloat16 (autograd's rule): half an ulp of rounding on top
        rounding = 2.0 ** -8 * ref[n].abs() if (dtype == torch.bfloat16 and n in ("kz", "qz", "v", "gl")) else 0.0
        excess = (diff - rounding).max().item()
        say(f"  d{n}: max err {diff.max().item():.3e} (past the output rounding {excess:.3e}) of scale {scale:.3e}")
        # a gradient whose own scale is below 1e-2 (cancellation in the softmax backward, e.g. at T = 2) is held to
        # 1e-6 absolute: the float32 rounding of the O(1) terms it is the difference of
        assert excess <= tol * max(scale, 1e-2), f"d{n}: max error {excess:.3e} vs scale {scale:.3e}"
    return grads


def test_grad_small_gate_mean_norm():
    check_case("small", 11, 2, 150, 3, 16, 16, 8, 8, overlap=0.7)


def test_grad_with_resets():
    check_case("resets", 12, 2, 200, 3, 16, 16, 8, 8, reset_p=0.03, overlap=0.7)


def test_grad_sum_mode_no_norm_no_gate_fixed_fades():
    check_case("plain", 13, 2, 130, 2, 8, 8, 6, 4, read_mode="sum", out_norm=False, gate=False,
               decays=[0.0, 1.0], learn_decay=False, overlap=0.5)


def test_grad_sixteen_picks():
    check_case("k16", 14, 1, 100, 2, 16, 8, 8, 16, overlap=0.7)


def test_grad_crowded_chunks_read_chains_past_the_staged_part():
    """n_sub = 4 gives M = 16 locations and k = 16 picks them all: every position writes every slot, so each chunk of
    both grad scans holds 64 * 16 - 16 = 1,008 later-writer chain entries, past the 384 a scan stages in LDS at
    k = 16; the rest are read from the chain plan in global memory."""
    check_case("crowded-k16", 21, 1, 200, 2, 16, 8, 4, 16, overlap=0.9)


def test_grad_layer_shape_bf16():
    """The layer shape of the validation workload (H=12, dh=64, d_a=64, M=1024, k=8), bfloat16 projections."""
    check_case("layer-bf16", 15, 1, 256, 12, 64, 64, 32, 8, dtype=torch.bfloat16, overlap=0.8, reset_p=0.01)


def test_backward_is_deterministic():
    t, reset = make(16, 1, 200, 4, 32, 16, 8, overlap=0.7)
    cfg = dict(k=8, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2)
    wgt = torch.randn(1, 200, 128, generator=torch.Generator().manual_seed(5))
    _, g1, _ = run_hip(t, reset, cfg, torch.float32, wgt)
    _, g2, _ = run_hip(t, reset, cfg, torch.float32, wgt)
    for n in NAMES:
        if g1[n] is not None:
            assert torch.equal(g1[n], g2[n]), n


def test_training_forward_equals_inference_forward():
    t, reset = make(17, 2, 190, 3, 16, 16, 8, overlap=0.7, reset_p=0.02)
    cfg = dict(k=8, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2)
    wgt = torch.zeros(2, 190, 48)
    r_train, _, dev = run_hip(t, reset, cfg, torch.float32, wgt)
    with torch.no_grad():
        r_inf = core.core_forward(dev["kz"], dev["qz"], dev["v"], dev["gl"], keys1=dev["keys1"], keys2=dev["keys2"],
                                  log_scale=dev["log_scale"], decay=dev["decay"], addr_b=dev["addr_b"],
                                  onorm_w=dev["onorm_w"], gate_bias=dev["gate_bias"], k=8,
                                  out_dtype=torch.float32, reset=reset.to("cuda"))
    assert torch.equal(r_train, r_inf.cpu())


# -- the module's training path -------------------------------------------------------------------------------------
def module_reference(m, x, reset, siw, sir):
    """float64 RunTimeSdm.forward of the module's parameters (prepare :195-213 with the oracle core, wo :247)."""
    P = {n: p.detach().double().cpu().clone().requires_grad_(p.requires_grad) for n, p in m.named_parameters()}
    x64 = x.detach().double().cpu().clone().requires_grad_(True)
    B, T, d = x64.shape
    H, d_a, dh = m.h, m.d_a, m.dh
    hx = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6) * P["norm.w"]
    kz = (hx @ P["wk.weight"].T).view(B, T, H, d_a)
    qz = (hx @ P["wq.weight"].T).view(B, T, H, d_a)
    V = (hx @ P["wv.weight"].T).view(B, T, H, dh)
    gl = hx @ P["wg.weight"].T + P["wg.bias"]
    lam = torch.sigmoid(P["decay_logit"]) if m.learn_decay else m.decays_fixed.double().cpu()
    cfg = dict(k=m.k, read_mode=m.read_mode, out_norm=m.out_norm, read_eps=m.read_eps, out_norm_eps=m.out_norm_eps)
    r = G.core_from_picks(kz, qz, V, gl, P["keys1"], P["keys2"], P["addr_b"], P["log_scale"], lam, P["onorm_w"],
                          None, siw, sir, cfg, reset=reset)
    y = r.reshape(B, T, d) @ P["wo.weight"].T
    return y, P, x64


def test_module_training_step_matches_the_oracle():
    torch.manual_seed(0)
    d, H, n_sub, d_a, k = 96, 4, 8, 16, 8
    m = RunTimeSdm(d, heads=H, n_sub=n_sub, d_a=d_a, k=k, decays=(0.6, 0.8, 0.95, 0.99), learn_decay=True,
                   addr_bias=0.2).to("cuda")
    for p in (m.wk.weight, m.wq.weight, m.wv.weight, m.wg.weight, m.wo.weight):
        torch.nn.init.xavier_uniform_(p)
    with torch.no_grad():
        m.wq.weight.copy_(0.7 * m.wk.weight + 0.3 * m.wq.weight)   # reads meet recent writes
        m.wg.bias.fill_(0.3)
    B, T = 2, 160
    x = torch.randn(B, T, d, device="cuda", requires_grad=True)
    reset = torch.rand(B, T, device="cuda") < 0.02
    say(f"[grad] module: B={B} T={T} d={d} H={H} n_sub={n_sub} d_a={d_a} k={k} learn_decay")
    y = m(x, reset)
    wgt = torch.randn(B, T, d, generator=torch.Generator().manual_seed(3)).to("cuda")
    (y * wgt).sum().backward()
    torch.cuda.synchronize()
    with torch.no_grad():   # the picks of the module's own projections (the same fused product)
        proj = torch.cat(m._project_train(x)[:2], -1)
        kz, qz = proj[..., :H * d_a], proj[..., H * d_a:2 * H * d_a]
        siw, _, _ = core.address(kz, m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)
        sir, _, _ = core.address(qz, m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)
    y_ref, P, x64 = module_reference(m, x, reset.cpu(), siw.permute(0, 2, 1, 3).long().cpu(),
                                     sir.permute(0, 2, 1, 3).long().cpu())
    assert (y.detach().double().cpu() - y_ref).abs().max().item() <= 2e-5 * max(1.0, y_ref.abs().max().item())
    (y_ref * wgt.double().cpu()).sum().backward()
    pairs = [("x", x.grad, x64.grad)] + [(n, p.grad, P[n].grad) for n, p in m.named_parameters()]
    for n, g, gr in pairs:
        scale = gr.abs().max().item()
        e = (g.double().cpu() - gr).abs().max().item()
        say(f"  d{n}: max err {e:.3e} of scale {scale:.3e}")
        assert e <= 1e-4 * max(scale, 1e-12), f"d{n}: {e:.3e} vs {scale:.3e}"
    # the module's inference forward gives the same output
    with torch.no_grad():
        y_inf = m(x.detach(), reset)
    assert (y_inf - y.detach()).abs().max().item() <= 1e-5 * max(1.0, y.abs().max().item())


@pytest.mark.parametrize("T", [1, 2, 63, 65, 129])
def test_grad_lengths_around_chunk_edges(T):
    """Sequence lengths of one position, a partial chunk, and just past one and two chunks of 64."""
    check_case(f"T={T}", 20 + T, 3, T, 2, 8, 8, 6, 4, overlap=0.7, reset_p=0.05)


def test_grad_sum_mode_with_resets_and_fixed_gate_free_fades():
    check_case("sum-resets", 30, 2, 140, 3, 16, 16, 8, 8, read_mode="sum", out_norm=True, gate=True,
               reset_p=0.04, overlap=0.6)


def test_grad_empty_batch_returns_nothing_to_do():
    t, _ = make(31, 1, 10, 2, 8, 8, 6)
    dev = {n: (None if t[n] is None else t[n].to("cuda")) for n in NAMES}
    z = torch.empty(0, 10, 16, device="cuda")
    r = core.SdmCoreFunction.apply(z.requires_grad_(True), z.clone().requires_grad_(True),
                                   torch.empty(0, 10, 16, device="cuda", requires_grad=True), None, dev["keys1"],
                                   dev["keys2"], None, dev["log_scale"], dev["decay"], dev["onorm_w"], None,
                                   dict(k=4, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2))
    assert r.shape == (0, 10, 16)


# -- a whole OneSdmLM training step ---------------------------------------------------------------------------------
def _rms64(x, w):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w


def _mixer64(P, pre, m, x, reset, siw, sir):
    """float64 RunTimeSdm.forward (prepare :195-213 with the oracle core, wo :247) from the parameter dict P."""
    B, T, d = x.shape
    H, d_a, dh = m.h, m.d_a, m.dh
    hx = _rms64(x, P[pre + "norm.w"])
    kz = (hx @ P[pre + "wk.weight"].T).view(B, T, H, d_a)
    qz = (hx @ P[pre + "wq.weight"].T).view(B, T, H, d_a)
    V = (hx @ P[pre + "wv.weight"].T).view(B, T, H, dh)
    gl = hx @ P[pre + "wg.weight"].T + P[pre + "wg.bias"]
    lam = torch.sigmoid(P[pre + "decay_logit"])
    cfg = dict(k=m.k, read_mode=m.read_mode, out_norm=m.out_norm, read_eps=m.read_eps, out_norm_eps=m.out_norm_eps)
    r = G.core_from_picks(kz, qz, V, gl, P[pre + "keys1"], P[pre + "keys2"], P[pre + "addr_b"], P[pre + "log_scale"],
                          lam, P[pre + "onorm_w"], None, siw, sir, cfg, reset=reset)
    return r.reshape(B, T, d) @ P[pre + "wo.weight"].T


def test_onesdm_training_step_matches_the_oracle():
    """Two layers of [x + RunTimeSdm(x); x + SwiGLU(RMSNorm x)], final norm, tied head, BOS resets and learned fades:
    every parameter's gradient of a weighted sum of the logits against a float64 autograd model that runs the same
    picks (each mixer's picks from its own input in the GPU forward)."""
    from sdmchat_amd import OneSdmLM
    torch.manual_seed(0)
    Vv, d, L, H, n_sub, d_a, k = 50, 96, 2, 4, 8, 16, 8
    model = OneSdmLM(Vv, d=d, layers=L, mlp_f=128, heads=H, n_sub=n_sub, d_a=d_a, k=k, decays=(0.6, 0.8, 0.95, 0.99),
                     learn_decay=True, addr_bias=0.2, reset_at_bos=True, bos_id=0).cuda()
    with torch.no_grad():   # the zero-start output maps and gate weights would leave the mixers silent
        for m in model.mems:
            torch.nn.init.xavier_uniform_(m.wo.weight)
            torch.nn.init.xavier_uniform_(m.wg.weight)
            m.wq.weight.copy_(0.7 * m.wk.weight + 0.3 * m.wq.weight)
    idx = torch.randint(1, Vv, (2, 120), generator=torch.Generator().manual_seed(1))
    idx[0, 40] = idx[1, 77] = 0   # BOS: the memory is emptied there
    idx = idx.cuda()
    inputs = {}
    hooks = [m.register_forward_pre_hook(lambda mod, args, i=i: inputs.__setitem__(i, args[0].detach()))
             for i, m in enumerate(model.mems)]
    say(f"[grad] OneSdmLM: layers={L} d={d} V={Vv} B=2 T=120, resets at BOS, learned fades")
    logits = model(idx)
    for hk in hooks:
        hk.remove()
    wgt = torch.randn(logits.shape, generator=torch.Generator().manual_seed(2)).cuda()
    (logits * wgt).sum().backward()
    torch.cuda.synchronize()
    picks = []
    with torch.no_grad():
        for i, m in enumerate(model.mems):
            proj = torch.cat(m._project_train(inputs[i])[:2], -1)
            sw = core.address(proj[..., :H * d_a], m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)[0]
            sr = core.address(proj[..., H * d_a:2 * H * d_a], m.keys1, m.keys2, k, m.log_scale, addr_b=m.addr_b)[0]
            picks.append((sw.permute(0, 2, 1, 3).long().cpu(), sr.permute(0, 2, 1, 3).long().cpu()))
    P = {n: p.detach().double().cpu().clone().requires_grad_(True) for n, p in model.named_parameters()}
    reset = (idx == 0).cpu()
    x = P["emb.weight"][idx.cpu()]
    for i, m in enumerate(model.mems):
        x = x + _mixer64(P, f"mems.{i}.", m, x, reset, *picks[i])
        hm = _rms64(x, P[f"mnorms.{i}.w"])
        x = x + (torch.nn.functional.silu(hm @ P[f"mlps.{i}.gate.weight"].T) * (hm @ P[f"mlps.{i}.up.weight"].T)) \
            @ P[f"mlps.{i}.down.weight"].T
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


def _small_module(**kw):
    torch.manual_seed(3)
    m = RunTimeSdm(96, heads=4, n_sub=8, d_a=16, k=8, decays=(0.6, 0.8, 0.95, 0.99), addr_bias=0.2, **kw).to("cuda")
    with torch.no_grad():
        for p in (m.wk.weight, m.wq.weight, m.wv.weight, m.wg.weight, m.wo.weight):
            torch.nn.init.xavier_uniform_(p)
        m.wq.weight.copy_(0.7 * m.wk.weight + 0.3 * m.wq.weight)
    return m


def test_mem_in_grad_scales_the_gradient_into_x():
    """grad_scale (track4_sdmllm_models.py:170-174): the mixer's gradient into x is scaled by mem_in_grad; 0 sends
    none, 0.5 half of what 1 sends."""
    x = torch.randn(2, 100, 96, device="cuda")
    wgt = torch.randn(2, 100, 96, device="cuda")
    grads = {}
    for a in (1.0, 0.5, 0.0):
        m = _small_module(mem_in_grad=a)
        xg = x.clone().requires_grad_(True)
        (m(xg) * wgt).sum().backward()
        grads[a] = xg.grad
    assert grads[0.0] is None or torch.count_nonzero(grads[0.0]) == 0   # detached: x gets no gradient at all
    torch.testing.assert_close(grads[0.5], 0.5 * grads[1.0], rtol=1e-5, atol=1e-7)
    assert grads[1.0].abs().max() > 0


def test_training_under_bf16_autocast_tracks_float32():
    """The reference trains under bf16 autocast: the projections and wo run in bf16, the core on the bf16 projections.
    Gradients stay finite and near the float32 path's.  This is a sanity check, not the parity bar (that is
    test_grad_layer_shape_bf16 against the oracle): bf16 projections move near-tie picks, which are discrete, so the
    two paths differ by a few percent (4-9% measured at this small shape, M = 64 locations)."""
    m = _small_module()
    x = torch.randn(2, 128, 96, device="cuda")
    wgt = torch.randn(2, 128, 96, device="cuda")
    out = {}
    for mode in ("f32", "bf16"):
        m.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=mode == "bf16"):
            y = m(xg)
        (y.float() * wgt).sum().backward()
        out[mode] = {n: p.grad.detach().clone() for n, p in m.named_parameters()}
        out[mode]["x"] = xg.grad.detach().clone()
    for n, g32 in out["f32"].items():
        g16 = out["bf16"][n]
        assert torch.isfinite(g16).all(), n
        rel = ((g16 - g32).norm() / g32.norm().clamp_min(1e-12)).item()
        say(f"  d{n}: relative difference bf16 vs f32 {rel:.3e}")
        assert rel < 0.25, (n, rel)
