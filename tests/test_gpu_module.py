"""GPU tests of the drop-in RunTimeSdm module against the fp64 oracle and the reference self-test's closed forms.

References: RunTimeSdm (track4_onesdm_models.py:151-300); self-test zero start (:703-712), gate (:756-772),
previous-token head (:773-785).
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import RunTimeSdm, synthetic as S
from tests._gpu_util import DELTA, assert_close, check_core, say

pytestmark = pytest.mark.gpu


def build(cfg, p):
    m = RunTimeSdm(cfg["d"], heads=cfg["heads"], n_sub=cfg["n_sub"], d_a=cfg["d_a"], k=cfg["k"],
                   decays=tuple(float(v) for v in p["decays_fixed"]), write_gate=cfg.get("write_gate", True),
                   out_norm=cfg.get("out_norm", True), read_mode=cfg.get("read_mode", "mean"))
    m.load_state_dict({k: torch.from_numpy(v) for k, v in p.items()}, strict=True)
    return m.cuda().eval()


def _p64(p):
    q = {k: v.astype(np.float64) for k, v in p.items()}
    q["decay"] = q["decays_fixed"]
    return q


def test_module_fp32_end_to_end():
    """The fp32 validation workload (B=1, T=256, d=768, H=12, M=1024, k=8) from x to y against the fp64 oracle."""
    cfg = S.layer_cfg()
    p = S.layer_params(cfg, seed=62)           # seeds chosen so that no address has an fp64 margin below 2e-6
    x = S.layer_input(1, 256, 768, seed=1062)
    hx = O.rms_norm(x, np.ones(768))
    for w in ("wk.weight", "wq.weight"):
        z = (hx @ p[w].T.astype(np.float64)).reshape(256, 12, 64)
        assert O.topk_margin(z, p["keys1"], p["keys2"], 8).min() > DELTA
    m = build(cfg, p)
    say("module fp32")
    with torch.no_grad():
        y = m(torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.layer_forward(x, _p64(p), cfg)
    np.testing.assert_allclose(y, want, atol=1e-5, rtol=1e-5)
    assert m.last_gate.shape == (1, 256, 12)
    assert float(m.last_gate.min()) >= 0 and float(m.last_gate.max()) <= 1


def test_module_bf16_core_and_output_map():
    """bf16 activations: the core on the module's own projections (picks against the oracle, read-out against the
    fp64 recurrence on those picks), and y against the output map applied in float64 to the read-out (2e-3 plus half
    a bf16 ulp for the bf16 outputs)."""
    cfg = S.layer_cfg()
    p = S.layer_params(cfg, seed=63)
    x = torch.from_numpy(S.layer_input(2, 512, 768, seed=64)).cuda().to(torch.bfloat16)
    m = build(cfg, p)
    say("module bf16")
    with torch.no_grad():
        kz, qz, V, g = m._project(x, torch.bfloat16)
        y = m(x)
    f = [t.float().cpu().numpy() for t in (kz, qz, V, g)]
    po = dict(keys1=p["keys1"], keys2=p["keys2"], addr_b=p["addr_b"], log_scale=p["log_scale"],
              decay=p["decays_fixed"], onorm_w=p["onorm_w"], gate_bias=p["wg.bias"])
    check_core(*f, po, 8, dtype=torch.bfloat16, tol=2e-3)
    with torch.no_grad():
        from sdmchat_amd import core
        r = core.core_forward(kz, qz, V, g, keys1=m.keys1, keys2=m.keys2, log_scale=m.log_scale, decay=m.decay(),
                              addr_b=m.addr_b, onorm_w=m.onorm_w, gate_bias=m.wg.bias, k=8)
    wo = m.wo.weight.detach().to(torch.bfloat16).double().cpu().numpy()
    want_y = r.double().cpu().numpy() @ wo.T
    assert_close(y.float().cpu().numpy(), want_y, 2e-3, bf16_out=True, msg="y = r wo^T")


def test_zero_output_map_gives_exact_zero():
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    m = build(cfg, S.layer_params(cfg, seed=65))
    m.reset_init()
    with torch.no_grad():
        y = m(torch.randn(2, 50, 64, device="cuda"))
    assert torch.count_nonzero(y) == 0
    m.enabled = False
    with torch.no_grad():
        assert torch.count_nonzero(m(torch.randn(2, 50, 64, device="cuda"))) == 0


def test_previous_token_head():
    """Fade 0 and one shared address: y[t] = V[t-1] * (1/k) / (1/k + eps) and y[0] = 0 exactly."""
    torch.manual_seed(0)
    r = RunTimeSdm(8, heads=1, n_sub=4, d_a=4, k=4, decays=(0.0,), write_gate=False, out_norm=False, chunk=3)
    torch.nn.init.zeros_(r.wq.weight)
    torch.nn.init.zeros_(r.wk.weight)
    torch.nn.init.eye_(r.wo.weight)
    r = r.cuda().eval()
    x = torch.randn(1, 9, 8, device="cuda")
    with torch.no_grad():
        y = r(x)
        V = r.wv(r.norm(x).float())
    want = V[0, :-1] * 0.25 / (0.25 + r.read_eps)
    torch.testing.assert_close(y[0, 1:], want, atol=1e-5, rtol=1e-5)
    assert float(y[0, 0].abs().max()) == 0.0


def test_gate_near_zero_writes_nothing():
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    m = build(cfg, S.layer_params(cfg, seed=66))
    torch.nn.init.zeros_(m.wg.weight)
    torch.nn.init.constant_(m.wg.bias, -30.0)
    with torch.no_grad():
        y = m(torch.randn(1, 40, 64, device="cuda"))
    assert float(y.abs().max()) < 1e-6


def test_last_state_matches_oracle():
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    p = S.layer_params(cfg, seed=68, decays=(0.0, 0.5, 0.95, 1.0))   # no fp64 margin below 2e-6
    m = build(cfg, p)
    m.keep_state = True
    x = S.layer_input(2, 90, 64, seed=1068)
    hx = O.rms_norm(x, np.ones(64))
    for w in ("wk.weight", "wq.weight"):
        z = (hx @ p[w].T.astype(np.float64)).reshape(180, 4, 16)
        assert O.topk_margin(z, p["keys1"], p["keys2"], 8).min() > DELTA
    with torch.no_grad():
        y = m(torch.from_numpy(x).cuda())
    mem, cnt = m.last_state
    pp = _p64(p)
    B, T, H = 2, 90, 4
    kz = (hx @ pp["wk.weight"].T).reshape(B, T, H, 16)
    qz = (hx @ pp["wq.weight"].T).reshape(B, T, H, 16)
    V = (hx @ pp["wv.weight"].T).reshape(B, T, H, 16)
    gl = hx @ pp["wg.weight"].T + pp["wg.bias"]
    _, parts = O.core_forward(kz, qz, V, gl, dict(keys1=pp["keys1"], keys2=pp["keys2"], log_scale=pp["log_scale"],
                                                  decay=pp["decay"], onorm_w=pp["onorm_w"]),
                              dict(k=8), return_parts=True)
    np.testing.assert_allclose(mem.cpu().numpy(), parts["mem"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt.cpu().numpy(), parts["cnt"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(y.cpu().numpy(), O.layer_forward(x, pp, cfg), atol=1e-5, rtol=1e-5)
