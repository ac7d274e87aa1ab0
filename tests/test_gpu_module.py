"""GPU tests of the drop-in RunTimeSdm module against the fp64 oracle and the reference self-test's closed forms.

References: RunTimeSdm (track4_onesdm_models.py:151-300); self-test zero start (:703-712), gate (:756-772),
previous-token head (:773-785).
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import RunTimeSdm, core, synthetic as S
from tests._gpu_util import (DELTA, assert_close, check_picks, gpu_address, half_ulp_bf16, say,
                              scan_from_picks)

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


def _bf16(a):
    """float values rounded to bfloat16 (nearest even), as float64."""
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).double().numpy()


def _autocast_norm(x, w):
    """The reference's input norm before bf16 autocast's cast: bf16(bf16(x * rsqrt(mean x^2 + eps)) * w)
    (RMSNorm, SM:69-71), the scale in float32."""
    xf = np.asarray(x, np.float32)
    r = (1.0 / np.sqrt(np.mean(xf.astype(np.float64) ** 2, -1, keepdims=True) + 1e-6)).astype(np.float32)
    return _bf16(_bf16(xf * r) * np.asarray(w, np.float32))


def _autocast_projections(hx, p):
    """The reference's projections under bf16 autocast (OM:199-205), restated: bf16(hx . bf16(W)^T + bf16(b)) with
    the sum in float64.  Returns, per projection, the value and the sum of the |terms| (its error scale)."""
    out = {}
    for n in ("wk", "wq", "wv", "wg"):
        w = _bf16(p[f"{n}.weight"])
        y = hx @ w.T
        if n == "wg":
            y = y + _bf16(p["wg.bias"])
        out[n] = (_bf16(y), np.abs(hx) @ np.abs(w).T)
    return out


def test_module_bf16_end_to_end():
    """bf16 x -> y at the bench shape (B=8, T=2048, d=768, H=12, M=1,024, k=8), every stage against an
    independent restatement: the norm and the four projections against the reference's autocast roundings (at most
    one bf16 ulp apart, on under 0.1% of the values: the GEMM sums in a different order); every pick against the
    fp64 oracle (margin rule); then, for batch rows 0 and 7, the read-out of all 12 heads from the fp64 recurrence
    and y = bf16(r) wo^T in float64 (OM:247 under autocast), within 2e-3 plus half a bf16 ulp.  The gate bias is
    non-zero, so the gate logit's rounding (bf16(W_g hx + b), OM:205) is exercised."""
    cfg = S.layer_cfg()
    p = S.layer_params(cfg, seed=63)
    rng = np.random.Generator(np.random.PCG64(630))
    p["wg.bias"] = rng.uniform(-1.0, 1.0, 12).astype(np.float32)
    p["onorm_w"] = rng.uniform(0.5, 1.5, (12, 64)).astype(np.float32)
    x = _bf16(S.layer_input(8, 2048, 768, seed=64)).astype(np.float32)
    m = build(cfg, p)
    say("module bf16 end to end, B=8 T=2048")
    xd = torch.from_numpy(x).cuda().to(torch.bfloat16)
    with torch.no_grad():
        y = m(xd).float().cpu().numpy()
        kz, qz, V, g = (t.float().cpu().numpy() for t in m._project(xd, torch.bfloat16))
        hx = core.rms_norm(xd, m.norm.w, m.norm.eps, out_dtype=torch.bfloat16).double().cpu().numpy()
    rows = [0, 7]
    # the norm: the kernel sums the squares in another order, so a value may round the other way (two bf16 ulps)
    hx_ref = _autocast_norm(x[rows], p["norm.w"])
    dn = np.abs(hx[rows] - hx_ref)
    assert np.all(dn <= 4.0 * half_ulp_bf16(hx_ref)), "the input norm is more than two bf16 ulps off"
    say(f"  norm: {float(np.mean(dn > 0)):.2e} of the values differ from the float64 scale")
    assert float(np.mean(dn > 0)) < 1e-3
    # the projections of the kernel's normalised rows against float64 sums rounded to bf16
    ref = _autocast_projections(hx[rows], p)
    for name, got in (("wk", kz), ("wq", qz), ("wv", V), ("wg", g)):
        want, terms = ref[name]
        d = np.abs(got[rows].astype(np.float64) - want)
        # one bf16 ulp, plus the float32 accumulation error of a 768-term sum (768 * 2^-24 of the |terms|)
        lim = 2.0 * half_ulp_bf16(want) + 768 * 2.0 ** -24 * terms
        if not np.all(d <= lim):
            i = np.unravel_index(np.argmax(d - lim), d.shape)
            raise AssertionError(f"{name}: {int((d > lim).sum())} values past the bound; worst at {i}: got "
                                 f"{got[rows][i]!r} want {want[i]!r} terms {terms[i]!r}")
        frac = float(np.mean(d > 0))
        say(f"  {name}: {frac:.2e} of the values differ from the float64 sum rounded to bf16")
        assert frac < 2e-3, f"{name}: {frac:.2e} of the values differ"
    po = dict(keys1=p["keys1"], keys2=p["keys2"], addr_b=p["addr_b"], log_scale=p["log_scale"],
              decay=p["decays_fixed"], onorm_w=p["onorm_w"], gate_bias=np.zeros(12, np.float32))
    siw, _, ww = gpu_address(kz, po, 8, dtype=torch.bfloat16, gate=g)
    sir, _, wr = gpu_address(qz, po, 8, dtype=torch.bfloat16)
    flips = check_picks(kz, po, 8, siw, ww, g) + check_picks(qz, po, 8, sir, wr)
    say("picks that differ from the fp64 oracle (near-ties):", flips)
    wo = _bf16(p["wo.weight"])
    for b in rows:
        r, _ = scan_from_picks(siw[b:b + 1], ww[b:b + 1], sir[b:b + 1], wr[b:b + 1], V[b:b + 1], p["decays_fixed"],
                               12, "mean", True, p["onorm_w"], 1024)
        assert_close(y[b:b + 1], _bf16(r) @ wo.T, 2e-3, bf16_out=True, msg=f"y, batch row {b}")


def test_module_bf16_eval_equals_training_forward():
    """The inference forward and the differentiable forward (bf16 autocast, x requiring grad) of one module give the
    same bits: the same norm kernel, the same fused projection with the gate bias, the same core and wo."""
    cfg = S.layer_cfg()
    p = S.layer_params(cfg, seed=67)
    p["wg.bias"] = np.random.Generator(np.random.PCG64(670)).uniform(-1.0, 1.0, 12).astype(np.float32)
    m = build(cfg, p)
    x = torch.from_numpy(S.layer_input(2, 512, 768, seed=671)).cuda().to(torch.bfloat16)
    say("module eval vs training forward")
    with torch.no_grad():
        y_eval = m(x)
    xg = x.clone().requires_grad_(True)
    with torch.enable_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y_train = m(xg)
    assert y_train.dtype == y_eval.dtype == torch.bfloat16
    assert torch.equal(y_train.detach(), y_eval), float((y_train.detach().float() - y_eval.float()).abs().max())


def test_module_output_map_cache_follows_in_place_changes():
    """An in-place change of wo alone (no_grad) reaches the next bf16 forward: doubling wo doubles y exactly."""
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    m = build(cfg, S.layer_params(cfg, seed=69))
    x = torch.randn(2, 40, 64, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        y1 = m(x)
        m.wo.weight.mul_(2.0)
        y2 = m(x)
        m.wg.bias.add_(0.75)          # the gate bias lives in the fused projection: it must follow too
        y3 = m(x)
        m.wg.bias.sub_(0.75)
        y4 = m(x)
    assert torch.equal(y2, 2 * y1)
    assert not torch.equal(y3, y2)
    assert torch.equal(y4, y2)


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


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_last_gate_is_kept_apart_and_last_state_is_loud(dt):
    """After an inference forward the gate logits are the [B, T, H] copy the forward left in the module's own
    workspace (sdm_rt_gate_copy_offset; not a view that keeps the fused projection's buffer alive), equal to the
    projections' gate logits bit for bit, last_gate is their sigmoid, a second forward's gate replaces the first's,
    and reading last_state after a forward that did not write it (keep_state unset) raises instead of returning
    None; with keep_state it holds the state."""
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    p = S.layer_params(cfg, seed=70)
    m = build(cfg, p)
    x = torch.from_numpy(S.layer_input(2, 50, 64, seed=1070)).cuda().to(dt)
    x2 = torch.from_numpy(S.layer_input(2, 50, 64, seed=1071)).cuda().to(dt)
    for xx in (x2, x):
        with torch.no_grad():
            m(xx)
    g = m._gate_src[0]
    assert tuple(g.shape) == (2, 50, 4) and g.dtype == dt
    assert g.untyped_storage().data_ptr() == m._ws.buf.untyped_storage().data_ptr()   # the workspace's copy
    with torch.no_grad():
        g_ref = m._project(x, dt)[3]
    assert torch.equal(g, g_ref)
    gate = m.last_gate
    assert torch.equal(gate, torch.sigmoid(g_ref.float()))
    assert tuple(gate.shape) == (2, 50, 4) and float(gate.min()) >= 0 and float(gate.max()) <= 1
    with pytest.raises(RuntimeError, match="keep_state"):
        _ = m.last_state
    m.keep_state = True
    with torch.no_grad():
        m(x)
    mem, cnt = m.last_state
    assert tuple(mem.shape) == (2, 4, 64, 16) and tuple(cnt.shape) == (2, 4, 64)
