"""The bfloat16 whole model and its decode (configs 3-5: the PARTIAL and FULL OneSdmLM at d 768, 12 layers,
vocabulary 32,768, bf16 weights and activations, float32 memory; forward OM:525-555, decode OM:276-300 and 534-555)
against the fp64 oracle evaluated with the same bfloat16 casts (oracle.sdm_fp64 with round=bf16: after each map,
norm, silu, product, read-out, residual sum and the logits), stage by stage.

Every stage of the GPU run is checked on the GPU's own input to that stage: each mixer's output against
oracle.layer_forward of the mixer's input, each SwiGLU's input norm and output, each TrainedSdm's output, and the
logits against the final norm and tied head of the last residual sum, each within rtol 2e-3 / atol 2e-3 plus one
bfloat16 unit (both sides round each output to bfloat16, so a value whose unrounded sums straddle a rounding boundary
lands one unit apart).  Each sub-stage is fed the GPU's own input: the mixer's input norm, its four maps on the
GPU's normed input, and its core and output map on the GPU's projections, where the oracle's picks may differ from
the kernel's only at float32 score ties (DELTA, adopt_picks; the count is printed).  Why stage by stage: the GPU sums in float32 and the oracle in
float64, so an occasional value rounds to the neighbouring bfloat16, and across 12 layers these one-unit differences
compound (run from the tokens alone, the two evaluations' address scores drift apart by up to ~6e-3 by the last
layers), so a comparison of the logits from the tokens alone measures that drift (printed) rather than any one
stage.

- forward, B=1, T=128, both arms;
- decode (config 5's workload, shortened): 64 FULL-arm streams, 256 steps, on the steps' own picks;
- decode at full length: 64 streams x 32,768 steps: logits stay finite, streams are independent (a second batch that
  shares half the streams' tokens gives those streams bit-identical logits at every step), and a stream that meets a
  BOS equals, bit for bit, a fresh stream fed the same tokens from that BOS on;
- the layer's decode step over 32,768 steps (4 streams, bf16) against the fp64 recurrence on the kernel's picks,
  with fades 0.3, 0.5 and 1 among the heads (the state's scale is folded back into the slab every ~60 steps at 0.5).
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import DecodeGraph, core, synthetic as S
from tests._gpu_util import assert_close, bf16_round, core_inputs, gpu_address, gpu_decode, half_ulp_bf16, say

pytestmark = pytest.mark.gpu
ARMS = ["swiglu", "trained_sdm"]
# the tolerance of the run from the tokens alone (reported, not a bound): there the oracle's addresses drift from the
# GPU's by up to ~6e-3 in the last layers
DRIFT_TOL = 1e-2


def _cfg(m, rnd=O.bf16, log=None):
    c = dict(layers=m.n_layers, heads=m.mems[0].h, d_a=m.mems[0].d_a, k=m.mems[0].k, ffn=m.ffn,
             reset_at_bos=m.reset_at_bos, bos_id=m.bos_id, round=rnd, adopt_tol=DRIFT_TOL, adopt_log=log)
    if m.ffn == "sdm":
        s = m.sdms[0]
        c.update(sdm_heads=s.h, sdm_d_a=s.d_a, sdm_k=s.k)
    return c


def _params64(m):
    return {n: v.detach().double().cpu().numpy() for n, v in m.state_dict().items()}


def _close(got, want, what):
    """Two bfloat16 results of the same stage: |got - want| <= 2e-3 + 2e-3 |want| + one bfloat16 unit of want (both
    sides round their output, so values whose unrounded sums straddle a rounding boundary land one unit apart)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    lim = 2e-3 + 2e-3 * np.abs(want) + 2.0 * half_ulp_bf16(want)
    bad = np.abs(got - want) > lim
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} off; worst excess "
                           f"{float((np.abs(got - want) - lim).max()):.3e}")
    return float((np.abs(got - want) / lim).max())


def _check_logits(got, h, p, what, rows=2048):
    """GPU logits (..., V) against the oracle's hidden state h (..., d) times emb.weight^T rounded to bfloat16, in
    pieces of `rows` tokens; returns the largest |error| / (2e-3 + 2e-3 |want| + half a bf16 unit)."""
    E = p["emb.weight"]
    g2 = got.reshape(-1, got.shape[-1])
    h2 = h.reshape(-1, h.shape[-1])
    worst = 0.0
    for i in range(0, h2.shape[0], rows):
        want = O.bf16(h2[i:i + rows] @ E.T)
        worst = max(worst, _close(g2[i:i + rows].double().cpu().numpy(), want, f"{what}, tokens {i}..{i + rows}"))
    return worst


def _cat(ts, B):
    """Per-call tensors (B, t, w) or (B, w) -> (B, T, w) float64 numpy."""
    return torch.cat([t.reshape(B, -1, t.shape[-1]) for t in ts], 1).double().cpu().numpy()


class _Stages:
    """Records every stage call of a OneSdmLM run (forward, or the steps of a decode), stacked along the position
    axis: each mixer's input x, normed input hx, projections (kz, qz, V, gate logits), picks and output y; each
    SwiGLU's normed input and output; each TrainedSdm's input, normed input, query, picks and output."""

    def __init__(self, m):
        self.m = m
        self.rec = {}
        for i, mm in enumerate(m.mems):
            mm.keep_picks = True
            for name in ("forward", "step"):
                self._wrap(mm, name, ("mem", i))
            self._wrap_step_residual(mm, ("mem", i))
            self._wrap_step_embed(mm, ("mem", i))
        for i, sd in enumerate(getattr(m, "sdms", [])):
            sd.keep_picks = True
            self._wrap(sd, "forward", ("sdm", i))
            self._wrap_residual(sd, ("sdm", i))
        for i, ml in enumerate(getattr(m, "mlps", [])):
            self._wrap(ml, "forward", ("mlp", i))

    def _wrap(self, mod, name, key):
        orig = getattr(mod, name)

        def f(*a, **kw):
            x = a[0].detach().clone()
            hx = kw.get("hx")
            hx = None if hx is None else hx.detach().clone()
            out = orig(*a, **kw)
            r = dict(x=x, hx=hx, y=out.detach().clone())
            if key[0] == "mem":
                r["proj"] = tuple(t.detach().clone() for t in mod.last_projections)
                r["picks"] = tuple(s_[..., :mod.k] for s_ in mod.last_picks)
            elif key[0] == "sdm":
                r["q"] = mod.last_q.detach().clone()
                r["picks"] = mod.last_si
            self.rec.setdefault(key, []).append(r)
            return out
        setattr(mod, name, f)

    def _wrap_residual(self, mod, key):
        """TrainedSdm.forward_residual (the add in front of the layer folded into its table step): the layer's input
        is the returned sum, its normed input the kernel's hx (last_hx)."""
        orig = mod.forward_residual

        def f(x, y):
            s, out = orig(x, y)
            r = dict(x=s.detach().clone(), hx=mod.last_hx.detach().clone().reshape(s.shape), y=out.detach().clone(),
                     q=mod.last_q.detach().clone(), picks=mod.last_si)
            self.rec.setdefault(key, []).append(r)
            return s, out
        mod.forward_residual = f

    def _wrap_step_residual(self, mod, key):
        """RunTimeSdm.step_residual (the add in front of the mixer folded into its projection map): the mixer's input
        is the returned sum; its normed input, which the folded map keeps on chip, is the norm kernel's on that sum
        (the same bits: test_gemm_rows_residual_equals_add_norm_then_gemm_rows)."""
        orig = mod.step_residual

        def f(x, y, *a, **kw):
            s, out = orig(x, y, *a, **kw)
            hx = core.rms_norm(s, mod.norm.w, mod.norm.eps, out_dtype=torch.bfloat16)
            r = dict(x=s.detach().clone(), hx=hx, y=out.detach().clone(),
                     proj=tuple(t.detach().clone() for t in mod.last_projections),
                     picks=tuple(s_[..., :mod.k] for s_ in mod.last_picks))
            self.rec.setdefault(key, []).append(r)
            return s, out
        mod.step_residual = f

    def _wrap_step_embed(self, mod, key):
        """RunTimeSdm.step_embed (the embedding gather and the first norm folded into the first mixer's projection
        map): the mixer's input is the returned gathered rows; its normed input is the norm kernel's on them (the
        same bits: test_gemm_rows_embed_equals_gather_norm_then_gemm_rows)."""
        orig = mod.step_embed

        def f(idx, table, *a, **kw):
            x, out = orig(idx, table, *a, **kw)
            hx = core.rms_norm(x, mod.norm.w, mod.norm.eps, out_dtype=torch.bfloat16)
            r = dict(x=x.detach().clone(), hx=hx, y=out.detach().clone(),
                     proj=tuple(t.detach().clone() for t in mod.last_projections),
                     picks=tuple(s_[..., :mod.k] for s_ in mod.last_picks))
            self.rec.setdefault(key, []).append(r)
            return x, out
        mod.step_embed = f

    def get(self, key, B):
        rec = self.rec[key]
        out = {n: _cat([r[n] for r in rec], B) for n in ("x", "y")}
        if rec[0]["hx"] is not None:
            out["hx"] = _cat([r["hx"] for r in rec], B)
        if key[0] == "mem":
            out["proj"] = [_cat([r["proj"][j] for r in rec], B) for j in range(4)]
            T = out["x"].shape[1]   # (B, H, t, kk) per call -> (B * T, H, kk), token order b * T + t
            out["picks"] = tuple(torch.cat([r["picks"][j] for r in rec], 2).permute(0, 2, 1, 3)
                                 .reshape(B * T, -1, rec[0]["picks"][j].shape[-1]).cpu().numpy() for j in range(2))
        elif key[0] == "sdm":
            out["q"] = _cat([r["q"] for r in rec], B)
            T = out["x"].shape[1]
            out["picks"] = torch.cat([r["picks"].reshape(B, -1, *r["picks"].shape[1:]) for r in rec], 1) \
                .reshape(B * T, *rec[0]["picks"].shape[1:]).cpu().numpy()
        return out


def _norm_ok(got, x, w, what):
    """The GPU's RMSNorm kernel against the oracle's bfloat16 norm: at most two bfloat16 units apart (it sums the
    squares in another order)."""
    want = O.rms_norm(x, w, rnd=O.bf16)
    assert np.all(np.abs(got - want) <= 4.0 * half_ulp_bf16(want)), f"{what}: the input norm is more than two units off"


def _map_ok(got, hx, W, bias, what):
    """A bfloat16 map of the GPU's own normed input against the float64 sum rounded to bfloat16: one unit, plus the
    float32 accumulation error of a k-term sum (k 2^-24 of the |terms|)."""
    want = O.bf16(hx @ W.T + (0.0 if bias is None else bias))
    terms = np.abs(hx) @ np.abs(W).T
    lim = 2.0 * half_ulp_bf16(want) + hx.shape[-1] * 2.0 ** -24 * terms
    assert np.all(np.abs(got - want) <= lim), f"{what}: more than one unit off"


def _check_stages(m, rec, p, logits, idx, what):
    """Every stage of the recorded run against the oracle on the GPU's own inputs to it: the input norms and maps,
    the mixer's core and output map on the GPU's projections (the picks can then differ only at float32 score ties,
    DELTA), SwiGLU on its normed input, TrainedSdm on its query; then the logits on the GPU's last residual sum.
    Returns the adoption counts."""
    from tests._gpu_util import DELTA
    B, T = idx.shape
    reset = (idx == m.bos_id) if m.reset_at_bos else None
    log = []
    x_after = None
    H, d_a = m.mems[0].h, m.mems[0].d_a
    d = m.d
    for i in range(m.n_layers):
        r = rec.get(("mem", i), B)
        X, hx, Y = r["x"], r["hx"], r["y"]
        if x_after is not None:   # the mixer's input is the last stage's residual sum
            assert np.array_equal(X, x_after), f"layer {i}: the residual stream is not the last stage's sum"
        pre = f"mems.{i}."
        lp = {n[len(pre):]: v for n, v in p.items() if n.startswith(pre)}
        _norm_ok(hx, X, lp["norm.w"], f"{what}: mixer {i}")
        kz, qz, V, g = r["proj"]
        for name, got, bias in (("wk", kz, None), ("wq", qz, None), ("wv", V, None), ("wg", g, lp["wg.bias"])):
            _map_ok(got, hx, lp[f"{name}.weight"], bias, f"{what}: mixer {i} {name}")
        core_p = dict(keys1=lp["keys1"], keys2=lp["keys2"], log_scale=lp["log_scale"], decay=lp["decays_fixed"],
                      onorm_w=lp["onorm_w"])
        ccfg = dict(k=m.mems[i].k, adopt_tol=DELTA, adopt_log=log)
        rr = O.core_forward(kz.reshape(B, T, H, d_a) + lp["addr_b"], qz.reshape(B, T, H, d_a) + lp["addr_b"],
                            V.reshape(B, T, H, d // H), g, core_p, ccfg, reset=reset, forced=r["picks"])
        y_ref = O.bf16(O.bf16(rr.reshape(B, T, d)) @ lp["wo.weight"].T)
        _close(Y, y_ref, f"{what}: mixer {i}'s core and output map")
        R = O.bf16(X + Y)
        if m.ffn == "mlp":
            r2 = rec.get(("mlp", i), B)
            _norm_ok(r2["x"], R, p[f"mnorms.{i}.w"], f"{what}: SwiGLU {i}")
            y2 = O.swiglu(r2["x"], p[f"mlps.{i}.gate.weight"], p[f"mlps.{i}.up.weight"], p[f"mlps.{i}.down.weight"],
                          rnd=O.bf16)
        else:
            r2 = rec.get(("sdm", i), B)
            assert np.array_equal(r2["x"], R), f"layer {i}: TrainedSdm's input is not the mixer's residual sum"
            pre = f"sdms.{i}."
            sp = {n[len(pre):]: v for n, v in p.items() if n.startswith(pre)}
            sd = m.sdms[i]
            _norm_ok(r2["hx"], R, sp["norm.w"], f"{what}: TrainedSdm {i}")
            _map_ok(r2["q"], r2["hx"], sp["wq.weight"], None, f"{what}: TrainedSdm {i} wq")
            q = r2["q"].reshape(B * T, sd.h, sd.d_a)
            sv, si = O.pk_address(q, sp["keys1"], sp["keys2"], sd.k)
            sv, si = O.adopt_picks(q, sp["keys1"], sp["keys2"], sv, si, r2["picks"], DELTA, log)
            tr = O.table_read(si, O.address_weights(sv, sp["log_scale"]), sp["values"]).reshape(B, T, d)
            y2 = O.bf16(O.bf16(tr) @ sp["wo.weight"].T)
        _close(r2["y"], y2, f"{what}: layer {i}'s {m.ffn}")
        x_after = O.bf16(R + r2["y"])
    h = O.rms_norm(x_after, p["nf.w"], rnd=O.bf16)
    _check_logits(logits, h, p, f"{what}: logits")
    return log


@pytest.mark.parametrize("arm", ARMS)
def test_full_model_bf16_stages_and_logits_match_oracle(arm):
    """The bfloat16 forward (B=1, T=128) stage by stage on the GPU's own stage inputs; then, for the record, the
    logits of the oracle run from the tokens alone (its own residual stream, the GPU's picks adopted within 1e-2)."""
    m = S.full_model(arm).cuda().to(torch.bfloat16).eval()
    p = _params64(m)
    idx = S.model_tokens(1, 128, seed=44)
    rec = _Stages(m)
    say("full model bf16 stages", arm)
    with torch.no_grad():
        got = m(torch.from_numpy(idx).cuda())
    log = _check_stages(m, rec, p, got, idx, arm)
    say(f"  stage checks passed; {sum(log)} addresses took the GPU's pick at a bf16 tie ({len(log)} addressings)")
    # from the tokens alone: the drift of two bfloat16 evaluations (reported, not a parity bound)
    forced = {}
    for i in range(m.n_layers):
        forced[("mem", i)] = rec.get(("mem", i), 1)["picks"]
        if arm == "trained_sdm":
            forced[("sdm", i)] = rec.get(("sdm", i), 1)["picks"]
    log2 = []
    want = O.model_forward(idx, p, _cfg(m, log=log2), forced=forced)
    g = got.double().cpu().numpy()
    scale = np.abs(want).max()
    top1 = float(np.mean(g.argmax(-1) == want.argmax(-1)))
    say(f"  from the tokens alone: max |logit difference| / scale {np.abs(g - want).max() / scale:.2e}, top-1 "
        f"agreement {top1:.3f}, {sum(log2)} addresses adopted within {DRIFT_TOL:.0e}")


def test_config5_decode_bf16_stages_match_oracle():
    """64 FULL-arm streams decoded for 256 steps in bfloat16 (config 5's workload, shortened): every stage of every
    step on the steps' own inputs and picks (the oracle runs each stage over all 256 positions of its recorded
    inputs: the mixer's recurrence sees the same history), and every position's logits."""
    m = S.full_model("trained_sdm").cuda().to(torch.bfloat16).eval()
    p = _params64(m)
    B, T = 64, 256
    idx = S.model_tokens(B, T, seed=45)
    rec = _Stages(m)
    say("config 5 decode bf16 stages", B, "streams", T, "steps")
    tok = torch.from_numpy(idx).cuda()
    with torch.no_grad():
        st = m.decode_state(B)
        got = torch.stack([m.step(tok[:, t], st) for t in range(T)], 1)   # (B, T, V)
    log = _check_stages(m, rec, p, got, idx, "decode")
    say(f"  {sum(log)} addresses took the step's pick at a bf16 tie ({len(log)} addressings)")


def test_config5_decode_full_length_properties():
    """64 FULL-arm streams, 32,768 steps, bfloat16, HIP graphs of 64 steps.  Run A and run B share the tokens of
    streams 0-31 and differ in streams 32-63: at every step the logits of streams 0-31 are bit-identical in both
    (one stream's output does not depend on another's tokens) and finite; stream 5 meets a BOS (token 7) at step
    s = 30,720, and a fresh stream fed stream 5's tokens from s on gives bit-identical logits for 2,048 steps."""
    m = S.full_model("trained_sdm", reset_at_bos=True, bos_id=7).cuda().to(torch.bfloat16).eval()
    B, steps, total, s_bos = 64, 64, 32768, 30720
    gen = torch.Generator(device="cuda").manual_seed(46)
    say("config 5 decode full length", B, "streams", total, "steps")
    ok = torch.ones((), dtype=torch.bool, device="cuda")
    fin = torch.ones((), dtype=torch.bool, device="cuda")
    fresh_ok = torch.ones((), dtype=torch.bool, device="cuda")
    with torch.no_grad():
        sa, sb, sf = m.decode_state(B), m.decode_state(B), m.decode_state(1)
        ga, gb, gf = DecodeGraph(m, sa, steps=steps), DecodeGraph(m, sb, steps=steps), None
        differ = False
        for blk in range(total // steps):
            ta = torch.randint(0, m.V, (steps, B), device="cuda", generator=gen)
            ta[ta == 7] = 8
            tb = ta.clone()
            tb[:, 32:] = torch.randint(0, m.V, (steps, 32), device="cuda", generator=gen)
            tb[tb == 7] = 8
            t0 = blk * steps
            if t0 <= s_bos < t0 + steps:
                ta[s_bos - t0, 5] = 7
                tb[s_bos - t0, 5] = 7
            la = ga.run(ta).clone()
            lb = gb.run(tb)
            ok &= (la[:, :32].view(torch.int16) == lb[:, :32].view(torch.int16)).all()   # bit for bit
            fin &= torch.isfinite(la).all() & torch.isfinite(lb).all()
            differ = differ or (blk == 0 and not torch.equal(la[:, 32:], lb[:, 32:]))
            if t0 + steps > s_bos and t0 < s_bos + 2048:   # the fresh stream, from the BOS on
                lo = max(s_bos - t0, 0)
                if gf is None:   # its first steps up to the block's end, eagerly; then graphs of 64
                    for t in range(lo, steps):
                        fresh_ok &= (m.step(ta[t, 5:6], sf)[0].view(torch.int16) == la[t, 5].view(torch.int16)).all()
                    gf = DecodeGraph(m, sf, steps=steps)
                else:
                    lf = gf.run(ta[:, 5:6].contiguous())
                    fresh_ok &= (lf[:, 0].view(torch.int16) == la[:, 5].view(torch.int16)).all()
    torch.cuda.synchronize()
    assert sa.pos == sb.pos == total
    assert differ, "streams 32-63 should differ between the runs"
    assert bool(fin), "non-finite logits"
    assert bool(ok), "a stream's logits depend on another stream's tokens"
    assert bool(fresh_ok), "after a BOS a stream differs from a fresh stream fed the same tokens"


def test_layer_decode_32k_steps_against_recurrence():
    """The mixer's decode step (sdm_rt_decode_step) at the layer shape (H=12, dh=64, M=1,024, k=8), 4 streams,
    32,768 steps, bfloat16: every step's read-out against the fp64 recurrence (its per-head-fade form) on the
    kernel's picks, within 2e-3 plus half a bfloat16 unit; fades 0.3, 0.5 and 1 among the heads (fade 0 has its own
    tests in test_gpu_decode.py; the per-head-fade recurrence here needs a positive fade)."""
    decays = (0.5, 0.3, 1.0) + tuple(np.random.Generator(np.random.PCG64(47)).uniform(0.9, 0.999, 9))
    kz, qz, V, g, p = core_inputs(4, 32768, 12, 64, 64, 32, seed=48, decays=decays)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    say("layer decode 32k steps bf16")
    r_dec, _ = gpu_decode(kz, qz, V, g, p, 8, dtype=torch.bfloat16)
    siw, _, ww = gpu_address(kz, p, 8, dtype=torch.bfloat16, gate=g)
    sir, _, wr = gpu_address(qz, p, 8, dtype=torch.bfloat16)
    B, T, H, dh = 4, 32768, 12, 64
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    num, den = O.scan_recurrence_rescaled(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                          wr.astype(np.float64), Vb, p["decay"].astype(np.float64))
    r64 = O.finish(num, den, "mean", 1e-3, True, p["onorm_w"].astype(np.float64), 1e-2)
    assert_close(r_dec, r64.transpose(0, 2, 1, 3).reshape(B, T, H * dh), 2e-3, True, msg="32k-step decode read-out")
