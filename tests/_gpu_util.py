"""Shared helpers of the GPU parity tests: seeded core inputs, the HIP calls and the oracle on the same values."""
import sys

import numpy as np
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import core

# float32 resolution of a cosine score near 1: picks may differ from the oracle's (in set or in order) only where
# two slots' fp64 scores are closer than this
DELTA = 2.4e-7


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf16_round(a):
    """Round float32 values to bfloat16 and back (the values a bf16 tensor holds)."""
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def core_inputs(B, T, H, dh, d_a, n_sub, seed, decays=None, addr_bias=0.0, gate=True):
    """Projection-like inputs of the core: kz, qz (B, T, H*d_a), V (B, T, H*dh), gate logits (B, T, H) ~ N(0, 1),
    and parameters (keys N(0,1), log_scale ln 8, onorm_w ~ U(0.5, 1.5), fades)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    kz = rng.standard_normal((B, T, H * d_a)).astype(np.float32)
    qz = rng.standard_normal((B, T, H * d_a)).astype(np.float32)
    V = rng.standard_normal((B, T, H * dh)).astype(np.float32)
    g = (rng.standard_normal((B, T, H)) * 1.5).astype(np.float32) if gate else None
    if decays is None:
        decays = rng.uniform(0.9, 0.999, H)
    p = dict(keys1=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             keys2=rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
             addr_b=(rng.standard_normal((H, d_a)) * addr_bias).astype(np.float32),
             log_scale=np.full(H, np.log(8.0), np.float32) + rng.uniform(-0.5, 0.5, H).astype(np.float32),
             decay=np.asarray(decays, np.float32),
             onorm_w=rng.uniform(0.5, 1.5, (H, dh)).astype(np.float32),
             gate_bias=rng.uniform(-0.5, 0.5, H).astype(np.float32))
    return kz, qz, V, g, p


def to_dev(a, dtype):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def gpu_core(kz, qz, V, g, p, k, dtype=torch.float32, out_dtype=None, read_mode="mean", out_norm=True,
             state_in=None, want_state=False, fused=False, reset=None):
    """Run sdm_rt_forward; returns r (numpy float32, (B, T, H*dh)) and optionally the state."""
    if fused:   # one buffer with all four inputs side by side (the layout of a fused projection)
        parts = [kz, qz, V] + ([g] if g is not None else [])
        widths = [x.shape[-1] for x in parts]
        buf = torch.zeros(kz.shape[0], kz.shape[1], sum(widths) + 40, device="cuda", dtype=dtype)
        o = 0
        views = []
        for x, w in zip(parts, widths):
            buf[..., o:o + w] = to_dev(x, dtype)
            views.append(buf[..., o:o + w])
            o += w
        kz_d, qz_d, V_d = views[:3]
        g_d = views[3] if g is not None else None
    else:
        kz_d, qz_d, V_d, g_d = (to_dev(x, dtype) for x in (kz, qz, V, g))
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    st = None
    if state_in is not None:
        st = (torch.from_numpy(state_in[0].astype(np.float32)).cuda(),
              torch.from_numpy(state_in[1].astype(np.float32)).cuda())
    res = core.core_forward(kz_d, qz_d, V_d, g_d, keys1=tp["keys1"], keys2=tp["keys2"], log_scale=tp["log_scale"],
                            decay=tp["decay"], addr_b=tp["addr_b"], onorm_w=tp["onorm_w"],
                            gate_bias=tp["gate_bias"] if g is not None else None, k=k, read_mode=read_mode,
                            out_norm=out_norm, out_dtype=out_dtype, state_in=st, want_state=want_state,
                            reset=None if reset is None else torch.from_numpy(np.asarray(reset, bool)).cuda())
    torch.cuda.synchronize()
    if want_state:
        r, (m, c) = res
        return r.float().cpu().numpy(), (m.cpu().numpy(), c.cpu().numpy())
    return res.float().cpu().numpy()


def gpu_address(z, p, k, dtype=torch.float32, gate=None):
    """sdm_rt_address on (B, T, H*d_a) addresses -> slots, scores, weights as numpy (B, H, T, kk)."""
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    s, v, w = core.address(to_dev(z, dtype), tp["keys1"], tp["keys2"], k, log_scale=tp["log_scale"],
                           addr_b=tp["addr_b"], gate_logits=to_dev(gate, dtype),
                           gate_bias=tp["gate_bias"] if gate is not None else None)
    torch.cuda.synchronize()
    return s.cpu().numpy(), v.cpu().numpy(), w.cpu().numpy()


def oracle_core(kz, qz, V, g, p, k, read_mode="mean", out_norm=True):
    """fp64 oracle of the core on the same values (kz/qz get addr_b, gate logits get gate_bias here)."""
    B, T, _ = V.shape
    H = p["keys1"].shape[0]
    d_a = 2 * p["keys1"].shape[2]
    dh = V.shape[-1] // H
    kz4 = kz.astype(np.float64).reshape(B, T, H, d_a) + p["addr_b"]
    qz4 = qz.astype(np.float64).reshape(B, T, H, d_a) + p["addr_b"]
    gl = None if g is None else g.astype(np.float64) + p["gate_bias"]
    cp = {n: p[n].astype(np.float64) for n in ("keys1", "keys2", "log_scale", "decay", "onorm_w")}
    cfg = dict(k=k, read_mode=read_mode, out_norm=out_norm)
    r, parts = O.core_forward(kz4, qz4, V.astype(np.float64).reshape(B, T, H, dh), gl, cp, cfg, return_parts=True)
    return r.reshape(B, T, H * dh), parts


def valid_picks(z, keys1, keys2, k, si):
    """Per (token, head): the picks are distinct and each scores (fp64) no lower than the kk-th best location minus
    DELTA -- an equally good pick set.  z (N, H, d_a); si (N, H, kk)."""
    g = O.full_grid(np.asarray(z, np.float64), np.asarray(keys1, np.float64), np.asarray(keys2, np.float64))
    kk = si.shape[-1]
    cut = -np.sort(-g, axis=-1)[..., kk - 1]
    got = np.take_along_axis(g, si.astype(np.int64), -1)
    distinct = np.array([len(set(r)) == kk for r in si.reshape(-1, kk).tolist()]).reshape(si.shape[:-1])
    return distinct & np.all(got >= cut[..., None] - DELTA, -1)


def min_margin(z, p, k):
    """Smallest fp64 top-k margin over every (token, head) address of (B, T, H*d_a) addresses."""
    B, T, W = z.shape
    H = p["keys1"].shape[0]
    d_a = W // H
    zz = z.astype(np.float64).reshape(B * T, H, d_a) + p["addr_b"]
    return float(O.topk_margin(zz, p["keys1"].astype(np.float64), p["keys2"].astype(np.float64), k).min())


def scan_from_picks(siw, ww, sir, wr, V, lam, H, read_mode="mean", out_norm=True, onorm_w=None, M=None,
                    rescaled=False):
    """fp64 recurrence + finish from given picks/weights (B, H, T, kk) and values V (B, T, H*dh).  rescaled: the
    recurrence with the fade carried per head (oracle scan_recurrence_rescaled: the same values, a step touches only
    its picked rows; no final state, returned as None)."""
    B, T, W = V.shape
    dh = W // H
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    args = (siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64), wr.astype(np.float64), Vb,
            np.asarray(lam, np.float64))
    if rescaled:
        num, den = O.scan_recurrence_rescaled(*args)
        mem = cnt = None
    else:
        num, den, mem, cnt = O.scan_recurrence(*args, (np.zeros((B, H, M, dh)), np.zeros((B, H, M))))
    r = O.finish(num, den, read_mode, 1e-3, out_norm, None if onorm_w is None else onorm_w.astype(np.float64), 1e-2)
    return r.transpose(0, 2, 1, 3).reshape(B, T, W), (mem, cnt)



def half_ulp_bf16(x):
    """Half the spacing of bfloat16 numbers (8 significant bits) around |x|: the most a correct rounding of x to
    bfloat16 can move it."""
    a = np.maximum(np.abs(np.asarray(x, np.float64)), 1e-30)
    return np.exp2(np.floor(np.log2(a)) - 8)


def assert_close(got, want, tol, bf16_out=False, msg=""):
    """|got - want| <= tol + tol * |want| (+ half a bf16 ulp of want when got was rounded to bfloat16)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    lim = tol + tol * np.abs(want) + (half_ulp_bf16(want) if bf16_out else 0.0)
    err = np.abs(got - want)
    bad = err > lim
    assert not bad.any(), (f"{msg}: {bad.sum()} of {bad.size} off; worst excess {float((err - lim).max()):.3e} "
                           f"at |want| {float(np.abs(want)[np.unravel_index(np.argmax(err - lim), err.shape)]):.3e}")


def tokens(a):
    """(B, H, T, kk) -> (B*T, H, kk)."""
    B, H, T, kk = a.shape
    return a.transpose(0, 2, 1, 3).reshape(B * T, H, kk)


def pick_diffs(zz, k1, k2, si_a, si_b):
    """(N, H) mask of the addresses whose ordered pick lists si_a, si_b (N, H, kk) differ, after checking that every
    difference is a tie: at each position the two slots' fp64 scores agree within DELTA."""
    diff = si_a != si_b
    rows = np.unique(np.argwhere(diff.any(-1))[:, 0])
    if len(rows):
        g = O.full_grid(np.asarray(zz[rows], np.float64), k1, k2)
        sa = np.take_along_axis(g, si_a[rows].astype(np.int64), -1)
        sb = np.take_along_axis(g, si_b[rows].astype(np.int64), -1)
        gap = np.abs(sa - sb)[diff[rows]]
        assert np.all(gap < DELTA), f"picks differ with an fp64 score gap of {float(gap.max()):.3e}"
    return diff.any(-1)


def check_picks(z, p, k, si, w, gate=None):
    """Kernel picks / weights (B, H, T, kk) of addresses z (B, T, H*d_a) against the fp64 oracle: the ordered pick
    lists agree except at ties (pick_diffs: two slots' fp64 scores within DELTA); weights agree (2e-6) where the
    lists agree.  Returns the number of (token, head) addresses whose picks differ."""
    B, T, W = z.shape
    H = p["keys1"].shape[0]
    d_a = W // H
    zz = z.astype(np.float64).reshape(B * T, H, d_a) + p["addr_b"]
    k1, k2 = p["keys1"].astype(np.float64), p["keys2"].astype(np.float64)
    osv, osi = O.pk_address(zz, k1, k2, k)
    gsi = tokens(si)
    same = ~pick_diffs(zz, k1, k2, osi, gsi)
    gl = None if gate is None else O.sigmoid(gate.astype(np.float64).reshape(B * T, H) + p["gate_bias"])
    ow = O.address_weights(osv, p["log_scale"].astype(np.float64), gl)
    np.testing.assert_allclose(tokens(w)[same], ow[same], atol=2e-6, rtol=2e-6)
    return int((~same).sum())


def check_core(kz, qz, V, g, p, k, dtype=torch.float32, out_dtype=None, tol=1e-5, read_mode="mean", out_norm=True,
               fused=False, slabs=None, rescaled=False):
    """sdm_rt_forward against the fp64 oracle in two parts: (1) the addressing kernel's picks and weights against
    the oracle's (check_picks); (2) the read-out against the fp64 recurrence + finish driven by those same picks and
    weights.  When no pick differs, the read-out is also compared with the fully independent oracle.  ``slabs``
    restricts (2) to a list of (b, h); rescaled runs (2) on the oracle's per-head-fade recurrence (long sequences,
    every slab) and skips the independent oracle.  Returns the number of differing picks."""
    out_dtype = out_dtype or dtype
    bf16_out = out_dtype == torch.bfloat16
    B, T, _ = V.shape
    H = p["keys1"].shape[0]
    dh = V.shape[-1] // H
    M = p["keys1"].shape[1] ** 2
    say("core", dtype, "->", out_dtype, "B", B, "T", T, "H", H, "dh", dh, "M", M, "k", k)
    r = gpu_core(kz, qz, V, g, p, k, dtype=dtype, out_dtype=out_dtype, read_mode=read_mode, out_norm=out_norm,
                 fused=fused)
    siw, _, ww = gpu_address(kz, p, k, dtype=dtype, gate=g)
    sir, _, wr = gpu_address(qz, p, k, dtype=dtype)
    flips = check_picks(kz, p, k, siw, ww, g) + check_picks(qz, p, k, sir, wr)
    on = p["onorm_w"] if out_norm else None
    if slabs is None:
        want, _ = scan_from_picks(siw, ww, sir, wr, V, p["decay"], H, read_mode, out_norm, on, M, rescaled)
        assert_close(r, want, tol, bf16_out, "read-out given the kernel's picks")
        if flips == 0 and not rescaled:
            full, _ = oracle_core(kz, qz, V, g, p, k, read_mode, out_norm)
            assert_close(r, full, tol, bf16_out, "read-out against the independent oracle")
    else:
        for b, h in slabs:
            sl = slice(h * dh, (h + 1) * dh)
            want, _ = scan_from_picks(siw[b:b + 1, h:h + 1], ww[b:b + 1, h:h + 1], sir[b:b + 1, h:h + 1],
                                      wr[b:b + 1, h:h + 1], V[b:b + 1, :, sl], p["decay"][h:h + 1], 1, read_mode,
                                      out_norm, None if on is None else on[h:h + 1], M)
            assert_close(r[b:b + 1, :, sl], want, tol, bf16_out, f"slab b={b} h={h}")
    return flips


def gpu_decode(kz, qz, V, g, p, k, dtype=torch.float32, out_dtype=None, read_mode="mean", out_norm=True,
               reset=None, state=None, last=True):
    """Run sdm_rt_decode_step once per position (B streams, T steps); returns r (numpy float32, (B, T, H*dh)) and
    the final DecodeState.  reset: (B, T) bool or None; state: a DecodeState to continue from, or None (empty, with
    the last-write slots when ``last``)."""
    B, T = V.shape[0], V.shape[1]
    H, n_sub, half = p["keys1"].shape
    dh = V.shape[2] // H
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    kz_d, qz_d, V_d, g_d = (to_dev(x, dtype) for x in (kz, qz, V, g))
    if state is None:
        state = core.DecodeState.empty(B, H, n_sub * n_sub, dh, "cuda", core.pick_pitch(k, n_sub) if last else None)
    rs = None if reset is None else torch.from_numpy(np.asarray(reset, bool)).cuda()
    ws = core.CoreWorkspace()
    outs = []
    for t in range(T):
        outs.append(core.decode_step(
            kz_d[:, t], qz_d[:, t], V_d[:, t], None if g_d is None else g_d[:, t], state, keys1=tp["keys1"],
            keys2=tp["keys2"], log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"],
            onorm_w=tp["onorm_w"], gate_bias=tp["gate_bias"] if g is not None else None, k=k, read_mode=read_mode,
            out_norm=out_norm, reset=None if rs is None else rs[:, t], out_dtype=out_dtype, workspace=ws))
    torch.cuda.synchronize()
    r = torch.stack(outs, 1) if outs else torch.zeros(B, 0, H * dh)
    return r.float().cpu().numpy(), state
