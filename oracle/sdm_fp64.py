"""float64 numpy restatement of the run-time SDM mixer -- TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function names the reference lines it restates (``OM`` = experiments/track4/sdmllm/track4_onesdm_models.py,
``SM`` = experiments/track4/sdmllm/track4_sdmllm_models.py).  Ties in every top-k are broken towards the lowest
index (a stable descending sort), the rule the product kernels implement.

Shapes: B batch rows, T positions, H heads, dh = d / H value width, d_a address width (two halves), n_sub sub-keys
per half, M = n_sub**2 locations per head, k picks per token and head.
"""
import numpy as np


def normalize_rows(x, eps=1e-12):
    """x / max(||x||_2, eps) along the last axis (torch.nn.functional.normalize, used at OM:137-140)."""
    n = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    return x / np.maximum(n, eps)


def stable_topk_desc(v, k):
    """Top-k along the last axis, sorted descending, equal values ordered by lowest index first."""
    order = np.argsort(-v, axis=-1, kind="stable")[..., :k]
    return np.take_along_axis(v, order, axis=-1), order


def half_scores(z, keys1, keys2):
    """Cosine of each address half against every unit sub-key (OM:136-140).

    z (N, H, d_a); keys (H, n_sub, d_a/2) -> s1, s2 (N, H, n_sub) float64."""
    z = np.asarray(z, np.float64)
    half = z.shape[-1] // 2
    u1 = normalize_rows(z[..., :half])
    u2 = normalize_rows(z[..., half:])
    k1 = normalize_rows(np.asarray(keys1, np.float64))
    k2 = normalize_rows(np.asarray(keys2, np.float64))
    return np.einsum("nhd,hsd->nhs", u1, k1), np.einsum("nhd,hsd->nhs", u2, k2)


def pk_address(z, keys1, keys2, k):
    """Exact product-key top-k (OM:134-148): top c1 = min(k, n_sub) per half, combine the c1 x c1 grid with score
    (v1 + v2) / 2, keep the top kk = min(k, c1^2), slot id = i1 * n_sub + i2.

    Returns sv (N, H, kk) descending and si (N, H, kk) int64."""
    n_sub = keys1.shape[1]
    s1, s2 = half_scores(z, keys1, keys2)
    c1 = min(k, n_sub)
    v1, i1 = stable_topk_desc(s1, c1)
    v2, i2 = stable_topk_desc(s2, c1)
    comb = ((v1[..., :, None] + v2[..., None, :]) * 0.5).reshape(*v1.shape[:-1], c1 * c1)
    kk = min(k, c1 * c1)
    sv, sc = stable_topk_desc(comb, kk)
    a, b = sc // c1, sc % c1
    si = np.take_along_axis(i1, a, -1) * n_sub + np.take_along_axis(i2, b, -1)
    return sv, si


def adopt_picks(z, keys1, keys2, sv, si, forced, tol, log=None):
    """Where another implementation's ordered picks ``forced`` (N, H, kk) differ from the oracle's si, check that
    each difference is a tie within ``tol`` (the two slots' fp64 scores at that position) and take the forced
    picks, with their fp64 scores.  Comparing a whole model with the HIP path needs this: its float32 inputs to a
    layer differ from the oracle's float64 ones by rounding, so near ties may resolve the other way.  Appends the
    number of adopted addresses to ``log``."""
    forced = np.asarray(forced).astype(np.int64)
    diff = si != forced
    rows = diff.any(-1)                  # (N, H)
    if rows.any():
        tok = np.flatnonzero(rows.any(-1))   # tokens with a differing head
        g = full_grid(np.asarray(z, np.float64)[tok], keys1, keys2)
        s_own = np.take_along_axis(g, si[tok], -1)
        s_got = np.take_along_axis(g, forced[tok], -1)
        gap = np.abs(s_own - s_got)[diff[tok]]
        if not np.all(gap < tol):
            raise AssertionError(f"picks differ away from a tie: fp64 score gap {float(gap.max()):.3e} >= {tol:.1e}")
        si = np.where(rows[..., None], forced, si)
        sv = np.array(sv)
        sv[tok] = np.where(rows[tok][..., None], s_got, sv[tok])
    if log is not None:
        log.append(int(rows.sum()))
    return sv, si


def full_grid(z, keys1, keys2):
    """Every location's score (s1[i] + s2[j]) / 2 at flat index i * n_sub + j: (N, H, n_sub^2)."""
    s1, s2 = half_scores(z, keys1, keys2)
    g = (s1[..., :, None] + s2[..., None, :]) * 0.5
    return g.reshape(*g.shape[:-2], -1)


def pk_address_bruteforce(z, keys1, keys2, k):
    """Top-k over the whole n_sub^2 grid (the brute-force search of the reference self-test, OM:694-702)."""
    n_sub = keys1.shape[1]
    kk = min(k, min(k, n_sub) ** 2)
    return stable_topk_desc(full_grid(z, keys1, keys2), kk)


def topk_margin(z, keys1, keys2, k):
    """fp64 gap between the kk-th and (kk+1)-th best location score (inf when every location is picked).

    A pick that differs from another implementation's by float32 rounding can only occur where this is tiny."""
    n_sub = keys1.shape[1]
    kk = min(k, min(k, n_sub) ** 2)
    g = full_grid(z, keys1, keys2)
    if g.shape[-1] <= kk:
        return np.full(g.shape[:-1], np.inf)
    part = -np.sort(-g, axis=-1)
    return part[..., kk - 1] - part[..., kk]


def topk_margin_pruned(z, keys1, keys2, k):
    """topk_margin without the whole grid: the (kk+1) best locations all lie in the grid of each half's kk+1 best
    sub-keys (a location ranked r in its half is beaten by r locations of its column), so that grid decides the
    margin exactly."""
    n_sub = keys1.shape[1]
    kk = min(k, min(k, n_sub) ** 2)
    if n_sub * n_sub <= kk:
        return np.full(np.asarray(z).shape[:-1], np.inf)
    s1, s2 = half_scores(z, keys1, keys2)
    c = min(kk + 1, n_sub)
    v1 = -np.sort(-s1, axis=-1)[..., :c]
    v2 = -np.sort(-s2, axis=-1)[..., :c]
    g = ((v1[..., :, None] + v2[..., None, :]) * 0.5).reshape(*v1.shape[:-1], c * c)
    part = -np.sort(-g, axis=-1)
    return part[..., kk - 1] - part[..., kk]


def softmax(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def rms_norm(x, w, eps=1e-6, rnd=None):
    """RMSNorm (SM:63-71): x * rsqrt(mean(x^2) + eps) * w, in float64.  rnd: the rounding of a reduced-precision
    evaluation (bf16 below), applied where the module casts: ``(x_f * rsqrt(...)).to(x.dtype) * w`` (SM:69-71)."""
    x = np.asarray(x, np.float64)
    n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return n * w if rnd is None else rnd(rnd(n) * w)


def bf16(a):
    """The nearest bfloat16 (ties to even) of each value, as float64: what a bfloat16 tensor holds after a result is
    cast to it.  float64 values are rounded to float32 first (the GPU computes in float32, then casts)."""
    a32 = np.asarray(a, np.float32)
    u = a32.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(a32), r, a32).astype(np.float64)


def _no_round(a):
    return a


def address_weights(sv, log_scale, gate=None):
    """softmax(e^{log_scale} * score) over the k picks, times the write gate when given (OM:203-207).

    sv (N, H, kk); log_scale (H,); gate (N, H) or None."""
    w = softmax(sv * np.exp(np.asarray(log_scale, np.float64))[None, :, None], axis=-1)
    if gate is not None:
        w = w * gate[..., None]
    return w


def scan_recurrence(siw, ww, sir, wr, V, lam, state=None, reset=None):
    """The token recurrence of the memory (OM:276-300): (empty at a reset,) read, then write.

    siw, sir (B, H, T, k) int; ww, wr (B, H, T, k); V (B, H, T, dh); lam (H,).
    state: optional (mem (B, H, M, dh), cnt (B, H, M)) to start from; M is taken from it or from max slot id.
    reset: optional (B, T) bool; where set, the memory of that batch row is emptied before position t reads
    (OM:287-289).
    Returns num (B, H, T, dh), den (B, H, T), mem, cnt (the state after the last write)."""
    B, H, T, k = siw.shape
    dh = V.shape[-1]
    if state is None:
        M = int(max(siw.max(initial=0), sir.max(initial=0))) + 1
        mem = np.zeros((B, H, M, dh))
        cnt = np.zeros((B, H, M))
    else:
        mem = np.array(state[0], np.float64)
        cnt = np.array(state[1], np.float64)
    lam = np.asarray(lam, np.float64)
    bi = np.arange(B)[:, None, None]
    hi = np.arange(H)[None, :, None]
    num = np.zeros((B, H, T, dh))
    den = np.zeros((B, H, T))
    for t in range(T):
        if reset is not None:
            live = (~np.asarray(reset[:, t], bool)).astype(np.float64)
            mem *= live[:, None, None, None]
            cnt *= live[:, None, None]
        rows = sir[:, :, t]                                  # (B, H, k)
        got = mem[bi, hi, rows]                              # (B, H, k, dh)
        num[:, :, t] = np.einsum("bhk,bhkd->bhd", wr[:, :, t], got)
        den[:, :, t] = np.einsum("bhk,bhk->bh", wr[:, :, t], cnt[bi, hi, rows])
        mem *= lam[None, :, None, None]
        cnt *= lam[None, :, None]
        wrow = siw[:, :, t]
        np.add.at(mem, (bi, hi, wrow), ww[:, :, t, :, None] * V[:, :, t, None, :])
        np.add.at(cnt, (bi, hi, wrow), ww[:, :, t])
    return num, den, mem, cnt


def scan_recurrence_rescaled(siw, ww, sir, wr, V, lam, reset=None):
    """scan_recurrence (OM:276-300) from an empty memory without resets, the fade carried as one factor per head: with
    mem_t = lam^t * P_t, a step reads lam^t * P at its read rows and adds (write) / lam^(t+1) to P at its write rows,
    so it touches 2k rows instead of fading all M; when a head's factor falls below 1e-100 it is folded into P (one
    pass over that head's memory).  The same values up to float64 rounding (checked against scan_recurrence in
    tests/test_oracle_scan.py); every lam must be above 0 (use scan_recurrence for a fade of 0).  reset: optional
    (B, T) bool, as in scan_recurrence (that batch row's memory emptied before position t reads, OM:287-289).
    Returns num (B, H, T, dh), den (B, H, T)."""
    B, H, T, k = siw.shape
    dh = V.shape[-1]
    M = int(max(siw.max(initial=0), sir.max(initial=0))) + 1
    lam = np.asarray(lam, np.float64)
    if T and not np.min(lam) > 0:
        raise ValueError("scan_recurrence_rescaled: a fade of 0; use scan_recurrence")
    P = np.zeros((B, H, M, dh))
    C = np.zeros((B, H, M))
    bi = np.arange(B)[:, None, None]
    hi = np.arange(H)[None, :, None]
    num = np.zeros((B, H, T, dh))
    den = np.zeros((B, H, T))
    S = np.ones(H)   # lam^t
    for t in range(T):
        if reset is not None and np.any(reset[:, t]):
            dead = np.asarray(reset[:, t], bool)
            P[dead] = 0.0
            C[dead] = 0.0
        rows = sir[:, :, t]
        num[:, :, t] = np.einsum("bhk,bhkd->bhd", wr[:, :, t], P[bi, hi, rows]) * S[None, :, None]
        den[:, :, t] = np.einsum("bhk,bhk->bh", wr[:, :, t], C[bi, hi, rows]) * S[None, :]
        S = S * lam
        low = S < 1e-100
        if low.any():   # fold the small factor into the memory of those heads
            P[:, low] *= S[low][None, :, None, None]
            C[:, low] *= S[low][None, :, None]
            S = np.where(low, 1.0, S)
        wrow = siw[:, :, t]
        inv = (1.0 / S)[None, :, None]
        np.add.at(P, (bi, hi, wrow), (ww[:, :, t] * inv)[..., None] * V[:, :, t, None, :])
        np.add.at(C, (bi, hi, wrow), ww[:, :, t] * inv)
    return num, den


def scan_closed_form(siw, ww, sir, wr, V, lam):
    """The same read written as the double sum of the closed form (O(T^2 k^2), tiny inputs only):
    num_t = sum_{s<t} lam^(t-1-s) sum_{i,j} wr[t,i] ww[s,j] [sir[t,i] == siw[s,j]] V_s; den with V -> 1."""
    B, H, T, k = siw.shape
    num = np.zeros(V.shape)
    den = np.zeros((B, H, T))
    for b in range(B):
        for h in range(H):
            for t in range(T):
                for s in range(t):
                    match = (sir[b, h, t][:, None] == siw[b, h, s][None, :])
                    c = float(np.sum(wr[b, h, t][:, None] * ww[b, h, s][None, :] * match))
                    f = float(lam[h]) ** (t - 1 - s)
                    num[b, h, t] += f * c * V[b, h, s]
                    den[b, h, t] += f * c
    return num, den


def finish(num, den, read_mode="mean", read_eps=1e-3, out_norm=True, onorm_w=None, out_norm_eps=1e-2):
    """Mean (or sum) read and the per-head output RMS norm (OM:243-246), before the output map.

    num (B, H, T, dh), den (B, H, T) -> r (B, H, T, dh)."""
    r = num / (den[..., None] + read_eps) if read_mode == "mean" else np.array(num)
    if out_norm:
        r = r / np.sqrt(np.mean(r * r, axis=-1, keepdims=True) + out_norm_eps) * onorm_w[None, :, None, :]
    return r


def core_forward(kz, qz, V, gate_logits, p, cfg, return_parts=False, reset=None, forced=None):
    """The SDM core between the projections and the output map.

    kz, qz (B, T, H, d_a) already include addr_b; V (B, T, H, dh); gate_logits (B, T, H) or None (gate off).
    p: dict with keys1, keys2, log_scale, decay, onorm_w.  cfg: dict with k, read_mode, read_eps, out_norm,
    out_norm_eps (and adopt_tol, adopt_log for ``forced``).  forced: None or another implementation's (siw, sir)
    picks (N, H, kk), taken at ties (adopt_picks).  Returns r (B, T, H, dh) in float64."""
    B, T, H, d_a = kz.shape
    k = cfg["k"]
    N = B * T
    zw = np.asarray(kz, np.float64).reshape(N, H, d_a)
    zr = np.asarray(qz, np.float64).reshape(N, H, d_a)
    svw, siw = pk_address(zw, p["keys1"], p["keys2"], k)
    svr, sir = pk_address(zr, p["keys1"], p["keys2"], k)
    if forced is not None:
        tol, log = cfg.get("adopt_tol", 1e-5), cfg.get("adopt_log")
        svw, siw = adopt_picks(zw, p["keys1"], p["keys2"], svw, siw, forced[0], tol, log)
        svr, sir = adopt_picks(zr, p["keys1"], p["keys2"], svr, sir, forced[1], tol, log)
    gate = None if gate_logits is None else sigmoid(np.asarray(gate_logits, np.float64).reshape(N, H))
    ww = address_weights(svw, p["log_scale"], gate)
    wr = address_weights(svr, p["log_scale"], None)
    kk = siw.shape[-1]

    def bh(a):
        return a.reshape(B, T, H, kk).transpose(0, 2, 1, 3)
    Vb = np.asarray(V, np.float64).transpose(0, 2, 1, 3)
    n_sub = p["keys1"].shape[1]
    M = n_sub * n_sub
    state = (np.zeros((B, H, M, Vb.shape[-1])), np.zeros((B, H, M)))
    num, den, mem, cnt = scan_recurrence(bh(siw), bh(ww), bh(sir), bh(wr), Vb, p["decay"], state, reset=reset)
    r = finish(num, den, cfg.get("read_mode", "mean"), cfg.get("read_eps", 1e-3), cfg.get("out_norm", True),
               p.get("onorm_w"), cfg.get("out_norm_eps", 1e-2)).transpose(0, 2, 1, 3)
    if return_parts:
        return r, dict(svw=svw, siw=siw, svr=svr, sir=sir, ww=ww, wr=wr, num=num, den=den, mem=mem, cnt=cnt)
    return r


def layer_forward(x, p, cfg, reset=None, forced=None):
    """Whole RunTimeSdm.forward in float64 (OM:195-213 prepare, OM:249-274 forward, OM:243-247 finish).

    x (B, T, d); p holds the module's parameters under their state_dict names ('norm.w', 'wk.weight', ...,
    'decays_fixed' as 'decay').  cfg["round"] (default none): the rounding of a bfloat16 evaluation (``bf16``),
    applied where a bfloat16 layer casts: the input norm, each projection (the gate logit with its bias), the
    read-out and the output map (the core computes in float32 between its bfloat16 inputs and output).  Returns
    y (B, T, d)."""
    x = np.asarray(x, np.float64)
    B, T, d = x.shape
    H = cfg["heads"]
    d_a = cfg["d_a"]
    dh = d // H
    rnd = cfg.get("round")
    r_ = rnd or _no_round
    hx = rms_norm(x, p["norm.w"], rnd=rnd)
    kz = r_(hx @ p["wk.weight"].T).reshape(B, T, H, d_a) + p["addr_b"]
    qz = r_(hx @ p["wq.weight"].T).reshape(B, T, H, d_a) + p["addr_b"]
    V = r_(hx @ p["wv.weight"].T).reshape(B, T, H, dh)
    g = r_(hx @ p["wg.weight"].T + p["wg.bias"]) if cfg.get("write_gate", True) else None
    core_p = dict(keys1=p["keys1"], keys2=p["keys2"], log_scale=p["log_scale"], decay=p["decay"],
                  onorm_w=p.get("onorm_w"))
    r = core_forward(kz, qz, V, g, core_p, cfg, reset=reset, forced=forced)
    return r_(r_(r.reshape(B, T, d)) @ p["wo.weight"].T)


def table_read(si, w, values):
    """The weighted read of picked table rows (TrainedSdm.forward's embedding_bag, OM:448-455).

    si (N, H, kk) int, w (N, H, kk), values (H, M, dh) -> (N, H, dh)."""
    H = values.shape[0]
    rows = np.asarray(values, np.float64)[np.arange(H)[None, :, None], si]   # (N, H, kk, dh)
    return np.einsum("nhk,nhkd->nhd", np.asarray(w, np.float64), rows)


def trained_sdm_forward(x, p, cfg, return_parts=False, forced=None):
    """TrainedSdm.forward (OM:414-457) in float64: RMSNorm, the query map, pk_address, softmax(exp(log_scale) *
    score), the weighted sum of the picked value rows, the output map.  p: norm.w, wq.weight, keys1, keys2, values,
    log_scale, wo.weight.  cfg: heads, d_a, k."""
    B, T, d = x.shape
    H, d_a, k = cfg["heads"], cfg["d_a"], cfg["k"]
    rnd = cfg.get("round")
    r_ = rnd or _no_round
    hx = rms_norm(np.asarray(x, np.float64), p["norm.w"], rnd=rnd)
    q = r_(hx @ np.asarray(p["wq.weight"], np.float64).T).reshape(B * T, H, d_a)
    sv, si = pk_address(q, p["keys1"], p["keys2"], k)
    if forced is not None:
        sv, si = adopt_picks(q, p["keys1"], p["keys2"], sv, si, forced, cfg.get("adopt_tol", 1e-5),
                             cfg.get("adopt_log"))
    w = address_weights(sv, p["log_scale"])
    r = r_(table_read(si, w, p["values"]).reshape(B, T, d))
    y = r_(r @ np.asarray(p["wo.weight"], np.float64).T)
    if return_parts:
        return y, dict(q=q, sv=sv, si=si, w=w, r=r)
    return y


def silu(x):
    return x / (1.0 + np.exp(-x))


def swiglu(x, gate_w, up_w, down_w, rnd=None):
    """down(silu(gate x) * up x) (track4_sdmllm_models.py:89-97).  rnd: a bfloat16 evaluation's casts, after each
    map, after silu and after the product (torch's bfloat16 ops compute in float32 and cast each result)."""
    if rnd is None:
        return (silu(x @ gate_w.T) * (x @ up_w.T)) @ down_w.T
    return rnd(rnd(rnd(silu(rnd(x @ gate_w.T))) * rnd(x @ up_w.T)) @ down_w.T)


def model_forward(idx, p, cfg, margins=None, forced=None, return_hidden=False):
    """OneSdmLM.forward (OM:471-555, archive off) in float64: embedding, per layer x + RunTimeSdm(x, reset) and
    x + SwiGLU(RMSNorm x) (ffn 'mlp') or x + TrainedSdm(x) (ffn 'sdm'), final RMSNorm, tied head.

    idx (B, T) int; p: the model's state dict as float64 arrays; cfg: layers, heads, d_a, k, ffn, mem, tie,
    reset_at_bos, bos_id, sdm_heads, sdm_d_a, sdm_k and the mixer options of core_forward.  When ``margins`` is a
    list, the smallest fp64 top-k margin of every addressing is appended to it.  forced: None or a dict of another
    implementation's picks, {("mem", i): (siw, sir), ("sdm", i): si} as (N, H, kk) arrays, taken at ties
    (adopt_picks, cfg["adopt_tol"]; the adopted counts go to cfg["adopt_log"]).  cfg["round"]: the rounding of a
    bfloat16 model (``bf16``; p then holds the bfloat16 weights), applied at every cast of a bfloat16 forward: each
    layer's (layer_forward, trained_sdm_forward, swiglu), each residual sum, the final norm and the logits.  Returns
    logits (B, T, V), or with return_hidden the normalised hidden state (B, T, d) the tied head reads (the logits
    are then that times emb.weight^T, rounded like them)."""
    E = p["emb.weight"]
    x = E[np.asarray(idx)]
    B, T, d = x.shape
    rnd = cfg.get("round")
    r_ = rnd or _no_round
    reset = (np.asarray(idx) == cfg.get("bos_id", 0)) if cfg.get("reset_at_bos") else None
    for i in range(cfg["layers"]):
        if cfg.get("mem", True):
            pre = f"mems.{i}."
            lp = {n[len(pre):]: v for n, v in p.items() if n.startswith(pre)}
            lp["decay"] = lp["decays_fixed"] if "decays_fixed" in lp else 1.0 / (1.0 + np.exp(-lp["decay_logit"]))
            if margins is not None:
                H, d_a = cfg["heads"], cfg["d_a"]
                hx = rms_norm(x, lp["norm.w"])
                for wn in ("wk.weight", "wq.weight"):
                    z = (hx @ lp[wn].T).reshape(B * T, H, d_a) + lp["addr_b"]
                    margins.append(float(topk_margin(z, lp["keys1"], lp["keys2"], cfg["k"]).min()))
            x = r_(x + layer_forward(x, lp, cfg, reset, None if forced is None else forced[("mem", i)]))
        if cfg.get("ffn", "mlp") == "mlp":
            x = r_(x + swiglu(rms_norm(x, p[f"mnorms.{i}.w"], rnd=rnd), p[f"mlps.{i}.gate.weight"],
                              p[f"mlps.{i}.up.weight"], p[f"mlps.{i}.down.weight"], rnd=rnd))
        elif cfg["ffn"] == "sdm":
            pre = f"sdms.{i}."
            sp = {n[len(pre):]: v for n, v in p.items() if n.startswith(pre)}
            scfg = dict(heads=cfg["sdm_heads"], d_a=cfg["sdm_d_a"], k=cfg["sdm_k"], adopt_tol=cfg.get("adopt_tol", 1e-5),
                        adopt_log=cfg.get("adopt_log"), round=rnd)
            y, parts = trained_sdm_forward(x, sp, scfg, return_parts=True,
                                           forced=None if forced is None else forced[("sdm", i)])
            if margins is not None:
                margins.append(float(topk_margin(parts["q"], sp["keys1"], sp["keys2"], scfg["k"]).min()))
            x = r_(x + y)
    h = rms_norm(x, p["nf.w"], rnd=rnd)
    if return_hidden:
        return h
    return r_(h @ (E.T if cfg.get("tie", True) else p["head.weight"].T))
