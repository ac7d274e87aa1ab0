"""float64 torch restatement of the SDM core with the picks held fixed, for its gradient -- TEST INFRASTRUCTURE ONLY
(see ``oracle/__init__.py``).

The reference trains RunTimeSdm by torch autograd of its chunked dense forward (OM = experiments/track4/sdmllm/
track4_onesdm_models.py, RunTimeSdm.prepare :195-213, _chunk :215-241, finish :243-247, under checkpoint :259-268).
topk and the slot ids carry no gradient, so for fixed picks the core is a smooth function of the projections and the
parameters; this module writes that function in float64 torch ops (CPU) and lets autograd differentiate it:
  * scores sv_j = (<u1, k1^[i1_j]> + <u2, k2^[i2_j]>) / 2 with u = F.normalize of the address halves (z + addr_b) and
    k^ = F.normalize of the sub-keys (pk_address :134-148, read at the picks: the values topk returns);
  * ww = softmax(e^log_scale sv_w) * sigmoid(gate logit + gate bias), wr = softmax(e^log_scale sv_r) (:203-207);
  * the closed form of the read, K[t][s] = lam^(t-1-s) [s < t] [same segment] sum_ij wr[t,i] ww[s,j] [match]
    (the dense chunk of :222-236 over the whole sequence), num = K V, den = K 1;
  * finish (:243-246) without wo.

Pinning: ``tests/test_oracle_grad.py`` checks the forward against ``sdm_fp64.core_forward`` (the token recurrence)
and every gradient against central finite differences of ``sdm_fp64.core_forward``; it also checks the identity
lam dL/dlam = sum_t t P_t - sum_s (s+1) Q_s (P_t = sum_i wr dwr, Q_s = sum_j ww dww) on this module's autograd.
"""
import torch
import torch.nn.functional as F


def _lam_powers(lam, T, reset=None, B=1):
    """D[b, h, t, s] = lam_h^(t-1-s) for s < t in the same segment, else 0 (OM:222-225, 229-233)."""
    pos = torch.arange(T, dtype=torch.float64)
    e = pos[:, None] - 1 - pos[None, :]
    mask = (e >= 0).to(torch.float64)
    D = torch.pow(lam[:, None, None], e.clamp(min=0)[None]) * mask[None]        # (H, T, T)
    D = D[None].expand(B, -1, -1, -1)
    if reset is not None:
        seg = torch.cumsum(torch.as_tensor(reset).to(torch.int64), 1)            # (B, T)
        same = (seg[:, :, None] == seg[:, None, :]).to(torch.float64)
        D = D * same[:, None]
    return D


def pick_scores(z, addr_b, keys1, keys2, si):
    """Mean half-cosine of each pick: z (B, T, H, d_a) before addr_b, si (B, T, H, kk) slot ids -> (B, T, H, kk)."""
    B, T, H, d_a = z.shape
    half = d_a // 2
    n_sub = keys1.shape[1]
    zz = z + (addr_b if addr_b is not None else 0.0)
    u1 = F.normalize(zz[..., :half], dim=-1, eps=1e-12)
    u2 = F.normalize(zz[..., half:], dim=-1, eps=1e-12)
    k1 = F.normalize(keys1, dim=-1, eps=1e-12)
    k2 = F.normalize(keys2, dim=-1, eps=1e-12)
    si = torch.as_tensor(si).to(torch.int64)
    hidx = torch.arange(H)[None, None, :, None]
    g1 = k1[hidx, si // n_sub]                                                  # (B, T, H, kk, half)
    g2 = k2[hidx, si % n_sub]
    v1 = (g1 * u1[..., None, :]).sum(-1)
    v2 = (g2 * u2[..., None, :]).sum(-1)
    return 0.5 * (v1 + v2)


def read_from_weights(siw, ww, sir, wr, V, lam, M, reset=None, read_mode="mean", read_eps=1e-3, out_norm=True,
                      onorm_w=None, out_norm_eps=1e-2):
    """r (B, T, H, dh) from per-pick weights: siw, sir (B, T, H, kk) int; ww, wr (B, T, H, kk); V (B, T, H, dh)."""
    B, T, H, kk = ww.shape
    siw = torch.as_tensor(siw).to(torch.int64).permute(0, 2, 1, 3)
    sir = torch.as_tensor(sir).to(torch.int64).permute(0, 2, 1, 3)
    W = torch.zeros(B, H, T, M, dtype=torch.float64).scatter_add(3, siw, ww.permute(0, 2, 1, 3))
    R = torch.zeros(B, H, T, M, dtype=torch.float64).scatter_add(3, sir, wr.permute(0, 2, 1, 3))
    K = torch.matmul(R, W.transpose(-1, -2)) * _lam_powers(lam, T, reset, B)   # (B, H, T, T)
    Vb = V.permute(0, 2, 1, 3)
    num = torch.matmul(K, Vb)
    den = K.sum(-1, keepdim=True)
    r = num / (den + read_eps) if read_mode == "mean" else num
    if out_norm:
        r = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + out_norm_eps) * onorm_w[None, :, None, :]
    return r.permute(0, 2, 1, 3)


def core_from_picks(kz, qz, V, gate_logits, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias, siw, sir,
                    cfg, reset=None):
    """The SDM core for fixed picks, float64 torch (differentiable in every tensor argument).

    kz, qz (B, T, H, d_a) before addr_b; V (B, T, H, dh); gate_logits (B, T, H) before gate_bias, or None (no
    gate); siw, sir (B, T, H, kk) slot ids.  cfg: k, read_mode, read_eps, out_norm, out_norm_eps.
    Returns r (B, T, H, dh)."""
    n_sub = keys1.shape[1]
    tau = torch.exp(log_scale)[None, None, :, None]
    svw = pick_scores(kz, addr_b, keys1, keys2, siw)
    svr = pick_scores(qz, addr_b, keys1, keys2, sir)
    ww = torch.softmax(svw * tau, -1)
    wr = torch.softmax(svr * tau, -1)
    if gate_logits is not None:
        gl = gate_logits + (gate_bias if gate_bias is not None else 0.0)
        ww = ww * torch.sigmoid(gl)[..., None]
    return read_from_weights(siw, ww, sir, wr, V, decay, n_sub * n_sub, reset, cfg.get("read_mode", "mean"),
                             cfg.get("read_eps", 1e-3), cfg.get("out_norm", True), onorm_w,
                             cfg.get("out_norm_eps", 1e-2))


def table_from_picks(q, keys1, keys2, log_scale, values, si):
    """TrainedSdm's read for fixed picks (OM:438-455): scores at the picks, softmax(e^log_scale sv), the weighted sum
    of the picked value rows.  q (B, T, H, d_a); si (B, T, H, kk); values (H, M, dh) -> r (B, T, H, dh)."""
    sv = pick_scores(q, None, keys1, keys2, si)
    w = torch.softmax(sv * torch.exp(log_scale)[None, None, :, None], -1)
    H = values.shape[0]
    si = torch.as_tensor(si).to(torch.int64)
    rows = values[torch.arange(H)[None, None, :, None], si]                    # (B, T, H, kk, dh)
    return (w[..., None] * rows).sum(-2)
