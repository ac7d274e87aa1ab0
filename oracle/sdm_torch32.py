"""torch float32 CPU restatement of the run-time SDM mixer -- TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

It follows the reference's op sequence so that, run on the CPU with the same torch build, its addressing bits match
the reference's: ``F.normalize`` of each half and of the sub-keys, ``einsum("nhd,hsd->nhs")``, ``topk`` per half,
the (v1 + v2) * 0.5 grid and a second ``topk`` (OM:134-148).  The scan is the dense chunk form (OM:215-241) driven by
a chunk loop (OM:249-274), and the token recurrence (OM:276-300) is restated as well.  It is the timed CPU baseline
of ``bench.py`` (forward only, ``torch.no_grad``).

``OM`` = experiments/track4/sdmllm/track4_onesdm_models.py, ``SM`` = experiments/track4/sdmllm/track4_sdmllm_models.py.
Parameters are passed as a dict keyed by the module's state_dict names ('norm.w', 'wk.weight', ..., 'keys1',
'keys2', 'addr_b', 'log_scale', 'decays_fixed', 'onorm_w').
"""
import torch
import torch.nn.functional as F


def pk_address(z, keys1, keys2, k):
    """OM:134-148.  z (N, H, d_a) float32; keys (H, n_sub, d_a/2) -> sv (N, H, kk) descending, si (N, H, kk)."""
    half = z.shape[-1] // 2
    n_sub = keys1.shape[1]
    unit1 = F.normalize(keys1, dim=-1).to(z.dtype)
    unit2 = F.normalize(keys2, dim=-1).to(z.dtype)
    s1 = torch.einsum("nhd,hsd->nhs", F.normalize(z[..., :half], dim=-1), unit1)
    s2 = torch.einsum("nhd,hsd->nhs", F.normalize(z[..., half:], dim=-1), unit2)
    c1 = min(k, n_sub)
    v1, i1 = s1.topk(c1, dim=-1)
    v2, i2 = s2.topk(c1, dim=-1)
    grid = ((v1.unsqueeze(-1) + v2.unsqueeze(-2)) * 0.5).flatten(-2)
    kk = min(k, c1 * c1)
    sv, flat = grid.topk(kk, dim=-1)
    row = torch.div(flat, c1, rounding_mode="floor")
    si = i1.gather(-1, row) * n_sub + i2.gather(-1, flat - row * c1)
    return sv, si


def rms_norm(x, w, eps=1e-6):
    """SM:69-71: float math, cast back to x's dtype, times the weight."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


def prepare(x, p, cfg):
    """OM:195-213: norm, the four projections, both addressings, softmax weights and the write gate.

    Returns (siw, ww, sir, wr) as (B, H, T, kk) and V as (B, H, T, dh)."""
    B, T, d = x.shape
    H, d_a, k = cfg["heads"], cfg["d_a"], cfg["k"]
    dh = d // H
    hx = rms_norm(x, p["norm.w"]).float()
    scale = p["log_scale"].exp()[None, :, None]
    kz = (hx @ p["wk.weight"].t()).view(B * T, H, d_a) + p["addr_b"]
    qz = (hx @ p["wq.weight"].t()).view(B * T, H, d_a) + p["addr_b"]
    svw, siw = pk_address(kz, p["keys1"], p["keys2"], k)
    svr, sir = pk_address(qz, p["keys1"], p["keys2"], k)
    ww = torch.softmax(svw * scale, -1)
    wr = torch.softmax(svr * scale, -1)
    if cfg.get("write_gate", True):
        gate = torch.sigmoid(hx @ p["wg.weight"].t() + p["wg.bias"])
    else:
        gate = hx.new_ones(B, T, H)
    ww = ww * gate.reshape(B * T, H, 1)
    kk = siw.shape[-1]

    def by_head(a):
        return a.view(B, T, H, kk).transpose(1, 2)
    V = (hx @ p["wv.weight"].t()).view(B, T, H, dh).transpose(1, 2)
    return by_head(siw), by_head(ww), by_head(sir), by_head(wr), V


def scan_chunk(siw, ww, sir, wr, Vc, mem, cnt, lam, M):
    """OM:215-241 without the segment masks: one chunk of L positions in parallel through dense (L, M) weights."""
    B, H, L, _ = siw.shape
    Aw = torch.zeros(B, H, L, M, dtype=torch.float32).scatter_add(3, siw, ww)
    Ar = torch.zeros(B, H, L, M, dtype=torch.float32).scatter_add(3, sir, wr)
    pos = torch.arange(L, dtype=torch.float32)
    gap = pos[:, None] - 1 - pos[None, :]                      # t - 1 - s
    lam4 = lam[None, :, None, None]
    fade = torch.pow(lam4, gap.clamp(min=0)) * (gap >= 0).float()
    fade_in = torch.pow(lam4, pos[None, None, :, None])
    tail = torch.pow(lam4, (L - 1 - pos)[None, None, :, None])
    ov = torch.matmul(Ar, Aw.transpose(-1, -2)) * fade
    num = torch.matmul(ov, Vc) + torch.matmul(Ar, mem) * fade_in
    den = ov.sum(-1, keepdim=True) + torch.matmul(Ar, cnt[..., None]) * fade_in
    At = Aw * tail
    mem = mem * torch.pow(lam4, float(L)) + torch.matmul(At.transpose(-1, -2), Vc)
    cnt = cnt * torch.pow(lam[None, :, None], float(L)) + At.sum(2)
    return num, den, mem, cnt


def finish(num, den, p, cfg, B, T, dtype):
    """OM:243-247: mean (or sum) read, per-head RMS norm, heads concatenated, then the output map."""
    d = cfg["d"]
    r = num / (den + cfg.get("read_eps", 1e-3)) if cfg.get("read_mode", "mean") == "mean" else num
    if cfg.get("out_norm", True):
        r = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + cfg.get("out_norm_eps", 1e-2)) * p["onorm_w"][None, :, None, :]
    flat = r.transpose(1, 2).reshape(B, T, d)
    return (flat @ p["wo.weight"].t()).to(dtype), flat


def forward(x, p, cfg, chunk=None, return_parts=False):
    """OM:249-274 (reset=None): chunk loop over the prepared sequence, then finish.  Every call starts empty."""
    B, T, d = x.shape
    H = cfg["heads"]
    M = cfg["n_sub"] ** 2
    dh = d // H
    chunk = chunk or cfg.get("chunk", 128)
    siw, ww, sir, wr, V = prepare(x, p, cfg)
    lam = p["decays_fixed"]
    mem = torch.zeros(B, H, M, dh, dtype=torch.float32)
    cnt = torch.zeros(B, H, M, dtype=torch.float32)
    nums, dens = [], []
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        n_, d_, mem, cnt = scan_chunk(siw[:, :, c0:c1], ww[:, :, c0:c1], sir[:, :, c0:c1], wr[:, :, c0:c1],
                                      V[:, :, c0:c1], mem, cnt, lam, M)
        nums.append(n_)
        dens.append(d_)
    y, flat = finish(torch.cat(nums, 2), torch.cat(dens, 2), p, cfg, B, T, x.dtype)
    if return_parts:
        return y, dict(siw=siw, ww=ww, sir=sir, wr=wr, V=V, mem=mem, cnt=cnt, r=flat)
    return y


def forward_sequential(x, p, cfg):
    """OM:276-300 (reset=None): token recurrence with sparse gathers and scatters."""
    B, T, d = x.shape
    H = cfg["heads"]
    M = cfg["n_sub"] ** 2
    dh = d // H
    siw, ww, sir, wr, V = prepare(x, p, cfg)
    lam = p["decays_fixed"][None, :, None]
    mem = torch.zeros(B, H, M, dh, dtype=torch.float32)
    cnt = torch.zeros(B, H, M, dtype=torch.float32)
    nums, dens = [], []
    for t in range(T):
        rows = sir[:, :, t]
        got = mem.gather(2, rows[..., None].expand(-1, -1, -1, dh))
        nums.append((wr[:, :, t, :, None] * got).sum(2))
        dens.append((wr[:, :, t] * cnt.gather(2, rows)).sum(-1, keepdim=True))
        wrow = siw[:, :, t]
        add = torch.zeros_like(mem).scatter_add(2, wrow[..., None].expand(-1, -1, -1, dh),
                                                ww[:, :, t, :, None] * V[:, :, t, None, :])
        mem = mem * lam[..., None] + add
        cnt = cnt * lam + torch.zeros_like(cnt).scatter_add(2, wrow, ww[:, :, t])
    y, _ = finish(torch.stack(nums, 2), torch.stack(dens, 2), p, cfg, B, T, x.dtype)
    return y
