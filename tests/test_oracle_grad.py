"""Pins of the float64 gradient oracle (oracle/sdm_grad64.py), CPU only.

* its forward equals the token recurrence of oracle/sdm_fp64.py (core_forward) for the same picks;
* every gradient it gives (autograd) equals central finite differences of sdm_fp64.core_forward, which recomputes the
  picks (the test checks they do not move), for kz, qz, V, gate logits, both sub-key sets, addr_b, log_scale, the
  fades, onorm_w and the gate bias -- with and without resets, gate, mean read and out-norm;
* the identity the HIP backward uses for the fade: lam dL/dlam = sum_t t P_t - sum_s (s+1) Q_s with
  P_t = sum_i wr[t,i] dL/dwr[t,i] and Q_s = sum_j ww[s,j] dL/dww[s,j].
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from oracle import sdm_grad64 as G


def make_case(seed, B=1, T=14, H=2, dh=4, d_a=4, n_sub=3, k=2, gate=True, reset=False):
    rng = np.random.default_rng(seed)
    c = dict(
        kz=rng.standard_normal((B, T, H, d_a)), qz=rng.standard_normal((B, T, H, d_a)),
        V=rng.standard_normal((B, T, H, dh)), gl=rng.standard_normal((B, T, H)) if gate else None,
        keys1=rng.standard_normal((H, n_sub, d_a // 2)), keys2=rng.standard_normal((H, n_sub, d_a // 2)),
        addr_b=0.3 * rng.standard_normal((H, d_a)), log_scale=np.log(8.0) + 0.2 * rng.standard_normal(H),
        decay=rng.uniform(0.3, 0.95, H), onorm_w=1.0 + 0.2 * rng.standard_normal((H, dh)),
        gate_bias=0.3 * rng.standard_normal(H) if gate else None,
        reset=(rng.random((B, T)) < 0.2) if reset else None)
    return c


def np_forward(c, cfg):
    """sdm_fp64.core_forward on the case (addr_b and the gate bias added here); returns r and the picks."""
    p = dict(keys1=c["keys1"], keys2=c["keys2"], log_scale=c["log_scale"], decay=c["decay"], onorm_w=c["onorm_w"])
    gl = None if c["gl"] is None else c["gl"] + c["gate_bias"]
    r, parts = O.core_forward(c["kz"] + c["addr_b"], c["qz"] + c["addr_b"], c["V"], gl, p, cfg, return_parts=True,
                              reset=c["reset"])
    B, T, H, _ = c["kz"].shape
    kk = parts["siw"].shape[-1]
    return r, parts["siw"].reshape(B, T, H, kk), parts["sir"].reshape(B, T, H, kk)


NAMES = ("kz", "qz", "V", "gl", "keys1", "keys2", "addr_b", "log_scale", "decay", "onorm_w", "gate_bias")


def torch_forward(c, cfg, siw, sir, grad=False):
    t = {n: (None if c[n] is None else torch.tensor(c[n], dtype=torch.float64, requires_grad=grad)) for n in NAMES}
    r = G.core_from_picks(t["kz"], t["qz"], t["V"], t["gl"], t["keys1"], t["keys2"], t["addr_b"], t["log_scale"],
                          t["decay"], t["onorm_w"], t["gate_bias"], siw, sir, cfg, reset=c["reset"])
    return r, t


CASES = [
    (dict(k=2, read_mode="mean", out_norm=True), dict(gate=True, reset=True)),
    (dict(k=2, read_mode="sum", out_norm=False), dict(gate=False, reset=False)),
    (dict(k=3, read_mode="mean", out_norm=True), dict(gate=True, reset=False, n_sub=4)),
]


@pytest.mark.parametrize("cfg,shape", CASES)
def test_forward_equals_the_token_recurrence(cfg, shape):
    c = make_case(1, **shape)
    r_np, siw, sir = np_forward(c, cfg)
    r_t, _ = torch_forward(c, cfg, siw, sir)
    np.testing.assert_allclose(r_t.numpy(), r_np, rtol=0, atol=1e-12)


@pytest.mark.parametrize("cfg,shape", CASES)
def test_gradients_equal_finite_differences(cfg, shape):
    c = make_case(2, **shape)
    r_np, siw, sir = np_forward(c, cfg)
    wgt = np.random.default_rng(7).standard_normal(r_np.shape)
    r_t, t = torch_forward(c, cfg, siw, sir, grad=True)
    (r_t * torch.tensor(wgt)).sum().backward()
    h = 1e-6
    for name in NAMES:
        if c[name] is None:
            continue
        if t[name].grad is None:   # a parameter the configuration does not read (onorm_w without the out-norm)
            assert name == "onorm_w" and not cfg["out_norm"]
            continue
        grad = t[name].grad.numpy()
        base = c[name]
        for idx in np.ndindex(base.shape):
            vals = []
            for sgn in (1.0, -1.0):
                cc = dict(c)
                x = np.array(base, np.float64)
                x[idx] += sgn * h
                cc[name] = x
                r, sw, sr = np_forward(cc, cfg)
                assert np.array_equal(sw, siw) and np.array_equal(sr, sir), f"picks moved at {name}{idx}"
                vals.append(float(np.sum(r * wgt)))
            fd = (vals[0] - vals[1]) / (2 * h)
            assert abs(fd - grad[idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, grad[idx])


def test_fade_gradient_identity():
    """lam dL/dlam equals sum_t t P_t - sum_s (s+1) Q_s (per head, summed over batch rows), with resets."""
    cfg = dict(k=3, read_mode="mean", out_norm=True)
    c = make_case(3, B=2, T=40, H=3, dh=5, d_a=6, n_sub=4, k=3, gate=True, reset=True)
    c["decay"] = np.array([0.2, 0.9, 1.0])
    r_np, siw, sir = np_forward(c, cfg)
    p = dict(keys1=c["keys1"], keys2=c["keys2"], log_scale=c["log_scale"], decay=c["decay"], onorm_w=c["onorm_w"])
    _, parts = O.core_forward(c["kz"] + c["addr_b"], c["qz"] + c["addr_b"], c["V"], c["gl"] + c["gate_bias"], p, cfg,
                              return_parts=True, reset=c["reset"])
    B, T, H, kk = siw.shape
    ww = torch.tensor(parts["ww"].reshape(B, T, H, kk), requires_grad=True)
    wr = torch.tensor(parts["wr"].reshape(B, T, H, kk), requires_grad=True)
    lam = torch.tensor(c["decay"], requires_grad=True)
    r = G.read_from_weights(siw, ww, sir, wr, torch.tensor(c["V"]), lam, 16, c["reset"], "mean", 1e-3, True,
                            torch.tensor(c["onorm_w"]), 1e-2)
    np.testing.assert_allclose(r.detach().numpy(), r_np, rtol=0, atol=1e-12)
    wgt = torch.tensor(np.random.default_rng(8).standard_normal(r.shape))
    (r * wgt).sum().backward()
    P = (wr * wr.grad).sum(-1).detach()      # (B, T, H)
    Q = (ww * ww.grad).sum(-1).detach()
    t = torch.arange(T, dtype=torch.float64)[None, :, None]
    rhs = (t * P - (t + 1) * Q).sum((0, 1))
    lhs = lam.detach() * lam.grad
    np.testing.assert_allclose(lhs.numpy(), rhs.numpy(), rtol=1e-10, atol=1e-12)
    assert abs(lhs[2].item()) > 1e-3   # a non-trivial fade gradient is checked


@pytest.mark.parametrize("n_sub,k", [(4, 3), (5, 6)])
def test_table_gradients_equal_finite_differences(n_sub, k):
    """TrainedSdm's read for fixed picks (sdm_grad64.table_from_picks): its value equals sdm_fp64's pk_address +
    address_weights + table_read, and its autograd gradients (q, both sub-key sets, log_scale, the value tables)
    equal central finite differences of that numpy forward, which recomputes the picks (checked not to move)."""
    rng = np.random.default_rng(11 + n_sub)
    B, T, H, d_a, dh = 1, 6, 2, 4, 3
    c = dict(q=rng.standard_normal((B, T, H, d_a)), keys1=rng.standard_normal((H, n_sub, d_a // 2)),
             keys2=rng.standard_normal((H, n_sub, d_a // 2)), log_scale=np.log(8.0) + 0.2 * rng.standard_normal(H),
             values=rng.standard_normal((H, n_sub * n_sub, dh)))

    def np_read(cc):
        sv, si = O.pk_address(cc["q"].reshape(B * T, H, d_a), cc["keys1"], cc["keys2"], k)
        w = O.address_weights(sv, cc["log_scale"])
        return O.table_read(si, w, cc["values"]).reshape(B, T, H, dh), si

    r_np, si = np_read(c)
    kk = si.shape[-1]
    t = {n: torch.tensor(v, requires_grad=True) for n, v in c.items()}
    r = G.table_from_picks(t["q"], t["keys1"], t["keys2"], t["log_scale"], t["values"], si.reshape(B, T, H, kk))
    np.testing.assert_allclose(r.detach().numpy(), r_np, rtol=0, atol=1e-12)
    wgt = np.random.default_rng(5).standard_normal(r_np.shape)
    (r * torch.tensor(wgt)).sum().backward()
    h = 1e-6
    for name, base in c.items():
        grad = t[name].grad.numpy()
        for idx in np.ndindex(base.shape):
            vals = []
            for sgn in (1.0, -1.0):
                cc = dict(c)
                x = np.array(base, np.float64)
                x[idx] += sgn * h
                cc[name] = x
                rr, s2 = np_read(cc)
                assert np.array_equal(s2, si), f"picks moved at {name}{idx}"
                vals.append(float(np.sum(rr * wgt)))
            fd = (vals[0] - vals[1]) / (2 * h)
            assert abs(fd - grad[idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, grad[idx])
