"""Host-side contract of the drop-in TrainedSdm module (CPU only): constructor, state_dict names and shapes, default
initialisation, loud failures; and the oracle's table read against a plain loop.

Reference: TrainedSdm (track4_onesdm_models.py:414-457).
"""
import math

import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import TrainedSdm


def test_state_dict_contract_and_default_init():
    m = TrainedSdm(768, 64, heads=1, d_a=32, k=16, seed=2)
    sd = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert sd == {"norm.w": (768,), "wq.weight": (32, 768), "keys1": (1, 64, 16), "keys2": (1, 64, 16),
                  "values": (1, 4096, 768), "log_scale": (1,), "wo.weight": (768, 768)}
    g = torch.Generator().manual_seed(9876 + 2)
    assert torch.equal(m.keys1.data, torch.randn(1, 64, 16, generator=g))
    assert torch.equal(m.keys2.data, torch.randn(1, 64, 16, generator=g))
    assert torch.count_nonzero(m.values) == 0
    torch.testing.assert_close(m.log_scale.data, torch.full((1,), math.log(8.0)))
    assert not TrainedSdm(64, 8, heads=2, d_a=8, learn_scale=False).log_scale.requires_grad


def test_constructor_rejects_what_the_reference_asserts():
    for kw in (dict(d=60, heads=8), dict(d=64, d_a=7), dict(d=64, heads=4, d_a=32)):
        d = kw.pop("d")
        with pytest.raises(ValueError):
            TrainedSdm(d, 8, **kw)


def test_no_cpu_fallback():
    m = TrainedSdm(64, 8, heads=2, d_a=16, k=8)
    x = torch.randn(1, 3, 64)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm device"):
        m(x)
    with pytest.raises(RuntimeError, match="ROCm device"):   # the training path has no CPU fallback either
        m(x)


def test_oracle_table_read_is_the_weighted_row_sum():
    rng = np.random.Generator(np.random.PCG64(5))
    N, H, kk, M, dh = 7, 3, 4, 10, 5
    si = np.stack([np.stack([rng.choice(M, kk, replace=False) for _ in range(H)]) for _ in range(N)])
    w = rng.random((N, H, kk))
    vals = rng.standard_normal((H, M, dh))
    want = np.zeros((N, H, dh))
    for n in range(N):
        for h in range(H):
            for j in range(kk):
                want[n, h] += w[n, h, j] * vals[h, si[n, h, j]]
    np.testing.assert_allclose(O.table_read(si, w, vals), want, atol=1e-12)


def test_onesdm_model_contract():
    """OneSdmLM (track4_onesdm_models.py:471-555): module names, zero-start mixers and tables, the matched TrainedSdm
    size, and the archive refused instead of silently dropped."""
    from sdmchat_amd import OneSdmLM
    from sdmchat_amd.model import matched_sdm_n_sub
    m = OneSdmLM(101, d=64, layers=2, mlp_f=96, heads=4, n_sub=8, d_a=16, k=8)
    keys = set(m.state_dict())
    for k in ("emb.weight", "mems.1.keys1", "mems.0.decays_fixed", "mlps.0.gate.weight", "mlps.1.down.weight",
              "mnorms.1.w", "nf.w"):
        assert k in keys, k
    assert "head.weight" not in keys
    assert all(torch.count_nonzero(mm.wo.weight) == 0 for mm in m.mems)
    s = OneSdmLM(101, d=64, layers=1, heads=4, n_sub=8, d_a=16, ffn="sdm", tie=False)
    assert s.sdm_d_a == 16 and s.sdms[0].n_sub == matched_sdm_n_sub(64, 688, 4, 16)
    assert torch.count_nonzero(s.sdms[0].values) == 0 and "head.weight" in s.state_dict()
    with pytest.raises(NotImplementedError):
        OneSdmLM(101, d=64, layers=1, heads=4, n_sub=8, d_a=16, archive=True)
