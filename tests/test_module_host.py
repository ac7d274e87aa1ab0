"""Host-side contract of the drop-in RunTimeSdm module (CPU only): constructor, state_dict names and shapes,
default initialisation, and loud failures instead of any CPU fallback.

Reference: RunTimeSdm.__init__ (track4_onesdm_models.py:154-185), reset_init (:187-190), forward signature (:249).
"""
import math

import pytest
import torch

from sdmchat_amd import RunTimeSdm

EXPECTED = {   # d=768, heads=12, n_sub=32, d_a=64 (the layer workload)
    "norm.w": (768,), "wk.weight": (768, 768), "wq.weight": (768, 768), "wv.weight": (768, 768),
    "wg.weight": (12, 768), "wg.bias": (12,), "wo.weight": (768, 768), "keys1": (12, 32, 32), "keys2": (12, 32, 32),
    "addr_b": (12, 64), "log_scale": (12,), "decays_fixed": (12,), "onorm_w": (12, 64),
}


def make(**kw):
    args = dict(heads=12, n_sub=32, d_a=64, k=8, decays=tuple([0.95] * 12))
    args.update(kw)
    return RunTimeSdm(768, **args)


def test_state_dict_contract():
    sd = make().state_dict()
    assert {k: tuple(v.shape) for k, v in sd.items()} == EXPECTED


def test_learned_decay_and_no_out_norm_variants():
    sd = make(learn_decay=True, out_norm=False).state_dict()
    assert "decay_logit" in sd and "decays_fixed" not in sd and "onorm_w" not in sd
    m = make(learn_decay=True)
    torch.testing.assert_close(m.decay(), torch.full((12,), 0.95), atol=1e-6, rtol=0)


def test_default_init_follows_the_seeded_generator():
    m = make(seed=3, addr_bias=0.5, addr_scale=4.0)
    g = torch.Generator().manual_seed(4321 + 3)
    k1 = torch.randn(12, 32, 32, generator=g)
    k2 = torch.randn(12, 32, 32, generator=g)
    ab = torch.randn(12, 64, generator=g) * 0.5
    assert torch.equal(m.keys1.data, k1) and torch.equal(m.keys2.data, k2) and torch.equal(m.addr_b.data, ab)
    torch.testing.assert_close(m.log_scale.data, torch.full((12,), math.log(4.0)))
    m.reset_init()
    assert torch.count_nonzero(m.wo.weight) == 0 and torch.count_nonzero(m.wg.weight) == 0


def test_constructor_rejects_what_the_reference_asserts():
    with pytest.raises(ValueError):
        RunTimeSdm(770, heads=12, decays=(0.9,) * 12)
    with pytest.raises(ValueError):
        RunTimeSdm(768, heads=12, d_a=63, decays=(0.9,) * 12)
    with pytest.raises(ValueError):
        RunTimeSdm(768, heads=12, decays=(0.9,) * 11)


def test_no_cpu_fallback():
    m = make()
    x = torch.randn(1, 4, 768)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm device"):
        m(x)
    with pytest.raises(RuntimeError, match="ROCm device"):   # the training path has no CPU fallback either
        m(x)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm device"):
        m(x, reset=torch.zeros(1, 4, dtype=torch.bool))
    with torch.no_grad(), pytest.raises(ValueError, match="reset must be"):
        m(x, reset=torch.zeros(1, 5, dtype=torch.bool))


def test_disabled_returns_zeros_without_the_library():
    m = make()
    m.enabled = False
    x = torch.randn(2, 3, 768)
    assert torch.equal(m(x), torch.zeros_like(x))


def test_memory_parameters_and_the_leak_control():
    """OneSdmLM.memory_parameters (track4_onesdm_models.py:557-558) names the mixers' parameters; set_leak
    (:560-564) sets every mixer's _leak, and a mixer forward with the control on raises (the kernels compute only
    the causal recurrence) instead of returning a causal result the control expects to differ."""
    from sdmchat_amd.model import OneSdmLM
    lm = OneSdmLM(64, d=32, layers=2, mlp_f=48, heads=2, n_sub=4, d_a=8, k=4, decays=(0.5, 0.9))
    names = lm.memory_parameters()
    want = {n for n, _ in lm.named_parameters() if n.startswith("mems.")}
    assert names == want and "mems.0.keys1" in names and "mems.1.onorm_w" in names
    assert not any(n.startswith("mlps.") or n.startswith("emb") for n in names)
    lm.set_leak(True)
    assert all(m._leak for m in lm.mems)
    with pytest.raises(NotImplementedError, match="causality control"):
        lm.mems[0](torch.zeros(1, 3, 32))
    lm.set_leak(False)
    assert not any(m._leak for m in lm.mems)
