"""Seeded synthetic layer parameters and inputs for the run-time SDM mixer workloads.

Everything is drawn with numpy's PCG64 from an integer seed, so the same arrays are produced on any machine.
Parameter names and shapes are the state_dict of the reference's ``RunTimeSdm`` (track4_onesdm_models.py:154-185):
2-D weights Xavier-uniform U(+-sqrt(6 / (fan_in + fan_out))), wg.bias 0, norm.w = onorm_w = 1, keys1/keys2 ~ N(0, 1),
addr_b 0, log_scale ln 8, per-head fades decays_fixed ~ U(0.9, 0.999); inputs x ~ N(0, 1).
"""
import math

import numpy as np

# The single-layer workloads: a fp32 validation shape and the bf16 throughput shape.
LAYER_SMALL = dict(B=1, T=256, d=768, heads=12, n_sub=32, d_a=64, k=8)
LAYER_BENCH = dict(B=8, T=2048, d=768, heads=12, n_sub=32, d_a=64, k=8)


def layer_cfg(d=768, heads=12, n_sub=32, d_a=64, k=8, chunk=128, **extra):
    """Constructor-style configuration of one layer (mean read, out-norm on, write gate on)."""
    cfg = dict(d=d, heads=heads, n_sub=n_sub, d_a=d_a, k=k, chunk=chunk, read_mode="mean", read_eps=1e-3,
               out_norm=True, out_norm_eps=1e-2, write_gate=True)
    cfg.update(extra)
    return cfg


def xavier(rng, fan_out, fan_in):
    bound = math.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-bound, bound, size=(fan_out, fan_in)).astype(np.float32)


def layer_params(cfg, seed=0, decay_range=(0.9, 0.999), decays=None):
    """float32 numpy parameters keyed by state_dict name."""
    rng = np.random.Generator(np.random.PCG64(seed))
    d, H, n_sub, d_a = cfg["d"], cfg["heads"], cfg["n_sub"], cfg["d_a"]
    dh = d // H
    p = {
        "norm.w": np.ones(d, np.float32),
        "wk.weight": xavier(rng, H * d_a, d),
        "wq.weight": xavier(rng, H * d_a, d),
        "wv.weight": xavier(rng, d, d),
        "wg.weight": xavier(rng, H, d),
        "wg.bias": np.zeros(H, np.float32),
        "wo.weight": xavier(rng, d, d),
        "keys1": rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
        "keys2": rng.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
        "addr_b": np.zeros((H, d_a), np.float32),
        "log_scale": np.full(H, math.log(8.0), np.float32),
        "onorm_w": np.ones((H, dh), np.float32),
    }
    if decays is None:
        p["decays_fixed"] = rng.uniform(decay_range[0], decay_range[1], size=H).astype(np.float32)
    else:
        p["decays_fixed"] = np.asarray(decays, np.float32)
    return p


def layer_input(B, T, d, seed=1):
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((B, T, d)).astype(np.float32)


# The whole-model workloads: the PARTIAL arm (SwiGLU of hidden 2,048 after each mixer) and the FULL arm (a TrainedSdm
# of 4,096 slots, one head of width 768, k 16), 12 layers of d 768, vocabulary 32,768.
MODEL_FULL = dict(V=32768, d=768, layers=12, mlp_f=2048, heads=12, n_sub=32, d_a=64, k=8)
ARMS = {"swiglu": dict(ffn="mlp"), "trained_sdm": dict(ffn="sdm", sdm_n_sub=64, sdm_heads=1, sdm_k=16)}


def full_model(arm, seed=5, **over):
    """A OneSdmLM of the whole-model workload with seeded weights (CPU, float32): the reference's initialisation
    (torch.manual_seed(seed)) with the zero-start maps (the mixers' wo and wg, the TrainedSdm output maps and value
    tables) filled with N(0, 0.02), so every layer carries signal; fades U(0.9, 0.999) per head."""
    import torch

    from .model import OneSdmLM

    kw = dict(MODEL_FULL)
    kw.update(ARMS[arm])
    kw.update(over)
    V = kw.pop("V")
    kw.setdefault("decays", tuple(float(v) for v in np.random.Generator(np.random.PCG64(3)).uniform(0.9, 0.999,
                                                                                                     kw["heads"])))
    torch.manual_seed(seed)
    m = OneSdmLM(V, **kw)
    gen = torch.Generator().manual_seed(seed + 6)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith(("wo.weight", "wg.weight", "values")):
                p.normal_(0.0, 0.02, generator=gen)
    return m


def model_tokens(B, T, V=32768, seed=11):
    """Seeded uniform token ids (B, T) int64."""
    return np.random.Generator(np.random.PCG64(seed)).integers(0, V, size=(B, T)).astype(np.int64)
