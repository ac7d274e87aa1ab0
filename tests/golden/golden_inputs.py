"""Deterministic inputs of the golden fixtures (numpy PCG64 only), shared by make_golden.py, which feeds them to the
reference, and the tests, which feed them to the oracle and the HIP path.  Parameters are keyed by the reference's
state_dict names (experiments/track4/sdmllm/track4_onesdm_models.py:154-185, :414-436, :471-521)."""
import math

import numpy as np


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _xavier(r, fan_out, fan_in):
    b = math.sqrt(6.0 / (fan_in + fan_out))
    return r.uniform(-b, b, size=(fan_out, fan_in)).astype(np.float32)


def digest(a):
    """A checksum of an array's bytes (the tests check that the regenerated inputs are the recorded ones)."""
    import hashlib
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest()[:8], np.int64)[0]


def bf16_round(a):
    """float32 values rounded to bfloat16 (nearest, ties to even), returned as float32."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


# --- the addressing of the layer workload: 2,048 tokens x 12 heads of bf16-rounded write-key projections ---------
def layer_addresses(seed=21, N=2048, d=768, H=12, d_a=64, n_sub=32):
    """z (N, H, d_a) float32 (bf16 values: x ~ N(0, 1) times a Xavier-uniform wk, computed in float64, rounded to
    float32 then bfloat16) and sub-keys keys1, keys2 (H, n_sub, d_a / 2) ~ N(0, 1) float32."""
    r = _rng(seed)
    x = r.standard_normal((N, d))
    w = _xavier(r, H * d_a, d).astype(np.float64)
    z = bf16_round((x @ w.T).astype(np.float32)).reshape(N, H, d_a)
    k1 = r.standard_normal((H, n_sub, d_a // 2)).astype(np.float32)
    k2 = r.standard_normal((H, n_sub, d_a // 2)).astype(np.float32)
    return z, k1, k2


# --- the addresses of the bench workload ------------------------------------------------------------------------
def bench_addresses():
    """The write keys and read queries of the layer bench workload (B=8, T=2048, d=768, 12 heads of M=1,024, d_a 64,
    k=8; parameters sdmchat_amd.synthetic.layer_params(seed=0), input layer_input(seed=1)) as a bfloat16 layer forms
    them: x rounded to bfloat16, the input norm x rsqrt(mean x^2 + 1e-6) rounded to bfloat16 (norm.w is 1), the
    wk and wq maps summed in float64 and rounded to bfloat16 (addr_b is 0).  Returns zw, zr (16,384, 12, 64) float32
    and keys1, keys2 (12, 32, 32) float32.  (The GPU's own float32 maps may round an occasional value the other
    way; these are the fixture's addresses, fed as they are to every implementation.)"""
    from sdmchat_amd import synthetic as S
    cfg = S.layer_cfg()
    p = S.layer_params(cfg, seed=0)
    x = bf16_round(S.layer_input(8, 2048, 768, seed=1)).astype(np.float64).reshape(8 * 2048, 768)
    hx = bf16_round((x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6)).astype(np.float32)).astype(np.float64)
    zw = bf16_round((hx @ p["wk.weight"].astype(np.float64).T).astype(np.float32)).reshape(-1, 12, 64)
    zr = bf16_round((hx @ p["wq.weight"].astype(np.float64).T).astype(np.float32)).reshape(-1, 12, 64)
    return zw, zr, p["keys1"], p["keys2"]


# --- one RunTimeSdm layer ----------------------------------------------------------------------------------------
def layer_case(name, seed):
    """(constructor kwargs, state dict of float32 arrays, x (B, T, d) float32) of a named layer case:
    'b1_t256' -- B=1, T=256, d=768, 12 heads, M=1,024, d_a 64, k 8, fades U(0.9, 0.999), chunk 128;
    'edge'    -- B=2, T=40, d=32, 4 heads, n_sub 6, d_a 8, k 4, fades (0, 1, 0, 1), chunk 7."""
    r = _rng(seed)
    if name == "b1_t256":
        B, T, d, H, n_sub, d_a, k, chunk = 1, 256, 768, 12, 32, 64, 8, 128
        decays = r.uniform(0.9, 0.999, size=H).astype(np.float32)
    elif name == "edge":
        B, T, d, H, n_sub, d_a, k, chunk = 2, 40, 32, 4, 6, 8, 4, 7
        decays = np.array([0.0, 1.0, 0.0, 1.0], np.float32)
    else:
        raise ValueError(name)
    dh = d // H
    kw = dict(d=d, heads=H, n_sub=n_sub, d_a=d_a, k=k, decays=tuple(float(v) for v in decays), chunk=chunk)
    p = {
        "norm.w": r.uniform(0.5, 1.5, size=d).astype(np.float32),
        "wk.weight": _xavier(r, H * d_a, d),
        "wq.weight": _xavier(r, H * d_a, d),
        "wv.weight": _xavier(r, d, d),
        "wg.weight": _xavier(r, H, d),
        "wg.bias": r.uniform(-1.0, 1.0, size=H).astype(np.float32),
        "wo.weight": _xavier(r, d, d),
        "keys1": r.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
        "keys2": r.standard_normal((H, n_sub, d_a // 2)).astype(np.float32),
        "addr_b": (r.standard_normal((H, d_a)) * 0.3).astype(np.float32),
        "log_scale": np.full(H, math.log(8.0), np.float32),
        "decays_fixed": decays,
        "onorm_w": r.uniform(0.5, 1.5, size=(H, dh)).astype(np.float32),
    }
    x = r.standard_normal((B, T, d)).astype(np.float32)
    return kw, p, x


# --- a tiny OneSdmLM of each arm ---------------------------------------------------------------------------------
MODEL_KW = dict(V=97, d=64, layers=2, mlp_f=96, heads=4, n_sub=8, d_a=16, k=8, decays=(0.0, 0.6, 0.95, 1.0),
                sdm_n_sub=10, sdm_heads=2, sdm_d_a=16, sdm_k=8, reset_at_bos=True, bos_id=3, addr_bias=0.2)


def model_params(shapes, seed):
    """A float32 state dict for the given {name: shape} (sorted by name): every 2-D map and table N(0, 0.1) (the
    value tables N(0, 0.3)), norm weights U(0.5, 1.5), sub-keys N(0, 1), log_scale ln 8, the mixer's addr_b N(0, 0.2),
    gate bias U(-1, 1); fades are buffers and keep MODEL_KW's."""
    r = _rng(seed)
    p = {}
    for n in sorted(shapes):
        s = tuple(shapes[n])
        if n.endswith("decays_fixed"):
            p[n] = np.asarray(MODEL_KW["decays"], np.float32)
        elif n.endswith("log_scale"):
            p[n] = np.full(s, math.log(8.0), np.float32)
        elif n.endswith(("keys1", "keys2")):
            p[n] = r.standard_normal(s).astype(np.float32)
        elif n.endswith(("norm.w", "nf.w", "onorm_w")) or (n.startswith("mnorms.") and n.endswith(".w")):
            p[n] = r.uniform(0.5, 1.5, size=s).astype(np.float32)
        elif n.endswith("addr_b"):
            p[n] = (r.standard_normal(s) * 0.2).astype(np.float32)
        elif n.endswith("wg.bias"):
            p[n] = r.uniform(-1.0, 1.0, size=s).astype(np.float32)
        elif n.endswith("values"):
            p[n] = (r.standard_normal(s) * 0.3).astype(np.float32)
        else:
            p[n] = (r.standard_normal(s) * 0.1).astype(np.float32)
    return p


def model_tokens(seed, B=2, T=70, V=97, bos=3):
    r = _rng(seed)
    idx = r.integers(0, V, size=(B, T))
    idx[0, [0, 25, 64]] = bos
    idx[1, 40] = bos
    return idx.astype(np.int64)
