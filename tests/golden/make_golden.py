"""Write the product-key addressing golden vectors from the reference implementation.

Run in a container that holds the reference checkout (it is read from REF_DIR below, never copied):

    python tests/golden/make_golden.py

Only the addressing function ``pk_address`` (experiments/track4/sdmllm/track4_onesdm_models.py:134-148) is imported:
the exact float32 bits of its scores (CPU ``F.normalize`` and ``einsum`` summation order) and the order ``topk``
gives exactly equal scores cannot be fixed by any closed form, so they are recorded here as data.  Inputs are drawn
from numpy PCG64 seeds and stored next to the outputs, so the fixture is self-contained.

Output: tests/golden/pk_address_golden.npz with, per case NAME, arrays NAME.z (N, H, d_a) float32,
NAME.keys1 / NAME.keys2 (H, n_sub, d_a/2) float32, NAME.k (scalar), NAME.sv (N, H, kk) float32 and NAME.si
(N, H, kk) int16 as returned by the reference (descending order).

``python tests/golden/make_golden.py runtime`` writes tests/golden/runtime_sdm_golden.npz from the reference's
``pk_address``, ``RunTimeSdm`` (:151-300) and ``OneSdmLM`` (:471-555), on the inputs of golden_inputs.py (numpy
PCG64; only seeds and a checksum of each input are stored, the tests regenerate the inputs):
  addr.*     the reference's picks (si int16, sv float32) of the 24,576 layer-workload addresses
             (golden_inputs.layer_addresses: 2,048 tokens x 12 heads, bf16-rounded projections)
  b1_t256.*, edge.*   RunTimeSdm.forward in float32 on the CPU (no autocast): y, and the picks of prepare
             (siw, sir int16 [B, H, T, kk]); b1_t256 = B1 T256 d768 H12 M1024 k8, edge = d32 H4 n_sub 6 k4 chunk 7
             with fades 0 and 1.  Seeds are searched (with the oracle, fp64) for inputs whose every addressing has
             a top-k margin above 2e-6, so the picks are the same in any correct float32 or float64 evaluation.
  model_mlp.*, model_sdm.*   the logits of a tiny OneSdmLM of each arm (golden_inputs.MODEL_KW, reset at BOS), with
             the same margin search.

``python tests/golden/make_golden.py bench`` writes tests/golden/bench_ties_golden.npz: the reference's ordered picks
(si int16, sv float32) at every address of the bench workload (golden_inputs.bench_addresses: the 393,216 write keys
and read queries of B=8, T=2048, 12 heads) where two consecutive of its 9 best fp64 scores lie within 1e-5 (the
pick or the order of the picks is a near-tie), their flat (token, head) indices (near_w, near_r), a checksum of
each address set, and a checksum of the reference's whole ordered pick array of each set (int16, (393,216 / 2, 8)):
a test that splices the recorded near-tie rows into its own picks reproduces that checksum exactly when every other
address's picks equal the reference's.
"""
import os
import sys

import numpy as np
import torch

REF_DIR = "/root/reference/experiments/track4/sdmllm"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "pk_address_golden.npz")


def cases():
    def rng(s):
        return np.random.Generator(np.random.PCG64(s))

    out = {}
    # the layer workload's addressing: 12 heads, 32 sub-keys per 32-dim half (1,024 locations), k = 8
    r = rng(11)
    out["layer"] = dict(z=r.standard_normal((256, 12, 64)), keys1=r.standard_normal((12, 32, 32)),
                        keys2=r.standard_normal((12, 32, 32)), k=8)
    # the reference's default mixer shape: d_a 32 (16-dim halves), k 16
    r = rng(12)
    out["default16"] = dict(z=r.standard_normal((96, 4, 32)), keys1=r.standard_normal((4, 32, 16)),
                            keys2=r.standard_normal((4, 32, 16)), k=16)
    # the reference self-test shapes: n_sub 6 (36 locations), d_a 8, k 5; and n_sub 9 with 6-dim halves
    r = rng(13)
    out["tiny6"] = dict(z=r.standard_normal((30, 4, 8)), keys1=r.standard_normal((4, 6, 4)),
                        keys2=r.standard_normal((4, 6, 4)), k=5)
    r = rng(14)
    out["selftest9"] = dict(z=r.standard_normal((30, 2, 12)), keys1=r.standard_normal((2, 9, 6)),
                            keys2=r.standard_normal((2, 9, 6)), k=5)
    # k larger than n_sub: c1 = n_sub = 4, kk = min(8, 16) = 8
    r = rng(15)
    out["k_gt_nsub"] = dict(z=r.standard_normal((40, 3, 8)), keys1=r.standard_normal((3, 4, 4)),
                            keys2=r.standard_normal((3, 4, 4)), k=8)
    # every location picked: n_sub 2, k 8 -> c1 2, kk 4 = M
    r = rng(16)
    out["all_picked"] = dict(z=r.standard_normal((20, 2, 6)), keys1=r.standard_normal((2, 2, 3)),
                             keys2=r.standard_normal((2, 2, 3)), k=8)
    # exact ties: a zero address (every score 0), one-dim halves (every score +-1), repeated sub-keys
    r = rng(17)
    z = r.standard_normal((64, 4, 64))
    z[::4] = 0.0
    z[1::4, :, :32] = 0.0
    k1 = r.standard_normal((4, 32, 32))
    k2 = r.standard_normal((4, 32, 32))
    k1[:, 16:] = k1[:, :16]
    k2[:, 1::2] = k2[:, ::2] * 3.0
    out["ties"] = dict(z=z, keys1=k1, keys2=k2, k=8)
    r = rng(18)
    out["sign_halves"] = dict(z=r.standard_normal((48, 2, 2)), keys1=r.standard_normal((2, 5, 1)),
                              keys2=r.standard_normal((2, 5, 1)), k=4)
    return out


def main():
    sys.path.insert(0, REF_DIR)
    import track4_onesdm_models as ref  # noqa: E402  (reference checkout, this container only)

    torch.set_num_threads(1)
    blob = {}
    for name, c in cases().items():
        z = torch.from_numpy(c["z"].astype(np.float32))
        k1 = torch.from_numpy(c["keys1"].astype(np.float32))
        k2 = torch.from_numpy(c["keys2"].astype(np.float32))
        with torch.no_grad():
            sv, si = ref.pk_address(z, k1, k2, c["k"])
        blob[f"{name}.z"] = z.numpy()
        blob[f"{name}.keys1"] = k1.numpy()
        blob[f"{name}.keys2"] = k2.numpy()
        blob[f"{name}.k"] = np.int64(c["k"])
        blob[f"{name}.sv"] = sv.numpy().astype(np.float32)
        blob[f"{name}.si"] = si.numpy().astype(np.int16)
        print(name, tuple(z.shape), "k", c["k"], "->", tuple(si.shape), flush=True)
    np.savez_compressed(OUT, **blob)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


def _layer_margin(kw, p, x):
    """The smallest fp64 top-k margin of both addressings of a layer (the oracle's restatement of prepare)."""
    from oracle import sdm_fp64 as O
    B, T, d = x.shape
    H, d_a, k = kw["heads"], kw["d_a"], kw["k"]
    hx = O.rms_norm(x.astype(np.float64), p["norm.w"].astype(np.float64))
    m = np.inf
    for wn in ("wk.weight", "wq.weight"):
        z = (hx @ p[wn].astype(np.float64).T).reshape(B * T, H, d_a) + p["addr_b"]
        m = min(m, float(O.topk_margin(z, p["keys1"], p["keys2"], k).min()))
    return m


def runtime_main():
    sys.path.insert(0, REF_DIR)
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    import track4_onesdm_models as ref  # noqa: E402  (reference checkout, this container only)
    from oracle import sdm_fp64 as O  # noqa: E402
    from tests.golden import golden_inputs as G  # noqa: E402

    torch.set_num_threads(4)
    blob = {}
    # 1. the layer workload's addressing
    z, k1, k2 = G.layer_addresses()
    with torch.no_grad():
        sv, si = ref.pk_address(torch.from_numpy(z), torch.from_numpy(k1), torch.from_numpy(k2), 8)
    blob["addr.seed"] = np.int64(21)
    blob["addr.digest"] = G.digest(z)
    blob["addr.k"] = np.int64(8)
    blob["addr.si"] = si.numpy().astype(np.int16)
    blob["addr.sv"] = sv.numpy().astype(np.float32)
    print("addr", z.shape, "->", tuple(si.shape), flush=True)
    # 2. RunTimeSdm.forward at B1 T256 (the layer's float32 validation workload) and the edge shape
    for name, seed0 in (("b1_t256", 100), ("edge", 200)):
        for seed in range(seed0, seed0 + 60):
            kw, p, x = G.layer_case(name, seed)
            if _layer_margin(kw, p, x) > 2e-6:
                break
        else:
            raise RuntimeError(f"{name}: no seed with clean margins")
        m = ref.RunTimeSdm(kw["d"], heads=kw["heads"], n_sub=kw["n_sub"], d_a=kw["d_a"], k=kw["k"],
                           decays=kw["decays"], chunk=kw["chunk"])
        m.load_state_dict({n: torch.from_numpy(v) for n, v in p.items()}, strict=True)
        m.eval()
        with torch.no_grad():
            xt = torch.from_numpy(x)
            y = m(xt)
            siw, _, sir, _, _ = m.prepare(xt)
        blob[f"{name}.seed"] = np.int64(seed)
        blob[f"{name}.digest"] = G.digest(x)
        blob[f"{name}.y"] = y.numpy().astype(np.float32)
        blob[f"{name}.siw"] = siw.numpy().astype(np.int16)
        blob[f"{name}.sir"] = sir.numpy().astype(np.int16)
        print(name, "seed", seed, "y", tuple(y.shape), flush=True)
    # 3. tiny OneSdmLM logits of both arms
    for ffn in ("mlp", "sdm"):
        kw = dict(G.MODEL_KW)
        V = kw.pop("V")
        for seed in range(300, 360):
            torch.manual_seed(seed)
            mdl = ref.OneSdmLM(V, ffn=ffn, seed=seed, **kw)
            shapes = {n: tuple(t.shape) for n, t in mdl.state_dict().items()}
            p = G.model_params(shapes, seed)
            idx = G.model_tokens(seed)
            cfg = dict(layers=kw["layers"], heads=kw["heads"], d_a=kw["d_a"], k=kw["k"], ffn=ffn,
                       reset_at_bos=True, bos_id=kw["bos_id"], sdm_heads=kw["sdm_heads"], sdm_d_a=kw["sdm_d_a"],
                       sdm_k=kw["sdm_k"])
            margins = []
            O.model_forward(idx, {n: v.astype(np.float64) for n, v in p.items()}, cfg, margins)
            if min(margins) > 2e-6:
                break
        else:
            raise RuntimeError(f"model {ffn}: no seed with clean margins")
        mdl.load_state_dict({n: torch.from_numpy(v) for n, v in p.items()}, strict=True)
        mdl.eval()
        with torch.no_grad():
            logits = mdl(torch.from_numpy(idx))
        blob[f"model_{ffn}.seed"] = np.int64(seed)
        blob[f"model_{ffn}.idx"] = idx.astype(np.int16)
        blob[f"model_{ffn}.logits"] = logits.numpy().astype(np.float32)
        print("model", ffn, "seed", seed, "logits", tuple(logits.shape), flush=True)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "runtime_sdm_golden.npz")
    np.savez_compressed(out, **blob)
    print("wrote", out, os.path.getsize(out), "bytes")


def _order_gap(O, z, keys1, keys2, k):
    """Per address, the smallest fp64 gap between consecutive scores among its kk + 1 best locations: below it, a
    float32 evaluation may pick (the kk-th against the next) or order (two picks) differently from float64.  The
    kk + 1 best lie in the grid of each half's kk + 1 best sub-keys (oracle.sdm_fp64.topk_margin_pruned)."""
    n_sub = keys1.shape[1]
    kk = min(k, min(k, n_sub) ** 2)
    s1, s2 = O.half_scores(z, keys1, keys2)
    c = min(kk + 1, n_sub)
    v1 = -np.sort(-s1, axis=-1)[..., :c]
    v2 = -np.sort(-s2, axis=-1)[..., :c]
    g = -np.sort(-((v1[..., :, None] + v2[..., None, :]) * 0.5).reshape(*v1.shape[:-1], c * c), axis=-1)[..., :kk + 1]
    return (g[..., :-1] - g[..., 1:]).min(-1)


def bench_main(margin=1e-5):
    """The reference's picks at the near-ties of the bench workload's 393,216 addresses (golden_inputs.
    bench_addresses: write keys and read queries of B=8, T=2048, 12 heads): every address where two consecutive of
    its kk + 1 best fp64 scores lie within ``margin`` (where a float32 evaluation may order or pick differently from
    float64), with the reference's ordered picks si and scores sv there."""
    sys.path.insert(0, REF_DIR)
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    import track4_onesdm_models as ref  # noqa: E402  (reference checkout, this container only)
    from oracle import sdm_fp64 as O  # noqa: E402
    from tests.golden import golden_inputs as G  # noqa: E402

    torch.set_num_threads(8)
    zw, zr, k1, k2 = G.bench_addresses()
    blob = {"bench.k": np.int64(8), "bench.margin": np.float64(margin)}
    for name, z in (("w", zw), ("r", zr)):
        mg = _order_gap(O, z.astype(np.float64), k1.astype(np.float64), k2.astype(np.float64), 8)
        near = np.flatnonzero(mg.reshape(-1) < margin)   # flat (token, head) indices
        with torch.no_grad():
            sv, si = ref.pk_address(torch.from_numpy(z), torch.from_numpy(k1), torch.from_numpy(k2), 8)
        H = z.shape[1]
        blob[f"bench.digest_{name}"] = G.digest(z)
        blob[f"bench.near_{name}"] = near.astype(np.int32)
        blob[f"bench.si_{name}"] = si.numpy().reshape(-1, H, 8).reshape(-1, 8)[near].astype(np.int16)
        blob[f"bench.sv_{name}"] = sv.numpy().reshape(-1, 8)[near].astype(np.float32)
        blob[f"bench.all_digest_{name}"] = G.digest(si.numpy().reshape(-1, 8).astype(np.int16))
        print(name, z.shape, "near-ties below", margin, ":", len(near), flush=True)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bench_ties_golden.npz")
    np.savez_compressed(out, **blob)
    print("wrote", out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    if sys.argv[1:] == ["runtime"]:
        runtime_main()
    elif sys.argv[1:] == ["bench"]:
        bench_main()
    else:
        main()
