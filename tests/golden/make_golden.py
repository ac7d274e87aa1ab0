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


if __name__ == "__main__":
    main()
