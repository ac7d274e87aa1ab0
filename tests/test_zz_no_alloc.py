"""GPU parity of sdm_rt_forward_noalloc (the forward on the library's fixed scratch array, for callers that cannot
allocate) with sdm_rt_forward (the same kernels on a caller's workspace): identical read-outs and final state on two
calls in a row, the second smaller, both through the C-ABI; and a call beyond the scratch fails without launching."""
import numpy as np
import pytest
import torch

from sdmchat_amd import _lib, core
from tests._gpu_util import core_inputs, say

pytestmark = pytest.mark.gpu


def _run(kz, qz, V, g, p, no_alloc, want_state=True):
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    kz_d, qz_d, V_d, g_d = (torch.from_numpy(a).cuda().to(torch.bfloat16) for a in (kz, qz, V, g))
    r, (mem, cnt) = core.core_forward(kz_d, qz_d, V_d, g_d, keys1=tp["keys1"], keys2=tp["keys2"],
                                      log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"],
                                      onorm_w=tp["onorm_w"], gate_bias=tp["gate_bias"], k=8, want_state=want_state,
                                      no_alloc=no_alloc)
    torch.cuda.synchronize()
    return r, mem, cnt


def test_noalloc_forward_equals_workspace_forward():
    # the layer shape (12 heads, dh 64, d_a 64, M 1024, k 8): B=4, T=1000, then B=2, T=333
    for B, T, seed in ((4, 1000, 91), (2, 333, 92)):
        kz, qz, V, g, p = core_inputs(B, T, 12, 64, 64, 32, seed=seed)
        say("noalloc forward", B, T)
        r0, m0, c0 = _run(kz, qz, V, g, p, no_alloc=False)
        r1, m1, c1 = _run(kz, qz, V, g, p, no_alloc=True)
        assert torch.equal(r0, r1), f"B={B} T={T}: read-outs differ"
        assert torch.equal(m0, m1) and torch.equal(c0, c1), f"B={B} T={T}: final state differs"


def test_noalloc_forward_rejects_a_call_beyond_its_scratch():
    kz, qz, V, g, p = core_inputs(1, 8, 12, 64, 64, 32, seed=93)
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    big = torch.zeros(40, 2048, 12 * 64, dtype=torch.bfloat16, device="cuda")   # 40 x 2048 positions need > 128 MiB
    bigk = torch.zeros(40, 2048, 12 * 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.SdmRtError, match="scratch"):
        core.core_forward(bigk, bigk, big, None, keys1=tp["keys1"], keys2=tp["keys2"], log_scale=tp["log_scale"],
                          decay=tp["decay"], onorm_w=tp["onorm_w"], k=8, no_alloc=True)
