"""GPU parity of the SDM core (sdm_rt_forward: addressing + scan + finish) against the fp64 oracle.

References: RunTimeSdm.prepare / _chunk / forward / finish (track4_onesdm_models.py:195-274, :243-246) and
forward_sequential (:276-300), whose token recurrence the oracle restates.

Each case is checked in two parts (tests/_gpu_util.check_core): the picks and weights of the addressing kernel
against the oracle's (picks identical wherever the fp64 score gap is >= 2.4e-7, weights within 2e-6), then the
read-out against the fp64 recurrence driven by those picks -- plus the fully independent oracle when no pick
differs.  Tolerances: float32 1e-5 (abs and rel); bfloat16 2e-3, plus half a bfloat16 ulp for outputs that are
themselves rounded to bfloat16.
"""
import numpy as np
import pytest
import torch

from tests._gpu_util import bf16_round, check_core, core_inputs, gpu_core, say

pytestmark = pytest.mark.gpu


def test_layer_small_fp32():
    """The fp32 validation workload: B=1, T=256, H=12, dh=64, d_a=64, M=1024, k=8."""
    check_core(*core_inputs(1, 256, 12, 64, 64, 32, seed=41), 8)


def test_layer_small_bf16():
    kz, qz, V, g, p = core_inputs(1, 256, 12, 64, 64, 32, seed=42)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3)


def test_bf16_inputs_fp32_out_and_fused_layout():
    """bf16 activations read from one fused buffer, read-out kept in float32: the arithmetic between the bf16 inputs
    and the output is float32, so the float32 tolerance applies."""
    kz, qz, V, g, p = core_inputs(2, 100, 12, 64, 64, 32, seed=43)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, out_dtype=torch.float32, tol=1e-5, fused=True)


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 130, 200])
def test_ragged_lengths_and_extreme_fades(T):
    """Lengths around the 64-position chunk, with fades 0 (previous-token head) and 1 (never fades)."""
    decays = [0.0, 1.0, 0.5, 0.9, 0.99, 0.999, 0.0, 1.0]
    check_core(*core_inputs(2, T, 8, 16, 16, 8, seed=44 + T, decays=decays, addr_bias=0.3), 8)


@pytest.mark.parametrize("read_mode,out_norm,gate", [("sum", True, True), ("mean", False, True), ("sum", False, False),
                                                     ("mean", True, False)])
def test_read_modes_norm_and_gate(read_mode, out_norm, gate):
    check_core(*core_inputs(1, 150, 4, 32, 32, 16, seed=45, gate=gate), 8, read_mode=read_mode, out_norm=out_norm)


def test_small_fades_rescale_the_slab_often():
    """Fades 0.05-0.3 push the slab multiplier below 2^-60 every chunk, exercising the rescale path."""
    check_core(*core_inputs(1, 400, 4, 16, 16, 8, seed=52, decays=(0.05, 0.1, 0.2, 0.3)), 8)


def test_reference_selftest_shape():
    """d=32, 4 heads of width 8, n_sub 6 (36 locations), d_a 8, k 5, fades (0, 0.7, 0.95, 1) -- the reference's
    self-test layer (track4_onesdm_models.py:704)."""
    check_core(*core_inputs(2, 23, 4, 8, 8, 6, seed=46, decays=(0.0, 0.7, 0.95, 1.0)), 5)


def test_reference_default_shape_k16():
    """The reference's default mixer: 4 heads of width 64, d_a 32, n_sub 32, k 16, fades (0, 0.8, 0.99, 1)."""
    check_core(*core_inputs(2, 160, 4, 64, 32, 32, seed=47, decays=(0.0, 0.8, 0.99, 1.0)), 16)


def test_state_carry_equals_one_pass():
    """Starting from the state another call left equals one pass over the concatenated sequence (kernel against
    itself, float32)."""
    kz, qz, V, g, p = core_inputs(2, 300, 6, 16, 16, 12, seed=48, decays=(0.0, 0.6, 0.9, 0.99, 1.0, 0.95))
    r_all, (m_all, c_all) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    cut = 137
    r1, st = gpu_core(kz[:, :cut], qz[:, :cut], V[:, :cut], g[:, :cut], p, 8, want_state=True)
    r2, (m2, c2) = gpu_core(kz[:, cut:], qz[:, cut:], V[:, cut:], g[:, cut:], p, 8, state_in=st, want_state=True)
    np.testing.assert_allclose(np.concatenate([r1, r2], 1), r_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(m2, m_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(c2, c_all, atol=1e-5, rtol=1e-5)


def test_final_state_matches_oracle_recurrence():
    from oracle import sdm_fp64 as O
    from tests._gpu_util import gpu_address
    kz, qz, V, g, p = core_inputs(2, 150, 4, 16, 16, 8, seed=53, decays=(0.0, 0.5, 0.97, 1.0))
    _, (mem, cnt) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    siw, _, ww = gpu_address(kz, p, 8, gate=g)
    sir, _, wr = gpu_address(qz, p, 8)
    Vb = V.astype(np.float64).reshape(2, 150, 4, 16).transpose(0, 2, 1, 3)
    _, _, m64, c64 = O.scan_recurrence(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                       wr.astype(np.float64), Vb, p["decay"].astype(np.float64),
                                       (np.zeros((2, 4, 64, 16)), np.zeros((2, 4, 64))))
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)


def test_zero_length_and_empty_batch():
    kz, qz, V, g, p = core_inputs(2, 0, 4, 8, 8, 4, seed=49)
    r, (m, c) = gpu_core(kz, qz, V, g, p, 4, want_state=True)
    assert r.shape == (2, 0, 32) and np.all(m == 0) and np.all(c == 0)
    kz, qz, V, g, p = core_inputs(0, 5, 4, 8, 8, 4, seed=50)
    assert gpu_core(kz, qz, V, g, p, 4).shape == (0, 5, 32)
    # no positions with a state in: the state out is that state (copied by a kernel, no memset or copy node)
    kz, qz, V, g, p = core_inputs(2, 0, 4, 8, 8, 4, seed=51)
    rng = np.random.default_rng(51)
    st = (rng.standard_normal((2, 4, 16, 8)).astype(np.float32), rng.random((2, 4, 16)).astype(np.float32))
    r, (m, c) = gpu_core(kz, qz, V, g, p, 4, state_in=st, want_state=True)
    assert r.shape == (2, 0, 32) and np.array_equal(m, st[0]) and np.array_equal(c, st[1])


def test_bench_shape_bf16():
    """B=8, T=2048, H=12, bf16: every pick against the oracle, and the read-out of all 96 (batch row, head) slabs
    against the fp64 recurrence (its per-head-fade form) on the kernel's picks."""
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=51)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    flips = check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3, rescaled=True)
    say("bench-shape picks that differ from the oracle (all at near-ties):", flips)


@pytest.mark.parametrize("T,H,dh,d_a,n_sub", [(64, 4, 16, 16, 8), (150, 4, 16, 16, 8), (150, 12, 64, 64, 32)])
def test_resets_match_the_oracle(T, H, dh, d_a, n_sub):
    """BOS resets (forward(x, reset), OM:229-233): the memory is emptied before the position reads.  Resets at chunk
    starts, inside chunks, twice in one chunk, at the last position, and a row without any; fades 0, 0.5, 0.97, 1
    (and the layer shape's: two column groups per slab sharing the out-norm)."""
    from oracle import sdm_fp64 as O
    from tests._gpu_util import assert_close, gpu_address
    B = 3
    decays = (0.0, 0.5, 0.97, 1.0) * (H // 4)
    kz, qz, V, g, p = core_inputs(B, T, H, dh, d_a, n_sub, seed=90 + T, decays=decays)
    reset = np.zeros((B, T), bool)
    reset[0, [0, 20, 31, T - 1]] = True
    reset[1, [1, 63]] = True
    if T > 64:
        reset[1, [64, 100, 101]] = True
    r, (mem, cnt) = gpu_core(kz, qz, V, g, p, 8, want_state=True, reset=reset)
    siw, _, ww = gpu_address(kz, p, 8, gate=g)
    sir, _, wr = gpu_address(qz, p, 8)
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    num, den, m64, c64 = O.scan_recurrence(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                           wr.astype(np.float64), Vb, p["decay"].astype(np.float64),
                                           (np.zeros((B, H, n_sub ** 2, dh)), np.zeros((B, H, n_sub ** 2))),
                                           reset=reset)
    r64 = O.finish(num, den, "mean", 1e-3, True, p["onorm_w"].astype(np.float64), 1e-2)
    assert_close(r, r64.transpose(0, 2, 1, 3).reshape(B, T, H * dh), 1e-5, msg="read-out with resets")
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)
    # a reset at position 0 changes nothing but rounding (the memory starts empty; the slab's scale restarts at 1)
    reset0 = np.zeros((B, T), bool)
    reset0[:, 0] = True
    np.testing.assert_allclose(gpu_core(kz, qz, V, g, p, 8, reset=reset0), gpu_core(kz, qz, V, g, p, 8),
                               atol=1e-5, rtol=1e-5)


def test_module_forward_with_resets_equals_decode_steps():
    """RunTimeSdm.forward(x, reset) = RunTimeSdm.step token by token with the same resets (float32)."""
    from sdmchat_amd import RunTimeSdm, synthetic as S
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    prm = S.layer_params(cfg, seed=91, decays=(0.0, 0.6, 0.97, 1.0))
    m = RunTimeSdm(64, heads=4, n_sub=8, d_a=16, k=8, decays=tuple(float(v) for v in prm["decays_fixed"]))
    m.load_state_dict({n: torch.from_numpy(v) for n, v in prm.items()}, strict=True)
    m = m.cuda().eval()
    x = torch.from_numpy(S.layer_input(2, 90, 64, seed=92)).cuda()
    reset = torch.zeros(2, 90, dtype=torch.bool, device="cuda")
    reset[0, 30] = reset[0, 70] = reset[1, 64] = True
    with torch.no_grad():
        y = m(x, reset)
        st = m.decode_state(2)
        ys = torch.stack([m.step(x[:, t], st, reset=reset[:, t]) for t in range(90)], 1)
    torch.cuda.synchronize()
    np.testing.assert_allclose(ys.cpu().numpy(), y.cpu().numpy(), atol=2e-5, rtol=1e-4)


def test_crowded_chunks_read_past_the_staged_plan():
    """A large address bias sends every token to nearly the same locations: each position reads most earlier ones of
    its chunk and each location has many writers, so a plan's variable part (later writers, in-chunk contributions)
    runs past the 4 KB the scan stages in LDS and the rest is read from the plan in global memory.  The workspace's
    plan sizes show that the overflow happened."""
    import torch
    from sdmchat_amd import core
    kz, qz, V, g, p = core_inputs(2, 200, 4, 16, 16, 8, seed=91, addr_bias=4.0)
    check_core(kz, qz, V, g, p, 8)
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    ws = core.CoreWorkspace()
    core.core_forward(*(torch.from_numpy(a).cuda() for a in (kz, qz, V, g)), keys1=tp["keys1"], keys2=tp["keys2"],
                      log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"], onorm_w=tp["onorm_w"],
                      gate_bias=tp["gate_bias"], k=8, workspace=ws)
    torch.cuda.synchronize()
    n_plans = 2 * 4 * ((200 + 63) // 64)
    sizes = ws.buf[:4 * n_plans].cpu().view(torch.int32)   # the workspace starts with the plans' variable-part sizes
    say(f"variable-part bytes per plan: max {int(sizes.max())}, mean {float(sizes.float().mean()):.0f}")
    assert int(sizes.max()) > 4096
