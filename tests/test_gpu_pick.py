"""GPU parity of the pick scan (pick plans + pick_scan_kernel), the scan sdm_rt_forward runs for picks of at most 8,
head_dim a multiple of 32 and up to 1,024 locations, against the fp64 oracle.

References: RunTimeSdm._chunk / forward / finish (track4_onesdm_models.py:215-274, :243-246) and the token
recurrence of forward_sequential (:276-300) that the oracle restates; reset at BOS (:229-233, :287-289).

The shapes here all take the pick path (head widths 32, 64 and 96, half widths 8 and 16, 64 or 256 locations); the
cases mirror tests/test_gpu_core.py's for the other scan: lengths around the chunk, fades 0 and 1, the slab rescale,
state carry, the final state, resets, crowded chunks whose plans overflow what the scan stages in LDS, unaligned
value rows, three column groups sharing the out-norm, and the read modes.  Tolerances as there: float32 1e-5,
bfloat16 2e-3 plus half a bfloat16 ulp.
"""
import numpy as np
import pytest
import torch

from tests._gpu_util import assert_close, bf16_round, check_core, core_inputs, gpu_address, gpu_core, say

pytestmark = pytest.mark.gpu

PICK_PLAN_VAR = 2 * 64 * 8 * 12   # offset of a pick plan's variable part (after its 12-byte read and write records)


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 130, 200])
def test_ragged_lengths_and_extreme_fades(T):
    decays = [0.0, 1.0, 0.5, 0.9, 0.99, 0.999, 0.0, 1.0]
    check_core(*core_inputs(2, T, 8, 32, 16, 8, seed=144 + T, decays=decays, addr_bias=0.3), 8)


def test_small_fades_rescale_the_slab_often():
    check_core(*core_inputs(1, 400, 4, 32, 16, 8, seed=152, decays=(0.05, 0.1, 0.2, 0.3)), 8)


@pytest.mark.parametrize("read_mode,out_norm,gate,dh", [("sum", True, True, 32), ("mean", False, True, 64),
                                                        ("sum", False, False, 32), ("mean", True, False, 64)])
def test_read_modes_norm_and_gate(read_mode, out_norm, gate, dh):
    check_core(*core_inputs(1, 150, 4, dh, 32, 16, seed=145 + dh, gate=gate), 8, read_mode=read_mode,
               out_norm=out_norm)


def test_three_column_groups_share_the_out_norm():
    """head_dim 96: three workgroups per slab add their partial sums of squares in one order."""
    check_core(*core_inputs(2, 170, 2, 96, 16, 8, seed=146), 8)


def test_fewer_picks_than_the_pitch():
    """k = 5 of 64 locations: picks 5..7 of every record are pads (row M, weight 0)."""
    check_core(*core_inputs(2, 140, 4, 32, 16, 8, seed=147, decays=(0.0, 0.7, 0.95, 1.0)), 5)


def test_float32_values_bfloat16_out_and_unaligned_rows():
    kz, qz, V, g, p = core_inputs(2, 100, 4, 64, 32, 16, seed=148)
    check_core(kz, qz, V, g, p, 8, dtype=torch.float32, out_dtype=torch.bfloat16, tol=2e-3)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, out_dtype=torch.float32, tol=1e-5, fused=True)


def test_state_carry_equals_one_pass():
    kz, qz, V, g, p = core_inputs(2, 300, 4, 32, 16, 8, seed=149, decays=(0.0, 0.6, 0.99, 1.0))
    r_all, (m_all, c_all) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    cut = 137
    r1, st = gpu_core(kz[:, :cut], qz[:, :cut], V[:, :cut], g[:, :cut], p, 8, want_state=True)
    r2, (m2, c2) = gpu_core(kz[:, cut:], qz[:, cut:], V[:, cut:], g[:, cut:], p, 8, state_in=st, want_state=True)
    np.testing.assert_allclose(np.concatenate([r1, r2], 1), r_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(m2, m_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(c2, c_all, atol=1e-5, rtol=1e-5)


def test_final_state_matches_oracle_recurrence():
    from oracle import sdm_fp64 as O
    B, T, H, dh = 2, 150, 4, 32
    kz, qz, V, g, p = core_inputs(B, T, H, dh, 16, 8, seed=153, decays=(0.0, 0.5, 0.97, 1.0))
    _, (mem, cnt) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    siw, _, ww = gpu_address(kz, p, 8, gate=g)
    sir, _, wr = gpu_address(qz, p, 8)
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    _, _, m64, c64 = O.scan_recurrence(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                       wr.astype(np.float64), Vb, p["decay"].astype(np.float64),
                                       (np.zeros((B, H, 64, dh)), np.zeros((B, H, 64))))
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("T,dh", [(64, 32), (150, 32), (150, 64)])
def test_resets_match_the_oracle(T, dh):
    from oracle import sdm_fp64 as O
    B, H, n_sub = 3, 4, 8
    kz, qz, V, g, p = core_inputs(B, T, H, dh, 16, n_sub, seed=190 + T + dh, decays=(0.0, 0.5, 0.97, 1.0))
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


def test_crowded_chunks_read_past_the_staged_plan():
    """A large address bias sends every token to nearly the same locations: positions have dozens of in-chunk read
    contributions (past the eight a pick plan keeps in its records) and slots many later writers, so the variable
    parts run past the 4 KB the scan stages in LDS and the rest is read from the plan in global memory.  The
    workspace shows that pick plans were written (their headers, at the pick plan's offset, hold the sizes) and
    that they overflowed."""
    from sdmchat_amd import core
    B, T, H = 2, 200, 4
    kz, qz, V, g, p = core_inputs(B, T, H, 32, 16, 8, seed=191, addr_bias=4.0)
    check_core(kz, qz, V, g, p, 8)
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    ws = core.CoreWorkspace()
    core.core_forward(*(torch.from_numpy(a).cuda() for a in (kz, qz, V, g)), keys1=tp["keys1"], keys2=tp["keys2"],
                      log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"], onorm_w=tp["onorm_w"],
                      gate_bias=tp["gate_bias"], k=8, workspace=ws)
    torch.cuda.synchronize()
    n_plans = B * H * ((T + 63) // 64)
    buf = ws.buf.cpu()
    sizes = buf[:4 * n_plans].view(torch.int32)
    say(f"variable-part bytes per plan: max {int(sizes.max())}, mean {float(sizes.float().mean()):.0f}")
    assert int(sizes.max()) > 4096
    off_plans = (4 * n_plans + 255) // 256 * 256
    stride = (len(buf) - off_plans) // n_plans   # an upper bound; the plans sit at a fixed stride from off_plans
    hdr = buf[off_plans + PICK_PLAN_VAR:off_plans + PICK_PLAN_VAR + 4].view(torch.int32)
    assert int(hdr[0]) == int(sizes[0]) and stride > PICK_PLAN_VAR


def test_bench_shape_fp32():
    """The bench shape in float32 (the float32 validation build's arithmetic: float32 projections, values and
    read-out): every pick against the oracle and every slab's read-out against the fp64 recurrence within 1e-5."""
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=181)
    flips = check_core(kz, qz, V, g, p, 8, dtype=torch.float32, tol=1e-5, rescaled=True)
    say("bench-shape float32 picks that differ from the oracle (all at near-ties):", flips)


def test_bench_shape_with_resets_bf16():
    """Packed documents at the bench shape (forward(x, reset), OM:229-233): BOS resets every 100-700 positions, one
    row without any, resets at a chunk's last and first positions and at the last position; bf16.  Every slab's
    read-out against the fp64 recurrence with the resets on the kernel's picks."""
    from oracle import sdm_fp64 as O
    from tests._gpu_util import assert_close, gpu_address, gpu_core
    B, T, H, dh = 8, 2048, 12, 64
    kz, qz, V, g, p = core_inputs(B, T, H, dh, 64, 32, seed=191)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    rng = np.random.Generator(np.random.PCG64(192))
    reset = np.zeros((B, T), bool)
    for b in range(B):
        t = int(rng.integers(0, 50))
        while t < T:
            reset[b, t] = True
            t += int(rng.integers(100, 700))
    reset[3] = False
    reset[5, [63, 64, 2047]] = True
    say("bench shape with resets:", int(reset.sum()), "resets")
    r = gpu_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, reset=reset)
    siw, _, ww = gpu_address(kz, p, 8, dtype=torch.bfloat16, gate=g)
    sir, _, wr = gpu_address(qz, p, 8, dtype=torch.bfloat16)
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    num, den = O.scan_recurrence_rescaled(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                          wr.astype(np.float64), Vb, p["decay"].astype(np.float64), reset=reset)
    r64 = O.finish(num, den, "mean", 1e-3, True, p["onorm_w"].astype(np.float64), 1e-2)
    assert_close(r, r64.transpose(0, 2, 1, 3).reshape(B, T, H * dh), 2e-3, True, msg="read-out with resets")


def test_bench_shape_state_carry_fp32():
    """The bench shape in two calls of 1,024 positions, the second starting from the state the first left
    (state_in / state_out over whole slabs of 1,024 locations), equals one call over 2,048 positions: the read-out
    and the final state, float32."""
    from tests._gpu_util import gpu_core
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=201)
    r_all, (m_all, c_all) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    cut = 1024
    r1, st = gpu_core(kz[:, :cut], qz[:, :cut], V[:, :cut], g[:, :cut], p, 8, want_state=True)
    r2, (m2, c2) = gpu_core(kz[:, cut:], qz[:, cut:], V[:, cut:], g[:, cut:], p, 8, state_in=st, want_state=True)
    np.testing.assert_allclose(np.concatenate([r1, r2], 1), r_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(m2, m_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(c2, c_all, atol=1e-5, rtol=1e-5)


def test_bench_shape_crowded_bf16():
    """The bench shape with addresses that crowd (a large address bias: tokens pick nearly the same locations, many
    contributions past the eight a record keeps and slots with many later writers; variable parts past the 4 KB the
    scan stages, read from the plan), bf16: every pick against the oracle and every slab's read-out against the fp64
    recurrence on the kernel's picks."""
    from sdmchat_amd import core
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=171, addr_bias=4.0)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    flips = check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3, rescaled=True)
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    ws = core.CoreWorkspace()
    core.core_forward(*(torch.from_numpy(a).cuda().to(torch.bfloat16) for a in (kz, qz, V, g)), keys1=tp["keys1"],
                      keys2=tp["keys2"], log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"],
                      onorm_w=tp["onorm_w"], gate_bias=tp["gate_bias"], k=8, workspace=ws)
    torch.cuda.synchronize()
    sizes = ws.buf[:4 * 8 * 12 * 32].cpu().view(torch.int32)
    say(f"crowded bench shape: {flips} picks at near-ties; variable parts mean {float(sizes.float().mean()):.0f} B, "
        f"max {int(sizes.max())} B, {float((sizes > 4096).float().mean()) * 100:.0f}% past the staged 4 KB")
    assert int(sizes.max()) > 4096


def _repeat(a, pattern):
    """Positions that repeat tokens: 'same' one token per batch row, 'cycle3' three tokens in turn, 'three_in_four'
    one token at three positions of every four and fresh ones at the fourth."""
    out = a.copy()
    T = a.shape[1]
    if pattern == "same":
        out[:] = a[:, :1]
    elif pattern == "cycle3":
        out[:] = a[:, np.arange(T) % 3]
    else:
        keep = np.arange(T) % 4 != 3
        out[:, keep] = a[:, :1]
    return out


@pytest.mark.parametrize("pattern", ["same", "cycle3", "three_in_four"])
def test_repeated_tokens_crowd_every_chunk(pattern):
    """Addresses of repeated tokens, the scan's slowest input: the first positions of every chunk own slots with up
    to 63 later writers ('same': 63, 'three_in_four': 47; a wave with a slot of 32 or more writes in teams of eight
    lanes, which also take the wave's other owned slots, here the fresh tokens'; 'cycle3': ~20, the owners' own
    walk), and positions have up to 63 in-chunk read contributions ('same': the last waves' positions past 40 load
    their entries together).  With resets, fades 0 ... 1 and a fade that rescales the slab every chunk: read-out
    and final state against the fp64 recurrence on the kernel's picks."""
    from oracle import sdm_fp64 as O
    B, T, H, dh, n_sub = 3, 200, 4, 64, 8
    kz, qz, V, g, p = core_inputs(B, T, H, dh, 16, n_sub, seed=301, decays=(0.0, 0.3, 0.97, 1.0))
    kz, qz, g = _repeat(kz, pattern), _repeat(qz, pattern), _repeat(g, pattern)
    reset = np.zeros((B, T), bool)
    reset[1, [5, 64, 100]] = True
    reset[2, [63, 130, 131]] = True
    r, (mem, cnt) = gpu_core(kz, qz, V, g, p, 8, want_state=True, reset=reset)
    siw, _, ww = gpu_address(kz, p, 8, gate=g)
    sir, _, wr = gpu_address(qz, p, 8)
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    num, den, m64, c64 = O.scan_recurrence(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                           wr.astype(np.float64), Vb, p["decay"].astype(np.float64),
                                           (np.zeros((B, H, n_sub ** 2, dh)), np.zeros((B, H, n_sub ** 2))),
                                           reset=reset)
    r64 = O.finish(num, den, "mean", 1e-3, True, p["onorm_w"].astype(np.float64), 1e-2)
    assert_close(r, r64.transpose(0, 2, 1, 3).reshape(B, T, H * dh), 1e-5, msg=f"read-out, {pattern} tokens")
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_crowded_slabs_early_write_sums_give_the_same_bits(dtype):
    """A slab with a crowded chunk (a plan's variable part past 4 KB) runs the chunk step whose owners sum their
    writes before the read barrier; that step and the plain one give the same bits.  Batch rows of one repeated
    token (crowded) beside rows of varied tokens, with resets and a fade that rescales the slab every chunk: the
    read-out and the final state with the default threshold, with every slab on the plain step and with every slab
    on the early step are equal bit for bit."""
    from sdmchat_amd import core
    B, T, H, dh, n_sub = 4, 300, 4, 64, 16
    kz, qz, V, g, p = core_inputs(B, T, H, dh, 32, n_sub, seed=307, decays=(0.0, 0.3, 0.97, 1.0))
    for arr in (kz, qz, g):   # rows 0 and 2: one repeated token
        arr[0] = arr[0, :1]
        arr[2] = arr[2, :1]
    reset = np.zeros((B, T), bool)
    reset[0, [70, 200]] = True
    reset[1, [5, 64]] = True
    if dtype == torch.bfloat16:
        kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    outs = []
    try:
        for nbytes in (None, 1 << 30, 0):   # default, every slab plain, every slab early
            core.set_crowded_threshold(nbytes)
            say("crowded threshold", nbytes, dtype)
            outs.append(gpu_core(kz, qz, V, g, p, 8, dtype=dtype, want_state=True, reset=reset))
    finally:
        core.set_crowded_threshold(None)
    (r0, (m0, c0)) = outs[0]
    for r, (m, c) in outs[1:]:
        assert np.array_equal(r.view(np.uint32), r0.view(np.uint32))
        assert np.array_equal(m.view(np.uint32), m0.view(np.uint32))
        assert np.array_equal(c.view(np.uint32), c0.view(np.uint32))
    assert np.isfinite(r0).all()


def test_bench_shape_one_repeated_token_bf16():
    """The bench shape with one repeated token per batch row (every chunk: 8 slots of 63 later writers, positions of
    up to 63 in-chunk contributions, variable parts past the staged 4 KB), bf16: every pick against the oracle and
    every slab's read-out against the fp64 recurrence on the kernel's picks."""
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=303)
    kz, qz, g = (_repeat(a, "same") for a in (kz, qz, g))
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3, rescaled=True)


def test_long_sequence_32k_positions_bf16():
    """T = 32,768 positions in one call (512 chunks per slab: the scan's table of plan sizes near the end of its LDS),
    one batch row, 12 heads, bf16: every pick against the oracle and the read-out of every slab against the fp64
    recurrence on the kernel's picks (its per-head-fade form, the factor folded into the memory as it shrinks)."""
    kz, qz, V, g, p = core_inputs(1, 32768, 12, 64, 64, 32, seed=161)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    flips = check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3, rescaled=True)
    say("T=32768 picks that differ from the oracle (all at near-ties):", flips)


def test_bench_shape_slabs_bf16():
    """B=8, T=2048, H=12 in bfloat16 (the bench workload): picks against the oracle and the read-out of all 96
    slabs against the fp64 recurrence on the kernel's picks (the per-head-fade form of the recurrence)."""
    kz, qz, V, g, p = core_inputs(8, 2048, 12, 64, 64, 32, seed=151)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    flips = check_core(kz, qz, V, g, p, 8, dtype=torch.bfloat16, tol=2e-3, rescaled=True)
    say("bench-shape picks that differ from the oracle (all at near-ties):", flips)


@pytest.mark.parametrize("k,what", [(8, "pick scan"), (16, "chunk scan")])
def test_a_wait_that_gives_up_is_reported(k, what):
    """The out-norm's wait for the other column group of a slab is bounded; when it gives up the chunk's read-outs
    are NaN and sdm_rt_status reports SDM_RT_ETIMEOUT.  The test makes every wait give up at once from the host
    (sdm_rt_set_wait_limit(0): the waits do not even look at the partner's sum), so every kernel still runs to its
    end; then the default limit is restored and the same call is clean.  k = 8 runs the pick scan, k = 16 (pitch
    16) the chunk scan; head_dim 64 gives two column groups in both."""
    from sdmchat_amd import _lib, core
    kz, qz, V, g, p = core_inputs(2, 200, 4, 64, 32, 16, seed=211)
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    args = [torch.from_numpy(a).cuda() for a in (kz, qz, V, g)]
    kw = dict(keys1=tp["keys1"], keys2=tp["keys2"], log_scale=tp["log_scale"], decay=tp["decay"], addr_b=tp["addr_b"],
              onorm_w=tp["onorm_w"], gate_bias=tp["gate_bias"], k=k, check=True)
    core.set_wait_limit(0)
    try:
        out = torch.zeros(2, 200, 4 * 64, device="cuda")
        with pytest.raises(_lib.SdmRtError, match="gave up"):
            core.core_forward(*args, out=out, **kw)
        torch.cuda.synchronize()
        assert bool(torch.isnan(out).all()), f"{what}: a given-up wait must leave NaN read-outs"
    finally:
        core.set_wait_limit(None)
    r = core.core_forward(*args, **kw)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(r).all())
    assert_close(r.cpu().numpy(), gpu_core(kz, qz, V, g, p, k), 0.0, msg=f"{what}: clean call after the error path")
