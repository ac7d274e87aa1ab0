"""GPU parity of the decode step (sdm_rt_decode_step): one token per stream, state carried between calls.

Reference: RunTimeSdm.forward_sequential (track4_onesdm_models.py:276-300), the token recurrence (empty at a reset,
read, then write), which the oracle restates (oracle.sdm_fp64.scan_recurrence).  The decode step addresses with the
same kernels as sdm_rt_forward, so its picks are the forward's; its read-outs are checked against the fp64
recurrence driven by those picks (float32 1e-5, bfloat16 2e-3 plus half a bfloat16 ulp) and against the forward over
the same tokens.
"""
import numpy as np
import pytest
import torch

from oracle import sdm_fp64 as O
from sdmchat_amd import core
from tests._gpu_util import assert_close, bf16_round, core_inputs, gpu_address, gpu_core, gpu_decode, say

pytestmark = pytest.mark.gpu


def _oracle_read(kz, qz, V, g, p, k, reset=None, read_mode="mean", out_norm=True):
    """fp64 recurrence (with resets) on the kernels' own picks and weights -> r (B, T, H*dh)."""
    B, T = V.shape[0], V.shape[1]
    H = p["keys1"].shape[0]
    dh = V.shape[2] // H
    siw, _, ww = gpu_address(kz, p, k, gate=g)
    sir, _, wr = gpu_address(qz, p, k)
    M = p["keys1"].shape[1] ** 2
    Vb = V.astype(np.float64).reshape(B, T, H, dh).transpose(0, 2, 1, 3)
    num, den, mem, cnt = O.scan_recurrence(siw.astype(np.int64), ww.astype(np.float64), sir.astype(np.int64),
                                           wr.astype(np.float64), Vb, p["decay"].astype(np.float64),
                                           (np.zeros((B, H, M, dh)), np.zeros((B, H, M))), reset=reset)
    r = O.finish(num, den, read_mode, 1e-3, out_norm, p["onorm_w"].astype(np.float64), 1e-2)
    return r.transpose(0, 2, 1, 3).reshape(B, T, H * dh), mem, cnt


@pytest.mark.parametrize("d_a,last", [(16, True), (16, False), (12, True)])
def test_decode_matches_oracle_and_forward_fp32(d_a, last):
    """d_a 16: one launch (addressing on the matrix cores); d_a 12: an addressing launch, then the step.  last:
    with and without the last-write slots (a head of decay 0 zeroes those rows, or its whole slab)."""
    decays = (0.0, 1.0, 0.5, 0.97)
    kz, qz, V, g, p = core_inputs(3, 150, 4, 16, d_a, 8, seed=71, decays=decays, addr_bias=0.3)
    say("decode fp32", V.shape, d_a, last)
    r_dec, st = gpu_decode(kz, qz, V, g, p, 8, last=last)
    r64, m64, c64 = _oracle_read(kz, qz, V, g, p, 8)
    np.testing.assert_allclose(r_dec, r64, atol=1e-5, rtol=1e-5)
    mem, cnt = (t.cpu().numpy() for t in st.state())
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)
    r_fwd, (mf, cf) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    np.testing.assert_allclose(r_dec, r_fwd, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(mem, mf, atol=1e-5, rtol=1e-5)


def test_decode_layer_shape_bf16():
    """64 streams of the layer shape (H=12, dh=64, d_a=64, M=1024, k=8), bf16 activations, 40 steps."""
    kz, qz, V, g, p = core_inputs(64, 40, 12, 64, 64, 32, seed=72)
    kz, qz, V, g = (bf16_round(a) for a in (kz, qz, V, g))
    say("decode bf16 layer shape", V.shape)
    r_dec, _ = gpu_decode(kz, qz, V, g, p, 8, dtype=torch.bfloat16)
    r64, _, _ = _oracle_read(kz, qz, V, g, p, 8)
    assert_close(r_dec, r64, 2e-3, bf16_out=True, msg="bf16 decode read-out")


@pytest.mark.parametrize("read_mode,out_norm,gate", [("sum", True, True), ("mean", False, False)])
def test_decode_read_modes(read_mode, out_norm, gate):
    kz, qz, V, g, p = core_inputs(2, 70, 4, 32, 32, 16, seed=73, gate=gate)
    r_dec, _ = gpu_decode(kz, qz, V, g, p, 8, read_mode=read_mode, out_norm=out_norm)
    r64, _, _ = _oracle_read(kz, qz, V, g, p, 8, read_mode=read_mode, out_norm=out_norm)
    np.testing.assert_allclose(r_dec, r64, atol=1e-5, rtol=1e-5)


def test_decode_resets():
    """Per-stream resets (a BOS empties that stream's memory before it reads, OM:287-289)."""
    kz, qz, V, g, p = core_inputs(3, 90, 4, 16, 16, 8, seed=74, decays=(0.3, 1.0, 0.9, 0.99))
    reset = np.zeros((3, 90), bool)
    reset[0, 0] = reset[0, 40] = reset[1, 63] = reset[2, 89] = True
    r_dec, st = gpu_decode(kz, qz, V, g, p, 8, reset=reset)
    r64, m64, c64 = _oracle_read(kz, qz, V, g, p, 8, reset=reset)
    np.testing.assert_allclose(r_dec, r64, atol=1e-5, rtol=1e-5)
    mem, cnt = (t.cpu().numpy() for t in st.state())
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)


def test_decode_zero_fade_with_resets():
    """Heads of decay 0 (only the last step's writes remain: those rows are zeroed, not the slab) across resets."""
    kz, qz, V, g, p = core_inputs(3, 80, 4, 16, 16, 8, seed=81, decays=(0.0, 0.0, 1.0, 0.5))
    reset = np.zeros((3, 80), bool)
    reset[0, 0] = reset[0, 33] = reset[1, 1] = reset[2, 79] = True
    r_dec, st = gpu_decode(kz, qz, V, g, p, 8, reset=reset)
    r64, m64, c64 = _oracle_read(kz, qz, V, g, p, 8, reset=reset)
    np.testing.assert_allclose(r_dec, r64, atol=1e-5, rtol=1e-5)
    mem, cnt = (t.cpu().numpy() for t in st.state())
    np.testing.assert_allclose(mem, m64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c64, atol=1e-5, rtol=1e-5)
    last = st.last.cpu().numpy()
    assert (last[:, :2, 0] >= 0).all() and (last[:, 2:, 0] == -2).all()   # decay-0 heads keep their write slots


def test_decode_small_fades_rescale_the_state():
    """Fades 0 and 0.05-0.3 push the state scale below 2^-60 within a few dozen steps (every step for 0)."""
    kz, qz, V, g, p = core_inputs(2, 120, 4, 16, 16, 8, seed=75, decays=(0.0, 0.05, 0.3, 1.0))
    r_dec, st = gpu_decode(kz, qz, V, g, p, 8)
    r64, m64, _ = _oracle_read(kz, qz, V, g, p, 8)
    np.testing.assert_allclose(r_dec, r64, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(st.state()[0].cpu().numpy(), m64, atol=1e-5, rtol=1e-5)
    assert float(st.scale.min()) >= 2.0 ** -60


def test_decode_continues_a_forward_state():
    """forward over the first 100 tokens, then 60 decode steps from its state = forward over all 160 tokens."""
    kz, qz, V, g, p = core_inputs(2, 160, 4, 16, 16, 8, seed=76, decays=(0.0, 0.6, 0.95, 1.0))
    r_all, (m_all, c_all) = gpu_core(kz, qz, V, g, p, 8, want_state=True)
    cut = 100
    _, (m1, c1) = gpu_core(kz[:, :cut], qz[:, :cut], V[:, :cut], g[:, :cut], p, 8, want_state=True)
    st = core.DecodeState.from_state(torch.from_numpy(m1).cuda(), torch.from_numpy(c1).cuda(), core.pick_pitch(8, 16))
    r2, st = gpu_decode(kz[:, cut:], qz[:, cut:], V[:, cut:], g[:, cut:], p, 8, state=st)
    np.testing.assert_allclose(r2, r_all[:, cut:], atol=1e-5, rtol=1e-5)
    mem, cnt = (t.cpu().numpy() for t in st.state())
    np.testing.assert_allclose(mem, m_all, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cnt, c_all, atol=1e-5, rtol=1e-5)


def test_module_step_equals_forward():
    """RunTimeSdm.step token by token = RunTimeSdm.forward over the sequence (projections, core and wo), fp32."""
    from sdmchat_amd import RunTimeSdm, synthetic as S
    cfg = S.layer_cfg(d=64, heads=4, n_sub=8, d_a=16, k=8)
    prm = S.layer_params(cfg, seed=77, decays=(0.0, 0.6, 0.97, 1.0))
    m = RunTimeSdm(64, heads=4, n_sub=8, d_a=16, k=8, decays=tuple(float(v) for v in prm["decays_fixed"]))
    m.load_state_dict({n: torch.from_numpy(v) for n, v in prm.items()}, strict=True)
    m = m.cuda().eval()
    x = torch.from_numpy(S.layer_input(3, 50, 64, seed=78)).cuda()
    with torch.no_grad():
        y = m(x)
        st = m.decode_state(3)
        ys = torch.stack([m.step(x[:, t], st) for t in range(50)], 1)
    torch.cuda.synchronize()
    np.testing.assert_allclose(ys.cpu().numpy(), y.cpu().numpy(), atol=2e-5, rtol=1e-4)


def test_decode_graph_replays_match_eager():
    """Decode steps captured in a HIP graph: every replay (three, with eager work and synchronisations between them)
    equals the same steps run eagerly from the same state."""
    kz, qz, V, g, p = core_inputs(4, 1, 4, 16, 16, 8, seed=79, decays=(0.0, 0.5, 0.9, 1.0))
    tp = {n: torch.from_numpy(v).cuda() for n, v in p.items()}
    kz_d, qz_d, V_d, g_d = (torch.from_numpy(a[:, 0]).cuda() for a in (kz, qz, V, g))
    prm = core._params("cuda", tp["keys1"], tp["keys2"], tp["addr_b"], tp["log_scale"], tp["decay"], tp["onorm_w"],
                       tp["gate_bias"])
    ws = core.CoreWorkspace()

    def step(st, out):
        core.decode_step(kz_d, qz_d, V_d, g_d, st, keys1=tp["keys1"], keys2=tp["keys2"], log_scale=tp["log_scale"],
                         decay=tp["decay"], k=8, out=out, workspace=ws, params=prm)

    eager, ge = core.DecodeState.empty(4, 4, 64, 16, "cuda", 8), torch.empty(4, 64, device="cuda")
    graphed, gg = core.DecodeState.empty(4, 4, 64, 16, "cuda", 8), torch.empty(4, 64, device="cuda")
    step(core.DecodeState.empty(4, 4, 64, 16, "cuda", 8), torch.empty(4, 64, device="cuda"))   # sizes the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(graphed, gg)
        step(graphed, gg)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        step(eager, ge)
        step(eager, ge)
        junk = torch.randn(1000, device="cuda").sum()   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(gg, ge), f"replay {rep}: read-out differs"
        assert torch.equal(graphed.mem, eager.mem) and torch.equal(graphed.cnt, eager.cnt)
        assert torch.equal(graphed.scale, eager.scale) and torch.equal(graphed.last, eager.last)
        del junk
