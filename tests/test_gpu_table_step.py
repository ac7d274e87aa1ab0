"""GPU tests of sdm_rt_table_step (core.table_step), TrainedSdm's read for a few tokens in one launch
(track4_onesdm_models.py:438-455: the query map, pk_address :134-148 and the weighted read): it must give, bit for
bit, what the three separate entry points give (sdm_rt_gemm_rows for the query map, sdm_rt_address, sdm_rt_table_read),
whose parity with the oracle the other tests check.  Shapes cover every addressing mode (32 and 64 sub-keys per half,
full and masked grids, 8 and 16 picks), d_a 32 and 64 and 1 ... 256 tokens."""
import pytest
import torch

from sdmchat_amd import TrainedSdm, core
from tests._gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,n_sub,d_a,k,d,rows", [(1, 64, 32, 16, 768, 64),    # the FULL model's table layer
                                                  (1, 64, 32, 16, 768, 1),
                                                  (1, 64, 32, 16, 768, 256),
                                                  (2, 32, 32, 8, 256, 37),     # full 32 x 32 grid
                                                  (3, 20, 64, 12, 192, 5),     # masked grid, 16 picks
                                                  (2, 48, 64, 8, 128, 64),     # 64 sub-keys, masked
                                                  (1, 64, 64, 8, 64, 9),       # 64 sub-keys, full, 8 picks
                                                  (1, 32, 32, 8, 1024, 5)])    # head_dim 1,024: the read's limit
def test_table_step_equals_map_address_and_read(H, n_sub, d_a, k, d, rows):
    g = torch.Generator(device="cpu").manual_seed(H * 1000 + n_sub + d_a + k + rows)
    dh = d // H
    hx = torch.randn(1, rows, d, generator=g).to(torch.bfloat16).cuda()
    wq = (torch.randn(H * d_a, d, generator=g) * d ** -0.5).to(torch.bfloat16).cuda()
    keys1 = torch.randn(H, n_sub, d_a // 2, generator=g).cuda()
    keys2 = torch.randn(H, n_sub, d_a // 2, generator=g).cuda()
    log_scale = (torch.full((H,), 2.0) + torch.rand(H, generator=g) * 0.5).cuda()
    values = torch.randn(H, n_sub * n_sub, dh, generator=g).to(torch.bfloat16).cuda()
    say("table_step", H, n_sub, d_a, k, d, rows)
    with torch.no_grad():
        r, si, sc, w, q = core.table_step(hx, wq, keys1, keys2, log_scale, values, k, want_q=True)
        q_ref = core.linear(hx, wq, as_matmul=True)
        si_ref, sc_ref, w_ref = core.address(q_ref, keys1, keys2, k, log_scale, padded=True)
        r_ref = core.table_read(si_ref, w_ref, values, k, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref)
    assert torch.equal(si, si_ref)
    assert torch.equal(sc, sc_ref) and torch.equal(w, w_ref)
    assert torch.equal(r, r_ref)


def test_trained_sdm_decode_shape_takes_the_one_launch_read():
    """TrainedSdm.forward on a few bfloat16 tokens (a decode step) runs the read in one launch and gives the same
    output, picks and queries as the separate calls (a forward of more tokens than the one-launch read takes)."""
    torch.manual_seed(5)
    m = TrainedSdm(768, 64, heads=1, d_a=32, k=16).cuda().to(torch.bfloat16).eval()
    with torch.no_grad():
        m.values.normal_()
        m.wo.weight.normal_(std=0.03)
    x = torch.randn(1, 300, 768, device="cuda").to(torch.bfloat16)   # 300 tokens: the separate calls
    m.keep_picks = True
    with torch.no_grad():
        y_all = m(x)
        si_all, q_all = m.last_si.clone(), m.last_q.clone()
        y_few = m(x[:, :64])                                           # 64 tokens: one launch
        assert core.table_step_fits(x[:, :64], m.wq.weight, m.values, 32)
    # the query map of more than 256 rows is the GEMM library's: compare the one-launch read with the separate
    # calls on the same 64 rows instead
    with torch.no_grad():
        hx = core.rms_norm(x[:, :64], m.norm.w, m.norm.eps, out_dtype=torch.bfloat16)
        q_ref = core.linear(hx, m.wq.weight, as_matmul=True)
        si_ref, _, w_ref = core.address(q_ref, m.keys1, m.keys2, m.k, m.log_scale, padded=True)
        r_ref = core.table_read(si_ref, w_ref, m.values, m.k, out_dtype=torch.bfloat16)
        y_ref = core.linear(r_ref, m.wo.weight, as_matmul=True)
    assert torch.equal(m.last_q, q_ref)
    assert torch.equal(y_few, y_ref)
    assert y_all.shape == (1, 300, 768) and si_all.shape[0] == 300 and q_all.shape == (1, 300, 32)


@pytest.mark.parametrize("H,n_sub,d_a,k,rows,inplace", [(1, 64, 32, 16, 64, True),    # the FULL model's table layer
                                                        (1, 64, 32, 16, 1, True),
                                                        (1, 64, 32, 16, 256, False),
                                                        (1, 64, 32, 16, 7, True),     # an odd token count
                                                        (2, 32, 32, 8, 37, False),    # two heads: not in place
                                                        (3, 20, 64, 12, 5, False)])
def test_table_step_residual_equals_add_norm_then_table_step(H, n_sub, d_a, k, rows, inplace):
    """sdm_rt_table_step_residual (the residual add and TrainedSdm's input norm folded in front of the table step)
    gives, bit for bit, what sdm_rt_add_rms_norm and then sdm_rt_table_step give: the residual sum, the normed rows,
    the queries, the picks, scores and weights and the read; x is summed in place only when asked, with one head."""
    d = 768
    g = torch.Generator(device="cpu").manual_seed(7 * H + n_sub + d_a + k + rows)
    dh = d // H
    x = torch.randn(1, rows, d, generator=g).to(torch.bfloat16).cuda()
    y = (torch.randn(1, rows, d, generator=g) * 0.5).to(torch.bfloat16).cuda()
    nw = (1.0 + 0.2 * torch.randn(d, generator=g)).cuda()
    wq = (torch.randn(H * d_a, d, generator=g) * d ** -0.5).to(torch.bfloat16).cuda()
    keys1 = torch.randn(H, n_sub, d_a // 2, generator=g).cuda()
    keys2 = torch.randn(H, n_sub, d_a // 2, generator=g).cuda()
    log_scale = (torch.full((H,), 2.0) + torch.rand(H, generator=g) * 0.5).cuda()
    values = torch.randn(H, n_sub * n_sub, dh, generator=g).to(torch.bfloat16).cuda()
    say("table_step_residual", H, n_sub, d_a, k, rows, inplace)
    with torch.no_grad():
        x_ref = x.clone()
        s_ref, hx_ref = core.add_rms_norm(x_ref, y, nw, 1e-6, out_dtype=torch.bfloat16)
        r_ref, si_ref, sc_ref, w_ref, q_ref = core.table_step(hx_ref, wq, keys1, keys2, log_scale, values, k,
                                                              want_q=True)
        x_in = x.clone()
        s, r, si, sc, w, q, hx = core.table_step_residual(x_in, y, nw, 1e-6, wq, keys1, keys2, log_scale, values, k,
                                                          want_q=True, inplace=inplace, want_hx=True)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref) and torch.equal(hx, hx_ref) and torch.equal(q, q_ref)
    assert torch.equal(si, si_ref) and torch.equal(sc, sc_ref) and torch.equal(w, w_ref)
    assert torch.equal(r, r_ref)
    if inplace and H == 1:
        assert s.data_ptr() == x_in.data_ptr()
    else:
        assert torch.equal(x_in, x), "x changed although the sum was not asked in place"


def test_onesdm_decode_with_the_folded_add_equals_the_separate_add():
    """A OneSdmLM with TrainedSdm layers of width 768 decoding in bfloat16: the steps whose residual adds run inside
    the table step (TrainedSdm.forward_residual) and inside the mixers' projection maps (RunTimeSdm.step_residual),
    and whose embedding gather and first norm run inside the first mixer's map (RunTimeSdm.step_embed), give the same
    logits, bit for bit, as the steps with the separate gather, norm and add-and-norm kernels, with the folds in
    several combinations and with none."""
    from sdmchat_amd import OneSdmLM
    torch.manual_seed(11)
    m = OneSdmLM(512, d=768, layers=3, heads=4, n_sub=16, d_a=32, k=8, ffn="sdm", sdm_n_sub=32, sdm_heads=1,
                 sdm_k=16).cuda().to(torch.bfloat16).eval()
    with torch.no_grad():
        for sd in m.sdms:
            sd.values.normal_()
            sd.wo.weight.normal_(std=0.03)
        for mm in m.mems:
            mm.wo.weight.normal_(std=0.03)
    toks = torch.randint(0, 512, (6, 24), device="cuda")
    say("onesdm decode, folded adds against separate adds")
    calls = {"table": 0, "mixer": 0, "embed": 0}

    def counting(mod, key, name="residual_fits"):
        fits = getattr(type(mod), name)

        def f(a, b):
            ok = fits(mod, a, b)
            calls[key] += int(ok)
            return ok
        return f

    outs = []
    for table_fold, mixer_fold, embed_fold in ((True, True, True), (True, False, False), (False, True, True),
                                               (False, False, False), (False, False, True)):
        for sd in m.sdms:
            sd.residual_fits = counting(sd, "table") if table_fold else (lambda x, y: False)
        for mm in m.mems:
            mm.residual_fits = counting(mm, "mixer") if mixer_fold else (lambda x, y: False)
            mm.embed_fits = counting(mm, "embed", "embed_fits") if embed_fold else (lambda idx, table: False)
        st = m.decode_state(24)
        with torch.no_grad():
            outs.append(torch.stack([m.step(toks[t], st) for t in range(6)]))
    for mod in list(m.sdms) + list(m.mems):
        del mod.residual_fits
    for mm in m.mems:
        del mm.embed_fits
    assert calls["table"] > 0 and calls["mixer"] > 0 and calls["embed"] > 0, calls   # every fold ran
    for o in outs[1:]:
        assert torch.equal(outs[0], o)
    assert torch.isfinite(outs[0].float()).all()
