"""GPU tests of the prepared sub-key pieces (sdm_rt_prepare_key_pieces): the bfloat16 scoring with the pieces that
_params prepares gives the same picks, scores, weights and read-outs, bit for bit, as the scoring that derives them
itself (params.key_pieces NULL), for the addressing (32 and 64 sub-keys per half, with an address bias), the core
forward and the decode step."""
import pytest
import torch

from sdmchat_amd import _lib, core
from tests._gpu_util import core_inputs, say

pytestmark = pytest.mark.gpu


def _both(p, dev):
    """(params with prepared pieces, the same params without, and with pieces whose stated size is too small for the
    shape: not read)."""
    tp = {n: (torch.from_numpy(v).to(dev) if v is not None else None) for n, v in p.items()}
    with_p = core._params(dev, tp["keys1"], tp["keys2"], tp["addr_b"], tp["log_scale"], tp["decay"], tp["onorm_w"],
                          tp["gate_bias"])
    assert with_p[0].key_pieces and with_p[0].key_pieces_bytes > 0, "pieces prepared"
    prm = _lib.SdmRtParams(*[getattr(with_p[0], f) for f, _ in _lib.SdmRtParams._fields_[:-2]])
    short = _lib.SdmRtParams(*[getattr(with_p[0], f) for f, _ in _lib.SdmRtParams._fields_])
    short.key_pieces_bytes = with_p[0].key_pieces_bytes - 16
    return tp, with_p, (prm, with_p[1]), (short, with_p[1])


@pytest.mark.parametrize("n_sub,d_a", [(32, 64), (64, 32), (16, 32), (32, 16)])
def test_address_with_prepared_pieces_equals_derived(n_sub, d_a):
    dev = torch.device("cuda")
    H, k = 4, 8
    kz, qz, V, g, p = core_inputs(2, 96, H, 32, d_a, n_sub, seed=n_sub + d_a, addr_bias=0.3)
    tp, with_p, without, short = _both(p, dev)
    z = torch.from_numpy(kz).to(dev).to(torch.bfloat16)
    gl = torch.from_numpy(g).to(dev).to(torch.bfloat16)
    say("key pieces: address", n_sub, d_a)
    outs = []
    for prm in (with_p, without, short):
        with torch.no_grad():
            outs.append(core.address(z, tp["keys1"], tp["keys2"], k, tp["log_scale"], addr_b=tp["addr_b"],
                                     gate_logits=gl, gate_bias=tp["gate_bias"], params=prm))
        torch.cuda.synchronize()
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)


def test_core_forward_and_decode_with_prepared_pieces_equal_derived():
    dev = torch.device("cuda")
    B, T, H, dh, d_a, n_sub, k = 2, 256, 4, 64, 64, 32, 8
    kz, qz, V, g, p = core_inputs(B, T, H, dh, d_a, n_sub, seed=5, addr_bias=0.2)
    tp, with_p, without, _ = _both(p, dev)
    t = [torch.from_numpy(a).to(dev).to(torch.bfloat16) for a in (kz, qz, V, g)]
    kw = dict(keys1=tp["keys1"], keys2=tp["keys2"], log_scale=tp["log_scale"], decay=tp["decay"],
              addr_b=tp["addr_b"], onorm_w=tp["onorm_w"], gate_bias=tp["gate_bias"], k=k)
    say("key pieces: core forward and decode")
    outs, steps = [], []
    for prm in (with_p, without):
        with torch.no_grad():
            outs.append(core.core_forward(*t, params=prm, **kw))
            st = core.DecodeState.empty(B, H, n_sub * n_sub, dh, dev, core.pick_pitch(k, n_sub))
            steps.append(torch.stack([core.decode_step(t[0][:, i], t[1][:, i], t[2][:, i], t[3][:, i], st,
                                                       params=prm, out_dtype=torch.bfloat16, **kw)
                                      for i in range(8)]))
        torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(steps[0], steps[1])
