"""The C-ABI library loads and exports every function include/sdm_rt.h declares; argument validation runs on the host
before anything is launched, so it is checked here without a GPU."""
import ctypes
import os
import re

import pytest

from sdmchat_amd import _lib, core

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(sdm_rt_\w+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "build the library first (python -m sdmchat_amd.build)"
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = declared_functions()
    assert {"sdm_rt_forward", "sdm_rt_address", "sdm_rt_workspace_bytes", "sdm_rt_last_error"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def _dims(**over):
    d = dict(B=8, T=2048, heads=12, head_dim=64, addr_dim=64, n_sub=32, k=8)
    d.update(over)
    return core.make_dims(d["B"], d["T"], d["heads"], d["head_dim"], d["addr_dim"], d["n_sub"], d["k"])


def test_workspace_and_pitch():
    lib = _lib.load()
    dims = _dims()
    ws = lib.sdm_rt_workspace_bytes(ctypes.byref(dims))
    plans = 8 * 12 * (2048 // 64)               # one plan per 64 positions of one head of one batch row
    assert ws >= plans * 64 * (8 * 6 + 8 * 8) + 8 * 2048 * 12 * 64 * 4   # picks and write records, fp32 read-out
    assert ws < plans * 32768 + 8 * 2048 * 12 * 64 * 4 + (1 << 20)
    assert lib.sdm_rt_pick_pitch(ctypes.byref(dims)) == 8
    assert lib.sdm_rt_pick_pitch(ctypes.byref(_dims(k=16, addr_dim=32))) == 16
    assert lib.sdm_rt_pick_pitch(ctypes.byref(_dims(k=5, n_sub=6))) == 8


@pytest.mark.parametrize("over,msg", [
    (dict(head_dim=12), "head_dim"),
    (dict(addr_dim=7), "addr_dim"),
    (dict(k=0), "top_k"),
    (dict(k=32, n_sub=32), "<= 16"),
    (dict(n_sub=300), "65535"),
    (dict(heads=0), "heads"),
])
def test_invalid_dims_are_rejected_before_launch(over, msg):
    lib = _lib.load()
    dims = _dims(**over)
    assert lib.sdm_rt_workspace_bytes(ctypes.byref(dims)) == 0
    prm = _lib.SdmRtParams()
    one = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), one, 4096, one, 4096, one, 4096, None, 0, 0, None, one, 4096, 0,
                            None, None, None, None, one, 1 << 30, None)
    assert rc != 0
    assert msg in lib.sdm_rt_last_error().decode()


def test_missing_pointers_and_small_workspace_are_rejected():
    lib = _lib.load()
    dims = _dims()
    prm = _lib.SdmRtParams()
    one = ctypes.c_void_p(16)
    rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), one, 4096, one, 4096, one, 4096, one, 4096, 0, None, one, 4096, 0,
                            None, None, None, None, one, 1 << 30, None)
    assert rc == -1 and "keys1" in lib.sdm_rt_last_error().decode()
    prm = _lib.SdmRtParams(one, one, None, one, one, one, None)
    rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), one, 4096, one, 4096, one, 4096, one, 4096, 0, None, one, 4096, 0,
                            None, None, None, None, one, 1024, None)
    assert rc == -2 and "workspace" in lib.sdm_rt_last_error().decode()
    rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), one, 4096, one, 4096, one, 4096, None, 0, 0, None, one, 4096, 0,
                            None, None, None, None, one, 1 << 30, None)
    assert rc == -1 and "gate_logits" in lib.sdm_rt_last_error().decode()
    rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), one, 4096, one, 4096, one, 4096, one, 4096, 7, None, one, 4096, 0,
                            None, None, None, None, one, 1 << 30, None)
    assert rc == -1 and "dtype" in lib.sdm_rt_last_error().decode()


def test_rms_norm_validation():
    lib = _lib.load()
    one = ctypes.c_void_p(16)
    assert lib.sdm_rt_rms_norm(one, 12, 1, 4, 12, one, 1e-6, one, 12, 1, None) == -3   # d not a multiple of 8
    assert "multiple of 8" in lib.sdm_rt_last_error().decode()
    assert lib.sdm_rt_rms_norm(one, 8, 1, 4, 16, one, 1e-6, one, 16, 1, None) == -1    # row stride < d
    assert lib.sdm_rt_rms_norm(one, 16, 5, 4, 16, one, 1e-6, one, 16, 1, None) == -1   # unknown dtype
    assert lib.sdm_rt_rms_norm(None, 16, 1, 0, 16, None, 1e-6, None, 16, 1, None) == 0  # no rows: nothing to do


def test_decode_step_validation():
    """sdm_rt_decode_step checks its arguments on the host: one token per stream, a state, enough workspace."""
    lib = _lib.load()
    dims = _dims(B=4, T=1)
    need = lib.sdm_rt_decode_workspace_bytes(ctypes.byref(dims))
    assert 0 < need < (1 << 20)
    assert lib.sdm_rt_decode_workspace_bytes(ctypes.byref(_dims(k=0))) == 0
    prm = _lib.SdmRtParams(*([ctypes.c_void_p(256)] * 7))
    fake = ctypes.c_void_p(256)
    I, F = _lib.SDM_RT_F32, _lib.SDM_RT_F32

    def call(d, state=fake, ws_bytes=need):
        return lib.sdm_rt_decode_step(ctypes.byref(d), ctypes.byref(prm), fake, 768, fake, 768, fake, 768, fake, 12,
                                      I, None, state, state, state, None, fake, 768, F, fake, ws_bytes, None)
    assert call(_dims(B=4, T=2)) == -1 and b"seq_len must be 1" in lib.sdm_rt_last_error()
    assert call(dims, state=None) == -1 and b"state" in lib.sdm_rt_last_error()
    assert call(dims, ws_bytes=need - 1) == -2 and b"workspace" in lib.sdm_rt_last_error()
    assert call(_dims(B=0, T=1)) == 0


def test_forward_noalloc_rejects_calls_beyond_its_scratch():
    """sdm_rt_forward_noalloc runs on a fixed 128 MiB scratch; a call whose workspace is larger fails on the host,
    before any device call."""
    lib = _lib.load()
    cap = lib.sdm_rt_noalloc_scratch_bytes()
    assert cap == 128 << 20
    big = _dims(B=32, T=2048)
    assert lib.sdm_rt_workspace_bytes(ctypes.byref(big)) > cap
    prm = _lib.SdmRtParams(*([ctypes.c_void_p(256)] * 7))
    fake = ctypes.c_void_p(256)
    F = _lib.SDM_RT_F32
    rc = lib.sdm_rt_forward_noalloc(ctypes.byref(big), ctypes.byref(prm), fake, 768, fake, 768, fake, 768, fake, 12,
                                    F, None, fake, 768, F, None, None, None, None, None)
    assert rc == -2 and b"scratch" in lib.sdm_rt_last_error()


def test_backward_validation():
    """sdm_rt_forward_train / sdm_rt_backward check their arguments on the host before any launch."""
    lib = _lib.load()
    dims = _dims(B=2, T=100)
    need = lib.sdm_rt_backward_workspace_bytes(ctypes.byref(dims))
    # dnum (N x H*dh float32) and the per-pick partial dots of both scans are the bulk of it
    N = 2 * 100
    assert need >= 4 * N * 12 * 64 + 2 * 4 * 2 * N * 12 * 8
    assert lib.sdm_rt_backward_workspace_bytes(ctypes.byref(_dims(addr_dim=130))) == 0   # d_a > 64
    prm = _lib.SdmRtParams(*([ctypes.c_void_p(256)] * 7))
    fake = ctypes.c_void_p(256)
    saved = _lib.SdmRtSaved(*([fake] * 8))
    grads = _lib.SdmRtGrads(fake, 768, fake, 768, fake, 768, fake, 12, *([None] * 7))
    F = _lib.SDM_RT_F32

    def bwd(d=dims, sv=saved, gr=grads, ws=need, dy_stride=768):
        return lib.sdm_rt_backward(ctypes.byref(d), ctypes.byref(prm), fake, 768, fake, 768, fake, 768, fake, 12, F,
                                   None, ctypes.byref(sv) if sv is not None else None, fake, dy_stride, F,
                                   ctypes.byref(gr) if gr is not None else None, fake, ws, None)
    assert bwd(sv=None) == -1 and b"saved" in lib.sdm_rt_last_error()
    assert bwd(gr=None) == -1 and b"grads" in lib.sdm_rt_last_error()
    assert bwd(ws=need - 1) == -2 and b"workspace" in lib.sdm_rt_last_error()
    assert bwd(dy_stride=700) == -1 and b"stride" in lib.sdm_rt_last_error()
    no_gl = _lib.SdmRtGrads(fake, 768, fake, 768, fake, 768, None, 0, *([None] * 7))
    assert bwd(gr=no_gl) == -1 and b"d_gate_logits" in lib.sdm_rt_last_error()
    assert bwd(d=_dims(B=0, T=100)) == 0
    rc = lib.sdm_rt_forward_train(ctypes.byref(dims), ctypes.byref(prm), fake, 768, fake, 768, fake, 768, fake, 12,
                                  F, None, fake, 768, F, None, fake, 1 << 30, None)
    assert rc == -1 and b"saved" in lib.sdm_rt_last_error()


def test_table_step_residual_arguments_are_checked_before_launch():
    """The folded table step takes the layer width 768 only, and sums in place only with one head."""
    lib = _lib.load()
    one = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    prm = _lib.SdmRtParams(one, one, None, one, None, None, None)

    def call(dims, d, sum_out):
        return lib.sdm_rt_table_step_residual(ctypes.byref(dims), ctypes.byref(prm), one, d, ctypes.c_void_p(32), d,
                                              one, 1e-6, sum_out, d, None, 0, d, one, d, one, None, 0, one, None,
                                              None, one, 4096, None)
    dims1 = core.make_dims(1, 64, 1, 768, 32, 64, 16, out_norm=False, write_gate=False)
    assert call(dims1, 512, one) != 0 and "768" in lib.sdm_rt_last_error().decode()
    dims2 = core.make_dims(1, 64, 2, 384, 32, 32, 8, out_norm=False, write_gate=False)
    assert call(dims2, 768, one) != 0 and "one head" in lib.sdm_rt_last_error().decode()
    assert call(dims1, 768, ctypes.c_void_p(32)) != 0 and "alias y" in lib.sdm_rt_last_error().decode()


def test_gemm_rows_residual_arguments_are_checked_before_launch():
    """The folded projection map takes k = 768, at most 256 tiles of 64 x 32, and no aliasing of its outputs with
    x, y or each other."""
    lib = _lib.load()
    x, y, nw, s, w, o = (ctypes.c_void_p(16 * i) for i in range(1, 7))   # never dereferenced: validation fails first

    def call(rows, n, k, s_out=s, out=o):
        return lib.sdm_rt_gemm_rows_residual(x, k, y, k, nw, 1e-6, s_out, k, w, k, None, out, n, rows, n, k, None)
    assert call(64, 2560, 512) != 0 and "768" in lib.sdm_rt_last_error().decode()
    assert call(64, 100, 768) != 0 and "multiple of 32" in lib.sdm_rt_last_error().decode()
    assert call(193, 2560, 768) != 0 and "256 tiles" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, s_out=x) != 0 and "alias" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, out=y) != 0 and "alias" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, out=s) != 0 and "alias" in lib.sdm_rt_last_error().decode()
    assert call(0, 2560, 768) == 0   # no rows: nothing to do


def test_gemm_rows_embed_arguments_are_checked_before_launch():
    """The folded embedding map takes k = 768, n a multiple of 32, at most 256 tiles of 64 x 32, a vocabulary of at
    least one row and no aliasing of its outputs with the table or each other."""
    lib = _lib.load()
    idx, t, nw, xo, w, o = (ctypes.c_void_p(16 * i) for i in range(1, 7))   # never dereferenced

    def call(rows, n, k, vocab=100, x_out=xo, out=o):
        return lib.sdm_rt_gemm_rows_embed(idx, t, k, vocab, nw, 1e-6, x_out, k, w, k, None, out, n, rows, n, k, None)
    assert call(64, 2560, 512) != 0 and "768" in lib.sdm_rt_last_error().decode()
    assert call(64, 100, 768) != 0 and "multiple of 32" in lib.sdm_rt_last_error().decode()
    assert call(193, 2560, 768) != 0 and "256 tiles" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, vocab=0) != 0 and "vocab" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, x_out=t) != 0 and "alias" in lib.sdm_rt_last_error().decode()
    assert call(64, 2560, 768, out=xo) != 0 and "alias" in lib.sdm_rt_last_error().decode()
    assert call(0, 2560, 768) == 0   # no rows: nothing to do


def test_prepare_key_pieces_checks_its_buffer():
    """The prepared sub-key pieces: their size for a shape, none for a shape without matrix-core scoring, and a
    buffer too small refused before launch."""
    lib = _lib.load()
    dims = core.make_dims(1, 1, 4, 8, 64, 32, 1)
    need = lib.sdm_rt_key_pieces_bytes(ctypes.byref(dims))
    assert need == 4 * (4 * 2 * 32 * 2 * 24 + 4 * 2 * 32)
    one = ctypes.c_void_p(16)
    prm = _lib.SdmRtParams(one, one, None, one, None, None, None)
    assert lib.sdm_rt_prepare_key_pieces(ctypes.byref(dims), ctypes.byref(prm), one, need - 16, None) != 0
    assert "needed" in lib.sdm_rt_last_error().decode()
    wide = core.make_dims(1, 1, 4, 8, 64, 128, 1)   # 128 sub-keys per half: no matrix-core scoring
    assert lib.sdm_rt_key_pieces_bytes(ctypes.byref(wide)) == 0
