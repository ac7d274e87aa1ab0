"""ctypes binding of ``libsdm_rt.so`` (the C ABI declared in include/sdm_rt.h).

The library is loaded from ``sdmchat_amd/lib/libsdm_rt.so`` (built by ``python -m sdmchat_amd.build``).  There is no
fallback: if the library is missing or a symbol is absent, loading raises.
"""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libsdm_rt.so")

SDM_RT_F32 = 0
SDM_RT_BF16 = 1

# every function the header declares, with its ctypes signature
c_void_p = ctypes.c_void_p
c_i64 = ctypes.c_int64


class SdmRtDims(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("addr_dim", ctypes.c_int32),
        ("n_sub", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("read_mean", ctypes.c_int32),
        ("out_norm", ctypes.c_int32),
        ("write_gate", ctypes.c_int32),
        ("read_eps", ctypes.c_float),
        ("out_norm_eps", ctypes.c_float),
    ]


class SdmRtParams(ctypes.Structure):
    _fields_ = [
        ("keys1", c_void_p),
        ("keys2", c_void_p),
        ("addr_b", c_void_p),
        ("log_scale", c_void_p),
        ("decay", c_void_p),
        ("onorm_w", c_void_p),
        ("gate_bias", c_void_p),
        ("key_pieces", c_void_p),
        ("key_pieces_bytes", ctypes.c_size_t),
    ]


class SdmRtSaved(ctypes.Structure):
    _fields_ = [
        ("slots_w", c_void_p),
        ("weights_w", c_void_p),
        ("scores_w", c_void_p),
        ("slots_r", c_void_p),
        ("weights_r", c_void_p),
        ("scores_r", c_void_p),
        ("read", c_void_p),
        ("den", c_void_p),
    ]


class SdmRtGrads(ctypes.Structure):
    _fields_ = [
        ("d_kz", c_void_p),
        ("d_kz_row_stride", c_i64),
        ("d_qz", c_void_p),
        ("d_qz_row_stride", c_i64),
        ("d_v", c_void_p),
        ("d_v_row_stride", c_i64),
        ("d_gate_logits", c_void_p),
        ("d_gate_row_stride", c_i64),
        ("d_keys1", c_void_p),
        ("d_keys2", c_void_p),
        ("d_addr_b", c_void_p),
        ("d_log_scale", c_void_p),
        ("d_onorm_w", c_void_p),
        ("d_gate_bias", c_void_p),
        ("d_log_decay", c_void_p),
    ]


SIGNATURES = {
    "sdm_rt_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_pick_pitch": (ctypes.c_int32, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_address": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                      c_void_p, c_i64, c_void_p, c_i64, ctypes.c_int,
                                      c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_forward": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                      c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                      ctypes.c_int, c_void_p,
                                      c_void_p, c_i64, ctypes.c_int,
                                      c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "sdm_rt_forward_noalloc": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                              c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                              ctypes.c_int, c_void_p,
                                              c_void_p, c_i64, ctypes.c_int,
                                              c_void_p, c_void_p, c_void_p, c_void_p,
                                              c_void_p]),
    "sdm_rt_decode_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_decode_step": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                          c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                          ctypes.c_int, c_void_p,
                                          c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_i64, ctypes.c_int,
                                          c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_table_read": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), c_void_p, c_void_p, c_void_p, ctypes.c_int,
                                         c_void_p, c_i64, ctypes.c_int, c_void_p]),
    "sdm_rt_gate_copy_offset": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_table_step": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams), c_void_p, c_i64,
                                         ctypes.c_int32, c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_i64, c_void_p]),
    "sdm_rt_table_step_residual": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams), c_void_p,
                                                  c_i64, c_void_p, c_i64, c_void_p, ctypes.c_float, c_void_p, c_i64,
                                                  c_void_p, c_i64, ctypes.c_int32, c_void_p, c_i64, c_void_p,
                                                  c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_i64,
                                                  c_void_p]),
    "sdm_rt_rms_norm": (ctypes.c_int, [c_void_p, c_i64, ctypes.c_int, c_i64, ctypes.c_int32, c_void_p,
                                       ctypes.c_float, c_void_p, c_i64, ctypes.c_int, c_void_p]),
    "sdm_rt_add_rms_norm": (ctypes.c_int, [c_void_p, c_i64, c_void_p, c_i64, ctypes.c_int, c_i64, ctypes.c_int32,
                                           c_void_p, ctypes.c_float, c_void_p, c_i64, c_void_p, c_i64, ctypes.c_int,
                                           c_void_p]),
    "sdm_rt_silu_mul": (ctypes.c_int, [c_void_p, c_i64, ctypes.c_int, c_i64, ctypes.c_int32, c_void_p, c_i64,
                                       c_void_p]),
    "sdm_rt_key_pieces_bytes": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_prepare_key_pieces": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams), c_void_p,
                                                 ctypes.c_size_t, c_void_p]),
    "sdm_rt_gemm_rows": (ctypes.c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_i64,
                                        ctypes.c_int32, ctypes.c_int32, c_void_p]),
    "sdm_rt_gemm_rows_residual": (ctypes.c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, ctypes.c_float,
                                                 c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_i64,
                                                 ctypes.c_int32, ctypes.c_int32, c_void_p]),
    "sdm_rt_gemm_rows_embed": (ctypes.c_int, [c_void_p, c_void_p, c_i64, c_i64, c_void_p, ctypes.c_float, c_void_p,
                                              c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_i64, ctypes.c_int32,
                                              ctypes.c_int32, c_void_p]),
    "sdm_rt_forward_train": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                            c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                            ctypes.c_int, c_void_p,
                                            c_void_p, c_i64, ctypes.c_int,
                                            ctypes.POINTER(SdmRtSaved), c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_backward_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_backward": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                       c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                       ctypes.c_int, c_void_p, ctypes.POINTER(SdmRtSaved),
                                       c_void_p, c_i64, ctypes.c_int,
                                       ctypes.POINTER(SdmRtGrads), c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_table_backward_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SdmRtDims)]),
    "sdm_rt_table_backward": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), ctypes.POINTER(SdmRtParams),
                                             c_void_p, c_i64, ctypes.c_int,
                                             c_void_p, c_void_p, c_void_p,
                                             c_void_p, ctypes.c_int,
                                             c_void_p, c_i64, ctypes.c_int,
                                             c_void_p, c_i64, c_void_p,
                                             c_void_p, c_void_p, c_void_p,
                                             c_void_p, ctypes.c_size_t, c_void_p]),
    "sdm_rt_status": (ctypes.c_int, [ctypes.POINTER(SdmRtDims), c_void_p, c_void_p]),
    "sdm_rt_set_wait_limit": (None, [c_i64]),
    "sdm_rt_set_crowded_threshold": (None, [ctypes.c_int32]),
    "sdm_rt_last_error": (ctypes.c_char_p, []),
}

SDM_RT_ETIMEOUT = -5

_LIB = None


def load(path=None):
    """Load (once) and return the library with every declared signature set."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"run-time SDM HIP library not built: {p} is missing (python -m sdmchat_amd.build)")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


class SdmRtError(RuntimeError):
    pass


def check(rc, lib=None):
    if rc != 0:
        lib = lib or load()
        raise SdmRtError(f"sdm_rt status {rc}: {lib.sdm_rt_last_error().decode()}")
