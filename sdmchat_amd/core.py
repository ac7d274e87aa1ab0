"""torch-facing wrappers of the C ABI: the SDM core on device tensors.

Tensors must live on a ROCm device.  Activations are [B, T, width] with unit stride in the last dimension and a
uniform row stride (a slice of a wider fused projection output is fine).  All work is queued on the current torch
stream; nothing synchronises.
"""
import ctypes

import torch
from torch.utils.weak import WeakIdKeyDictionary

from . import _lib

_DT = {torch.float32: _lib.SDM_RT_F32, torch.bfloat16: _lib.SDM_RT_BF16}


def make_dims(B, T, heads, head_dim, addr_dim, n_sub, k, read_mode="mean", out_norm=True, write_gate=True,
              read_eps=1e-3, out_norm_eps=1e-2):
    return _lib.SdmRtDims(int(B), int(T), int(heads), int(head_dim), int(addr_dim), int(n_sub), int(k),
                          1 if read_mode == "mean" else 0, 1 if out_norm else 0, 1 if write_gate else 0,
                          float(read_eps), float(out_norm_eps))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _rows16(t2):
    """A 2-D view whose rows are contiguous and all start 16-byte aligned."""
    es = t2.element_size()
    return t2.stride(1) == 1 and t2.data_ptr() % 16 == 0 and (t2.stride(0) * es) % 16 == 0


def _f32(t, device):
    if t is None:
        return None
    return t.detach().to(device=device, dtype=torch.float32).contiguous()


def _rows(x, name, B, T, width):
    """Row stride (elements) of a [B, T, >=width] activation whose B*T rows are uniformly strided."""
    if x.dim() != 3 or x.shape[0] != B or x.shape[1] != T or x.shape[2] < width:
        raise ValueError(f"{name}: expected [B={B}, T={T}, >={width}], got {tuple(x.shape)}")
    if x.dtype not in _DT:
        raise ValueError(f"{name}: dtype {x.dtype} is not float32 or bfloat16")
    if x.numel() == 0:
        return width
    if x.stride(2) != 1:
        raise ValueError(f"{name}: last dimension must have unit stride")
    if B > 1 and T > 0 and x.stride(0) != T * x.stride(1):
        raise ValueError(f"{name}: rows must be uniformly strided (stride(0) == T * stride(1))")
    return x.stride(1)


def _rows2(x, name, B, width):
    """Row stride (elements) of a [B, >=width] activation with unit stride in the last dimension."""
    if x.dim() != 2 or x.shape[0] != B or x.shape[1] < width:
        raise ValueError(f"{name}: expected [B={B}, >={width}], got {tuple(x.shape)}")
    if x.dtype not in _DT:
        raise ValueError(f"{name}: dtype {x.dtype} is not float32 or bfloat16")
    if x.numel() and x.stride(1) != 1:
        raise ValueError(f"{name}: last dimension must have unit stride")
    return x.stride(0) if B > 1 else max(x.shape[1], width)


def _params(device, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias):
    """The SdmRtParams of these parameters (float32, contiguous copies where needed) with the sub-key pieces of the
    bfloat16 scoring prepared from them (sdm_rt_prepare_key_pieces, one launch).  Returns (params, held tensors);
    build them again after a parameter changes (ParamCache does)."""
    held = [_f32(t, device) for t in (keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias)]
    prm = _lib.SdmRtParams(*[_ptr(t) for t in held])
    H, n_sub, half = held[0].shape
    dims = make_dims(1, 1, H, 8, 2 * half, n_sub, 1)
    lib = _lib.load()
    nbytes = lib.sdm_rt_key_pieces_bytes(ctypes.byref(dims))
    if nbytes:
        pieces = torch.empty(nbytes, dtype=torch.uint8, device=held[0].device)
        stream = torch.cuda.current_stream(pieces.device).cuda_stream
        _lib.check(lib.sdm_rt_prepare_key_pieces(ctypes.byref(dims), ctypes.byref(prm), _ptr(pieces), nbytes,
                                                 ctypes.c_void_p(stream)), lib)
        prm.key_pieces = _ptr(pieces)
        prm.key_pieces_bytes = nbytes
        held.append(pieces)
    return prm, held


class ParamCache:
    """The float32, contiguous copies of a module's core parameters and their SdmRtParams, rebuilt only when one of
    the source tensors changes (data pointer or version)."""

    def __init__(self):
        self.key = None
        self.value = None

    def get(self, device, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias, decay_source=None):
        """decay may be a callable computing it; decay_source is then the tensor it derives from (the cache key)."""
        srcs = (keys1, keys2, addr_b, log_scale, decay_source if callable(decay) else decay, onorm_w, gate_bias)
        key = (device,) + tuple(None if t is None else (t.data_ptr(), t._version, t.dtype) for t in srcs)
        if self.key != key:
            dec = decay() if callable(decay) else decay
            self.value = _params(device, keys1, keys2, addr_b, log_scale, dec, onorm_w, gate_bias)
            self.key = key
        return self.value


def workspace_bytes(dims):
    return _lib.load().sdm_rt_workspace_bytes(ctypes.byref(dims))


def address(z, keys1, keys2, k, log_scale, addr_b=None, gate_logits=None, gate_bias=None, padded=False,
            params=None):
    """Product-key addressing of one address set (pk_address + softmax weights [+ gate]).

    z [B, T, H * d_a]; keys [H, n_sub, d_a/2].  Returns slots int32, scores and weights float32, each
    [B, H, T, kk] (descending score order, ties to the lower index)."""
    lib = _lib.load()
    B, T = z.shape[0], z.shape[1]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dims = make_dims(B, T, H, 8, d_a, n_sub, k, out_norm=False, write_gate=gate_logits is not None)
    zs = _rows(z, "z", B, T, H * d_a)
    gs = 0
    if gate_logits is not None:
        if gate_logits.dtype != z.dtype:
            raise ValueError("gate_logits must have the dtype of z")
        gs = _rows(gate_logits, "gate_logits", B, T, H)
    dev = z.device
    if params is None:   # the addressing reads no fade
        params = _params(dev, keys1, keys2, addr_b, log_scale, None, None, gate_bias)
    prm, held = params
    pitch = lib.sdm_rt_pick_pitch(ctypes.byref(dims))
    if pitch <= 0:
        raise _lib.SdmRtError(lib.sdm_rt_last_error().decode() or "invalid dimensions")
    kk = min(k, min(k, n_sub) ** 2)
    slots = torch.empty(B, H, T, pitch, dtype=torch.int32, device=dev)
    scores = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    weights = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_address(ctypes.byref(dims), ctypes.byref(prm), _ptr(z), zs, _ptr(gate_logits), gs, _DT[z.dtype],
                            _ptr(slots), _ptr(scores), _ptr(weights), None, 0, ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    del held
    if padded:   # the kernel's own [B, H, T, pitch] arrays (pads: slot -1, weight 0)
        return slots, scores, weights
    return slots[..., :kk], scores[..., :kk], weights[..., :kk]


def gate_copy(workspace, B, T, H, dh, d_a, n_sub, k, dtype, read_mode="mean", out_norm=True, read_eps=1e-3,
              out_norm_eps=1e-2):
    """The gate logits that the last core_forward on ``workspace`` read, [B, T, H] in ``dtype`` (the projections'
    dtype): a view of the copy sdm_rt_forward leaves in its workspace (sdm_rt_gate_copy_offset), valid until the
    workspace is next used.  The dimensions must be those of that call."""
    lib = _lib.load()
    dims = make_dims(B, T, H, dh, d_a, n_sub, k, read_mode, out_norm, True, read_eps, out_norm_eps)
    off = lib.sdm_rt_gate_copy_offset(ctypes.byref(dims))
    n = B * T * H * torch.empty(0, dtype=dtype).element_size()
    buf = workspace.buf
    if off == 0 or buf is None or buf.numel() < off + n:
        raise RuntimeError("gate_copy: the workspace holds no gate copy for these dimensions")
    return buf[off:off + n].view(dtype).view(B, T, H)


class CoreWorkspace:
    """A reusable device workspace (grows on demand)."""

    def __init__(self):
        self.buf = None

    def get(self, nbytes, device):
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        return self.buf


def core_forward(kz, qz, v, gate_logits, *, keys1, keys2, log_scale, decay, addr_b=None, onorm_w=None,
                 gate_bias=None, k, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2,
                 out_dtype=None, out=None, state_in=None, want_state=False, workspace=None, params=None, reset=None,
                 no_alloc=False, check=False):
    """The SDM core between the projections and the output map (RunTimeSdm.forward minus wk/wq/wv/wg and wo).

    kz, qz [B, T, H * d_a]; v [B, T, H * dh]; gate_logits [B, T, H] or None (no write gate); all share one dtype,
    each with its own uniform row stride.  Returns r [B, T, H * dh] (out_dtype, default v's dtype) and, when want_state, the final
    (mem [B, H, M, dh], cnt [B, H, M]) float32 state.  ``params`` may carry a prepared (SdmRtParams, held) pair.
    reset [B, T] bool or None: where set, the memory is emptied before that position reads (forward(x, reset),
    track4_onesdm_models.py:229-233).  no_alloc: run on the library's fixed scratch (sdm_rt_forward_noalloc) instead
    of a workspace.  check: synchronise the stream afterwards and raise SdmRtError if one of the scan's bounded
    waits gave up (sdm_rt_status: the read-outs of that chunk are NaN)."""
    lib = _lib.load()
    B, T = v.shape[0], v.shape[1]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    width = v.shape[2]
    dh = width // H
    dims = make_dims(B, T, H, dh, d_a, n_sub, k, read_mode, out_norm, gate_logits is not None, read_eps, out_norm_eps)
    dt = v.dtype
    for name, x in (("kz", kz), ("qz", qz), ("gate_logits", gate_logits)):
        if x is not None and x.dtype != dt:
            raise ValueError(f"{name} has dtype {x.dtype}, expected {dt}")
    vs = _rows(v, "v", B, T, H * dh)
    ks = _rows(kz, "kz", B, T, H * d_a)
    qs = _rows(qz, "qz", B, T, H * d_a)
    gs = 0 if gate_logits is None else _rows(gate_logits, "gate_logits", B, T, H)
    dev = v.device
    if params is None:
        params = _params(dev, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias)
    prm = params[0]
    out_dtype = out_dtype or dt
    if out is None:
        out = torch.empty(B, T, H * dh, dtype=out_dtype, device=dev)
    ostride = _rows(out, "out", B, T, H * dh)
    M = n_sub * n_sub
    mem_in = cnt_in = mem_out = cnt_out = None
    if state_in is not None:
        mem_in = state_in[0].to(device=dev, dtype=torch.float32).contiguous()
        cnt_in = state_in[1].to(device=dev, dtype=torch.float32).contiguous()
        if tuple(mem_in.shape) != (B, H, M, dh) or tuple(cnt_in.shape) != (B, H, M):
            raise ValueError("state_in must be (mem [B, H, M, dh], cnt [B, H, M])")
    if want_state:
        mem_out = torch.empty(B, H, M, dh, dtype=torch.float32, device=dev)
        cnt_out = torch.empty(B, H, M, dtype=torch.float32, device=dev)
    rs = None
    if reset is not None:
        if tuple(reset.shape) != (B, T):
            raise ValueError(f"reset must be [B={B}, T={T}]")
        rs = reset.to(device=dev, dtype=torch.uint8).contiguous()
    stream = torch.cuda.current_stream(dev).cuda_stream
    if no_alloc:
        rc = lib.sdm_rt_forward_noalloc(ctypes.byref(dims), ctypes.byref(prm), _ptr(kz), ks, _ptr(qz), qs, _ptr(v),
                                        vs, _ptr(gate_logits), gs, _DT[dt], _ptr(rs), _ptr(out), ostride,
                                        _DT[out_dtype], _ptr(mem_in), _ptr(cnt_in), _ptr(mem_out), _ptr(cnt_out),
                                        ctypes.c_void_p(stream))
    else:
        nbytes = lib.sdm_rt_workspace_bytes(ctypes.byref(dims))  # 0 for invalid dims: the call below reports why
        ws = (workspace or CoreWorkspace()).get(nbytes, dev)
        rc = lib.sdm_rt_forward(ctypes.byref(dims), ctypes.byref(prm), _ptr(kz), ks, _ptr(qz), qs, _ptr(v), vs,
                                _ptr(gate_logits), gs, _DT[dt], _ptr(rs), _ptr(out), ostride, _DT[out_dtype],
                                _ptr(mem_in), _ptr(cnt_in), _ptr(mem_out), _ptr(cnt_out), _ptr(ws), ws.numel(),
                                ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    if check:
        rc = lib.sdm_rt_status(ctypes.byref(dims), None if no_alloc else _ptr(ws), ctypes.c_void_p(stream))
        _lib.check(rc, lib)
    if want_state:
        return out, (mem_out, cnt_out)
    return out


def set_wait_limit(polls):
    """Polls a forward's wait for the other column groups of a slab makes before it gives up, process-wide
    (sdm_rt_set_wait_limit): None or a negative value restores the default, 0 makes every wait give up at once (for
    tests of the error path)."""
    _lib.load().sdm_rt_set_wait_limit(-1 if polls is None else int(polls))


def set_crowded_threshold(nbytes):
    """The plan size above which the forward's pick scan treats a slab as crowded and sums its owners' writes before
    the read barrier, process-wide (sdm_rt_set_crowded_threshold): None or a negative value restores the default
    (4,096 bytes); the results are the same bits either way."""
    _lib.load().sdm_rt_set_crowded_threshold(-1 if nbytes is None else int(nbytes))


def table_read(slots, weights, values, k, out_dtype=torch.float32, out=None):
    """The weighted read of picked table rows (TrainedSdm.forward's embedding_bag, track4_onesdm_models.py:448-455).

    slots, weights [B, H, T, pitch] as address() returns them (the first kk entries are the picks); values
    [H, M, dh] float32 or bfloat16 (M = n_sub^2).  Returns out [B, T, H * dh] in out_dtype: the float32 sum over
    the picks of weight * row."""
    lib = _lib.load()
    B, H, T, pitch = slots.shape
    Hv, M, dh = values.shape
    n_sub = int(round(M ** 0.5))
    if Hv != H or n_sub * n_sub != M:
        raise ValueError(f"values must be [H={H}, n_sub^2, dh], got {tuple(values.shape)}")
    if slots.dtype != torch.int32 or weights.dtype != torch.float32 or tuple(weights.shape) != tuple(slots.shape):
        raise ValueError("slots must be int32 and weights float32, both [B, H, T, pitch]")
    if values.dtype not in _DT:
        raise ValueError(f"values: dtype {values.dtype} is not float32 or bfloat16")
    dims = make_dims(B, T, H, dh, 2, n_sub, k, out_norm=False, write_gate=False)
    want = lib.sdm_rt_pick_pitch(ctypes.byref(dims))
    kk = min(k, min(k, n_sub) ** 2)
    if pitch < kk or want <= 0:
        raise ValueError(f"slots hold {pitch} picks per (token, head); k={k}, n_sub={n_sub} needs {kk}")
    if pitch != want:   # repack into the kernel's pitch (pads: slot -1, weight 0)
        ps = torch.full((B, H, T, want), -1, dtype=torch.int32, device=slots.device)
        pw = torch.zeros((B, H, T, want), dtype=torch.float32, device=slots.device)
        ps[..., :kk] = slots[..., :kk]
        pw[..., :kk] = weights[..., :kk]
        slots, weights = ps, pw
    dev = values.device
    sl, wt, vals = slots.contiguous(), weights.contiguous(), values.detach().contiguous()
    if out is None:
        out = torch.empty(B, T, H * dh, dtype=out_dtype, device=dev)
    ostride = _rows(out, "out", B, T, H * dh)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_table_read(ctypes.byref(dims), _ptr(sl), _ptr(wt), _ptr(vals), _DT[vals.dtype], _ptr(out), ostride,
                               _DT[out.dtype], ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return out


TABLE_STEP_MAX = 256   # token counts up to this take sdm_rt_table_step (the query map's sums as sdm_rt_gemm_rows')


def table_step_fits(hx, wq, values, d_a):
    """Whether sdm_rt_table_step serves this TrainedSdm read: bfloat16 inputs, map and tables, at most
    TABLE_STEP_MAX tokens, d_a 32 or 64, the layer width a multiple of 64, head_dim a multiple of 8 up to 1,024, no
    autograd."""
    d = hx.shape[-1]
    rows = hx.numel() // d if d else 0
    return (hx.is_cuda and hx.dtype == torch.bfloat16 and wq.dtype == torch.bfloat16
            and values.dtype == torch.bfloat16 and 0 < rows <= TABLE_STEP_MAX and d % 64 == 0 and d_a in (32, 64)
            and values.shape[-1] % 8 == 0 and values.shape[-1] <= 1024
            and not (torch.is_grad_enabled() and any(t.requires_grad for t in (hx, wq, values))))


def table_step(hx, wq, keys1, keys2, log_scale, values, k, params=None, want_q=False):
    """TrainedSdm's read for a few tokens in one launch (sdm_rt_table_step): q = hx wq^T, its product-key picks and
    the weighted read of the picked rows, bit for bit what linear(), address(padded=True) and table_read() give.
    hx [B, T, d] bf16, wq [H * d_a, d] bf16, values [H, M, dh] bf16.  Returns (r [B, T, H * dh] bf16, slots, scores,
    weights [B, H, T, pitch], q [B, T, H * d_a] or None)."""
    lib = _lib.load()
    B, T, d = hx.shape
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dh = values.shape[-1]
    dims = make_dims(B, T, H, dh, d_a, n_sub, k, out_norm=False, write_gate=False)
    x2 = hx.reshape(B * T, d)
    if not _rows16(x2):
        x2 = x2.contiguous()
    wq = wq if _rows16(wq) else wq.contiguous()
    vals = values.detach().contiguous()
    dev = hx.device
    if params is None:
        params = _params(dev, keys1, keys2, None, log_scale, None, None, None)
    prm, held = params
    pitch = lib.sdm_rt_pick_pitch(ctypes.byref(dims))
    if pitch <= 0:
        raise _lib.SdmRtError(lib.sdm_rt_last_error().decode() or "invalid dimensions")
    slots = torch.empty(B, H, T, pitch, dtype=torch.int32, device=dev)
    scores = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    weights = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    out = torch.empty(B, T, H * dh, dtype=torch.bfloat16, device=dev)
    q = torch.empty(B, T, H * d_a, dtype=torch.bfloat16, device=dev) if want_q else None
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_table_step(ctypes.byref(dims), ctypes.byref(prm), _ptr(x2), x2.stride(0), d, _ptr(wq), wq.stride(0),
                               _ptr(vals), _ptr(q), H * d_a, _ptr(slots), _ptr(scores), _ptr(weights), _ptr(out),
                               H * dh, ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    del held
    return out, slots, scores, weights, q


def table_step_residual_fits(x, y, wq, values, d_a):
    """Whether sdm_rt_table_step_residual serves this residual add and TrainedSdm read: table_step_fits on x, y of
    x's shape and dtype, both contiguous, and the layer width 768."""
    return (x.shape[-1] == TABLE_STEP_FOLD_D and y.shape == x.shape and y.dtype == x.dtype and x.is_contiguous()
            and y.is_contiguous() and y.is_cuda and table_step_fits(x, wq, values, d_a)
            and not (torch.is_grad_enabled() and (x.requires_grad or y.requires_grad)))


TABLE_STEP_FOLD_D = 768   # the layer width of sdm_rt_table_step_residual


def table_step_residual(x, y, norm_w, eps, wq, keys1, keys2, log_scale, values, k, params=None, want_q=False,
                        inplace=True, want_hx=False):
    """The residual add, TrainedSdm's input norm and its read in one launch (sdm_rt_table_step_residual):
    s = x + y, hx = rms_norm(s, norm_w, eps) in bf16, then table_step on hx; bit for bit add_rms_norm followed by
    table_step.  x, y [B, T, 768] bf16, contiguous.  s is written into x when ``inplace`` (one head only; otherwise
    into a new tensor).  Returns (s, r, slots, scores, weights, q, hx); q and hx are None unless asked for."""
    lib = _lib.load()
    B, T, d = x.shape
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dh = values.shape[-1]
    dims = make_dims(B, T, H, dh, d_a, n_sub, k, out_norm=False, write_gate=False)
    wq = wq if _rows16(wq) else wq.contiguous()
    vals = values.detach().contiguous()
    dev = x.device
    if params is None:
        params = _params(dev, keys1, keys2, None, log_scale, None, None, None)
    prm, held = params
    pitch = lib.sdm_rt_pick_pitch(ctypes.byref(dims))
    if pitch <= 0:
        raise _lib.SdmRtError(lib.sdm_rt_last_error().decode() or "invalid dimensions")
    s = x if (inplace and H == 1) else torch.empty_like(x)
    wf = _f32_weight(norm_w, dev)
    slots = torch.empty(B, H, T, pitch, dtype=torch.int32, device=dev)
    scores = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    weights = torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev)
    out = torch.empty(B, T, H * dh, dtype=torch.bfloat16, device=dev)
    q = torch.empty(B, T, H * d_a, dtype=torch.bfloat16, device=dev) if want_q else None
    hx = torch.empty(B, T, d, dtype=torch.bfloat16, device=dev) if want_hx else None
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_table_step_residual(ctypes.byref(dims), ctypes.byref(prm), _ptr(x), d, _ptr(y), d, _ptr(wf),
                                        float(eps), _ptr(s), d, _ptr(hx), d, d, _ptr(wq), wq.stride(0), _ptr(vals),
                                        _ptr(q), H * d_a, _ptr(slots), _ptr(scores), _ptr(weights), _ptr(out), H * dh,
                                        ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    del held
    return s, out, slots, scores, weights, q, hx


class DecodeState:
    """State of B decode streams: the true memory is ``scale * mem`` and the true counts ``scale * cnt``
    (mem [B, H, M, dh], cnt [B, H, M], scale [B, H], float32, on the device).  Keeping the scale apart lets a decode
    step fade the whole state in O(1).  ``last`` [B, H, pitch] int32 (or None) holds the slots of the last step's
    writes where that step left nothing else (a head of decay 0), so the next step zeroes only those rows: -1 marks
    an unused entry, -2 in entry 0 a slab whose other rows are unknown."""

    def __init__(self, mem, cnt, scale, last=None):
        B, H, M, dh = mem.shape
        if tuple(cnt.shape) != (B, H, M) or tuple(scale.shape) != (B, H):
            raise ValueError("DecodeState needs mem [B, H, M, dh], cnt [B, H, M] and scale [B, H]")
        for t in (mem, cnt, scale):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device != mem.device:
                raise ValueError("DecodeState tensors must be contiguous float32 on one device")
        if last is not None and (last.dtype != torch.int32 or last.dim() != 3 or tuple(last.shape[:2]) != (B, H)
                                 or not last.is_contiguous() or last.device != mem.device):
            raise ValueError("DecodeState.last must be contiguous int32 [B, H, pitch] on the state's device")
        self.mem, self.cnt, self.scale, self.last = mem, cnt, scale, last

    @classmethod
    def empty(cls, B, H, M, dh, device, pitch=None):
        last = None if pitch is None else torch.full((B, H, pitch), -1, dtype=torch.int32, device=device)
        return cls(torch.zeros(B, H, M, dh, device=device), torch.zeros(B, H, M, device=device),
                   torch.ones(B, H, device=device), last)

    @classmethod
    def from_state(cls, mem, cnt, pitch=None):
        """Continue from a true state, e.g. the (mem, cnt) of core_forward(..., want_state=True)."""
        mem = mem.detach().to(torch.float32).contiguous().clone()
        cnt = cnt.detach().to(torch.float32).contiguous().clone()
        last = None
        if pitch is not None:
            last = torch.full(mem.shape[:2] + (pitch,), -1, dtype=torch.int32, device=mem.device)
            last[..., 0] = -2
        return cls(mem, cnt, torch.ones(mem.shape[:2], device=mem.device), last)

    def state(self):
        """The true (mem, cnt), as forward's last_state holds them (a format conversion, not a decode step)."""
        return self.mem * self.scale[..., None, None], self.cnt * self.scale[..., None]

    def nbytes(self):
        """Device bytes the state holds."""
        return sum(t.numel() * t.element_size() for t in (self.mem, self.cnt, self.scale, self.last) if t is not None)


def pick_pitch(k, n_sub):
    """Entries per address of the pick arrays (sdm_rt_pick_pitch): the kept picks rounded up to 8."""
    c1 = min(k, n_sub)
    kk = min(k, c1 * c1)
    return (kk + 7) // 8 * 8


def decode_step(kz, qz, v, gate_logits, state, *, keys1, keys2, log_scale, decay, addr_b=None, onorm_w=None,
                gate_bias=None, k, read_mode="mean", out_norm=True, read_eps=1e-3, out_norm_eps=1e-2, reset=None,
                out_dtype=None, out=None, workspace=None, params=None):
    """One token for each of B streams (RunTimeSdm.forward_sequential's recurrence, one step): optional reset, read,
    then faded write, updating ``state`` (a DecodeState) in place.

    kz, qz [B, H * d_a]; v [B, H * dh]; gate_logits [B, H] or None; reset [B] bool or None.  Returns r [B, H * dh]
    (before wo), out_dtype defaulting to v's dtype."""
    lib = _lib.load()
    B = v.shape[0]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dh = v.shape[1] // H
    M = n_sub * n_sub
    dims = make_dims(B, 1, H, dh, d_a, n_sub, k, read_mode, out_norm, gate_logits is not None, read_eps,
                     out_norm_eps)
    dt = v.dtype
    for name, x in (("kz", kz), ("qz", qz), ("gate_logits", gate_logits)):
        if x is not None and x.dtype != dt:
            raise ValueError(f"{name} has dtype {x.dtype}, expected {dt}")
    ks = _rows2(kz, "kz", B, H * d_a)
    qs = _rows2(qz, "qz", B, H * d_a)
    vs = _rows2(v, "v", B, H * dh)
    gs = 0 if gate_logits is None else _rows2(gate_logits, "gate_logits", B, H)
    if tuple(state.mem.shape) != (B, H, M, dh):
        raise ValueError(f"state holds {tuple(state.mem.shape)}, expected [B={B}, H={H}, M={M}, dh={dh}]")
    if state.last is not None and state.last.shape[2] != pick_pitch(k, n_sub):
        raise ValueError(f"state.last has pitch {state.last.shape[2]}, expected {pick_pitch(k, n_sub)}")
    dev = v.device
    if params is None:
        params = _params(dev, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias)
    prm = params[0]
    rs = None
    if reset is not None:
        if tuple(reset.shape) != (B,):
            raise ValueError(f"reset must be [B={B}]")
        rs = reset.to(device=dev, dtype=torch.uint8).contiguous()
    out_dtype = out_dtype or dt
    if out is None:
        out = torch.empty(B, H * dh, dtype=out_dtype, device=dev)
    ostride = _rows2(out, "out", B, H * dh)
    nbytes = lib.sdm_rt_decode_workspace_bytes(ctypes.byref(dims))
    ws = (workspace or CoreWorkspace()).get(nbytes, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_decode_step(ctypes.byref(dims), ctypes.byref(prm), _ptr(kz), ks, _ptr(qz), qs, _ptr(v), vs,
                                _ptr(gate_logits), gs, _DT[dt], _ptr(rs), _ptr(state.mem), _ptr(state.cnt),
                                _ptr(state.scale), _ptr(state.last), _ptr(out), ostride, _DT[out_dtype], _ptr(ws), ws.numel(),
                                ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return out


_W32 = WeakIdKeyDictionary()


def _f32_weight(w, device):
    """A norm weight as the contiguous float32 device vector the kernels read; a conversion is kept per weight
    tensor until the tensor changes in place (its version counter), so a bfloat16 model converts each weight once."""
    if w.dtype == torch.float32 and w.device == device and w.is_contiguous():
        return w.detach()
    hit = _W32.get(w)
    if hit is not None and hit[0] == w._version and hit[1].device == device:
        return hit[1]
    f = w.detach().to(device=device, dtype=torch.float32).contiguous()
    _W32[w] = (w._version, f)
    return f


def rms_norm(x, w, eps=1e-6, out_dtype=None, out=None):
    """RMSNorm of the last dimension with the reference's rounding (track4_sdmllm_models.py:63-71):
    cast_out(cast_in(x * rsqrt(mean(x^2) + eps)) * w), float32 math; out_dtype defaults to x.dtype."""
    if x.device.type != "cuda":
        raise RuntimeError("rms_norm needs a ROCm device tensor")
    if x.dtype not in _DT:
        raise ValueError(f"rms_norm: dtype {x.dtype} is not float32 or bfloat16")
    d = x.shape[-1]
    x2 = x.reshape(-1, d)
    if x2.numel() and not _rows16(x2):   # the kernel reads rows in 16-byte pieces
        x2 = x2.contiguous()
    out_dtype = out_dtype or x.dtype
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    o2 = out.view(-1, d)
    wf = _f32_weight(w, x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.sdm_rt_rms_norm(_ptr(x2), x2.stride(0) if x2.numel() else d, _DT[x.dtype], x2.shape[0], d, _ptr(wf),
                             float(eps), _ptr(o2), o2.stride(0) if o2.numel() else d, _DT[out_dtype],
                             ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return out


class RmsNormFunction(torch.autograd.Function):
    """rms_norm as an autograd function: the forward on the RMSNorm kernel (the reference's rounding, SM:63-71), the
    backward of y = x * rsqrt(mean(x^2) + eps) * w in float32 with the casts taken as identities, as autograd takes
    the reference's ``.to(x.dtype)``.  apply(x, w, eps, out_dtype) -> y."""

    @staticmethod
    def forward(ctx, x, w, eps, out_dtype):
        ctx.save_for_backward(x, w)
        ctx.eps = eps
        return rms_norm(x, w, eps, out_dtype=out_dtype)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        xf = x.float()
        r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + ctx.eps)
        n = xf * r
        g = dy.float()
        gw = g * w.float()
        dx = r * (gw - n * (gw * n).mean(-1, keepdim=True)) if ctx.needs_input_grad[0] else None
        dw = (g * n).reshape(-1, n.shape[-1]).sum(0) if ctx.needs_input_grad[1] else None
        return (None if dx is None else dx.to(x.dtype), None if dw is None else dw.to(w.dtype), None, None)


# -- training: forward with saved tensors, backward, and the autograd Function -------------------------------------

def add_rms_norm(x, y, w, eps=1e-6, out_dtype=None, inplace=True):
    """The residual add and the next RMSNorm in one kernel: s = x + y (in x's dtype; written into x when
    ``inplace``), returns (s, rms_norm(s, w, eps, out_dtype)) (OneSdmLM.residual's x + layer(x), then a norm)."""
    if x.device.type != "cuda":
        raise RuntimeError("add_rms_norm needs a ROCm device tensor")
    if x.dtype not in _DT or y.dtype != x.dtype or x.shape != y.shape:
        raise ValueError("add_rms_norm: x and y must have one shape and dtype (float32 or bfloat16)")
    d = x.shape[-1]
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("add_rms_norm: x and y must be contiguous")
    s = x if inplace else torch.empty_like(x)
    out_dtype = out_dtype or x.dtype
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    wf = _f32_weight(w, x.device)
    lib = _lib.load()
    rows = x.numel() // d
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.sdm_rt_add_rms_norm(_ptr(x), d, _ptr(y), d, _DT[x.dtype], rows, d, _ptr(wf), float(eps), _ptr(s), d,
                                 _ptr(out), d, _DT[out_dtype], ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return s, out


def silu_mul(gate_up):
    """SwiGLU's silu(g) * u on a fused [gate | up] projection [..., 2 f], with torch's roundings."""
    if gate_up.device.type != "cuda" or gate_up.dtype not in _DT:
        raise ValueError("silu_mul needs a float32 or bfloat16 ROCm tensor")
    f2 = gate_up.shape[-1]
    g2 = gate_up.reshape(-1, f2)
    if g2.numel() and not _rows16(g2):   # the kernel reads rows in 16-byte pieces
        g2 = g2.contiguous()
    out = torch.empty(gate_up.shape[:-1] + (f2 // 2,), dtype=gate_up.dtype, device=gate_up.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(gate_up.device).cuda_stream
    rc = lib.sdm_rt_silu_mul(_ptr(g2), g2.stride(0), _DT[gate_up.dtype], g2.shape[0], f2 // 2, _ptr(out), f2 // 2,
                             ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return out


GEMM_ROWS_MAX = 256   # row counts up to this use sdm_rt_gemm_rows; larger products go to the GEMM library


def linear(x, w, bias=None, as_matmul=False):
    """F.linear(x, w, bias) (y = x w^T + bias).  A bfloat16 product of a few rows (a decode step's projections:
    at most GEMM_ROWS_MAX rows of x, w [n, k] with n a multiple of 32 and k of 64) runs on sdm_rt_gemm_rows, float32
    sums and the bias added before the one rounding, as the GEMM library rounds; every other product is F.linear
    (torch.matmul(x, w.t()) with ``as_matmul``, for the call sites written that way)."""
    k = x.shape[-1]
    n = w.shape[0]
    rows = x.numel() // k if k else 0
    fits = (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and w.dim() == 2
            and w.shape[1] == k and (bias is None or (bias.dtype == torch.bfloat16 and bias.numel() == n))
            and 0 < rows <= GEMM_ROWS_MAX and n % 32 == 0 and n > 0 and k % 64 == 0 and k > 0
            and not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, w, bias))))
    if not fits:
        if as_matmul and bias is None:
            return torch.matmul(x, w.t())
        return torch.nn.functional.linear(x, w, bias)
    x2 = x.reshape(rows, k)
    if not _rows16(x2):
        x2 = x2.contiguous()
    if not _rows16(w):
        w = w.contiguous()
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    y = torch.empty(x.shape[:-1] + (n,), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.sdm_rt_gemm_rows(_ptr(x2), x2.stride(0), _ptr(w), w.stride(0), _ptr(bias), _ptr(y), n, rows, n, k,
                              ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return y


GEMM_ROWS_FOLD_K = 768   # the layer width of sdm_rt_gemm_rows_residual


def linear_residual_fits(x, y, w, bias=None):
    """Whether sdm_rt_gemm_rows_residual serves this residual add, input norm and map: x, y bf16 of one shape,
    contiguous, with 768 columns; w [n, 768] bf16 with n a positive multiple of 32 (bias bf16 [n] or None); at most
    256 tiles of 64 rows x 32 columns; no autograd recording."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and y.dtype == x.dtype and y.shape == x.shape
            and x.is_contiguous() and y.is_contiguous() and x.shape[-1] == GEMM_ROWS_FOLD_K):
        return False
    if not (w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[1] == GEMM_ROWS_FOLD_K and w.shape[0] % 32 == 0
            and w.shape[0] > 0 and (bias is None or (bias.dtype == torch.bfloat16 and bias.numel() == w.shape[0]))):
        return False
    rows = x.numel() // GEMM_ROWS_FOLD_K
    if rows == 0 or (w.shape[0] // 32) * ((rows + 63) // 64) > 256:
        return False
    return not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, y, w, bias)))


def linear_residual(x, y, norm_w, eps, w, bias=None):
    """The residual add, the next layer's input norm and its map in one launch (sdm_rt_gemm_rows_residual):
    s = x + y, hx = rms_norm(s, norm_w, eps) in bf16, out = linear(hx, w, bias); bit for bit add_rms_norm followed by
    linear.  x, y [..., 768] bf16, contiguous (linear_residual_fits).  s is a new tensor (every workgroup reads x and y
    while the first column's write the sums).  Returns (s, out)."""
    k = GEMM_ROWS_FOLD_K
    n = w.shape[0]
    rows = x.numel() // k
    w = w if _rows16(w) else w.contiguous()
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    s = torch.empty_like(x)
    out = torch.empty(x.shape[:-1] + (n,), dtype=torch.bfloat16, device=x.device)
    wf = _f32_weight(norm_w, x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.sdm_rt_gemm_rows_residual(_ptr(x), k, _ptr(y), k, _ptr(wf), float(eps), _ptr(s), k, _ptr(w), w.stride(0),
                                       _ptr(bias), _ptr(out), n, rows, n, k, ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return s, out


def linear_embed_fits(idx, table, w, bias=None):
    """Whether sdm_rt_gemm_rows_embed serves this embedding, first norm and map: idx int64 [rows] on the GPU, table
    [vocab, 768] bf16 with 16-byte aligned rows, w and bias as linear_residual_fits takes them, at most 256 tiles of
    64 rows x 32 columns, no autograd recording."""
    if not (idx.is_cuda and idx.dtype == torch.int64 and idx.dim() == 1 and idx.numel() > 0):
        return False
    if not (table.is_cuda and table.dtype == torch.bfloat16 and table.dim() == 2
            and table.shape[1] == GEMM_ROWS_FOLD_K and _rows16(table)):
        return False
    if not (w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[1] == GEMM_ROWS_FOLD_K and w.shape[0] % 32 == 0
            and w.shape[0] > 0 and (bias is None or (bias.dtype == torch.bfloat16 and bias.numel() == w.shape[0]))):
        return False
    if (w.shape[0] // 32) * ((idx.numel() + 63) // 64) > 256:
        return False
    return not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (table, w, bias)))


def linear_embed(idx, table, norm_w, eps, w, bias=None):
    """The embedding gather, the first layer's input norm and its map in one launch (sdm_rt_gemm_rows_embed):
    x = table[idx], hx = rms_norm(x, norm_w, eps) in bf16, out = linear(hx, w, bias); bit for bit the gather, rms_norm
    and linear.  idx int64 [rows], each in [0, vocab) (one outside is clamped into it, not reported)
    (linear_embed_fits).  Returns (x, out), x [rows, 768] a new tensor."""
    k = GEMM_ROWS_FOLD_K
    n = w.shape[0]
    rows = idx.numel()
    idx = idx.contiguous()
    w = w if _rows16(w) else w.contiguous()
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    x = torch.empty(rows, k, dtype=torch.bfloat16, device=idx.device)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=idx.device)
    wf = _f32_weight(norm_w, idx.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(idx.device).cuda_stream
    rc = lib.sdm_rt_gemm_rows_embed(_ptr(idx), _ptr(table), table.stride(0), table.shape[0], _ptr(wf), float(eps),
                                    _ptr(x), k, _ptr(w), w.stride(0), _ptr(bias), _ptr(out), n, rows, n, k,
                                    ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return x, out


def _dims_of(kz, v, keys1, k, read_mode, out_norm, gated, read_eps, out_norm_eps):
    B, T = v.shape[0], v.shape[1]
    H, n_sub, half = keys1.shape
    dh = v.shape[2] // H
    return make_dims(B, T, H, dh, 2 * half, n_sub, k, read_mode, out_norm, gated, read_eps, out_norm_eps)


def core_forward_train(kz, qz, v, gate_logits, *, params, k, read_mode="mean", out_norm=True, read_eps=1e-3,
                       out_norm_eps=1e-2, out_dtype=torch.float32, reset=None, workspace=None):
    """core_forward (empty start, no state out) that also keeps what core_backward needs.

    params: a prepared (SdmRtParams, held) pair (_params).  Returns (r [B, T, H * dh] out_dtype, saved dict of
    device tensors: slots_w/weights_w/scores_w, slots_r/weights_r/scores_r [B, H, T, pitch], read [B, T, H * dh] and
    den [B, T, H] float32)."""
    lib = _lib.load()
    keys1 = params[1][0]
    B, T = v.shape[0], v.shape[1]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dh = v.shape[2] // H
    dims = _dims_of(kz, v, keys1, k, read_mode, out_norm, gate_logits is not None, read_eps, out_norm_eps)
    dt = v.dtype
    for name, x in (("kz", kz), ("qz", qz), ("gate_logits", gate_logits)):
        if x is not None and x.dtype != dt:
            raise ValueError(f"{name} has dtype {x.dtype}, expected {dt}")
    vs = _rows(v, "v", B, T, H * dh)
    ks = _rows(kz, "kz", B, T, H * d_a)
    qs = _rows(qz, "qz", B, T, H * d_a)
    gs = 0 if gate_logits is None else _rows(gate_logits, "gate_logits", B, T, H)
    dev = v.device
    pitch = lib.sdm_rt_pick_pitch(ctypes.byref(dims))
    if pitch <= 0:
        raise _lib.SdmRtError(lib.sdm_rt_last_error().decode() or "invalid dimensions")
    saved = dict(
        slots_w=torch.empty(B, H, T, pitch, dtype=torch.int32, device=dev),
        weights_w=torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev),
        scores_w=torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev),
        slots_r=torch.empty(B, H, T, pitch, dtype=torch.int32, device=dev),
        weights_r=torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev),
        scores_r=torch.empty(B, H, T, pitch, dtype=torch.float32, device=dev),
        read=torch.empty(B, T, H * dh, dtype=torch.float32, device=dev),
        den=torch.empty(B, T, H, dtype=torch.float32, device=dev),
    )
    sv = _lib.SdmRtSaved(*[_ptr(saved[n]) for n in ("slots_w", "weights_w", "scores_w", "slots_r", "weights_r",
                                                    "scores_r", "read", "den")])
    out = torch.empty(B, T, H * dh, dtype=out_dtype, device=dev)
    rs = None
    if reset is not None:
        if tuple(reset.shape) != (B, T):
            raise ValueError(f"reset must be [B={B}, T={T}]")
        rs = reset.to(device=dev, dtype=torch.uint8).contiguous()
    saved["reset"] = rs
    nbytes = lib.sdm_rt_workspace_bytes(ctypes.byref(dims))
    ws = (workspace or CoreWorkspace()).get(nbytes, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_forward_train(ctypes.byref(dims), ctypes.byref(params[0]), _ptr(kz), ks, _ptr(qz), qs, _ptr(v),
                                  vs, _ptr(gate_logits), gs, _DT[dt], _ptr(rs), _ptr(out), H * dh, _DT[out_dtype],
                                  ctypes.byref(sv), _ptr(ws), ws.numel(), ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return out, saved


def core_backward(kz, qz, v, gate_logits, saved, dy, *, params, k, read_mode="mean", out_norm=True, read_eps=1e-3,
                  out_norm_eps=1e-2, workspace=None):
    """Gradients of the core for dy = d loss / d r (r from core_forward_train with the same inputs and params).

    Returns a dict of float32 device tensors: kz, qz [B, T, H * d_a], v [B, T, H * dh], gate_logits [B, T, H] (None
    without the gate), keys1, keys2, addr_b, log_scale, onorm_w (None without the out-norm), gate_bias, log_decay
    (lam * d loss / d lam)."""
    lib = _lib.load()
    keys1 = params[1][0]
    B, T = v.shape[0], v.shape[1]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    dh = v.shape[2] // H
    gated = gate_logits is not None
    dims = _dims_of(kz, v, keys1, k, read_mode, out_norm, gated, read_eps, out_norm_eps)
    vs = _rows(v, "v", B, T, H * dh)
    ks = _rows(kz, "kz", B, T, H * d_a)
    qs = _rows(qz, "qz", B, T, H * d_a)
    gs = 0 if gate_logits is None else _rows(gate_logits, "gate_logits", B, T, H)
    if dy.dtype not in _DT:
        dy = dy.float()
    if dy.dim() != 3 or dy.stride(2) != 1:
        dy = dy.contiguous()
    dys = _rows(dy, "dy", B, T, H * dh)
    dev = v.device
    f32 = dict(dtype=torch.float32, device=dev)
    g = dict(kz=torch.empty(B, T, H * d_a, **f32), qz=torch.empty(B, T, H * d_a, **f32),
             v=torch.empty(B, T, H * dh, **f32), gate_logits=torch.empty(B, T, H, **f32) if gated else None,
             keys1=torch.empty(H, n_sub, half, **f32), keys2=torch.empty(H, n_sub, half, **f32),
             addr_b=torch.empty(H, d_a, **f32), log_scale=torch.empty(H, **f32),
             onorm_w=torch.empty(H, dh, **f32) if out_norm else None, gate_bias=torch.empty(H, **f32),
             log_decay=torch.empty(H, **f32))
    gr = _lib.SdmRtGrads(_ptr(g["kz"]), H * d_a, _ptr(g["qz"]), H * d_a, _ptr(g["v"]), H * dh,
                         _ptr(g["gate_logits"]), H, _ptr(g["keys1"]), _ptr(g["keys2"]), _ptr(g["addr_b"]),
                         _ptr(g["log_scale"]), _ptr(g["onorm_w"]), _ptr(g["gate_bias"]), _ptr(g["log_decay"]))
    sv = _lib.SdmRtSaved(*[_ptr(saved[n]) for n in ("slots_w", "weights_w", "scores_w", "slots_r", "weights_r",
                                                    "scores_r", "read", "den")])
    nbytes = lib.sdm_rt_backward_workspace_bytes(ctypes.byref(dims))
    ws = (workspace or CoreWorkspace()).get(nbytes, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_backward(ctypes.byref(dims), ctypes.byref(params[0]), _ptr(kz), ks, _ptr(qz), qs, _ptr(v), vs,
                             _ptr(gate_logits), gs, _DT[v.dtype], _ptr(saved["reset"]), ctypes.byref(sv), _ptr(dy),
                             dys, _DT[dy.dtype], ctypes.byref(gr), _ptr(ws), ws.numel(), ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return g


class SdmCoreFunction(torch.autograd.Function):
    """The SDM core as an autograd function: forward sdm_rt_forward_train, backward sdm_rt_backward.

    apply(kz, qz, v, gate_logits, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias, cfg) -> r float32
    [B, T, H * dh].  kz, qz, v, gate_logits share one dtype (float32 or bfloat16); gate_logits, addr_b, onorm_w and
    gate_bias may be None.  cfg: dict with k, read_mode, out_norm, read_eps, out_norm_eps, reset ([B, T] bool or
    None) and optionally workspace (a CoreWorkspace).  The picks carry no gradient (as topk in the reference)."""

    @staticmethod
    def forward(ctx, kz, qz, v, gate_logits, keys1, keys2, addr_b, log_scale, decay, onorm_w, gate_bias, cfg):
        if v.device.type != "cuda":
            raise RuntimeError("the SDM core needs ROCm device tensors")
        params = _params(v.device, keys1, keys2, addr_b, log_scale, decay, onorm_w if cfg["out_norm"] else None,
                         gate_bias)
        opts = dict(k=cfg["k"], read_mode=cfg["read_mode"], out_norm=cfg["out_norm"], read_eps=cfg["read_eps"],
                    out_norm_eps=cfg["out_norm_eps"])
        r, saved = core_forward_train(kz, qz, v, gate_logits, params=params, reset=cfg.get("reset"),
                                      workspace=cfg.get("workspace"), **opts)
        ctx.opts = opts
        ctx.params = params
        ctx.saved = saved
        ctx.workspace = cfg.get("workspace")
        ctx.has = (gate_logits is not None, addr_b is not None, onorm_w is not None, gate_bias is not None)
        ctx.dtypes = (kz.dtype, keys1.dtype, log_scale.dtype, decay.dtype)
        ctx.save_for_backward(kz, qz, v, gate_logits, decay)
        return r

    @staticmethod
    def backward(ctx, dr):
        kz, qz, v, gate_logits, decay = ctx.saved_tensors
        g = core_backward(kz, qz, v, gate_logits, ctx.saved, dr, params=ctx.params, workspace=ctx.workspace,
                          **ctx.opts)
        has_g, has_ab, has_on, has_gb = ctx.has
        dt = ctx.dtypes[0]
        need = ctx.needs_input_grad

        def cast(t, like_dtype, i):
            return t.to(like_dtype) if (t is not None and need[i]) else None
        d_decay = None
        if need[8]:
            lam = decay.detach().to(torch.float32)
            d_decay = torch.where(lam > 0, g["log_decay"] / torch.where(lam > 0, lam, torch.ones_like(lam)),
                                  torch.zeros_like(lam)).to(decay.dtype)
        return (cast(g["kz"], dt, 0), cast(g["qz"], dt, 1), cast(g["v"], dt, 2),
                cast(g["gate_logits"], dt, 3) if has_g else None,
                cast(g["keys1"], ctx.dtypes[1], 4), cast(g["keys2"], ctx.dtypes[1], 5),
                cast(g["addr_b"], ctx.dtypes[1], 6) if has_ab else None,
                cast(g["log_scale"], ctx.dtypes[2], 7), d_decay,
                cast(g["onorm_w"], ctx.dtypes[1], 9) if has_on else None,
                cast(g["gate_bias"], ctx.dtypes[1], 10) if has_gb else None, None)


def table_backward(q, slots, weights, scores, values, dy, *, k, params, workspace=None):
    """Gradients of TrainedSdm's table read for fixed picks (sdm_rt_table_backward).

    q [B, T, H * d_a]; slots, weights, scores [B, H, T, pitch] from address(q, ..., padded=True); values [H, M, dh];
    dy [B, T, H * dh] the gradient of the read.  params: the (SdmRtParams, held) pair of keys1, keys2 and log_scale.
    Returns a dict of float32 device tensors q, values, keys1, keys2, log_scale."""
    lib = _lib.load()
    keys1 = params[1][0]
    B, T = q.shape[0], q.shape[1]
    H, n_sub, half = keys1.shape
    d_a = 2 * half
    Hv, M, dh = values.shape
    dims = make_dims(B, T, H, dh, d_a, n_sub, k, out_norm=False, write_gate=False)
    qs = _rows(q, "q", B, T, H * d_a)
    if dy.dtype not in _DT:
        dy = dy.float()
    if dy.dim() != 3 or dy.stride(2) != 1:
        dy = dy.contiguous()
    dys = _rows(dy, "dy", B, T, H * dh)
    vals = values.detach().contiguous()
    dev = q.device
    f32 = dict(dtype=torch.float32, device=dev)
    g = dict(q=torch.empty(B, T, H * d_a, **f32), values=torch.empty(H, M, dh, **f32),
             keys1=torch.empty(H, n_sub, half, **f32), keys2=torch.empty(H, n_sub, half, **f32),
             log_scale=torch.empty(H, **f32))
    nbytes = lib.sdm_rt_table_backward_workspace_bytes(ctypes.byref(dims))
    ws = (workspace or CoreWorkspace()).get(nbytes, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.sdm_rt_table_backward(ctypes.byref(dims), ctypes.byref(params[0]), _ptr(q), qs, _DT[q.dtype],
                                   _ptr(slots), _ptr(weights), _ptr(scores), _ptr(vals), _DT[vals.dtype], _ptr(dy),
                                   dys, _DT[dy.dtype], _ptr(g["q"]), H * d_a, _ptr(g["values"]), _ptr(g["keys1"]),
                                   _ptr(g["keys2"]), _ptr(g["log_scale"]), _ptr(ws), ws.numel(),
                                   ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    return g


class TableSdmFunction(torch.autograd.Function):
    """TrainedSdm's layer between the query map and wo as an autograd function: forward sdm_rt_address +
    sdm_rt_table_read, backward sdm_rt_table_backward.

    apply(q, keys1, keys2, log_scale, values, cfg) -> r float32 [B, T, H * dh]; q [B, T, H * d_a] float32 or
    bfloat16; cfg: dict with k and optionally workspace.  After the call cfg["slots"] holds the picks
    [B, H, T, pitch].  The picks carry no gradient (as topk in the reference)."""

    @staticmethod
    def forward(ctx, q, keys1, keys2, log_scale, values, cfg):
        if q.device.type != "cuda":
            raise RuntimeError("the table layer needs ROCm device tensors")
        params = _params(q.device, keys1, keys2, None, log_scale, None, None, None)
        slots, scores, weights = address(q, keys1, keys2, cfg["k"], log_scale, padded=True, params=params)
        r = table_read(slots, weights, values, cfg["k"], out_dtype=torch.float32)
        cfg["slots"] = slots
        ctx.k = cfg["k"]
        ctx.params = params
        ctx.workspace = cfg.get("workspace")
        ctx.dtypes = (q.dtype, keys1.dtype, log_scale.dtype, values.dtype)
        ctx.save_for_backward(q, values, slots, scores, weights)
        return r

    @staticmethod
    def backward(ctx, dr):
        q, values, slots, scores, weights = ctx.saved_tensors
        g = table_backward(q, slots, weights, scores, values, dr, k=ctx.k, params=ctx.params,
                           workspace=ctx.workspace)
        need = ctx.needs_input_grad
        dq, dk, dl, dv = ctx.dtypes
        return (g["q"].to(dq) if need[0] else None, g["keys1"].to(dk) if need[1] else None,
                g["keys2"].to(dk) if need[2] else None, g["log_scale"].to(dl) if need[3] else None,
                g["values"].to(dv) if need[4] else None, None)
