"""TrainedSdm: the trained product-key table layer of SDMCHAT (experiments/track4/sdmllm/track4_onesdm_models.py:414-457)
on the MI355X kernels.

A drop-in for the reference module: the same constructor, parameter names, shapes and initialisation (a
``Generator(9876 + seed)`` draws keys1 then keys2; values start at zero), so a reference state dict loads with
``strict=True``.  The forward runs the RMSNorm kernel, the query map as one GEMM, the product-key addressing kernel
(sdm_rt_address: top-k of the n_sub^2 slots and the softmax weights) and the weighted table read (sdm_rt_table_read,
the reference's embedding_bag), then the output map.  There is no CPU or torch fallback.

Training: with autograd recording the norm, the query map and wo run as the reference's torch ops (under the
caller's autocast) and the layer between them through ``core.TableSdmFunction``, whose backward is the HIP
``sdm_rt_table_backward`` (gradients of the query, the sub-keys, log_scale and the value tables).
"""
import math

import torch
import torch.nn as nn

from . import core
from .runtime_sdm import RMSNorm


class TrainedSdm(nn.Module):
    """x [B, T, d] -> y [B, T, d]: per token and head, the softmax-weighted sum of the k table rows that the
    query's product-key address picks (track4_onesdm_models.py:414-457).  It never mixes positions."""

    def __init__(self, d, n_sub, heads=4, d_a=32, k=32, scale=8.0, learn_scale=True, seed=0):
        super().__init__()
        if not (d % heads == 0 and d_a % 2 == 0 and heads * d_a <= d):
            raise ValueError("TrainedSdm needs d % heads == 0, an even d_a and heads * d_a <= d")
        g = torch.Generator().manual_seed(9876 + seed)
        self.d, self.h, self.dh, self.d_a, self.k = d, heads, d // heads, d_a, k
        self.n_sub, self.M = n_sub, n_sub * n_sub
        self.norm = RMSNorm(d)
        self.wq = nn.Linear(d, heads * d_a, bias=False)
        self.keys1 = nn.Parameter(torch.randn(heads, n_sub, d_a // 2, generator=g))
        self.keys2 = nn.Parameter(torch.randn(heads, n_sub, d_a // 2, generator=g))
        self.values = nn.Parameter(torch.zeros(heads, self.M, self.dh))
        self.log_scale = nn.Parameter(torch.full((heads,), math.log(scale)), requires_grad=learn_scale)
        self.wo = nn.Linear(d, d, bias=False)
        self.last_si = None
        self.keep_picks = False   # set True to keep the last forward's queries in last_q
        self.last_q = None
        self.last_hx = None
        self._cast = None
        self._prm = core.ParamCache()

    def reset_init(self):
        """Zero start: every read is exactly zero, so the layer adds nothing at init (track4_onesdm_models.py:433-436)."""
        nn.init.zeros_(self.values)

    def _check(self, x):
        if x.device.type != "cuda":
            raise RuntimeError("TrainedSdm HIP path needs a ROCm device tensor")
        if x.dim() != 3 or x.shape[-1] != self.d:
            raise ValueError(f"expected x of shape [B, T, {self.d}], got {tuple(x.shape)}")

    def _compute_dtype(self, x):
        if x.dtype == torch.bfloat16:
            return torch.bfloat16
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            return torch.bfloat16
        if x.dtype == torch.float32:
            return torch.float32
        raise ValueError(f"unsupported input dtype {x.dtype}")

    def _weights(self, dt):
        """wq and wo in the compute dtype, cached until either changes."""
        ws = (self.wq.weight, self.wo.weight)
        key = (dt,) + tuple((w.data_ptr(), w._version) for w in ws)
        if self._cast is None or self._cast[0] != key:
            self._cast = (key,) + tuple(w.detach().to(dt) for w in ws)
        return self._cast[1], self._cast[2]

    def _picks(self, x, dt, hx=None):
        """RMSNorm, the query map and the addressing: slots, scores, weights [B, H, T, pitch].  hx: the normed input
        when the caller computed it."""
        if hx is None:
            hx = core.rms_norm(x, self.norm.w, self.norm.eps, out_dtype=dt)
        q = core.linear(hx, self._weights(dt)[0], as_matmul=True)
        if self.keep_picks:
            self.last_q = q
        prm = self._prm.get(x.device, self.keys1, self.keys2, None, self.log_scale, None, None, None)
        return core.address(q, self.keys1, self.keys2, self.k, self.log_scale, padded=True, params=prm)

    def address(self, x):
        """x (B, T, d) -> soft weights (B*T, h, kk) and slot ids (B*T, h, kk), as the reference's address()."""
        self._check(x)
        B, T, _ = x.shape
        with torch.autocast("cuda", enabled=False):
            si, _, w = self._picks(x, self._compute_dtype(x))
        kk = min(self.k, min(self.k, self.n_sub) ** 2)
        return (w[..., :kk].permute(0, 2, 1, 3).reshape(B * T, self.h, kk),
                si[..., :kk].permute(0, 2, 1, 3).reshape(B * T, self.h, kk).long())

    def _training(self, x):
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _forward_train(self, x):
        """The differentiable forward (track4_onesdm_models.py:438-455): q = wq(norm(x).float()).float(), the table
        layer through TableSdmFunction, wo."""
        B, T, _ = x.shape
        q = self.wq(self.norm(x).float()).float()
        cfg = dict(k=self.k)
        r = core.TableSdmFunction.apply(q, self.keys1, self.keys2, self.log_scale, self.values, cfg)
        kk = min(self.k, min(self.k, self.n_sub) ** 2)
        self.last_si = cfg["slots"][..., :kk].permute(0, 2, 1, 3).reshape(B * T, self.h, kk)
        return self.wo(r).to(x.dtype)

    def forward(self, x, hx=None):
        """x [B, T, d] -> y [B, T, d].  hx: rms_norm(x) in the compute dtype, when the caller has it (inference)."""
        self._check(x)
        if self._training(x):
            return self._forward_train(x)
        B, T, _ = x.shape
        dt = self._compute_dtype(x)
        with torch.autocast("cuda", enabled=False):
            if hx is None:
                hx = core.rms_norm(x, self.norm.w, self.norm.eps, out_dtype=dt)
            wq, wo = self._weights(dt)
            if core.table_step_fits(hx, wq, self.values, self.d_a):   # a few tokens: the read in one launch
                prm = self._prm.get(x.device, self.keys1, self.keys2, None, self.log_scale, None, None, None)
                r, si, _, _, q = core.table_step(hx, wq, self.keys1, self.keys2, self.log_scale, self.values, self.k,
                                                 params=prm, want_q=self.keep_picks)
                if self.keep_picks:
                    self.last_q = q
            else:
                si, _, w = self._picks(x, dt, hx)
                r = core.table_read(si, w, self.values, self.k, out_dtype=dt)
            y = core.linear(r, wo, as_matmul=True).to(x.dtype)
        kk = min(self.k, min(self.k, self.n_sub) ** 2)
        self.last_si = si[..., :kk].permute(0, 2, 1, 3).reshape(B * T, self.h, kk)
        return y

    def residual_fits(self, x, y):
        """Whether forward_residual serves x + y for this layer: inference, bfloat16, contiguous, width 768, at most
        core.TABLE_STEP_MAX tokens (a decode step)."""
        if not x.is_cuda or x.dtype != torch.bfloat16 or self._training(x) or torch.is_autocast_enabled("cuda"):
            return False
        wq, _ = self._weights(torch.bfloat16)
        return core.table_step_residual_fits(x, y, wq, self.values, self.d_a)

    def forward_residual(self, x, y):
        """The residual add in front of this layer and the layer, inference only: s = x + y (OneSdmLM's
        x = x + stage(x), track4_onesdm_models.py:540-547), then forward(s); the add, the input norm and the read in
        one launch (core.table_step_residual).  x, y [..., d] bfloat16, contiguous (residual_fits).  s is written into
        x with one head.  With keep_picks, last_hx keeps the normed input.  Returns (s, forward(s))."""
        shape = x.shape
        x3, y3 = x.reshape(-1, 1, shape[-1]) if x.dim() == 2 else x, y.reshape(-1, 1, shape[-1]) if y.dim() == 2 else y
        B, T, _ = x3.shape
        with torch.autocast("cuda", enabled=False):
            wq, wo = self._weights(torch.bfloat16)
            prm = self._prm.get(x.device, self.keys1, self.keys2, None, self.log_scale, None, None, None)
            s, r, si, _, _, q, hx = core.table_step_residual(x3, y3, self.norm.w, self.norm.eps, wq, self.keys1,
                                                             self.keys2, self.log_scale, self.values, self.k,
                                                             params=prm, want_q=self.keep_picks,
                                                             want_hx=self.keep_picks)
            if self.keep_picks:
                self.last_q, self.last_hx = q, hx
            out = core.linear(r, wo, as_matmul=True)
        kk = min(self.k, min(self.k, self.n_sub) ** 2)
        self.last_si = si[..., :kk].permute(0, 2, 1, 3).reshape(B * T, self.h, kk)
        return s.reshape(shape), out.reshape(shape)
