"""RunTimeSdm: drop-in replacement of the reference's run-time SDM mixer, backed by HIP kernels for gfx950.

Mirrors ``RunTimeSdm`` of experiments/track4/sdmllm/track4_onesdm_models.py:151-300: the same constructor arguments,
parameter and buffer names and shapes (so ``load_state_dict(strict=True)`` accepts the reference's checkpoints under
``mems.{i}.<name>``), the same default initialisation (nn.Linear layers built in the same order, sub-keys and
address bias drawn from ``torch.Generator().manual_seed(4321 + seed)``, :159-185) and the same
``forward(x, reset=None) -> Tensor[B, T, d]`` in ``x.dtype``.

What runs where: the input RMSNorm, the four input projections (two GEMMs: [wk; wq; wg] and wv; one of both for a
decode step's few rows) and the output map ``wo`` are dense ops (hipBLASLt, or sdm_rt_gemm_rows for a few rows); the
SDM core between them -- product-key addressing, softmax weights, write gate, the
faded write / causal read of the memory and the mean read with its per-head norm -- is one call into
``libsdm_rt.so`` (sdm_rt_forward).  There is no CPU or pure-torch fallback: a missing library, a CPU tensor or an
unsupported option raises.

Training: with autograd recording (grad enabled and x or a parameter requiring grad) forward takes the reference's
own torch path for the input norm (with grad_scale), the projections and wo, and runs the core through
``core.SdmCoreFunction``, whose backward is ``sdm_rt_backward``: the gradients reach every parameter (the sub-keys,
addr_b, log_scale, decay_logit with learn_decay, onorm_w, the projections and the gate bias) as under the
reference's autograd of its chunked form (:259-268).
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import core


def grad_scale(x, alpha):
    """Identity forward; the gradient into x is scaled by alpha (track4_sdmllm_models.py:170-174)."""
    if alpha == 1.0:
        return x
    xd = x.detach()
    return xd if alpha == 0.0 else xd + alpha * (x - xd)


class RMSNorm(nn.Module):
    """RMSNorm with a weight named ``w`` (track4_sdmllm_models.py:63-71): float math, cast back, times w."""

    def __init__(self, d, eps=1e-6):
        super().__init__()
        self.w = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.w


class RunTimeSdm(nn.Module):
    """A Kanerva memory with M = n_sub^2 locations per head, written and read while the sequence is read."""

    def __init__(self, d, heads=4, n_sub=32, d_a=32, k=16, decays=(0.0, 0.8, 0.99, 1.0), learn_decay=False,
                 write_gate=True, gate_bias=0.0, read_mode="mean", out_norm=True, addr_scale=8.0, learn_scale=True,
                 chunk=128, read_eps=1e-3, mem_in_grad=1.0, out_norm_eps=1e-2, addr_bias=0.0, seed=0):
        super().__init__()
        if d % heads != 0 or d_a % 2 != 0 or len(decays) != heads or read_mode not in ("mean", "sum"):
            raise ValueError("need d % heads == 0, even d_a, one decay per head and read_mode 'mean' or 'sum'")
        gen = torch.Generator().manual_seed(4321 + seed)
        self.d, self.h, self.dh, self.k, self.d_a, self.n_sub = d, heads, d // heads, k, d_a, n_sub
        self.M = n_sub * n_sub
        self.chunk, self.read_mode, self.read_eps, self.mem_in_grad = chunk, read_mode, read_eps, mem_in_grad
        self.write_gate, self.out_norm, self.learn_decay = write_gate, out_norm, learn_decay
        self.out_norm_eps = out_norm_eps
        self.enabled = True
        self._leak = False        # the reference's test-only causality control (OM:165, 223); see forward
        self.keep_state = False   # set True to fill last_state (costs one state write per call)
        self.keep_picks = False   # set True to fill last_picks, last_addresses and last_projections (an extra
                                  # addressing per call, forward and step)
        self.last_picks = self.last_addresses = self.last_projections = None
        self.norm = RMSNorm(d)
        self.wk = nn.Linear(d, heads * d_a, bias=False)
        self.wq = nn.Linear(d, heads * d_a, bias=False)
        self.wv = nn.Linear(d, d, bias=False)
        self.wg = nn.Linear(d, heads, bias=True)
        self.wo = nn.Linear(d, d, bias=False)
        self.keys1 = nn.Parameter(torch.randn(heads, n_sub, d_a // 2, generator=gen))
        self.keys2 = nn.Parameter(torch.randn(heads, n_sub, d_a // 2, generator=gen))
        self.addr_b = nn.Parameter(torch.randn(heads, d_a, generator=gen) * addr_bias)
        self.log_scale = nn.Parameter(torch.full((heads,), math.log(addr_scale)), requires_grad=learn_scale)
        lam = torch.tensor(decays, dtype=torch.float32)
        if learn_decay:
            self.decay_logit = nn.Parameter(torch.logit(lam.clamp(1e-4, 1 - 1e-4)))
        else:
            self.register_buffer("decays_fixed", lam, persistent=True)
        if out_norm:
            self.onorm_w = nn.Parameter(torch.ones(heads, self.dh))
        self.gate_bias0 = gate_bias
        self._gate_src = None
        self.last_gate = None
        self._last_state = None
        self._state_skipped = False
        self._fused = None
        self._ws = core.CoreWorkspace()
        self._prm = core.ParamCache()

    def reset_init(self):
        """Zero output map and gate weights, constant gate bias (track4_onesdm_models.py:187-190)."""
        nn.init.zeros_(self.wo.weight)
        nn.init.zeros_(self.wg.weight)
        nn.init.constant_(self.wg.bias, self.gate_bias0)

    def decay(self):
        """Per-head fade (track4_onesdm_models.py:192-193)."""
        return torch.sigmoid(self.decay_logit) if self.learn_decay else self.decays_fixed

    # -- fused input projection ----------------------------------------------------------------------------------
    def _rows_a(self):
        """Rows of the first projection map, [wk; wq; wg] padded to a multiple of 256 (a shape hipBLASLt runs well)."""
        rows = 2 * self.h * self.d_a + (self.h if self.write_gate else 0)
        return (rows + 255) // 256 * 256

    def _fused_weight(self, dtype):
        """The projections in one buffer, [wk; wq; wg; zero rows up to _rows_a(); wv], the matching bias (zero
        except wg.bias on the gate rows; None without the write gate) and wo, all in ``dtype``, cached until one of
        these tensors changes (data pointer or in-place version).  The sequence forward maps the two row ranges
        separately (two GEMMs of 1,792 and 768 columns at the layer shape run faster than one of 2,560 with the
        bias); a decode step maps the whole buffer at once."""
        ws = (self.wk.weight, self.wq.weight, self.wg.weight, self.wv.weight)
        srcs = ws + (self.wg.bias, self.wo.weight)
        key = (dtype, ws[0].device, self.write_gate) + tuple((t.data_ptr(), t._version) for t in srcs)
        if self._fused is not None and self._fused[0] == key:
            return self._fused[1:]
        H, d_a, d = self.h, self.d_a, self.d
        ra = self._rows_a()
        o_g = 2 * H * d_a
        W = torch.zeros(ra + d, self.d, dtype=dtype, device=ws[0].device)
        W[:o_g].copy_(torch.cat([self.wk.weight.detach(), self.wq.weight.detach()], 0))
        W[ra:].copy_(self.wv.weight.detach())
        bias = None
        if self.write_gate:   # the gate logit rounds once, as the reference's wg(hx) under autocast (OM:205)
            W[o_g:o_g + H].copy_(self.wg.weight.detach())
            bias = torch.zeros(ra + d, dtype=dtype, device=ws[0].device)
            bias[o_g:o_g + H].copy_(self.wg.bias.detach())
        wo = self.wo.weight.detach().to(dtype)
        self._fused = (key, W, bias, wo)
        return W, bias, wo

    def _core_params(self, device):
        """The core's float32 parameters, converted once per change of the module's tensors (no gate bias: it is
        the fused projection's bias)."""
        return self._prm.get(device, self.keys1, self.keys2, self.addr_b, self.log_scale, self.decay,
                             self.onorm_w if self.out_norm else None, None,
                             decay_source=self.decay_logit if self.learn_decay else self.decays_fixed)

    def _check(self, x, reset):
        if reset is not None and (reset.dim() != 2 or tuple(reset.shape) != tuple(x.shape[:2])):
            raise ValueError(f"reset must be [B, T] = {tuple(x.shape[:2])}, got {tuple(reset.shape)}")
        if x.device.type != "cuda":
            raise RuntimeError("RunTimeSdm HIP core needs a ROCm device tensor")
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

    def _project(self, x, dt, hx=None):
        """RMSNorm then the projections wk, wq, wv, wg (prepare, track4_onesdm_models.py:197-206): one GEMM for
        [wk; wq; wg] and one for wv (one GEMM of the whole buffer for a few rows).  Returns views kz, qz
        [B, T, H * d_a] and gate logits [B, T, H] (None without the write gate) of the first map's output, and V
        [B, T, d].  The gate bias is the GEMM's bias, so W_g hx + b rounds to dt once, as wg(hx) does; addr_b is
        added inside the core.  hx: the normed input when the caller computed it (in dt, as the norm below gives
        it)."""
        H, d_a = self.h, self.d_a
        if hx is None:
            hx = core.rms_norm(x, self.norm.w, self.norm.eps, out_dtype=dt)   # the norm, then the cast to dt
        W, bias = self._fused_weight(dt)[:2]
        ra = self._rows_a()
        if hx.numel() // hx.shape[-1] <= core.GEMM_ROWS_MAX:
            proj = core.linear(hx, W, bias)                            # [B, T, ra + d]
            pa, V = proj[..., :ra], proj[..., ra:]
        else:
            pa = core.linear(hx, W[:ra], None if bias is None else bias[:ra])
            V = core.linear(hx, W[ra:])
        o_q, o_g = H * d_a, 2 * H * d_a
        g = pa[..., o_g:o_g + H] if self.write_gate else None
        return pa[..., :o_q], pa[..., o_q:o_g], V, g

    def _training(self, x):
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _project_train(self, x):
        """The differentiable prepare (:195-206) up to the projections: the input norm on the RMSNorm kernel
        (core.RmsNormFunction, with its float32 backward) and the same two maps as inference ([wk; wq; wg] padded,
        with the gate bias, then wv), so both forwards compute the same values.  Under autocast the GEMMs run in its
        dtype, as in the reference.  Returns kz, qz, V, g (None without the write gate)."""
        H, d_a = self.h, self.d_a
        hx = core.RmsNormFunction.apply(grad_scale(x, self.mem_in_grad), self.norm.w, self.norm.eps,
                                        torch.promote_types(x.dtype, self.norm.w.dtype)).float()
        Wa = torch.cat([self.wk.weight, self.wq.weight] + ([self.wg.weight] if self.write_gate else []), 0)
        rows = Wa.shape[0]
        ra = self._rows_a()
        Wa = F.pad(Wa, (0, 0, 0, ra - rows))
        o_q, o_g = H * d_a, 2 * H * d_a
        # the gate bias inside the projection, so the logit rounds once, as wg(hx) does
        bias = F.pad(self.wg.bias, (o_g, ra - rows)) if self.write_gate else None
        pa = F.linear(hx, Wa, bias)
        V = F.linear(hx, self.wv.weight)
        g = pa[..., o_g:o_g + H] if self.write_gate else None
        return pa[..., :o_q], pa[..., o_q:o_g], V, g

    def _forward_train(self, x, reset):
        """The differentiable forward: _project_train, the core through SdmCoreFunction, finish's wo (:247)."""
        B, T, _ = x.shape
        H = self.h
        kz, qz, V, g = self._project_train(x)
        cfg = dict(k=self.k, read_mode=self.read_mode, out_norm=self.out_norm, read_eps=self.read_eps,
                   out_norm_eps=self.out_norm_eps, reset=reset, workspace=self._ws)
        r = core.SdmCoreFunction.apply(kz, qz, V, g, self.keys1, self.keys2, self.addr_b, self.log_scale,
                                       self.decay(), self.onorm_w if self.out_norm else None, None, cfg)
        y = self.wo(r).to(x.dtype)
        self._gate_src = (g.detach().contiguous() if g is not None else None, None, (B, T, H), x.device)
        self._last_gate = None
        self._last_state, self._state_skipped = None, False
        return y

    def forward(self, x, reset=None, hx=None):
        """x [B, T, d] -> y [B, T, d] in x.dtype; every call starts from an empty memory
        (track4_onesdm_models.py:249-274).  reset [B, T] bool: where True the memory is emptied before that position
        reads (a BOS starts a new document, :229-233).  With ``keep_state`` set, ``last_state`` receives (mem, cnt)
        (inference only).  With autograd recording the forward is differentiable (SdmCoreFunction).  hx: the input
        norm rms_norm(x) in the compute dtype, when the caller has it (inference only)."""
        B, T, _ = x.shape
        if not self.enabled:
            return torch.zeros_like(x)
        if self._leak:
            raise NotImplementedError(
                "RunTimeSdm._leak (set_leak) is the reference self-test's causality control, a mask of its dense "
                "chunk algorithm (track4_onesdm_models.py:223) that lets a position read later writes of its chunk; "
                "the HIP kernels compute only the causal recurrence")
        self._check(x, reset)
        if self._training(x):
            return self._forward_train(x, reset)
        dt = self._compute_dtype(x)
        H = self.h
        with torch.autocast("cuda", enabled=False):
            kz, qz, V, g = self._project(x, dt, hx)
            wo = self._fused_weight(dt)[2]
            res = core.core_forward(
                kz, qz, V, g, keys1=self.keys1, keys2=self.keys2, log_scale=self.log_scale, decay=self.decay(),
                addr_b=self.addr_b, onorm_w=self.onorm_w if self.out_norm else None,
                gate_bias=None, k=self.k, read_mode=self.read_mode,
                out_norm=self.out_norm, read_eps=self.read_eps, out_norm_eps=self.out_norm_eps, out_dtype=dt,
                want_state=self.keep_state, workspace=self._ws, reset=reset, params=self._core_params(x.device))
            r, state = (res if self.keep_state else (res, None))
            y = torch.matmul(r, wo.t()).to(x.dtype)
            if self.keep_picks:   # the same addressing kernels as the core's, on the same projections
                prm = self._core_params(x.device)
                self.last_addresses = (kz, qz)   # before addr_b
                self.last_projections = (kz, qz, V, g)
                self.last_picks = tuple(
                    core.address(z, self.keys1, self.keys2, self.k, self.log_scale, addr_b=self.addr_b,
                                 params=prm)[0] for z in (kz, qz))
            # the gate logits as the forward left them in its workspace ([B, T, H]: a view of the projection
            # buffer would keep the whole buffer, ~59 MB at B=8, T=2048, until the next forward, and a copy costs a
            # launch); the workspace is this module's, so the view holds until the next forward replaces it;
            # last_gate applies the sigmoid when first read
            g_keep = None if g is None else core.gate_copy(
                self._ws, B, T, H, self.dh, self.d_a, self.n_sub, self.k, dt, self.read_mode, self.out_norm,
                self.read_eps, self.out_norm_eps)
        self._gate_src = (g_keep, None, (B, T, H), x.device)
        self._last_gate = None
        self._last_state, self._state_skipped = state, not self.keep_state
        return y

    @property
    def last_state(self):
        """(mem [B, H, M, dh], cnt [B, H, M]) float32 after the last forward's final position, as the reference
        sets it on every call (track4_onesdm_models.py:273).  Writing it costs a state write per call (25.6 MB at
        B=8, T=2048), so the forward writes it only with ``keep_state`` set; reading it after a forward that skipped
        it raises instead of returning a stale or missing value."""
        if self._state_skipped:
            raise RuntimeError("RunTimeSdm.last_state: set keep_state = True before the forward to receive the final "
                               "state (it is not written by default: 25.6 MB per call at B=8, T=2048)")
        return self._last_state

    @last_state.setter
    def last_state(self, value):
        self._last_state, self._state_skipped = value, False

    @property
    def last_gate(self):
        """The write gate of the last forward, [B, T, H] float32 (prepare, track4_onesdm_models.py:205, 212);
        computed from the kept gate logits when first read."""
        if self._last_gate is None and self._gate_src is not None:
            g, bias, shape, dev = self._gate_src
            self._last_gate = (torch.sigmoid(g.float() + (bias.float() if bias is not None else 0.0))
                               if g is not None else torch.ones(shape, device=dev))
            self._gate_src = None
        return self._last_gate

    @last_gate.setter
    def last_gate(self, value):
        self._last_gate = value
        self._gate_src = None

    # -- decoding ----------------------------------------------------------------------------------------------------
    def decode_state(self, batch, device=None):
        """An empty state for ``batch`` decode streams (a core.DecodeState)."""
        device = device if device is not None else self.keys1.device
        return core.DecodeState.empty(batch, self.h, self.M, self.dh, device, core.pick_pitch(self.k, self.n_sub))

    def step(self, x, state, reset=None, hx=None):
        """One token for each of B streams: x [B, d] (or [B, 1, d]) -> y of the same shape, with the recurrence of
        forward_sequential (track4_onesdm_models.py:276-300) carried in ``state`` (updated in place).  reset [B] bool
        or None empties a stream's memory before its token reads (a BOS, :287-289)."""
        squeeze = x.dim() == 3
        x2 = x.reshape(x.shape[0], x.shape[-1]) if squeeze else x
        if not self.enabled:
            return torch.zeros_like(x)
        self._check(x2.unsqueeze(1), None)
        if self._training(x2):
            raise RuntimeError("RunTimeSdm.step is inference only: call it under torch.no_grad() or "
                               "torch.inference_mode()")
        dt = self._compute_dtype(x2)
        with torch.autocast("cuda", enabled=False):
            kz, qz, V, g = self._project(x2.unsqueeze(1), dt, None if hx is None else hx.reshape(x2.shape[0], 1, -1))
            y = self._step_projected(kz, qz, V, g, state, reset, dt, x.dtype)
        return y.reshape(x.shape)

    def _step_projected(self, kz, qz, V, g, state, reset, dt, out_dtype):
        """The step after the projections (kz, qz, V, g: [B, 1, ...] views): the decode step, then wo."""
        wo = self._fused_weight(dt)[2]
        r = core.decode_step(
            kz[:, 0], qz[:, 0], V[:, 0], None if g is None else g[:, 0], state, keys1=self.keys1,
            keys2=self.keys2, log_scale=self.log_scale, decay=self.decay(), addr_b=self.addr_b,
            onorm_w=self.onorm_w if self.out_norm else None, gate_bias=None,
            k=self.k, read_mode=self.read_mode, out_norm=self.out_norm, read_eps=self.read_eps,
            out_norm_eps=self.out_norm_eps, reset=reset, out_dtype=dt, workspace=self._ws,
            params=self._core_params(kz.device))
        y = core.linear(r, wo, as_matmul=True).to(out_dtype)
        if self.keep_picks:   # the addressing kernels on the step's rows: the decode step's own picks
            prm = self._core_params(kz.device)
            self.last_addresses = (kz, qz)
            self.last_projections = (kz, qz, V, g)
            self.last_picks = tuple(
                core.address(z, self.keys1, self.keys2, self.k, self.log_scale, addr_b=self.addr_b,
                             params=prm)[0] for z in (kz, qz))
        return y

    def residual_fits(self, x, y):
        """Whether step_residual serves a step on x + y: bf16 rows of the layer width, few enough for the folded
        map (core.linear_residual_fits on the whole projection buffer), inference."""
        if not self.enabled or x.dim() not in (2, 3) or x.shape[-1] != self.d or x.device.type != "cuda":
            return False
        if x.dtype != torch.bfloat16 or self._training(x) or torch.is_autocast_enabled("cuda"):
            return False
        W, bias = self._fused_weight(torch.bfloat16)[:2]
        return core.linear_residual_fits(x, y, W, bias)

    def step_residual(self, x, y, state, reset=None):
        """step() on the residual stream's next value s = x + y (OneSdmLM's x = x + layer(x) in front of this mixer,
        track4_onesdm_models.py:540-547): the add, the input norm and the whole projection map run in one launch
        (core.linear_residual), bit for bit add_rms_norm followed by step(s, hx=...).  x, y [B, d] (or [B, 1, d])
        bf16 (residual_fits).  Returns (s, out), each of x's shape."""
        if not self.residual_fits(x, y):
            raise ValueError("step_residual: the folded map does not take these rows (see residual_fits)")
        x2 = x.reshape(-1, self.d)
        B = x2.shape[0]
        H, d_a = self.h, self.d_a
        dt = torch.bfloat16
        W, bias = self._fused_weight(dt)[:2]
        ra = self._rows_a()
        s, proj = core.linear_residual(x2, y.reshape(-1, self.d), self.norm.w, self.norm.eps, W, bias)
        proj = proj.view(B, 1, -1)
        pa, V = proj[..., :ra], proj[..., ra:]
        o_q, o_g = H * d_a, 2 * H * d_a
        g = pa[..., o_g:o_g + H] if self.write_gate else None
        out = self._step_projected(pa[..., :o_q], pa[..., o_q:o_g], V, g, state, reset, dt, x.dtype)
        return s.reshape(x.shape), out.reshape(x.shape)

    def embed_fits(self, idx, table):
        """Whether step_embed serves a step on table[idx]: bf16 rows of the layer width, few enough for the folded
        map (core.linear_embed_fits on the whole projection buffer), inference."""
        if not self.enabled or self.d != core.GEMM_ROWS_FOLD_K or self._training(table):
            return False
        if torch.is_autocast_enabled("cuda") or table.dtype != torch.bfloat16:
            return False
        W, bias = self._fused_weight(torch.bfloat16)[:2]
        return core.linear_embed_fits(idx, table, W, bias)

    def step_embed(self, idx, table, state, reset=None):
        """step() on the embedded tokens x = table[idx] (OneSdmLM's embedding in front of its first layer,
        track4_onesdm_models.py:534-535): the gather, the input norm and the whole projection map run in one launch
        (core.linear_embed), bit for bit the gather, rms_norm and step(x, hx=...).  idx [B] int64, table [vocab, d]
        bf16 (embed_fits).  Returns (x, out), each [B, d]."""
        if not self.embed_fits(idx, table):
            raise ValueError("step_embed: the folded map does not take these tokens (see embed_fits)")
        B = idx.shape[0]
        H, d_a = self.h, self.d_a
        dt = torch.bfloat16
        W, bias = self._fused_weight(dt)[:2]
        ra = self._rows_a()
        x, proj = core.linear_embed(idx, table, self.norm.w, self.norm.eps, W, bias)
        proj = proj.view(B, 1, -1)
        pa, V = proj[..., :ra], proj[..., ra:]
        o_q, o_g = H * d_a, 2 * H * d_a
        g = pa[..., o_g:o_g + H] if self.write_gate else None
        out = self._step_projected(pa[..., :o_q], pa[..., o_q:o_g], V, g, state, reset, dt, dt)
        return x, out.reshape(B, self.d)

    def forward_sequential(self, x, reset=None):
        """The token recurrence of the reference (track4_onesdm_models.py:276-300).  It is the same function as
        forward; the HIP core computes it once, so this is forward."""
        return self.forward(x, reset)
