"""Drop-in PathOrderedGeometricMHA backed by the gfx950 HIP kernels.

Usage in the reference's experiment scripts (their plugin API is a module
name resolved with importlib, experiments/session_cherry.py:278,445):

    python session_cherry.py --attn-module holonomyawareattention_amd.attention_kernel

Interface (kernel/attention_fast_chunked.py:43-61, kernel/attention_kernel.py:193-218):
  PathOrderedGeometricMHA(d_model, n_heads=4, dropout=0.0, edge_scale=0.1, mode="causal")
  forward(x (B,L,D), attn_mask (L,L) bool | None, return_geometry=False)
      -> (y (B,L,D), None | {"C": P (B,H,L,d,d), "H": Hol (B,H,d,d)})
  attributes h, d, m_dim, edge_scale, scale, mode, link_mode, qkv, out,
  gqproj, gkproj, edge_mlp, dropout (same state_dict keys).

Rotation model: each head's d dims carry floor(d/3) SO(3) blocks (dims
3b..3b+2); the generator emits m_dim = 3*floor(d/3) link parameters per head,
block b's three being the skew entries (0,1), (0,2), (1,2) of its 3x3 block in
the reference's row-major upper-triangle order (core/utils.py:20-26). Leftover
dims (d mod 3) are not rotated. This is the reference's dense SO(d) model
restricted to block-diagonal generators.

Dispatch follows the reference's kernel module (kernel/attention_kernel.py:
203-213): mode == "causal" with attn_mask exactly tril(L) runs the causal
kernels (holo_attn_fwd; return_geometry is also supported); every other call
-- no mask, the ring mask or any (L, L) boolean mask, inert mode -- runs the
exact-path kernels (holo_attn_masked_fwd), where the reference falls back to
kernel/attention_fast.py. Both need x on the GPU; active attention dropout
(training, dropout > 0) runs on the exact path's dropout kernels when
exact_backward is on and raises otherwise; anything else unsupported raises
NotImplementedError (there is no CPU path).
Under autograd the projections are ordinary differentiable torch GEMMs and the
scan + attention core is one autograd function whose backward is the gfx950
backward (holo_attn_bwd; the reference recomputes its forward under autograd,
kernel/attention_kernel.py:174-187); that backward covers the causal + tril
path. Other calls under autograd (any other mask, inert mode, return_geometry)
run their forward as with gradients off and return outputs whose backward
raises NotImplementedError, unless exact_backward is on: then any mask and
inert mode run the exact path's differentiable pair (holo_attn_masked_train_fwd,
holo_attn_masked_bwd); the geometry output has no gfx950 backward.
"""
from __future__ import annotations

import math
import weakref
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, kernels


class _Verified:
    """Remembers that a tensor passed a check, without keeping it alive: a
    weak reference plus its address and version counter. A later tensor
    matches only if it is the same live object, unmodified since (so a new
    tensor placed at a freed tensor's address never matches)."""

    __slots__ = ("ref", "key")

    def __init__(self, t: torch.Tensor, extra=()):
        self.ref = weakref.ref(t)
        self.key = (t.data_ptr(), t._version, *extra)

    def matches(self, t: torch.Tensor, extra=()) -> bool:
        return self.ref() is t and self.key == (t.data_ptr(), t._version, *extra)


def _is_exact_tril(mask: Optional[torch.Tensor], L: int) -> bool:
    """True iff mask is exactly tril(L) (kernel/attention_kernel.py:193-199)."""
    if mask is None or tuple(mask.shape) != (L, L):
        return False
    tril = torch.ones(L, L, dtype=torch.bool, device=mask.device).tril()
    return torch.equal(mask.bool(), tril)


class _MatmulF32Out(torch.autograd.Function):
    """x2 (N, D) @ w^T with an fp32 output (the generator projections: link
    parameters are never rounded to bf16). The backward rounds the incoming
    fp32 gradient to x's dtype for its two GEMMs."""

    @staticmethod
    def forward(ctx, x2, w):
        ctx.save_for_backward(x2, w)
        if x2.dtype == torch.float32:
            return x2 @ w.t()
        return torch.mm(x2, w.t(), out_dtype=torch.float32)

    @staticmethod
    def backward(ctx, dg):
        x2, w = ctx.saved_tensors
        dgl = dg.to(x2.dtype)
        dx = dgl @ w if ctx.needs_input_grad[0] else None
        dw = dgl.t() @ x2 if ctx.needs_input_grad[1] else None
        return dx, dw


class _ForwardOnly(torch.autograd.Function):
    """Attaches outputs computed without autograd (the exact path, the
    geometry output) to the inputs they depend on: forward returns them
    unchanged, backward raises NotImplementedError, so a forward under autograd
    (e.g. an eval() model outside torch.no_grad()) works and only an actual
    backward through these outputs fails."""

    @staticmethod
    def forward(ctx, what: str, n_out: int, *tensors):
        ctx.what = what
        outs = tuple(t.view_as(t) for t in tensors[:n_out])
        return outs[0] if n_out == 1 else outs

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            f"holonomyawareattention_amd kernel path does not support this call: the gradient of {ctx.what} "
            "(the gfx950 backward covers causal mode with attn_mask == tril(L) and no geometry output)")


class _PathAttention(torch.autograd.Function):
    """o (B,L,H,d) = scan + causal attention + back-rotation of q, k, v (views
    of qkv (B,L,H,3d)) under the links of the fp32 generator output g
    ((B,L,2*H*m) = [gq | gk] for the additive generator, (B,L,H*m) for the
    interaction MLP). Backward: holo_attn_bwd, returning dqkv and dg."""

    @staticmethod
    def forward(ctx, qkv, g, edge_scale, scale, additive, d):
        B, L, H, _ = qkv.shape
        m = 3 * (d // 3)
        gq, gk = _PathAttention._gviews(g, B, L, H, m, additive)
        qh, kh, vh_t, P, _ = kernels.geom_scan(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:],
                                                gq, gk, edge_scale, p_format="f32")
        lse = torch.empty((B, H, qh.shape[2]), dtype=torch.float32, device=qkv.device)
        o = kernels.attention(qh, kh, vh_t, P, d, scale, lse=lse)
        ctx.save_for_backward(g, qh, kh, vh_t, P, lse, o)
        ctx.cfg = (edge_scale, scale, additive, d, H, m, tuple(qkv.shape))
        return o

    @staticmethod
    def _gviews(g, B, L, H, m, additive):
        if additive:
            return g[..., :H * m].view(B, L, H, m), g[..., H * m:].view(B, L, H, m)
        return g.view(B, L, H, m), None

    @staticmethod
    def backward(ctx, do):
        g, qh, kh, vh_t, P, lse, o = ctx.saved_tensors
        es, scale, additive, d, H, m, shp = ctx.cfg
        B, L = shp[0], shp[1]
        dqkv = torch.empty(shp, dtype=o.dtype, device=o.device)
        dg = torch.empty_like(g)
        gq, gk = _PathAttention._gviews(g, B, L, H, m, additive)
        dgq, dgk = _PathAttention._gviews(dg, B, L, H, m, additive)
        kernels.attention_backward(gq, gk, es, qh, kh, vh_t, P, lse, o, do.contiguous(), d, scale,
                                   dqkv[..., :d], dqkv[..., d:2 * d], dqkv[..., 2 * d:], dgq, dgk)
        return dqkv, dg, None, None, None, None


class _ExactPathAttention(torch.autograd.Function):
    """o (B,L,H,d) of the exact path (any mask, causal mode with the wrap
    branch through the holonomy, or inert mode) from the q, k, v views of qkv
    and the fp32 generator output g (layouts of _PathAttention): geom_scan in
    the call's mode + holo_attn_masked_train_fwd. Backward:
    holo_attn_masked_bwd, returning dqkv and dg (the closing edge's share of
    dg included in causal mode). drop = (p, seed) applies attention dropout
    (holo_attn_masked_dropout_fwd / _bwd, the keep mask regenerated from the
    seed in the backward); None = no dropout."""

    @staticmethod
    def forward(ctx, qkv, g, edge_scale, scale, additive, d, mask, mode, drop=None):
        B, L, H, _ = qkv.shape
        m = 3 * (d // 3)
        p, seed = drop if drop is not None else (0.0, 0)
        gq, gk = _PathAttention._gviews(g, B, L, H, m, additive)
        qh, kh, vh_t, P, hol = kernels.geom_scan(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:], gq, gk,
                                                 edge_scale, want_hol=mode == "causal", p_format="f32", mode=mode)
        o, lse = kernels.attention_masked_train(qh, kh, vh_t, P, hol, d, scale, mode=mode, mask=mask,
                                                dropout_p=p, seed=seed)
        ctx.save_for_backward(g, qh, kh, vh_t, P, hol, lse, o, mask)
        ctx.cfg = (edge_scale, scale, additive, d, H, m, tuple(qkv.shape), mode, p, seed)
        return o

    @staticmethod
    def backward(ctx, do):
        g, qh, kh, vh_t, P, hol, lse, o, mask = ctx.saved_tensors
        es, scale, additive, d, H, m, shp, mode, p, seed = ctx.cfg
        B, L = shp[0], shp[1]
        dqkv = torch.empty(shp, dtype=o.dtype, device=o.device)
        dg = torch.empty_like(g)
        gq, gk = _PathAttention._gviews(g, B, L, H, m, additive)
        dgq, dgk = _PathAttention._gviews(dg, B, L, H, m, additive)
        kernels.attention_masked_backward(gq, gk, es, qh, kh, vh_t, P, hol, lse, o, do.contiguous(), d, scale,
                                          dqkv[..., :d], dqkv[..., d:2 * d], dqkv[..., 2 * d:], dgq, dgk,
                                          mode=mode, mask=mask, dropout_p=p, seed=seed)
        return dqkv, dg, None, None, None, None, None, None, None


class PathOrderedGeometricMHA(nn.Module):
    def __init__(self, d_model: int, n_heads: int = 4, dropout: float = 0.0,
                 edge_scale: float = 0.1, mode: str = "causal"):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError("d_model must be divisible by n_heads")
        if mode not in ("causal", "inert"):
            raise ValueError("mode must be 'causal' or 'inert'")
        self.h = n_heads
        self.d = d_model // n_heads
        self.n_blocks = self.d // 3
        self.m_dim = 3 * self.n_blocks
        self.edge_scale = edge_scale
        self.scale = 1.0 / math.sqrt(self.d)
        self.mode = mode

        self.qkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.out = nn.Linear(d_model, d_model, bias=False)
        self.dropout = nn.Dropout(dropout)
        self.gqproj = nn.Linear(d_model, self.m_dim * n_heads, bias=False)
        self.gkproj = nn.Linear(d_model, self.m_dim * n_heads, bias=False)
        self.edge_mlp = nn.Sequential(
            nn.Linear(2 * d_model, 4 * d_model), nn.GELU(),
            nn.Linear(4 * d_model, self.m_dim * n_heads),
        )
        self.link_mode = "interaction"
        # Options of this build (not reference attributes; defaults keep the
        # validated behaviour). fp16_operands: the bf16 inference path stores
        # the transported q, k, v in fp16 (11-bit significands; a value
        # beyond +-65504 becomes inf); False keeps bf16 operands, whose range
        # is fp32's. check_status: read the scan's status word after each
        # inference forward (one host synchronisation) and raise RuntimeError
        # if a carry wait timed out (outputs NaN) or an fp16 operand
        # overflowed; off, the word is never read. fused_interaction: the
        # bf16 interaction generator's edge MLP on the hand-written GEMM
        # (holo_edge_hidden_fwd with q/k/v in the same launch, then
        # holo_gemm_f32out_fwd) instead of torch's GEMMs and GELU; off by
        # default: these two entry points have been executed on the CPU
        # only, never on a GPU. exact_backward: under autograd, calls off the
        # causal + tril path (any other mask, inert mode) run a
        # differentiable exact path (holo_attn_masked_train_fwd and
        # holo_attn_masked_bwd) instead of a forward whose backward raises,
        # and active attention dropout (training, dropout.p > 0) runs there
        # (holo_attn_masked_dropout_fwd / _bwd) as the reference's exact path
        # applies it, instead of raising; off by default for the same reason.
        self.fp16_operands = True
        self.check_status = False
        self.fused_interaction = False
        self.exact_backward = False
        self._wcat_src = None          # _Verified of each weight behind _wcat
        self._wcat = None
        self._mask_ok = None           # _Verified of the last mask found to be tril(L)
        # profiling hook: when set to a sequence of 5 torch.cuda.Event, forward
        # records them on the launch stream around its four stages (link
        # inputs, geometry scan, attention, out-projection); no host sync
        self._stage_events = None

    # ---- dispatch predicate (kernel/attention_kernel.py:203-208) ----
    def _unsupported_reason(self, x, attn_mask, causal_implied: bool = False) -> Optional[str]:
        if not x.is_cuda:
            return "input is not on the GPU"
        if self._dropout_active() and causal_implied:
            return "attention dropout is active (prefill and decode apply none)"
        if self._dropout_active() and not getattr(self, "exact_backward", False):
            return ("attention dropout is active (the exact path's dropout kernels run it when exact_backward "
                    "is on)")
        if x.dtype not in (torch.float32, torch.bfloat16):
            return f"dtype {x.dtype} (float32 and bfloat16 are supported)"
        if self.link_mode not in ("additive", "interaction"):
            return f"link_mode={self.link_mode!r}"
        if causal_implied:                    # prefill / decode: the causal tril path by definition
            return None if self.mode == "causal" else f"mode={self.mode!r} (decode runs the causal mode)"
        L = x.shape[1]
        if attn_mask is not None and (tuple(attn_mask.shape) != (L, L) or attn_mask.device != x.device):
            return f"attn_mask must be an ({L}, {L}) tensor on {x.device}"
        return None

    def _dropout_active(self) -> bool:
        """nn.Dropout(p) on the attention weights acts: training and p > 0."""
        return self.training and self.dropout.p != 0.0

    def _tril_path(self, attn_mask, L: int) -> bool:
        """causal mode with attn_mask exactly tril(L): the reference's kernel
        path (kernel/attention_kernel.py:203-208), here the causal kernels
        with their fused backward. The check runs once per mask tensor: the
        verdict is kept for the same live tensor object while it is unmodified
        (a weak reference plus its version counter, never its address alone)."""
        if self.mode != "causal" or attn_mask is None:
            return False
        if self._mask_ok is not None and self._mask_ok.matches(attn_mask, (tuple(attn_mask.shape),)):
            return True
        if not _is_exact_tril(attn_mask, L):
            return False
        self._mask_ok = _Verified(attn_mask, (tuple(attn_mask.shape),))
        return True

    def _kernel_supported(self, x, attn_mask, return_geometry=False) -> bool:
        """The reference's dispatch predicate (kernel/attention_kernel.py:203-208):
        True for calls on its kernel path (causal + tril, no dropout, GPU).
        Every other GPU call runs the exact-path kernels (holo_attn_masked_fwd)."""
        return self._unsupported_reason(x, attn_mask) is None and self._tril_path(attn_mask, x.shape[1])

    def _cat_weight(self, mods) -> torch.Tensor:
        """Row-concatenated weights of `mods` for one GEMM, rebuilt unless every
        weight is the same live tensor, unmodified, as at the last build."""
        ws = tuple(mod.weight for mod in mods)
        src = self._wcat_src
        if src is None or len(src) != len(ws) or not all(v.matches(w, (w.dtype, w.device, tuple(w.shape)))
                                                         for v, w in zip(src, ws)):
            with torch.no_grad():
                self._wcat = torch.cat([w.detach() for w in ws], dim=0)
            self._wcat_src = tuple(_Verified(w, (w.dtype, w.device, tuple(w.shape))) for w in ws)
        return self._wcat

    def _fused_projection_ok(self, x: torch.Tensor) -> bool:
        """holo_qkvg_proj_fwd's conditions, so that every input it would
        refuse takes the library GEMMs instead: bf16, additive generator, K a
        multiple of 64, output widths multiples of 4, 16-byte aligned pointers
        and row strides, and operands within the kernel's 32-bit buffer
        offsets (M * row stride and max(3D, H*m) * K bf16 elements below
        2 GiB)."""
        if x.dim() != 3:
            return False
        B, L, D = (int(n) for n in x.shape)
        n_gen = self.h * self.m_dim
        ws = (self.qkv.weight, self.gqproj.weight, self.gkproj.weight)
        if not (x.dtype == torch.bfloat16 and self.link_mode == "additive" and D % 64 == 0
                and n_gen % 4 == 0 and n_gen > 0 and x.stride(-1) == 1
                and all(w.dtype == torch.bfloat16 and w.is_contiguous() and w.data_ptr() % 16 == 0 for w in ws)):
            return False
        rs, view = kernels.token_rows_stride(x)
        if view and (x.data_ptr() % 16 != 0 or rs % 8 != 0):
            return False
        return B * L * rs * 2 <= 0x7fffffff and max(3 * D, n_gen) * D * 2 <= 0x7fffffff

    def _fused_interaction_ok(self, x: torch.Tensor) -> bool:
        """The conditions of holo_edge_hidden_fwd and holo_gemm_f32out_fwd
        for the interaction generator (fused_interaction on): bf16, the edge
        MLP as built (Linear with bias, exact GELU, Linear), contiguous
        16-byte aligned bf16 weights, D a multiple of 64, and every operand
        within the kernels' 32-bit buffer offsets (weights counted to the end
        of their last 256-row tile)."""
        if not (getattr(self, "fused_interaction", False) and self.link_mode == "interaction" and x.dim() == 3):
            return False
        B, L, D = (int(n) for n in x.shape)
        l1, act, l2 = self.edge_mlp[0], self.edge_mlp[1], self.edge_mlp[2]
        n_gen = self.h * self.m_dim
        if not (isinstance(act, nn.GELU) and act.approximate == "none" and l1.bias is not None):
            return False
        ws = (self.qkv.weight, l1.weight, l1.bias, l2.weight)
        if not (x.dtype == torch.bfloat16 and D % 64 == 0 and n_gen % 4 == 0 and x.stride(-1) == 1
                and tuple(l1.weight.shape) == (4 * D, 2 * D) and tuple(l2.weight.shape) == (n_gen, 4 * D)
                and all(w.dtype == torch.bfloat16 and w.is_contiguous() and w.data_ptr() % 16 == 0 for w in ws)):
            return False
        rs, view = kernels.token_rows_stride(x)
        if view and (x.data_ptr() % 16 != 0 or rs % 8 != 0):
            return False
        tile = lambda n: (n + 255) // 256 * 256
        lim = 0x7fffffff
        return (B * L * rs * 2 <= lim and 3 * D * D * 2 <= lim and tile(4 * D) * 2 * D * 2 <= lim
                and B * L * 4 * D * 2 <= lim and tile(n_gen) * 4 * D * 2 <= lim)

    def _link_inputs(self, x: torch.Tensor, fused: bool = False):
        """q, k, v views (B,L,H,d) and generator views gq, gk (B,L,H,m).

        The generator leaves the GEMM in fp32 whatever x's dtype: link angle
        errors accumulate along the path, so the link parameters are never
        rounded to bf16 (additive: one extra GEMM with an fp32 output;
        interaction: the edge MLP's last layer). fused=True (bf16, additive)
        runs q/k/v and the generator as one hand-written GEMM
        (holo_qkvg_proj_fwd) that returns gq = g_t = gq(x_t) + gk(x_{t+1})
        and gk = None: the scan's direct mode, a_t = edge_scale * g_t. With
        fused=True and fused_interaction on (bf16, interaction), q/k/v and the
        edge MLP run on holo_edge_hidden_fwd and holo_gemm_f32out_fwd."""
        B, L, D = x.shape
        H, d, m = self.h, self.d, self.m_dim
        if fused and self._fused_projection_ok(x):
            qkv, g = kernels.qkvg_projection(x, self.qkv.weight, self.gqproj.weight, self.gkproj.weight)
            qkv = qkv.view(B, L, H, 3 * d)
            return qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:], g.view(B, L, H, m), None
        x2 = x.reshape(B * L, D)
        if self.link_mode == "additive":
            if x.dtype == torch.float32:
                y5 = F.linear(x, self._cat_weight((self.qkv, self.gqproj, self.gkproj)))
                qkv = y5[..., :3 * D].view(B, L, H, 3 * d)
                g = y5[..., 3 * D:]
            else:
                qkv = F.linear(x, self.qkv.weight).view(B, L, H, 3 * d)
                wg = self._cat_weight((self.gqproj, self.gkproj))
                g = torch.mm(x2, wg.t(), out_dtype=torch.float32).view(B, L, 2 * H * m)
            gq = g[..., :H * m].view(B, L, H, m)
            gk = g[..., H * m:].view(B, L, H, m)
        elif fused and self._fused_interaction_ok(x):
            qkv, hid = kernels.edge_hidden(x, self.qkv.weight, self.edge_mlp[0].weight, self.edge_mlp[0].bias)
            qkv = qkv.view(B, L, H, 3 * d)
            lin2 = self.edge_mlp[2]
            gq = kernels.edge_out(hid, lin2.weight).view(B, L, H, m)
            gk = None if lin2.bias is None else lin2.bias.detach().float().view(1, 1, H, m).expand(B, L, H, m)
        else:
            qkv = F.linear(x, self.qkv.weight).view(B, L, H, 3 * d)
            hid = self.edge_mlp[1](self.edge_mlp[0](self._pairs(x))).reshape(B * L, 4 * D)
            lin2 = self.edge_mlp[2]
            if x.dtype == torch.float32:
                gq = F.linear(hid, lin2.weight).view(B, L, H, m)
            else:
                gq = torch.mm(hid, lin2.weight.t(), out_dtype=torch.float32).view(B, L, H, m)
            if lin2.bias is not None:   # a_t = es * (g_t + bias): the scan adds the bias per head
                gk = lin2.bias.detach().float().view(1, 1, H, m).expand(B, L, H, m)
            else:
                gk = None
        return qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:], gq, gk

    @staticmethod
    def _pairs(x: torch.Tensor) -> torch.Tensor:
        """[x_t ; x_{(t+1) mod L}] (B, L, 2D), the edge MLP's input
        (core/attention_fast_chunked.py:74-75), written in two copies."""
        B, L, D = x.shape
        pair = torch.empty((B, L, 2 * D), dtype=x.dtype, device=x.device)
        pair[..., :D] = x
        pair[:, :L - 1, D:] = x[:, 1:]
        pair[:, L - 1, D:] = x[:, 0]
        return pair

    def _edge_params(self, pair: torch.Tensor) -> torch.Tensor:
        """Interaction generator on (..., 2D) pairs [x_t ; x_{t+1}]
        (core/attention_fast_chunked.py:73-77): (N, H*m) with the last layer
        written in fp32 (differentiable)."""
        hid = self.edge_mlp[1](self.edge_mlp[0](pair)).reshape(-1, 4 * self.h * self.d)
        lin2 = self.edge_mlp[2]
        if pair.dtype == torch.float32:
            return F.linear(hid, lin2.weight, lin2.bias)
        g = _MatmulF32Out.apply(hid, lin2.weight)
        if lin2.bias is not None:
            g = g + lin2.bias.float()
        return g

    def _forward_autograd(self, x: torch.Tensor, exact_mask: Optional[Tuple[Optional[torch.Tensor]]] = None,
                          drop: Optional[Tuple[float, int]] = None) -> torch.Tensor:
        """Differentiable forward: torch GEMMs for the projections and the
        generator, _PathAttention for the core (causal + tril) or, with
        exact_mask = (attn_mask,), _ExactPathAttention (the exact path in the
        module's mode, attn_mask None = every pair; drop = (p, seed): with
        attention dropout)."""
        B, L, D = x.shape
        H, d, m = self.h, self.d, self.m_dim
        qkv = F.linear(x, self.qkv.weight).view(B, L, H, 3 * d)
        additive = self.link_mode == "additive"
        if additive:
            wg = torch.cat([self.gqproj.weight, self.gkproj.weight], 0)
            g = _MatmulF32Out.apply(x.reshape(B * L, D), wg).view(B, L, 2 * H * m)
        else:
            pair = torch.cat([x, torch.roll(x, shifts=-1, dims=1)], dim=-1)
            g = self._edge_params(pair).view(B, L, H * m)
        if exact_mask is not None:
            mask = exact_mask[0]
            mask = None if mask is None else mask.detach().to(torch.bool)
            o = _ExactPathAttention.apply(qkv, g, self.edge_scale, self.scale, additive, d, mask, self.mode, drop)
        else:
            o = _PathAttention.apply(qkv, g, self.edge_scale, self.scale, additive, d)
        return F.linear(o.reshape(B, L, D), self.out.weight)

    def _op_dtype(self, x: torch.Tensor) -> torch.dtype:
        """Operand type of the transported q, k, v on the causal inference
        path: fp16 for bf16 activations (11-bit significands on the matrix
        cores at the bf16 rate; the parity bar needs them) unless
        fp16_operands is off, fp32 otherwise."""
        if x.dtype == torch.bfloat16 and getattr(self, "fp16_operands", True):
            return torch.float16
        return x.dtype

    def _status_word(self, device: torch.device) -> Optional[torch.Tensor]:
        """A one-element int32 device tensor for the scan's status word when
        check_status is on, else None (the word is never copied or read)."""
        return torch.zeros(1, dtype=torch.int32, device=device) if getattr(self, "check_status", False) else None

    @staticmethod
    def _raise_on_status(status: Optional[torch.Tensor]) -> None:
        """Reads the status word (a host synchronisation) and raises for any
        bit set: HOLO_WS_TIMEOUT (a chained carry wait ran out of polls; the
        outputs are NaN) or HOLO_WS_OVERFLOW (a transported value exceeded
        fp16's range and was stored as inf)."""
        if status is None:
            return
        word = int(status.item())
        if word == 0:
            return
        what = []
        if word & _lib.HOLO_WS_TIMEOUT:
            what.append("a chained carry wait timed out (outputs NaN)")
        if word & _lib.HOLO_WS_OVERFLOW:
            what.append("a transported q/k/v value exceeded fp16's range (stored as inf; "
                        "set fp16_operands = False to keep bf16 operands)")
        raise RuntimeError(f"holonomyawareattention_amd: scan status 0x{word:x}: " + "; ".join(what or ["unknown bits"]))

    @staticmethod
    def _p_format(x: torch.Tensor, return_geometry: bool) -> str:
        """Storage of the prefix rotations between the scan and the attention
        epilogue: int16 quaternions (half the bytes, quantisation ~6e-5 of a
        rotated vector, well below bf16 rounding) on the bf16 path, fp32 for
        fp32 runs and whenever the geometry is returned."""
        return "snorm16" if x.dtype == torch.bfloat16 and not return_geometry else "f32"

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                return_geometry: bool = False
                ) -> Tuple[torch.Tensor, Optional[Dict[str, torch.Tensor]]]:
        reason = self._unsupported_reason(x, attn_mask)
        if reason is not None:
            raise NotImplementedError(
                f"holonomyawareattention_amd kernel path does not support this call: {reason}")
        B, L, D = x.shape
        if self._dropout_active():
            return self._forward_dropout(x, attn_mask, return_geometry)
        tril = self._tril_path(attn_mask, L)
        params = [p for p in self.parameters() if p.requires_grad]
        track = torch.is_grad_enabled() and (x.requires_grad or bool(params))
        if track:
            if tril and not return_geometry:
                return self._forward_autograd(x), None
            if not tril and not return_geometry and getattr(self, "exact_backward", False):
                return self._forward_autograd(x, exact_mask=(attn_mask,)), None
            with torch.no_grad():
                y, geo = self._forward_exact(x, attn_mask, return_geometry) if not tril else \
                    self._forward_kernels(x, True)
            what = "the geometry output" if tril else \
                ("inert mode" if self.mode != "causal" else "an attention mask other than tril(L)")
            deps = [x] + params
            if geo is None:
                return _ForwardOnly.apply(what, 1, y, *deps), None
            y, C, Hm = _ForwardOnly.apply(what, 3, y, geo["C"], geo["H"], *deps)
            return y, {"C": C, "H": Hm}
        if not tril:
            return self._forward_exact(x, attn_mask, return_geometry)
        return self._forward_kernels(x, return_geometry)

    def _forward_dropout(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor], return_geometry: bool
                         ) -> Tuple[torch.Tensor, Optional[Dict[str, torch.Tensor]]]:
        """Active attention dropout (exact_backward on): as the reference's
        kernel module sends such calls to its exact path
        (kernel/attention_kernel.py:203-213 -> kernel/attention_fast.py:160),
        every mask -- tril(L) included -- runs the exact path's differentiable
        pair with dropout (holo_attn_masked_dropout_fwd / _bwd). The keep mask
        comes from a fresh 64-bit seed drawn from torch's default CPU
        generator (so torch.manual_seed makes it repeatable) and is
        regenerated by the backward. The geometry output (return_geometry)
        does not depend on dropout; it comes from a separate forward without
        gradients, as elsewhere."""
        seed = int(torch.randint(0, 2 ** 63 - 1, (), dtype=torch.int64).item())
        y = self._forward_autograd(x, exact_mask=(attn_mask,), drop=(float(self.dropout.p), seed))
        if not return_geometry:
            return y, None
        with torch.no_grad():
            _, geo = self._forward_exact(x, attn_mask, True)
        params = [p for p in self.parameters() if p.requires_grad]
        if torch.is_grad_enabled() and (x.requires_grad or bool(params)):
            C, Hm = _ForwardOnly.apply("the geometry output", 2, geo["C"], geo["H"], x, *params)
            geo = {"C": C, "H": Hm}
        return y, geo

    def _forward_kernels(self, x: torch.Tensor, return_geometry: bool
                         ) -> Tuple[torch.Tensor, Optional[Dict[str, torch.Tensor]]]:
        """The causal + tril forward on the gfx950 kernels, without autograd."""
        B, L, D = x.shape
        ev = self._stage_events
        with torch.no_grad():
            if ev is not None:
                ev[0].record()
            q, k, v, gq, gk = self._link_inputs(x, fused=True)
            if ev is not None:
                ev[1].record()
            status = self._status_word(x.device)
            qh, kh, vh_t, P, hol = kernels.geom_scan(q, k, v, gq, gk, self.edge_scale,
                                                     want_hol=return_geometry,
                                                     p_format=self._p_format(x, return_geometry),
                                                     op_dtype=self._op_dtype(x), status=status)
            if ev is not None:
                ev[2].record()
            o = kernels.attention(qh, kh, vh_t, P, self.d, self.scale, out_dtype=x.dtype)
            if ev is not None:
                ev[3].record()
            y = F.linear(o.view(B, L, D), self.out.weight)
            if ev is not None:
                ev[4].record()
        self._raise_on_status(status)
        if not return_geometry:
            return y, None
        d = self.d
        C = kernels.quat_to_dense(P, d).to(x.dtype)
        Hm = kernels.quat_to_dense(hol, d).to(x.dtype)
        return y, {"C": C, "H": Hm}

    def _forward_exact(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor], return_geometry: bool
                       ) -> Tuple[torch.Tensor, Optional[Dict[str, torch.Tensor]]]:
        """Every call off the causal + tril path: any mask (None = every pair,
        e.g. the ring mask of core/utils.py:59-75), causal mode (the wrap branch
        through the holonomy) or inert mode, as the reference's kernel module
        runs them on its exact path (kernel/attention_kernel.py:211-213 ->
        kernel/attention_fast.py:129-166). Rows whose mask allows no key are NaN,
        as there."""
        B, L, D = x.shape
        causal = self.mode == "causal"
        ev = self._stage_events
        with torch.no_grad():
            if ev is not None:
                ev[0].record()
            q, k, v, gq, gk = self._link_inputs(x, fused=True)
            if ev is not None:
                ev[1].record()
            status = self._status_word(x.device)
            qh, kh, vh_t, P, hol = kernels.geom_scan(q, k, v, gq, gk, self.edge_scale,
                                                     want_hol=causal or return_geometry,
                                                     p_format=self._p_format(x, return_geometry),
                                                     mode=self.mode, status=status)
            if ev is not None:
                ev[2].record()
            o = kernels.attention_masked(qh, kh, vh_t, P, hol, self.d, self.scale, mode=self.mode,
                                         mask=attn_mask)
            if ev is not None:
                ev[3].record()
            y = F.linear(o.view(B, L, D), self.out.weight)
            if ev is not None:
                ev[4].record()
        self._raise_on_status(status)
        if not return_geometry:
            return y, None
        C = kernels.quat_to_dense(P, self.d).to(x.dtype)
        Hm = kernels.quat_to_dense(hol, self.d).to(x.dtype)
        return y, {"C": C, "H": Hm}

    # ---- incremental decode (no counterpart in the reference) ----
    def prefill(self, x: torch.Tensor, capacity: Optional[int] = None) -> Tuple[torch.Tensor, "DecodeState"]:
        """Causal forward of the prefix x (B, T, D) -- the same kernels as
        `forward` -- plus the state that `decode_step` continues from: the
        prefix's transported keys and values (global frame) in caches of
        `capacity` positions (default T + 256, rounded up to 64), P_{T-1} and
        the link inputs of token T-1."""
        reason = self._unsupported_reason(x, None, causal_implied=True)
        if reason is not None:
            raise NotImplementedError(f"holonomyawareattention_amd prefill: {reason}")
        B, T, D = x.shape
        H, d = self.h, self.d
        cap = T + 256 if capacity is None else int(capacity)
        cap = (max(cap, T + 1) + 63) // 64 * 64
        with torch.no_grad():
            q, k, v, gq, gk = self._link_inputs(x)
            qh, kh, vh_t, P, _ = kernels.geom_scan(q, k, v, gq, gk, self.edge_scale, p_format="f32")
            o = kernels.attention(qh, kh, vh_t, P, d, self.scale)
            y = F.linear(o.view(B, T, D), self.out.weight)
            Dp, Tp = kh.shape[-1], kh.shape[2]
            kc = torch.zeros((B, H, cap, Dp), dtype=x.dtype, device=x.device)
            vc = torch.zeros((B, H, cap // 64, Dp, 64), dtype=x.dtype, device=x.device)
            kc[:, :, :Tp] = kh
            vc[:, :, :Tp // 64] = vh_t
            st = DecodeState(kc, vc, P[:, :, T - 1].contiguous(), T,
                             gq[:, T - 1].contiguous() if self.link_mode == "additive" else x[:, T - 1].clone())
        return y, st

    def decode_step(self, x_t: torch.Tensor, state: "DecodeState") -> torch.Tensor:
        """Output (B, 1, D) for the next token x_t (B, 1, D) after the tokens in
        `state` (from `prefill` or earlier steps); equals row t of `forward`
        over the whole sequence. Updates `state`."""
        B, L, D = x_t.shape
        if L != 1:
            raise ValueError("decode_step takes one token per sequence (B, 1, D)")
        if self._dropout_active():
            raise NotImplementedError("holonomyawareattention_amd decode_step: attention dropout is active "
                                      "(prefill and decode apply none)")
        t = state.t
        if t >= state.capacity:
            raise ValueError(f"decode cache full ({state.capacity} positions)")
        H, d = self.h, self.d
        with torch.no_grad():
            if self.link_mode == "additive":
                q, k, v, gq, gk = self._link_inputs(x_t)
                kernels.decode_geom(q[:, 0], k[:, 0], v[:, 0], state.g_prev, gk[:, 0], self.edge_scale, t,
                                    state.P, state.qh, state.kh, state.vh)
                state.g_prev = gq[:, 0].contiguous()
            else:
                qkv = F.linear(x_t, self.qkv.weight).view(B, H, 3 * d)
                g = self._edge_params(torch.cat([state.g_prev, x_t[:, 0]], dim=-1)).view(B, H, self.m_dim)
                kernels.decode_geom(qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:], g, None,
                                    self.edge_scale, t, state.P, state.qh, state.kh, state.vh)
                state.g_prev = x_t[:, 0].clone()
            if state.workspace is None:        # sized once for the last position of the cache
                n = kernels.decode_workspace_bytes(B, H, d, state.capacity - 1)
                state.workspace = torch.empty(max(n, 16), dtype=torch.uint8, device=x_t.device)
            o = kernels.decode_attention(state.qh, state.kh, state.vh, state.P, t, d, self.scale,
                                         workspace=state.workspace)
            y = F.linear(o.view(B, 1, D), self.out.weight)
        state.t = t + 1
        return y


class DecodeState:
    """Caches and running geometry of `PathOrderedGeometricMHA.decode_step`:
    kh (B, H, capacity, Dp) and vh (B, H, capacity/64, Dp, 64) transported keys
    and values in the frame of token 0, P (B, H, nb, 4) fp32 = P_{t-1}, t = the
    next token's position, g_prev = the link inputs of token t-1 (gq in
    additive mode, x_{t-1} in interaction mode)."""

    def __init__(self, kh, vh, P, t, g_prev):
        self.kh, self.vh, self.P, self.t, self.g_prev = kh, vh, P, t, g_prev
        self.capacity = int(kh.shape[2])
        self.qh = torch.empty((kh.shape[0], kh.shape[1], kh.shape[3]), dtype=kh.dtype, device=kh.device)
        self.workspace = None
