"""Host-side behaviour of the drop-in module: constructor, attributes,
state_dict keys, dispatch predicate and the errors of unsupported calls."""
from __future__ import annotations

import math

import pytest
import torch

from holonomyawareattention_amd.attention_kernel import PathOrderedGeometricMHA, _is_exact_tril

REFERENCE_KEYS = {"qkv.weight", "out.weight", "gqproj.weight", "gkproj.weight",
                  "edge_mlp.0.weight", "edge_mlp.0.bias", "edge_mlp.2.weight", "edge_mlp.2.bias"}


def test_constructor_mirrors_reference():
    m = PathOrderedGeometricMHA(192, n_heads=4, edge_scale=0.05)
    assert (m.h, m.d, m.n_blocks, m.m_dim) == (4, 48, 16, 48)
    assert m.scale == pytest.approx(1 / math.sqrt(48))
    assert m.mode == "causal" and m.link_mode == "interaction" and m.edge_scale == 0.05
    assert set(m.state_dict()) == REFERENCE_KEYS
    assert tuple(m.gqproj.weight.shape) == (4 * 48, 192)
    assert tuple(m.edge_mlp[2].weight.shape) == (4 * 48, 4 * 192)
    m16 = PathOrderedGeometricMHA(64, n_heads=4)          # d = 16: five blocks, one free dim
    assert (m16.n_blocks, m16.m_dim) == (5, 15)
    with pytest.raises(ValueError):
        PathOrderedGeometricMHA(100, n_heads=3)
    with pytest.raises(ValueError):
        PathOrderedGeometricMHA(96, n_heads=2, mode="ring")


def test_exact_tril_predicate():
    T = 7
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    assert _is_exact_tril(tril, T)
    assert not _is_exact_tril(None, T)
    assert not _is_exact_tril(tril[:-1, :-1], T)
    ring = tril.clone(); ring[0, T - 1] = True
    assert not _is_exact_tril(ring, T)
    assert _is_exact_tril(tril.int(), T)


def test_dispatch_between_tril_and_exact_paths():
    """causal + exactly tril(L) is the reference's kernel path
    (kernel/attention_kernel.py:203-208); every other mask or mode goes to the
    exact-path kernels (its kernel/attention_fast.py fallback)."""
    T = 9
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    ring = tril.clone(); ring[0, T - 1] = True
    causal = PathOrderedGeometricMHA(24, n_heads=2)
    inert = PathOrderedGeometricMHA(24, n_heads=2, mode="inert")
    assert causal._tril_path(tril, T)
    assert causal._tril_path(tril, T)                     # cached by tensor identity
    assert not causal._tril_path(None, T) and not causal._tril_path(ring, T)
    assert not inert._tril_path(tril, T)


@pytest.mark.parametrize("kind", ["cpu", "inert", "nomask", "ring", "dropout", "dtype"])
def test_unsupported_calls_raise(kind):
    """No CPU path, and no attention dropout unless exact_backward is on: such
    calls raise NotImplementedError (the guarded reference's exception,
    kernel/attention_fast_chunked.py:106-114) whatever the mask and mode."""
    T = 6
    m = PathOrderedGeometricMHA(24, n_heads=2, mode="inert" if kind == "inert" else "causal",
                                dropout=0.1 if kind == "dropout" else 0.0)
    x = torch.randn(1, T, 24, dtype=torch.float16 if kind == "dtype" else torch.float32)
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    if kind == "nomask":
        mask = None
    if kind == "ring":
        mask = mask.clone(); mask[0, T - 1] = True
    if kind == "dropout":
        m.train()
    with pytest.raises(NotImplementedError):
        m(x, attn_mask=mask)
    assert not m._kernel_supported(x, mask)


def test_forward_only_outputs_raise_on_backward():
    """The outputs of calls with no gfx950 backward (exact path, geometry
    output) pass through unchanged and keep the graph to x and the parameters;
    backward raises NotImplementedError naming the call."""
    from holonomyawareattention_amd.attention_kernel import _ForwardOnly
    x = torch.randn(2, 3, requires_grad=True)
    w = torch.nn.Parameter(torch.randn(3))
    y0, c0 = torch.randn(2, 3), torch.randn(4)
    y = _ForwardOnly.apply("inert mode", 1, y0, x, w)
    assert y.requires_grad and torch.equal(y.detach(), y0)
    with pytest.raises(NotImplementedError, match="inert mode"):
        y.sum().backward()
    y, c = _ForwardOnly.apply("the geometry output", 2, y0, c0, x, w)
    assert torch.equal(y.detach(), y0) and torch.equal(c.detach(), c0) and c.requires_grad
    with pytest.raises(NotImplementedError, match="geometry output"):
        (y.sum() + c.sum()).backward()
    with torch.no_grad():
        y = _ForwardOnly.apply("x", 1, y0, x, w)
    assert not y.requires_grad


def test_fused_projection_predicate_follows_the_abi_limits():
    """Inputs the hand-written projection GEMM refuses (holo_qkvg_proj_fwd:
    row strides not a multiple of 8 elements, operands above its 32-bit buffer
    offsets) take the library GEMMs instead of raising. The large inputs are
    never written (torch.empty leaves the pages untouched): only the
    metadata is read."""
    D, H = 1536, 16
    m = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=0.05).to(torch.bfloat16)
    m.link_mode = "additive"
    big = lambda B, T: torch.empty(B, T, D, dtype=torch.bfloat16)
    assert m._fused_projection_ok(torch.empty(2, 8, D, dtype=torch.bfloat16))
    assert m._fused_projection_ok(big(64, 8192))                      # 1.61e9 bytes of x: inside
    assert not m._fused_projection_ok(big(128, 8192))                 # 3.2e9 bytes: beyond 2 GiB
    assert not m._fused_projection_ok(torch.empty(2, 8, D + 4, dtype=torch.bfloat16)[..., :D])  # row stride 1540
    assert m._fused_projection_ok(torch.empty(2, 8, D + 8, dtype=torch.bfloat16)[..., :D])      # row stride 1544
    assert m._fused_projection_ok(torch.empty(2, 9, D, dtype=torch.bfloat16)[:, ::2])           # copied rows
    assert not m._fused_projection_ok(torch.empty(2, 8, D, dtype=torch.bfloat16)[..., 1:D - 63])  # D' % 64 != 0
    m.link_mode = "interaction"
    assert not m._fused_projection_ok(torch.empty(2, 8, D, dtype=torch.bfloat16))
    m32 = PathOrderedGeometricMHA(D, n_heads=H)
    m32.link_mode = "additive"
    assert not m32._fused_projection_ok(torch.empty(2, 8, D))


def test_fused_interaction_predicate_follows_the_abi_limits():
    """fused_interaction is off by default; on, the interaction generator
    takes holo_edge_hidden_fwd / holo_gemm_f32out_fwd only where their
    conditions hold (bf16, exact GELU with a first-layer bias, widths
    multiples of 4, the hidden activations within 2 GiB); every other input
    keeps the library GEMMs. Metadata only: the large inputs are never
    written."""
    D, H = 1536, 16
    m = PathOrderedGeometricMHA(D, n_heads=H, edge_scale=0.05).to(torch.bfloat16)
    x = torch.empty(2, 8, D, dtype=torch.bfloat16)
    assert m.fused_interaction is False and not m._fused_interaction_ok(x)
    m.fused_interaction = True
    assert m._fused_interaction_ok(x)
    big = lambda B, T: torch.empty(B, T, D, dtype=torch.bfloat16)
    assert m._fused_interaction_ok(big(16, 8192))             # hidden (131072, 6144) bf16: 1.61e9 bytes
    assert not m._fused_interaction_ok(big(32, 8192))         # 3.2e9 bytes: beyond 2 GiB
    assert not m._fused_interaction_ok(torch.empty(2, 8, D + 4, dtype=torch.bfloat16)[..., :D])
    m.link_mode = "additive"
    assert not m._fused_interaction_ok(x)
    m.link_mode = "interaction"
    m.edge_mlp[1] = torch.nn.GELU(approximate="tanh")
    assert not m._fused_interaction_ok(x)
    m.edge_mlp[1] = torch.nn.GELU()
    assert m._fused_interaction_ok(x)
    assert not m._fused_interaction_ok(x.float())
    m2 = PathOrderedGeometricMHA(128, n_heads=2).to(torch.bfloat16)      # H*m = 2*63: not a multiple of 4
    m2.fused_interaction = True
    assert not m2._fused_interaction_ok(torch.empty(2, 8, 128, dtype=torch.bfloat16))
    m4 = PathOrderedGeometricMHA(128, n_heads=4).to(torch.bfloat16)      # H*m = 4*30
    m4.fused_interaction = True
    assert m4._fused_interaction_ok(torch.empty(2, 8, 128, dtype=torch.bfloat16))


def test_fused_interaction_reaches_the_edge_gemms(monkeypatch):
    """With fused_interaction on, the kernel path's link inputs come from
    kernels.edge_hidden (q/k/v + hidden layer) and kernels.edge_out (g, fp32),
    with the second layer's bias handed to the scan as a per-head constant
    (gk with row stride 0). Stand-ins record the calls (no GPU here)."""
    from holonomyawareattention_amd import attention_kernel as AK
    B, T, D, H = 2, 6, 128, 4
    calls = []

    def fake_hidden(x, w_qkv, w1, b1):
        calls.append(("hidden", w_qkv is m.qkv.weight, w1 is m.edge_mlp[0].weight, b1 is m.edge_mlp[0].bias))
        return (torch.arange(B * T * 3 * D, dtype=torch.float32).reshape(B, T, 3 * D).to(torch.bfloat16),
                torch.zeros(B, T, 4 * D, dtype=torch.bfloat16))

    def fake_out(hid, w2):
        calls.append(("out", tuple(hid.shape), w2 is m.edge_mlp[2].weight))
        return torch.ones(B, T, H * m.m_dim)

    monkeypatch.setattr(AK.kernels, "edge_hidden", fake_hidden)
    monkeypatch.setattr(AK.kernels, "edge_out", fake_out)
    m = PathOrderedGeometricMHA(D, n_heads=H).to(torch.bfloat16)
    m.fused_interaction = True
    x = torch.randn(B, T, D).to(torch.bfloat16)
    q, k, v, gq, gk = m._link_inputs(x, fused=True)
    assert calls == [("hidden", True, True, True), ("out", (B, T, 4 * D), True)]
    d = D // H
    qkv = torch.arange(B * T * 3 * D, dtype=torch.float32).reshape(B, T, H, 3 * d).to(torch.bfloat16)
    assert torch.equal(q, qkv[..., :d]) and torch.equal(k, qkv[..., d:2 * d]) and torch.equal(v, qkv[..., 2 * d:])
    assert gq.dtype == torch.float32 and tuple(gq.shape) == (B, T, H, m.m_dim)
    assert gk.stride()[:2] == (0, 0) and torch.equal(gk[0, 0], m.edge_mlp[2].bias.float().view(H, m.m_dim))


def test_status_word_and_operand_options_reach_the_scan(monkeypatch):
    """check_status passes a status word to the scan and raises on any bit
    the scan set (carry time-out, fp16 overflow); off, no word is passed.
    fp16_operands=False keeps bf16 operands on the bf16 path. The kernel
    wrappers are replaced by stand-ins that record their arguments (no GPU
    here); only the module's plumbing is under test."""
    from holonomyawareattention_amd import attention_kernel as AK, _lib
    B, T, D, H = 1, 5, 24, 2
    seen = {}

    def fake_scan(q, k, v, gq, gk, es, want_hol=False, p_format="f32", mode="causal", op_dtype=None,
                  status=None, static_scratch=False):
        seen["status"], seen["op_dtype"] = status, op_dtype
        if status is not None:
            status.fill_(seen.get("word", 0))
        return None, None, None, None, None

    def fake_attention(qh, kh, vh_t, P, d, scale, out=None, lse=None, out_dtype=None):
        return torch.zeros(B, T, H, d, dtype=out_dtype or torch.float32)

    monkeypatch.setattr(AK.kernels, "geom_scan", fake_scan)
    monkeypatch.setattr(AK.kernels, "attention", fake_attention)
    m = PathOrderedGeometricMHA(D, n_heads=H).eval()
    m.link_mode = "additive"
    x = torch.randn(B, T, D)
    m._forward_kernels(x, False)
    assert seen["status"] is None and seen["op_dtype"] == torch.float32
    m.check_status = True
    m._forward_kernels(x, False)
    assert seen["status"] is not None and seen["status"].dtype == torch.int32
    for word, needle in ((_lib.HOLO_WS_OVERFLOW, "fp16"), (_lib.HOLO_WS_TIMEOUT, "timed out")):
        seen["word"] = word
        with pytest.raises(RuntimeError, match=needle):
            m._forward_kernels(x, False)
    xb = torch.randn(B, T, D).to(torch.bfloat16)
    assert m._op_dtype(xb) == torch.float16
    m.fp16_operands = False
    assert m._op_dtype(xb) == torch.bfloat16 and m._op_dtype(x) == torch.float32


def test_exact_backward_option_routes_autograd_through_the_exact_path(monkeypatch):
    """exact_backward on: a call off the causal + tril path under autograd
    runs _ExactPathAttention, whose forward takes the scan in the module's
    mode and holo_attn_masked_train_fwd, and whose backward takes
    holo_attn_masked_bwd with the same mode, mask and saved state; gradients
    then reach the weights. Off (the default): the forward-only outputs'
    backward raises. Stand-ins for the kernel wrappers (no GPU here)."""
    from holonomyawareattention_amd import attention_kernel as AK
    B, T, D, H = 1, 6, 24, 2
    d = D // H
    seen = {}

    def fake_scan(q, k, v, gq, gk, es, want_hol=False, p_format="f32", mode="causal", op_dtype=None,
                  status=None, static_scratch=False):
        seen["scan"] = (mode, want_hol, p_format, gk is None)
        P = torch.zeros(B, H, T, d // 3, 4)
        hol = torch.zeros(B, H, d // 3, 4) if want_hol else None
        return torch.zeros(1), torch.zeros(1), torch.zeros(1), P, hol

    def fake_train(qh, kh, vh_t, P, hol, d_, scale, mode="causal", mask=None, dropout_p=0.0, seed=0, offset=0):
        seen["train"] = (mode, None if mask is None else mask.clone(), hol is not None)
        seen["train_drop"] = (dropout_p, seed, offset)
        return torch.ones(B, T, H, d_), torch.zeros(B, H, 64)

    def fake_bwd(gq, gk, es, qh, kh, vh_t, P, hol, lse, o, dout, d_, scale, dq, dk, dv, dgq, dgk, mode="causal",
                 mask=None, workspace=None, dropout_p=0.0, seed=0, offset=0):
        seen["bwd"] = (mode, None if mask is None else mask.clone(), tuple(dout.shape))
        seen["bwd_drop"] = (dropout_p, seed, offset)
        for t in (dq, dk, dv, dgq) + ((dgk,) if dgk is not None else ()):
            t.fill_(1.0)

    monkeypatch.setattr(AK.kernels, "geom_scan", fake_scan)
    monkeypatch.setattr(AK.kernels, "attention_masked_train", fake_train)
    monkeypatch.setattr(AK.kernels, "attention_masked_backward", fake_bwd)
    ring = torch.zeros(T, T, dtype=torch.bool)
    for i in range(T):
        ring[i, [i, (i - 1) % T, (i + 1) % T]] = True
    for mode, link in (("causal", "additive"), ("inert", "interaction")):
        seen.clear()
        m = PathOrderedGeometricMHA(D, n_heads=H, mode=mode)
        m.link_mode = link
        m.exact_backward = True
        x = torch.randn(B, T, D, requires_grad=True)
        y = m._forward_autograd(x, exact_mask=(ring,))
        assert seen["scan"] == (mode, mode == "causal", "f32", link == "interaction")
        assert seen["train"][0] == mode and torch.equal(seen["train"][1], ring) and seen["train"][2] == (mode == "causal")
        y.sum().backward()
        assert seen["bwd"][0] == mode and torch.equal(seen["bwd"][1], ring) and seen["bwd"][2] == (B, T, H, d)
        assert seen["train_drop"] == seen["bwd_drop"] == (0.0, 0, 0)
        assert x.grad is not None and m.qkv.weight.grad is not None
        assert (m.gqproj.weight.grad if link == "additive" else m.edge_mlp[0].weight.grad) is not None
    m = PathOrderedGeometricMHA(D, n_heads=H)
    assert m.exact_backward is False

    # active attention dropout: every mask (tril included) runs the exact
    # pair with the module's p and one fresh seed, which the backward gets
    # too; the seed comes from torch's CPU generator (repeatable under
    # torch.manual_seed)
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    m = PathOrderedGeometricMHA(D, n_heads=H, dropout=0.25)
    assert m._dropout_active() and not m.eval()._dropout_active()
    m.train()
    m.exact_backward = True
    seeds = []
    for rep in range(3):
        seen.clear()
        if rep < 2:
            torch.manual_seed(11)
        x = torch.randn(B, T, D, requires_grad=True)
        y, geo = m._forward_dropout(x, tril, False)
        assert geo is None and torch.equal(seen["train"][1], tril) and seen["train"][0] == "causal"
        y.sum().backward()
        p_, seed, off = seen["train_drop"]
        assert p_ == 0.25 and off == 0 and 0 <= seed < 2 ** 63 and seen["bwd_drop"] == (p_, seed, off)
        seeds.append(seed)
    assert seeds[0] == seeds[1] != seeds[2]
    # prefill and decode apply no dropout: they refuse it, exact_backward or not
    # (a stand-in for a GPU tensor: the reason is decided before any data is read)
    import types
    gpu_like = types.SimpleNamespace(is_cuda=True, dtype=torch.float32, shape=(B, T, D))
    assert "prefill and decode" in m._unsupported_reason(gpu_like, None, causal_implied=True)
    with pytest.raises(NotImplementedError, match="dropout"):
        m.decode_step(torch.randn(B, 1, D), None)
    m.exact_backward = False
    assert "exact_backward" in m._unsupported_reason(gpu_like, None)
    m.eval()
    assert m._unsupported_reason(gpu_like, None) is None


def test_forward_only_outputs_without_exact_backward():
    """With exact_backward off, the module's forward under autograd for a
    non-tril call keeps returning outputs whose backward raises."""
    from holonomyawareattention_amd.attention_kernel import _ForwardOnly
    x = torch.randn(2, 3, requires_grad=True)
    y = _ForwardOnly.apply("an attention mask other than tril(L)", 1, x * 2, x)
    with pytest.raises(NotImplementedError, match="tril"):
        y.sum().backward()
