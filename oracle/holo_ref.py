"""CPU oracle for the path-ordered (holonomy) attention forward.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this module: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only
as the checker (or, in bench.py, as the timed CPU baseline), never as the code
path being measured or shipped.

Three restatements of the reference algorithm (SiddhiMali/HolonomyAwareAttention),
all written from the reference's behaviour, not copied:

* ``forward_chunked`` follows ``core/attention_fast_chunked.py`` step by step in
  the caller's dtype (fp32 or fp64): per-head interleaved QKV split (:69-71),
  generator times ``edge_scale`` (:73-84), dense skew (``core/utils.py:4-27``)
  and ``torch.matrix_exp`` (``core/utils.py:30-52``), strictly sequential
  left-multiplied prefix products (:89-95), P^T transports (:108-110), the
  wrap branch with Hol^T (:112-117), key blocks of BLOCK_K=64 with an online
  softmax and ``finfo.min`` masking (:119-166), normalisation, P back-rotation
  and the out-projection (:168-173). The SO(3)-block rotation model is run by
  scattering the block parameters into the dense skew layout (every other
  entry zero), which the reference's own code then computes exactly.
* ``forward_blocks`` computes the same function in fp64 with the structure made
  explicit: closed-form Rodrigues 3x3 blocks, a 3x3 sequential scan, plain
  causal softmax (the wrap branch is always masked under tril). It is the fast
  checker for large slices; it is pinned against ``forward_chunked`` and the
  golden fixtures at small sizes.
* ``forward_arc_walk`` is the brute-force O(L^3) definition of
  ``core/attention.py:156-192`` (walk the ring arc j -> i composing edge
  rotations; inert mode: endpoint transport C_i^T C_j), any mask, for tiny L.
* ``forward_exact_blocks`` / ``exact_attention64`` restate the reference's
  exact path for every mode and mask (``kernel/attention_fast.py:84-166``,
  which the reference's kernel module runs off its kernel path): the wrap
  branch through Hol, the inert endpoint transport, -inf masking; fp64 on the
  block structure.

Pinning (every function has at least one independent check in tests/):
  skew_from_vec / block scatter / geometry / forward_chunked
        -> golden vectors written by importing the reference
           (tests/golden/make_golden.py), both link modes, fp64 and fp32;
  rodrigues -> torch.linalg.matrix_exp in fp64, G^T G = I, det = +1,
           exp(0)=I, exp(A)exp(-A)=I, small-angle series, angle pi;
  scan  -> brute-force products, P_0 = I, orthogonality;
  forward_exact_blocks -> forward_arc_walk for causal and inert mode with no
           mask, the ring mask (core/utils.py:59-75) and random masks;
           forward_blocks under causal + tril; at edge_scale = 0 torch's
           scaled_dot_product_attention with the same boolean mask (NaN rows
           where a row allows nothing, as torch.softmax gives).
  forward_blocks -> forward_chunked (fp64), flat-connection reduction
           (edge_scale = 0 gives torch's causal scaled_dot_product_attention),
           gauge invariance, causal prefix consistency, forward_arc_walk.
  exact_backward64 / link_grad_closed -> central differences of
           exact_attention64 through geometry_blocks (causal and inert, no
           mask, random and ring masks, the closing edge included); under
           tril the tril backward oracle (pinned to torch autograd);
           planted mistakes fail (tests/test_oracle_exact_backward.py).
  philox4x32_10 -> the published known-answer vectors of Philox4x32-10
           (Random123: zero, all-ones and pi-digit counters and keys);
  dropout_keep -> kept fraction within binomial bounds, rows independent of
           the row subset asked for, p = 0 keeps everything;
  exact_attention64 / exact_backward64 with keep -> p = 0 gives the
           dropout-free result; with drop_scale = 1 the outputs of a keep
           mask and of its complement sum to the dropout-free output
           (dropout acts on the softmax weights of both branches); the
           gradients by central differences under a fixed keep mask, with
           planted mistakes failing (tests/test_oracle_dropout.py).
  decoder_forward -> at edge_scale = 0 (P = I) a stack of torch's own pre-LN
           nn.TransformerEncoderLayer (GELU, causal mask, zero attention
           biases, the per-head interleaved qkv rows reordered into torch's
           [q; k; v] layout) in float64; causal prefix consistency.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch

BLOCK_K = 64          # key-block width of core/attention_fast_chunked.py:33


# --------------------------------------------------------------------------
# rotation-model helpers
# --------------------------------------------------------------------------
def n_blocks(d: int) -> int:
    """Number of SO(3) blocks per head: floor(d/3); leftover dims are identity."""
    return d // 3


def block_param_count(d: int) -> int:
    return 3 * n_blocks(d)


def dense_index(i: int, j: int, d: int) -> int:
    """Position of entry (i, j), i < j, in the row-major upper-triangle vector
    that core/utils.py:20-26 reads (i outer, j inner)."""
    return i * d - i * (i + 1) // 2 + (j - i - 1)


def block_to_dense_map(d: int) -> np.ndarray:
    """dense index of each block parameter: block b, component c in
    (a01, a02, a12) of A_b = [[0,a01,a02],[-a01,0,a12],[-a02,-a12,0]]."""
    out = []
    for b in range(n_blocks(d)):
        r = 3 * b
        out += [dense_index(r, r + 1, d), dense_index(r, r + 2, d),
                dense_index(r + 1, r + 2, d)]
    return np.asarray(out, dtype=np.int64)


def dense_rows_from_block(w_blk: torch.Tensor, n_heads: int, d: int) -> torch.Tensor:
    """Scatter a block-layout generator matrix (H*m_blk, ...) into the
    reference's dense layout (H*d(d-1)/2, ...), zeros elsewhere."""
    mb, md = block_param_count(d), d * (d - 1) // 2
    mp = torch.as_tensor(block_to_dense_map(d))
    w = w_blk.reshape(n_heads, mb, *w_blk.shape[1:])
    out = w.new_zeros(n_heads, md, *w_blk.shape[1:])
    out[:, mp] = w
    return out.reshape(n_heads * md, *w_blk.shape[1:])


def skew_from_vec(v: torch.Tensor, d: int) -> torch.Tensor:
    """Row-major upper-triangle vector -> skew matrix (core/utils.py:4-27):
    A[i,j] = v[idx], A[j,i] = -v[idx], idx running i-major over i < j."""
    *prefix, m = v.shape
    if m != d * (d - 1) // 2:
        raise ValueError(f"Expected last dim {d * (d - 1) // 2}, got {m}")
    rows, cols = torch.triu_indices(d, d, offset=1)
    A = v.new_zeros(*prefix, d, d)
    A[..., rows, cols] = v
    A[..., cols, rows] = -v
    return A


def so_exp(A: torch.Tensor) -> torch.Tensor:
    """core/utils.py:30-52: the matrix exponential (torch's routine)."""
    return torch.matrix_exp(A)


# --------------------------------------------------------------------------
# restatement of core/attention_fast_chunked.py
# --------------------------------------------------------------------------
def _linear(x, w, b=None):
    y = x @ w.transpose(0, 1)
    return y if b is None else y + b


def generator_params(x: torch.Tensor, W: Dict[str, torch.Tensor], n_heads: int,
                     edge_scale: float, link_mode: str) -> torch.Tensor:
    """Block-layout link parameters a (B, H, T, m_blk) for the T edges
    t -> t+1 (mod T); edge T-1 is the closing edge.
    additive:    a_t = (gq(x_t) + gk(x_{t+1})) * edge_scale     (:80-84)
    interaction: a_t = edge_mlp([x_t ; x_{t+1}]) * edge_scale   (:73-79)
    """
    B, T, D = x.shape
    d = D // n_heads
    m = block_param_count(d)
    if link_mode == "additive":
        gq = _linear(x, W["gqproj.weight"]).view(B, T, n_heads, m).transpose(1, 2)
        gk = _linear(x, W["gkproj.weight"]).view(B, T, n_heads, m).transpose(1, 2)
        return (gq + torch.roll(gk, shifts=-1, dims=2)) * edge_scale
    if link_mode == "interaction":
        pair = torch.cat([x, torch.roll(x, shifts=-1, dims=1)], dim=-1)
        h = torch.nn.functional.gelu(_linear(pair, W["edge_mlp.0.weight"], W["edge_mlp.0.bias"]))
        a = _linear(h, W["edge_mlp.2.weight"], W["edge_mlp.2.bias"])
        return a.view(B, T, n_heads, m).transpose(1, 2) * edge_scale
    raise ValueError(f"unknown link_mode {link_mode!r}")


def split_qkv(x: torch.Tensor, w_qkv: torch.Tensor, n_heads: int):
    """Per-head interleaved split of x W_qkv^T: columns [q_h | k_h | v_h] for
    each head h (core/attention_fast_chunked.py:69-71). Returns (B,H,T,d) x3."""
    B, T, D = x.shape
    d = D // n_heads
    qkv = _linear(x, w_qkv).view(B, T, n_heads, 3 * d)
    q, k, v = qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:]
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)


def geometry_chunked(x: torch.Tensor, W: Dict[str, torch.Tensor], n_heads: int,
                     edge_scale: float, link_mode: str = "additive",
                     a: Optional[torch.Tensor] = None):
    """q, k, v, P, Hol as core/attention_fast_chunked.py:63-96 computes them,
    on the dense d x d layout. `a` (B,H,T,m_blk) overrides the generator."""
    B, T, D = x.shape
    d = D // n_heads
    q, k, v = split_qkv(x, W["qkv.weight"], n_heads)
    if a is None:
        a = generator_params(x, W, n_heads, edge_scale, link_mode)
    md = d * (d - 1) // 2
    a_dense = a.new_zeros(B, n_heads, T, md)
    a_dense[..., torch.as_tensor(block_to_dense_map(d))] = a
    G_adj = so_exp(skew_from_vec(a_dense[:, :, :-1], d))
    G_close = so_exp(skew_from_vec(a_dense[:, :, -1], d))
    eye = torch.eye(d, dtype=x.dtype)
    P = torch.empty(B, n_heads, T, d, d, dtype=x.dtype)
    P[:, :, 0] = eye
    Pt = eye.expand(B, n_heads, d, d).clone()
    for t in range(T - 1):
        Pt = G_adj[:, :, t] @ Pt                 # left-multiply (:93)
        P[:, :, t + 1] = Pt
    Hol = G_close @ P[:, :, T - 1]
    return q, k, v, P, Hol


def attention_core_chunked(q, k, v, P, Hol, scale: float, block_k: int = BLOCK_K):
    """Transport, key-block online softmax with the (masked) wrap branch, and
    back-rotation, as core/attention_fast_chunked.py:105-171 with a tril mask.
    Returns the per-head outputs (B, H, T, d) before the out-projection."""
    B, H, L, d = q.shape
    dtype = q.dtype
    qh = torch.einsum("bhide,bhid->bhie", P, q)          # P_i^T q_i
    kh_all = torch.einsum("bhjde,bhjd->bhje", P, k)
    vh_all = torch.einsum("bhjde,bhjd->bhje", P, v)
    kh_wrap = torch.einsum("bhef,bhje->bhjf", Hol, kh_all)
    vh_wrap = torch.einsum("bhef,bhje->bhjf", Hol, vh_all)
    neg = torch.finfo(dtype).min
    m_run = torch.full((B, H, L), neg, dtype=dtype)
    l_run = torch.zeros((B, H, L), dtype=dtype)
    o_run = torch.zeros((B, H, L, d), dtype=dtype)
    idx = torch.arange(L)
    for k0 in range(0, L, block_k):
        k1 = min(k0 + block_k, L)
        jj = idx[k0:k1]
        base = (idx.view(L, 1) >= jj.view(1, -1)).view(1, 1, L, -1)
        s_base = torch.einsum("bhie,bhje->bhij", qh, kh_all[:, :, k0:k1]) * scale
        s_wrap = torch.einsum("bhie,bhje->bhij", qh, kh_wrap[:, :, k0:k1]) * scale
        s = torch.where(base, s_base, s_wrap)
        s = s.masked_fill(~base, neg)            # tril: allowed == (i >= j)
        m_new = torch.maximum(m_run, s.max(dim=-1).values)
        corr = torch.exp(m_run - m_new)
        p = torch.exp(s - m_new.unsqueeze(-1))
        l_run = l_run * corr + p.sum(dim=-1)
        cb = torch.einsum("bhij,bhje->bhie", p * base, vh_all[:, :, k0:k1])
        cw = torch.einsum("bhij,bhje->bhie", p * ~base, vh_wrap[:, :, k0:k1])
        o_run = o_run * corr.unsqueeze(-1) + cb + cw
        m_run = m_new
    o_run = o_run / l_run.clamp_min(1e-20).unsqueeze(-1)
    return torch.einsum("bhide,bhie->bhid", P, o_run)   # P_i o_i


def forward_chunked(x: torch.Tensor, W: Dict[str, torch.Tensor], n_heads: int,
                    edge_scale: float, link_mode: str = "additive",
                    a: Optional[torch.Tensor] = None, return_geometry: bool = False):
    """y = PathOrderedGeometricMHA.forward(x, tril) of the reference chunked
    implementation, in x's dtype. W holds block-layout weights (torch tensors
    of x's dtype)."""
    B, T, D = x.shape
    d = D // n_heads
    q, k, v, P, Hol = geometry_chunked(x, W, n_heads, edge_scale, link_mode, a)
    o = attention_core_chunked(q, k, v, P, Hol, 1.0 / math.sqrt(d))
    y = _linear(o.transpose(1, 2).reshape(B, T, D), W["out.weight"])
    if return_geometry:
        return y, {"C": P, "H": Hol}
    return y


# --------------------------------------------------------------------------
# block-structured fp64 restatement (fast checker for large slices)
# --------------------------------------------------------------------------
def rodrigues(a: np.ndarray) -> np.ndarray:
    """exp of A = [[0,a0,a1],[-a0,0,a2],[-a1,-a2,0]] for a (..., 3), float64:
    I + (sin th / th) A + ((1 - cos th) / th^2) A^2, th = |a|, with the
    Taylor series of both coefficients below th = 1e-4."""
    a = np.asarray(a, dtype=np.float64)
    a0, a1, a2 = a[..., 0], a[..., 1], a[..., 2]
    z = np.zeros_like(a0)
    A = np.stack([np.stack([z, a0, a1], -1),
                  np.stack([-a0, z, a2], -1),
                  np.stack([-a1, -a2, z], -1)], -2)
    th2 = a0 * a0 + a1 * a1 + a2 * a2
    th = np.sqrt(th2)
    small = th < 1e-4
    ths = np.where(small, 1.0, th)
    s1 = np.where(small, 1.0 - th2 / 6.0 + th2 * th2 / 120.0, np.sin(ths) / ths)
    s2 = np.where(small, 0.5 - th2 / 24.0 + th2 * th2 / 720.0, (1.0 - np.cos(ths)) / (ths * ths))
    eye = np.broadcast_to(np.eye(3), A.shape)
    return eye + s1[..., None, None] * A + s2[..., None, None] * (A @ A)


def prefix_blocks(G: np.ndarray) -> np.ndarray:
    """P_0 = I, P_{t+1} = G_t P_t along axis -4 of G (..., T-1, nb, 3, 3);
    returns (..., T, nb, 3, 3)."""
    *lead, Tm1, nb, _, _ = G.shape
    P = np.empty((*lead, Tm1 + 1, nb, 3, 3), dtype=np.float64)
    cur = np.broadcast_to(np.eye(3), (*lead, nb, 3, 3)).copy()
    P[..., 0, :, :, :] = cur
    for t in range(Tm1):
        cur = G[..., t, :, :, :] @ cur
        P[..., t + 1, :, :, :] = cur
    return P


def apply_blocks_T(P: np.ndarray, u: np.ndarray) -> np.ndarray:
    """u^_t = P_t^T u_t on the block dims of u (..., T, d); leftover dims pass."""
    nb = P.shape[-3]
    out = u.copy()
    ub = u[..., :3 * nb].reshape(*u.shape[:-1], nb, 3)
    out[..., :3 * nb] = np.einsum("...bij,...bi->...bj", P, ub).reshape(*u.shape[:-1], 3 * nb)
    return out


def apply_blocks(P: np.ndarray, u: np.ndarray) -> np.ndarray:
    """u_t = P_t u^_t on the block dims."""
    nb = P.shape[-3]
    out = u.copy()
    ub = u[..., :3 * nb].reshape(*u.shape[:-1], nb, 3)
    out[..., :3 * nb] = np.einsum("...bij,...bj->...bi", P, ub).reshape(*u.shape[:-1], 3 * nb)
    return out


def causal_attention64(qh: np.ndarray, kh: np.ndarray, vh: np.ndarray, scale: float,
                       q_block: int = 256) -> np.ndarray:
    """softmax(q k^T * scale + causal) v over (..., T, d), float64, query-blocked."""
    T = qh.shape[-2]
    out = np.empty_like(qh)
    for i0 in range(0, T, q_block):
        i1 = min(T, i0 + q_block)
        s = np.matmul(qh[..., i0:i1, :], np.swapaxes(kh[..., :i1, :], -1, -2)) * scale
        mask = np.arange(i0, i1)[:, None] >= np.arange(i1)[None, :]
        s = np.where(mask, s, -np.inf)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[..., i0:i1, :] = np.matmul(p, vh[..., :i1, :])
    return out


def attention_rows64(qh: np.ndarray, kh: np.ndarray, vh: np.ndarray, scale: float,
                     rows: np.ndarray) -> np.ndarray:
    """Rows `rows` (query positions) of causal_attention64: query i attends to
    keys 0..i. qh, kh, vh (..., T, d) float64 -> (..., len(rows), d)."""
    rows = np.asarray(rows)
    i1 = int(rows.max()) + 1
    s = np.matmul(qh[..., rows, :], np.swapaxes(kh[..., :i1, :], -1, -2)) * scale
    s = np.where(rows[:, None] >= np.arange(i1)[None, :], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vh[..., :i1, :])


def ring_mask(T: int) -> np.ndarray:
    """Local ring mask of core/utils.py:59-75: token i may attend to itself and
    to its ring neighbours (i - 1) mod T and (i + 1) mod T (True = allowed)."""
    m = np.zeros((T, T), dtype=bool)
    i = np.arange(T)
    m[i, i] = True
    m[i, (i - 1) % T] = True
    m[i, (i + 1) % T] = True
    return m


def exact_attention64(q: np.ndarray, k: np.ndarray, v: np.ndarray, P: np.ndarray, Hol: np.ndarray,
                      scale: float, mask: Optional[np.ndarray] = None, mode: str = "causal",
                      keep: Optional[np.ndarray] = None, drop_scale: float = 1.0) -> np.ndarray:
    """Per-head outputs (B, H, T, d) of the reference's exact path for any
    mask and mode (kernel/attention_fast.py:129-162, which
    kernel/attention_kernel.py:211-213 runs for every call off the kernel
    path), float64, on the block structure.

    The reference transports key/value j to query i by G_arc[i, j] =
    P_i P_j^T (i >= j) or P_i Hol P_j^T (i < j) in causal mode (:130-141) and
    by P_i^T P_j in inert mode (:142-144), masks disallowed scores with -inf
    (:154-157; a row with no allowed key gives NaN, as torch.softmax does) and
    returns sum_j a_ij G_arc[i, j] v_j. In transported coordinates
    (u^ = P^T u in causal mode, u' = P u in inert mode):
      causal: s_ij = q^_i . (Hol k^_j if i < j else k^_j),
              o_i  = P_i (sum_{j<=i} a_ij v^_j + Hol sum_{j>i} a_ij v^_j)
      inert:  s_ij = q'_i . k'_j,   o_i = P_i^T sum_j a_ij v'_j
    q, k, v (B, H, T, d); P (B, H, T, nb, 3, 3); Hol (B, H, nb, 3, 3);
    mask (T, T) bool or None (everything allowed). Attention dropout
    (kernel/attention_fast.py:160, an nn.Dropout on the softmax weights):
    keep (B, H, T, T) bool (dropout_keep) multiplies a_ij by
    keep_ij * drop_scale (1 / (1 - p)) after the softmax."""
    T = q.shape[-2]
    allowed = np.ones((T, T), dtype=bool) if mask is None else np.asarray(mask, dtype=bool)
    if mode == "causal":
        qh, kh, vh = (apply_blocks_T(P, u) for u in (q, k, v))
        Hb = Hol[:, :, None]                                  # broadcast over tokens
        khw, vhw = apply_blocks(Hb, kh), apply_blocks(Hb, vh)
        base = np.arange(T)[:, None] >= np.arange(T)[None, :]
        s = np.where(base, np.einsum("...id,...jd->...ij", qh, kh),
                     np.einsum("...id,...jd->...ij", qh, khw)) * scale
    elif mode == "inert":
        qh, kh, vh = (apply_blocks(P, u) for u in (q, k, v))
        s = np.einsum("...id,...jd->...ij", qh, kh) * scale
    else:
        raise ValueError(mode)
    s = np.where(allowed, s, -np.inf)
    with np.errstate(invalid="ignore"):
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=-1, keepdims=True)
    if keep is not None:
        p = np.where(keep, p * drop_scale, 0.0)
    if mode == "causal":
        oh = np.einsum("...ij,...jd->...id", np.where(base, p, 0.0), vh) + \
            np.einsum("...ij,...jd->...id", np.where(base, 0.0, p), vhw)
        return apply_blocks(P, oh)
    return apply_blocks_T(P, np.einsum("...ij,...jd->...id", p, vh))


# --------------------------------------------------------------------------
# attention dropout's keep mask
# --------------------------------------------------------------------------
# Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as
# easy as 1, 2, 3", SC 2011): ten rounds of two 32x32->64-bit products on a
# 128-bit counter under a 64-bit key bumped by Weyl increments.
PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def philox4x32_10(ctr: np.ndarray, key: Tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 of counters ctr (..., 4) uint32 under key (k0, k1):
    (..., 4) uint32. Each round maps (c0, c1, c2, c3) to
    (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)) and then
    bumps the key by PHILOX_W."""
    ctr = np.asarray(ctr, dtype=np.uint32)
    c = [ctr[..., i].astype(np.uint64) for i in range(4)]
    m32 = np.uint64(0xFFFFFFFF)
    k0, k1 = np.uint64(int(key[0]) & 0xFFFFFFFF), np.uint64(int(key[1]) & 0xFFFFFFFF)
    M0, M1 = np.uint64(PHILOX_M[0]), np.uint64(PHILOX_M[1])
    for _ in range(10):
        p0, p1 = M0 * c[0], M1 * c[2]                 # exact: both factors below 2^32
        c = [(p1 >> np.uint64(32)) ^ c[1] ^ k0, p1 & m32, (p0 >> np.uint64(32)) ^ c[3] ^ k1, p0 & m32]
        k0 = (k0 + np.uint64(PHILOX_W[0])) & m32
        k1 = (k1 + np.uint64(PHILOX_W[1])) & m32
    return np.stack(c, -1).astype(np.uint32)


def dropout_threshold(p: float) -> int:
    """The 32-bit threshold of drop probability p (0 <= p < 1, taken as a
    float32): a pair is kept when its random word is >= round(p * 2^32)
    (ties to even), capped at 2^32 - 1."""
    t = float(np.float32(p)) * 4294967296.0
    return min(int(round(t)), 0xFFFFFFFF)


def dropout_keep(B: int, H: int, T: int, p: float, seed: int, offset: int = 0,
                 rows: Optional[np.ndarray] = None) -> np.ndarray:
    """Keep mask (B, H, T, T) bool of attention dropout with probability p:
    pair (i, j) of head (b, h) is kept when word j % 4 of
    philox4x32_10((i, j // 4, b H + h, offset), (seed mod 2^32, seed // 2^32))
    is >= dropout_threshold(p). rows (optional index array) limits i to
    those rows: (B, H, len(rows), T)."""
    i = np.arange(T, dtype=np.uint64) if rows is None else np.asarray(rows, dtype=np.uint64)
    j = np.arange(T, dtype=np.uint64)
    bh = np.arange(B * H, dtype=np.uint64).reshape(B, H, 1, 1)
    ctr = np.empty((B, H, len(i), (T + 3) // 4, 4), dtype=np.uint32)
    ctr[..., 0] = i.reshape(1, 1, -1, 1)
    ctr[..., 1] = np.arange((T + 3) // 4, dtype=np.uint64).reshape(1, 1, 1, -1)
    ctr[..., 2] = bh
    ctr[..., 3] = int(offset) & 0xFFFFFFFF
    words = philox4x32_10(ctr, (int(seed) & 0xFFFFFFFF, (int(seed) >> 32) & 0xFFFFFFFF))
    words = words.reshape(B, H, len(i), -1)[..., :T]
    return words >= np.uint32(dropout_threshold(p))


def geometry_blocks(a: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """a (B,H,T,m_blk) -> P (B,H,T,nb,3,3) and Hol (B,H,nb,3,3), float64."""
    B, H, T, m = a.shape
    nb = m // 3
    G = rodrigues(a.reshape(B, H, T, nb, 3))
    P = prefix_blocks(G[:, :, :-1])
    Hol = G[:, :, -1] @ P[:, :, -1]
    return P, Hol


def forward_blocks(x: np.ndarray, W: Dict[str, np.ndarray], n_heads: int,
                   edge_scale: float, link_mode: str = "additive",
                   a: Optional[np.ndarray] = None, return_parts: bool = False):
    """float64 forward on the block structure. x (B,T,D); W block-layout."""
    x = np.asarray(x, dtype=np.float64)
    B, T, D = x.shape
    H = n_heads
    d = D // H
    Wt = {k: torch.as_tensor(np.asarray(w, dtype=np.float64)) for k, w in W.items()}
    xt = torch.as_tensor(x)
    q, k, v = (t.numpy() for t in split_qkv(xt, Wt["qkv.weight"], H))
    if a is None:
        a = generator_params(xt, Wt, H, edge_scale, link_mode).numpy()
    P, Hol = geometry_blocks(np.asarray(a, dtype=np.float64))
    qh, kh, vh = (apply_blocks_T(P, u) for u in (q, k, v))
    oh = causal_attention64(qh, kh, vh, 1.0 / math.sqrt(d))
    o = apply_blocks(P, oh)
    y = o.transpose(0, 2, 1, 3).reshape(B, T, D) @ np.asarray(W["out.weight"], np.float64).T
    if return_parts:
        return y, dict(q=q, k=k, v=v, a=a, P=P, Hol=Hol, qh=qh, kh=kh, vh=vh, oh=oh, o=o)
    return y


def forward_exact_blocks(x: np.ndarray, W: Dict[str, np.ndarray], n_heads: int, edge_scale: float,
                         link_mode: str = "additive", mask: Optional[np.ndarray] = None,
                         mode: str = "causal", a: Optional[np.ndarray] = None,
                         return_parts: bool = False):
    """float64 forward of the layer for any mask and mode (the reference's
    exact path, kernel/attention_fast.py:84-166); with mode "causal" and a tril
    mask it is forward_blocks."""
    x = np.asarray(x, dtype=np.float64)
    B, T, D = x.shape
    H = n_heads
    d = D // H
    Wt = {k: torch.as_tensor(np.asarray(w, dtype=np.float64)) for k, w in W.items()}
    xt = torch.as_tensor(x)
    q, k, v = (t.numpy() for t in split_qkv(xt, Wt["qkv.weight"], H))
    if a is None:
        a = generator_params(xt, Wt, H, edge_scale, link_mode).numpy()
    P, Hol = geometry_blocks(np.asarray(a, dtype=np.float64))
    o = exact_attention64(q, k, v, P, Hol, 1.0 / math.sqrt(d), mask, mode)
    y = o.transpose(0, 2, 1, 3).reshape(B, T, D) @ np.asarray(W["out.weight"], np.float64).T
    if return_parts:
        return y, dict(q=q, k=k, v=v, a=a, P=P, Hol=Hol, o=o)
    return y


def blocks_to_dense(Pb: np.ndarray, d: int) -> np.ndarray:
    """(..., nb, 3, 3) block rotations -> (..., d, d) with identity leftovers."""
    nb = Pb.shape[-3]
    out = np.zeros((*Pb.shape[:-3], d, d), dtype=Pb.dtype)
    for b in range(nb):
        out[..., 3 * b:3 * b + 3, 3 * b:3 * b + 3] = Pb[..., b, :, :]
    for r in range(3 * nb, d):
        out[..., r, r] = 1.0
    return out


# --------------------------------------------------------------------------
# brute-force definition (core/attention.py:156-192), tiny L only
# --------------------------------------------------------------------------
def forward_arc_walk(x: np.ndarray, W: Dict[str, np.ndarray], n_heads: int,
                     edge_scale: float, link_mode: str = "additive", mask="tril",
                     mode: str = "causal") -> np.ndarray:
    """Transport key/value j to query i by walking the ring arc j -> j+1 -> ...
    -> i with the edge rotations (crossing the closing edge when i < j), then
    softmax over the allowed keys. float64, O(L^3). `mask`: "tril" (default),
    None (everything allowed) or a (T, T) bool array; a row with no allowed key
    is NaN (softmax over -inf only). mode "inert" replaces the walk by the
    endpoint transport C_i^T C_j of the prefix products C_t = G_{t-1}...G_0
    (core/attention.py:150-167)."""
    x = np.asarray(x, dtype=np.float64)
    B, T, D = x.shape
    H = n_heads
    d = D // H
    Wt = {k: torch.as_tensor(np.asarray(w, dtype=np.float64)) for k, w in W.items()}
    xt = torch.as_tensor(x)
    q, k, v = (t.numpy() for t in split_qkv(xt, Wt["qkv.weight"], H))
    a = generator_params(xt, Wt, H, edge_scale, link_mode).numpy()
    G = blocks_to_dense(rodrigues(a.reshape(B, H, T, -1, 3)), d)     # (B,H,T,d,d)
    if isinstance(mask, str):
        allowed = np.tril(np.ones((T, T), dtype=bool))
    else:
        allowed = np.ones((T, T), dtype=bool) if mask is None else np.asarray(mask, dtype=bool)
    C = np.empty((B, H, T, d, d))
    C[:, :, 0] = np.eye(d)
    for t in range(T - 1):
        C[:, :, t + 1] = G[:, :, t] @ C[:, :, t]
    out = np.zeros((B, H, T, d))
    for i in range(T):
        Kt = np.zeros((B, H, T, d))
        Vt = np.zeros((B, H, T, d))
        for j in range(T):
            if mode == "inert":
                U = np.swapaxes(C[:, :, i], -1, -2) @ C[:, :, j]
            else:
                U = np.broadcast_to(np.eye(d), (B, H, d, d)).copy()
                t = j
                while t != i:
                    U = G[:, :, t] @ U
                    t = (t + 1) % T
            Kt[:, :, j] = np.einsum("bhdf,bhf->bhd", U, k[:, :, j])
            Vt[:, :, j] = np.einsum("bhdf,bhf->bhd", U, v[:, :, j])
        s = np.einsum("bhd,bhjd->bhj", q[:, :, i], Kt) / math.sqrt(d)
        s = np.where(allowed[i], s, -np.inf)
        with np.errstate(invalid="ignore"):
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(-1, keepdims=True)
        out[:, :, i] = np.einsum("bhj,bhjd->bhd", p, Vt)
    return out.transpose(0, 2, 1, 3).reshape(B, T, D) @ np.asarray(W["out.weight"], np.float64).T


# --------------------------------------------------------------------------
# decoder stack (experiments/session_cherry.py:286-294 block, :315-327 hidden)
# --------------------------------------------------------------------------
def _layer_norm64(h: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """nn.LayerNorm over the last dim (biased variance), float64."""
    mu = h.mean(axis=-1, keepdims=True)
    var = ((h - mu) ** 2).mean(axis=-1, keepdims=True)
    return (h - mu) / np.sqrt(var + eps) * w + b


def _gelu64(x: np.ndarray) -> np.ndarray:
    """nn.GELU() (exact erf form), float64."""
    return torch.nn.functional.gelu(torch.as_tensor(x)).numpy()


def decoder_forward(tokens: np.ndarray, W: Dict[str, np.ndarray], n_layers: int, n_heads: int,
                    edge_scale: float, link_mode: str = "additive",
                    return_hidden: bool = False) -> np.ndarray:
    """float64 forward of the pre-LN decoder: h = embed[tokens]; per block
    h += attention(ln1(h)) (forward_blocks) and h += ff(ln2(h)) with
    ff = Linear -> GELU -> Linear (session_cherry.py:292-294); logits = h W_lm^T."""
    W = {k: np.asarray(v, dtype=np.float64) for k, v in W.items()}
    h = W["embed.weight"][np.asarray(tokens)]
    for i in range(n_layers):
        p = f"blocks.{i}."
        core = {k[len(p) + 5:]: v for k, v in W.items() if k.startswith(p + "core.")}
        a = _layer_norm64(h, W[p + "ln1.weight"], W[p + "ln1.bias"])
        h = h + forward_blocks(a, core, n_heads, edge_scale, link_mode)
        a = _layer_norm64(h, W[p + "ln2.weight"], W[p + "ln2.bias"])
        f = _gelu64(a @ W[p + "ff.0.weight"].T + W[p + "ff.0.bias"])
        h = h + f @ W[p + "ff.2.weight"].T + W[p + "ff.2.bias"]
    if return_hidden:
        return h
    return h @ W["lm_head.weight"].T


# --------------------------------------------------------------------------
# backward of the block-structured forward (float64)
# --------------------------------------------------------------------------
def _blocks3(u: np.ndarray, nb: int) -> np.ndarray:
    return u[..., :3 * nb].reshape(*u.shape[:-1], nb, 3)


def link_grad_from_cross(a: np.ndarray, P: np.ndarray, c: np.ndarray) -> np.ndarray:
    """dL/da_t (B,H,T,nb,3) from the per-token cross-product sums c (B,H,T,nb,3).

    With E_t = P_t^T dL/dP_t, the reverse recursion of P_{t+1} = G_t P_t gives
    M_t = P_t^T Lambda_t = sum_{s>=t} E_s, and G_t^T dL/dG_t = P_t M_{t+1} P_t^T.
    Only its antisymmetric part reaches a: vee(W - W^T) = P_t m_{t+1} with
    m = sum_{s>t} c_s, c_s = vee(E_s - E_s^T). The skew vector a = (a01, a02, a12)
    is phi = (-a12, a02, -a01) in the standard hat map, and
    dL/dphi = J_r(phi)^T g, J_r^T g = g + al phi x g + be phi x (phi x g),
    al = (1 - cos th) / th^2, be = (th - sin th) / th^3. The closing edge
    (t = T-1) only enters the holonomy: its gradient is zero."""
    suf = np.cumsum(c[..., ::-1, :, :], axis=-3)[..., ::-1, :, :]        # m_t = sum_{s>=t} c_s
    m_next = np.zeros_like(c)
    m_next[..., :-1, :, :] = suf[..., 1:, :, :]
    g = np.einsum("...bij,...bj->...bi", P, m_next)                      # P_t m_{t+1}
    phi = np.stack([-a[..., 2], a[..., 1], -a[..., 0]], -1)
    th2 = (phi * phi).sum(-1)
    th = np.sqrt(th2)
    small = th < 1e-3
    ths = np.where(small, 1.0, th)
    al = np.where(small, 0.5 - th2 / 24.0 + th2 * th2 / 720.0, (1.0 - np.cos(ths)) / (ths * ths))
    be = np.where(small, 1.0 / 6.0 - th2 / 120.0 + th2 * th2 / 5040.0, (ths - np.sin(ths)) / (ths ** 3))
    pxg = np.cross(phi, g)
    dphi = g + al[..., None] * pxg + be[..., None] * np.cross(phi, pxg)
    da = np.stack([-dphi[..., 2], dphi[..., 1], -dphi[..., 0]], -1)
    da[..., -1, :, :] = 0.0
    return da


def link_grad_closed(a: np.ndarray, P: np.ndarray, c: np.ndarray, c_hol: np.ndarray) -> np.ndarray:
    """dL/da_t (B,H,T,nb,3) when the loss also depends on the holonomy
    Hol = G_{T-1} P_{T-1} (the exact path's wrap branch): Hol is P_T of the
    same recursion, so its cross-product sum c_hol (B,H,nb,3) is a virtual
    token T's. Every suffix m_t gains c_hol, and the closing edge t = T-1
    gets P_{T-1} c_hol (in link_grad_from_cross it has no later token)."""
    cc = np.concatenate([c, c_hol[..., None, :, :]], axis=-3)            # tokens 0..T
    suf = np.cumsum(cc[..., ::-1, :, :], axis=-3)[..., ::-1, :, :]      # m_t = sum_{s>=t} c_s, t = 0..T
    m_next = suf[..., 1:, :, :]                                          # m_{t+1}, t = 0..T-1
    g = np.einsum("...bij,...bj->...bi", P, m_next)
    return _link_param_grad(a, g)


def _link_param_grad(a: np.ndarray, g: np.ndarray) -> np.ndarray:
    """dL/da from g = P_t m_{t+1} (the SO(3) right Jacobian step of
    link_grad_from_cross)."""
    phi = np.stack([-a[..., 2], a[..., 1], -a[..., 0]], -1)
    th2 = (phi * phi).sum(-1)
    th = np.sqrt(th2)
    small = th < 1e-3
    ths = np.where(small, 1.0, th)
    al = np.where(small, 0.5 - th2 / 24.0 + th2 * th2 / 720.0, (1.0 - np.cos(ths)) / (ths * ths))
    be = np.where(small, 1.0 / 6.0 - th2 / 120.0 + th2 * th2 / 5040.0, (ths - np.sin(ths)) / (ths ** 3))
    pxg = np.cross(phi, g)
    dphi = g + al[..., None] * pxg + be[..., None] * np.cross(phi, pxg)
    return np.stack([-dphi[..., 2], dphi[..., 1], -dphi[..., 0]], -1)


def exact_backward64(q: np.ndarray, k: np.ndarray, v: np.ndarray, a: np.ndarray, do: np.ndarray, scale: float,
                     mask: Optional[np.ndarray] = None, mode: str = "causal", plant: str = "",
                     keep: Optional[np.ndarray] = None, drop_scale: float = 1.0) -> Dict[str, np.ndarray]:
    """Gradients of <do, exact_attention64(q, k, v, P(a), Hol(a), ...)>
    (the exact path for any mask and mode) with respect to q, k, v (B,H,T,d)
    and the link parameters a (B,H,T,m) of all T edges, in float64. Rows
    must allow at least one key.

    Causal mode, in the path frame (u^ = P^T u), with qw = Hol^T q^ and
    dow = Hol^T do^ the wrap branch's operands (pairs i < j):
      dS = p (dA - delta), dA_ij = do^_i . v^_j (i >= j) or dow_i . v^_j,
      delta_i = do^_i . u_i (u_i = P_i^T o_i),
      dq^ = scale (dS_base k^ + Hol dS_wrap k^),
      dk^ = scale (dS_base^T q^ + dS_wrap^T qw) = dk_base + dkw,
      dv^ = p_base^T do^ + p_wrap^T dow = dv_base + dvw.
    The per-token cross sums c_t = u x do^ + dq^ x q^ + dk^ x k^ + dv^ x v^
    are those of the tril path; the holonomy adds the virtual token
    c_hol = sum_j k^_j x dkw_j + v^_j x dvw_j (Hol^T dL/dHol, antisymmetric
    part), see link_grad_closed.
    Inert mode is the same algebra with P replaced by Q = P^T (u' = P u): the
    cross sums c'_t in the primed frame give c_t = -P_t^T c'_t, and there is
    no holonomy (the closing edge's gradient is zero).
    With attention dropout (keep, drop_scale as for exact_attention64) the
    output weights are A = p z, z = keep * drop_scale: dv^ and dvw take A in
    place of p, the gradient of p is z dA, and delta_i = sum_j p_ij z_ij dA_ij
    is still do^_i . u_i, since u is formed with A.
    `plant` (tests only) introduces one named mistake, so that the tests can
    show their checks detect it."""
    T = q.shape[-2]
    nb = a.shape[-1] // 3
    P, Hol = geometry_blocks(a)
    allowed = np.ones((T, T), dtype=bool) if mask is None else np.asarray(mask, dtype=bool)
    b3 = lambda u: _blocks3(u, nb)
    mm = lambda x, y: np.einsum("...ij,...jd->...id", x, y)
    mmT = lambda x, y: np.einsum("...ij,...id->...jd", x, y)
    dot = lambda x, y: np.einsum("...id,...jd->...ij", x, y)
    if mode == "causal":
        qh, kh, vh, doh = (apply_blocks_T(P, u) for u in (q, k, v, do))
        Hb = Hol[:, :, None]
        qw, dow = apply_blocks_T(Hb, qh), apply_blocks_T(Hb, doh)
        if plant == "hol_not_transposed":
            qw = apply_blocks(Hb, qh)
        base = np.arange(T)[:, None] >= np.arange(T)[None, :]
        s = np.where(base, dot(qh, kh), dot(qw, kh)) * scale
    elif mode == "inert":
        qh, kh, vh, doh = (apply_blocks(P, u) for u in (q, k, v, do))
        base = np.ones((T, T), dtype=bool)
        s = dot(qh, kh) * scale
    else:
        raise ValueError(mode)
    s = np.where(allowed, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    z = 1.0 if keep is None else np.where(keep, drop_scale, 0.0)
    if plant == "dropout_before_softmax" and keep is not None:
        p = np.where(keep, p, 0.0)
        p = p / p.sum(-1, keepdims=True)
        z = 1.0
    A = p * z
    Ab, Aw = np.where(base, A, 0.0), np.where(base, 0.0, A)
    if mode == "causal":
        dA = np.where(base, dot(doh, vh), dot(dow, vh))
        u = mm(Ab, vh) + apply_blocks(Hb, mm(Aw, vh))
    else:
        dA = dot(doh, vh)
        u = mm(A, vh)
    delta = (doh * u).sum(-1, keepdims=True)
    dS = p * ((dA if plant == "dropout_grad_unscaled" else z * dA) - delta)
    dSb, dSw = np.where(base, dS, 0.0), np.where(base, 0.0, dS)
    dqh = scale * mm(dSb, kh)
    dkh = scale * mmT(dSb, qh)
    dvh = mmT(Ab, doh)
    if mode == "causal":
        dqh = dqh + apply_blocks(Hb, scale * mm(dSw, kh))
        dkw, dvw = scale * mmT(dSw, qw), mmT(Aw, dow)
        dkh, dvh = dkh + dkw, dvh + dvw
    c = (np.cross(b3(u), b3(doh)) + np.cross(b3(dqh), b3(qh)) + np.cross(b3(dkh), b3(kh))
         + np.cross(b3(dvh), b3(vh)))
    ab = a.reshape(*a.shape[:-1], nb, 3)
    if mode == "causal":
        c_hol = (np.cross(b3(kh), b3(dkw)) + np.cross(b3(vh), b3(dvw))).sum(-3)
        if plant == "no_holonomy_torque":
            c_hol = 0.0 * c_hol
        da = link_grad_closed(ab, P, c, c_hol)
        back = apply_blocks
    else:
        c = -np.einsum("...bji,...bj->...bi", P, c)                       # c_t = -P_t^T c'_t
        if plant == "inert_torque_sign":
            c = -c
        elif plant == "inert_torque_frame":
            c = np.einsum("...bij,...bj->...bi", P, np.einsum("...bij,...bj->...bi", P, c))
        da = link_grad_from_cross(ab, P, c)
        back = apply_blocks_T
    return {"dq": back(P, dqh), "dk": back(P, dkh), "dv": back(P, dvh), "da": da.reshape(a.shape),
            "dqh": dqh, "dkh": dkh, "dvh": dvh, "delta": delta[..., 0]}


def attention_backward64(qh, kh, vh, oh, doh, scale):
    """Causal softmax attention backward in float64: (dqh, dkh, dvh)."""
    T = qh.shape[-2]
    s = np.einsum("...id,...jd->...ij", qh, kh) * scale
    mask = np.tril(np.ones((T, T), dtype=bool))
    s = np.where(mask, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    dvh = np.einsum("...ij,...id->...jd", p, doh)
    dp = np.einsum("...id,...jd->...ij", doh, vh)
    delta = (doh * oh).sum(-1, keepdims=True)
    ds = p * (dp - delta)
    dqh = np.einsum("...ij,...jd->...id", ds, kh) * scale
    dkh = np.einsum("...ij,...id->...jd", ds, qh) * scale
    return dqh, dkh, dvh


def backward_blocks(x: np.ndarray, W: Dict[str, np.ndarray], n_heads: int, edge_scale: float,
                    dy: np.ndarray, link_mode: str = "additive") -> Dict[str, np.ndarray]:
    """Gradients of <dy, forward_blocks(x)> in float64: the input x, every
    weight, and the intermediates the fused backward produces (dq, dk, dv in
    the reference frame, da the link parameters' gradient)."""
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    B, T, D = x.shape
    H = n_heads
    d = D // H
    nb = n_blocks(d)
    _, pt = forward_blocks(x, W, H, edge_scale, link_mode, return_parts=True)
    P = pt["P"]
    wout = np.asarray(W["out.weight"], np.float64)
    o_flat = pt["o"].transpose(0, 2, 1, 3).reshape(B, T, D)
    do = (dy @ wout).reshape(B, T, H, d).transpose(0, 2, 1, 3)
    doh = apply_blocks_T(P, do)
    dqh, dkh, dvh = attention_backward64(pt["qh"], pt["kh"], pt["vh"], pt["oh"], doh, 1.0 / math.sqrt(d))
    c = (np.cross(_blocks3(pt["oh"], nb), _blocks3(doh, nb)) + np.cross(_blocks3(dqh, nb), _blocks3(pt["qh"], nb))
         + np.cross(_blocks3(dkh, nb), _blocks3(pt["kh"], nb)) + np.cross(_blocks3(dvh, nb), _blocks3(pt["vh"], nb)))
    da = link_grad_from_cross(pt["a"].reshape(B, H, T, nb, 3), P, c).reshape(B, H, T, 3 * nb)
    dq, dk, dv = (apply_blocks(P, g) for g in (dqh, dkh, dvh))
    dqkv = np.concatenate([dq, dk, dv], -1).transpose(0, 2, 1, 3).reshape(B, T, 3 * D)   # [q_h | k_h | v_h]
    grads = {"dq": dq, "dk": dk, "dv": dv, "da": da, "dqh": dqh, "dkh": dkh, "dvh": dvh, "doh": doh,
             "out.weight": dy.reshape(-1, D).T @ o_flat.reshape(-1, D),
             "qkv.weight": dqkv.reshape(-1, 3 * D).T @ x.reshape(-1, D)}
    dx = dqkv @ np.asarray(W["qkv.weight"], np.float64)
    m = 3 * nb
    dg = edge_scale * da.transpose(0, 2, 1, 3)                    # (B, T, H, m): dL/d(generator output)
    if link_mode == "additive":
        dgq = dg.reshape(B, T, H * m)
        dgk = np.roll(dg, 1, axis=1).reshape(B, T, H * m)        # gk_{t+1} enters edge t
        for name, g in (("gqproj.weight", dgq), ("gkproj.weight", dgk)):
            grads[name] = g.reshape(-1, H * m).T @ x.reshape(-1, D)
            dx = dx + g @ np.asarray(W[name], np.float64)
    else:
        xt = torch.as_tensor(x).requires_grad_(True)
        Wt = {k: torch.as_tensor(np.asarray(v, np.float64)).requires_grad_(True)
              for k, v in W.items() if k.startswith("edge_mlp")}
        pair = torch.cat([xt, torch.roll(xt, shifts=-1, dims=1)], dim=-1)
        h = torch.nn.functional.gelu(_linear(pair, Wt["edge_mlp.0.weight"], Wt["edge_mlp.0.bias"]))
        g_out = _linear(h, Wt["edge_mlp.2.weight"], Wt["edge_mlp.2.bias"])
        g_out.backward(torch.as_tensor(dg.reshape(B, T, H * m)))
        dx = dx + xt.grad.numpy()
        for k, v in Wt.items():
            grads[k] = v.grad.numpy()
    grads["x"] = dx
    return grads
