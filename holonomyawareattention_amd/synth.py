"""Counter-based, platform-independent synthetic inputs.

Every synthetic tensor used by the tests, the golden fixtures and the benchmark
is produced here from an integer seed and a stream name, so that the same
values can be regenerated on any machine without shipping tensors.

Generator: SplitMix64 on the element counter (Steele, Lea & Flood, "Fast
splittable pseudorandom number generators", OOPSLA 2014), 53-bit uniforms in
(0, 1), and the Box-Muller transform (both the cosine and the sine branch are
used, so element 2j and 2j+1 share one uniform pair).
"""
from __future__ import annotations

import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, name: str) -> np.uint64:
    """64-bit key of the stream `name` under `seed` (crc32 of the name)."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * np.uint64(0x100000001B3)
        base = base ^ np.uint64(zlib.crc32(name.encode()))
        return _mix(np.array([base], dtype=np.uint64))[0]


def uniform(seed: int, name: str, n: int, offset: int = 0) -> np.ndarray:
    """n float64 uniforms in (0, 1) for counters offset .. offset+n-1."""
    key = stream_key(seed, name)
    ctr = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = _mix(key + (ctr + np.uint64(1)) * _GOLDEN)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, name: str, shape, std: float = 1.0) -> np.ndarray:
    """float64 array of N(0, std^2) values, row-major over `shape`."""
    shape = tuple(int(s) for s in shape)
    n = int(np.prod(shape)) if shape else 1
    npair = (n + 1) // 2
    out = np.empty(2 * npair, dtype=np.float64)
    step = 1 << 22                                  # bound the temporaries
    for p0 in range(0, npair, step):
        p1 = min(npair, p0 + step)
        u = uniform(seed, name, 2 * (p1 - p0), offset=2 * p0)
        r = np.sqrt(-2.0 * np.log(u[0::2]))
        ang = (2.0 * np.pi) * u[1::2]
        out[2 * p0:2 * p1:2] = r * np.cos(ang)
        out[2 * p0 + 1:2 * p1:2] = r * np.sin(ang)
    out = out[:n]
    if std != 1.0:
        out *= std
    return out.reshape(shape)


def layer_inputs(seed: int, B: int, T: int, d_model: int, n_heads: int,
                 link_mode: str = "additive"):
    """Seeded inputs for one path-ordered attention layer (block rotation model).

    x ~ N(0,1) of shape (B,T,D); projection and generator weights ~ N(0, 1/D)
    (nn.Linear layout: (out_features, in_features)). The generator weights
    have H*m rows with m = 3*(d//3) block parameters per head. For
    link_mode="interaction" the two-layer edge MLP gets N(0, 1/fan_in) weights
    and N(0, 0.1^2) biases, so the bias path is exercised.
    Returns a dict of float64 numpy arrays.
    """
    D, H = d_model, n_heads
    d = D // H
    m = 3 * (d // 3)
    std = 1.0 / np.sqrt(D)
    out = {
        "x": normal(seed, "x", (B, T, D)),
        "qkv.weight": normal(seed, "qkv.weight", (3 * D, D), std),
        "out.weight": normal(seed, "out.weight", (D, D), std),
        "gqproj.weight": normal(seed, "gqproj.weight", (H * m, D), std),
        "gkproj.weight": normal(seed, "gkproj.weight", (H * m, D), std),
    }
    if link_mode == "interaction":
        out["edge_mlp.0.weight"] = normal(seed, "edge_mlp.0.weight", (4 * D, 2 * D), 1.0 / np.sqrt(2 * D))
        out["edge_mlp.0.bias"] = normal(seed, "edge_mlp.0.bias", (4 * D,), 0.1)
        out["edge_mlp.2.weight"] = normal(seed, "edge_mlp.2.weight", (H * m, 4 * D), 1.0 / np.sqrt(4 * D))
        out["edge_mlp.2.bias"] = normal(seed, "edge_mlp.2.bias", (H * m,), 0.1)
    return out


def uniform_ints(seed: int, name: str, shape, high: int) -> np.ndarray:
    """int64 array uniform in [0, high), row-major over `shape`."""
    shape = tuple(int(s) for s in shape)
    n = int(np.prod(shape)) if shape else 1
    u = uniform(seed, name, n)
    return np.minimum((u * high).astype(np.int64), high - 1).reshape(shape)


def decoder_inputs(seed: int, vocab: int, d_model: int, n_heads: int, n_layers: int,
                   link_mode: str = "additive"):
    """Seeded weights of a `HoloDecoder` (keys = its state_dict keys).

    Embedding ~ N(0, 1); per block the attention weights of `layer_inputs`
    (a seed of its own per block), LayerNorm weights 1 + N(0, 0.1^2) and
    biases N(0, 0.1^2) (so the affine part is exercised), MLP weights
    N(0, 1/fan_in) with N(0, 0.1^2) biases; LM head N(0, 1/d_model).
    Returns a dict of float64 numpy arrays.
    """
    D = d_model
    out = {"embed.weight": normal(seed, "embed.weight", (vocab, D))}
    for i in range(n_layers):
        p = f"blocks.{i}."
        core = layer_inputs(seed * 1000003 + i + 1, 1, 1, D, n_heads, link_mode)
        core.pop("x")
        for k, v in core.items():
            out[p + "core." + k] = v
        for ln in ("ln1", "ln2"):
            out[p + ln + ".weight"] = 1.0 + normal(seed, p + ln + ".weight", (D,), 0.1)
            out[p + ln + ".bias"] = normal(seed, p + ln + ".bias", (D,), 0.1)
        out[p + "ff.0.weight"] = normal(seed, p + "ff.0.weight", (4 * D, D), 1.0 / np.sqrt(D))
        out[p + "ff.0.bias"] = normal(seed, p + "ff.0.bias", (4 * D,), 0.1)
        out[p + "ff.2.weight"] = normal(seed, p + "ff.2.weight", (D, 4 * D), 1.0 / np.sqrt(4 * D))
        out[p + "ff.2.bias"] = normal(seed, p + "ff.2.bias", (D,), 0.1)
    out["lm_head.weight"] = normal(seed, "lm_head.weight", (vocab, D), 1.0 / np.sqrt(D))
    return out
