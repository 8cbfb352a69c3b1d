"""Deterministic inputs for the golden fixtures: splitmix64 counters -> Box-Muller normals.

The fixtures store only the reference's outputs; the weights and inputs that produced them are
regenerated here from (name, shape, std), so the committed files stay small. numpy only, so the
same values come out on every machine. Weight values are rounded to bf16 (round to nearest
even), the form the HIP stack stores them in."""
from __future__ import annotations

import zlib

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(name: str, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """float32 N(mean, std^2) of `shape`, a pure function of (name, shape)."""
    n = int(np.prod(shape)) if len(shape) else 1
    seed = np.uint64(zlib.crc32(name.encode()) * 0x100000001)
    i = np.arange((n + 1) // 2, dtype=np.uint64) * np.uint64(2)
    with np.errstate(over="ignore"):
        a = _splitmix64(seed + i)
        b = _splitmix64(seed + i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return (mean + std * z).astype(np.float32).reshape(shape)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) & np.uint64(0xFFFF0000)
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(x))


def weight(name: str, shape, std: float, mean: float = 0.0) -> np.ndarray:
    return bf16_round(normal(name, shape, std, mean))


# Shapes shared by make_fixtures.py and the tests that read the fixtures.
CFG = dict(d_model=256, hk=2, hv=4, dk=128, n_heads=4, n_kv=2, head_dim=256, rotary_dim=64,
           rope_theta=1e7, eps=1e-6)
KINDS = ["delta", "delta", "delta", "attn"]


def layer_weights(prefix: str, kind: str, c: dict = CFG) -> dict:
    """One block's weights in the stack's naming (float32 holding bf16 values)."""
    dm, hk, hv, d = c["d_model"], c["hk"], c["hv"], c["dk"]
    H, KV, HD = c["n_heads"], c["n_kv"], c["head_dim"]
    W = {"norm1": weight(prefix + "norm1", (dm,), 0.1)}
    if kind == "delta":
        C = 2 * hk * d + hv * d
        W.update(w_qkv=weight(prefix + "w_qkv", (C, dm), 0.06), w_z=weight(prefix + "w_z", (hv * d, dm), 0.06),
                 w_b=weight(prefix + "w_b", (hv, dm), 0.06), w_a=weight(prefix + "w_a", (hv, dm), 0.06),
                 conv_w=weight(prefix + "conv_w", (C, 4), 0.3), a_log=weight(prefix + "a_log", (hv,), 0.5),
                 dt_bias=weight(prefix + "dt_bias", (hv,), 0.5),
                 gnorm_w=weight(prefix + "gnorm_w", (d,), 0.1, 1.0),
                 w_out=weight(prefix + "w_out", (dm, hv * d), 0.02))
    else:
        W.update(w_q=weight(prefix + "w_q", (2 * H * HD, dm), 0.06), w_k=weight(prefix + "w_k", (KV * HD, dm), 0.06),
                 w_v=weight(prefix + "w_v", (KV * HD, dm), 0.06), w_o=weight(prefix + "w_o", (dm, H * HD), 0.02),
                 q_norm=weight(prefix + "q_norm", (HD,), 0.1), k_norm=weight(prefix + "k_norm", (HD,), 0.1))
    return W


def feeds(prefix: str, B: int, lengths, d_model: int = CFG["d_model"], std: float = 1.0):
    return [normal(f"{prefix}x{i}", (B, T, d_model), std) for i, T in enumerate(lengths)]
