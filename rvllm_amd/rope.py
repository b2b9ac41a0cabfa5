"""RoPE angle tables for rvkv_attn_prep.

rope_cos_sin follows src/model.rs:224-250: theta_j = rope_theta **
(-2 j / head_dim), divided by factors[j] when Llama-3 frequency factors are
given; angle[i, j] = positions[i] * theta_j; the tables are cos and sin of
the angles, f32 [n, head_dim / 2]. Like the reference, the table is built
once per forward on the host (positions are host-side bookkeeping) and
shared by every layer; it is a few KB per step, not part of the hot path.
"""
from __future__ import annotations

import numpy as np


def rope_cos_sin(rope_theta: float, head_dim: int, positions,
                 factors=None):
    half = head_dim // 2
    # Every step is an f32 operation of the reference; pow, cos and sin are
    # evaluated in f64 and rounded once, which gives the correctly rounded
    # f32 result.
    expo = (np.float32(-2.0) * np.arange(half, dtype=np.float32)
            / np.float32(head_dim))
    theta = np.power(np.float64(np.float32(rope_theta)),
                     expo.astype(np.float64)).astype(np.float32)
    if factors is not None:
        theta = theta / np.asarray(factors, np.float32)
    pos = np.asarray(positions).astype(np.float32).reshape(-1, 1)
    angle = (pos * theta.reshape(1, half)).astype(np.float64)
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
