"""CPU restatement of the decoder-step operations around the attention path
(qwen_kernels.cu:13-107: embedding gather, RMSNorm, bias, residual, RoPE in the
rotate-half form, SwiGLU, argmax) and of a Qwen2-shaped decoder forward built from
them (qwen_serve.cu:90-175), in float64 numpy.  Test infrastructure only: the
tests compare the HIP kernels and the GPU model with these on the same inputs.
"""
from __future__ import annotations

import numpy as np


def embed_gather(table, ids):
    """qwen_kernels.cu:13-20; ids outside the table give zero rows."""
    ids = np.asarray(ids)
    V = table.shape[0]
    out = np.zeros((len(ids), table.shape[1]), np.float64)
    ok = (ids >= 0) & (ids < V)
    out[ok] = table[ids[ok]].astype(np.float64)
    return out


def rmsnorm(x, w, eps):
    """qwen_kernels.cu:24-40: x * rsqrt(mean(x^2) + eps) * w per row."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(w, np.float64)


def rope(x, pos, D, theta):
    """qwen_kernels.cu:64-79, rotate-half: x [rows, heads, D], pos [rows]."""
    x = np.asarray(x, np.float64).copy()
    hd = D // 2
    t = np.arange(hd, dtype=np.float64)
    inv = theta ** (-2.0 * t / D)
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]       # [rows, hd]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., :hd].copy(), x[..., hd:].copy()
    x[..., :hd] = x1 * c - x2 * s
    x[..., hd:] = x2 * c + x1 * s
    return x


def silu_mul(gate, up):
    """qwen_kernels.cu:98-104."""
    g = np.asarray(gate, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, np.float64)


def argmax(logits):
    """First index of the row maximum (qwen_kernels.cu argmax)."""
    return np.argmax(np.asarray(logits), axis=-1)


def linear(x, w):
    """y = x w^T (the reference's cuBLAS linear layers)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
