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


def _r16(a):
    """Round to fp16 and back: the GPU stores every kernel's output in fp16."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def decoder_logits(W, cfg, tokens, logits_from=0, round16=True):
    """Teacher-forced forward of one token sequence through the Qwen2-shaped decoder
    (qwen_serve.cu:97-121 for every position at once: causal attention over the
    prefix), returning float64 logits [T, vocab].  W maps names to fp16 arrays
    (kvcache_amd.model.QwenModel.tensor layout: [out, in] row-major); fp16 rounding is
    applied where the GPU stores a kernel's output, arithmetic is float32 (GEMMs) and
    float64 (norms, softmax).  Rows before `logits_from` are left out of the lm_head
    (the returned array still has T rows; those are zero).  round16=False runs the
    same statements in float64 without the fp16 stores (the form compared with the
    Hugging Face Qwen2 forward)."""
    H, Hq, Hkv, D = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    I, V = cfg.inter, cfg.vocab
    tok = np.asarray(tokens)
    T = len(tok)
    if round16:
        f32, r16 = (lambda a: np.asarray(a, np.float32)), _r16
    else:
        f32 = r16 = lambda a: np.asarray(a, np.float64)
    embed = W["embed"].reshape(V, H)
    x = f32(embed[tok])
    pos = np.arange(T)
    mask = np.triu(np.ones((T, T), bool), 1)
    g = Hq // Hkv
    for l in range(cfg.layers):
        w = lambda n, shape: f32(W[f"{n}.{l}"].reshape(shape))
        n = r16(rmsnorm(x, w("ln1", (H,)), cfg.eps))
        q = r16(r16(n @ w("wq", (Hq * D, H)).T) + w("bq", (Hq * D,)))
        k = r16(r16(n @ w("wk", (Hkv * D, H)).T) + w("bk", (Hkv * D,)))
        v = r16(r16(n @ w("wv", (Hkv * D, H)).T) + w("bv", (Hkv * D,)))
        q = r16(rope(q.reshape(T, Hq, D), pos, D, cfg.theta))
        k = r16(rope(k.reshape(T, Hkv, D), pos, D, cfg.theta))
        v = v.reshape(T, Hkv, D).astype(np.float64)
        att = np.empty((T, Hq, D))
        for h in range(Hq):
            s = q[:, h].astype(np.float64) @ k[:, h // g].astype(np.float64).T / np.sqrt(D)
            s[mask] = -np.inf
            s = np.exp(s - s.max(axis=1, keepdims=True))
            att[:, h] = (s / s.sum(axis=1, keepdims=True)) @ v[:, h // g]
        att = r16(att.reshape(T, Hq * D))
        x = r16(x + r16(att @ w("wo", (H, Hq * D)).T))
        n = r16(rmsnorm(x, w("ln2", (H,)), cfg.eps))
        a = r16(silu_mul(r16(n @ w("wg", (I, H)).T), r16(n @ w("wu", (I, H)).T)))
        x = r16(x + r16(a @ w("wd", (H, I)).T))
    out = np.zeros((T, V), np.float64)
    n = r16(rmsnorm(x[logits_from:], f32(W["norm"]), cfg.eps))
    out[logits_from:] = n @ f32(embed).T
    return out


def teacher_forced_check(logits_cpu, prompt_len, generated, margin):
    """Generated token i is predicted at position prompt_len - 1 + i.  Returns
    (exact matches, list of (i, gpu token, cpu top token, cpu logit gap)) for the
    mismatches whose CPU gap exceeds `margin` (near-ties within it are tolerated)."""
    exact, bad = 0, []
    for i, t in enumerate(generated):
        row = logits_cpu[prompt_len - 1 + i]
        top = int(np.argmax(row))
        if top == int(t):
            exact += 1
        elif row[top] - row[int(t)] > margin:
            bad.append((i, int(t), top, float(row[top] - row[int(t)])))
    return exact, bad
