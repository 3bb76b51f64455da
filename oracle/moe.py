"""GLM-style MoE block: sigmoid top-k router, clamped SwiGLU experts, weighted combine.

Test infrastructure only: see the package docstring for who may import this.

Restates native/glm53/moe_ref.py:25-112 (semantics) and native/kernels/moe.vyb:1-170:
  scores = sigmoid(logits); choice = scores + bias (selection only)
  idx = top-k of choice (descending; ties -> lower expert id)
  w = scores[idx] / (sum + 1e-20) * scale
  expert FFN: g = min(gate(x), L); u = clip(up(x), -L, L); e = down(silu(g) * u)
  out = sum_i w_i e_i + shared(x)   (shared expert: weight 1, same clamp)
"""

import numpy as np

SCALE = 2.5
SWIGLU_LIMIT = 10.0


def sigmoid(x):
    x = np.asarray(x, np.float64)
    return 1.0 / (1.0 + np.exp(-x))


def route_logits(logits, topk=8, bias=None, scale=SCALE):
    """logits [T, E] -> (idx int64 [T, topk], w float64 [T, topk]) (moe_ref.py:68-78)."""
    scores = sigmoid(logits)
    choice = scores if bias is None else scores + np.asarray(bias, np.float64)[None, :]
    idx = np.argsort(-choice, axis=-1, kind="stable")[:, :topk]
    w = np.take_along_axis(scores, idx, axis=-1)
    w = w / (w.sum(axis=-1, keepdims=True) + 1e-20) * scale
    return idx, w


def swiglu(g, u, limit=SWIGLU_LIMIT):
    """Clamped SwiGLU (moe_ref.py:81-84)."""
    g = np.minimum(np.asarray(g, np.float64), limit)
    u = np.clip(np.asarray(u, np.float64), -limit, limit)
    return (g * sigmoid(g)) * u


def ffn_rows(x, wg, wu, wd, limit=SWIGLU_LIMIT):
    """x [S, H]; weights in GGUF row layout (out x in): wg/wu [I, H], wd [H, I]."""
    x = np.asarray(x, np.float64)
    return swiglu(x @ np.asarray(wg, np.float64).T, x @ np.asarray(wu, np.float64).T,
                  limit) @ np.asarray(wd, np.float64).T


def moe_forward(x, logits, experts, shared, topk=8, bias=None, scale=SCALE,
                limit=SWIGLU_LIMIT):
    """x [T, H]; experts: callable e -> (wg, wu, wd) row layout; shared: (wg, wu, wd).

    Returns (out float64 [T, H], idx, w). Each (token, expert) FFN is computed once.
    """
    x = np.asarray(x, np.float64)
    idx, w = route_logits(logits, topk, bias, scale)
    T = x.shape[0]
    out = np.zeros_like(x)
    for e in np.unique(idx):
        toks, lanes = np.nonzero(idx == e)
        wg, wu, wd = experts(int(e))
        y = ffn_rows(x[toks], wg, wu, wd, limit)
        out[toks] += w[toks, lanes][:, None] * y
    out += ffn_rows(x, *shared, limit=limit)
    return out, idx, w


def bucket(idx, n_experts):
    """Per-expert token buckets: (counts [E], offsets [E+1], rows [T*k] of (t*k + slot)).

    Rows are grouped by expert in ascending expert id; within an expert in ascending
    (token, slot) order. This is the layout the grouped GEMM consumes.
    """
    idx = np.asarray(idx)
    T, k = idx.shape
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    order = np.argsort(flat, kind="stable")
    return counts, offsets, order
