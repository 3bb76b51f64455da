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


def router_logits_f64(x, w):
    """Router logits [T, E] = x [T, H] w [E, H]^T in float64 in the library's summation order
    (H % 32 == 0): wave q of 4 sums the quarter [q H/4, (q+1) H/4), lane l of 64 the elements
    q H/4 + 512 k + 8 l + j in (k, j) order, each as a product then a sum; the 64 lane sums fold
    as s_l + s_(l xor d), d = 32 .. 1; the wave sums add as ((w0 + w1) + w2) + w3
    (glm_engine.vyb:2728-2745 computes the same float64 matmul in its own order)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    T, H = x.shape
    E = w.shape[0]
    Hq = H // 4
    lanes = np.arange(64)
    out = np.empty((T, E))
    for t in range(T):
        ws = []
        for q in range(4):
            part = np.zeros((E, 64))
            for k in range(0, Hq, 512):
                for j in range(8):
                    h = q * Hq + k + 8 * lanes + j
                    ok = (k + 8 * lanes) < Hq
                    hh = np.where(ok, h, 0)
                    part = np.where(ok[None, :], part + x[t, hh][None, :] * w[:, hh], part)
            for d in (32, 16, 8, 4, 2, 1):
                part = part + part[:, lanes ^ d]
            ws.append(part[:, 0])
        out[t] = ((ws[0] + ws[1]) + ws[2]) + ws[3]
    return out


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


def fixture_route(lg32, bias, topk=8, scale=SCALE):
    """moe_route's selection and weights (native/kernels/moe.vyb:53-89) from float32 logits:
    greedy rounds, each taking the first expert (ascending id) whose sigmoid(logit) + bias is
    strictly above both -1e9 and every other unused choice, expert 0 when none is; weights
    sigmoid(logit[idx]) / (sum + 1e-20) * scale summed in lane order. float64."""
    lg = np.asarray(lg32, np.float64)
    S, E = lg.shape
    sc = sigmoid(lg) + np.asarray(bias, np.float64)[None, :]
    idx = np.zeros((S, topk), np.int64)
    for s in range(S):
        used = np.zeros(E, bool)
        for l in range(topk):
            cand = np.where(used | ~(sc[s] > -1e9), -np.inf, sc[s])
            best = int(np.argmax(cand)) if np.isfinite(cand).any() else 0
            idx[s, l] = best
            used[best] = True
    raw = sigmoid(np.take_along_axis(lg, idx, axis=1))
    tot = np.zeros(S)
    for l in range(topk):
        tot = tot + raw[:, l]
    return idx, raw / (tot[:, None] + 1e-20) * scale


def fixture_block(y, G, bias, wg_e, wu_e, wd_e, wg_s, wu_s, wd_s, topk=8, scale=SCALE,
                  limit=SWIGLU_LIMIT):
    """The reference's MoE fixture kernels (native/kernels/moe.vyb:1-170) in float64: weights dense
    [in][out] (gate/up [H][I], down [I][H]); every routed lane uses the one expert (wg_e, wu_e,
    wd_e), lane topk is the shared expert. Returns (LG float64 [S, E], idx [S, topk], w [S, topk],
    act float64 [S, topk + 1, I], out float64 [S, H]); routing runs on float32-rounded logits
    as the kernels store them."""
    y = np.asarray(y, np.float64)
    lg = y @ np.asarray(G, np.float64).T
    idx, w = fixture_route(lg.astype(np.float32), bias, topk, scale)
    a_e = swiglu(y @ np.asarray(wg_e, np.float64), y @ np.asarray(wu_e, np.float64), limit)
    a_s = swiglu(y @ np.asarray(wg_s, np.float64), y @ np.asarray(wu_s, np.float64), limit)
    act = np.concatenate([np.repeat(a_e[:, None, :], topk, axis=1), a_s[:, None, :]], axis=1)
    part = a_e @ np.asarray(wd_e, np.float64)
    out = np.zeros_like(part)
    for l in range(topk):
        out = out + w[:, l:l + 1] * part
    out = out + a_s @ np.asarray(wd_s, np.float64)
    return lg, idx, w, act, out
