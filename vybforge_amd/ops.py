"""Host-side mirror of the reference's packed-weight call surface, on torch device tensors.

The reference host picks a kernel by GGUF type id (``gemv_h``/``gemm_h``,
native/host/ridge_decode.vyb:295-328) and fills a parameter block
(``set_gemv``/``set_gemm``, ridge_decode.vyb:264-279). Here the same choice is
``gemv(ty, ...)``/``dequant(ty, ...)`` and the parameters travel as C-ABI arguments.
All calls are asynchronous on torch's current stream and allocate only their outputs.
"""

import math

import torch

from . import _lib
from ._lib import BF16, F16, F32, F64, Q4_GGML, Q4_INTERLEAVED, call  # noqa: F401

GGML_Q4_0 = 2   # ggml_type ids, as the reference dispatches on them
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q5_K = 13
GGML_Q6_K = 14
GGML_IQ2_S = 22
KQUANTS = (GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_IQ2_S)

BLOCK_BYTES = {GGML_Q4_0: 18, GGML_Q8_0: 34, GGML_Q4_K: 144, GGML_Q5_K: 176, GGML_Q6_K: 210, GGML_IQ2_S: 82}
BLOCK_WEIGHTS = {GGML_Q4_0: 32, GGML_Q8_0: 32, GGML_Q4_K: 256, GGML_Q5_K: 256, GGML_Q6_K: 256, GGML_IQ2_S: 256}

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: F64}


def _dt(t):
    try:
        return _DT[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def _ptr(t):
    if t is None:
        return 0
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def row_bytes(ty, K):
    return (K // BLOCK_WEIGHTS[ty]) * BLOCK_BYTES[ty]


# ---- shape checks: the C-ABI sees only pointers, so every size is checked against the tensors
# here, before a launch could read or write past them

def _nbytes(t):
    return t.numel() * t.element_size()


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _check_weights(W, ty, rows, K, what="W"):
    _need(W is not None and _nbytes(W) >= rows * row_bytes(ty, K),
          f"{what} holds {_nbytes(W) if W is not None else 0} B, fewer than {rows} rows of {row_bytes(ty, K)} B")


def _check_out(out, shape, what="out"):
    _need(out.numel() == math.prod(shape), f"{what} has {out.numel()} elements, expected {tuple(shape)}")


def _check_residual(residual, out):
    if residual is not None:
        _need(residual.dtype == out.dtype and residual.numel() == out.numel(),
              "residual must have the output's dtype and shape")


def dequant(ty, W, nblocks, out_dtype=torch.float32, order=Q4_GGML, out=None):
    """Decode nblocks packed blocks to out [nblocks*32] (the bit-exact gate path)."""
    _need(_nbytes(W) >= nblocks * BLOCK_BYTES.get(ty, 0), "W holds fewer than nblocks blocks")
    if out is None:
        out = torch.empty(nblocks * 32, dtype=out_dtype, device=W.device)
    _check_out(out, (nblocks * 32,))
    if ty == GGML_Q4_0:
        call("vybdq_dequant_q4_0", _ptr(W), _ptr(out), nblocks, order, _dt(out.dtype), _stream())
    elif ty == GGML_Q8_0:
        call("vybdq_dequant_q8_0", _ptr(W), _ptr(out), nblocks, _dt(out.dtype), _stream())
    else:
        raise ValueError(f"unsupported GGUF type {ty}")
    return out


def dequant_any(ty, W, n, out_dtype=torch.float32, out=None):
    """Decode the first n weights of a packed tensor of GGML type ty (vybdq_dequant)."""
    _need(ty in BLOCK_BYTES and n % BLOCK_WEIGHTS[ty] == 0, "n must be whole blocks of a known type")
    _need(_nbytes(W) >= n // BLOCK_WEIGHTS[ty] * BLOCK_BYTES[ty], "W holds fewer than n weights")
    if out is None:
        out = torch.empty(n, dtype=out_dtype, device=W.device)
    _check_out(out, (n,))
    call("vybdq_dequant", ty, _ptr(W), _ptr(out), n, _dt(out.dtype), _stream())
    return out


def gemv(ty, W, X, N, K, y_dtype=torch.float32, residual=None, order=Q4_GGML, out=None):
    """Y[m, n] = RS[m, n] + sum_k X[m, k] W[n, k]; X [M, K] or [K]; returns Y [M, N] or [N]."""
    squeeze = X.dim() == 1
    _need(X.shape[-1] == K, f"X has {X.shape[-1]} columns, K = {K}")
    X2 = X.reshape(1, K) if squeeze else X
    M = X2.shape[0]
    _need(ty in BLOCK_BYTES, f"unsupported GGUF type {ty}")
    _check_weights(W, ty, N, K)
    if out is None:
        out = torch.empty((M, N), dtype=y_dtype, device=X.device)
    _check_out(out, (M, N))
    if residual is not None and residual.dtype != out.dtype:
        raise TypeError("residual must have the output dtype")
    _check_residual(residual, out)
    if ty == GGML_Q4_0:
        call("vybdq_gemv_q4_0", _ptr(W), _ptr(X2), _ptr(out), M, N, K, _dt(X2.dtype), _dt(out.dtype),
             _ptr(residual), order, _stream())
    elif ty == GGML_Q8_0:
        call("vybdq_gemv_q8_0", _ptr(W), _ptr(X2), _ptr(out), M, N, K, _dt(X2.dtype), _dt(out.dtype),
             _ptr(residual), _stream())
    elif ty in KQUANTS:
        call("vybdq_gemv", ty, _ptr(W), _ptr(X2), _ptr(out), M, N, K, _dt(X2.dtype), _dt(out.dtype),
             _ptr(residual), _stream())
    else:
        raise ValueError(f"unsupported GGUF type {ty}")
    return out.reshape(N) if squeeze else out


def gemv_q4_0_seg3(X, K, segs, order=Q4_GGML):
    """Fused q4_0 GEMVs sharing X. segs: list of up to 3 (W, Y, N) with Y preallocated."""
    _need(X.numel() == K, f"X holds {X.numel()} elements, K = {K}")
    for i, (W, Y, N) in enumerate(segs):
        _check_weights(W, GGML_Q4_0, N, K, f"segment {i} W")
        _check_out(Y, (N,), f"segment {i} Y")
    args = []
    for i in range(3):
        if i < len(segs):
            W, Y, N = segs[i]
            args += [_ptr(W), _ptr(Y), N, _dt(Y.dtype)]
        else:
            args += [0, 0, 0, F32]
    call("vybdq_gemv_q4_0_seg3", _ptr(X), K, _dt(X.dtype), order, *args, _stream())


def gemv_seg3(ty, X, K, segs):
    """Fused GEMVs of GGUF type ty sharing X [M, K] (or [K]) in one launch (vybdq_gemv_seg3).
    segs: up to 3 (W, Y, N) or (W, Y, N, residual) with Y preallocated [M, N] (or [N])."""
    _need(X.shape[-1] == K, f"X has {X.shape[-1]} columns, K = {K}")
    X2 = X.reshape(1, K) if X.dim() == 1 else X
    M = X2.shape[0]
    for i, seg in enumerate(segs):
        W, Y, N = seg[:3]
        RS = seg[3] if len(seg) > 3 else None
        if N > 0:
            _need(Y.numel() == M * N, f"segment {i}: Y holds {Y.numel()} elements, expected {M} x {N}")
            _check_weights(W, ty, N, K, f"segment {i}: W")
            _need(RS is None or (RS.dtype == Y.dtype and RS.numel() == Y.numel()), f"segment {i}: residual must match Y")
    args = []
    for i in range(3):
        if i < len(segs) and segs[i][2] > 0:
            W, Y, N = segs[i][:3]
            RS = segs[i][3] if len(segs[i]) > 3 else None
            args += [_ptr(W), _ptr(Y), N, _dt(Y.dtype), _ptr(RS)]
        else:
            args += [0, 0, 0, F32, 0]
    call("vybdq_gemv_seg3", ty, _ptr(X2), M, K, _dt(X2.dtype), *args, _stream())


def quant_q8_act(X, out=None):
    """xq8 quantizer: X [M, K] -> (Xq int8 [M, K], Xs float32 [M, K/32]); out: preallocated (Xq, Xs)."""
    X2 = X.reshape(-1, X.shape[-1])
    M, K = X2.shape
    if out is None:
        q = torch.empty((M, K), dtype=torch.int8, device=X.device)
        d = torch.empty((M, K // 32), dtype=torch.float32, device=X.device)
    else:
        q, d = out
    _need(q.dtype == torch.int8 and q.numel() == M * K, "Xq must be int8 [M, K]")
    _need(d.dtype == torch.float32 and d.numel() == M * (K // 32), "Xs must be float32 [M, K/32]")
    call("vybdq_quant_q8_act", _ptr(X2), _ptr(q), _ptr(d), M, K, _dt(X2.dtype), _stream())
    return q, d


XQ8_TYPES = (GGML_Q4_K, GGML_Q5_K, GGML_IQ2_S)


def _check_xq8(Xq, Xs, K):
    _need(Xq.dtype == torch.int8 and Xq.numel() == K, f"Xq must be int8 [{K}]")
    _need(Xs.dtype == torch.float32 and Xs.numel() == K // 32, f"Xs must be float32 [{K // 32}]")


def gemv_xq8(ty, W, Xq, Xs, N, K, y_dtype=torch.float32, residual=None, out=None):
    """Decode GEMV on one xq8 row (vybdq_gemv_xq8): Y[n] = RS[n] + sum_k W[n, k] Xs[k/32] Xq[k];
    ty Q4_K, Q5_K or IQ2_S. Returns Y [N]."""
    _need(ty in XQ8_TYPES, f"xq8 GEMV: unsupported GGUF type {ty}")
    _check_xq8(Xq, Xs, K)
    _check_weights(W, ty, N, K)
    if out is None:
        out = torch.empty(N, dtype=y_dtype, device=Xq.device)
    _need(out.numel() == N, f"out must hold {N} elements")
    _need(residual is None or (residual.dtype == out.dtype and residual.numel() == N), "residual must match out")
    call("vybdq_gemv_xq8", ty, _ptr(W), _ptr(Xq), _ptr(Xs), _ptr(out), N, K, _dt(out.dtype), _ptr(residual),
         _stream())
    return out


def gemv_xq8_seg3(ty, Xq, Xs, K, segs):
    """Fused xq8 GEMVs sharing one xq8 row (vybdq_gemv_xq8_seg3). segs: up to 3 (W, Y, N) or
    (W, Y, N, residual) with Y preallocated [N]."""
    _need(ty in XQ8_TYPES, f"xq8 GEMV: unsupported GGUF type {ty}")
    _check_xq8(Xq, Xs, K)
    args = []
    for i in range(3):
        if i < len(segs) and segs[i][2] > 0:
            W, Y, N = segs[i][:3]
            RS = segs[i][3] if len(segs[i]) > 3 else None
            _check_weights(W, ty, N, K, f"segment {i}: W")
            _need(Y.numel() == N, f"segment {i}: Y must hold {N} elements")
            _need(RS is None or (RS.dtype == Y.dtype and RS.numel() == N), f"segment {i}: residual must match Y")
            args += [_ptr(W), _ptr(Y), N, _dt(Y.dtype), _ptr(RS)]
        else:
            args += [0, 0, 0, F32, 0]
    call("vybdq_gemv_xq8_seg3", ty, _ptr(Xq), _ptr(Xs), K, *args, _stream())


# ---- persistent GEMV chain ---------------------------------------------------------------

def rmsnorm_q8(X, W, eps, y_dtype=None, f32_copy=False, q8=True):
    """RMSNorm of the rows of X [M, N] (or [N]) with the q8 copy of its float32 output
    (vybdq_rmsnorm_q8). Returns (Y or None, Y32 or None, Xq or None, Xs or None)."""
    X2 = X.reshape(1, -1) if X.dim() == 1 else X
    M, N = X2.shape
    _need(W.numel() == N and W.dtype == X2.dtype, "W must be [N] of X's dtype")
    dev = X.device
    Y = torch.empty((M, N), dtype=y_dtype, device=dev) if y_dtype is not None else None
    Y32 = torch.empty((M, N), dtype=torch.float32, device=dev) if f32_copy else None
    Xq = torch.empty((M, N), dtype=torch.int8, device=dev) if q8 else None
    Xs = torch.empty((M, N // 32), dtype=torch.float32, device=dev) if q8 else None
    call("vybdq_rmsnorm_q8", _ptr(X2), _ptr(W), _ptr(Y), _ptr(Y32), _ptr(Xq), _ptr(Xs), M, N, float(eps),
         _dt(X2.dtype), _dt(Y.dtype) if Y is not None else F32, _stream())
    return Y, Y32, Xq, Xs


def swiglu_q8(G, U, h_dtype=torch.float32, q8=True):
    """h = silu(G) * U elementwise with the q8 copy of float32(h) (vybdq_swiglu_q8).
    Returns (H or None, Xq or None, Xs or None)."""
    n = G.numel()
    _need(U.numel() == n and U.dtype == G.dtype, "U must match G")
    dev = G.device
    H = torch.empty(n, dtype=h_dtype, device=dev) if h_dtype is not None else None
    Xq = torch.empty(n, dtype=torch.int8, device=dev) if q8 else None
    Xs = torch.empty(n // 32, dtype=torch.float32, device=dev) if q8 else None
    call("vybdq_swiglu_q8", _ptr(G), _ptr(U), _ptr(H), _ptr(Xq), _ptr(Xs), n, _dt(G.dtype),
         _dt(H.dtype) if H is not None else F32, _stream())
    return H, Xq, Xs


PBLOCK_WORDS = 32        # one stage = the reference's GEMV p-block, 256-byte stride
_YE = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 258, torch.float64: 8}
_XE = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 258}


class Stage:
    """A stage descriptor plus the tensors it points at (kept alive as long as the stage)."""

    def __init__(self, words, refs):
        self.words = words
        self.refs = refs


def pblock(X, K, segs, residual=None, order=Q4_GGML):
    """One stage descriptor (int64 [32]) in the reference GEMV p-block layout.

    segs: up to 3 (W, Y, N) with preallocated Y; W@0 X@8 Y@16 M@24 N@32 K@40 YE@48
    W2@56 NS2@64 Y2@72 YE2@80 W3@88 NS3@96 Y3@104 YE3@112 RS@120 GRID@128 XE@136 ORDER@144.
    The returned Stage holds references to X, W, Y and residual: a descriptor must never
    outlive the memory it points to.
    """
    import numpy as np
    pb = np.zeros(PBLOCK_WORDS, np.int64)
    pb[1], pb[3], pb[5] = _ptr(X), 1, K
    slots = [(0, 2, 4, 6), (7, 9, 8, 10), (11, 13, 12, 14)]
    for i, (W, Y, N) in enumerate(segs):
        w, y, n, ye = slots[i]
        pb[w], pb[y], pb[n], pb[ye] = _ptr(W), _ptr(Y), N, _YE[Y.dtype]
    for i in range(len(segs), 3):
        pb[slots[i][3]] = 8
    pb[15] = _ptr(residual)
    pb[17] = _XE[X.dtype]
    pb[18] = order
    refs = (X, residual) + tuple(t for seg in segs for t in seg[:2])
    return Stage(pb, refs)


class GemvChain:
    """A device-resident chain of GEMV stages run by one persistent launch per call."""

    def __init__(self, ty, stages, device):
        import numpy as np
        self.ty = ty
        self.n = len(stages)
        self.refs = [st.refs for st in stages]
        words = [st.words for st in stages]
        self.max_k = max(int(pb[5]) for pb in words)
        self.pb = torch.from_numpy(np.stack(words)).to(device)
        nbytes = _lib.lib.vybdq_chain_workspace_size(self.n)
        self.ws = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=device)

    def __call__(self):
        call("vybdq_gemv_chain", self.ty, _ptr(self.pb), self.n, PBLOCK_WORDS * 8, self.max_k,
             _ptr(self.ws), _stream())

    def status(self):
        torch.cuda.synchronize()
        return _lib.lib.vybdq_chain_status(_ptr(self.ws))


# ---- EXL3 --------------------------------------------------------------------------------

EXL3_MCG = _lib.EXL3_MCG


def exl3_decode_tiles(trellis, K, N, out_dtype=torch.float16, codebook=_lib.EXL3_MCG):
    """trellis uint16/int16 [K/16, N/16, 64] -> rotated-basis What [K, N]."""
    _need(trellis.numel() == K * N // 4 and trellis.element_size() == 2, "trellis must be 16-bit [K/16, N/16, 64]")
    out = torch.empty((K, N), dtype=out_dtype, device=trellis.device)
    call("vybdq_exl3_decode_tiles", _ptr(trellis), _ptr(out), K, N, codebook, _dt(out_dtype), _stream())
    return out


def exl3_dequant(trellis, suh, svh, K, N, out_dtype=torch.float32, codebook=_lib.EXL3_MCG):
    """Full W [K, N] = diag(suh) Hs What Hs diag(svh)."""
    _need(trellis.numel() == K * N // 4 and trellis.element_size() == 2, "trellis must be 16-bit [K/16, N/16, 64]")
    _need(suh.numel() == K and svh.numel() == N, "suh must hold K and svh N values")
    out = torch.empty((K, N), dtype=out_dtype, device=trellis.device)
    call("vybdq_dequant_exl3", _ptr(trellis), _ptr(suh), _ptr(svh), _ptr(out), K, N, codebook,
         _dt(out_dtype), _stream())
    return out


class Exl3Linear:
    """x [B, K] -> y [B, N] through the fused EXL3 GEMM, with its workspace."""

    def __init__(self, trellis, suh, svh, K, N, codebook=_lib.EXL3_MCG, max_batch=16):
        _need(trellis.numel() == K * N // 4 and trellis.element_size() == 2, "trellis must be 16-bit [K/16, N/16, 64]")
        _need(suh.numel() == K and svh.numel() == N and suh.dtype == svh.dtype == torch.float16,
              "suh must be fp16 [K] and svh fp16 [N]")
        self.t, self.suh, self.svh, self.K, self.N, self.cb = trellis, suh, svh, K, N, codebook
        nbytes = max(_lib.lib.vybdq_exl3_workspace_size(b, K, N) for b in (1, 2, 4, 8, max_batch))
        if nbytes < 0:
            raise ValueError("unsupported EXL3 shape")
        # zero-filled once: the arrival counters at its start must be zero (each call leaves them so)
        self.ws = torch.zeros(nbytes + 256, dtype=torch.uint8, device=trellis.device)
        self.ws_ptr = (self.ws.data_ptr() + 255) // 256 * 256
        self.ws_bytes = nbytes

    def __call__(self, X, y_dtype=torch.float32, out=None):
        B = X.shape[0]
        _need(X.dim() == 2 and X.shape[1] == self.K, f"X must be [B, {self.K}]")
        if out is None:
            out = torch.empty((B, self.N), dtype=y_dtype, device=X.device)
        _check_out(out, (B, self.N))
        call("vybdq_exl3_gemm", _ptr(self.t), _ptr(self.suh), _ptr(self.svh), _ptr(X), _ptr(out), B,
             self.K, self.N, self.cb, _dt(X.dtype), _dt(out.dtype), self.ws_ptr, self.ws_bytes, _stream())
        return out


# ---- prefill GEMM and MoE ------------------------------------------------------------------

def gemm(ty, W, X, N, K, y_dtype=torch.float32, residual=None, out=None, workspace=None):
    """Y [M, N] = X [M, K] W^T (+ residual) through the dequant MFMA GEMM.

    workspace: a GemmWorkspace (split-K partials) or None for the unsplit GEMM."""
    M = X.shape[0]
    _need(X.dim() == 2 and X.shape[1] == K, f"X must be [M, {K}]")
    _need(ty in BLOCK_BYTES, f"unsupported GGUF type {ty}")
    _check_weights(W, ty, N, K)
    if out is None:
        out = torch.empty((M, N), dtype=y_dtype, device=X.device)
    _check_out(out, (M, N))
    _check_residual(residual, out)
    if workspace is None:
        call("vybdq_gemm", ty, _ptr(W), _ptr(X), _ptr(out), M, N, K, _dt(X.dtype), _dt(out.dtype), 0,
             _ptr(residual), _stream())
    else:
        call("vybdq_gemm_ws", ty, _ptr(W), _ptr(X), _ptr(out), M, N, K, _dt(X.dtype), _dt(out.dtype), 0,
             _ptr(residual), workspace.ptr, workspace.nbytes, _stream())
    return out


def gemm_q8_0_i8(W, Xq, Xs, N, K, y_dtype=torch.float32, residual=None, out=None, workspace=None):
    """int8 path: Y [M, N] from xq8-quantized activations (Xq int8 [M, K], Xs float32 [M, K/32])
    and packed Q8_0 rows W, through int8 MFMA with per-block float32 scaling."""
    M = Xq.shape[0]
    _need(Xq.dtype == torch.int8 and Xq.numel() == M * K, f"Xq must be int8 [M, {K}]")
    _need(Xs.dtype == torch.float32 and Xs.numel() == M * (K // 32), f"Xs must be float32 [M, {K // 32}]")
    _check_weights(W, GGML_Q8_0, N, K)
    if out is None:
        out = torch.empty((M, N), dtype=y_dtype, device=Xq.device)
    _check_out(out, (M, N))
    _check_residual(residual, out)
    ws, nb = (workspace.ptr, workspace.nbytes) if workspace is not None else (0, 0)
    call("vybdq_gemm_q8_0_i8", _ptr(W), _ptr(Xq), _ptr(Xs), _ptr(out), M, N, K, _dt(out.dtype), 0, _ptr(residual),
         ws, nb, _stream())
    return out


class GemmWorkspace:
    """256-byte aligned workspace for vybdq_gemm_ws (int8=False) or vybdq_gemm_q8_0_i8 (int8=True),
    sized for the given (M, N, K) shapes."""

    def __init__(self, shapes, device, ty=GGML_Q8_0, int8=False):
        if int8:
            sizes = [_lib.lib.vybdq_gemm_q8_0_i8_workspace_size(M, N, K) for M, N, K in shapes]
        else:
            sizes = [_lib.lib.vybdq_gemm_workspace_size(ty, M, N, K) for M, N, K in shapes]
        self.nbytes = max(sizes + [0])
        self.buf = torch.zeros(self.nbytes + 256, dtype=torch.uint8, device=device)
        self.ptr = (self.buf.data_ptr() + 255) // 256 * 256 if self.nbytes else 0


def router_logits(X, W, y_dtype=torch.float64):
    """Y [T, E] = X [T, H] W^T (W [E, H]) accumulated in float64 (vybdq_router_logits)."""
    T, H = X.shape
    E = W.shape[0]
    _need(W.dim() == 2 and W.shape[1] == H, "W must be [E, H]")
    Y = torch.empty((T, E), dtype=y_dtype, device=X.device)
    call("vybdq_router_logits", _ptr(X), _dt(X.dtype), _ptr(W), _dt(W.dtype), _ptr(Y), _dt(Y.dtype), T, E, H,
         _stream())
    return Y


def moe_route(logits, topk, bias=None, scale=2.5):
    T, E = logits.shape
    _need(bias is None or (bias.numel() == E and bias.dtype == torch.float32), "bias must be float32 [E]")
    idx = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device)
    call("vybdq_moe_route", _ptr(logits), _dt(logits.dtype), _ptr(bias), _ptr(idx), _ptr(w), T, E, topk,
         float(scale), _stream())
    return idx, w


class MoeLayer:
    """GLM-style MoE layer over packed expert tensors (GGUF row layout, stacked per expert)."""

    def __init__(self, ty, w_gate, w_up, w_down, H, I, E, topk=8, shared=None, scale=2.5, limit=10.0,
                 bias=None):
        _check_weights(w_gate, ty, E * I, H, "w_gate")
        _check_weights(w_up, ty, E * I, H, "w_up")
        _check_weights(w_down, ty, E * H, I, "w_down")
        if shared:
            _check_weights(shared[0], ty, I, H, "shared gate")
            _check_weights(shared[1], ty, I, H, "shared up")
            _check_weights(shared[2], ty, H, I, "shared down")
        _need(bias is None or (bias.numel() == E and bias.dtype == torch.float32), "bias must be float32 [E]")
        self.ty, self.H, self.I, self.E, self.topk = ty, H, I, E, topk
        self.w = (w_gate, w_up, w_down)
        self.shared = shared
        self.scale, self.limit, self.bias = scale, limit, bias
        self._ws = None
        self._ws_t = 0

    def _workspace(self, T, device):
        if self._ws is None or self._ws_t < T:
            n = _lib.lib.vybdq_moe_workspace_size(T, self.H, self.I, self.E, self.topk)
            if n < 0:
                raise ValueError("unsupported MoE shape")
            self._ws = torch.empty(n + 256, dtype=torch.uint8, device=device)
            self._ws_t = T
            self._ws_bytes = n
        return (self._ws.data_ptr() + 255) // 256 * 256, self._ws_bytes

    def __call__(self, x, logits, out_dtype=torch.float32, out=None, routing=False, noalloc=False):
        """out [T, H] for x [T, H] and logits [T, E]. noalloc: run through
        vybdq_moe_forward_noalloc (the library's per-GPU scratch instead of this layer's workspace)."""
        T = x.shape[0]
        _need(x.dim() == 2 and x.shape[1] == self.H, f"x must be [T, {self.H}]")
        _need(logits.dim() == 2 and tuple(logits.shape) == (T, self.E), f"logits must be [T, {self.E}]")
        if out is None:
            out = torch.empty((T, self.H), dtype=out_dtype, device=x.device)
        _check_out(out, (T, self.H))
        idx = w = None
        if routing:
            idx = torch.empty((T, self.topk), dtype=torch.int32, device=x.device)
            w = torch.empty((T, self.topk), dtype=torch.float32, device=x.device)
        sg, su, sd = self.shared if self.shared else (None, None, None)
        args = (self.ty, _ptr(x), _dt(x.dtype), _ptr(logits), _dt(logits.dtype),
                _ptr(self.bias), _ptr(self.w[0]), _ptr(self.w[1]), _ptr(self.w[2]), _ptr(sg), _ptr(su), _ptr(sd),
                _ptr(out), _dt(out.dtype), _ptr(idx), _ptr(w), T, self.H, self.I, self.E, self.topk,
                float(self.scale), float(self.limit))
        if noalloc:
            call("vybdq_moe_forward_noalloc", *args, _stream())
        else:
            ws, nb = self._workspace(T, x.device)
            call("vybdq_moe_forward", *args, ws, nb, _stream())
        return (out, idx, w) if routing else out


EXL3_EXPERT_FIELDS = ("gate_proj.trellis", "gate_proj.suh", "gate_proj.svh", "up_proj.trellis", "up_proj.suh",
                      "up_proj.svh", "down_proj.trellis", "down_proj.suh", "down_proj.svh")


class MoeExl3Layer:
    """The GLM-5.3 MoE layer with EXL3 4-bpw routed experts and a bf16 shared expert
    (vybdq_moe_forward_exl3; the reference's native/glm53/glm_engine.vyb:2728-2990).

    experts: E sequences of the 9 device tensors of EXL3_EXPERT_FIELDS (trellis int16
    [in/16, out/16, 64], suh fp16 [in], svh fp16 [out]; gate/up in = H, out = I; down in = I, out = H),
    wherever they live in device memory. shared: (gate [I, H], up [I, H], down [H, I]) bf16 or None.
    bias: the e_score_correction_bias (float32 [E], selection only) or None."""

    def __init__(self, experts, H, I, topk=8, shared=None, scale=2.5, limit=10.0, bias=None):
        E = len(experts)
        _need(E >= 1 and H % 128 == 0 and I % 128 == 0, "need experts and H, I multiples of 128")
        shapes = ((H // 16, I // 16, 64), (H,), (I,)) * 2 + ((I // 16, H // 16, 64), (I,), (H,))
        addrs = []
        for e, ts in enumerate(experts):
            _need(len(ts) == 9, f"expert {e}: need the 9 tensors {EXL3_EXPERT_FIELDS}")
            for f, (t, shp) in enumerate(zip(ts, shapes)):
                ok = (t.element_size() == 2 and t.numel() == math.prod(shp) and t.is_cuda and t.is_contiguous() and
                      (f % 3 != 0 or t.data_ptr() % 16 == 0) and (f % 3 == 0 or t.dtype == torch.float16))
                _need(ok, f"expert {e} {EXL3_EXPERT_FIELDS[f]}: expected 16-bit {shp}")
                addrs.append(t.data_ptr())
        dev = experts[0][0].device
        self.table = torch.tensor(addrs, dtype=torch.int64).to(dev)
        self.experts = [tuple(ts) for ts in experts]  # the table holds their addresses
        if shared is not None:
            for t, shp, what in zip(shared, ((I, H), (I, H), (H, I)), ("gate", "up", "down")):
                _need(t.dtype == torch.bfloat16 and tuple(t.shape) == shp and t.data_ptr() % 16 == 0,
                      f"shared {what} must be bf16 {shp}")
        _need(bias is None or (bias.numel() == E and bias.dtype == torch.float32), "bias must be float32 [E]")
        self.H, self.I, self.E, self.topk = H, I, E, topk
        self.shared, self.scale, self.limit, self.bias = shared, scale, limit, bias
        self._ws, self._ws_bytes = None, 0

    def _workspace(self, T, device):
        n = _lib.lib.vybdq_moe_exl3_workspace_size(T, self.H, self.I, self.E, self.topk)
        if n < 0:
            raise ValueError("unsupported MoE shape")
        if self._ws is None or self._ws_bytes < n:
            self._ws = torch.empty(n + 256, dtype=torch.uint8, device=device)
            self._ws_bytes = n
        return (self._ws.data_ptr() + 255) // 256 * 256, self._ws_bytes

    def __call__(self, x, logits, out_dtype=torch.float32, out=None, routing=False):
        """out [T, H] for x [T, H] and logits [T, E] (and the routing when routing=True)."""
        T = x.shape[0]
        _need(x.dim() == 2 and x.shape[1] == self.H, f"x must be [T, {self.H}]")
        _need(logits.dim() == 2 and tuple(logits.shape) == (T, self.E), f"logits must be [T, {self.E}]")
        if out is None:
            out = torch.empty((T, self.H), dtype=out_dtype, device=x.device)
        _check_out(out, (T, self.H))
        idx = w = None
        if routing:
            idx = torch.empty((T, self.topk), dtype=torch.int32, device=x.device)
            w = torch.empty((T, self.topk), dtype=torch.float32, device=x.device)
        sg, su, sd = self.shared if self.shared else (None, None, None)
        ws, nb = self._workspace(T, x.device)
        call("vybdq_moe_forward_exl3", _ptr(x), _dt(x.dtype), _ptr(logits), _dt(logits.dtype), _ptr(self.bias),
             _ptr(self.table), _ptr(sg), _ptr(su), _ptr(sd), _ptr(out), _dt(out.dtype), _ptr(idx), _ptr(w), T, self.H,
             self.I, self.E, self.topk, float(self.scale), float(self.limit), ws, nb, _stream())
        return (out, idx, w) if routing else out
