"""Host-side mirror of the qwen35 Gated-DeltaNet operators, on HIP.

Names and argument meaning follow the reference (inference/core/matvec.c,
inference/core/engine.c):

    gdn_gates(alpha, beta, dt_bias, ssm_a)      engine.c:788-793
    gdn_step(S, q, k, v, gate, beta, n_k)       l2norm (engine.c:826-827) +
                                                gdn_state_update (matvec.c:975-1004)
    gdn_chunk(S, q, k, v, gate, beta, n_k)      the same over T tokens in order
    gdn_conv(x, conv_state, conv_w)             conv1d_update + silu (matvec.c:956-968,
                                                engine.c:809-812) over T tokens
    gdn_gated_norm(x, z, w, n_heads)            rmsnorm_gated per v-head (matvec.c:1007-1021)
    gdn_decode(S, conv_in, conv_out, qkv, ...)  one decode token of the layer, all of the above
                                                in one launch (engine.c:786-847)

S is the fp32 state [n_v, d, d] (S[h, j, :] is column j, the reference's
transposed storage), updated in place unless S_out names another buffer (then
S keeps the state before the call).  Tensors are torch fp32 tensors on the
GPU; every call goes through libyllm_hip.so on the current stream, with no CPU
fallback.
"""
from __future__ import annotations

import torch

from ._lib import F16, F32, YhipError, check, lib

L2_EPS = 1e-6  # the qwen35 GDN l2norm epsilon (engine.c:826-827 passes the model's norm eps)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _f32_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda or t.dtype != torch.float32:
            raise YhipError(-22, "GDN tensors must be fp32 on the GPU")


def _rows(t: torch.Tensor) -> tuple[int, int]:
    """(rows, row stride in floats) of a 2-D view with unit inner stride."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise YhipError(-22, "expected a 2-D tensor with contiguous rows")
    return t.shape[0], t.stride(0)


def gdn_gates(alpha: torch.Tensor, beta: torch.Tensor, dt_bias: torch.Tensor, ssm_a: torch.Tensor,
              gate: torch.Tensor | None = None) -> torch.Tensor:
    """alpha, beta: [T, n_v] (beta is replaced by sigmoid(beta)); returns the
    log-decay gate [T, n_v] = softplus(alpha + dt_bias) * ssm_a (written to
    `gate` when given)."""
    _f32_gpu(alpha, beta, dt_bias, ssm_a)
    if alpha.dim() == 1:
        alpha, beta = alpha.unsqueeze(0), beta.unsqueeze(0)
    if not (alpha.is_contiguous() and beta.is_contiguous()) or alpha.shape != beta.shape:
        raise YhipError(-22, "gdn_gates: alpha and beta must be contiguous [T, n_v]")
    T, n_v = alpha.shape
    if dt_bias.numel() != n_v or ssm_a.numel() != n_v:
        raise YhipError(-22, "gdn_gates: dt_bias and ssm_a must have n_v elements")
    if gate is None:
        gate = torch.empty_like(alpha)
    elif gate.shape != alpha.shape or not gate.is_contiguous():
        raise YhipError(-22, "gdn_gates: gate must be contiguous [T, n_v]")
    check(lib().yhip_gdn_gates(beta.data_ptr(), gate.data_ptr(), alpha.data_ptr(), dt_bias.data_ptr(),
                               ssm_a.data_ptr(), T, n_v, _stream()))
    return gate


def gdn_chunk_workspace_bytes(T: int, n_v: int, d: int) -> int:
    return int(lib().yhip_gdn_chunk_workspace(T, n_v, d))


def _state_out(S: torch.Tensor, S_out: torch.Tensor | None) -> int:
    if S_out is None:
        return S.data_ptr()
    _f32_gpu(S_out)
    if S_out.shape != S.shape or not S_out.is_contiguous():
        raise YhipError(-22, "gdn: S_out must be contiguous and shaped like S")
    return S_out.data_ptr()


def gdn_chunk(S: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor,
              beta: torch.Tensor, n_k: int, eps: float = L2_EPS, out: torch.Tensor | None = None,
              workspace: torch.Tensor | None = None, chunked: bool = True,
              S_out: torch.Tensor | None = None) -> torch.Tensor:
    """T tokens in order.  q, k: [T, >= n_k*d]; v: [T, >= n_v*d]; gate, beta:
    [T, n_v].  Returns out [T, n_v*d]; the state after the last token goes
    to S (in place) or to S_out when given (S then keeps the state before the
    call).  eps <= 0 skips the q/k normalisation.  chunked=True uses the
    chunked form (with `workspace`, allocated here when not given);
    chunked=False runs the token-by-token recurrence."""
    _f32_gpu(S, q, k, v, gate, beta)
    if S.dim() != 3 or S.shape[1] != S.shape[2] or not S.is_contiguous():
        raise YhipError(-22, "gdn: S must be contiguous [n_v, d, d]")
    so = _state_out(S, S_out)
    n_v, d = S.shape[0], S.shape[1]
    T, qs = _rows(q)
    Tk, ks = _rows(k)
    Tv, vs = _rows(v)
    if Tk != T or Tv != T or ks != qs:
        raise YhipError(-22, "gdn: q, k, v must have T rows, q and k the same row stride")
    if gate.shape != (T, n_v) or beta.shape != (T, n_v) or not (gate.is_contiguous() and beta.is_contiguous()):
        raise YhipError(-22, "gdn: gate and beta must be contiguous [T, n_v]")
    if out is None:
        out = torch.empty((T, n_v * d), dtype=torch.float32, device=S.device)
    _f32_gpu(out)
    To, os_ = _rows(out)
    if To != T:
        raise YhipError(-22, "gdn: out must have T rows")
    ws_bytes = gdn_chunk_workspace_bytes(T, n_v, d) if chunked else 0
    if ws_bytes and (workspace is None or workspace.numel() * workspace.element_size() < ws_bytes):
        workspace = torch.empty(ws_bytes // 4, dtype=torch.float32, device=S.device)
    ws_ptr = workspace.data_ptr() if ws_bytes else None
    check(lib().yhip_gdn_chunk(S.data_ptr(), so, out.data_ptr(), os_, q.data_ptr(), k.data_ptr(), qs, v.data_ptr(), vs,
                               gate.data_ptr(), beta.data_ptr(), T, n_k, n_v, d, float(eps), ws_ptr, ws_bytes,
                               _stream()))
    return out


def gdn_step(S: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor,
             beta: torch.Tensor, n_k: int, eps: float = L2_EPS, out: torch.Tensor | None = None) -> torch.Tensor:
    """One token: q, k [n_k*d], v [n_v*d], gate, beta [n_v]; returns out [n_v*d]."""
    _f32_gpu(S, q, k, v, gate, beta)
    if S.dim() != 3 or S.shape[1] != S.shape[2] or not S.is_contiguous():
        raise YhipError(-22, "gdn: S must be contiguous [n_v, d, d]")
    n_v, d = S.shape[0], S.shape[1]
    for t, n in ((q, n_k * d), (k, n_k * d), (v, n_v * d), (gate, n_v), (beta, n_v)):
        if t.numel() != n or not t.is_contiguous():
            raise YhipError(-22, "gdn_step: q, k [n_k*d], v [n_v*d], gate, beta [n_v], contiguous")
    if out is None:
        out = torch.empty(n_v * d, dtype=torch.float32, device=S.device)
    check(lib().yhip_gdn_step(S.data_ptr(), out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                              gate.data_ptr(), beta.data_ptr(), n_k, n_v, d, float(eps), _stream()))
    return out


def gdn_conv(x: torch.Tensor, conv_state: torch.Tensor, conv_w: torch.Tensor, silu: bool = True,
             out: torch.Tensor | None = None, state_out: torch.Tensor | None = None) -> torch.Tensor:
    """x: [T, dim] rows (row stride free); conv_state: fp32 [kwidth, dim]
    delay line, updated in place (or, with `state_out`, left as it was and
    the new line written there); conv_w: fp32 [dim, kwidth].  Returns
    silu(conv) rows [T, dim] (a new tensor unless `out` is given; out must
    not overlap x)."""
    _f32_gpu(x, conv_state, conv_w)
    T, xs = _rows(x)
    if conv_state.dim() != 2 or not conv_state.is_contiguous():
        raise YhipError(-22, "gdn_conv: conv_state must be contiguous [kwidth, dim]")
    kwidth, dim = conv_state.shape
    if conv_w.shape != (dim, kwidth) or not conv_w.is_contiguous():
        raise YhipError(-22, "gdn_conv: conv_w must be contiguous [dim, kwidth]")
    if x.shape[1] < dim:
        raise YhipError(-22, "gdn_conv: x rows must hold dim channels")
    if out is None:
        out = torch.empty((T, dim), dtype=torch.float32, device=x.device)
    _f32_gpu(out)
    To, os_ = _rows(out)
    if To != T:
        raise YhipError(-22, "gdn_conv: out must have T rows")
    if state_out is not None:
        _f32_gpu(state_out)
        if state_out.shape != conv_state.shape or not state_out.is_contiguous():
            raise YhipError(-22, "gdn_conv: state_out must be contiguous [kwidth, dim]")
    so = state_out.data_ptr() if state_out is not None else conv_state.data_ptr()
    check(lib().yhip_gdn_conv(out.data_ptr(), os_, x.data_ptr(), xs, conv_state.data_ptr(), so, conv_w.data_ptr(),
                              T, dim, kwidth, int(silu), _stream()))
    return out


def gdn_gated_norm(x: torch.Tensor, z: torch.Tensor, w: torch.Tensor, n_heads: int, eps: float = L2_EPS,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """x, z: [T, n_heads*head_dim] rows; w: [head_dim] fp32 or f16.  Returns
    rmsnorm(x, w) * silu(z) per head (into `out`, which may be x)."""
    _f32_gpu(x, z)
    T, xs = _rows(x)
    Tz, zs = _rows(z)
    head_dim = w.numel()
    if Tz != T or x.shape[1] < n_heads * head_dim or z.shape[1] < n_heads * head_dim:
        raise YhipError(-22, "gdn_gated_norm: x and z must be [T, n_heads*head_dim]")
    if not w.is_cuda or w.dtype not in (torch.float32, torch.float16) or not w.is_contiguous():
        raise YhipError(-22, "gdn_gated_norm: w must be a contiguous fp32 or f16 GPU tensor")
    if out is None:
        out = torch.empty((T, n_heads * head_dim), dtype=torch.float32, device=x.device)
    _f32_gpu(out)
    Ty, ys = _rows(out)
    if Ty != T:
        raise YhipError(-22, "gdn_gated_norm: out must have T rows")
    check(lib().yhip_gdn_gated_norm(out.data_ptr(), ys, x.data_ptr(), xs, z.data_ptr(), zs, w.data_ptr(),
                                    F16 if w.dtype == torch.float16 else F32, T, n_heads, head_dim,
                                    float(eps), _stream()))
    return out


def gdn_decode(S: torch.Tensor, conv_in: torch.Tensor, conv_out: torch.Tensor, qkv: torch.Tensor, z: torch.Tensor,
               alpha: torch.Tensor, beta_raw: torch.Tensor, conv_w: torch.Tensor, dt_bias: torch.Tensor,
               ssm_a: torch.Tensor, norm_w: torch.Tensor, n_k: int, l2_eps: float = L2_EPS,
               norm_eps: float = L2_EPS, y: torch.Tensor | None = None,
               S_out: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token of a GDN layer (engine.c:786-847 after the
    projections): gates, conv1d + silu, l2norm, state update, gated RMSNorm.
    S [n_v, d, d] updated in place (or into S_out); conv_in -> conv_out the delay line
    [kwidth, conv_dim] before / after the token (two buffers, swap them each
    token); qkv [conv_dim] = q | k | v; z [n_v*d]; alpha, beta_raw, dt_bias,
    ssm_a [n_v]; conv_w [conv_dim, kwidth]; norm_w [d] fp32 or f16.
    Returns y [n_v*d]."""
    _f32_gpu(S, conv_in, conv_out, qkv, z, alpha, beta_raw, conv_w, dt_bias, ssm_a)
    n_v, d = S.shape[0], S.shape[1]
    kwidth, conv_dim = conv_in.shape
    if S.shape != (n_v, d, d) or not S.is_contiguous() or conv_out.shape != conv_in.shape:
        raise YhipError(-22, "gdn_decode: S must be contiguous [n_v, d, d]; conv_in / conv_out [kwidth, conv_dim]")
    if conv_dim != (2 * n_k + n_v) * d or conv_w.shape != (conv_dim, kwidth):
        raise YhipError(-22, "gdn_decode: conv_dim must be (2*n_k + n_v)*d and conv_w [conv_dim, kwidth]")
    for t in (conv_in, conv_out, qkv, z, alpha, beta_raw, conv_w, dt_bias, ssm_a, norm_w):
        if not t.is_contiguous():
            raise YhipError(-22, "gdn_decode: tensors must be contiguous")
    if qkv.numel() < conv_dim or z.numel() < n_v * d or min(alpha.numel(), beta_raw.numel(), dt_bias.numel(),
                                                            ssm_a.numel()) < n_v or norm_w.numel() != d:
        raise YhipError(-22, "gdn_decode: input sizes do not match the heads")
    if not norm_w.is_cuda or norm_w.dtype not in (torch.float32, torch.float16):
        raise YhipError(-22, "gdn_decode: norm_w must be fp32 or f16 on the GPU")
    if y is None:
        y = torch.empty(n_v * d, dtype=torch.float32, device=S.device)
    _f32_gpu(y)
    so = _state_out(S, S_out)
    check(lib().yhip_gdn_decode(S.data_ptr(), so, conv_in.data_ptr(), conv_out.data_ptr(), y.data_ptr(), qkv.data_ptr(),
                                z.data_ptr(), alpha.data_ptr(), beta_raw.data_ptr(), conv_w.data_ptr(),
                                dt_bias.data_ptr(), ssm_a.data_ptr(), norm_w.data_ptr(),
                                F16 if norm_w.dtype == torch.float16 else F32, n_k, n_v, d, kwidth, float(l2_eps),
                                float(norm_eps), _stream()))
    return y
