"""Host-side mirror of the reference's per-layer attention operators, on HIP.

Names and argument meaning follow the reference operators that the C ABI
replaces (inference/cuda/cuda_kernels.h:50-63, inference/core/engine.c):

    kv_store(cache, k, v, pos_start)          engine.c:1068-1072 / 518-529
    attn_decode(q, cache, pos, n_heads)       engine.c:1074-1096
    attn_decode_batch(q, caches, lens, ...)   the same per sequence, batched
    attn_prefill(q, cache, pos_start, ...)    engine.c:532-563
    gate=...                                  engine.c:959-960 (qwen35)

Tensors are torch tensors on the GPU (torch is used for device memory and
streams only); every call goes through libyllm_hip.so on the current torch
stream.  Errors raise YhipError with the library's message; there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import BF16, F16, F32, YhipError, check, lib

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise YhipError(-22, f"unsupported dtype {t.dtype}") from None


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need_gpu(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None:
            if not t.is_cuda:
                raise YhipError(-22, "tensor must be on the GPU")
            if not t.is_contiguous():
                raise YhipError(-22, "tensor must be contiguous")


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


@dataclass
class LayerKV:
    """One layer's KV cache of one sequence in HBM.

    k: f16 [n_kv, kv_stride, head_dim]           (row = position)
    v: f16 [n_kv, kv_stride // 32, head_dim, 32] (32-position tiles, d-major)
    """

    k: torch.Tensor
    v: torch.Tensor

    @property
    def n_kv(self) -> int:
        return self.k.shape[0]

    @property
    def kv_stride(self) -> int:
        return self.k.shape[1]

    @property
    def head_dim(self) -> int:
        return self.k.shape[2]

    @classmethod
    def empty(cls, n_kv: int, head_dim: int, max_seq: int, device: str | torch.device = "cuda",
              zero: bool = True) -> "LayerKV":
        stride = round_up(max(max_seq, 1), 64)
        alloc = torch.zeros if zero else torch.empty
        k = alloc((n_kv, stride, head_dim), dtype=torch.float16, device=device)
        v = alloc((n_kv, stride // 32, head_dim, 32), dtype=torch.float16, device=device)
        return cls(k, v)


def kv_store(cache: LayerKV, k: torch.Tensor, v: torch.Tensor, pos_start: int) -> None:
    """Store rows pos_start..pos_start+B-1; k, v: [B, n_kv*head_dim] (f32/f16/bf16)."""
    _need_gpu(k, v, cache.k, cache.v)
    if k.dim() == 1:
        k, v = k.unsqueeze(0), v.unsqueeze(0)
    if k.shape != v.shape or k.dtype != v.dtype or k.shape[1] != cache.n_kv * cache.head_dim:
        raise YhipError(-22, f"kv_store: k {tuple(k.shape)} / v {tuple(v.shape)} do not match the cache")
    check(lib().yhip_kv_store(_ptr(cache.k), _ptr(cache.v), _ptr(k), _ptr(v), _dtype_code(k), pos_start,
                              k.shape[0], cache.n_kv, cache.head_dim, cache.kv_stride, _stream()))


ROPE_NONE, ROPE_PAIRS, ROPE_HALF, ROPE_MROPE = 0, 1, 2, 3


def _rows(t: torch.Tensor, width: int, name: str) -> tuple[torch.Tensor, int]:
    """A [B, >=width] fp32 matrix with unit column stride; returns (t, row stride)."""
    if t.dim() == 1:
        t = t.unsqueeze(0)
    if t.dim() != 2 or t.dtype != torch.float32 or t.stride(1) != 1 or t.shape[1] < width:
        raise YhipError(-22, f"rope_kv_store: {name} must be fp32 [B, >={width}] with unit column stride")
    return t, (t.stride(0) if t.shape[0] > 1 else t.shape[1])


def rope_kv_store(cache: LayerKV, q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor, pos_start: int,
                  n_heads: int, rope: int, theta: float, n_rot: int = 0, q_out: torch.Tensor | None = None,
                  q_out_dtype: torch.dtype = torch.float32) -> torch.Tensor | None:
    """RoPE on q and k for rows at positions pos_start.. (engine.c:1054-1072,
    qwen35 engine.c:910-934), k and v stored into the cache like kv_store.

    q [B, n_heads*head_dim], k and v [B, n_kv*head_dim], fp32, rows may be
    strided slices of one projection output.  rope: ROPE_PAIRS (llama),
    ROPE_HALF (qwen), ROPE_MROPE (qwen35, first n_rot dims) or ROPE_NONE.
    Returns the rotated q (q_out, allocated in q_out_dtype if not given;
    q_out may be q itself), or None when q is None."""
    for t in (q, k, v, q_out):
        if t is not None and not t.is_cuda:
            raise YhipError(-22, "tensor must be on the GPU")
    d = cache.head_dim
    k, ks = _rows(k, cache.n_kv * d, "k")
    v, vs = _rows(v, cache.n_kv * d, "v")
    B = k.shape[0]
    qs = qos = 0
    qdt = F32
    if q is not None:
        q, qs = _rows(q, n_heads * d, "q")
        if q_out is None:
            q_out = torch.empty((B, n_heads * d), dtype=q_out_dtype, device=q.device)
        if q_out.dim() != 2 or q_out.stride(1) != 1 or q_out.shape[0] != B or q_out.shape[1] < n_heads * d:
            raise YhipError(-22, "rope_kv_store: q_out must be [B, >=n_heads*head_dim] with unit column stride")
        qos = q_out.stride(0) if B > 1 else q_out.shape[1]
        qdt = _dtype_code(q_out)
        if q.shape[0] != B:
            raise YhipError(-22, "rope_kv_store: q, k, v row counts differ")
    if v.shape[0] != B:
        raise YhipError(-22, "rope_kv_store: q, k, v row counts differ")
    check(lib().yhip_rope_kv_store(_ptr(q_out) if q is not None else None, qdt, qos, _ptr(q), qs, _ptr(k), ks,
                                   _ptr(v), vs, _ptr(cache.k), _ptr(cache.v), pos_start, B, n_heads, cache.n_kv,
                                   d, cache.kv_stride, rope, n_rot, theta, _stream()))
    return q_out if q is not None else None


def o_proj_workspace_bytes(B: int, hidden: int, qdim: int, w_dtype: torch.dtype,
                           att_dtype: torch.dtype = torch.float32) -> int:
    return int(lib().yhip_o_proj_workspace(B, hidden, qdim, _DT[w_dtype], _DT[att_dtype]))


def o_proj(x: torch.Tensor, att: torch.Tensor, w: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """x[b] += w . att[b] in place (engine.c:969-973: matmul(att_out, SLOT_O) and
    the residual add).  x [B, hidden] f32, att [B, qdim] f32, w [hidden, qdim]
    f16 or f32 (att f16 with f16 weights); rows of x and att may be strided.
    Returns x."""
    for t in (x, att, w):
        if not t.is_cuda:
            raise YhipError(-22, "tensor must be on the GPU")
    if x.dim() == 1:
        x, att = x.unsqueeze(0), att.unsqueeze(0)
    if x.dtype != torch.float32 or att.dtype not in (torch.float32, torch.float16) or x.stride(1) != 1 \
            or att.stride(1) != 1:
        raise YhipError(-22, "o_proj: x (f32) and att (f32 / f16) must be rows with unit column stride")
    if not w.is_contiguous() or w.dim() != 2 or w.shape[1] != att.shape[1] or w.shape[0] != x.shape[1]:
        raise YhipError(-22, f"o_proj: w {tuple(w.shape)} does not match att {tuple(att.shape)} / x {tuple(x.shape)}")
    B, hidden, qdim = x.shape[0], w.shape[0], w.shape[1]
    need = o_proj_workspace_bytes(B, hidden, qdim, w.dtype, att.dtype)
    ws = _workspace(need, x.device, workspace)
    xs = x.stride(0) if B > 1 else hidden
    ats = att.stride(0) if B > 1 else qdim
    check(lib().yhip_o_proj(_ptr(x), xs, _ptr(att), _dtype_code(att), ats, _ptr(w), _dtype_code(w), B, hidden,
                            qdim, _ptr(ws),
                            ws.numel() * ws.element_size() if ws is not None else 0, _stream()))
    return x


def kv_from_engine(cache: LayerKV, eng_k: torch.Tensor, eng_v: torch.Tensor) -> None:
    """Fill rows 0..n-1 from engine-layout f16 rows [n, n_kv*head_dim] (yllm.h:109)."""
    _need_gpu(eng_k, eng_v)
    check(lib().yhip_kv_from_engine(_ptr(cache.k), _ptr(cache.v), _ptr(eng_k), _ptr(eng_v), eng_k.shape[0],
                                    cache.n_kv, cache.head_dim, cache.kv_stride, _stream()))


def kv_to_engine(cache: LayerKV, n_rows: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Rows 0..n_rows-1 in the engine layout, as f16 [n_rows, n_kv*head_dim]."""
    kd = cache.n_kv * cache.head_dim
    ek = torch.empty((n_rows, kd), dtype=torch.float16, device=cache.k.device)
    ev = torch.empty_like(ek)
    check(lib().yhip_kv_to_engine(_ptr(ek), _ptr(ev), _ptr(cache.k), _ptr(cache.v), n_rows, cache.n_kv,
                                  cache.head_dim, cache.kv_stride, _stream()))
    return ek, ev


def decode_workspace_bytes(n_seq: int, max_len: int, total_len: int, n_heads: int, n_kv: int,
                           head_dim: int) -> int:
    return int(lib().yhip_attn_decode_workspace(n_seq, max_len, total_len, n_heads, n_kv, head_dim))


def decode_workspace(nbytes: int, device: torch.device | str = "cuda") -> torch.Tensor:
    """A decode workspace of at least nbytes (see yhip_attn_decode_workspace)."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def _workspace(nbytes: int, device: torch.device, ws: torch.Tensor | None) -> torch.Tensor | None:
    if nbytes == 0:
        return ws
    if ws is not None and ws.numel() * ws.element_size() >= nbytes:
        return ws
    return decode_workspace(nbytes, device)


def attn_decode(q: torch.Tensor, cache: LayerKV, pos: int, n_heads: int, gate: torch.Tensor | None = None,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One query token at position pos over keys 0..pos. q: f32 [n_heads*head_dim]."""
    _need_gpu(q, gate)
    d = cache.head_dim
    if q.dtype != torch.float32 or q.numel() != n_heads * d:
        raise YhipError(-22, "attn_decode: q must be f32 [n_heads*head_dim]")
    if out is None:
        out = torch.empty(n_heads * d, dtype=torch.float32, device=q.device)
    nbytes = decode_workspace_bytes(1, pos + 1, pos + 1, n_heads, cache.n_kv, d)
    ws = _workspace(nbytes, q.device, workspace)
    check(lib().yhip_attn_decode(_ptr(out), _ptr(q), _ptr(cache.k), _ptr(cache.v), pos, n_heads, cache.n_kv,
                                 d, cache.kv_stride, _ptr(gate), _ptr(ws), nbytes, _stream()))
    return out


def attn_decode_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: LayerKV, pos: int, n_heads: int,
                     rope: int, theta: float, n_rot: int = 0, gate: torch.Tensor | None = None,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """rope_kv_store of the token at pos followed by attn_decode, in one
    launch (same result, same cache bits).  q [n_heads*head_dim], k and v
    [n_kv*head_dim]: the token's raw fp32 rows (contiguous); q is not
    modified; k and v are rotated / stored into the cache at pos."""
    _need_gpu(q, k, v, gate)
    d = cache.head_dim
    if (q.dtype != torch.float32 or k.dtype != torch.float32 or v.dtype != torch.float32 or
            q.numel() != n_heads * d or k.numel() != cache.n_kv * d or v.numel() != cache.n_kv * d):
        raise YhipError(-22, "attn_decode_rope: q, k, v must be the token's f32 rows")
    if out is None:
        out = torch.empty(n_heads * d, dtype=torch.float32, device=q.device)
    nbytes = decode_workspace_bytes(1, pos + 1, pos + 1, n_heads, cache.n_kv, d)
    ws = _workspace(nbytes, q.device, workspace)
    check(lib().yhip_attn_decode_rope(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(cache.k), _ptr(cache.v), pos,
                                      n_heads, cache.n_kv, d, cache.kv_stride, rope, n_rot, theta, _ptr(gate),
                                      _ptr(ws), nbytes, _stream()))
    return out


class DecodeBatch:
    """Device tables (K/V base pointers per sequence) for attn_decode_batch."""

    def __init__(self, caches: list[LayerKV]):
        if not caches:
            raise YhipError(-22, "DecodeBatch: no sequences")
        c0 = caches[0]
        for c in caches:
            if (c.n_kv, c.head_dim, c.kv_stride) != (c0.n_kv, c0.head_dim, c0.kv_stride):
                raise YhipError(-22, "DecodeBatch: caches must share n_kv, head_dim and kv_stride")
        dev = c0.k.device
        self.caches = caches
        self.kptrs = torch.tensor([c.k.data_ptr() for c in caches], dtype=torch.int64, device=dev)
        self.vptrs = torch.tensor([c.v.data_ptr() for c in caches], dtype=torch.int64, device=dev)
        self.n_kv, self.head_dim, self.kv_stride = c0.n_kv, c0.head_dim, c0.kv_stride


def attn_decode_batch(q: torch.Tensor, batch: DecodeBatch, lens: list[int] | np.ndarray, n_heads: int,
                      gate: torch.Tensor | None = None, out: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None,
                      lens_dev: torch.Tensor | None = None) -> torch.Tensor:
    """q: f32 [n_seq, n_heads*head_dim]; lens[i] keys for sequence i (0: a zero output row)."""
    _need_gpu(q, gate)
    n_seq = len(batch.caches)
    d = batch.head_dim
    lens = np.asarray(lens, dtype=np.int64)
    if q.dtype != torch.float32 or q.shape != (n_seq, n_heads * d) or lens.shape != (n_seq,):
        raise YhipError(-22, "attn_decode_batch: q must be f32 [n_seq, n_heads*head_dim] and lens [n_seq]")
    if lens_dev is None:
        lens_dev = torch.tensor(lens.astype(np.int32), dtype=torch.int32, device=q.device)
    if out is None:
        out = torch.empty((n_seq, n_heads * d), dtype=torch.float32, device=q.device)
    max_len, total = int(lens.max()), int(lens.sum())
    nbytes = decode_workspace_bytes(n_seq, max_len, total, n_heads, batch.n_kv, d)
    ws = _workspace(nbytes, q.device, workspace)
    gstride = gate.shape[-1] if gate is not None else 0
    check(lib().yhip_attn_decode_batch(_ptr(out), out.shape[1], _ptr(q), q.shape[1], _ptr(batch.kptrs),
                                       _ptr(batch.vptrs), _ptr(lens_dev), n_seq, max_len, total, n_heads,
                                       batch.n_kv, d, batch.kv_stride, _ptr(gate), gstride, _ptr(ws), nbytes,
                                       _stream()))
    return out


def prefill_workspace_bytes(B: int, max_end: int, n_heads: int, n_kv: int, head_dim: int) -> int:
    """Workspace of every attn_prefill of B tokens ending at or before max_end."""
    return int(lib().yhip_attn_prefill_workspace(B, max_end, n_heads, n_kv, head_dim))


def prefill_workspace(nbytes: int, device: torch.device | str = "cuda") -> torch.Tensor:
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def attn_prefill(q: torch.Tensor, cache: LayerKV, pos_start: int, n_heads: int,
                 out_dtype: torch.dtype = torch.float32, gate: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """B prompt tokens at positions pos_start.. ; q: [B, n_heads*head_dim] (f32/f16/bf16).
    q, out and gate may be row slices of larger matrices (unit column stride).
    A launch with few work items splits the keys over a workspace (allocated
    here unless given; see prefill_workspace_bytes)."""
    for t in (q, gate, out):
        if t is not None and (not t.is_cuda or t.dim() != 2 or t.stride(1) != 1):
            raise YhipError(-22, "attn_prefill: q, out and gate must be GPU rows with unit column stride")
    d = cache.head_dim
    if q.shape[1] != n_heads * d:
        raise YhipError(-22, "attn_prefill: q must be [B, n_heads*head_dim]")
    B = q.shape[0]
    if out is None:
        out = torch.empty((B, n_heads * d), dtype=out_dtype, device=q.device)
    if out.shape[0] != B or out.shape[1] != n_heads * d:
        raise YhipError(-22, "attn_prefill: out must be [B, n_heads*head_dim]")
    nbytes = prefill_workspace_bytes(B, pos_start + B, n_heads, cache.n_kv, d)
    ws = _workspace(nbytes, q.device, workspace)
    qs = q.stride(0) if B > 1 else q.shape[1]
    os_ = out.stride(0) if B > 1 else out.shape[1]
    gs = (gate.stride(0) if B > 1 else gate.shape[1]) if gate is not None else 0
    check(lib().yhip_attn_prefill(_ptr(out), _dtype_code(out), os_, _ptr(q), _dtype_code(q), qs, _ptr(cache.k),
                                  _ptr(cache.v), pos_start, B, n_heads, cache.n_kv, d, cache.kv_stride, _ptr(gate),
                                  gs, _ptr(ws), ws.numel() * ws.element_size() if ws is not None else 0,
                                  _stream()))
    return out


# ---- seeded synthetic inputs (host) ----------------------------------------

def synth_normal(seed: int, n: int, sigma: float = 0.5, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().yhip_synth_normal(seed, first, sigma, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n)
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """In place: nearest f16-representable values, reference rounding."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().yhip_synth_round_f16(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size)
    return x


def round_bf16(x: np.ndarray) -> np.ndarray:
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().yhip_synth_round_bf16(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size)
    return x


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().yhip_host_f32_to_f16(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out
