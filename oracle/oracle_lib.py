"""ctypes wrappers for the CPU oracle (oracle/liboracle.so) and for the
reference built from its own sources (oracle/_ref/libyref.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the checker / the timed CPU path,
never as part of the product."""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int, c_uint16, c_uint32, c_uint64
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libyref.so"

FP = POINTER(c_float)
HP = POINTER(c_uint16)


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(FP)


def hp(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(HP)


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        L = ctypes.CDLL(str(path))
        L.yo_threads.restype = c_int
        L.yo_threads.argtypes = []
        L.yo_f16_to_f32.restype = c_float
        L.yo_f16_to_f32.argtypes = [c_uint16]
        L.yo_f32_to_f16.restype = c_uint16
        L.yo_f32_to_f16.argtypes = [c_float]
        L.yo_bf16_to_f16.restype = c_uint16
        L.yo_bf16_to_f16.argtypes = [c_uint16]
        L.yo_f32_to_f16_buf.argtypes = [FP, HP, ctypes.c_size_t]
        L.yo_softmax.argtypes = [FP, c_uint32]
        L.yo_l2norm.argtypes = [FP, c_uint32, c_float]
        L.yo_kv_store.argtypes = [HP, HP, FP, FP, c_uint32, c_uint32, c_uint32]
        L.yo_attn_decode.argtypes = [FP, FP, HP, HP, c_uint32, c_uint32, c_uint32, c_uint32]
        L.yo_attn_prefill.argtypes = [FP, FP, HP, HP, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                      c_uint32]
        L.yo_gate_sigmoid.argtypes = [FP, FP, c_uint32]
        L.yo_gdn_gates.argtypes = [FP, FP, FP, FP, FP, c_uint32]
        L.yo_conv1d_update.argtypes = [FP, FP, FP, c_uint32, c_uint32]
        L.yo_conv_silu_sequence.argtypes = [FP, FP, FP, c_uint32, c_uint32, c_uint32]
        L.yo_rmsnorm_gated.argtypes = [FP, FP, ctypes.c_void_p, ctypes.c_int, FP, c_uint32, c_float]
        L.yo_rope.argtypes = [FP, c_uint32, c_uint32, c_float, c_int, c_uint32]
        L.yo_matmul.argtypes = [FP, FP, ctypes.c_void_p, c_int, c_uint32, c_uint32]
        L.yo_o_proj.argtypes = [FP, FP, ctypes.c_void_p, c_int, c_uint32, c_uint32, c_uint32]
        L.yo_rope_kv_store.argtypes = [FP, FP, FP, HP, HP, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_int,
                                       c_uint32, c_float]
        L.yo_gdn_state_update.argtypes = [FP, FP, FP, FP, FP, FP, FP, c_uint32, c_uint32, c_uint32, c_uint32]
        L.yo_gdn_sequence.argtypes = [FP, FP, FP, FP, FP, FP, FP, c_uint32, c_uint32, c_uint32, c_uint32,
                                      c_uint32, c_float]
        self.L = L

    # conversions
    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.L.yo_f32_to_f16_buf(fp(x), hp(out), x.size)
        return out

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        return np.array([self.L.yo_f16_to_f32(int(v)) for v in np.ravel(h)], dtype=np.float32).reshape(h.shape)

    def softmax(self, v: np.ndarray) -> np.ndarray:
        v = np.array(v, dtype=np.float32)
        self.L.yo_softmax(fp(v), v.size)
        return v

    def kv_store(self, kc, vc, k, v, pos_start, kv_dim):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        self.L.yo_kv_store(hp(kc), hp(vc), fp(k), fp(v), pos_start, k.size // kv_dim, kv_dim)

    def decode(self, q, kc, vc, pos, n_heads, n_kv, hd) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.empty(n_heads * hd, dtype=np.float32)
        self.L.yo_attn_decode(fp(out), fp(q), hp(kc), hp(vc), pos, n_heads, n_kv, hd)
        return out

    def prefill(self, q, kc, vc, pos_start, B, n_heads, n_kv, hd) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.empty((B, n_heads * hd), dtype=np.float32)
        self.L.yo_attn_prefill(fp(out), fp(q), hp(kc), hp(vc), pos_start, B, n_heads, n_kv, hd, n_heads * hd)
        return out

    def gate_sigmoid(self, x, gate) -> np.ndarray:
        x = np.array(x, dtype=np.float32)
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        self.L.yo_gate_sigmoid(fp(x), fp(gate), x.size)
        return x

    def gdn_gates(self, alpha_raw, beta_raw, dt, a):
        beta = np.array(beta_raw, dtype=np.float32)
        gate = np.empty_like(beta)
        self.L.yo_gdn_gates(fp(beta), fp(gate), fp(np.ascontiguousarray(alpha_raw, dtype=np.float32)),
                            fp(np.ascontiguousarray(dt, dtype=np.float32)),
                            fp(np.ascontiguousarray(a, dtype=np.float32)), beta.size)
        return beta, gate

    def gdn_step(self, S, q, k, v, gate, beta, n_k, hk, n_v, hv):
        S = np.array(S, dtype=np.float32)
        out = np.empty(n_v * hv, dtype=np.float32)
        self.L.yo_gdn_state_update(fp(S), fp(out), fp(np.ascontiguousarray(q, np.float32)),
                                   fp(np.ascontiguousarray(k, np.float32)), fp(np.ascontiguousarray(v, np.float32)),
                                   fp(np.ascontiguousarray(gate, np.float32)),
                                   fp(np.ascontiguousarray(beta, np.float32)), n_k, hk, n_v, hv)
        return S, out

    def gdn_sequence(self, S, q, k, v, gate, beta, T, n_k, hk, n_v, hv, eps):
        S = np.array(S, dtype=np.float32)
        q = np.array(q, dtype=np.float32)
        k = np.array(k, dtype=np.float32)
        out = np.empty((T, n_v * hv), dtype=np.float32)
        self.L.yo_gdn_sequence(fp(S), fp(out), fp(q), fp(k), fp(np.ascontiguousarray(v, np.float32)),
                               fp(np.ascontiguousarray(gate, np.float32)),
                               fp(np.ascontiguousarray(beta, np.float32)), T, n_k, hk, n_v, hv, eps)
        return S, out, q, k


def _conv_args(state, x, w):
    return (np.array(state, dtype=np.float32, order="C", copy=True), np.array(x, dtype=np.float32, order="C", copy=True),
            np.ascontiguousarray(w, dtype=np.float32))


def _oracle_conv(self, state, x, w, kwidth):
    """matvec.c:956-968 over the rows of x: returns (new state, conv rows)."""
    st, xr, wc = _conv_args(state, x, w)
    dim = xr.shape[-1]
    for row in xr.reshape(-1, dim):
        self.L.yo_conv1d_update(fp(st), fp(row), fp(wc), dim, kwidth)
    return st, xr


def _oracle_conv_silu(self, state, x, w, kwidth):
    """engine.c:809-812 over T rows: conv then silu; returns (state, rows)."""
    st, xr, wc = _conv_args(state, x, w)
    T, dim = xr.shape
    self.L.yo_conv_silu_sequence(fp(st), fp(xr), fp(wc), T, dim, kwidth)
    return st, xr


def _oracle_rmsnorm_gated(self, x, w, z, eps):
    """matvec.c:1007-1021 per row of x (w f32, or f16 bits as uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    z = np.ascontiguousarray(z, dtype=np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    w_f16 = int(w.dtype == np.uint16)
    w = np.ascontiguousarray(w)
    for yr, xr, zr in zip(y.reshape(-1, n), x.reshape(-1, n), z.reshape(-1, n)):
        self.L.yo_rmsnorm_gated(fp(yr), fp(xr), w.ctypes.data_as(ctypes.c_void_p), w_f16, fp(zr), n, eps)
    return y


def _rope_rows(fn, x, pos, d):
    """Apply fn(head, pos) to every head of d floats of x [B][..., n*d]; row b at pos[b]."""
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    rows = y.reshape(y.shape[0], -1, d)
    for b in range(rows.shape[0]):
        for h in range(rows.shape[1]):
            head = np.ascontiguousarray(rows[b, h])
            fn(head, int(pos[b]))
            rows[b, h] = head
    return y


def _oracle_rope(self, x, pos, d, theta, kind, n_rot=0):
    """yo_rope over every head of every row of x [B][n*d] (row b at position pos[b])."""
    return _rope_rows(lambda h, p: self.L.yo_rope(fp(h), d, p, theta, kind, n_rot), x, pos, d)


def _oracle_rope_kv_store(self, q, k, v, pos_start, n_heads, n_kv, d, theta, kind, n_rot=0):
    """yo_rope_kv_store on B rows: returns (rotated q, K rows, V rows) with
    the caches as engine rows pos_start..pos_start+B-1 [B][n_kv*d] (u16)."""
    q = np.array(q, np.float32, order="C", copy=True)
    k = np.array(k, np.float32, order="C", copy=True)
    v = np.ascontiguousarray(v, np.float32)
    B = q.shape[0]
    kvd = n_kv * d
    kc = np.zeros((pos_start + B, kvd), np.uint16)
    vc = np.zeros_like(kc)
    self.L.yo_rope_kv_store(fp(q), fp(k), fp(v), hp(kc), hp(vc), pos_start, B, n_heads, n_kv, d, kind, n_rot,
                            theta)
    return q, kc[pos_start:], vc[pos_start:]


def _oracle_matmul(self, x, w):
    """yo_matmul of one row x [in] with w [out][in] (f32, or f16 bits as uint16)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w)
    y = np.empty(w.shape[0], np.float32)
    self.L.yo_matmul(fp(y), fp(x), w.ctypes.data_as(ctypes.c_void_p), int(w.dtype == np.uint16), w.shape[0],
                     w.shape[1])
    return y


def _oracle_o_proj(self, x, att, w):
    """yo_o_proj: x [B][hidden] + matmul(att [B][qdim], w [hidden][qdim]) per row (new array)."""
    x = np.array(x, np.float32, order="C", copy=True)
    att = np.ascontiguousarray(att, np.float32)
    w = np.ascontiguousarray(w)
    self.L.yo_o_proj(fp(x), fp(att), w.ctypes.data_as(ctypes.c_void_p), int(w.dtype == np.uint16), x.shape[0],
                     w.shape[0], w.shape[1])
    return x


Oracle.matmul = _oracle_matmul
Oracle.o_proj = _oracle_o_proj
Oracle.rope = _oracle_rope
Oracle.rope_kv_store = _oracle_rope_kv_store
Oracle.conv = _oracle_conv
Oracle.conv_silu = _oracle_conv_silu
Oracle.rmsnorm_gated = _oracle_rmsnorm_gated


class Ref:
    """The reference compiled from its own sources (oracle/_ref)."""

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (make -C oracle ref)")
        L = ctypes.CDLL(str(path))
        L.f16_to_f32.restype = c_float
        L.f16_to_f32.argtypes = [c_uint16]
        L.f32_to_f16_buf.argtypes = [FP, HP, ctypes.c_size_t]
        L.bf16_to_f16.restype = c_uint16
        L.bf16_to_f16.argtypes = [c_uint16]
        L.softmax.argtypes = [FP, c_uint32]
        L.l2norm_inplace.argtypes = [FP, c_uint32, c_float]
        L.gdn_state_update.argtypes = [FP, FP, FP, FP, FP, FP, FP, c_uint32, c_uint32, c_uint32, c_uint32]
        L.conv1d_update.argtypes = [FP, FP, ctypes.c_void_p, c_uint32, c_uint32]
        L.rmsnorm_gated.argtypes = [FP, FP, ctypes.c_void_p, FP, c_uint32, c_float, c_uint32]
        L.matmul.argtypes = [FP, FP, ctypes.c_void_p, c_uint32, c_uint32, c_uint32]
        L.rope_inplace.argtypes = [FP, c_uint32, c_uint32, c_float]
        L.rope_inplace_qwen.argtypes = [FP, c_uint32, c_uint32, c_float]
        L.rope_inplace_mrope.argtypes = [FP, c_uint32, c_uint32, c_uint32, c_float]
        L.yrng.restype = c_uint64
        L.yrng.argtypes = [POINTER(c_uint64)]
        L.ysrand.restype = c_uint64
        L.ysrand.argtypes = [c_uint64]
        L.yr_decode.restype = c_int
        L.yr_decode.argtypes = [c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, HP, HP, FP, FP, FP, c_float,
                                FP, HP, HP, FP]
        L.yr_prefill.restype = c_int
        L.yr_prefill.argtypes = [c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, HP, HP, FP, FP, FP,
                                 c_float, FP, HP, HP, FP]
        L.yr_gated.restype = c_int
        L.yr_gated.argtypes = [c_uint32, c_uint32, c_uint32, c_uint32, HP, HP, FP, FP, FP, FP, c_float, FP, FP,
                               HP, HP, FP]
        L.yr_gdn.restype = c_int
        L.yr_gdn.argtypes = [c_uint32, c_uint32, c_uint32, FP, FP, FP, FP, FP, c_float, FP, FP, FP, FP, FP, FP,
                             FP, FP]
        self.L = L

    def conv(self, state, x, w, kwidth):
        """The reference's conv1d_update (matvec.c:956) over the rows of x."""
        st, xr, wc = _conv_args(state, x, w)
        dim = xr.shape[-1]
        for row in xr.reshape(-1, dim):
            self.L.conv1d_update(fp(st), fp(row), wc.ctypes.data_as(ctypes.c_void_p), dim, kwidth)
        return st, xr

    def rmsnorm_gated(self, x, w, z, eps):
        """The reference's rmsnorm_gated (matvec.c:1007) per row (w f32 or f16 bits)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        z = np.ascontiguousarray(z, dtype=np.float32)
        y = np.empty_like(x)
        n = x.shape[-1]
        dtype = 0 if w.dtype == np.uint16 else 1  # DT_F16 = 0, DT_F32 = 1 (llf.h:14-15)
        w = np.ascontiguousarray(w)
        for yr, xr, zr in zip(y.reshape(-1, n), x.reshape(-1, n), z.reshape(-1, n)):
            self.L.rmsnorm_gated(fp(yr), fp(xr), w.ctypes.data_as(ctypes.c_void_p), fp(zr), n, eps, dtype)
        return y

    def rope(self, x, pos, d, theta, kind, n_rot=0):
        """The reference's rope_inplace (kind 1), rope_inplace_qwen (2) or
        rope_inplace_mrope (3) (matvec.c:890-939) on every head of x."""
        L = self.L
        fns = {0: lambda h, p: None,
               1: lambda h, p: L.rope_inplace(fp(h), d, p, theta),
               2: lambda h, p: L.rope_inplace_qwen(fp(h), d, p, theta),
               3: lambda h, p: L.rope_inplace_mrope(fp(h), d, n_rot, p, theta)}
        return _rope_rows(fns[kind], x, pos, d)

    def matmul(self, x, w):
        """The reference's matmul (matvec.c:785): DT_F32 for f32 w, DT_F16 for f16 bits."""
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w)
        y = np.empty(w.shape[0], np.float32)
        self.L.matmul(fp(y), fp(x), w.ctypes.data_as(ctypes.c_void_p), w.shape[0], w.shape[1],
                      0 if w.dtype == np.uint16 else 1)  # DT_F16 = 0, DT_F32 = 1 (llf.h:14-15)
        return y

    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.L.f32_to_f16_buf(fp(x), hp(out), x.size)
        return out

    def decode(self, arch, n_heads, n_kv, hd, pos, kprev, vprev, wq, wk, wv, xval=1.0):
        hidden, kvd = n_heads * hd, n_kv * hd
        q = np.empty(hidden, np.float32)
        kr = np.empty((pos + 1, kvd), np.uint16)
        vr = np.empty((pos + 1, kvd), np.uint16)
        att = np.empty(hidden, np.float32)
        kp = np.ascontiguousarray(kprev if pos else np.zeros((1, kvd), np.uint16), np.uint16)
        vp = np.ascontiguousarray(vprev if pos else np.zeros((1, kvd), np.uint16), np.uint16)
        rc = self.L.yr_decode(arch, n_heads, n_kv, hd, pos, hp(kp), hp(vp), fp(np.float32(wq)), fp(np.float32(wk)),
                              fp(np.float32(wv)), xval, fp(q), hp(kr), hp(vr), fp(att))
        assert rc == 0, f"yr_decode rc={rc}"
        return q, kr, vr, att

    def prefill(self, arch, n_heads, n_kv, hd, pos_start, B, kprev, vprev, wq, wk, wv, xval=1.0):
        hidden, kvd = n_heads * hd, n_kv * hd
        q = np.empty((B, hidden), np.float32)
        kr = np.empty((pos_start + B, kvd), np.uint16)
        vr = np.empty((pos_start + B, kvd), np.uint16)
        att = np.empty((B, hidden), np.float32)
        kp = np.ascontiguousarray(kprev if pos_start else np.zeros((1, kvd), np.uint16), np.uint16)
        vp = np.ascontiguousarray(vprev if pos_start else np.zeros((1, kvd), np.uint16), np.uint16)
        rc = self.L.yr_prefill(arch, n_heads, n_kv, hd, pos_start, B, hp(kp), hp(vp),
                               fp(np.ascontiguousarray(wq, np.float32)), fp(np.ascontiguousarray(wk, np.float32)),
                               fp(np.ascontiguousarray(wv, np.float32)), xval, fp(q), hp(kr), hp(vr), fp(att))
        assert rc == 0, f"yr_prefill rc={rc}"
        return q, kr, vr, att

    def gated(self, n_heads, n_kv, hd, pos, kprev, vprev, wq, wg, wk, wv, xval=1.0):
        hidden, kvd = n_heads * hd, n_kv * hd
        q = np.empty(hidden, np.float32)
        g = np.empty(hidden, np.float32)
        kr = np.empty((pos + 1, kvd), np.uint16)
        vr = np.empty((pos + 1, kvd), np.uint16)
        att = np.empty(hidden, np.float32)
        kp = np.ascontiguousarray(kprev if pos else np.zeros((1, kvd), np.uint16), np.uint16)
        vp = np.ascontiguousarray(vprev if pos else np.zeros((1, kvd), np.uint16), np.uint16)
        rc = self.L.yr_gated(n_heads, n_kv, hd, pos, hp(kp), hp(vp), fp(np.float32(wq)), fp(np.float32(wg)),
                             fp(np.float32(wk)), fp(np.float32(wv)), xval, fp(q), fp(g), hp(kr), hp(vr), fp(att))
        assert rc == 0, f"yr_gated rc={rc}"
        return q, g, kr, vr, att

    def gdn(self, n_k, n_v, hd, wqkv, walpha, wbeta, dt, a, S, xval=1.0):
        S = np.array(S, dtype=np.float32)
        q = np.empty(n_k * hd, np.float32)
        k = np.empty(n_k * hd, np.float32)
        v = np.empty(n_v * hd, np.float32)
        ar = np.empty(n_v, np.float32)
        br = np.empty(n_v, np.float32)
        beta = np.empty(n_v, np.float32)
        gate = np.empty(n_v, np.float32)
        rc = self.L.yr_gdn(n_k, n_v, hd, fp(np.float32(wqkv)), fp(np.float32(walpha)), fp(np.float32(wbeta)),
                           fp(np.float32(dt)), fp(np.float32(a)), xval, fp(S), fp(q), fp(k), fp(v), fp(ar),
                           fp(br), fp(beta), fp(gate))
        assert rc == 0, f"yr_gdn rc={rc}"
        return dict(S=S, q=q, k=k, v=v, alpha_raw=ar, beta_raw=br, beta=beta, gate=gate)


def engine_to_headmajor(kc: np.ndarray, vc: np.ndarray, n_kv: int, hd: int, stride: int):
    """Engine rows [n, n_kv*hd] (u16) -> the HIP cache geometry, zero padded:
    K [n_kv, stride, hd] and V [n_kv, stride/32, hd, 32] (32-position tiles, d-major)."""
    n = kc.shape[0]
    K = np.zeros((n_kv, stride, hd), np.uint16)
    Vt = np.zeros((n_kv, hd, stride), np.uint16)
    K[:, :n, :] = kc.reshape(n, n_kv, hd).transpose(1, 0, 2)
    Vt[:, :, :n] = vc.reshape(n, n_kv, hd).transpose(1, 2, 0)
    V = Vt.reshape(n_kv, hd, stride // 32, 32).transpose(0, 2, 1, 3).copy()
    return K, V


def untile_v(V: np.ndarray) -> np.ndarray:
    """V [n_kv, stride/32, hd, 32] -> [n_kv, hd, stride] (column = position)."""
    n_kv, nt, hd, t = V.shape
    return V.transpose(0, 2, 1, 3).reshape(n_kv, hd, nt * t)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
