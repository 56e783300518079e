"""Gated DeltaNet on the GPU vs the oracle (engine.c:786-831, matvec.c:942-1004).

Inputs follow the fifth configuration's recipe: q, k, v ~ 0.5*N(0,1) from the
seeded generator; gates from alpha, beta ~ 0.5*N with dt_bias = 0 and
ssm_a = -1; q/k are L2-normalised inside the kernel (eps 1e-6).  Outputs and
the final state must be within relative L2 1e-3 of the fp32 oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 1e-3
EPS = 1e-6


def gen(seed, n, sigma=0.5):
    from yllm_amd.attention import synth_normal

    return synth_normal(seed, n, sigma)


def rel_l2(a, b):
    return float(np.linalg.norm((np.asarray(a) - np.asarray(b)).ravel()) / max(np.linalg.norm(np.ravel(b)), 1e-30))


def inputs(seed, T, n_k, n_v, d, s0_scale=0.0):
    q = gen(seed, T * n_k * d).reshape(T, n_k * d)
    k = gen(seed + 1, T * n_k * d).reshape(T, n_k * d)
    v = gen(seed + 2, T * n_v * d).reshape(T, n_v * d)
    alpha = gen(seed + 3, T * n_v).reshape(T, n_v)
    beta_raw = gen(seed + 4, T * n_v).reshape(T, n_v)
    S0 = (gen(seed + 5, n_v * d * d, s0_scale) if s0_scale else np.zeros(n_v * d * d, np.float32)).reshape(n_v, d, d)
    return q, k, v, alpha, beta_raw, S0


def oracle_gates(oracle, alpha, beta_raw, dt, a):
    beta = np.empty_like(beta_raw)
    gate = np.empty_like(alpha)
    for t in range(alpha.shape[0]):
        beta[t], gate[t] = oracle.gdn_gates(alpha[t], beta_raw[t], dt, a)
    return beta, gate


def to_dev(cuda, *xs):
    return [torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(cuda) for x in xs]


def test_gdn_gates_match_oracle(cuda, oracle):
    from yllm_amd.gdn import gdn_gates

    T, n_v = 37, 16
    alpha = gen(11, T * n_v, 2.0).reshape(T, n_v)
    beta_raw = gen(12, T * n_v, 2.0).reshape(T, n_v)
    dt = gen(13, n_v, 1.0)
    a = -np.abs(gen(14, n_v, 1.0)) - 0.1
    want_b, want_g = oracle_gates(oracle, alpha, beta_raw, dt, a)
    al, be, dtd, ad = to_dev(cuda, alpha, beta_raw, dt, a)
    gate = gdn_gates(al, be, dtd, ad)
    assert np.allclose(be.cpu().numpy(), want_b, rtol=2e-6, atol=1e-7)
    assert np.allclose(gate.cpu().numpy(), want_g, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("n_k,n_v,d", [(16, 16, 128), (2, 4, 64), (4, 2, 128), (3, 3, 64)])
def test_gdn_step_matches_oracle(cuda, oracle, n_k, n_v, d):
    from yllm_amd.gdn import gdn_step

    q, k, v, alpha, beta_raw, S0 = inputs(100 + d + n_k, 1, n_k, n_v, d, s0_scale=0.05)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, _, _ = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, 1, n_k, d, n_v, d, EPS)
    S, qd, kd, vd, gd, bd = to_dev(cuda, S0, q[0], k[0], v[0], gate[0], beta[0])
    out = gdn_step(S, qd, kd, vd, gd, bd, n_k, EPS).cpu().numpy()
    e_o, e_s = rel_l2(out, o_want[0]), rel_l2(S.cpu().numpy().ravel(), S_want)
    print(f"gdn step {n_k}/{n_v} d={d}: out {e_o:.3e} state {e_s:.3e}")
    assert e_o <= TOL and e_s <= TOL


@pytest.mark.parametrize("chunked", [False, True], ids=["tokenwise", "chunked"])
@pytest.mark.parametrize("T,n_k,n_v,d", [(1, 16, 16, 128), (31, 16, 16, 128), (33, 4, 8, 128), (64, 16, 16, 128),
                                         (65, 2, 4, 64), (100, 2, 4, 64), (130, 4, 2, 128), (300, 16, 16, 128)])
def test_gdn_chunk_matches_oracle(cuda, oracle, T, n_k, n_v, d, chunked):
    from yllm_amd.gdn import gdn_chunk

    q, k, v, alpha, beta_raw, S0 = inputs(200 + T, T, n_k, n_v, d, s0_scale=0.02)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, _, _ = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, T, n_k, d, n_v, d, EPS)
    S, qd, kd, vd, gd, bd = to_dev(cuda, S0, q, k, v, gate, beta)
    out = gdn_chunk(S, qd, kd, vd, gd, bd, n_k, EPS, chunked=chunked).cpu().numpy()
    e_o, e_s = rel_l2(out, o_want), rel_l2(S.cpu().numpy().ravel(), S_want)
    rows = max(rel_l2(out[t], o_want[t]) for t in range(T))
    print(f"gdn chunk T={T} {n_k}/{n_v} d={d} chunked={chunked}: out {e_o:.3e} (worst row {rows:.3e}) "
          f"state {e_s:.3e}")
    assert e_o <= TOL and e_s <= TOL and rows <= 3 * TOL


@pytest.mark.parametrize("chunked", [False, True], ids=["tokenwise", "chunked"])
def test_gdn_chunk_interleaved_layout_and_prenormalised(cuda, oracle, chunked):
    """q, k, v as slices of one [T, conv_channels] row (the engine's qkv
    buffer, engine.c:820-823) and q/k normalised by the caller (eps <= 0)."""
    from yllm_amd.gdn import gdn_chunk

    T, n_k, n_v, d = 145, 2, 4, 128
    q, k, v, alpha, beta_raw, S0 = inputs(301, T, n_k, n_v, d)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, qn, kn = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, T, n_k, d, n_v, d, EPS)
    qkv = np.concatenate([qn, kn, v], axis=1)
    (qkv_d, S, gd, bd) = to_dev(cuda, qkv, S0, gate, beta)
    kd0 = n_k * d
    out = gdn_chunk(S, qkv_d[:, :kd0], qkv_d[:, kd0:2 * kd0], qkv_d[:, 2 * kd0:], gd, bd, n_k, eps=0.0,
                    chunked=chunked)
    assert rel_l2(out.cpu().numpy(), o_want) <= TOL
    assert rel_l2(S.cpu().numpy().ravel(), S_want) <= TOL


@pytest.mark.parametrize("chunked,cut", [(False, 37), (True, 64)], ids=["tokenwise", "chunked"])
def test_gdn_chunk_split_is_exact(cuda, chunked, cut):
    """Running T tokens in one call or as two calls (state carried in S) gives
    identical bits: token by token the arithmetic does not depend on how
    tokens are staged, and in the chunked form a cut on a chunk boundary
    leaves every chunk's computation unchanged."""
    from yllm_amd.gdn import gdn_chunk

    T, n_k, n_v, d = 200, 16, 16, 128
    q, k, v, alpha, beta_raw, S0 = inputs(400, T, n_k, n_v, d, s0_scale=0.02)
    gate = -np.log1p(np.exp(alpha)).astype(np.float32)
    beta = (1 / (1 + np.exp(-beta_raw))).astype(np.float32)
    Sa, qd, kd, vd, gd, bd = to_dev(cuda, S0, q, k, v, gate, beta)
    Sb = Sa.clone()
    full = gdn_chunk(Sa, qd, kd, vd, gd, bd, n_k, chunked=chunked)
    first = gdn_chunk(Sb, qd[:cut], kd[:cut], vd[:cut], gd[:cut].contiguous(), bd[:cut].contiguous(), n_k,
                      chunked=chunked)
    second = gdn_chunk(Sb, qd[cut:], kd[cut:], vd[cut:], gd[cut:].contiguous(), bd[cut:].contiguous(), n_k,
                       chunked=chunked)
    assert torch.equal(full, torch.cat([first, second]))
    assert torch.equal(Sa, Sb)


@pytest.mark.parametrize("chunked", [False, True], ids=["tokenwise", "chunked"])
def test_gdn_full_size_prefill(cuda, oracle, chunked):
    """The fifth configuration's GDN layer: 4096 tokens, 16 heads, d = 128."""
    from yllm_amd.gdn import gdn_chunk, gdn_gates

    T, n_k, n_v, d = 4096, 16, 16, 128
    q, k, v, alpha, beta_raw, S0 = inputs(0x5EED0005, T, n_k, n_v, d)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, _, _ = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, T, n_k, d, n_v, d, EPS)
    S, qd, kd, vd, al, be = to_dev(cuda, S0, q, k, v, alpha, beta_raw)
    gd = gdn_gates(al, be, *to_dev(cuda, np.zeros(n_v), -np.ones(n_v)))
    out = gdn_chunk(S, qd, kd, vd, gd, be, n_k, chunked=chunked).cpu().numpy()
    e_o, e_s = rel_l2(out, o_want), rel_l2(S.cpu().numpy().ravel(), S_want)
    print(f"gdn full T={T} chunked={chunked}: out {e_o:.3e} state {e_s:.3e}")
    assert e_o <= TOL and e_s <= TOL


# ---------------------------------------------------------------- neighbours

def conv_inputs(seed, T, dim, kw, stride=None):
    stride = stride or dim
    x = gen(seed, T * stride, 1.0).reshape(T, stride)
    st = gen(seed + 1, kw * dim, 1.0).reshape(kw, dim)
    w = gen(seed + 2, dim * kw, 0.5).reshape(dim, kw)
    return x, st, w


@pytest.mark.parametrize("T,dim,kw", [(1, 96, 4), (2, 96, 4), (7, 40, 3), (8, 256, 4), (37, 300, 4), (129, 1024, 2),
                                      (64, 64, 1), (33, 130, 8)])
def test_gdn_conv_bits_match_oracle(cuda, oracle, T, dim, kw):
    """Without silu the conv outputs and the new delay line are the
    reference's bits (conv1d_update order, no contraction)."""
    from yllm_amd.gdn import gdn_conv

    x, st, w = conv_inputs(500 + T + dim, T, dim, kw)
    st_want, rows_want = oracle.conv(st, x, w, kw)
    xd, sd, wd = to_dev(cuda, x, st, w)
    out = gdn_conv(xd, sd, wd, silu=False).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), rows_want.view(np.uint32))
    assert np.array_equal(sd.cpu().numpy().view(np.uint32), st_want.view(np.uint32))


def test_gdn_conv_silu_strided_and_split(cuda, oracle):
    """conv + silu on qkv rows with extra columns (row stride > dim), against
    the oracle to 2e-6; and 200 tokens in one call or as 3 + 197 (the delay
    line carries the state) give the same bits."""
    from yllm_amd.gdn import gdn_conv

    T, dim, kw, stride = 200, 192, 4, 256
    x, st, w = conv_inputs(601, T, dim, kw, stride)
    st_want, rows_want = oracle.conv_silu(st, x[:, :dim], w, kw)
    xd, sd, wd = to_dev(cuda, x, st, w)
    sd2 = sd.clone()
    out = gdn_conv(xd, sd, wd)
    assert rel_l2(out.cpu().numpy(), rows_want) <= 2e-7
    assert np.allclose(out.cpu().numpy(), rows_want, rtol=2e-6, atol=1e-7)
    assert np.array_equal(sd.cpu().numpy(), st_want)
    parts = torch.cat([gdn_conv(xd[:3], sd2, wd), gdn_conv(xd[3:], sd2, wd)])
    assert torch.equal(parts, out) and torch.equal(sd2, sd)


def test_gdn_conv_full_size(cuda, oracle):
    """The fifth configuration's layer: 4096 tokens, 2*16*128 + 16*128 = 6144
    channels, kernel width 4."""
    from yllm_amd.gdn import gdn_conv

    T, dim, kw = 4096, 6144, 4
    x, st, w = conv_inputs(0x5EED0105, T, dim, kw)
    st_want, rows_want = oracle.conv(st, x, w, kw)
    xd, sd, wd = to_dev(cuda, x, st, w)
    out = gdn_conv(xd, sd, wd, silu=False).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), rows_want.view(np.uint32))
    assert np.array_equal(sd.cpu().numpy().view(np.uint32), st_want.view(np.uint32))


@pytest.mark.parametrize("w_f16", [False, True], ids=["w_f32", "w_f16"])
@pytest.mark.parametrize("T,n_heads,hd", [(1, 16, 128), (37, 4, 64), (5, 3, 256), (130, 16, 128)])
def test_gdn_gated_norm_matches_oracle(cuda, oracle, T, n_heads, hd, w_f16):
    from yllm_amd.gdn import gdn_gated_norm

    x = gen(700 + T, T * n_heads * hd, 0.7).reshape(T, n_heads * hd)
    z = gen(701 + T, T * n_heads * hd, 2.0).reshape(T, n_heads * hd)
    w = (gen(702, hd, 0.2) + np.float32(1.0)).astype(np.float32)
    wo = oracle.f32_to_f16(w) if w_f16 else w
    want = oracle.rmsnorm_gated(x.reshape(-1, hd), wo, z.reshape(-1, hd), np.float32(EPS)).reshape(T, -1)
    xd, zd = to_dev(cuda, x, z)
    wd = torch.from_numpy(wo.view(np.float16) if w_f16 else w).to(cuda)
    got = gdn_gated_norm(xd, zd, wd, n_heads).cpu().numpy()
    assert np.allclose(got, want, rtol=3e-6, atol=1e-7), float(np.abs(got - want).max())
    # in place, as the engine applies it
    gdn_gated_norm(xd, zd, wd, n_heads, out=xd)
    assert np.allclose(xd.cpu().numpy(), want, rtol=3e-6, atol=1e-7)
