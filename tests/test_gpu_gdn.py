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


@pytest.mark.parametrize("T,n_k,n_v,d", [(65, 2, 4, 64), (197, 4, 8, 128), (300, 16, 16, 128), (200, 32, 32, 128)],
                         ids=["d64-2chunks", "d128-4chunks-ragged", "16heads", "32heads-one-part"])
def test_gdn_chunk_out_of_place_matches_oracle(cuda, oracle, T, n_k, n_v, d):
    """The chunked form with the state out of place: two workgroups per 16
    state rows whenever they fit the GPU (32 heads of 128 do not: one per
    slice), each writing half of every chunk's token tiles.  Against the
    oracle, and bit for bit the in-place result."""
    from yllm_amd.gdn import gdn_chunk

    q, k, v, alpha, beta_raw, S0 = inputs(900 + T, T, n_k, n_v, d, s0_scale=0.02)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, _, _ = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, T, n_k, d, n_v, d, EPS)
    S_in, S_ip, qd, kd, vd, gd, bd = to_dev(cuda, S0, S0, q, k, v, gate, beta)
    S_op = torch.full_like(S_in, float("nan"))
    out_op = gdn_chunk(S_in, qd, kd, vd, gd, bd, n_k, EPS, S_out=S_op)
    out_ip = gdn_chunk(S_ip, qd, kd, vd, gd, bd, n_k, EPS)
    torch.cuda.synchronize()
    out = out_op.cpu().numpy()
    e_o, e_s = rel_l2(out, o_want), rel_l2(S_op.cpu().numpy().ravel(), S_want)
    rows = max(rel_l2(out[t], o_want[t]) for t in range(T))
    print(f"gdn chunk out of place T={T} {n_k}/{n_v} d={d}: out {e_o:.3e} (worst row {rows:.3e}) state {e_s:.3e}")
    assert e_o <= TOL and e_s <= TOL and rows <= 3 * TOL
    assert torch.equal(out_op.view(torch.int32), out_ip.view(torch.int32))
    assert torch.equal(S_op.view(torch.int32), S_ip.view(torch.int32))
    assert np.array_equal(S_in.cpu().numpy().view(np.uint32), S0.view(np.uint32))


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


def test_gdn_chunk_long_ragged_split_is_exact(cuda, oracle):
    """2100 tokens (33 chunks, the last one of 52 tokens) in one chunked call
    give the bits of two calls of 1024 and 1076 tokens (a cut on a chunk
    boundary), and match the oracle."""
    from yllm_amd.gdn import gdn_chunk

    T, cut, n_k, n_v, d = 2100, 1024, 4, 8, 64
    q, k, v, alpha, beta_raw, S0 = inputs(0x91ECE, T, n_k, n_v, d, s0_scale=0.02)
    beta, gate = oracle_gates(oracle, alpha, beta_raw, np.zeros(n_v, np.float32), -np.ones(n_v, np.float32))
    S_want, o_want, _, _ = oracle.gdn_sequence(S0.ravel(), q, k, v, gate, beta, T, n_k, d, n_v, d, EPS)
    Sa, qd, kd, vd, gd, bd = to_dev(cuda, S0, q, k, v, gate, beta)
    Sb = Sa.clone()
    full = gdn_chunk(Sa, qd, kd, vd, gd, bd, n_k, EPS)
    first = gdn_chunk(Sb, qd[:cut], kd[:cut], vd[:cut], gd[:cut].contiguous(), bd[:cut].contiguous(), n_k, EPS)
    second = gdn_chunk(Sb, qd[cut:], kd[cut:], vd[cut:], gd[cut:].contiguous(), bd[cut:].contiguous(), n_k, EPS)
    assert torch.equal(full, torch.cat([first, second]))
    assert torch.equal(Sa, Sb)
    assert rel_l2(full.cpu().numpy(), o_want) <= TOL
    assert rel_l2(Sa.cpu().numpy().ravel(), S_want) <= TOL


def test_gdn_chunk_graph_replays(cuda):
    """The chunked form (gates in, workspace allocated inside the capture)
    captured in a graph: every replay, with eager work and synchronisations
    between them, gives the eager bits."""
    from yllm_amd.gdn import gdn_chunk

    T, n_k, n_v, d = 2304, 16, 16, 128
    q, k, v, alpha, beta_raw, S0 = inputs(0x6A4F, T, n_k, n_v, d, s0_scale=0.02)
    gate = -np.log1p(np.exp(alpha)).astype(np.float32)
    beta = (1 / (1 + np.exp(-beta_raw))).astype(np.float32)
    S_init, qd, kd, vd, gd, bd = to_dev(cuda, S0, q, k, v, gate, beta)
    S = S_init.clone()
    want = gdn_chunk(S, qd, kd, vd, gd, bd, n_k, EPS)
    S_want = S.clone()
    S.copy_(S_init)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gdn_chunk(S, qd, kd, vd, gd, bd, n_k, EPS)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = gdn_chunk(S, qd, kd, vd, gd, bd, n_k, EPS)
    for i in range(3):
        S.copy_(S_init)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
        assert torch.equal(S, S_want), f"replay {i}"
        junk = torch.randn(1 << 20, device=S.device)
        torch.cuda.synchronize()
        del junk


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


# ------------------------------------------------------- fused decode token

def _layer_inputs(seed, T, n_k, n_v, d, kw, w_f16, oracle):
    conv_dim = (2 * n_k + n_v) * d
    qkv = gen(seed, T * conv_dim, 1.0).reshape(T, conv_dim)
    z = gen(seed + 1, T * n_v * d, 1.0).reshape(T, n_v * d)
    alpha = gen(seed + 2, T * n_v, 1.0).reshape(T, n_v)
    beta_raw = gen(seed + 3, T * n_v, 1.0).reshape(T, n_v)
    conv_w = gen(seed + 4, conv_dim * kw, 0.5).reshape(conv_dim, kw)
    dt = gen(seed + 5, n_v, 0.5)
    a = -np.abs(gen(seed + 6, n_v, 1.0)) - 0.1
    norm_w = (gen(seed + 7, d, 0.1) + 1.0).astype(np.float32)
    if w_f16:
        norm_w = oracle.f32_to_f16(norm_w)
    st0 = gen(seed + 8, kw * conv_dim, 1.0).reshape(kw, conv_dim)
    S0 = gen(seed + 9, n_v * d * d, 0.05).reshape(n_v, d, d)
    return qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, st0, S0


def _oracle_layer(oracle, S, st, qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, n_k, n_v, d, kw):
    """engine.c:786-847 token by token from the pinned oracle pieces."""
    ys = []
    for t in range(qkv.shape[0]):
        st, rows = oracle.conv_silu(st, qkv[t][None], conv_w, kw)
        beta, gate = oracle.gdn_gates(alpha[t], beta_raw[t], dt, a)
        r = rows[0]
        S, out, _, _ = oracle.gdn_sequence(S, r[:n_k * d], r[n_k * d:2 * n_k * d], r[2 * n_k * d:], gate, beta, 1,
                                           n_k, d, n_v, d, EPS)
        ys.append(oracle.rmsnorm_gated(out.reshape(n_v, d), norm_w, z[t].reshape(n_v, d), np.float32(EPS)).ravel())
    return S, st, np.stack(ys)


@pytest.mark.parametrize("oop", [False, True], ids=["in_place", "ping_pong"])
@pytest.mark.parametrize("n_k,n_v,d,kw,w_f16", [
    (16, 16, 128, 4, False),  # the fifth configuration's GDN layer
    (2, 4, 64, 4, True),
    (4, 8, 128, 3, False),
    (1, 3, 64, 1, False),
    (4, 12, 128, 6, True),  # conv width past 4 (eight taps loaded), 12 heads: a partial group of 8
    (8, 24, 64, 8, False),
])
def test_gdn_decode_matches_oracle(cuda, oracle, n_k, n_v, d, kw, w_f16, oop):
    """In place (one workgroup per head) and with the state alternating
    between two buffers as the device backend keeps it (several workgroups
    per head, each storing its share of the columns)."""
    from yllm_amd.gdn import gdn_decode

    T = 5
    qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, st0, S0 = _layer_inputs(3100 + d + kw, T, n_k, n_v, d, kw,
                                                                             w_f16, oracle)
    S_want, st_want, y_want = _oracle_layer(oracle, S0, st0, qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, n_k,
                                            n_v, d, kw)
    S, st_a, st_b, qkv_t, z_t, al, br, cw, dtt, at = to_dev(cuda, S0, st0, np.zeros_like(st0), qkv, z, alpha,
                                                             beta_raw, conv_w, dt, a)
    nw = torch.from_numpy(norm_w).to(cuda)
    nw = nw.view(torch.float16) if w_f16 else nw
    ys = []
    S_b = torch.full_like(S, float("nan"))
    for t in range(T):
        ys.append(gdn_decode(S, st_a, st_b, qkv_t[t], z_t[t], al[t], br[t], cw, dtt, at, nw, n_k,
                             S_out=S_b if oop else None).cpu().numpy())
        st_a, st_b = st_b, st_a
        if oop:
            S, S_b = S_b, S
    y = np.stack(ys)
    err_y = max(rel_l2(y[t], y_want[t]) for t in range(T))
    err_s = rel_l2(S.cpu().numpy(), S_want)
    print(f"gdn_decode n_k={n_k} n_v={n_v} d={d} kw={kw}: y max rel_l2 {err_y:.2e}, state {err_s:.2e}")
    assert err_y <= 1e-5 and err_s <= 1e-5
    # the delay line holds the inputs themselves: bit for bit
    assert np.array_equal(st_a.cpu().numpy().view(np.uint32), st_want.view(np.uint32))


def test_gdn_prefill_then_decode_tokens(cuda, oracle):
    """A 70-token prefill through gdn_conv + gdn_gates + gdn_chunk (chunked) +
    gdn_gated_norm, then 4 decode tokens through gdn_decode: the delay line
    and the state hand over between the two paths (the oracle runs all 74
    tokens one by one)."""
    from yllm_amd.gdn import (gdn_chunk, gdn_chunk_workspace_bytes, gdn_conv, gdn_decode, gdn_gated_norm,
                              gdn_gates)

    n_k, n_v, d, kw, T0, T1 = 4, 8, 128, 4, 70, 4
    T = T0 + T1
    qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, st0, S0 = _layer_inputs(3300, T, n_k, n_v, d, kw, False, oracle)
    S_want, _, y_want = _oracle_layer(oracle, S0, st0, qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, n_k, n_v, d,
                                      kw)
    S, st_a, st_b, qkv_t, z_t, al, br, cw, dtt, at, nw = to_dev(cuda, S0, st0, np.zeros_like(st0), qkv, z, alpha,
                                                                 beta_raw, conv_w, dt, a, norm_w)
    kd = n_k * d
    xc = gdn_conv(qkv_t[:T0], st_a, cw)
    beta = br[:T0].clone()
    gate = torch.empty_like(beta)
    gdn_gates(al[:T0], beta, dtt, at, gate=gate)
    ws = torch.empty(gdn_chunk_workspace_bytes(T0, n_v, d) // 4, device=cuda)
    out = gdn_chunk(S, xc[:, :kd], xc[:, kd:2 * kd], xc[:, 2 * kd:], gate, beta, n_k, workspace=ws)
    y_pre = gdn_gated_norm(out, z_t[:T0], nw, n_v).cpu().numpy()
    ys = []
    for t in range(T0, T):
        ys.append(gdn_decode(S, st_a, st_b, qkv_t[t], z_t[t], al[t], br[t], cw, dtt, at, nw, n_k).cpu().numpy())
        st_a, st_b = st_b, st_a
    err_pre = rel_l2(y_pre, y_want[:T0])
    err_dec = max(rel_l2(ys[i], y_want[T0 + i]) for i in range(T1))
    err_s = rel_l2(S.cpu().numpy(), S_want)
    print(f"prefill {T0} + decode {T1}: prefill y {err_pre:.2e}, decode y {err_dec:.2e}, state {err_s:.2e}")
    assert err_pre <= TOL and err_dec <= TOL and err_s <= TOL


@pytest.mark.parametrize("T,chunked", [(1, True), (33, False), (130, True)],
                         ids=["T1", "T33-tokenwise", "T130-chunked"])
def test_gdn_out_of_place_state_matches_in_place(cuda, T, chunked):
    """A state written to S_out (as the device backend alternates two
    buffers) is the in-place result bit for bit, with the same outputs, and
    the state before the call is left untouched; likewise the conv delay line
    with state_out and the fused decode token."""
    from yllm_amd.gdn import gdn_chunk, gdn_conv, gdn_decode

    n_k, n_v, d = 4, 8, 128
    q, k, v, alpha, beta_raw, S0 = inputs(4100 + T, T, n_k, n_v, d, s0_scale=0.05)
    gate, beta = -np.abs(alpha) * 0.1, 1.0 / (1.0 + np.exp(-beta_raw))
    S_ip, S_in, qd, kd, vd, gd, bd = to_dev(cuda, S0, S0, q[:T], k[:T], v[:T], gate[:T], beta[:T])
    S_op = torch.full_like(S_in, float("nan"))
    out_ip = gdn_chunk(S_ip, qd, kd, vd, gd, bd, n_k, chunked=chunked)
    out_op = gdn_chunk(S_in, qd, kd, vd, gd, bd, n_k, chunked=chunked, S_out=S_op)
    torch.cuda.synchronize()
    assert torch.equal(out_ip.view(torch.int32), out_op.view(torch.int32))
    assert torch.equal(S_op.view(torch.int32), S_ip.view(torch.int32))
    assert np.array_equal(S_in.cpu().numpy().view(np.uint32), S0.view(np.uint32))

    Tc, dim, kw = T + 7, 320, 4  # one run (T <= 8) and several
    x, st, w = conv_inputs(4200 + T, Tc, dim, kw)
    xd, st_ip, st_in, wd = to_dev(cuda, x, st, st, w)
    st_op = torch.full_like(st_in, float("nan"))
    for rows in (slice(0, min(Tc, 8)), slice(0, Tc)):
        st_ip.copy_(st_in)
        o_ip = gdn_conv(xd[rows], st_ip, wd)
        o_op = gdn_conv(xd[rows], st_in, wd, state_out=st_op)
        assert torch.equal(o_ip, o_op) and torch.equal(st_op, st_ip)
        assert np.array_equal(st_in.cpu().numpy().view(np.uint32), st.view(np.uint32))

    if T == 1:
        n_v2, dd, kw2 = 16, 128, 4
        conv_dim = (2 * 16 + n_v2) * dd
        qkv, z = gen(4301, conv_dim, 1.0), gen(4302, n_v2 * dd, 1.0)
        al, br = gen(4303, n_v2, 1.0), gen(4304, n_v2, 1.0)
        cw = gen(4305, conv_dim * kw2, 0.5).reshape(conv_dim, kw2)
        dt, a = gen(4306, n_v2, 0.5), -np.abs(gen(4307, n_v2, 1.0)) - 0.1
        nw = (gen(4308, dd, 0.1) + 1.0).astype(np.float32)
        line = gen(4309, kw2 * conv_dim, 1.0).reshape(kw2, conv_dim)
        S2 = gen(4310, n_v2 * dd * dd, 0.05).reshape(n_v2, dd, dd)
        t = to_dev(cuda, S2, S2, line, np.zeros_like(line), np.zeros_like(line), qkv, z, al, br, cw, dt, a, nw)
        Sa, Sb, l0, la, lb, qkv_t, z_t, al_t, br_t, cw_t, dt_t, a_t, nw_t = t
        Sb_out = torch.full_like(Sb, float("nan"))
        ya = gdn_decode(Sa, l0, la, qkv_t, z_t, al_t, br_t, cw_t, dt_t, a_t, nw_t, 16)
        yb = gdn_decode(Sb, l0, lb, qkv_t, z_t, al_t, br_t, cw_t, dt_t, a_t, nw_t, 16, S_out=Sb_out)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb) and torch.equal(Sb_out, Sa) and torch.equal(la, lb)
        assert np.array_equal(Sb.cpu().numpy().view(np.uint32), S2.view(np.uint32))
