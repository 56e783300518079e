"""Fused RoPE + KV store on the GPU vs the oracle (engine.c:1054-1072 llama /
qwen, engine.c:910-934 qwen35; matvec.c:890-939).

q, k, v are fp32 slices of one projection row [B, (n_heads + 2 n_kv) * d].
The rotated q must agree with the oracle to a few fp32 ulps (the angles are
bit for bit the reference's, the device cosf / sinf differ by an ulp or two);
the K cache holds the reference f16 rounding of the rotated k (equal bits
except where the rotated value sits within an fp32 ulp or two of an f16
rounding boundary: then one f16 ulp apart, or, among f16 subnormals, within
the fp32 error); the V cache holds the reference
rounding of v bit for bit; rows outside the stored range are untouched.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import rel_l2, untile_v

pytestmark = pytest.mark.gpu
SENTINEL = 0x7777  # cache fill that the store must leave alone outside its rows
TOL_ATT = 1e-3    # attention outputs: max relative L2 error vs the fp32 CPU oracle


def gen(seed, shape, sigma=1.0):
    from yllm_amd.attention import synth_normal

    return synth_normal(seed, int(np.prod(shape)), sigma).reshape(shape)


def fused_rows(seed, B, nh, nkv, d):
    """One projection row per token: [q | k | v], and the three fp32 slices as numpy."""
    qd, kvd = nh * d, nkv * d
    x = gen(seed, (B, qd + 2 * kvd))
    return x, x[:, :qd], x[:, qd:qd + kvd], x[:, qd + kvd:]


def sentinel_cache(cuda, nkv, d, rows):
    from yllm_amd.attention import LayerKV

    cache = LayerKV.empty(nkv, d, rows, device=cuda, zero=False)
    cache.k.view(torch.int16).fill_(SENTINEL)
    cache.v.view(torch.int16).fill_(SENTINEL)
    return cache


def cache_bits(cache):
    torch.cuda.synchronize()
    K = cache.k.view(torch.int16).cpu().numpy().view(np.uint16)
    V = untile_v(cache.v.view(torch.int16).cpu().numpy().view(np.uint16))  # [n_kv, d, stride]
    return K, V


def f16_ulps(a, b):
    """|a - b| in f16 ulps for finite same-sign bit patterns."""
    ia, ib = a.astype(np.int32), b.astype(np.int32)
    same_sign = (ia & 0x8000) == (ib & 0x8000)
    return np.where(same_sign, np.abs(ia - ib), 1 << 16)


def f16_close(got_bits, want_bits, abs_err):
    """Rounded values at most one f16 ulp apart, or (near zero, where f16 ulps
    are finer than the fp32 error) within the fp32 error bound abs_err."""
    g = got_bits.view(np.float16).astype(np.float64)
    w = want_bits.view(np.float16).astype(np.float64)
    return np.abs(g - w) <= np.maximum(np.abs(w) * 2.0 ** -10, abs_err + 2.0 ** -24)


def check_k(K, want_bits, pos, nkv, d, scale):
    """K rows pos.. of the head-major cache vs the oracle's f16 bits [B, nkv*d]."""
    got = K[:, pos[0]:pos[-1] + 1, :].transpose(1, 0, 2).reshape(len(pos), nkv * d)
    equal = float((got == want_bits).mean())
    close = f16_close(got, want_bits, 4e-6 * scale)
    print(f"  K bits equal {equal:.6f}, all within 1 ulp or the fp32 bound: {bool(close.all())}")
    assert close.all() and equal >= 0.999


CASES = [
    # kind, n_heads, n_kv, head_dim, n_rot, theta, pos_start, B
    (1, 14, 2, 64, 0, 10000.0, 500, 12),          # llama pairs, the 0.5B head shape
    (2, 28, 4, 128, 0, 1000000.0, 0, 33),         # qwen halves
    (3, 16, 2, 256, 64, 10000000.0, 130000, 5),   # qwen35 M-RoPE, far positions
    (1, 32, 8, 128, 0, 500000.0, 131000, 64),     # llama3-like at 128k
    (0, 8, 8, 128, 0, 10000.0, 3, 4),             # no rope: plain store
    (3, 4, 1, 64, 64, 10000.0, 7, 1),             # M-RoPE over every dim, one token
]


@pytest.mark.parametrize("kind,nh,nkv,d,n_rot,theta,ps,B", CASES)
def test_rope_kv_store_matches_oracle(cuda, oracle, kind, nh, nkv, d, n_rot, theta, ps, B):
    from yllm_amd.attention import rope_kv_store

    x, q, k, v = fused_rows(1000 + kind * 10 + B, B, nh, nkv, d)
    pos = np.arange(ps, ps + B)
    th = np.float32(theta)
    want_q = oracle.rope(q, pos, d, th, kind, n_rot)
    want_k = oracle.f32_to_f16(oracle.rope(k, pos, d, th, kind, n_rot))
    want_v = oracle.f32_to_f16(np.ascontiguousarray(v))
    rows = ps + B + 70
    cache = sentinel_cache(cuda, nkv, d, rows)
    xt = torch.from_numpy(x).to(cuda)
    qd, kvd = nh * d, nkv * d
    got_q = rope_kv_store(cache, xt[:, :qd], xt[:, qd:qd + kvd], xt[:, qd + kvd:], ps, nh, kind, float(th),
                          n_rot=n_rot)
    got_q = got_q.cpu().numpy()
    err = np.abs(got_q - want_q).max()
    print(f"rope kind={kind} {nh}/{nkv} d={d} pos {ps}..{ps + B - 1}: q max err {err:.2e}")
    assert err <= 4e-6 * max(1.0, float(np.abs(q).max()))
    K, V = cache_bits(cache)
    check_k(K, want_k, pos, nkv, d, max(1.0, float(np.abs(k).max())))
    got_v = V[:, :, ps:ps + B].transpose(2, 0, 1).reshape(B, kvd)
    assert np.array_equal(got_v, want_v)
    # nothing outside rows ps..ps+B-1
    outside = np.ones(K.shape[1], bool)
    outside[ps:ps + B] = False
    assert (K[:, outside, :] == SENTINEL).all() and (V[:, :, outside] == SENTINEL).all()


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16])
def test_rope_q_out_dtypes(cuda, oracle, odt):
    from yllm_amd.attention import round_bf16, rope_kv_store

    nh, nkv, d, B, ps = 12, 2, 128, 9, 77
    x, q, k, v = fused_rows(1201, B, nh, nkv, d)
    want = oracle.rope(q, np.arange(ps, ps + B), d, np.float32(1e6), 2, 0)
    cache = sentinel_cache(cuda, nkv, d, ps + B)
    xt = torch.from_numpy(x).to(cuda)
    qd, kvd = nh * d, nkv * d
    got = rope_kv_store(cache, xt[:, :qd], xt[:, qd:qd + kvd], xt[:, qd + kvd:], ps, nh, 2, 1e6,
                        q_out_dtype=odt)
    assert got.dtype == odt
    got = got.view(torch.int16).cpu().numpy().view(np.uint16)
    if odt == torch.float16:
        ref_bits = want.astype(np.float16).view(np.uint16)
    else:
        ref_bits = (round_bf16(want.ravel().copy()).view(np.uint32) >> 16).astype(np.uint16).reshape(want.shape)
    if odt == torch.float16:
        assert f16_close(got, ref_bits, 4e-6 * max(1.0, float(np.abs(q).max()))).all()
    else:  # bf16 keeps the f32 exponent range: neighbours are one integer step apart
        assert f16_ulps(got, ref_bits).max() <= 1
    assert (got == ref_bits).mean() >= 0.999


def test_rope_in_place_and_k_only(cuda, oracle):
    from yllm_amd.attention import rope_kv_store

    nh, nkv, d, B, ps = 8, 2, 64, 6, 40
    x, q, k, v = fused_rows(1301, B, nh, nkv, d)
    pos = np.arange(ps, ps + B)
    want_q = oracle.rope(q, pos, d, np.float32(1e4), 1, 0)
    cache = sentinel_cache(cuda, nkv, d, 128)
    xt = torch.from_numpy(x).to(cuda)
    qd, kvd = nh * d, nkv * d
    qv = xt[:, :qd]
    out = rope_kv_store(cache, qv, xt[:, qd:qd + kvd], xt[:, qd + kvd:], ps, nh, 1, 1e4, q_out=qv)
    assert out.data_ptr() == qv.data_ptr()
    assert np.abs(xt[:, :qd].cpu().numpy() - want_q).max() <= 4e-6 * max(1.0, float(np.abs(q).max()))
    # k and v stored, the rest of the row unchanged
    assert np.array_equal(xt[:, qd:].cpu().numpy(), x[:, qd:])
    # q = None: only the store
    cache2 = sentinel_cache(cuda, nkv, d, 128)
    assert rope_kv_store(cache2, None, xt[:, qd:qd + kvd], xt[:, qd + kvd:], ps, nh, 1, 1e4) is None
    K1, V1 = cache_bits(cache)
    K2, V2 = cache_bits(cache2)
    assert np.array_equal(K1, K2) and np.array_equal(V1, V2)


def test_rope_then_prefill_matches_oracle(cuda, oracle):
    """Two rope_kv_store calls (a prompt, then a continuation) feed the causal
    prefill; the attention output matches the oracle's rope + store + prefill."""
    from yllm_amd.attention import attn_prefill, rope_kv_store

    nh, nkv, d, theta = 16, 2, 256, np.float32(1e7)
    B0, B1 = 70, 45
    cache = sentinel_cache(cuda, nkv, d, B0 + B1)
    kc, vc, qs = [], [], []
    for ps, B, seed in ((0, B0, 1401), (B0, B1, 1402)):
        x, q, k, v = fused_rows(seed, B, nh, nkv, d)
        pos = np.arange(ps, ps + B)
        qs.append(oracle.rope(q, pos, d, theta, 3, 64))
        kc.append(oracle.f32_to_f16(oracle.rope(k, pos, d, theta, 3, 64)))
        vc.append(oracle.f32_to_f16(np.ascontiguousarray(v)))
        xt = torch.from_numpy(x).to(cuda)
        qd, kvd = nh * d, nkv * d
        q_rot = rope_kv_store(cache, xt[:, :qd], xt[:, qd:qd + kvd], xt[:, qd + kvd:], ps, nh, 3, float(theta),
                              n_rot=64)
    got = attn_prefill(q_rot, cache, B0, nh).float().cpu().numpy()
    # the oracle attends with the K bits the GPU stored (equal up to the rare one-ulp case)
    K, _ = cache_bits(cache)
    k_bits = K[:, :B0 + B1, :].transpose(1, 0, 2).reshape(B0 + B1, nkv * d)
    assert f16_close(k_bits, np.concatenate(kc), 4e-6 * 4).all()
    want = oracle.prefill(qs[1], k_bits, np.concatenate(vc), B0, B1, nh, nkv, d)
    err = rel_l2(got, want)
    print(f"rope + prefill qwen35 heads: rel_l2 {err:.3e}")
    assert err <= 1e-3


def test_rope_kv_store_full_size_sampled_rows(cuda, oracle):
    """8192 tokens of the qwen35 attention shape (16 q / 2 kv heads of 256,
    M-RoPE over 64 dims, theta 1e7) in one call; rows sampled across the
    batch are checked against the oracle (RoPE is per token)."""
    from yllm_amd.attention import rope_kv_store

    nh, nkv, d, B = 16, 2, 256, 8192
    x, q, k, v = fused_rows(1501, B, nh, nkv, d)
    cache = sentinel_cache(cuda, nkv, d, B)
    xt = torch.from_numpy(x).to(cuda)
    qd, kvd = nh * d, nkv * d
    got_q = rope_kv_store(cache, xt[:, :qd], xt[:, qd:qd + kvd], xt[:, qd + kvd:], 0, nh, 3, 1e7, n_rot=64)
    K, V = cache_bits(cache)
    got_q = got_q.cpu().numpy()
    rows = np.array([0, 1, 63, 64, 1000, 4095, 4096, 8191])
    th = np.float32(1e7)
    want_q = oracle.rope(q[rows], rows, d, th, 3, 64)
    assert np.abs(got_q[rows] - want_q).max() <= 4e-6 * max(1.0, float(np.abs(q).max()))
    want_k = oracle.f32_to_f16(oracle.rope(k[rows], rows, d, th, 3, 64))
    got_k = K[:, rows, :].transpose(1, 0, 2).reshape(len(rows), kvd)
    assert f16_close(got_k, want_k, 4e-6 * max(1.0, float(np.abs(k).max()))).all()
    # V everywhere: the store is the plain reference rounding
    assert np.array_equal(V[:, :, :B].transpose(2, 0, 1).reshape(B, kvd), oracle.f32_to_f16(np.ascontiguousarray(v)))
    # dims past n_rot are copied unrotated: their K bits are exactly the rounding of k
    kk = K[:, :B, :].transpose(1, 0, 2).reshape(B, nkv, d)[:, :, 64:]
    assert np.array_equal(kk, oracle.f32_to_f16(np.ascontiguousarray(k.reshape(B, nkv, d)[:, :, 64:])))


# ---------------------------------------------- RoPE + KV store + decode, fused

@pytest.mark.parametrize("kind,nh,nkv,d,pos,n_rot,gated", [
    ("pairs", 32, 8, 128, 4095, 0, False),
    ("pairs", 32, 8, 128, 32767, 0, False),    # many splits; the token in the last
    ("half", 14, 2, 64, 512, 0, False),
    ("mrope", 16, 2, 256, 4351, 64, True),     # the hybrid group's gated layer
    ("mrope", 16, 2, 256, 0, 64, True),        # the token is the only key
    ("none", 28, 4, 128, 127, 0, False),       # the token ends a 128-key split
    ("pairs", 8, 8, 64, 128, 0, False),        # the token starts a split
    ("pairs", 32, 8, 128, 39999, 0, False),    # splits of 1280 keys: K loaded as MFMA operands
    ("half", 16, 8, 256, 39999, 0, True),      # the same at d 256, gated
])
def test_decode_rope_matches_oracle_and_two_launches(cuda, oracle, kind, nh, nkv, d, pos, n_rot, gated):
    """yhip_attn_decode_rope against the oracle (the reference's RoPE, store
    and decode) and against yhip_rope_kv_store + yhip_attn_decode on a copy
    of the same cache.  The fused path takes the host's cosf / sinf of the
    reference's angles, the two-launch path the device's: q and the stored
    key may differ by an fp32 / f16 ulp, and a score an ulp apart can round
    its probability to the neighbouring f16 (2^-11 of that key's weight), so
    the two outputs agree to 1e-4 rel-L2 -- and bit for bit when nothing is
    rotated; the values and the earlier rows are bit for bit the same."""
    from yllm_amd.attention import (ROPE_HALF, ROPE_MROPE, ROPE_NONE, ROPE_PAIRS, LayerKV, attn_decode,
                                    attn_decode_rope, kv_store, rope_kv_store)

    rope = {"pairs": ROPE_PAIRS, "half": ROPE_HALF, "mrope": ROPE_MROPE, "none": ROPE_NONE}[kind]
    theta = 1e7 if kind == "mrope" else 1e4
    qd, kvd = nh * d, nkv * d
    a = LayerKV.empty(nkv, d, pos + 41, device=cuda)
    K0, V0 = gen(401 + d, (pos, kvd)), gen(402 + d, (pos, kvd))
    if pos > 0:
        kv_store(a, torch.from_numpy(K0).to(cuda), torch.from_numpy(V0).to(cuda), 0)
    b = LayerKV(a.k.clone(), a.v.clone())
    row, q, k, v = fused_rows(403 + d, 1, nh, nkv, d)
    gate = gen(404 + d, (qd,)) if gated else None

    # the oracle: the token's RoPE + store, then the decode over rows 0..pos
    q_rot, kc_t, vc_t = oracle.rope_kv_store(q, k, v, pos, nh, nkv, d, np.float32(theta), rope, n_rot)
    kc = np.concatenate([oracle.f32_to_f16(K0), kc_t]) if pos else kc_t
    vc = np.concatenate([oracle.f32_to_f16(V0), vc_t]) if pos else vc_t
    want = oracle.decode(q_rot[0], kc, vc, pos, nh, nkv, d)
    if gated:
        want = oracle.gate_sigmoid(want, gate)

    rt = torch.from_numpy(row[0]).to(cuda)
    qt, kt, vt = rt[:qd], rt[qd:qd + kvd], rt[qd + kvd:]
    gt = torch.from_numpy(gate).to(cuda) if gated else None
    q_before = qt.clone()
    got = attn_decode_rope(qt, kt, vt, b, pos, nh, rope, theta, n_rot=n_rot, gate=gt).cpu().numpy()
    assert torch.equal(qt, q_before)
    q2 = rope_kv_store(a, qt.view(1, -1), kt.view(1, -1), vt.view(1, -1), pos, nh, rope, theta, n_rot=n_rot)
    two = attn_decode(q2.view(-1), a, pos, nh, gate=gt).cpu().numpy()

    err, err2 = rel_l2(got, want), rel_l2(got, two)
    Ka, Va = cache_bits(a)
    Kb, Vb = cache_bits(b)
    kb_row = Kb[:, pos, :].reshape(-1)
    k_ref = kc_t[0].reshape(nkv, d).reshape(-1)
    ulps_ref = f16_ulps(kb_row, k_ref).max()
    ulps_two = f16_ulps(kb_row, Ka[:, pos, :].reshape(-1)).max()
    print(f"decode_rope {kind} {nh}/{nkv} d={d} pos={pos}: rel_l2 vs oracle {err:.2e}, vs two launches "
          f"{err2:.2e}; token K row vs oracle <= {ulps_ref} ulp, vs two launches <= {ulps_two} ulp")
    assert err <= TOL_ATT and err2 <= 1e-4
    if rope == ROPE_NONE:
        assert np.array_equal(got, two)
    # the fused launch rotates with the host's cosf / sinf of the reference's angles: the stored key is the
    # oracle's bit for bit; the two-launch path (device sincosf) may be an ulp apart
    assert ulps_ref == 0 and ulps_two <= 1
    # everything but the token's K row is bit for bit the two-launch path's
    Ka[:, pos, :] = Kb[:, pos, :]
    assert np.array_equal(Ka, Kb) and np.array_equal(Va, Vb)
