"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is compared bit for bit with (a) golden vectors that the
reference's own compiled code produced (tests/golden/make_golden.py), (b) the
reference built from its sources, live, when oracle/_ref is present, and
(c) closed forms / textbook routines that a plausible slip (wrong GQA index,
missing scale, transposed state, wrong rounding direction) would fail.
"""
from __future__ import annotations

import numpy as np
import pytest

from inputs import splitmix, uniform_pm1
from oracle_lib import rel_l2


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def prev_rows(oracle, seed, n, kvd):
    return oracle.f32_to_f16(uniform_pm1(seed, max(n, 1) * kvd).reshape(max(n, 1), kvd))[:n]


# ---------------------------------------------------------------- conversions

def test_f32_to_f16_golden(oracle, golden):
    got = oracle.f32_to_f16(golden["conv_f32"])
    assert np.array_equal(got, golden["conv_f32_to_f16"])


def test_f32_to_f16_rounds_ties_away_from_zero(oracle):
    # 1 + 2^-11 is exactly half way between 1 and 1+2^-10: RNE gives 0x3c00, the reference 0x3c01
    assert oracle.f32_to_f16(np.float32([1.0 + 2.0 ** -11]))[0] == 0x3C01
    assert oracle.f32_to_f16(np.float32([-(1.0 + 2.0 ** -11)]))[0] == 0xBC01
    # f32 subnormals flush to signed zero, overflow to inf
    assert list(oracle.f32_to_f16(np.float32([1e-40, -1e-40, 1e6, -1e6]))) == [0x0000, 0x8000, 0x7C00, 0xFC00]


def test_f32_to_f16_matches_numpy_off_ties(oracle):
    # away from exact ties the reference rounding equals IEEE round-to-nearest
    x = uniform_pm1(5, 20000, 4.0)
    np_bits = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16(x)
    mant = x.view(np.uint32) & 0x1FFF
    not_tie = mant != 0x1000
    assert np.array_equal(got[not_tie], np_bits[not_tie])


def test_f16_to_f32_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.isnan(got[nan]).all()


def test_f16_reference_known_answers(oracle):
    # tests/test_matvec.c:34-54 of the reference
    cases = {0x0000: 0.0, 0x3C00: 1.0, 0xBC00: -1.0, 0x0001: 5.960464477539063e-8,
             0x8001: -5.960464477539063e-8, 0x03F7: 6.049871444702148e-5, 0x83F7: -6.049871444702148e-5,
             0x0400: 6.103515625e-5}
    for h, v in cases.items():
        assert abs(float(oracle.L.yo_f16_to_f32(h)) - v) <= 1e-12
    assert np.isinf(oracle.L.yo_f16_to_f32(0x7C00)) and oracle.L.yo_f16_to_f32(0xFC00) < 0
    for h in (0x0000, 0x3C00, 0xBC00, 0x0400, 0x7BFF, 0x03FF, 0x8003, 0x3555, 0xC555, 0x03F7):
        assert oracle.L.yo_f32_to_f16(oracle.L.yo_f16_to_f32(h)) == h


def test_bf16_to_f16_golden(oracle, golden):
    got = np.array([oracle.L.yo_bf16_to_f16(int(v)) for v in golden["conv_bf16"]], np.uint16)
    assert np.array_equal(got, golden["conv_bf16_to_f16"])


def test_yrng_golden(golden):
    # the portable splitmix used for fixture inputs reproduces the reference yrng stream
    assert np.array_equal(splitmix(int(golden["yrng_seed"][0]), 16), golden["yrng_first16"])


# ----------------------------------------------------------- softmax / l2norm

def test_softmax_golden(oracle, golden):
    for i in range(4):
        got = oracle.softmax(golden[f"softmax{i}_in"])
        assert np.array_equal(bits(got), bits(golden[f"softmax{i}_out"]))


def test_softmax_reference_known_answer(oracle):
    # tests/test_matvec.c:230-239 of the reference
    v = oracle.softmax(np.float32([1.0, 2.0, 3.0]))
    s = np.exp(1.0) + np.exp(2.0) + np.exp(3.0)
    assert abs(v[0] - np.exp(1.0) / s) < 1e-6 and abs(v[2] - np.exp(3.0) / s) < 1e-6
    assert abs(v.sum() - 1.0) < 1e-6


def test_l2norm_golden(oracle, golden):
    for i in range(2):
        v = np.array(golden[f"l2norm{i}_in"], np.float32)
        oracle.L.yo_l2norm(v.ctypes.data_as(__import__("oracle_lib").FP), v.size, np.float32(1e-6))
        assert np.array_equal(bits(v), bits(golden[f"l2norm{i}_out"]))


# ------------------------------------------------------------------ attention

def _decode_case(oracle, golden, name):
    arch, nh, nkv, hd, pos = (int(x) for x in golden[f"{name}_meta"])
    seeds = golden[f"{name}_seeds"]
    kvd = nkv * hd
    kc = np.concatenate([prev_rows(oracle, int(seeds[0]), pos, kvd), golden[f"{name}_knew"]])
    vc = np.concatenate([prev_rows(oracle, int(seeds[1]), pos, kvd), golden[f"{name}_vnew"]])
    return (nh, nkv, hd, pos), golden[f"{name}_q"], kc, vc


@pytest.mark.parametrize("name", ["dec_cfg1", "dec_qwen", "dec_pos0"])
def test_decode_golden(oracle, golden, name):
    (nh, nkv, hd, pos), q, kc, vc = _decode_case(oracle, golden, name)
    out = oracle.decode(q, kc, vc, pos, nh, nkv, hd)
    assert np.array_equal(bits(out), bits(golden[f"{name}_att"]))


@pytest.mark.parametrize("name", ["pre_llama", "pre_qwen", "pre_ragged"])
def test_prefill_golden(oracle, golden, name):
    arch, nh, nkv, hd, ps, B = (int(x) for x in golden[f"{name}_meta"])
    seeds = golden[f"{name}_seeds"]
    kvd = nkv * hd
    kc = np.concatenate([prev_rows(oracle, int(seeds[0]), ps, kvd), golden[f"{name}_knew"]])
    vc = np.concatenate([prev_rows(oracle, int(seeds[1]), ps, kvd), golden[f"{name}_vnew"]])
    out = oracle.prefill(golden[f"{name}_q"], kc, vc, ps, B, nh, nkv, hd)
    assert np.array_equal(bits(out), bits(golden[f"{name}_att"]))


@pytest.mark.parametrize("name", ["gat_small", "gat_cfg5"])
def test_gated_golden(oracle, golden, name):
    nh, nkv, hd, pos = (int(x) for x in golden[f"{name}_meta"])
    seeds = golden[f"{name}_seeds"]
    kvd = nkv * hd
    kc = np.concatenate([prev_rows(oracle, int(seeds[0]), pos, kvd), golden[f"{name}_knew"]])
    vc = np.concatenate([prev_rows(oracle, int(seeds[1]), pos, kvd), golden[f"{name}_vnew"]])
    out = oracle.gate_sigmoid(oracle.decode(golden[f"{name}_q"], kc, vc, pos, nh, nkv, hd), golden[f"{name}_gate"])
    assert np.array_equal(bits(out), bits(golden[f"{name}_att"]))


def _attn_f64(q, kc, vc, positions, nh, nkv, hd):
    """fp64 brute force of softmax(q k^T / sqrt(d)) v with the reference GQA map."""
    K = kc.view(np.float16).astype(np.float64)
    V = vc.view(np.float16).astype(np.float64)
    q = np.asarray(q, np.float64).reshape(len(positions), nh, hd)
    out = np.zeros_like(q)
    for t, pos in enumerate(positions):
        for h in range(nh):
            kvh = h * nkv // nh
            k = K[: pos + 1, kvh * hd:(kvh + 1) * hd]
            v = V[: pos + 1, kvh * hd:(kvh + 1) * hd]
            s = k @ q[t, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = p @ v / p.sum()
    return out.reshape(len(positions), nh * hd)


@pytest.mark.parametrize("nh,nkv,hd,pos", [(4, 2, 64, 9), (6, 3, 64, 30), (8, 1, 128, 70), (3, 3, 64, 5)])
def test_decode_fp64_brute_force(oracle, nh, nkv, hd, pos):
    kvd = nkv * hd
    kc = oracle.f32_to_f16(uniform_pm1(41, (pos + 1) * kvd).reshape(pos + 1, kvd))
    vc = oracle.f32_to_f16(uniform_pm1(42, (pos + 1) * kvd).reshape(pos + 1, kvd))
    q = uniform_pm1(43, nh * hd, 1.5)
    out = oracle.decode(q, kc, vc, pos, nh, nkv, hd)
    want = _attn_f64(q, kc, vc, [pos], nh, nkv, hd)[0]
    assert rel_l2(out, want) < 1e-6


def test_attention_closed_forms(oracle):
    nh, nkv, hd = 4, 2, 64
    kvd = nkv * hd
    q = uniform_pm1(51, nh * hd, 2.0)
    v = oracle.f32_to_f16(uniform_pm1(52, 10 * kvd).reshape(10, kvd))
    k = oracle.f32_to_f16(uniform_pm1(53, 10 * kvd).reshape(10, kvd))
    V = v.view(np.float16).astype(np.float32)
    # one key: the output is that V row exactly
    out = oracle.decode(q, k[:1], v[:1], 0, nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):
        kvh = h * nkv // nh
        assert np.array_equal(out[h], V[0, kvh * hd:(kvh + 1) * hd])
    # identical keys: uniform weights, the output is the mean of V
    kk = np.repeat(k[:1], 10, axis=0)
    out = oracle.decode(q, kk, v, 9, nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):
        kvh = h * nkv // nh
        assert np.allclose(out[h], V[:, kvh * hd:(kvh + 1) * hd].mean(0), rtol=0, atol=1e-6)
    # heads of one group with the same query give the same output; other groups differ
    qq = np.tile(q[:hd], nh)
    out = oracle.decode(qq, k, v, 9, nh, nkv, hd).reshape(nh, hd)
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[2], out[3])
    assert not np.array_equal(out[0], out[2])


def test_prefill_causality(oracle):
    nh, nkv, hd, B = 4, 2, 64, 12
    kvd = nkv * hd
    q = uniform_pm1(61, B * nh * hd).reshape(B, nh * hd)
    k = oracle.f32_to_f16(uniform_pm1(62, B * kvd).reshape(B, kvd))
    v = oracle.f32_to_f16(uniform_pm1(63, B * kvd).reshape(B, kvd))
    base = oracle.prefill(q, k, v, 0, B, nh, nkv, hd)
    k2, v2 = k.copy(), v.copy()
    k2[7:] ^= 0x1234
    v2[7:] ^= 0x0F0F
    pert = oracle.prefill(q, k2, v2, 0, B, nh, nkv, hd)
    assert np.array_equal(bits(base[:7]), bits(pert[:7]))
    assert not np.array_equal(base[7:], pert[7:])
    # prefill row t equals decode at position t
    for t in (0, 5, 11):
        d = oracle.decode(q[t], k[: t + 1], v[: t + 1], t, nh, nkv, hd)
        assert np.array_equal(bits(d), bits(base[t]))


# ------------------------------------------------------------------------ GDN

@pytest.mark.parametrize("name", ["gdn_2_4", "gdn_4_2", "gdn_3_3"])
def test_gdn_golden(oracle, golden, name):
    nk, nv, hd = (int(x) for x in golden[f"{name}_meta"])
    seeds = golden[f"{name}_seeds"]
    dt = uniform_pm1(int(seeds[1]), nv, 1.0)
    a = -np.exp(uniform_pm1(int(seeds[2]), nv, 1.0)).astype(np.float32)
    beta, gate = oracle.gdn_gates(golden[f"{name}_alpha_raw"], golden[f"{name}_beta_raw"], dt, a)
    assert np.array_equal(bits(beta), bits(golden[f"{name}_beta"]))
    assert np.array_equal(bits(gate), bits(golden[f"{name}_gate"]))
    S0 = uniform_pm1(int(seeds[0]), nv * hd * hd, 0.2)
    S1, _ = oracle.gdn_step(S0, golden[f"{name}_q"], golden[f"{name}_k"], golden[f"{name}_v"], gate, beta, nk, hd,
                            nv, hd)
    assert np.array_equal(bits(S1), bits(golden[f"{name}_S"]))


def _gdn_f64(S, q, k, v, g, beta, nk, hk, nv, hv):
    """fp64 statement of the recurrence in matrix form: S_h (hk x hv)."""
    S = S.reshape(nv, hv, hk).transpose(0, 2, 1).astype(np.float64)  # [h][i][j] = state col j entry i
    out = np.zeros((nv, hv))
    for h in range(nv):
        kh = h % nk
        qq, kk = q[kh * hk:(kh + 1) * hk].astype(np.float64), k[kh * hk:(kh + 1) * hk].astype(np.float64)
        Sh = S[h] * np.exp(np.float64(g[h]))
        delta = (v[h * hv:(h + 1) * hv] - kk @ Sh) * beta[h]
        Sh = Sh + np.outer(kk, delta)
        S[h] = Sh
        out[h] = (qq @ Sh) / np.sqrt(hv)
    return S.transpose(0, 2, 1).reshape(-1), out.reshape(-1)


def test_gdn_step_fp64_matrix_form(oracle):
    nk, nv, hd = 2, 4, 32
    S = uniform_pm1(71, nv * hd * hd, 0.3)
    q, k = uniform_pm1(72, nk * hd, 0.2), uniform_pm1(73, nk * hd, 0.2)
    v = uniform_pm1(74, nv * hd)
    g = -np.abs(uniform_pm1(75, nv))
    beta = np.abs(uniform_pm1(76, nv))
    S1, out = oracle.gdn_step(S, q, k, v, g, beta, nk, hd, nv, hd)
    S_ref, out_ref = _gdn_f64(S, q, k, v, g, beta, nk, hd, nv, hd)
    assert rel_l2(S1, S_ref) < 1e-6 and rel_l2(out, out_ref) < 1e-5


def test_gdn_closed_forms(oracle):
    hd = 16
    # beta = 0: pure decay S <- exp(g) S, output (S q)/sqrt(d)
    S = uniform_pm1(81, hd * hd, 0.5)
    q, k, v = uniform_pm1(82, hd), uniform_pm1(83, hd), uniform_pm1(84, hd)
    S1, out = oracle.gdn_step(S, q, k, v, np.float32([-0.5]), np.float32([0.0]), 1, hd, 1, hd)
    assert np.allclose(S1, S * np.exp(-0.5), rtol=1e-6, atol=0)
    # g = 1 (log-gate 0), beta = 1, orthonormal keys from a zero state: S k_t returns v_t
    basis = np.eye(hd, dtype=np.float32)
    S = np.zeros(hd * hd, np.float32)
    vs = uniform_pm1(85, 5 * hd).reshape(5, hd)
    for t in range(5):
        S, _ = oracle.gdn_step(S, basis[t], basis[t], vs[t], np.float32([0.0]), np.float32([1.0]), 1, hd, 1, hd)
    for t in range(5):
        _, o = oracle.gdn_step(S, basis[t], basis[t + 5], np.zeros(hd, np.float32), np.float32([0.0]),
                               np.float32([0.0]), 1, hd, 1, hd)
        assert np.allclose(o * np.sqrt(hd), vs[t], atol=1e-6)
    # d = 1: scalar recursion s <- g s + beta (v - g s k) k
    s, g, b, kk, vv = 0.3, np.exp(-0.2), 0.7, 0.9, -0.4
    S1, o = oracle.gdn_step(np.float32([s]), np.float32([1.0]), np.float32([kk]), np.float32([vv]),
                            np.float32([-0.2]), np.float32([b]), 1, 1, 1, 1)
    want = g * s + b * (vv - g * s * kk) * kk
    assert abs(S1[0] - want) < 1e-6 and abs(o[0] - want) < 1e-6


# ----------------------------------------------------- live reference (if built)

@pytest.mark.parametrize("arch,nh,nkv,hd,pos", [(0, 8, 4, 64, 33), (1, 12, 3, 128, 77), (0, 7, 7, 64, 1)])
def test_decode_vs_reference_live(oracle, ref, arch, nh, nkv, hd, pos):
    kvd, hidden = nkv * hd, nh * hd
    kp = prev_rows(oracle, 91, pos, kvd)
    vp = prev_rows(oracle, 92, pos, kvd)
    sc = 1.0 / np.sqrt(hidden)
    q, kr, vr, att = ref.decode(arch, nh, nkv, hd, pos, kp, vp, uniform_pm1(93, hidden, 2 * sc),
                                uniform_pm1(94, kvd, 2 * sc), uniform_pm1(95, kvd, 2 * sc))
    out = oracle.decode(q, kr, vr, pos, nh, nkv, hd)
    assert np.array_equal(bits(out), bits(att))


def test_prefill_vs_reference_live(oracle, ref):
    nh, nkv, hd, ps, B = 8, 2, 64, 19, 21
    kvd, hidden = nkv * hd, nh * hd
    kp, vp = prev_rows(oracle, 101, ps, kvd), prev_rows(oracle, 102, ps, kvd)
    sc = 1.0 / np.sqrt(hidden)
    q, kr, vr, att = ref.prefill(1, nh, nkv, hd, ps, B, kp, vp,
                                 uniform_pm1(103, B * hidden, 2 * sc).reshape(B, hidden),
                                 uniform_pm1(104, B * kvd, 2 * sc).reshape(B, kvd),
                                 uniform_pm1(105, B * kvd, 2 * sc).reshape(B, kvd))
    # the rows the reference stored are the oracle's rounding of the same values
    out = oracle.prefill(q, kr, vr, ps, B, nh, nkv, hd)
    assert np.array_equal(bits(out), bits(att))


def test_gdn_vs_reference_live(oracle, ref):
    nk, nv, hd = 16, 16, 128
    conv = 2 * nk * hd + nv * hd
    S = uniform_pm1(111, nv * hd * hd, 0.2)
    dt, a = uniform_pm1(112, nv), -np.exp(uniform_pm1(113, nv))
    r = ref.gdn(nk, nv, hd, uniform_pm1(114, conv, 0.1), uniform_pm1(115, nv, 0.1), uniform_pm1(116, nv, 0.1),
                dt, a.astype(np.float32), S)
    beta, gate = oracle.gdn_gates(r["alpha_raw"], r["beta_raw"], dt, a.astype(np.float32))
    assert np.array_equal(bits(beta), bits(r["beta"])) and np.array_equal(bits(gate), bits(r["gate"]))
    S1, _ = oracle.gdn_step(S, r["q"], r["k"], r["v"], gate, beta, nk, hd, nv, hd)
    assert np.array_equal(bits(S1), bits(r["S"]))


# ---------------------------------------------------------------- GDN neighbours

def _conv_inputs(golden):
    dim, kw, T = (int(v) for v in golden["conv1d_meta"])
    s = [int(v) for v in golden["conv1d_seeds"]]
    return (uniform_pm1(s[0], kw * dim).reshape(kw, dim), uniform_pm1(s[1], T * dim, 2.0).reshape(T, dim),
            uniform_pm1(s[2], dim * kw, 0.7), kw)


def test_conv1d_golden(oracle, golden):
    """matvec.c:956-968 over 7 tokens: state and outputs bit for bit."""
    st0, x, w, kw = _conv_inputs(golden)
    st, rows = oracle.conv(st0, x, w, kw)
    assert np.array_equal(bits(st), bits(golden["conv1d_state"]))
    assert np.array_equal(bits(rows), bits(golden["conv1d_rows"]))


def test_conv1d_vs_reference_live(oracle, ref):
    st0 = uniform_pm1(61, 3 * 40).reshape(3, 40)
    x = uniform_pm1(62, 9 * 40, 3.0).reshape(9, 40)
    w = uniform_pm1(63, 40 * 3)
    a, b = oracle.conv(st0, x, w, 3), ref.conv(st0, x, w, 3)
    assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[1]), bits(b[1]))


def test_conv1d_closed_forms(oracle):
    """A single tap on the newest input is the identity; a single tap on the
    oldest reads the input kwidth-1 tokens back; silu(x) = x * sigmoid(x)."""
    dim, kw, T = 24, 4, 10
    x = uniform_pm1(71, T * dim, 3.0).reshape(T, dim)
    st0 = np.zeros((kw, dim), np.float32)
    w_new = np.zeros((dim, kw), np.float32)
    w_new[:, kw - 1] = 1.0
    st, rows = oracle.conv(st0, x, w_new, kw)
    assert np.array_equal(rows, x) and np.array_equal(st, x[-kw:])
    w_old = np.zeros((dim, kw), np.float32)
    w_old[:, 0] = 1.0
    _, rows = oracle.conv(st0, x, w_old, kw)
    assert np.array_equal(rows[kw - 1:], x[:T - kw + 1]) and not rows[:kw - 1].any()
    _, rows = oracle.conv_silu(st0, x, w_new, kw)
    x64 = x.astype(np.float64)
    assert np.allclose(rows, x64 / (1 + np.exp(-x64)), rtol=2e-7, atol=1e-7)


def test_rmsnorm_gated_golden(oracle, golden):
    s = [int(v) for v in golden["rmsg_seeds"]]
    n = 128
    x = uniform_pm1(s[0], 3 * n).reshape(3, n)
    z = uniform_pm1(s[1], 3 * n, 3.0).reshape(3, n)
    wf = (uniform_pm1(s[2], n, 0.5) + np.float32(1.0)).astype(np.float32)
    assert np.array_equal(bits(oracle.rmsnorm_gated(x, wf, z, np.float32(1e-6))), bits(golden["rmsg_f32"]))
    wh = oracle.f32_to_f16(wf)
    assert np.array_equal(bits(oracle.rmsnorm_gated(x, wh, z, np.float32(1e-6))), bits(golden["rmsg_f16"]))


def test_rmsnorm_gated_fp64(oracle):
    """Against the fp64 formula: y = x w / sqrt(mean(x^2) + eps) * z sigmoid(z)."""
    n = 128
    x = uniform_pm1(81, 5 * n, 2.0).reshape(5, n)
    z = uniform_pm1(82, 5 * n, 4.0).reshape(5, n)
    w = uniform_pm1(83, n, 0.3) + np.float32(1.0)
    y = oracle.rmsnorm_gated(x, w.astype(np.float32), z, np.float32(1e-6))
    x64, z64 = x.astype(np.float64), z.astype(np.float64)
    want = x64 * w / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * z64 / (1 + np.exp(-z64))
    assert np.allclose(y, want, rtol=3e-6, atol=1e-6)


# ---------------------------------------------------------------- RoPE

ROPE_NAMES = ["rope_pairs", "rope_half", "rope_mrope"]


def _rope_case(golden, name):
    kind, d, n_rot, seed = (int(v) for v in golden[f"{name}_meta"])
    pos = golden[f"{name}_pos"]
    x = uniform_pm1(seed, len(pos) * 3 * d, 2.0).reshape(len(pos), 3 * d)
    return kind, d, n_rot, golden[f"{name}_theta"][0], pos, x


@pytest.mark.parametrize("name", ROPE_NAMES)
def test_rope_golden(oracle, golden, name):
    kind, d, n_rot, theta, pos, x = _rope_case(golden, name)
    got = oracle.rope(x, pos, d, theta, kind, n_rot)
    assert np.array_equal(bits(got), bits(golden[f"{name}_out"]))


@pytest.mark.parametrize("kind,d,n_rot,theta", [(1, 128, 0, 500000.0), (2, 64, 0, 10000.0),
                                                (3, 128, 32, 1e6), (3, 64, 64, 10000.0)])
def test_rope_vs_reference_live(oracle, ref, kind, d, n_rot, theta):
    pos = np.array([3, 99, 1000, 65535, 200000], np.int64)
    x = uniform_pm1(121 + kind, len(pos) * 5 * d, 3.0).reshape(len(pos), 5 * d)
    want = ref.rope(x, pos, d, np.float32(theta), kind, n_rot)
    assert np.array_equal(bits(oracle.rope(x, pos, d, np.float32(theta), kind, n_rot)), bits(want))


def _rope_f64(x, pos, d, theta, kind, n_rot):
    """Textbook rotation in fp64, pairs chosen per kind (matvec.c:890-939)."""
    y = np.array(x, np.float64).reshape(len(pos), -1, d)
    span = n_rot if kind == 3 else d
    j = np.arange(span // 2)
    i0 = 2 * j if kind == 1 else j
    i1 = 2 * j + 1 if kind == 1 else j + span // 2
    freq = np.float64(theta) ** (-2.0 * j / span)
    for b, p in enumerate(pos):
        c, s = np.cos(freq * p), np.sin(freq * p)
        a0, a1 = y[b][:, i0].copy(), y[b][:, i1].copy()
        y[b][:, i0] = a0 * c - a1 * s
        y[b][:, i1] = a0 * s + a1 * c
    return y.reshape(len(pos), -1)


@pytest.mark.parametrize("kind,d,n_rot", [(1, 64, 0), (2, 128, 0), (3, 256, 64)])
def test_rope_fp64_rotation(oracle, kind, d, n_rot):
    # small positions: the float angle's error (pos * ulp(freq)) stays below 1e-5
    pos = np.arange(0, 64, 7)
    x = uniform_pm1(131, len(pos) * 2 * d).reshape(len(pos), 2 * d)
    got = oracle.rope(x, pos, d, np.float32(10000.0), kind, n_rot)
    assert np.abs(got - _rope_f64(x, pos, d, 10000.0, kind, n_rot)).max() < 2e-5


def test_rope_closed_forms(oracle):
    d = 64
    x = uniform_pm1(141, 4 * d).reshape(2, 2 * d)
    # position 0: cos 0 = 1, sin 0 = 0 exactly, every kind is the identity
    for kind, n_rot in ((0, 0), (1, 0), (2, 0), (3, 32)):
        assert np.array_equal(bits(oracle.rope(x, [0, 0], d, np.float32(1e4), kind, n_rot)), bits(x))
    # kind 0 (no rope) leaves every position alone
    assert np.array_equal(bits(oracle.rope(x, [5, 77], d, np.float32(1e4), 0, 0)), bits(x))
    # MROPE over all d dims is the qwen pairing with span d, bit for bit
    y3 = oracle.rope(x, [9, 1234], d, np.float32(1e6), 3, d)
    y2 = oracle.rope(x, [9, 1234], d, np.float32(1e6), 2, 0)
    assert np.array_equal(bits(y3), bits(y2))
    # MROPE leaves dims n_rot.. untouched
    y = oracle.rope(x, [9, 1234], d, np.float32(1e6), 3, 16).reshape(2, 2, d)
    assert np.array_equal(bits(y[:, :, 16:]), bits(x.reshape(2, 2, d)[:, :, 16:]))
    # the llama and qwen pairings are one permutation apart: interleave the
    # halves, rotate pairs (2j, 2j+1), de-interleave == rotate (j, j+d/2)
    perm = np.empty(d, np.int64)
    perm[0::2], perm[1::2] = np.arange(d // 2), np.arange(d // 2, d)
    xi = x.reshape(2, 2, d)[:, :, perm].reshape(2, 2 * d)
    yp = oracle.rope(xi, [3, 4000], d, np.float32(1e4), 1, 0).reshape(2, 2, d)
    yq = oracle.rope(x, [3, 4000], d, np.float32(1e4), 2, 0).reshape(2, 2, d)
    assert np.array_equal(bits(yp), bits(yq[:, :, perm]))
    # each rotation keeps the pair's length
    y = oracle.rope(x, [31, 31], d, np.float32(1e4), 1, 0).reshape(-1, 2)
    xr = x.reshape(-1, 2).astype(np.float64)
    assert np.allclose(np.hypot(y[:, 0], y[:, 1]), np.hypot(xr[:, 0], xr[:, 1]), rtol=1e-6)


@pytest.mark.parametrize("name", ROPE_NAMES)
def test_rope_kv_store_loop_golden(oracle, golden, name):
    # the per-token loop (engine.c:1054-1072) on rows [q | k | v] of one head
    # each: q and k are the golden rotations, the caches their f16 rounding
    kind, d, n_rot, theta, pos, x = _rope_case(golden, name)
    out = golden[f"{name}_out"]
    for b in (0, 3, 5, 7):
        q, kc, vc = oracle.rope_kv_store(x[b:b + 1, :d], x[b:b + 1, d:2 * d], x[b:b + 1, 2 * d:], int(pos[b]), 1, 1,
                                         d, theta, kind, n_rot)
        assert np.array_equal(bits(q[0]), bits(out[b, :d]))
        assert np.array_equal(kc[0], oracle.f32_to_f16(out[b, d:2 * d]))
        assert np.array_equal(vc[0], oracle.f32_to_f16(x[b, 2 * d:]))


def test_rope_kv_store_loop_gqa_rows(oracle):
    # several heads and consecutive rows: each head rotated on its own at its row's position
    nh, nkv, d, ps, B = 6, 2, 64, 30, 5
    q = uniform_pm1(151, B * nh * d).reshape(B, nh * d)
    k = uniform_pm1(152, B * nkv * d).reshape(B, nkv * d)
    v = uniform_pm1(153, B * nkv * d).reshape(B, nkv * d)
    qr, kc, vc = oracle.rope_kv_store(q, k, v, ps, nh, nkv, d, np.float32(1e4), 2)
    pos = np.arange(ps, ps + B)
    assert np.array_equal(bits(qr), bits(oracle.rope(q, pos, d, np.float32(1e4), 2)))
    assert np.array_equal(kc, oracle.f32_to_f16(oracle.rope(k, pos, d, np.float32(1e4), 2)))
    assert np.array_equal(vc, oracle.f32_to_f16(v))


# ---------------------------------------------------------------- o_proj

def _mm_case(golden, name):
    out, inn, f16, seed = (int(v) for v in golden[f"{name}_meta"])
    x = uniform_pm1(seed, 3 * inn, 2.0).reshape(3, inn)
    w = uniform_pm1(seed + 100, out * inn, 0.5).reshape(out, inn)
    return x, w, bool(f16)


@pytest.mark.parametrize("name", ["mm_f16", "mm_f32"])
def test_matmul_golden(oracle, golden, name):
    x, w, f16 = _mm_case(golden, name)
    if f16:
        w = oracle.f32_to_f16(w)
    got = np.stack([oracle.matmul(row, w) for row in x])
    assert np.array_equal(bits(got), bits(golden[f"{name}_y"]))


@pytest.mark.parametrize("out,inn,f16", [(64, 896, True), (33, 4096, False), (128, 128, True)])
def test_matmul_vs_reference_live(oracle, ref, out, inn, f16):
    x = uniform_pm1(161, inn, 3.0)
    w = uniform_pm1(162, out * inn).reshape(out, inn)
    if f16:
        w = oracle.f32_to_f16(w)
    assert np.array_equal(bits(oracle.matmul(x, w)), bits(ref.matmul(x, w)))


def test_matmul_and_o_proj_closed_forms(oracle):
    n = 64
    x = uniform_pm1(171, 2 * n).reshape(2, n)
    # identity weights give x back exactly, f32 or f16 (1.0 is exact in f16)
    eye = np.eye(n, dtype=np.float32)
    for w in (eye, oracle.f32_to_f16(eye)):
        assert np.array_equal(bits(oracle.matmul(x[0], w)), bits(x[0]))
    # a permutation matrix permutes; a row of twos doubles one element exactly
    perm = np.random.default_rng(5).permutation(n)
    assert np.array_equal(bits(oracle.matmul(x[0], eye[perm])), bits(x[0][perm]))
    # fp64 against a textbook product, f16 weights decoded exactly
    w16 = oracle.f32_to_f16(uniform_pm1(172, 48 * n).reshape(48, n))
    wd = w16.view(np.float16).astype(np.float64)
    y = oracle.matmul(x[1], w16)
    assert np.allclose(y, wd @ x[1].astype(np.float64), rtol=1e-5, atol=1e-5)
    # o_proj = residual + matmul per token, rows independent
    res = uniform_pm1(173, 2 * 48).reshape(2, 48)
    got = oracle.o_proj(res, x, w16)
    want = res.astype(np.float64) + x.astype(np.float64) @ wd.T
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    assert np.array_equal(bits(got[1]), bits((res[1] + oracle.matmul(x[1], w16)).astype(np.float32)))
