"""The workloads of the benchmark's configurations, run at their full size on
the GPU and checked against the CPU oracle.

- Config 3: batched decode, 64 sequences with lengths L_i = 1024 +
  floor(u * 31745) from the seeded generator (seed 0x5EED0003), 32 query /
  8 KV heads, head_dim 128, f16 KV -- one yhip_attn_decode_batch call with
  the production split plan; sequences compared with the oracle's decode
  (engine.c:1074-1096), the shortest and the longest among them.
- Config 5: the qwen35 hybrid group.  Three Gated-DeltaNet layers, each a
  4096-token prefill (conv1d + silu, gates, chunked recurrence, gated
  RMSNorm) followed by 256 decode tokens (the fused decode token), against
  the oracle's token-by-token layer (engine.c:786-847, matvec.c:942-1021);
  and the gated attention layer (16 / 2 heads, head_dim 256, M-RoPE over 64
  dims, bf16 prefill queries, sigmoid gate) as a 4096-token prefill and 256
  decode steps, against the oracle's RoPE + store (engine.c:910-934) and
  attention + gate (engine.c:935-960).

Bars as everywhere: relative L2 <= 1e-3 against the fp32 oracle (a bf16
output adds its own 2^-8 rounding bound)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3
SEED = 0x5EED0000


def normal(seed, n, sigma=0.5, first=0):
    from yllm_amd.attention import synth_normal

    return synth_normal(seed, n, sigma, first)


def config3_lengths(n_seq=64):
    """L_i = 1024 + floor(u_i * 31745), u_i = ((r_i >> 40) + 0.5) * 2^-24 with
    r_i the splitmix64 stream of seed 0x5EED0003 (the generator of
    platform.c:405-417)."""
    from inputs import splitmix

    r = splitmix(SEED + 3, n_seq)
    u = ((r >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0
    return np.minimum((1024 + np.floor(u * 31745)).astype(np.int64), 32768)


def test_config3_batched_decode_full_size(cuda, oracle):
    from yllm_amd.attention import (DecodeBatch, LayerKV, attn_decode_batch, decode_workspace_bytes, kv_store,
                                    round_f16)

    nh, nkv, hd, n_seq, cap = 32, 8, 128, 64, 32768
    kvd = nkv * hd
    lens = config3_lengths(n_seq)
    assert lens.min() >= 1024 and lens.max() <= 32768
    # distinct rows per sequence: sequence i reads a window of a 65536-row base
    # starting at row (7919 * i) mod 32768
    base_rows = 2 * cap
    Kb = round_f16(normal(SEED + 3, base_rows * kvd)).reshape(base_rows, kvd)
    Vb = round_f16(normal(SEED + 3, base_rows * kvd, first=base_rows * kvd)).reshape(base_rows, kvd)
    kt, vt = torch.from_numpy(Kb).to(cuda).half(), torch.from_numpy(Vb).to(cuda).half()
    offs = [(7919 * i) % cap for i in range(n_seq)]
    caches = []
    for i, L in enumerate(lens):
        c = LayerKV.empty(nkv, hd, cap, device=cuda, zero=False)
        kv_store(c, kt[offs[i]:offs[i] + int(L)], vt[offs[i]:offs[i] + int(L)], 0)
        caches.append(c)
    del kt, vt
    q = normal(SEED + 103, n_seq * nh * hd).reshape(n_seq, nh * hd)
    need = decode_workspace_bytes(n_seq, int(lens.max()), int(lens.sum()), nh, nkv, hd)
    assert need > 0  # the production plan splits the sequences
    got = attn_decode_batch(torch.from_numpy(q).to(cuda), DecodeBatch(caches), lens, nh).cpu().numpy()
    assert np.isfinite(got).all()
    order = np.argsort(lens)
    check = sorted(set([int(order[0]), int(order[-1])] + [int(order[j]) for j in (8, 16, 24, 32, 40, 48, 56)]))
    kc_all, vc_all = oracle.f32_to_f16(Kb), oracle.f32_to_f16(Vb)
    for i in check:
        L = int(lens[i])
        want = oracle.decode(q[i], kc_all[offs[i]:offs[i] + L], vc_all[offs[i]:offs[i] + L], L - 1, nh, nkv, hd)
        err = rel_l2(got[i], want)
        print(f"config 3 sequence {i} ({L} keys): rel_l2 {err:.3e}")
        assert err <= TOL


def _gdn_layer_inputs(li, T, n_h, d, kw):
    seed = SEED + 5 + 16 * li
    conv_dim = 3 * n_h * d
    qkv = normal(seed, T * conv_dim).reshape(T, conv_dim)
    z = normal(seed + 1, T * n_h * d).reshape(T, n_h * d)
    alpha = normal(seed + 2, T * n_h).reshape(T, n_h)
    beta_raw = normal(seed + 3, T * n_h).reshape(T, n_h)
    conv_w = normal(seed + 4, conv_dim * kw).reshape(conv_dim, kw)
    norm_w = (normal(seed + 5, d, 0.1) + 1.0).astype(np.float32)
    return qkv, z, alpha, beta_raw, conv_w, norm_w


@pytest.mark.parametrize("li", [0, 1, 2])
def test_config5_gdn_layer_prefill_then_decode(cuda, oracle, li):
    """One of the group's three GDN layers: 4096-token prefill (conv + silu,
    gates, chunked recurrence, gated RMSNorm) then 256 fused decode tokens,
    from a zero state and delay line; dt_bias 0, ssm_a -1.  The prefill's
    state goes out of place, as the device backend keeps it (the chained
    recurrence then runs two workgroups per state slice)."""
    from test_gpu_gdn import EPS, _oracle_layer
    from yllm_amd.gdn import gdn_chunk, gdn_chunk_workspace_bytes, gdn_conv, gdn_decode, gdn_gated_norm, gdn_gates

    n_h, d, kw, T0, T1 = 16, 128, 4, 4096, 256
    T = T0 + T1
    qkv, z, alpha, beta_raw, conv_w, norm_w = _gdn_layer_inputs(li, T, n_h, d, kw)
    dt, a = np.zeros(n_h, np.float32), -np.ones(n_h, np.float32)
    S0 = np.zeros((n_h, d, d), np.float32)
    st0 = np.zeros((kw, 3 * n_h * d), np.float32)
    S_want, _, y_want = _oracle_layer(oracle, S0, st0, qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w, n_h, n_h, d,
                                      kw)
    dev = [torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(cuda)
           for x in (S0, st0, np.zeros_like(st0), qkv, z, alpha, beta_raw, conv_w, dt, a, norm_w)]
    S, st_a, st_b, qkv_t, z_t, al, br, cw, dtt, at, nw = dev
    kd = n_h * d
    xc = gdn_conv(qkv_t[:T0], st_a, cw)
    beta = br[:T0].clone()
    gate = torch.empty_like(beta)
    gdn_gates(al[:T0], beta, dtt, at, gate=gate)
    ws = torch.empty(gdn_chunk_workspace_bytes(T0, n_h, d) // 4, device=cuda)
    S_pre = S
    S = torch.full_like(S_pre, float("nan"))
    out = gdn_chunk(S_pre, xc[:, :kd], xc[:, kd:2 * kd], xc[:, 2 * kd:], gate, beta, n_h, workspace=ws, S_out=S)
    y_pre = gdn_gated_norm(out, z_t[:T0], nw, n_h).cpu().numpy()
    ys = []
    for t in range(T0, T):
        ys.append(gdn_decode(S, st_a, st_b, qkv_t[t], z_t[t], al[t], br[t], cw, dtt, at, nw, n_h).cpu().numpy())
        st_a, st_b = st_b, st_a
    y_dec = np.stack(ys)
    err_pre = rel_l2(y_pre, y_want[:T0])
    rows_pre = max(rel_l2(y_pre[t], y_want[t]) for t in (0, 1, 63, 64, 2047, 4094, 4095))
    err_dec = max(rel_l2(y_dec[i], y_want[T0 + i]) for i in range(T1))
    err_s = rel_l2(S.cpu().numpy(), S_want)
    print(f"config 5 GDN layer {li}: prefill y {err_pre:.2e} (rows {rows_pre:.2e}), decode y max {err_dec:.2e}, "
          f"state {err_s:.2e}")
    assert err_pre <= TOL and rows_pre <= TOL and err_dec <= TOL and err_s <= TOL


def test_config5_gated_attention_prefill_then_decode(cuda, oracle):
    """The group's gated attention layer: M-RoPE (64 dims, theta 1e7) + KV
    store of 4096 prompt rows, causal prefill with bf16 queries and the
    sigmoid gate, bf16 out; then 256 decode steps, each the token's RoPE +
    store fused into a gated decode over keys 0..t (attn_decode_rope, the
    bench's decode step; test_gpu_rope checks its stored key against the
    oracle bit for bit and its output against the two-launch path to 1e-5)."""
    from yllm_amd.attention import (ROPE_MROPE, LayerKV, attn_decode_rope, attn_prefill, decode_workspace,
                                    decode_workspace_bytes, round_bf16, rope_kv_store)

    nh, nkv, hd, T0, T1, theta = 16, 2, 256, 4096, 256, np.float32(1e7)
    T = T0 + T1
    qd, kvd = nh * hd, nkv * hd
    seed = SEED + 5 + 64
    x = normal(seed, T * (qd + 2 * kvd)).reshape(T, qd + 2 * kvd)
    gate = normal(seed + 1, T * qd, 1.0).reshape(T, qd)
    # the oracle: rope + store of every row, then attention over its own cache
    q_rot, kc, vc = oracle.rope_kv_store(x[:, :qd], x[:, qd:qd + kvd], x[:, qd + kvd:], 0, nh, nkv, hd, theta,
                                         ROPE_MROPE, 64)
    xt = torch.from_numpy(x).to(cuda)
    gt = torch.from_numpy(gate).to(cuda)
    cache = LayerKV.empty(nkv, hd, T, device=cuda)
    q_pre = rope_kv_store(cache, xt[:T0, :qd], xt[:T0, qd:qd + kvd], xt[:T0, qd + kvd:], 0, nh, ROPE_MROPE,
                          float(theta), n_rot=64, q_out_dtype=torch.bfloat16)
    out_pre = attn_prefill(q_pre, cache, 0, nh, out_dtype=torch.bfloat16, gate=gt[:T0]).float().cpu().numpy()
    ws = decode_workspace(decode_workspace_bytes(1, T, T, nh, nkv, hd), cuda)
    dec = []
    for t in range(T0, T):
        dec.append(attn_decode_rope(xt[t, :qd], xt[t, qd:qd + kvd], xt[t, qd + kvd:], cache, t, nh, ROPE_MROPE,
                                    float(theta), n_rot=64, gate=gt[t], workspace=ws).cpu().numpy())
    # the stored K rows are the oracle's to an f16 ulp (device sin/cos), V bit for bit
    from yllm_amd.attention import kv_to_engine

    ek, ev = kv_to_engine(cache, T)
    gk = ek.view(torch.int16).cpu().numpy().view(np.uint16)
    gv = ev.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(gv, vc)
    assert np.abs(gk.astype(np.int32) - kc.astype(np.int32)).max() <= 1
    assert (gk == kc).mean() >= 0.999
    # prefill rows: the engine's attention + gate with the bf16-rounded rotated queries
    q_bf = round_bf16(np.ascontiguousarray(q_rot[:T0], np.float32).copy())
    for t in (0, 1, 127, 128, 1000, 2047, 3000, T0 - 2, T0 - 1):
        want = oracle.gate_sigmoid(oracle.decode(q_bf[t], kc[:t + 1], vc[:t + 1], t, nh, nkv, hd).ravel(), gate[t])
        err = rel_l2(out_pre[t], want)
        assert err <= TOL + 2.0 ** -8, f"prefill row {t}: rel_l2 {err:.3e}"
    worst = 0.0
    for i, t in enumerate(range(T0, T)):
        want = oracle.gate_sigmoid(oracle.decode(q_rot[t], kc[:t + 1], vc[:t + 1], t, nh, nkv, hd).ravel(), gate[t])
        err = rel_l2(dec[i], want)
        worst = max(worst, err)
        assert err <= TOL, f"decode step {t}: rel_l2 {err:.3e}"
    print(f"config 5 gated attention: decode max rel_l2 {worst:.3e}")
