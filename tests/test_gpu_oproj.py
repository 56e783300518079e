"""o_proj on the GPU vs the oracle (engine.c:969-973, matvec.c:98-122).

x[b] += W_o . att[b].  Up to 8 tokens the GEMV kernel keeps every product
and sum in f32 (the reference's arithmetic in another order); more tokens go
through the MFMA GEMM with f16 weights times the f16 hi + lo parts of f32 att
(about 22 bits of each activation), f16 weights times f16 att (the attention
kernel's f16 output) or, for f32 weights, the hi + lo parts of both.  Either way the
result must be within relative L2 1e-5 of the f32 oracle (the stated bar is
1e-3), on the updated x and on the product alone.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def gen(seed, shape, sigma=1.0):
    from yllm_amd.attention import synth_normal

    return synth_normal(seed, int(np.prod(shape)), sigma).reshape(shape)


def weights(oracle, seed, hidden, qdim, f16):
    w = gen(seed, (hidden, qdim), 1.0 / np.sqrt(qdim))
    return oracle.f32_to_f16(w) if f16 else w


def to_dev(cuda, w):
    t = torch.from_numpy(np.ascontiguousarray(w)).to(cuda)
    return t.view(torch.float16) if w.dtype == np.uint16 else t


@pytest.mark.parametrize("B,hidden,qdim,f16", [
    (1, 896, 896, True),      # decode, the 0.5B shape (14 heads x 64)
    (3, 4096, 4096, True),
    (8, 2048, 4096, True),    # the largest GEMV batch
    (1, 1000, 512, False),    # f32 weights, a hidden size that is no multiple of the rows per wave
    (9, 896, 896, True),      # the smallest GEMM batch
    (64, 4096, 4096, True),
    (300, 2048, 4096, True),
    (77, 1024, 2048, False),  # f32 GEMM
    (200, 4096, 4096, True),  # 256 x 256 tiles, a partial token tile
    (200, 1000, 904, False),  # f32 weights; hidden and qdim no multiples of the tiles or of 64
    (130, 520, 1032, True),   # the smallest 256-token tile config, ragged edges
    (64, 333, 904, True),     # the engine's 64-token chunk, ragged edges
])
def test_o_proj_matches_oracle(cuda, oracle, B, hidden, qdim, f16):
    from yllm_amd.attention import o_proj

    x0 = gen(2001 + B, (B, hidden))
    att = gen(2002 + B, (B, qdim), 0.5)
    w = weights(oracle, 2003 + B, hidden, qdim, f16)
    want = oracle.o_proj(x0, att, w)
    xt = torch.from_numpy(x0).to(cuda)
    o_proj(xt, torch.from_numpy(att).to(cuda), to_dev(cuda, w))
    got = xt.cpu().numpy()
    err = rel_l2(got, want)
    err_p = rel_l2(got.astype(np.float64) - x0, want.astype(np.float64) - x0)
    print(f"o_proj B={B} {hidden}x{qdim} {'f16' if f16 else 'f32'}: rel_l2 {err:.2e}, product only {err_p:.2e}")
    assert err <= TOL and err_p <= TOL
    assert max(rel_l2(got[b], want[b]) for b in range(B)) <= 3 * TOL


@pytest.mark.parametrize("B", [1, 6, 200])
def test_o_proj_f16_attention_output(cuda, oracle, B):
    """att written as f16 by the attention kernel: the GEMV widens it, the
    GEMM path runs one f16 GEMM; the oracle sees the same f16 values."""
    from yllm_amd.attention import o_proj

    hidden, qdim = 2048, 4096
    x0 = gen(2401 + B, (B, hidden))
    att16 = oracle.f32_to_f16(gen(2402 + B, (B, qdim), 0.5))
    w = weights(oracle, 2403 + B, hidden, qdim, True)
    want = oracle.o_proj(x0, att16.view(np.float16).astype(np.float32), w)
    xt = torch.from_numpy(x0).to(cuda)
    o_proj(xt, to_dev(cuda, att16), to_dev(cuda, w))
    err = rel_l2(xt.cpu().numpy(), want)
    print(f"o_proj f16 att B={B}: rel_l2 {err:.2e}")
    assert err <= TOL


def test_o_proj_strided_rows_and_repeat(cuda, oracle):
    """att and x as slices of wider rows; a second call adds again (x is the
    residual stream, updated in place); a smaller batch after a larger one."""
    from yllm_amd.attention import o_proj, o_proj_workspace_bytes

    hidden, qdim = 1024, 2048
    w = weights(oracle, 2101, hidden, qdim, True)
    wt = to_dev(cuda, w)
    ws = torch.empty(o_proj_workspace_bytes(40, hidden, qdim, torch.float16), dtype=torch.uint8, device=cuda)
    for B in (40, 12, 5):
        x0 = gen(2102 + B, (B, hidden + 64))
        att = gen(2103 + B, (B, qdim + 32), 0.5)
        xt = torch.from_numpy(x0).to(cuda)
        at = torch.from_numpy(att).to(cuda)
        o_proj(xt[:, 16:16 + hidden], at[:, 8:8 + qdim], wt, workspace=ws)
        o_proj(xt[:, 16:16 + hidden], at[:, 8:8 + qdim], wt, workspace=ws)
        got = xt.cpu().numpy()
        once = oracle.o_proj(x0[:, 16:16 + hidden], att[:, 8:8 + qdim], w)
        want = oracle.o_proj(once, att[:, 8:8 + qdim], w)
        assert rel_l2(got[:, 16:16 + hidden], want) <= TOL
        # the columns around the slice are untouched
        assert np.array_equal(got[:, :16], x0[:, :16]) and np.array_equal(got[:, 16 + hidden:], x0[:, 16 + hidden:])


def test_o_proj_full_size_sampled_rows(cuda, oracle):
    """8192 tokens of a 4096 x 4096 f16 o_proj in one call (the GEMM path);
    rows sampled across the batch are checked against the oracle."""
    from yllm_amd.attention import o_proj

    B, hidden, qdim = 8192, 4096, 4096
    w = weights(oracle, 2201, hidden, qdim, True)
    x0 = gen(2202, (B, hidden))
    att = gen(2203, (B, qdim), 0.5)
    xt = torch.from_numpy(x0).to(cuda)
    o_proj(xt, torch.from_numpy(att).to(cuda), to_dev(cuda, w))
    got = xt.cpu().numpy()
    rows = np.array([0, 1, 1000, 4095, 4096, 8191])
    want = oracle.o_proj(x0[rows], att[rows], w)
    assert rel_l2(got[rows], want) <= TOL


def test_o_proj_after_gated_decode(cuda, oracle):
    """The qwen35 step after attention (engine.c:958-973): split-K decode with
    the sigmoid gate in its epilogue, then o_proj into the residual stream."""
    from yllm_amd.attention import LayerKV, attn_decode, kv_store, o_proj

    nh, nkv, d, L, hidden = 16, 2, 256, 300, 1024
    kvd, qd = nkv * d, nh * d
    K = oracle.f32_to_f16(gen(2301, (L, kvd), 0.5)).view(np.float16).astype(np.float32)
    V = oracle.f32_to_f16(gen(2302, (L, kvd), 0.5)).view(np.float16).astype(np.float32)
    q = gen(2303, (qd,), 0.5)
    gate = gen(2304, (qd,))
    w = weights(oracle, 2305, hidden, qd, True)
    x0 = gen(2306, (1, hidden))
    cache = LayerKV.empty(nkv, d, L, device=cuda)
    kv_store(cache, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda), 0)
    att = attn_decode(torch.from_numpy(q).to(cuda), cache, L - 1, nh, gate=torch.from_numpy(gate).to(cuda))
    xt = torch.from_numpy(x0).to(cuda)
    o_proj(xt, att.view(1, -1), to_dev(cuda, w))
    kc, vc = oracle.f32_to_f16(K), oracle.f32_to_f16(V)
    att_want = oracle.gate_sigmoid(oracle.decode(q, kc, vc, L - 1, nh, nkv, d), gate)
    want = oracle.o_proj(x0, att_want[None, :], w)
    err = rel_l2(xt.cpu().numpy(), want)
    print(f"gated decode + o_proj: rel_l2 {err:.2e}")
    assert err <= 1e-3
