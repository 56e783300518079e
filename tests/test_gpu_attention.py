"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on
identical seeded inputs.

Bars: KV cache bits are identical (integer work); attention outputs are
within a relative L2 error of 1e-3 of the oracle (fp32 CPU reference of the
same loops), the north-star tolerance.  Full-size cases are checked through
properties that do not need the whole O(L^2) oracle: sampled prefill rows
against the oracle's decode at the same position (the two are the same
arithmetic, tests/test_oracle.py::test_prefill_causality)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import engine_to_headmajor, rel_l2, untile_v

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max relative L2 error vs the fp32 CPU oracle


def gen(seed, shape, sigma=0.5, f16=True):
    from yllm_amd.attention import round_f16, synth_normal

    n = int(np.prod(shape))
    x = synth_normal(seed, n, sigma)
    if f16:
        round_f16(x)
    return x.reshape(shape)


def make_cache(cuda, oracle, K, V, n_kv, hd, stride_rows=None, src=torch.float32):
    """Store rows through the HIP kv_store; return the cache and the oracle's engine-layout bits."""
    from yllm_amd.attention import LayerKV, kv_store

    L = K.shape[0]
    cache = LayerKV.empty(n_kv, hd, stride_rows or L, device=cuda)
    kt = torch.from_numpy(K).to(cuda).to(src)
    vt = torch.from_numpy(V).to(cuda).to(src)
    kv_store(cache, kt, vt, 0)
    # the engine sees the src-typed values as floats and rounds them itself
    kc, vc = oracle.f32_to_f16(kt.float().cpu().numpy()), oracle.f32_to_f16(vt.float().cpu().numpy())
    return cache, kc, vc


def cache_bits(cache):
    torch.cuda.synchronize()
    return cache.k.view(torch.int16).cpu().numpy().view(np.uint16), cache.v.view(torch.int16).cpu().numpy().view(
        np.uint16)


# ------------------------------------------------------------------- KV store

@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16])
def test_kv_store_bits_match_reference_rounding(cuda, oracle, golden, src):
    from yllm_amd.attention import LayerKV, kv_store

    n_kv, hd = 2, 64
    kvd = n_kv * hd
    vals = np.concatenate([golden["conv_f32"], gen(5, (4096,), 4.0, f16=False)])
    rows = len(vals) // kvd
    K = vals[: rows * kvd].reshape(rows, kvd).astype(np.float32)
    V = -K[::-1].copy()
    kt = torch.from_numpy(K).to(cuda).to(src)
    vt = torch.from_numpy(V).to(cuda).to(src)
    # what the engine would store: the reference rounding of the (already src-typed) values
    Kx, Vx = kt.float().cpu().numpy(), vt.float().cpu().numpy()
    cache = LayerKV.empty(n_kv, hd, rows + 5, device=cuda)
    kv_store(cache, kt[:17], vt[:17], 0)
    kv_store(cache, kt[17:], vt[17:], 17)  # second call continues at pos_start
    Kb, Vb = cache_bits(cache)
    Kw, Vw = engine_to_headmajor(oracle.f32_to_f16(Kx), oracle.f32_to_f16(Vx), n_kv, hd, cache.kv_stride)
    Vb, Vw = untile_v(Vb), untile_v(Vw)  # [n_kv, hd, position]
    nan = np.isnan(Kx).any(axis=1)
    assert np.array_equal(Kb[:, : rows][:, ~nan], Kw[:, : rows][:, ~nan])
    assert np.array_equal(Vb[:, :, : rows][:, :, ~nan[::-1]], Vw[:, :, : rows][:, :, ~nan[::-1]])
    # nothing outside the stored rows was touched
    assert not Kb[:, rows:].any() and not Vb[:, :, rows:].any()


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ps,B", [(37, 100), (64, 64), (5, 250)])
def test_kv_store_block_kernel_matches_element_path(cuda, oracle, src, ps, B):
    """The bulk store over 64-position blocks (16-byte aligned sources) and
    the element-wise path (a source one element off 16-byte alignment) write
    the same bits, those of the reference rounding, and nothing outside
    positions ps..ps+B-1."""
    from yllm_amd.attention import LayerKV, kv_store

    n_kv, hd = 2, 128
    kvd = n_kv * hd
    K, V = gen(71 + B, (B, kvd), 2.0, f16=False), gen(72 + B, (B, kvd), 2.0, f16=False)
    kt, vt = torch.from_numpy(K).to(cuda).to(src), torch.from_numpy(V).to(cuda).to(src)
    # the same rows at a data pointer 2 or 4 bytes past a 16-byte boundary
    kb = torch.empty(B * kvd + 1, dtype=src, device=cuda)
    vb = torch.empty(B * kvd + 1, dtype=src, device=cuda)
    kb[1:].copy_(kt.reshape(-1))
    vb[1:].copy_(vt.reshape(-1))
    km, vm = kb[1:].view(B, kvd), vb[1:].view(B, kvd)
    assert km.data_ptr() % 16 != 0
    blk, elt = LayerKV.empty(n_kv, hd, ps + B + 30, device=cuda), LayerKV.empty(n_kv, hd, ps + B + 30, device=cuda)
    kv_store(blk, kt, vt, ps)
    kv_store(elt, km, vm, ps)
    torch.cuda.synchronize()
    assert torch.equal(blk.k, elt.k) and torch.equal(blk.v, elt.v)
    Kb, Vb = cache_bits(blk)
    Kx, Vx = kt.float().cpu().numpy(), vt.float().cpu().numpy()
    Kw, Vw = engine_to_headmajor(oracle.f32_to_f16(Kx), oracle.f32_to_f16(Vx), n_kv, hd, -(-B // 64) * 64)
    assert np.array_equal(Kb[:, ps:ps + B], Kw[:, :B])
    assert np.array_equal(untile_v(Vb)[:, :, ps:ps + B], untile_v(Vw)[:, :, :B])
    assert not Kb[:, :ps].any() and not Kb[:, ps + B:].any()
    assert not untile_v(Vb)[:, :, :ps].any() and not untile_v(Vb)[:, :, ps + B:].any()


@pytest.mark.parametrize("src", [torch.float32, torch.bfloat16])
def test_kv_store_few_rows_matches_bulk(cuda, src):
    """Appending 1-3 rows at a time (the one-launch path) writes the same bits
    as one bulk store of all rows."""
    from yllm_amd.attention import LayerKV, kv_store

    n_kv, hd, rows = 2, 128, 70
    K, V = gen(61, (rows, n_kv * hd), f16=False), gen(62, (rows, n_kv * hd), f16=False)
    kt, vt = torch.from_numpy(K).to(cuda).to(src), torch.from_numpy(V).to(cuda).to(src)
    bulk, step = LayerKV.empty(n_kv, hd, rows, device=cuda), LayerKV.empty(n_kv, hd, rows, device=cuda)
    kv_store(bulk, kt, vt, 0)
    p, n = 0, 1
    while p < rows:
        m = min(n, rows - p)
        kv_store(step, kt[p:p + m], vt[p:p + m], p)
        p, n = p + m, n % 3 + 1
    torch.cuda.synchronize()
    assert torch.equal(bulk.k, step.k) and torch.equal(bulk.v, step.v)


def test_kv_engine_layout_round_trip(cuda, oracle):
    from yllm_amd.attention import LayerKV, kv_from_engine, kv_to_engine

    n_kv, hd, n = 4, 128, 300
    eng = oracle.f32_to_f16(gen(7, (2, n, n_kv * hd), f16=False))
    ek = torch.from_numpy(eng[0].view(np.int16)).to(cuda)
    ev = torch.from_numpy(eng[1].view(np.int16)).to(cuda)
    cache = LayerKV.empty(n_kv, hd, n, device=cuda)
    kv_from_engine(cache, ek, ev)
    Kb, Vb = cache_bits(cache)
    Kw, Vw = engine_to_headmajor(eng[0], eng[1], n_kv, hd, cache.kv_stride)
    assert np.array_equal(Kb, Kw) and np.array_equal(Vb, Vw)
    bk, bv = kv_to_engine(cache, n)
    assert np.array_equal(bk.view(torch.int16).cpu().numpy().view(np.uint16), eng[0])
    assert np.array_equal(bv.view(torch.int16).cpu().numpy().view(np.uint16), eng[1])


# --------------------------------------------------------------------- decode

def test_decode_reference_config1_fixture(cuda, oracle, golden):
    """Config 1 (14q/2kv, d=64, 512 keys) with the query and rows the reference engine produced."""
    from yllm_amd.attention import LayerKV, attn_decode, kv_from_engine
    from test_oracle import _decode_case

    (nh, nkv, hd, pos), q, kc, vc = _decode_case(oracle, golden, "dec_cfg1")
    cache = LayerKV.empty(nkv, hd, pos + 1, device=cuda)
    kv_from_engine(cache, torch.from_numpy(kc.view(np.int16)).to(cuda), torch.from_numpy(vc.view(np.int16)).to(cuda))
    out = attn_decode(torch.from_numpy(q).to(cuda), cache, pos, nh).cpu().numpy()
    err = rel_l2(out, golden["dec_cfg1_att"])
    print(f"config1 decode rel_l2 vs reference engine = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("nh,nkv,hd,L", [
    (14, 2, 64, 512), (32, 8, 128, 1), (32, 8, 128, 31), (32, 8, 128, 33), (32, 8, 128, 4097),
    (28, 4, 128, 2048), (6, 4, 64, 300), (16, 2, 256, 777), (8, 8, 128, 20000),
    (32, 16, 64, 6000), (24, 8, 256, 9000), (12, 8, 128, 7000),
    (8, 2, 64, 600), (8, 2, 128, 300), (32, 8, 128, 300), (6, 2, 64, 257),
    # splits of 1280 keys (more than 1024): K loaded as MFMA operands
    (8, 8, 64, 40000), (16, 8, 256, 40000)])
def test_decode_parity(cuda, oracle, nh, nkv, hd, L):
    """Split-K decode against the oracle; kv head counts that are multiples of
    8 with whole query-head groups run the kv-head-first grids (32/8, 8/8,
    32/16 with two kv heads per XCD, 24/8 at d 256), 12/8 the split-major
    ones; 600, 300 and 257 keys run unsplit with several blocks per wave and
    a partial last block."""
    from yllm_amd.attention import attn_decode

    kvd = nkv * hd
    K = gen(100 + L, (L, kvd))
    V = gen(200 + L, (L, kvd))
    q = gen(300 + L, (nh * hd,), f16=False)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    want = oracle.decode(q, kc, vc, L - 1, nh, nkv, hd)
    got = attn_decode(torch.from_numpy(q).to(cuda), cache, L - 1, nh).cpu().numpy()
    err = rel_l2(got, want)
    print(f"decode {nh}/{nkv} d={hd} L={L}: rel_l2={err:.3e}")
    assert err <= TOL


def test_decode_gated_parity(cuda, oracle):
    from yllm_amd.attention import attn_decode

    nh, nkv, hd, L = 16, 2, 256, 1500
    kvd = nkv * hd
    K, V = gen(11, (L, kvd)), gen(12, (L, kvd))
    q = gen(13, (nh * hd,))
    gate = gen(14, (nh * hd,), 1.0, f16=False)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd, src=torch.bfloat16)
    want = oracle.gate_sigmoid(oracle.decode(q, kc, vc, L - 1, nh, nkv, hd), gate)
    got = attn_decode(torch.from_numpy(q).to(cuda), cache, L - 1, nh, gate=torch.from_numpy(gate).to(cuda))
    err = rel_l2(got.cpu().numpy(), want)
    print(f"gated decode rel_l2={err:.3e}")
    assert err <= TOL


def test_decode_batch_ragged_parity(cuda, oracle):
    from yllm_amd.attention import DecodeBatch, LayerKV, attn_decode_batch, kv_store

    nh, nkv, hd = 32, 8, 128
    kvd = nkv * hd
    lens = [1, 95, 1024, 3001, 777, 64, 8191]
    stride = 8192
    caches, wants, qs = [], [], []
    for i, L in enumerate(lens):
        K, V = gen(400 + i, (L, kvd)), gen(500 + i, (L, kvd))
        q = gen(600 + i, (nh * hd,), f16=False)
        c = LayerKV.empty(nkv, hd, stride, device=cuda)
        kv_store(c, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda), 0)
        caches.append(c)
        qs.append(q)
        wants.append(oracle.decode(q, oracle.f32_to_f16(K), oracle.f32_to_f16(V), L - 1, nh, nkv, hd))
    batch = DecodeBatch(caches)
    got = attn_decode_batch(torch.from_numpy(np.stack(qs)).to(cuda), batch, lens, nh).cpu().numpy()
    for i, L in enumerate(lens):
        err = rel_l2(got[i], wants[i])
        print(f"batch seq {i} L={L}: rel_l2={err:.3e}")
        assert err <= TOL


def test_decode_workspace_reuse_across_calls(cuda, oracle):
    """One workspace serves many split-K calls of different lengths (stale
    partials of a longer call must never leak into a shorter one)."""
    from yllm_amd.attention import attn_decode, decode_workspace, decode_workspace_bytes

    nh, nkv, hd, L = 32, 8, 128, 9000
    kvd = nkv * hd
    K, V = gen(21, (L, kvd)), gen(22, (L, kvd))
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    ws = decode_workspace(decode_workspace_bytes(1, L, L, nh, nkv, hd), cuda)
    for i, n in enumerate([9000, 4500, 9000, 777, 8999, 9000]):
        q = gen(23 + i, (nh * hd,), f16=False)
        want = oracle.decode(q, kc[:n], vc[:n], n - 1, nh, nkv, hd)
        got = attn_decode(torch.from_numpy(q).to(cuda), cache, n - 1, nh, workspace=ws).cpu().numpy()
        err = rel_l2(got, want)
        print(f"reuse call {i} keys={n}: rel_l2={err:.3e}")
        assert err <= TOL


def test_decode_workspace_for_max_len_serves_every_position(cuda, oracle):
    """The engine sizes one decode workspace for max_seq and decodes at every
    position below it.  The split count is not monotone in the length (at
    32/8 heads, 4352 keys split 17 ways and 4096 keys 32 ways), so a
    workspace of yhip_attn_decode_workspace(1, 4352, ...) must serve every
    shorter call: each C call below gets exactly that many bytes."""
    from yllm_amd._lib import check, lib
    from yllm_amd.attention import decode_workspace, decode_workspace_bytes

    nh, nkv, hd, L = 32, 8, 128, 4352
    kvd = nkv * hd
    K, V = gen(41, (L, kvd)), gen(42, (L, kvd))
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    nbytes = decode_workspace_bytes(1, L, L, nh, nkv, hd)
    ws = decode_workspace(nbytes, cuda)
    q = gen(43, (nh * hd,), f16=False)
    qt = torch.from_numpy(q).to(cuda)
    out = torch.empty(nh * hd, dtype=torch.float32, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    for n in range(2900, L + 1):
        check(lib().yhip_attn_decode(out.data_ptr(), qt.data_ptr(), cache.k.data_ptr(), cache.v.data_ptr(), n - 1, nh,
                                     nkv, hd, cache.kv_stride, None, ws.data_ptr(), nbytes, stream))
        if n in (2900, 3000, 4096, 4097, 4224, L):
            want = oracle.decode(q, kc[:n], vc[:n], n - 1, nh, nkv, hd)
            err = rel_l2(out.cpu().numpy(), want)
            assert err <= TOL, f"{n} keys: rel_l2 {err:.3e}"


@pytest.mark.parametrize("nh,nkv", [(8, 2), (32, 8)])
@pytest.mark.parametrize("max_len", [100, 300, 5000])
def test_decode_batch_empty_sequence_gives_zeros(cuda, oracle, max_len, nh, nkv):
    """A sequence with no keys gets a zero output row, with one split
    (max_len 100) as with several (5000), gated or not; 8 kv heads take the
    kv-head-first grids (a kv head's splits and merges on one XCD)."""
    from yllm_amd.attention import DecodeBatch, LayerKV, attn_decode_batch, kv_store

    hd = 128
    kvd = nkv * hd
    lens = [max_len, 0, 37]
    caches, wants, qs = [], [], []
    gate = gen(49, (3, nh * hd), 1.0, f16=False)
    for i, L in enumerate(lens):
        K, V = gen(450 + i, (max(L, 1), kvd)), gen(550 + i, (max(L, 1), kvd))
        q = gen(650 + i, (nh * hd,), f16=False)
        c = LayerKV.empty(nkv, hd, max_len, device=cuda)
        kv_store(c, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda), 0)
        caches.append(c)
        qs.append(q)
        wants.append(None if L == 0 else
                     oracle.decode(q, oracle.f32_to_f16(K[:L]), oracle.f32_to_f16(V[:L]), L - 1, nh, nkv, hd))
    for g in (None, torch.from_numpy(gate).to(cuda)):
        out = torch.full((3, nh * hd), float("nan"), device=cuda)
        attn_decode_batch(torch.from_numpy(np.stack(qs)).to(cuda), DecodeBatch(caches), lens, nh, gate=g, out=out)
        got = out.cpu().numpy()
        assert (got[1] == 0).all()
        for i in (0, 2):
            want = wants[i] if g is None else oracle.gate_sigmoid(wants[i], gate[i])
            assert rel_l2(got[i], want) <= TOL


def test_decode_long_context_full_size(cuda, oracle):
    """Config 4 decode at its full size: 131072 keys, 32q/8kv, d=128 (split-K + LSE merge)."""
    from yllm_amd.attention import attn_decode

    nh, nkv, hd, L = 32, 8, 128, 131072
    kvd = nkv * hd
    K, V = gen(0x5EED0004, (L, kvd)), gen(0x5EED0104, (L, kvd))
    q = gen(0x5EED0204, (nh * hd,))
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    Kb, _ = cache_bits(cache)
    assert np.array_equal(Kb[3, 77777], kc[77777, 3 * hd:4 * hd])
    want = oracle.decode(q, kc, vc, L - 1, nh, nkv, hd)
    got = attn_decode(torch.from_numpy(q).to(cuda), cache, L - 1, nh).cpu().numpy()
    err = rel_l2(got, want)
    print(f"decode 131072 rel_l2={err:.3e}")
    assert err <= TOL


# -------------------------------------------------------------------- prefill

@pytest.mark.parametrize("nh,nkv,hd,ps,B,qdt,odt", [
    (28, 4, 128, 0, 300, torch.float16, torch.float32),
    (28, 4, 128, 100, 77, torch.float32, torch.float32),
    (14, 2, 64, 0, 129, torch.float32, torch.float16),
    (32, 8, 128, 5, 64, torch.bfloat16, torch.bfloat16),
    (6, 4, 64, 0, 1, torch.float32, torch.float32),
    (16, 2, 256, 30, 200, torch.bfloat16, torch.float32),
    # a query block with idle waves and three key tiles: the idle waves must
    # not restage tile 0 while the busy one still scores it
    (2, 1, 256, 0, 129, torch.float32, torch.float32),
    (4, 1, 128, 0, 129, torch.float16, torch.float32),
    (2, 2, 64, 0, 193, torch.float32, torch.float32),
    # head_dim 256 (32-key tiles, two waves per 32 queries): a start inside
    # a tile, GQA 8:1, many items; and f16 queries into bf16 output
    (8, 1, 256, 45, 300, torch.float16, torch.bfloat16),
    (32, 4, 256, 0, 1100, torch.float16, torch.float32),
])
def test_prefill_parity(cuda, oracle, nh, nkv, hd, ps, B, qdt, odt):
    from yllm_amd.attention import attn_prefill

    kvd = nkv * hd
    L = ps + B
    K, V = gen(700 + L, (L, kvd)), gen(800 + L, (L, kvd))
    q = gen(900 + L, (B, nh * hd))
    if qdt == torch.bfloat16:
        from yllm_amd.attention import round_bf16

        q = round_bf16(q.ravel().copy()).reshape(B, nh * hd)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    want = oracle.prefill(q, kc, vc, ps, B, nh, nkv, hd)
    qt = torch.from_numpy(q).to(cuda).to(qdt)
    got = attn_prefill(qt, cache, ps, nh, out_dtype=odt).float().cpu().numpy()
    err = rel_l2(got, want)
    print(f"prefill {nh}/{nkv} d={hd} ps={ps} B={B} q={qdt} out={odt}: rel_l2={err:.3e}")
    # a bf16-typed output adds its own rounding (up to 2^-9 relative per element)
    tol = TOL + (2.0 ** -8 if odt == torch.bfloat16 else 0.0)
    assert err <= tol
    # every row on its own, so one bad query cannot hide in the average
    rows = [rel_l2(got[i], want[i]) for i in range(B)]
    assert max(rows) <= 3 * tol


@pytest.mark.parametrize("nh,nkv,hd,B,qsig", [(28, 4, 128, 192, 1.0), (28, 4, 128, 192, 4.0), (28, 4, 128, 192, 8.0),
                                            (16, 2, 256, 130, 4.0), (8, 8, 64, 100, 8.0)])
def test_prefill_f32_queries_large_scores(cuda, oracle, nh, nkv, hd, B, qsig):
    """fp32 queries that f16 cannot represent, scaled up to scores of std
    ~qsig/2 (|s| up to ~20 at qsig 8), the peaked softmax of qsig 8 included:
    the kernel takes fp32 q as f16 hi + lo parts, so the scores keep
    fp32-level error."""
    from yllm_amd.attention import attn_prefill

    kvd = nkv * hd
    K, V = gen(1700 + hd, (B, kvd)), gen(1800 + hd, (B, kvd))
    q = gen(1900 + hd, (B, nh * hd), qsig, f16=False)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    want = oracle.prefill(q, kc, vc, 0, B, nh, nkv, hd)
    s0 = q[:, :hd] @ K[:, :hd].T / np.sqrt(hd)  # head 0's scores (before the causal mask)
    got = attn_prefill(torch.from_numpy(q).to(cuda), cache, 0, nh).cpu().numpy()
    err = rel_l2(got, want)
    rows = max(rel_l2(got[i], want[i]) for i in range(B))
    print(f"prefill f32 q sigma {qsig} {nh}/{nkv} d={hd}: head-0 score std {s0.std():.2f} max {np.abs(s0).max():.1f}, "
          f"rel_l2={err:.3e}, worst row {rows:.3e}")
    assert err <= TOL and rows <= 3 * TOL


@pytest.mark.parametrize("nh,nkv,hd,ps,B,plain", [
    (8, 2, 128, 448, 64, False),    # the engine's 64-token call: packed rows, split keys
    (16, 2, 256, 200, 64, False),   # the gated layer's head shape, pair mode
    (32, 4, 128, 0, 1024, True),    # 256 (query block, head) items: the plain mode
    (8, 8, 64, 0, 200, False),
])
def test_prefill_f32_queries_competing_large_scores(cuda, oracle, nh, nkv, hd, ps, B, plain):
    """Scores of 60..100 (and up to twice that where both picks are one key)
    with two keys competing: every query is built from two keys of its kv
    head in its causal range, q = c (k1/|k1|^2 + k2/|k2|^2) + noise, so both
    score about c/sqrt(d) and its softmax splits between them.  A score error
    of |s| 2^-11 (q rounded to f16) moves these outputs by ~1e-3 overall and
    ~4e-3 in the worst rows (computed in fp64 when the case was built); the
    kernel takes fp32 q as f16 hi + lo parts (two MFMAs), so the scores keep
    fp32-level error and the outputs stay well within 1e-3 of the fp32
    oracle."""
    from yllm_amd.attention import attn_prefill

    kvd = nkv * hd
    L = ps + B
    K, V = gen(2100 + hd, (L, kvd)), gen(2200 + hd, (L, kvd))
    rng = np.random.default_rng(2300 + hd)
    q = np.empty((B, nh * hd), np.float32)
    for b in range(B):
        for h in range(nh):
            kv = h * nkv // nh
            j1, j2 = rng.integers(0, ps + b + 1, size=2)
            k1, k2 = K[j1, kv * hd:(kv + 1) * hd], K[j2, kv * hd:(kv + 1) * hd]
            c = rng.uniform(60.0, 100.0) * np.sqrt(hd)
            q[b, h * hd:(h + 1) * hd] = c * (k1 / np.dot(k1, k1) + k2 / np.dot(k2, k2)) + rng.normal(0.0, 0.05, hd)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    top = np.array([np.max(q[b, :hd] @ K[: ps + b + 1, :hd].T) / np.sqrt(hd) for b in range(B)])  # head 0
    got = attn_prefill(torch.from_numpy(q).to(cuda), cache, ps, nh).cpu().numpy()
    if plain:
        rows = [0, 1, 127, 128, 500, B - 1]
        errs = [rel_l2(got[t], oracle.decode(q[t], kc[: ps + t + 1], vc[: ps + t + 1], ps + t, nh, nkv, hd))
                for t in rows]
        err = max(errs)
    else:
        want = oracle.prefill(q, kc, vc, ps, B, nh, nkv, hd)
        err = rel_l2(got, want)
        errs = [rel_l2(got[i], want[i]) for i in range(B)]
    print(f"prefill f32 q competing keys {nh}/{nkv} d={hd} ps={ps} B={B}: head-0 top score {top.min():.1f}.."
          f"{top.max():.1f} (median {np.median(top):.1f}), rel_l2={err:.3e}, worst row {max(errs):.3e}")
    assert np.median(top) >= 40.0
    assert err <= TOL and max(errs) <= 3 * TOL


def test_prefill_gated_parity(cuda, oracle):
    from yllm_amd.attention import attn_prefill

    nh, nkv, hd, B = 16, 2, 256, 96
    kvd = nkv * hd
    K, V = gen(31, (B, kvd)), gen(32, (B, kvd))
    q = gen(33, (B, nh * hd))
    gate = gen(34, (B, nh * hd), 1.0, f16=False)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    want = oracle.gate_sigmoid(oracle.prefill(q, kc, vc, 0, B, nh, nkv, hd).ravel(), gate.ravel())
    got = attn_prefill(torch.from_numpy(q).to(cuda), cache, 0, nh, gate=torch.from_numpy(gate).to(cuda))
    err = rel_l2(got.cpu().numpy().ravel(), want)
    print(f"gated prefill rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("nh,nkv,hd,ps,B,qdt,odt,gated", [
    # more (query block, head) items than resident 8-wave workgroups: each
    # workgroup walks several items, the next item's tiles load during the
    # previous one's last key step (f32 queries load at the item's start)
    (28, 4, 128, 0, 2048, torch.float32, torch.float32, False),
    # gated: every item issues its own loads; 3 kv heads: items are not
    # grouped per XCD; unaligned start and a partial last query block
    (24, 3, 128, 37, 2000, torch.float16, torch.float32, True),
    (32, 8, 64, 0, 2048, torch.bfloat16, torch.float16, False),
])
def test_prefill_resident_workgroups_sampled_rows(cuda, oracle, nh, nkv, hd, ps, B, qdt, odt, gated):
    from yllm_amd.attention import attn_prefill, round_bf16

    kvd = nkv * hd
    L = ps + B
    K, V = gen(1700 + L, (L, kvd)), gen(1800 + L, (L, kvd))
    q = gen(1900 + L, (B, nh * hd))
    if qdt == torch.bfloat16:
        q = round_bf16(q.ravel().copy()).reshape(B, nh * hd)
    gate = gen(2000 + L, (B, nh * hd), 1.0, f16=False) if gated else None
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    got = attn_prefill(torch.from_numpy(q).to(cuda).to(qdt), cache, ps, nh, out_dtype=odt,
                       gate=torch.from_numpy(gate).to(cuda) if gated else None).float().cpu().numpy()
    assert np.isfinite(got).all()
    tol = TOL + (2.0 ** -10 if odt == torch.float16 else 0.0)
    for b in (0, 1, 127, 128, 255, 640, 1023, 1024, 1500, B - 129, B - 2, B - 1):
        t = ps + b
        want = oracle.decode(q[b], kc[: t + 1], vc[: t + 1], t, nh, nkv, hd)
        if gated:
            want = oracle.gate_sigmoid(want.ravel(), gate[b].ravel())
        err = rel_l2(got[b].ravel(), want.ravel())
        assert err <= tol, f"row {b}: rel_l2={err:.3e}"


@pytest.mark.parametrize("nh,nkv,hd,L", [(28, 4, 128, 2048), (32, 8, 128, 8192)])
def test_prefill_full_size_sampled_rows(cuda, oracle, nh, nkv, hd, L):
    """Configs 2 and 4-prefill at full size: sampled rows against the oracle at their position,
    plus rows compared with the GPU decode kernel at the same position."""
    from yllm_amd.attention import attn_decode, attn_prefill

    kvd = nkv * hd
    K, V = gen(0x5EED0002 + L, (L, kvd)), gen(0x5EED0102 + L, (L, kvd))
    q = gen(0x5EED0202 + L, (L, nh * hd))
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    got = attn_prefill(torch.from_numpy(q).to(cuda).half(), cache, 0, nh).cpu().numpy()
    assert np.isfinite(got).all()
    for t in (0, 1, 63, 64, 127, 128, 1000, L // 2 + 17, L - 2, L - 1):
        want = oracle.decode(q[t], kc[: t + 1], vc[: t + 1], t, nh, nkv, hd)
        err = rel_l2(got[t], want)
        dec = attn_decode(torch.from_numpy(q[t]).to(cuda), cache, t, nh).cpu().numpy()
        assert err <= TOL, f"row {t}: rel_l2={err:.3e}"
        assert rel_l2(got[t], dec) <= TOL


# ------------------------------------------------------ prefill: engine chunks

@pytest.mark.parametrize("nh,nkv,hd,ps,B,qdt,odt,gated", [
    # the engine's 64-token chunks (engine.c:270-272, 622-653) at the start,
    # middle and end of an 8k prompt: packed rows, split keys
    (28, 4, 128, 0, 64, torch.float32, torch.float32, False),
    (28, 4, 128, 1984, 64, torch.float32, torch.float32, False),
    (32, 8, 128, 8128, 64, torch.float16, torch.float32, False),
    (16, 2, 256, 4032, 64, torch.bfloat16, torch.bfloat16, True),
    (16, 2, 256, 1001, 37, torch.float32, torch.float32, False),
    (4, 4, 256, 100, 200, torch.float16, torch.float32, True),
    (14, 2, 64, 2000, 64, torch.float32, torch.float16, False),
    # a wave's rows straddle two heads (B not a multiple of 32); uneven groups
    (28, 4, 128, 3001, 37, torch.float32, torch.float32, False),
    (6, 4, 64, 777, 50, torch.float32, torch.float32, True),
    (32, 8, 128, 5000, 1, torch.float32, torch.float32, False),
    # plain rows (B >= 128) with split keys: few (query block, head) items
    (8, 2, 128, 3000, 200, torch.float16, torch.float32, False),
])
def test_prefill_engine_chunk_parity(cuda, oracle, nh, nkv, hd, ps, B, qdt, odt, gated):
    from yllm_amd.attention import attn_prefill, prefill_workspace_bytes, round_bf16

    kvd = nkv * hd
    L = ps + B
    K, V = gen(2700 + L, (L, kvd)), gen(2800 + L, (L, kvd))
    q = gen(2900 + L, (B, nh * hd), f16=(qdt == torch.float16))
    if qdt == torch.bfloat16:
        q = round_bf16(q.ravel().copy()).reshape(B, nh * hd)
    gate = gen(3000 + L, (B, nh * hd), 1.0, f16=False) if gated else None
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    want = oracle.prefill(q, kc, vc, ps, B, nh, nkv, hd)
    if gated:
        want = oracle.gate_sigmoid(want.ravel(), gate.ravel()).reshape(B, nh * hd)
    qt = torch.from_numpy(q).to(cuda).to(qdt)
    gt = torch.from_numpy(gate).to(cuda) if gated else None
    tol = TOL + (2.0 ** -8 if odt == torch.bfloat16 else 2.0 ** -10 if odt == torch.float16 else 0.0)
    need = prefill_workspace_bytes(B, L, nh, nkv, hd)
    # with the key-split workspace (the mirror allocates it), then through the
    # C ABI without one: the same packing, unsplit
    from yllm_amd._lib import check, lib

    for split in (True, False):
        if split:
            out = attn_prefill(qt, cache, ps, nh, out_dtype=odt, gate=gt)
        else:
            out = torch.empty((B, nh * hd), dtype=odt, device=cuda)
            code = {torch.float32: 1, torch.float16: 0, torch.bfloat16: 2}
            check(lib().yhip_attn_prefill(out.data_ptr(), code[odt], nh * hd, qt.data_ptr(), code[qdt], nh * hd,
                                          cache.k.data_ptr(), cache.v.data_ptr(), ps, B, nh, nkv, hd, cache.kv_stride,
                                          gt.data_ptr() if gated else None, nh * hd if gated else 0, None, 0,
                                          torch.cuda.current_stream().cuda_stream))
        got = out.float().cpu().numpy()
        err = rel_l2(got, want)
        rows = max(rel_l2(got[i], want[i]) for i in range(B))
        print(f"chunk {nh}/{nkv} d={hd} ps={ps} B={B} {'split' if split else 'unsplit'} ({need} B): "
              f"rel_l2={err:.3e} worst row {rows:.3e}")
        assert np.isfinite(got).all()
        assert err <= tol and rows <= 3 * tol


def test_prefill_chunked_prompt_equals_single_launch(cuda, oracle):
    """A 2048-token prompt issued as 32 calls of 64 tokens (the engine's
    chunking, every call a split launch) gives the single launch's result to
    rounding, and both match the oracle's rows."""
    from yllm_amd.attention import attn_prefill, prefill_workspace, prefill_workspace_bytes

    nh, nkv, hd, L, C = 28, 4, 128, 2048, 64
    kvd = nkv * hd
    K, V = gen(0x5EED0002 + 7, (L, kvd)), gen(0x5EED0102 + 7, (L, kvd))
    q = gen(0x5EED0202 + 7, (L, nh * hd), f16=False)
    cache, kc, vc = make_cache(cuda, oracle, K, V, nkv, hd)
    qt = torch.from_numpy(q).to(cuda)
    whole = attn_prefill(qt, cache, 0, nh).cpu().numpy()
    out = torch.empty((L, nh * hd), device=cuda)
    ws = prefill_workspace(prefill_workspace_bytes(C, L, nh, nkv, hd), cuda)
    for p0 in range(0, L, C):
        attn_prefill(qt[p0:p0 + C], cache, p0, nh, out=out[p0:p0 + C], workspace=ws)
    chunked = out.cpu().numpy()
    assert rel_l2(chunked, whole) <= 2e-4
    for t in (0, 63, 64, 1000, 1983, 1984, 2047):
        want = oracle.decode(q[t], kc[: t + 1], vc[: t + 1], t, nh, nkv, hd)
        assert rel_l2(chunked[t], want) <= TOL
