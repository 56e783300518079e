"""CPU checks of the C-ABI library: it loads, exports every declared symbol,
validates arguments before touching the GPU, and its host-side helpers
(generator, conversions) agree with the oracle and the reference fixtures."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from inputs import splitmix

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(yhip_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol(hiplib):
    from yllm_amd._lib import SIGNATURES

    names = declared_symbols()
    assert names, "no declarations found"
    for n in sorted(names):
        assert hasattr(hiplib, n), f"{n} declared in include/ but not exported"
    assert names == set(SIGNATURES), "binding table and header disagree"


def test_version(hiplib):
    assert b"gfx950" in hiplib.yhip_version()


def _err(hiplib):
    return hiplib.yhip_last_error().decode()


P = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


@pytest.mark.parametrize("hd,nh,nkv,stride,msg", [
    (96, 8, 2, 128, "head_dim"),
    (128, 8, 0, 128, "n_kv_heads"),
    (128, 2, 4, 128, "n_kv_heads"),
    (128, 34, 2, 128, "16 query heads"),
    (128, 8, 2, 100, "multiple of 64"),
    (256, 8, 2, 1 << 22, "under 2 GiB"),   # 4M positions x 256 dims x 2 B = 2 GiB per kv head
])
def test_decode_rejects_bad_shapes(hiplib, hd, nh, nkv, stride, msg):
    rc = hiplib.yhip_attn_decode(P, P, P, P, 3, nh, nkv, hd, stride, None, None, 0, None)
    assert rc == -22 and msg in _err(hiplib)


def test_decode_rejects_null_and_range(hiplib):
    assert hiplib.yhip_attn_decode(None, P, P, P, 3, 8, 2, 128, 128, None, None, 0, None) == -22
    assert hiplib.yhip_attn_decode(P, P, P, P, 128, 8, 2, 128, 128, None, None, 0, None) == -22
    assert "pos" in _err(hiplib)


def test_decode_workspace_is_checked(hiplib):
    need = hiplib.yhip_attn_decode_workspace(1, 100000, 100000, 32, 8, 128)
    assert need > 0
    rc = hiplib.yhip_attn_decode(P, P, P, P, 99999, 32, 8, 128, 131072, None, P, 4096, None)
    assert rc == -28 and "workspace" in _err(hiplib)
    # a short context needs no split and no workspace
    assert hiplib.yhip_attn_decode_workspace(1, 64, 64, 32, 8, 128) == 0


@pytest.mark.parametrize("nh,nkv,hd,max_len", [(32, 8, 128, 4352), (28, 4, 128, 10000), (16, 2, 256, 4352),
                                               (14, 2, 64, 512), (32, 8, 128, 131072)])
def test_decode_workspace_serves_every_shorter_position(hiplib, nh, nkv, hd, max_len):
    """A single-sequence workspace sized for max_len serves every shorter call:
    the size never shrinks as max_len grows, although the split count is not
    monotone in the length (4352 keys at 32/8 split 17 ways, 4096 keys 32
    ways).  The engine sizes one workspace for max_seq."""
    ws = hiplib.yhip_attn_decode_workspace
    sizes = np.array([ws(1, L, L, nh, nkv, hd) for L in range(1, max_len + 1, 1 if max_len <= 20000 else 61)])
    assert (np.diff(sizes.astype(np.int64)) >= 0).all()
    assert sizes[-1] == ws(1, max_len, max_len, nh, nkv, hd)


def test_prefill_rejects_bad_args(hiplib):
    # positions past the cache
    rc = hiplib.yhip_attn_prefill(P, 1, 1024, P, 1, 1024, P, P, 100, 64, 8, 2, 128, 128, None, 0, None, 0, None)
    assert rc == -22 and "exceed" in _err(hiplib)
    # dtype
    rc = hiplib.yhip_attn_prefill(P, 7, 1024, P, 1, 1024, P, P, 0, 64, 8, 2, 128, 128, None, 0, None, 0, None)
    assert rc == -22 and "dtype" in _err(hiplib)
    # stride
    rc = hiplib.yhip_attn_prefill(P, 1, 1000, P, 1, 1024, P, P, 0, 64, 8, 2, 128, 128, None, 0, None, 0, None)
    assert rc == -22 and "stride" in _err(hiplib)
    # empty batch is a no-op
    assert hiplib.yhip_attn_prefill(P, 1, 1024, P, 1, 1024, P, P, 0, 0, 8, 2, 128, 128, None, 0, None, 0, None) == 0


def test_kv_store_rejects_overflow(hiplib):
    rc = hiplib.yhip_kv_store(P, P, P, P, 1, 120, 9, 2, 128, 128, None)
    assert rc == -22 and "exceed" in _err(hiplib)
    assert hiplib.yhip_kv_store(P, P, P, P, 1, 0, 0, 2, 128, 128, None) == 0


def test_host_f16_rounding_matches_reference(hiplib, golden):
    from yllm_amd.attention import f32_to_f16_bits

    # the same __host__ __device__ routine rounds on the GPU
    assert np.array_equal(f32_to_f16_bits(golden["conv_f32"]), golden["conv_f32_to_f16"])


def test_synth_normal_is_splitmix_box_muller(hiplib, golden):
    from yllm_amd.attention import synth_normal

    seed = int(golden["yrng_seed"][0])
    x = synth_normal(seed, 16, 0.5)
    r = golden["yrng_first16"]  # the reference yrng stream for this seed
    u = ((r >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0
    rad = np.sqrt(-2.0 * np.log(u[0::2]))
    z = np.empty(16)
    z[0::2] = rad * np.cos(2 * np.pi * u[1::2])
    z[1::2] = rad * np.sin(2 * np.pi * u[1::2])
    assert np.allclose(x, (0.5 * z).astype(np.float32), rtol=1e-6, atol=1e-7)
    # chunks are independent of where generation starts
    full = synth_normal(7, 1000)
    assert np.array_equal(full[333:777], synth_normal(7, 444, first=333))
    # the portable fixture generator walks the same stream
    assert np.array_equal(splitmix(seed, 16), r)
    # moments
    big = synth_normal(123, 200000, 0.5)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 0.5) < 0.01


def test_gdn_rejects_bad_args(hiplib):
    F = ctypes.c_float
    # head_dim outside {64, 128}
    rc = hiplib.yhip_gdn_chunk(P, None, P, 4096, P, P, 4096, P, 4096, P, P, 8, 16, 16, 256, F(1e-6), None, 0, None)
    assert rc == -22 and "head_dim" in _err(hiplib)
    # strides that do not cover the heads
    rc = hiplib.yhip_gdn_chunk(P, None, P, 2048, P, P, 1024, P, 2048, P, P, 8, 16, 16, 128, F(1e-6), None, 0, None)
    assert rc == -22 and "strides" in _err(hiplib)
    # misaligned q
    rc = hiplib.yhip_gdn_chunk(P, None, P, 2048, ctypes.c_void_p(0x1004), P, 2048, P, 2048, P, P, 8, 16, 16, 128, F(1e-6),
                               None, 0, None)
    assert rc == -22 and "aligned" in _err(hiplib)
    # null pointers
    rc = hiplib.yhip_gdn_step(None, P, P, P, P, P, P, 16, 16, 128, F(1e-6), None)
    assert rc == -22 and "null" in _err(hiplib)
    rc = hiplib.yhip_gdn_gates(P, None, P, P, P, 4, 16, None)
    assert rc == -22 and "null" in _err(hiplib)
    # no tokens is a no-op
    assert hiplib.yhip_gdn_chunk(P, None, P, 2048, P, P, 2048, P, 2048, P, P, 0, 16, 16, 128, F(1e-6), None, 0, None) == 0
    # a workspace that is too small for the chunked form
    rc = hiplib.yhip_gdn_chunk(P, None, P, 2048, P, P, 2048, P, 2048, P, P, 128, 16, 16, 128, F(1e-6), P, 4096, None)
    assert rc == -28 and "workspace" in _err(hiplib)
    assert hiplib.yhip_gdn_chunk_workspace(63, 16, 128) == 0
    # per (head, chunk): -W in bf16, Q~ and K~ in bf16 hi / lo, P likewise, U^T, gamma_last + pad
    assert hiplib.yhip_gdn_chunk_workspace(4096, 16, 128) == 64 * 16 * (64 * 128 // 2 + 2 * 64 * 128 + 64 * 64
                                                                     + 64 * 128 + 4) * 4
    assert hiplib.yhip_gdn_gates(P, P, P, P, P, 0, 16, None) == 0
    # an out-of-place state that overlaps the state (16 heads x 128 x 128 floats = 1 MiB) is refused
    S0 = ctypes.c_void_p(0x4000000)
    rc = hiplib.yhip_gdn_chunk(S0, ctypes.c_void_p(0x4000000 + 4096), P, 2048, P, P, 2048, P, 2048, P, P, 8, 16, 16,
                               128, F(1e-6), None, 0, None)
    assert rc == -22 and "S_out" in _err(hiplib)


def test_gdn_neighbours_reject_bad_args(hiplib):
    F = ctypes.c_float
    X, O = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x900000)  # never dereferenced
    # conv: kwidth outside 1..8, strides, overlap of out and x, nulls; T = 0 is a no-op
    rc = hiplib.yhip_gdn_conv(O, 512, X, 512, P, None, P, 4, 512, 9, 1, None)
    assert rc == -22 and "kwidth" in _err(hiplib)
    rc = hiplib.yhip_gdn_conv(O, 512, X, 256, P, None, P, 4, 512, 4, 1, None)
    assert rc == -22 and "strides" in _err(hiplib)
    rc = hiplib.yhip_gdn_conv(X, 512, X, 512, P, None, P, 4, 512, 4, 1, None)
    assert rc == -22 and "overlap" in _err(hiplib)
    rc = hiplib.yhip_gdn_conv(O, 512, X, 512, None, None, P, 4, 512, 4, 1, None)
    assert rc == -22 and "null" in _err(hiplib)
    assert hiplib.yhip_gdn_conv(O, 512, X, 512, P, None, P, 0, 512, 4, 1, None) == 0
    # an out-of-place delay line must not overlap the old one (4 rows x 512 channels)
    rc = hiplib.yhip_gdn_conv(O, 512, X, 512, ctypes.c_void_p(0x4000000), ctypes.c_void_p(0x4000000 + 8188), P, 4,
                              512, 4, 1, None)
    assert rc == -22 and "conv_state_out" in _err(hiplib)
    # gated norm: head_dim not a multiple of 64 or above 256, weight dtype, strides
    rc = hiplib.yhip_gdn_gated_norm(P, 2048, P, 2048, P, 2048, P, 1, 4, 16, 100, F(1e-6), None)
    assert rc == -22 and "head_dim" in _err(hiplib)
    rc = hiplib.yhip_gdn_gated_norm(P, 4096, P, 4096, P, 4096, P, 1, 4, 16, 512, F(1e-6), None)
    assert rc == -22 and "head_dim" in _err(hiplib)
    rc = hiplib.yhip_gdn_gated_norm(P, 2048, P, 2048, P, 2048, P, 2, 4, 16, 128, F(1e-6), None)
    assert rc == -22 and "w_dtype" in _err(hiplib)
    rc = hiplib.yhip_gdn_gated_norm(P, 2048, P, 1024, P, 2048, P, 1, 4, 16, 128, F(1e-6), None)
    assert rc == -22 and "strides" in _err(hiplib)
    assert hiplib.yhip_gdn_gated_norm(P, 2048, P, 2048, P, 2048, P, 1, 0, 16, 128, F(1e-6), None) == 0


def test_rope_kv_store_rejects_bad_args(hiplib):
    F = ctypes.c_float

    def call(q_out=P, qdt=1, qos=1024, q=P, qs=1024, ks=256, vs=256, pos=0, B=4, nh=8, nkv=2, d=128, kvs=64,
             rope=2, n_rot=0, k=P):
        return hiplib.yhip_rope_kv_store(q_out, qdt, qos, q, qs, k, ks, P, vs, P, P, pos, B, nh, nkv, d, kvs,
                                         rope, n_rot, F(1e6), None)

    assert call(rope=4) == -22 and "rope kind" in _err(hiplib)
    assert call(rope=3, n_rot=0) == -22 and "n_rot" in _err(hiplib)
    assert call(rope=3, n_rot=33) == -22 and "n_rot" in _err(hiplib)
    assert call(rope=3, n_rot=256) == -22 and "n_rot" in _err(hiplib)
    assert call(d=96) == -22 and "head_dim" in _err(hiplib)
    assert call(nh=40, qs=5120, qos=5120) == -22 and "16 query heads" in _err(hiplib)
    assert call(qdt=3) == -22 and "dtype" in _err(hiplib)
    assert call(ks=255) == -22 and "strides" in _err(hiplib)
    assert call(qs=1000) == -22 and "strides" in _err(hiplib)
    assert call(pos=61, B=4) == -22 and "kv_stride" in _err(hiplib)
    assert call(ks=257) == -22 and "aligned" in _err(hiplib)
    assert call(q=ctypes.c_void_p(0x1004)) == -22 and "aligned" in _err(hiplib)
    assert call(q_out=ctypes.c_void_p(0x1002), qdt=0) == -22 and "aligned" in _err(hiplib)
    assert call(k=None) == -22 and "null" in _err(hiplib)
    assert call(q=None) == -22 and "null" in _err(hiplib)
    # no q (q_out NULL) skips the q checks; B = 0 is a no-op
    assert call(q_out=None, q=None, qs=0, qos=0, B=0) == 0
    assert call(B=0, rope=3, n_rot=64) == 0


def test_o_proj_rejects_bad_args(hiplib):
    def call(x=P, xs=4096, att=P, adt=1, ats=4096, w=P, wdt=0, B=1, hidden=4096, qdim=4096, ws=None, wsb=0):
        return hiplib.yhip_o_proj(x, xs, att, adt, ats, w, wdt, B, hidden, qdim, ws, wsb, None)

    assert call(wdt=2) == -22 and "w_dtype" in _err(hiplib)      # bf16 slots: the reference reads them as f16
    assert call(adt=0, wdt=1) == -22 and "att_dtype" in _err(hiplib)  # f16 att needs f16 weights
    assert call(adt=2) == -22 and "att_dtype" in _err(hiplib)
    assert call(qdim=900) == -22 and "multiple of 8" in _err(hiplib)
    assert call(xs=4000) == -22 and "strides" in _err(hiplib)
    assert call(ats=4100) == -22 and "strides" in _err(hiplib)
    assert call(w=ctypes.c_void_p(0x1008)) == -22 and "aligned" in _err(hiplib)
    assert call(att=None) == -22 and "null" in _err(hiplib)
    # up to 8 tokens need no workspace; more need the f16 hi/lo parts of f32 att (and of f32 weights)
    assert hiplib.yhip_o_proj_workspace(8, 4096, 4096, 0, 1) == 0
    need16 = hiplib.yhip_o_proj_workspace(64, 4096, 4096, 0, 1)
    need32 = hiplib.yhip_o_proj_workspace(64, 4096, 4096, 1, 1)
    assert need16 == 2 * 64 * 4096 * 2
    assert need32 == need16 + 2 * 4096 * 4096 * 2
    assert hiplib.yhip_o_proj_workspace(64, 4096, 4096, 0, 0) == 0  # f16 att: one product, no parts
    assert call(B=64, ws=P, wsb=need16 - 1) == -28 and "workspace" in _err(hiplib)
    assert call(hidden=32768, qdim=32768) == -22  # the weights' byte offsets must fit 32 bits
    assert call(B=0) == 0


def test_gdn_decode_rejects_bad_args(hiplib):
    F = ctypes.c_float
    A, B = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x900000)  # delay lines, never dereferenced

    def call(S=P, cin=A, cout=B, nk=16, nv=16, d=128, kw=4, ndt=1, So=None):
        return hiplib.yhip_gdn_decode(S, So, cin, cout, P, P, P, P, P, P, P, P, P, ndt, nk, nv, d, kw, F(1e-6),
                                      F(1e-6), None)

    assert call(d=256) == -22 and "head_dim" in _err(hiplib)
    assert call(nk=4, nv=2) == -22 and "n_k_heads" in _err(hiplib)
    assert call(kw=9) == -22 and "kwidth" in _err(hiplib)
    assert call(ndt=2) == -22 and "dtype" in _err(hiplib)
    assert call(S=ctypes.c_void_p(0x1004)) == -22 and "aligned" in _err(hiplib)
    assert call(cout=ctypes.c_void_p(0x100000 + 64)) == -22 and "overlaps" in _err(hiplib)
    assert call(cin=None) == -22 and "null" in _err(hiplib)
    # an out-of-place state must not overlap the state (16 heads x 128 x 128 floats = 1 MiB)
    S0 = ctypes.c_void_p(0x4000000)
    assert call(S=S0, So=ctypes.c_void_p(0x4000000 + (1 << 20) - 16)) == -22 and "S_out" in _err(hiplib)
    assert call(S=S0, So=ctypes.c_void_p(0x4000000 + (1 << 20) + 8)) == -22 and "S_out" in _err(hiplib)


def test_decode_rope_rejects_bad_args(hiplib):
    F = ctypes.c_float
    args = lambda **kw: [kw.get("out", P), P, P, P, P, P, kw.get("pos", 0), 8, 8, 64, 64, kw.get("rope", 1),
                         kw.get("n_rot", 0), F(1e4), None, None, 0, None]
    assert hiplib.yhip_attn_decode_rope(*args(out=None)) == -22 and "null" in _err(hiplib)
    assert hiplib.yhip_attn_decode_rope(*args(pos=64)) == -22 and "kv_stride" in _err(hiplib)
    assert hiplib.yhip_attn_decode_rope(*args(rope=9)) == -22 and "rope" in _err(hiplib)
    assert hiplib.yhip_attn_decode_rope(*args(rope=3, n_rot=3)) == -22 and "n_rot" in _err(hiplib)
    assert hiplib.yhip_attn_decode_rope(*args(out=ctypes.c_void_p(0x1004))) == -22 and "aligned" in _err(hiplib)
    # 32k keys split: a workspace is needed
    big = [P, P, P, P, P, P, 32767, 32, 8, 128, 32768, 1, 0, F(1e4), None, None, 0, None]
    assert hiplib.yhip_attn_decode_rope(*big) == -28 and "workspace" in _err(hiplib)
