"""Write tests/golden/ref_vectors.npz from the reference built from its own
sources (oracle/_ref/libyref.so, `make -C oracle ref`).

Every expected value in the fixture is produced by the reference's compiled
code: its f32/f16/bf16 conversions (platform.c), softmax / l2norm /
gdn_state_update / rope_inplace* / matmul (matvec.c), yrng (platform.c), and the attention loops that
are inline in its per-layer forward (engine.c:1074-1096 decode, 532-563
batched prefill, 935-960 gated attention, 788-793 GDN gates), which
oracle/ref_driver.c runs on a synthetic one-block model.  Inputs that are
not produced by the reference (earlier KV rows, projection columns, GDN
states) are regenerated from the seeds stored here with tests/golden/inputs.py.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
sys.path.insert(0, str(HERE))

from inputs import uniform_pm1  # noqa: E402
from oracle_lib import Ref  # noqa: E402

OUT = HERE / "ref_vectors.npz"

# (name, arch, n_heads, n_kv, head_dim, pos): decode through engine_fwd_block_at
DECODE = [
    ("dec_cfg1", 0, 14, 2, 64, 511),      # the reference's CPU-runnable config
    ("dec_qwen", 1, 8, 2, 128, 100),
    ("dec_pos0", 0, 4, 1, 64, 0),         # single key: output = V row
]
# (name, arch, n_heads, n_kv, head_dim, pos_start, B): batched prefill path
PREFILL = [
    ("pre_llama", 0, 4, 2, 64, 40, 16),
    ("pre_qwen", 1, 28, 4, 128, 0, 6),    # config-2 head shape
    ("pre_ragged", 0, 6, 3, 64, 7, 17),   # odd sizes, GQA 2
]
# (name, n_heads, n_kv, head_dim, pos): qwen35 gated attention
GATED = [
    ("gat_small", 4, 2, 256, 63),
    ("gat_cfg5", 16, 2, 256, 130),        # config-5 head shape
]
# (name, n_k, n_v, hd): qwen35 GDN step
GDN = [("gdn_2_4", 2, 4, 16), ("gdn_4_2", 4, 2, 32), ("gdn_3_3", 3, 3, 64)]
# (name, kind, head_dim, n_rot, theta): RoPE of 3 heads at 8 positions
ROPE = [
    ("rope_pairs", 1, 64, 0, 10000.0),        # llama rope_inplace
    ("rope_half", 2, 128, 0, 1000000.0),      # qwen rope_inplace_qwen
    ("rope_mrope", 3, 256, 64, 10000000.0),   # qwen35 rope_inplace_mrope
]


def prev_rows(ref: Ref, seed: int, n: int, kvd: int) -> np.ndarray:
    return ref.f32_to_f16(uniform_pm1(seed, max(n, 1) * kvd).reshape(max(n, 1), kvd))[:n]


def main() -> None:
    ref = Ref()
    fx: dict[str, np.ndarray] = {}

    # ---- conversions: platform.c:316-391 ----
    edge = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, -1e-8, 6.1e-5, 5.96e-8,
                     2.98e-8, 2.99e-8, 1.0009765625, 1.00048828125, 1.000732421875, 3.0517578125e-05,
                     1e-40, -1e-40, np.inf, -np.inf, np.nan, 0.1, 0.2, 1.5e-5, 2.0 ** -15 * 1.5,
                     2.0 ** -24 * 1.5, 2.0 ** -25], dtype=np.float32)
    # exact ties of the f16 grid: the reference rounds them away from zero
    ties = ((np.arange(1, 65, dtype=np.float32) * 2 + 1) * np.float32(2.0 ** -11)).astype(np.float32)
    rnd = np.concatenate([uniform_pm1(11, 2048, 8.0), uniform_pm1(12, 1024, 1e-4),
                          uniform_pm1(13, 512, 70000.0)])
    f32 = np.concatenate([edge, ties, -ties, rnd]).astype(np.float32)
    fx["conv_f32"] = f32
    fx["conv_f32_to_f16"] = ref.f32_to_f16(f32)
    b = np.concatenate([np.array([0x0000, 0x8000, 0x7f80, 0xff80, 0x7fc1, 0x0001, 0x3800, 0x3880, 0x3870,
                                  0x4780, 0x4770, 0x477f, 0x3f80, 0xbf80], np.uint16),
                        (np.arange(4096, dtype=np.uint32) * 16 + 3).astype(np.uint16)])
    fx["conv_bf16"] = b
    fx["conv_bf16_to_f16"] = np.array([ref.L.bf16_to_f16(int(v)) for v in b], np.uint16)

    # ---- yrng: platform.c:405-417 ----
    import ctypes
    st = ctypes.c_uint64(ref.L.ysrand(0x5EED0001))
    fx["yrng_seed"] = np.array([0x5EED0001], np.uint64)
    fx["yrng_first16"] = np.array([ref.L.yrng(ctypes.byref(st)) for _ in range(16)], np.uint64)

    # ---- softmax / l2norm: matvec.c:1023-1031, 942-949 ----
    sm_in = [np.array([1.0, 2.0, 3.0], np.float32), uniform_pm1(21, 37, 6.0), uniform_pm1(22, 513, 30.0),
             np.array([-1e30, 0.0, 5.0, 5.0], np.float32)]
    for i, v in enumerate(sm_in):
        w = v.copy()
        from oracle_lib import fp
        ref.L.softmax(fp(w), w.size)
        fx[f"softmax{i}_in"] = v
        fx[f"softmax{i}_out"] = w
    for i, v in enumerate([uniform_pm1(31, 128, 0.3), uniform_pm1(32, 64, 1e-7)]):
        w = v.copy()
        ref.L.l2norm_inplace(fp(w), w.size, np.float32(1e-6))
        fx[f"l2norm{i}_in"] = v
        fx[f"l2norm{i}_out"] = w

    # ---- decode: engine.c:1074-1096 ----
    for ci, (name, arch, nh, nkv, hd, pos) in enumerate(DECODE):
        kvd, hidden = nkv * hd, nh * hd
        seeds = np.array([1000 + 10 * ci + j for j in range(5)], np.int64)
        kp, vp = prev_rows(ref, int(seeds[0]), pos, kvd), prev_rows(ref, int(seeds[1]), pos, kvd)
        sc = 1.0 / np.sqrt(hidden)
        q, kr, vr, att = ref.decode(arch, nh, nkv, hd, pos, kp, vp, uniform_pm1(int(seeds[2]), hidden, 2 * sc),
                                    uniform_pm1(int(seeds[3]), kvd, 2 * sc), uniform_pm1(int(seeds[4]), kvd, 2 * sc))
        assert np.array_equal(kr[:pos], kp) and np.array_equal(vr[:pos], vp)
        fx[f"{name}_meta"] = np.array([arch, nh, nkv, hd, pos], np.int64)
        fx[f"{name}_seeds"] = seeds
        fx[f"{name}_q"] = q
        fx[f"{name}_knew"] = kr[pos:]
        fx[f"{name}_vnew"] = vr[pos:]
        fx[f"{name}_att"] = att

    # ---- batched prefill: engine.c:532-563 ----
    for ci, (name, arch, nh, nkv, hd, ps, B) in enumerate(PREFILL):
        kvd, hidden = nkv * hd, nh * hd
        seeds = np.array([2000 + 10 * ci + j for j in range(5)], np.int64)
        kp, vp = prev_rows(ref, int(seeds[0]), ps, kvd), prev_rows(ref, int(seeds[1]), ps, kvd)
        sc = 1.0 / np.sqrt(hidden)
        wq = uniform_pm1(int(seeds[2]), B * hidden, 2 * sc).reshape(B, hidden)
        wk = uniform_pm1(int(seeds[3]), B * kvd, 2 * sc).reshape(B, kvd)
        wv = uniform_pm1(int(seeds[4]), B * kvd, 2 * sc).reshape(B, kvd)
        q, kr, vr, att = ref.prefill(arch, nh, nkv, hd, ps, B, kp, vp, wq, wk, wv)
        fx[f"{name}_meta"] = np.array([arch, nh, nkv, hd, ps, B], np.int64)
        fx[f"{name}_seeds"] = seeds
        fx[f"{name}_q"] = q
        fx[f"{name}_knew"] = kr[ps:]
        fx[f"{name}_vnew"] = vr[ps:]
        fx[f"{name}_att"] = att

    # ---- gated attention: engine.c:935-960 ----
    for ci, (name, nh, nkv, hd, pos) in enumerate(GATED):
        kvd, hidden = nkv * hd, nh * hd
        seeds = np.array([3000 + 10 * ci + j for j in range(6)], np.int64)
        kp, vp = prev_rows(ref, int(seeds[0]), pos, kvd), prev_rows(ref, int(seeds[1]), pos, kvd)
        sc = 1.0 / np.sqrt(hidden)
        q, g, kr, vr, att = ref.gated(nh, nkv, hd, pos, kp, vp, uniform_pm1(int(seeds[2]), hidden, 2 * sc),
                                      uniform_pm1(int(seeds[3]), hidden, 4 * sc),
                                      uniform_pm1(int(seeds[4]), kvd, 2 * sc), uniform_pm1(int(seeds[5]), kvd, 2 * sc))
        fx[f"{name}_meta"] = np.array([nh, nkv, hd, pos], np.int64)
        fx[f"{name}_seeds"] = seeds
        fx[f"{name}_q"] = q
        fx[f"{name}_gate"] = g
        fx[f"{name}_knew"] = kr[pos:]
        fx[f"{name}_vnew"] = vr[pos:]
        fx[f"{name}_att"] = att

    # ---- GDN: engine.c:786-831, matvec.c:975-1004 ----
    for ci, (name, nk, nv, hd) in enumerate(GDN):
        seeds = np.array([4000 + 10 * ci + j for j in range(6)], np.int64)
        conv = 2 * nk * hd + nv * hd
        S = uniform_pm1(int(seeds[0]), nv * hd * hd, 0.2)
        dt = uniform_pm1(int(seeds[1]), nv, 1.0)
        a = -np.exp(uniform_pm1(int(seeds[2]), nv, 1.0)).astype(np.float32)
        r = ref.gdn(nk, nv, hd, uniform_pm1(int(seeds[3]), conv, 0.1), uniform_pm1(int(seeds[4]), nv, 0.1),
                    uniform_pm1(int(seeds[5]), nv, 0.1), dt, a, S)
        fx[f"{name}_meta"] = np.array([nk, nv, hd], np.int64)
        fx[f"{name}_seeds"] = seeds
        for k in ("q", "k", "v", "alpha_raw", "beta_raw", "beta", "gate", "S"):
            fx[f"{name}_{k}"] = r[k]

    # ---- GDN neighbours: conv1d_update matvec.c:956-968, rmsnorm_gated 1007-1021 ----
    dim, kw, T = 96, 4, 7
    seeds = np.array([5001, 5002, 5003], np.int64)
    st0 = uniform_pm1(int(seeds[0]), kw * dim).reshape(kw, dim)
    x = uniform_pm1(int(seeds[1]), T * dim, 2.0).reshape(T, dim)
    w = uniform_pm1(int(seeds[2]), dim * kw, 0.7)
    st, rows = ref.conv(st0, x, w, kw)
    fx["conv1d_meta"] = np.array([dim, kw, T], np.int64)
    fx["conv1d_seeds"] = seeds
    fx["conv1d_state"] = st
    fx["conv1d_rows"] = rows
    n = 128
    seeds = np.array([5011, 5012, 5013], np.int64)
    xx = uniform_pm1(int(seeds[0]), 3 * n).reshape(3, n)
    zz = uniform_pm1(int(seeds[1]), 3 * n, 3.0).reshape(3, n)
    wf = (uniform_pm1(int(seeds[2]), n, 0.5) + np.float32(1.0)).astype(np.float32)
    fx["rmsg_seeds"] = seeds
    fx["rmsg_f32"] = ref.rmsnorm_gated(xx, wf, zz, np.float32(1e-6))
    fx["rmsg_f16"] = ref.rmsnorm_gated(xx, ref.f32_to_f16(wf), zz, np.float32(1e-6))

    # ---- RoPE: rope_inplace / rope_inplace_qwen / rope_inplace_mrope, matvec.c:890-939 ----
    pos = np.array([0, 1, 2, 17, 511, 4095, 32767, 131071], np.int64)
    for ri, (name, kind, d, n_rot, theta) in enumerate(ROPE):
        seed = 6001 + ri
        x = uniform_pm1(seed, len(pos) * 3 * d, 2.0).reshape(len(pos), 3 * d)
        fx[f"{name}_meta"] = np.array([kind, d, n_rot, seed], np.int64)
        fx[f"{name}_theta"] = np.float32([theta])
        fx[f"{name}_pos"] = pos
        fx[f"{name}_out"] = ref.rope(x, pos, d, np.float32(theta), kind, n_rot)

    # ---- o_proj matmul: matmul_f16 / matmul_f32, matvec.c:98-122 (dispatch 785-795) ----
    for name, out, inn, f16, seed in (("mm_f16", 96, 256, True, 7001), ("mm_f32", 40, 128, False, 7002)):
        x = uniform_pm1(seed, 3 * inn, 2.0).reshape(3, inn)
        w = uniform_pm1(seed + 100, out * inn, 0.5).reshape(out, inn)
        if f16:
            w = ref.f32_to_f16(w)
        fx[f"{name}_meta"] = np.array([out, inn, int(f16), seed], np.int64)
        fx[f"{name}_y"] = np.stack([ref.matmul(row, w) for row in x])

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(fx)} arrays)")


if __name__ == "__main__":
    main()
