"""yhip_attn_decode_batch_noalloc against yhip_attn_decode_batch.

The no-allocation entry point runs the same plan and kernels with the split-K
partials in the library's fixed per-device scratch, so its output must equal
the workspace entry point's bit for bit: checked on two calls in a row, the
second with a smaller input (fewer, shorter sequences, gated), whose plan
reuses the scratch the first call left behind.  Shapes whose partials exceed
the scratch are refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle_lib import rel_l2

pytestmark = pytest.mark.gpu


def _call(fn_name, out, q, batch, lens_dev, lens, nh, gate=None, ws=None):
    from yllm_amd._lib import check, lib

    L = lib()
    stream = torch.cuda.current_stream().cuda_stream
    max_len, total = int(max(lens)), int(sum(lens))
    gptr = gate.data_ptr() if gate is not None else None
    gstride = gate.shape[-1] if gate is not None else 0
    common = (out.data_ptr(), out.shape[1], q.data_ptr(), q.shape[1], batch.kptrs.data_ptr(), batch.vptrs.data_ptr(),
              lens_dev.data_ptr(), len(lens), max_len, total, nh, batch.n_kv, batch.head_dim, batch.kv_stride, gptr,
              gstride)
    if fn_name == "yhip_attn_decode_batch":
        check(L.yhip_attn_decode_batch(*common, ws.data_ptr(), ws.numel(), stream))
    else:
        check(L.yhip_attn_decode_batch_noalloc(*common, stream))


def _case(cuda, oracle, seed, lens, nh, nkv, hd, cap, gated):
    from yllm_amd.attention import DecodeBatch, LayerKV, kv_store, round_f16, synth_normal

    kvd = nkv * hd
    caches, data = [], []
    for i, L in enumerate(lens):
        K = round_f16(synth_normal(seed + 2 * i, L * kvd, 0.5)).reshape(L, kvd)
        V = round_f16(synth_normal(seed + 2 * i + 1, L * kvd, 0.5)).reshape(L, kvd)
        c = LayerKV.empty(nkv, hd, cap, device=cuda, zero=False)
        kv_store(c, torch.from_numpy(K).to(cuda), torch.from_numpy(V).to(cuda), 0)
        caches.append(c)
        data.append((K, V))
    q = synth_normal(seed + 999, len(lens) * nh * hd, 0.5).reshape(len(lens), nh * hd)
    gate = synth_normal(seed + 998, len(lens) * nh * hd, 1.0).reshape(len(lens), nh * hd) if gated else None
    return DecodeBatch(caches), data, q, gate


def test_noalloc_decode_matches_workspace_entry_point(cuda, oracle):
    from yllm_amd.attention import decode_workspace_bytes

    nh, nkv, hd, cap = 32, 8, 128, 20480
    first = [20000, 1, 7777, 12345, 300, 19999, 4096, 16384, 9000, 2500, 18000, 640, 11111, 5000, 15000, 20000]
    second = [3000, 129, 2048, 777, 2999]
    for seed, lens, gated in ((0x5EED0103, first, False), (0x5EED0203, second, True)):
        batch, data, q, gate = _case(cuda, oracle, seed, lens, nh, nkv, hd, cap, gated)
        need = decode_workspace_bytes(len(lens), max(lens), sum(lens), nh, nkv, hd)
        assert 0 < need <= 16 << 20
        qt = torch.from_numpy(q).to(cuda)
        gt = torch.from_numpy(gate).to(cuda) if gated else None
        lens_dev = torch.tensor(lens, dtype=torch.int32, device=cuda)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        want = torch.full((len(lens), nh * hd), float("nan"), device=cuda)
        got = torch.full((len(lens), nh * hd), float("nan"), device=cuda)
        _call("yhip_attn_decode_batch", want, qt, batch, lens_dev, lens, nh, gt, ws)
        _call("yhip_attn_decode_batch_noalloc", got, qt, batch, lens_dev, lens, nh, gt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{len(lens)} sequences: outputs differ"
        # and both are the engine's attention (the oracle) for a few sequences
        gn = got.cpu().numpy()
        for i in (0, 1, len(lens) - 1):
            K, V = data[i]
            L = lens[i]
            ref = oracle.decode(q[i], oracle.f32_to_f16(K), oracle.f32_to_f16(V), L - 1, nh, nkv, hd)
            if gated:
                ref = oracle.gate_sigmoid(ref, gate[i])
            assert rel_l2(gn[i], ref) <= 1e-3
        print(f"noalloc decode: {len(lens)} sequences, partials {need} bytes, equal to the workspace entry point")


def test_noalloc_decode_refuses_shapes_beyond_the_scratch(hiplib):
    import ctypes

    from yllm_amd._lib import lib

    P = ctypes.c_void_p(0x1000)  # never dereferenced: the size check fails first
    need = lib().yhip_attn_decode_workspace(64, 32768, 64 * 20000, 16, 2, 256)
    assert need > 16 << 20
    rc = lib().yhip_attn_decode_batch_noalloc(P, 4096, P, 4096, P, P, P, 64, 32768, 64 * 20000, 16, 2, 256, 32768,
                                              None, 0, None)
    assert rc == -28 and "scratch" in lib().yhip_last_error().decode()
