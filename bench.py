#!/usr/bin/env python3
"""Benchmark of the yllm attention hot path on one MI355X (gfx950).

Metric: attention decode GB/s (% of HBM peak) and prefill attention TFLOP/s
(% of bf16/f16 MFMA peak).  One "step" is one pass of the hot path over one
batch of synthetic input, with all inputs resident in HBM:

  prefill2k   (default) causal GQA prefill, 2048 tokens, 28 query / 4 KV
              heads, head_dim 128, f16 Q/K/V drawn N(0,1)*0.5 from seed
              0x5EED0002, f32 output -- one yhip_attn_prefill launch.
  prefill8k   the same at 8192 tokens, 32 / 8 heads.
  decode512   the reference's CPU-runnable decode: 14 query / 2 KV heads,
              head_dim 64, 512 keys, fp32 q (64 rotating layer caches).
  decode32k   one query token per head over a 32768-key cache, 32 / 8 heads,
              head_dim 128 -- one yhip_attn_decode call (split + merge
              kernels).  Steps rotate over 6 layer caches (768 MiB) so the
              256 MB MALL cannot serve repeats.
  decode128k  131072 keys, 32 / 8 heads (config 4), 2 layer caches.
  decode_batch 64 sequences, lengths uniform in [1024, 32768] from seed,
              32 / 8 heads -- one yhip_attn_decode_batch call.
  gdn4k       one Gated DeltaNet layer over a 4096-token prompt, 16 heads,
              d_k = d_v = 128, fp32 (the fifth configuration's GDN layer):
              yhip_gdn_gates + yhip_gdn_chunk from a zero state.
  rope8k      fused RoPE + KV store ahead of attention: 8192 tokens,
              32 / 8 heads of 128 (llama pairs, theta 5e5), f32 q/k/v
              slices of one projection row -> f16 q, f16 K/V cache.
  oproj8k     o_proj after prefill attention: x += W_o . att, 8192 tokens,
              W_o 4096 x 4096 f16, f16 att (the MFMA GEMM, residual fused).
  oproj64     the same for the engine's 64-token prefill chunk, f32 att.
  oproj1      the same for one decode token (the GEMV kernel, HBM-bound).
  kvstore8k   the KV store on its own: 8192 rows of K and V, 8 KV heads of
              128, f32 -> f16 with the reference rounding into the
              head-major cache (K rows, V 32-position tiles).
  gated4k     the qwen35 gated attention prefill of the fifth configuration:
              4096 tokens, 16 / 2 heads, head_dim 256, bf16 queries, f32
              sigmoid gate fused in the epilogue, bf16 out.
  hybrid      the fifth configuration end to end: 3 GDN layers + 1 gated
              attention layer (16 / 2 heads, d 256, bf16), 4096-token
              prefill then 256 decode steps; tokens/s over the whole pass,
              its roofline the sum of the phases' bounds (MFMA for the
              prefill attention and the GDN chunks, HBM for the decode
              steps' KV and recurrent-state traffic).

The default line reports prefill2k as `value`, decode32k and gdn4k under
"secondary".  The CPU baseline is the oracle restatement of the reference's
OpenMP loops (oracle/), timed on this host on a bounded sample, and the same
run checks the GPU output against it (relative L2).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12        # B/s, MI355X HBM3E
MFMA_F16_PEAK = 2.5e15   # FLOP/s, dense f16/bf16 MFMA
MFMA_F32_PEAK = 157.3e12  # FLOP/s, dense fp32 MFMA
METRIC = "attn decode GB/s (% HBM peak); prefill attn TFLOP/s (% MFMA peak)"
SEED = 0x5EED0000
ROTATE_BYTES = 300 << 20  # rotating input sets exceed the 256 MB MALL (Infinity Cache)
# the chain runs two workgroups per 16 state rows when they fit the GPU's 256
# CUs (its state goes out of place)
GDN_CHUNKED_KERNELS = "gdn_prep_kernel<%d> + gdn_chain_kernel<%d, %d>"
EAGER = False  # --eager: launch each step from the host (for counter collection)
CHUNKED_GDN = True  # --gdn-tokenwise: time the token-by-token GDN kernel instead


def synth(seed: int, n: int, first: int = 0) -> np.ndarray:
    from yllm_amd.attention import round_f16, synth_normal

    return round_f16(synth_normal(seed, n, 0.5, first))


def synth_raw(seed: int, n: int, first: int = 0) -> np.ndarray:
    from yllm_amd.attention import synth_normal

    return synth_normal(seed, n, 0.5, first)


def prefill_flops(L: int, nh: int, hd: int, pos_start: int = 0) -> float:
    # QK^T + PV over the causal triangle: 4 * n_q * d * sum_t (keys of token t)
    keys = sum(range(pos_start + 1, pos_start + L + 1))
    return 4.0 * nh * hd * keys


def time_steps(fn, steps: int, warmup: int, out=None, eager: bool = False, graph_per_step: bool = False):
    """Run fn(i) `warmup` times eagerly, capture steps warmup..warmup+steps-1
    in one HIP graph, replay it untimed for ~20 ms of GPU work (the clocks
    ramp up again after the capture) and time one more replay with HIP events
    on the replay stream, so host launch overhead is not part of the
    measurement.  The output of
    the replayed last step is checked bit for bit against the same step run
    eagerly.  With graph_per_step (a step of over a thousand launches whose
    inputs do not depend on i) one step is captured and its graph replayed
    `steps` times, which keeps the graph's size independent of `steps`.
    Returns (ms_per_step, ms per step of the graph's kernels)."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    if graph_per_step and not (EAGER or eager):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn(warmup)
        g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # untimed replays until ~20 ms of GPU work have run, as below
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
        per = start.elapsed_time(end)
        for _ in range(min(50, int(20.0 / max(per, 1e-3)))):
            g.replay()
        start.record()
        for _ in range(steps):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        if out is not None:
            replayed = out.clone()
            fn(warmup)
            torch.cuda.synchronize()
            if not torch.equal(replayed, out):
                raise RuntimeError("graph replay and eager run of the same step differ")
        return ms, ms
    if EAGER or eager:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(warmup + i)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        return ms, ms
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(warmup + i)
    g.replay()  # first replay uploads the graph
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # untimed replays until the GPU has run ~20 ms of this work (at most 50
    # replays): after the capture the clocks ramp up again, and a short timed
    # replay (50 steps of 0.14 ms) measured 6 % slower than a long one
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    per = start.elapsed_time(end)
    for _ in range(min(50, int(20.0 / max(per, 1e-3)))):
        g.replay()
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if out is not None:
        replayed = out.clone()
        fn(warmup + steps - 1)
        torch.cuda.synchronize()
        if not torch.equal(replayed, out):
            raise RuntimeError("graph replay and eager run of the same step differ")
    return ms, ms


def copy_ceiling_gbps() -> float:
    """Measured device-to-device copy bandwidth (read + write bytes), 1 GiB."""
    import torch

    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        b.copy_(a)
    end.record()
    torch.cuda.synchronize()
    gbps = 2.0 * 10 * a.numel() / (start.elapsed_time(end) * 1e-3) / 1e9
    # the two 1 GiB buffers go back to the driver: kept in torch's cache, the
    # next workload's buffers were carved out of them, and the 32k decode that
    # follows in the default run streamed its caches from there 4 % slower
    # (25.2 against 24.3 us) than from caches allocated on their own, as the
    # layer caches of an engine are
    del a, b
    torch.cuda.empty_cache()
    return gbps


# ------------------------------------------------------------------ workloads

def run_prefill(L: int, nh: int, nkv: int, hd: int, cfg: int, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.attention import LayerKV, attn_prefill, kv_store

    dev = torch.device("cuda:0")
    seed = SEED + cfg
    nq, nk = L * nh * hd, L * nkv * hd
    q = torch.from_numpy(synth(seed, nq).reshape(L, nh * hd)).to(dev).half()
    k = torch.from_numpy(synth(seed, nk, nq).reshape(L, nkv * hd)).to(dev).half()
    v = torch.from_numpy(synth(seed, nk, nq + nk).reshape(L, nkv * hd)).to(dev).half()
    # Consecutive steps rotate over copies of (q, cache, out) whose total
    # exceeds the 256 MB MALL, so every step reads its inputs from HBM.
    set_bytes = nq * 2 + 2 * nk * 2 + L * nh * hd * 4
    n_sets = max(1, -(-ROTATE_BYTES // set_bytes))
    qs, caches, outs = [], [], []
    for _ in range(n_sets):
        c = LayerKV.empty(nkv, hd, L, device=dev)
        kv_store(c, k, v, 0)
        qs.append(q.clone())
        caches.append(c)
        outs.append(torch.empty((L, nh * hd), dtype=torch.float32, device=dev))
    del q
    last = (warmup + steps - 1) % n_sets
    ms, kern_ms = time_steps(lambda i: attn_prefill(qs[i % n_sets], caches[i % n_sets], 0, nh, out=outs[i % n_sets]),
                             steps, warmup, outs[last])
    q, out = qs[last], outs[last]
    flops = prefill_flops(L, nh, hd)
    achieved = flops / (kern_ms * 1e-3)
    res = {
        "value": flops / (ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": ms,
        "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"causal GQA prefill attention, {L} tokens, {nh} query / {nkv} KV heads, "
                               f"head_dim {hd}, f16 Q/K/V N(0,1)*0.5 seed {hex(seed)}, f32 out; "
                               f"{n_sets} rotating input sets (> 256 MB MALL)",
                   "tokens": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "mfma", "kernel": "prefill_kernel<%d>" % hd, "achieved": achieved / 1e12,
                     "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s", "frac": achieved / MFMA_F16_PEAK,
                     "flops_per_launch": flops, "launch_ms": kern_ms, "traffic": traffic_of(f"prefill{L}")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_prefill(q, k, v, out, L, nh, nkv, hd)
    return res


def run_prefill_chunked(L: int, nh: int, nkv: int, hd: int, chunk: int, cfg: int, steps: int, warmup: int,
                        cpu: bool):
    """The prompt as the engine issues it: engine_forward_prefill hands the
    block at most 64 tokens per call (pb_cap, engine.c:270-272, 622-653), so
    an L-token prompt is L / chunk attention launches at positions 0, chunk,
    2 chunk, ...; a step is all of them (the K/V rows already stored)."""
    import torch

    from yllm_amd.attention import LayerKV, attn_prefill, kv_store, prefill_workspace, prefill_workspace_bytes

    dev = torch.device("cuda:0")
    seed = SEED + cfg
    nq, nk = L * nh * hd, L * nkv * hd
    q = torch.from_numpy(synth(seed, nq).reshape(L, nh * hd)).to(dev).half()
    k = torch.from_numpy(synth(seed, nk, nq).reshape(L, nkv * hd)).to(dev).half()
    v = torch.from_numpy(synth(seed, nk, nq + nk).reshape(L, nkv * hd)).to(dev).half()
    set_bytes = nq * 2 + 2 * nk * 2 + L * nh * hd * 4
    n_sets = max(1, -(-ROTATE_BYTES // set_bytes))
    qs, caches, outs = [], [], []
    for _ in range(n_sets):
        c = LayerKV.empty(nkv, hd, L, device=dev)
        kv_store(c, k, v, 0)
        qs.append(q.clone())
        caches.append(c)
        outs.append(torch.empty((L, nh * hd), dtype=torch.float32, device=dev))
    del q
    ws = prefill_workspace(prefill_workspace_bytes(chunk, L, nh, nkv, hd), dev)

    def step(i):
        qi, ci, oi = qs[i % n_sets], caches[i % n_sets], outs[i % n_sets]
        for p0 in range(0, L, chunk):
            attn_prefill(qi[p0:p0 + chunk], ci, p0, nh, out=oi[p0:p0 + chunk], workspace=ws)

    last = (warmup + steps - 1) % n_sets
    ms, kern_ms = time_steps(step, steps, warmup, outs[last])
    q, out = qs[last], outs[last]
    flops = prefill_flops(L, nh, hd)
    achieved = flops / (kern_ms * 1e-3)
    res = {
        "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms, "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"causal GQA prefill attention of a {L}-token prompt issued as the engine does, "
                               f"{L // chunk} calls of {chunk} tokens at positions 0, {chunk}, ...; {nh} query / "
                               f"{nkv} KV heads, head_dim {hd}, f16 Q/K/V N(0,1)*0.5 seed {hex(seed)}, f32 out; "
                               f"{n_sets} rotating input sets (> 256 MB MALL)",
                   "tokens": L, "chunk": chunk, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "mfma", "kernel": "prefill_kernel<%d> (+ prefill_merge_kernel<%d>), %d launches"
                     % (hd, hd, L // chunk), "achieved": achieved / 1e12, "peak": MFMA_F16_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": achieved / MFMA_F16_PEAK, "flops_per_launch": flops,
                     "launch_ms": kern_ms, "traffic": traffic_of(f"prefill{L}c{chunk}")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_prefill(q, k, v, out, L, nh, nkv, hd)
    return res


def decode_bytes(L: int, nkv: int, nh: int, hd: int) -> float:
    return float(L) * nkv * hd * 2 * 2 + 2.0 * nh * hd * 4  # K,V once (GQA-aware) + q in + out


def run_decode(L: int, nh: int, nkv: int, hd: int, cfg: int, n_layers: int, steps: int, warmup: int,
               cpu: bool, label: str, q_f32: bool = False):
    import torch

    from yllm_amd.attention import LayerKV, attn_decode, decode_workspace, decode_workspace_bytes, kv_store

    dev = torch.device("cuda:0")
    seed = SEED + cfg
    nk = L * nkv * hd
    k = torch.from_numpy(synth(seed, nk).reshape(L, nkv * hd)).to(dev).half()
    v = torch.from_numpy(synth(seed, nk, nk).reshape(L, nkv * hd)).to(dev).half()
    # q: f16-representable values, or (q_f32) the fp32 draws themselves, which the kernel takes as f16 hi + lo
    q = torch.from_numpy((synth_raw if q_f32 else synth)(seed, nh * hd, 2 * nk)).to(dev)
    caches = []
    for _ in range(n_layers):  # distinct HBM regions with the same contents
        c = LayerKV.empty(nkv, hd, L, device=dev, zero=False)
        kv_store(c, k, v, 0)
        caches.append(c)
    del k, v
    ws = decode_workspace(decode_workspace_bytes(1, L, L, nh, nkv, hd), dev)
    out = torch.empty(nh * hd, dtype=torch.float32, device=dev)
    ms, kern_ms = time_steps(lambda i: attn_decode(q, caches[i % n_layers], L - 1, nh, out=out, workspace=ws),
                             steps, warmup, out)
    nbytes = decode_bytes(L, nkv, nh, hd)
    achieved = nbytes / (kern_ms * 1e-3)
    one = L * hd * 4 <= 160 * 1024  # the library's plan runs such a context unsplit
    res = {
        "value": nbytes / (ms * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": ms,
        "tokens_per_s": 1.0 / (ms * 1e-3),
        "config": {"workload": f"{label}: decode attention, 1 sequence, {L} keys, {nh} query / {nkv} KV heads, "
                               f"head_dim {hd}, f16 KV N(0,1)*0.5 seed {hex(seed)}, "
                               f"{'fp32' if q_f32 else 'f16-valued'} q, "
                               f"{'one split per KV head (K+V <= 160 KiB per head), no merge' if one else 'split-K + LSE merge'}, "
                               f"{n_layers} rotating layer caches",
                   "keys": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "hbm", "kernel": ("decode_split_kernel<%d>" % hd if one else
                                                "decode_split_kernel<%d> + decode_merge_kernel<%d>" % (hd, hd)),
                     "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK, "bytes_per_launch": nbytes, "launch_ms": kern_ms,
                     "traffic": traffic_of(label)},
    }
    if cpu:
        res["cpu_baseline"] = cpu_decode(q, caches[0], out, L, nh, nkv, hd)
    return res


def run_decode_batch(nh: int, nkv: int, hd: int, n_seq: int, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.attention import (DecodeBatch, LayerKV, attn_decode_batch, decode_workspace,
                                    decode_workspace_bytes, kv_store)

    dev = torch.device("cuda:0")
    seed = SEED + 3
    # L_i = 1024 + floor(u * 31745), u from the yrng stream (splitmix64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + np.arange(1, n_seq + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        r = z ^ (z >> np.uint64(31))
    u = ((r >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0
    lens = np.minimum((1024 + np.floor(u * 31745)).astype(np.int64), 32768)
    kvd = nkv * hd
    base_k = torch.from_numpy(synth(seed, 32768 * kvd).reshape(32768, kvd)).to(dev).half()
    base_v = torch.from_numpy(synth(seed, 32768 * kvd, 32768 * kvd).reshape(32768, kvd)).to(dev).half()
    caches = []
    for L in lens:  # one engine-style cache of capacity 32768 per sequence
        c = LayerKV.empty(nkv, hd, 32768, device=dev, zero=False)
        kv_store(c, base_k[: int(L)], base_v[: int(L)], 0)
        caches.append(c)
    batch = DecodeBatch(caches)
    q = torch.from_numpy(synth(seed + 100, n_seq * nh * hd).reshape(n_seq, nh * hd)).to(dev)
    lens_dev = torch.tensor(lens.astype(np.int32), device=dev)
    ws = decode_workspace(decode_workspace_bytes(n_seq, int(lens.max()), int(lens.sum()), nh, nkv, hd), dev)
    out = torch.empty((n_seq, nh * hd), dtype=torch.float32, device=dev)
    ms, kern_ms = time_steps(lambda i: attn_decode_batch(q, batch, lens, nh, out=out, workspace=ws,
                                                         lens_dev=lens_dev), steps, warmup, out)
    nbytes = float(lens.sum()) * kvd * 2 * 2 + 2.0 * n_seq * nh * hd * 4
    achieved = nbytes / (kern_ms * 1e-3)
    res = {
        "value": nbytes / (ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms,
        "tokens_per_s": n_seq / (ms * 1e-3),
        "config": {"workload": f"batched decode, {n_seq} sequences, lengths U[1024,32768] (sum {int(lens.sum())}), "
                               f"{nh} query / {nkv} KV heads, head_dim {hd}, f16 KV",
                   "n_seq": n_seq, "sum_len": int(lens.sum()), "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "hbm", "kernel": "decode_split_kernel<%d> + decode_merge_kernel<%d>" % (hd, hd),
                     "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK, "bytes_per_launch": nbytes, "launch_ms": kern_ms,
                     "traffic": traffic_of("decode_batch")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_decode_batch(q, caches, lens, out, nh, nkv, hd)
    return res


def gdn_bytes(T: int, n_k: int, n_v: int, d: int) -> float:
    # q, k, v in, out, gates and beta in, state read + written (fp32)
    return 4.0 * (T * (2 * n_k * d + 2 * n_v * d + 3 * n_v) + 2 * n_v * d * d)


def gdn_flops(T: int, n_v: int, d: int) -> float:
    return 7.0 * d * d * n_v * T  # decay, two dots, update: the sequential form's count


def run_gdn(T: int, n_h: int, d: int, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.gdn import gdn_chunk, gdn_chunk_workspace_bytes, gdn_gates

    dev = torch.device("cuda:0")
    seed = SEED + 5
    n = T * n_h * d
    q = torch.from_numpy(synth_raw(seed, n).reshape(T, n_h * d)).to(dev)
    k = torch.from_numpy(synth_raw(seed, n, n).reshape(T, n_h * d)).to(dev)
    v = torch.from_numpy(synth_raw(seed, n, 2 * n).reshape(T, n_h * d)).to(dev)
    alpha = torch.from_numpy(synth_raw(seed, T * n_h, 3 * n).reshape(T, n_h)).to(dev)
    beta_raw = torch.from_numpy(synth_raw(seed, T * n_h, 3 * n + T * n_h).reshape(T, n_h)).to(dev)
    dt = torch.zeros(n_h, device=dev)
    a = -torch.ones(n_h, device=dev)
    # the state goes out of place, as the device backend alternates two state
    # buffers: S stays the zero state before the prompt, S2 takes the state
    # after it
    S = torch.zeros((n_h, d, d), device=dev)
    S2 = torch.empty_like(S)
    beta = torch.empty_like(beta_raw)
    gate = torch.empty_like(alpha)
    ws = torch.empty(max(gdn_chunk_workspace_bytes(T, n_h, d) // 4, 1), device=dev)
    # rotating copies of the inputs and output beyond the 256 MB MALL
    set_bytes = 4 * (4 * n + 2 * T * n_h)
    n_sets = max(1, -(-ROTATE_BYTES // set_bytes))
    sets = [(q.clone(), k.clone(), v.clone(), alpha.clone(), beta_raw.clone(), torch.empty((T, n_h * d), device=dev))
            for _ in range(n_sets)]

    def step(i):
        qi, ki, vi, ai, bi, oi = sets[i % n_sets]
        beta.copy_(bi)
        gdn_gates(ai, beta, dt, a, gate=gate)
        gdn_chunk(S, qi, ki, vi, gate, beta, n_h, out=oi, workspace=ws, chunked=CHUNKED_GDN, S_out=S2)

    ms, kern_ms = time_steps(step, steps, warmup, sets[(warmup + steps - 1) % n_sets][5])
    out = sets[(warmup + steps - 1) % n_sets][5]
    nbytes, flops = gdn_bytes(T, n_h, n_h, d), gdn_flops(T, n_h, d)
    # the arithmetic is fp32 (the reference's type): bound by the fp32 MFMA
    # peak or by HBM, whichever takes longer
    t_mfma, t_hbm = flops / MFMA_F32_PEAK, nbytes / HBM_PEAK
    t_roof = max(t_mfma, t_hbm)
    kern_s = kern_ms * 1e-3
    res = {
        "value": T / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3),
        "config": {"workload": f"Gated DeltaNet layer prefill, {T} tokens, {n_h} heads, d_k = d_v = {d}, fp32, "
                               f"q/k/v/alpha/beta N(0,1)*0.5 seed {hex(seed)}, dt_bias 0, ssm_a -1, "
                               f"gates + l2norm + recurrence ({'chunked' if CHUNKED_GDN else 'token by token'}); "
                               f"{n_sets} rotating input sets (> 256 MB MALL)",
                   "tokens": T, "heads": n_h, "head_dim": d},
        "roofline": {"bound": "mfma" if t_mfma >= t_hbm else "hbm",
                     "kernel": (GDN_CHUNKED_KERNELS % (d, d, 2 if 2 * n_h * d // 16 <= 256 else 1) if CHUNKED_GDN else
                                "gdn_kernel<%d>" % d) + " (+ gdn_gates_kernel)",
                     **({"achieved": flops / kern_s / 1e12, "peak": MFMA_F32_PEAK / 1e12, "unit": "TFLOP/s"}
                        if t_mfma >= t_hbm else
                        {"achieved": nbytes / kern_s / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s"}),
                     "frac": t_roof / kern_s, "bytes_per_launch": nbytes, "flops_per_launch": flops,
                     "launch_ms": kern_ms, "traffic": traffic_of(f"gdn{T}"),
                     "note": "fp32 arithmetic: frac = max(bytes / 8 TB/s, flops / 157.3 TFLOP/s fp32 MFMA) / "
                             "measured time; flops are the sequential form's 7*d^2 per head and token"},
        "gflops": flops / (ms * 1e-3) / 1e9,
    }
    if cpu:
        res["cpu_baseline"] = cpu_gdn(q, k, v, alpha, beta_raw, out, T, n_h, d)
    return res


def rope_bytes(L: int, nh: int, nkv: int, hd: int) -> float:
    """Algorithmic HBM bytes of one fused RoPE + KV store over L tokens: read
    q, k, v (f32), write q (f16) and the K and V cache rows (f16)."""
    return float(L) * hd * ((4 + 2) * nh + 2 * (4 + 2) * nkv)


def run_rope(L: int, nh: int, nkv: int, hd: int, theta: float, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.attention import ROPE_PAIRS, LayerKV, rope_kv_store

    dev = torch.device("cuda:0")
    seed = SEED + 6
    qd, kvd = nh * hd, nkv * hd
    width = qd + 2 * kvd
    x = torch.from_numpy(synth_raw(seed, L * width).reshape(L, width)).to(dev)
    # rotating copies of (projection rows, q out, cache) beyond the 256 MB MALL
    set_bytes = rope_bytes(L, nh, nkv, hd)
    n_sets = max(1, int(-(-ROTATE_BYTES // set_bytes)))
    sets = [(x.clone(), torch.empty((L, qd), dtype=torch.float16, device=dev),
             LayerKV.empty(nkv, hd, L, device=dev)) for _ in range(n_sets)]
    del x

    def step(i):
        xi, qo, c = sets[i % n_sets]
        rope_kv_store(c, xi[:, :qd], xi[:, qd:qd + kvd], xi[:, qd + kvd:], 0, nh, ROPE_PAIRS, theta, q_out=qo)

    last = sets[(warmup + steps - 1) % n_sets]
    ms, kern_ms = time_steps(step, steps, warmup, last[1])
    nbytes = rope_bytes(L, nh, nkv, hd)
    achieved = nbytes / (kern_ms * 1e-3)
    res = {
        "value": L / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"fused RoPE (llama pairs, theta {theta:g}) + KV store, {L} tokens at positions "
                               f"0..{L - 1}, {nh} query / {nkv} KV heads, head_dim {hd}; f32 q/k/v slices of one "
                               f"projection row N(0,1) seed {hex(seed)}, f16 q out, f16 K/V cache; "
                               f"{n_sets} rotating input sets (> 256 MB MALL)",
                   "tokens": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "hbm", "kernel": "rope_kv_kernel<%d,%d>" % (ROPE_PAIRS, hd), "achieved": achieved / 1e9,
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": achieved / HBM_PEAK,
                     "bytes_per_launch": nbytes, "launch_ms": kern_ms, "traffic": traffic_of(f"rope{L}")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_rope(last, L, nh, nkv, hd, theta)
    return res


def kvstore_bytes(L: int, nkv: int, hd: int) -> float:
    return float(L) * nkv * hd * 2 * (4 + 2)  # K and V: f32 read, f16 written


def run_kvstore(L: int, nkv: int, hd: int, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.attention import LayerKV, kv_store

    dev = torch.device("cuda:0")
    seed = SEED + 7
    kvd = nkv * hd
    k = torch.from_numpy(synth_raw(seed, L * kvd).reshape(L, kvd)).to(dev)
    v = torch.from_numpy(synth_raw(seed, L * kvd, L * kvd).reshape(L, kvd)).to(dev)
    # rotating copies of (k, v rows, cache) beyond the 256 MB MALL
    n_sets = max(1, int(-(-ROTATE_BYTES // kvstore_bytes(L, nkv, hd))))
    sets = [(k.clone(), v.clone(), LayerKV.empty(nkv, hd, L, device=dev, zero=False)) for _ in range(n_sets)]
    del k, v

    def step(i):
        ki, vi, c = sets[i % n_sets]
        kv_store(c, ki, vi, 0)

    last = sets[(warmup + steps - 1) % n_sets]
    ms, kern_ms = time_steps(step, steps, warmup, last[2].k)
    nbytes = kvstore_bytes(L, nkv, hd)
    achieved = nbytes / (kern_ms * 1e-3)
    res = {
        "value": achieved / 1e9, "unit": "GB/s", "ms_per_step": ms, "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"KV store: {L} rows at positions 0..{L - 1}, {nkv} KV heads, head_dim {hd}; "
                               f"f32 K/V rows N(0,1) seed {hex(seed)} -> f16 (the reference's round-half-up) "
                               f"into the head-major cache; {n_sets} rotating input sets (> 256 MB MALL)",
                   "tokens": L, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "hbm", "kernel": "kv_block_kernel", "achieved": achieved / 1e9,
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": achieved / HBM_PEAK,
                     "bytes_per_launch": nbytes, "launch_ms": kern_ms, "traffic": traffic_of(f"kvstore{L}")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_kvstore(last, L, nkv, hd)
    return res


def run_gated_prefill(L: int, nh: int, nkv: int, hd: int, steps: int, warmup: int, cpu: bool):
    import torch

    from yllm_amd.attention import LayerKV, attn_prefill, kv_store

    dev = torch.device("cuda:0")
    seed = SEED + 5
    nq, nk = L * nh * hd, L * nkv * hd
    q = torch.from_numpy(synth(seed, nq).reshape(L, nh * hd)).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(synth(seed, nk, nq).reshape(L, nkv * hd)).to(dev).half()
    v = torch.from_numpy(synth(seed, nk, nq + nk).reshape(L, nkv * hd)).to(dev).half()
    gate = torch.from_numpy(synth_raw(seed, nq, nq + 2 * nk).reshape(L, nh * hd)).to(dev)
    set_bytes = nq * 2 + 2 * nk * 2 + nq * 4 + nq * 2
    n_sets = max(1, -(-ROTATE_BYTES // set_bytes))
    sets = []
    for _ in range(n_sets):
        c = LayerKV.empty(nkv, hd, L, device=dev)
        kv_store(c, k, v, 0)
        sets.append((q.clone(), c, gate.clone(), torch.empty((L, nh * hd), dtype=torch.bfloat16, device=dev)))
    del q, gate

    def step(i):
        qi, c, gi, oi = sets[i % n_sets]
        attn_prefill(qi, c, 0, nh, gate=gi, out=oi)

    last = sets[(warmup + steps - 1) % n_sets]
    ms, kern_ms = time_steps(step, steps, warmup, last[3])
    flops = prefill_flops(L, nh, hd)
    achieved = flops / (kern_ms * 1e-3)
    res = {
        "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms, "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"qwen35 gated attention prefill: causal GQA over {L} tokens, {nh} query / {nkv} KV "
                               f"heads, head_dim {hd}; bf16 queries, f16 K/V, f32 sigmoid gate fused in the "
                               f"epilogue, bf16 out; N(0,1)*0.5 seed {hex(seed)}; {n_sets} rotating input sets "
                               f"(> 256 MB MALL)",
                   "tokens": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd},
        "roofline": {"bound": "mfma", "kernel": "prefill_kernel<%d>" % hd, "achieved": achieved / 1e12,
                     "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s", "frac": achieved / MFMA_F16_PEAK,
                     "flops_per_launch": flops, "launch_ms": kern_ms, "traffic": traffic_of(f"gated{L}")},
    }
    if cpu:
        res["cpu_baseline"] = cpu_gated_prefill(last, k, v, L, nh, nkv, hd)
    return res


def run_oproj(B: int, hidden: int, qdim: int, steps: int, warmup: int, cpu: bool):
    """o_proj x += W_o . att over B tokens, f16 weights; att f32 for one
    decode token (the engine's att_out), f16 for a prefill batch (the prefill
    kernel's f16 output)."""
    import torch

    from yllm_amd.attention import o_proj, o_proj_workspace_bytes

    dev = torch.device("cuda:0")
    seed = SEED + 7
    w = (torch.from_numpy(synth_raw(seed, hidden * qdim).reshape(hidden, qdim)).to(dev) / np.sqrt(qdim)).half()
    att = torch.from_numpy(synth_raw(seed, B * qdim, hidden * qdim).reshape(B, qdim)).to(dev) * 0.5
    gemv = B <= 8
    if B > 64:  # a prefill-sized batch: the attention kernel's f16 output
        att = att.half()
    x = torch.from_numpy(synth_raw(seed, B * hidden, hidden * qdim + B * qdim).reshape(B, hidden)).to(dev)
    # rotating (weights, att, x) sets beyond the 256 MB MALL
    att_dt, att_size = att.dtype, att.element_size()
    set_bytes = hidden * qdim * 2 + B * (qdim * att_size + hidden * 4)
    n_sets = max(1, int(-(-ROTATE_BYTES // set_bytes)))
    sets = [(w.clone(), att.clone(), x.clone()) for _ in range(n_sets)]
    x_ref = x.clone()
    del w, att, x
    ws = torch.empty(max(o_proj_workspace_bytes(B, hidden, qdim, torch.float16, att_dt), 256), dtype=torch.uint8,
                     device=dev)

    def step(i):
        wi, ai, xi = sets[i % n_sets]
        o_proj(xi, ai, wi, workspace=ws)

    last = sets[(warmup + steps - 1) % n_sets]
    # x accumulates from step to step, so no replay-vs-eager output check
    ms, kern_ms = time_steps(step, steps, warmup, None)
    flops = 2.0 * B * hidden * qdim
    nbytes = hidden * qdim * 2.0 + B * qdim * att_size + 2.0 * B * hidden * 4.0
    if gemv:
        roof = {"bound": "hbm", "kernel": "oproj_gemv_kernel<1,%d>" % (1 if B == 1 else 8),
                "achieved": nbytes / (kern_ms * 1e-3) / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": nbytes / (kern_ms * 1e-3) / HBM_PEAK, "bytes_per_launch": nbytes, "launch_ms": kern_ms,
                "traffic": traffic_of(f"oproj{B}")}
        value, unit = nbytes / (ms * 1e-3) / 1e9, "GB/s"
    else:
        roof = {"bound": "mfma", "kernel": ("oproj_gemm_kernel<%d,%d>" % ((2, 4) if B > 128 else (1, 1))) +
                ("" if att_dt == torch.float16 else " (+ oproj_split_kernel)"),
                "achieved": flops / (kern_ms * 1e-3) / 1e12, "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": flops / (kern_ms * 1e-3) / MFMA_F16_PEAK, "flops_per_launch": flops, "launch_ms": kern_ms,
                "traffic": traffic_of(f"oproj{B}")}
        value, unit = flops / (ms * 1e-3) / 1e12, "TFLOP/s"
    res = {
        "value": value, "unit": unit, "ms_per_step": ms, "tokens_per_s": B / (ms * 1e-3),
        "config": {"workload": f"o_proj x += W_o . att, {B} token(s), W_o {hidden} x {qdim} f16, "
                               f"{'f32' if att_dt == torch.float32 else 'f16'} att, f32 residual, N(0,1) seed {hex(seed)}; "
                               f"{n_sets} rotating sets (> 256 MB MALL)",
                   "tokens": B, "hidden": hidden, "qdim": qdim},
        "roofline": roof,
    }
    if cpu:
        res["cpu_baseline"] = cpu_oproj(last, x_ref, B, hidden, qdim)
    return res


def hybrid_phase_bounds(T, n_dec, n_gdn, hg, dg, kw, nh, nkv, da) -> dict:
    """Seconds each phase of the hybrid group takes at its roofline:
    prefill attention at the f16 MFMA peak (causal FLOPs); each GDN layer's
    chunked prefill at max(its algorithmic bytes at HBM peak, the
    sequential form's flops at the fp32 MFMA peak); the prefill's conv,
    gated norm and RoPE + KV store as HBM bytes; every decode token's
    gated-attention KV read (keys 0..t, K and V once), its q / gate / out
    and new K/V row, and per GDN layer the state read and written once plus
    its conv delay line and token rows, at HBM peak."""
    conv = 3 * hg * dg
    pre_attn = prefill_flops(T, nh, da) / MFMA_F16_PEAK
    gdn_chunk = n_gdn * max(gdn_bytes(T, hg, hg, dg) / HBM_PEAK, gdn_flops(T, hg, dg) / MFMA_F32_PEAK)
    # conv: rows in, rows out, delay line; gated norm: x, z in, y out; RoPE + store: q/k/v rows in, bf16 q, K/V out
    pre_io = (n_gdn * (T * conv * 4 * 2 + T * hg * dg * 4 * 3)
              + T * (nh * da * (4 + 2) + nkv * da * 2 * (4 + 2))) / HBM_PEAK
    dec = 0.0
    for t in range(T, T + n_dec):
        keys = t + 1
        dec += keys * nkv * da * 2 * 2 + nh * da * 4 * 3 + nkv * da * 2 * (4 + 2)
        dec += n_gdn * (hg * dg * dg * 4 * 2 + kw * conv * 4 * 2 + conv * 4 + hg * dg * 4 * 3)
    return {"prefill_attention": pre_attn, "prefill_gdn_chunks": gdn_chunk, "prefill_conv_norm_rope": pre_io,
            "decode_tokens": dec / HBM_PEAK}


def run_hybrid(steps: int, warmup: int, cpu: bool, n_dec: int = 256):
    """The fifth configuration: one group of 3 Gated-DeltaNet layers and 1
    gated GQA attention layer, a 4096-token prefill then n_dec decode steps.
    A GDN layer's GPU part is conv1d + silu over its qkv rows, the gates, the
    l2norm + recurrence, and the gated RMSNorm (the projections are not on
    this path)."""
    import torch

    from yllm_amd.attention import (ROPE_MROPE, LayerKV, attn_decode_rope, attn_prefill, decode_workspace,
                                    decode_workspace_bytes, rope_kv_store)
    from yllm_amd.gdn import gdn_chunk, gdn_chunk_workspace_bytes, gdn_conv, gdn_decode, gdn_gated_norm, gdn_gates

    dev = torch.device("cuda:0")
    seed = SEED + 5
    T, n_gdn, hg, dg, kw = 4096, 3, 16, 128, 4   # GDN: 16 heads, d_k = d_v = 128, conv width 4
    nh, nkv, da = 16, 2, 256                     # gated attention: 16 / 2 heads, d = 256
    L = T + n_dec
    kd, conv = hg * dg, 3 * hg * dg              # q, k: kd channels each; v: hg*dg
    first = [0]

    def draw(n, bf16=False, scale=None):
        x = synth_raw(seed, n, first[0])
        first[0] += n
        t = torch.from_numpy(x).to(dev)
        if scale is not None:
            t = t * scale
        return t.to(torch.bfloat16) if bf16 else t

    gd = [dict(qkv=draw(L * conv).view(L, conv), z=draw(L * hg * dg).view(L, -1),
               alpha=draw(L * hg).view(L, hg), beta_raw=draw(L * hg).view(L, hg),
               conv_w=draw(conv * kw, scale=0.5).view(conv, kw), norm_w=draw(dg, scale=0.1) + 1.0)
          for _ in range(n_gdn)]
    qd, kvd = nh * da, nkv * da
    at = dict(qkv=draw(L * (qd + 2 * kvd)).view(L, -1), gate=draw(L * qd).view(L, -1))
    dt = torch.zeros(hg, device=dev)
    a = -torch.ones(hg, device=dev)
    S = [torch.zeros((hg, dg, dg), device=dev) for _ in range(n_gdn)]
    S2 = [torch.zeros((hg, dg, dg), device=dev) for _ in range(n_gdn)]  # prefill and decode alternate S, S2
    cst = [torch.zeros((kw, conv), device=dev) for _ in range(n_gdn)]
    cst2 = [torch.zeros((kw, conv), device=dev) for _ in range(n_gdn)]
    beta = [torch.empty((L, hg), device=dev) for _ in range(n_gdn)]
    gate = [torch.empty((L, hg), device=dev) for _ in range(n_gdn)]
    xc = torch.empty((L, conv), device=dev)           # conv + silu rows: q | k | v
    gout = torch.empty((L, hg * dg), device=dev)
    ws = torch.empty(gdn_chunk_workspace_bytes(T, hg, dg) // 4, device=dev)
    cache = LayerKV.empty(nkv, da, L, device=dev)
    aout = torch.empty((L, nh * da), dtype=torch.bfloat16, device=dev)
    dout = torch.empty(nh * da, device=dev)
    dws = decode_workspace(decode_workspace_bytes(1, L, L, nh, nkv, da), dev)
    q_pre = torch.empty((T, qd), dtype=torch.bfloat16, device=dev)  # rotated prefill queries
    qkv = at["qkv"]

    def rope_store(t0, t1, q_out):
        rope_kv_store(cache, qkv[t0:t1, :qd], qkv[t0:t1, qd:qd + kvd], qkv[t0:t1, qd + kvd:], t0, nh, ROPE_MROPE,
                      1e7, n_rot=64, q_out=q_out)

    def gdn_layer_prefill(li):
        # the delay line and the state out of place (cst -> cst2, S -> S2),
        # as the device backend keeps them: the conv in one launch, where in
        # place takes a second for the line, and the chained recurrence on
        # two workgroups per state slice
        g = gd[li]
        gdn_conv(g["qkv"][:T], cst[li], g["conv_w"], out=xc[:T], state_out=cst2[li])
        gdn_chunk(S[li], xc[:T, :kd], xc[:T, kd:2 * kd], xc[:T, 2 * kd:], gate[li][:T], beta[li][:T], hg,
                  out=gout[:T], workspace=ws, S_out=S2[li])
        gdn_gated_norm(gout[:T], g["z"][:T], g["norm_w"], hg, out=gout[:T])

    def gdn_layer_step(li, t):
        # one launch per layer and token; the state and the delay line
        # alternate between two buffers each, as the device backend keeps
        # them (the prefill left the delay line in cst2 and the state in S2)
        g = gd[li]
        even = (t - T) % 2 == 0
        c_in, c_out = (cst2[li], cst[li]) if even else (cst[li], cst2[li])
        s_in, s_out = (S2[li], S[li]) if even else (S[li], S2[li])
        gdn_decode(s_in, c_in, c_out, g["qkv"][t], g["z"][t], g["alpha"][t], g["beta_raw"][t], g["conv_w"], dt, a,
                   g["norm_w"], hg, y=gout[t], S_out=s_out)

    def step(i):
        for li in range(n_gdn):
            S[li].zero_()
            cst[li].zero_()
            beta[li][:T].copy_(gd[li]["beta_raw"][:T])
            gdn_gates(gd[li]["alpha"][:T], beta[li][:T], dt, a, gate=gate[li][:T])
        # prefill
        for li in range(n_gdn):
            gdn_layer_prefill(li)
        rope_store(0, T, q_pre)
        attn_prefill(q_pre, cache, 0, nh, gate=at["gate"][:T], out=aout[:T])
        # decode
        for t in range(T, L):
            for li in range(n_gdn):
                gdn_layer_step(li, t)
            # RoPE + KV store of the token fused into the split-K decode
            attn_decode_rope(qkv[t, :qd], qkv[t, qd:qd + kvd], qkv[t, qd + kvd:], cache, t, nh, ROPE_MROPE, 1e7,
                             n_rot=64, gate=at["gate"][t], out=dout, workspace=dws)

    # one step is ~1300 launches: its graph is captured once and replayed
    ms, _ = time_steps(step, steps, warmup, dout, graph_per_step=True)
    phases = hybrid_phase_bounds(T, n_dec, n_gdn, hg, dg, kw, nh, nkv, da)
    ideal_ms = sum(phases.values()) * 1e3
    res = {
        "value": L / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "tokens_per_s": L / (ms * 1e-3),
        "config": {"workload": f"qwen35 hybrid group: {n_gdn} Gated-DeltaNet layers ({hg} heads, d {dg}, fp32: "
                               f"conv1d width {kw} + silu, gates, l2norm + recurrence, gated RMSNorm) + "
                               f"1 gated attention layer ({nh}/{nkv} heads, d {da}: M-RoPE over 64 dims + KV "
                               f"store from fp32 q/k/v rows, bf16 prefill queries, sigmoid gate); "
                               f"{T}-token prefill (chunked GDN, MFMA attention) then {n_dec} decode steps "
                               f"(fused GDN token per layer, one launch; RoPE + KV store fused into the split-K decode) per step; N(0,1)*0.5 seed "
                               f"{hex(seed)}",
                   "prefill_tokens": T, "decode_steps": n_dec},
        # no single kernel bounds the group: the roofline is the sum of its
        # phases' bounds, as a step rate (achieved / peak = ideal / measured)
        "roofline": {"bound": "mfma+hbm (sum of phase bounds)",
                     "kernel": "decode phase: gdn_decode_head_kernel<%d> x %d + decode_split_kernel<%d, ROPE> + "
                               "decode_merge_kernel<%d> per token" % (dg, n_gdn, da, da),
                     "achieved": 1e3 / ms, "peak": 1e3 / ideal_ms, "unit": "steps/s", "frac": ideal_ms / ms,
                     "ideal_ms": ideal_ms, "phase_bound_us": {k2: v2 * 1e6 for k2, v2 in phases.items()},
                     "launch_ms": ms, "traffic": None},
    }
    if cpu:
        torch.cuda.synchronize()
        li = n_gdn - 1  # the shared output rows hold the last GDN layer's results
        res["cpu_baseline"] = cpu_hybrid(
            {k2: v2.cpu().numpy() for k2, v2 in gd[li].items()}, (S2 if n_dec % 2 == 0 else S)[li].cpu().numpy(),
            gout.cpu().numpy(),
            qkv.cpu().numpy(), at["gate"].cpu().numpy(), aout.float().cpu().numpy(), dout.cpu().numpy(),
            T, n_dec, n_gdn, hg, dg, kw, nh, nkv, da)
    return res


# ---------------------------------------------------------------- CPU leg

def _oracle():
    sys.path.insert(0, str(ROOT / "oracle"))
    from oracle_lib import Oracle

    return Oracle()


def _host_desc(O) -> tuple[int, str]:
    cores = int(O.L.yo_threads())
    model = "unknown CPU"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return cores, model


def cpu_prefill(q, k, v, out, L, nh, nkv, hd):
    """The CPU oracle (OpenMP over heads, as the reference): the whole
    workload up to 2048 tokens; beyond, the last 64 query rows (the longest
    key ranges, ~10 s of the whole 8k pass's ~40 s would be too long for the
    default run), FLOP/s from the sample's own causal work."""
    O = _oracle()
    from oracle_lib import rel_l2

    p0 = 0 if L <= 2048 else L - 64
    qn = q[p0:].float().cpu().numpy()
    kc = O.f32_to_f16(k.float().cpu().numpy())
    vc = O.f32_to_f16(v.float().cpu().numpy())
    t0 = time.perf_counter()
    want = O.prefill(qn, kc, vc, p0, L - p0, nh, nkv, hd)
    dt = time.perf_counter() - t0
    cores, model = _host_desc(O)
    what = (f"the whole workload ({L} tokens, all heads)" if p0 == 0 else
            f"query rows {p0}..{L - 1} (the last {L - p0}, all heads, keys 0..row)")
    return {"value": prefill_flops(L - p0, nh, hd, p0) / dt / 1e12, "unit": "TFLOP/s", "cores": cores,
            "kind": "port", "sample": f"{what}, one pass, {dt:.2f} s; effective parallelism <= {nh} heads; {model}",
            "seconds": dt, "parity_rel_l2": rel_l2(out[p0:].cpu().numpy(), want)}


def cpu_kvstore(kv_set, L, nkv, hd):
    """The reference's store is the scalar f32_to_f16 per element
    (engine.c:1068-1072, platform.c:340-379); the oracle's restatement runs
    over all rows until ~2 s of CPU work.  The GPU cache's K rows and V tiles
    are compared bit for bit with it."""
    O = _oracle()
    torch = sys.modules["torch"]
    k, v, cache = kv_set
    kn, vn = k.cpu().numpy(), v.cpu().numpy()
    t0 = time.perf_counter()
    n = 0
    while True:
        kc = O.f32_to_f16(kn)
        vc = O.f32_to_f16(vn)
        n += 1
        dt = time.perf_counter() - t0
        if dt > 2.0:
            break
    torch.cuda.synchronize()
    kvd = nkv * hd
    gk = cache.k.view(torch.int16).cpu().numpy().view(np.uint16)[:, :L, :].transpose(1, 0, 2).reshape(L, kvd)
    gv = (cache.v.view(torch.int16).cpu().numpy().view(np.uint16)  # [nkv][L/32][hd][32]
          .transpose(1, 3, 0, 2).reshape(-1, nkv, hd)[:L].reshape(L, kvd))
    same = bool(np.array_equal(gk, kc.reshape(L, kvd)) and np.array_equal(gv, vc.reshape(L, kvd)))
    cores, model = _host_desc(O)
    return {"value": kvstore_bytes(L, nkv, hd) * n / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the whole workload ({L} rows, K and V), {n} passes, {dt:.2f} s, single thread as the "
                      f"reference's loop; {model}", "seconds": dt, "parity_bit_exact": same}


def cpu_gated_prefill(gset, k, v, L, nh, nkv, hd):
    """The oracle (OpenMP over heads, as the reference) on the last 64 query
    rows (the longest key ranges), the sigmoid gate applied as engine.c:959-960;
    FLOP/s from the sample's own causal work."""
    O = _oracle()
    from oracle_lib import rel_l2

    torch = sys.modules["torch"]
    q, _, gate, out = gset
    S = 64
    p0 = L - S
    qn = q[p0:].float().cpu().numpy()
    kc = O.f32_to_f16(k.float().cpu().numpy())
    vc = O.f32_to_f16(v.float().cpu().numpy())
    t0 = time.perf_counter()
    want = O.prefill(qn, kc, vc, p0, S, nh, nkv, hd)
    want = O.gate_sigmoid(want.ravel(), gate[p0:].cpu().numpy().ravel())
    dt = time.perf_counter() - t0
    torch.cuda.synchronize()
    got = out[p0:].float().cpu().numpy().ravel()
    from yllm_amd.attention import round_bf16

    cores, model = _host_desc(O)
    flops = prefill_flops(S, nh, hd, p0)
    # the output is bf16: against the f32 oracle the error includes bf16's own
    # rounding (2^-9 relative); against the oracle rounded to bf16 it is the
    # kernel's
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"query rows {p0}..{L - 1} (the last {S}, all heads, keys 0..row), one pass, {dt:.2f} s; "
                      f"effective parallelism <= {nh} heads; {model}",
            "seconds": dt, "parity_rel_l2": rel_l2(got, want),
            "parity_rel_l2_vs_bf16_rounded": rel_l2(got, round_bf16(np.array(want, np.float32, copy=True)))}


def cpu_rope(rope_set, L, nh, nkv, hd, theta):
    """The oracle's per-token loop (the reference's engine.c:1054-1072 is
    single-threaded) over a sample of tokens spread over the positions; the
    same rows of the GPU's q and caches are checked against it."""
    O = _oracle()
    x, qo, cache = rope_set
    qd, kvd = nh * hd, nkv * hd
    rows = np.unique(np.linspace(0, L - 1, min(L, 2048)).astype(np.int64))
    xs = x[rows].cpu().numpy()
    t0 = time.perf_counter()
    n = 0
    while True:  # whole passes over the sample until ~2 s of CPU work
        for r, row in zip(rows, xs):
            q, kc, vc = O.rope_kv_store(row[None, :qd], row[None, qd:qd + kvd], row[None, qd + kvd:], int(r), nh,
                                        nkv, hd, np.float32(theta), 1)
        n += len(rows)
        dt = time.perf_counter() - t0
        if dt > 2.0:
            break
    # parity of the sampled rows (the last pass left the last row's results; redo the sample for the check)
    qs, ks, vs = [], [], []
    for r, row in zip(rows, xs):
        q, kc, vc = O.rope_kv_store(row[None, :qd], row[None, qd:qd + kvd], row[None, qd + kvd:], int(r), nh,
                                    nkv, hd, np.float32(theta), 1)
        qs.append(q[0])
        ks.append(kc[0])
        vs.append(vc[0])
    torch = sys.modules["torch"]
    torch.cuda.synchronize()
    got_q = qo[rows].float().cpu().numpy()
    want_q = np.float16(np.stack(qs)).astype(np.float32)
    K = cache.k.view(torch.int16).cpu().numpy().view(np.uint16)[:, rows, :].transpose(1, 0, 2).reshape(len(rows), kvd)
    k_equal = float((K == np.stack(ks)).mean())
    cores = 1
    _, model = _host_desc(O)
    return {"value": n / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{len(rows)} tokens spread over positions 0..{L - 1}, passes until 2 s "
                      f"({n} tokens in {dt:.2f} s), one thread (the reference loop is serial); {model}",
            "seconds": dt, "q_max_abs_err_f16": float(np.abs(got_q - want_q).max()),
            "k_bits_equal_frac": k_equal}


def cpu_oproj(oproj_set, x_before, B, hidden, qdim):
    """The oracle's matmul_f16 rows (the reference runs them with OpenMP over
    output rows) on a sample of tokens; those rows of the GPU result are
    checked against it.  x_before is the set's residual before the timed
    steps; the GPU applied o_proj to it (warmup + steps) / n_sets times, so
    the check uses one fresh GPU call on a copy."""
    import torch

    from yllm_amd.attention import o_proj

    O = _oracle()
    from oracle_lib import rel_l2

    w, att, _ = oproj_set
    rows = np.unique(np.linspace(0, B - 1, min(B, 8)).astype(np.int64))
    xg = x_before.clone()
    o_proj(xg, att, w)
    torch.cuda.synchronize()
    wn = w.view(torch.int16).cpu().numpy().view(np.uint16)
    an = att[rows].float().cpu().numpy()
    xn = x_before[rows].cpu().numpy()
    t0 = time.perf_counter()
    n = 0
    while True:
        want = O.o_proj(xn, an, wn)
        n += len(rows)
        dt = time.perf_counter() - t0
        if dt > 2.0:
            break
    _, model = _host_desc(O)
    return {"value": n / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{len(rows)} tokens, passes until 2 s ({n} tokens in {dt:.2f} s), one thread; {model}",
            "seconds": dt, "parity_rel_l2": rel_l2(xg[rows].cpu().numpy(), want)}


def cpu_gdn(q, k, v, alpha, beta_raw, out, T, n_h, d):
    """The oracle's single-threaded recurrence (the reference's gdn_state_update
    has no OpenMP) over the whole sequence."""
    O = _oracle()
    from oracle_lib import rel_l2

    qn, kn, vn = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    al, br = alpha.cpu().numpy(), beta_raw.cpu().numpy()
    t0 = time.perf_counter()
    beta = np.empty_like(br)
    gate = np.empty_like(al)
    zeros, ones = np.zeros(n_h, np.float32), -np.ones(n_h, np.float32)
    for t in range(T):
        beta[t], gate[t] = O.gdn_gates(al[t], br[t], zeros, ones)
    S = np.zeros(n_h * d * d, np.float32)
    _, want, _, _ = O.gdn_sequence(S, qn, kn, vn, gate, beta, T, n_h, d, n_h, d, 1e-6)
    dt = time.perf_counter() - t0
    _, model = _host_desc(O)
    return {"value": T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"the whole workload ({T} tokens, {n_h} heads), one pass, {dt:.2f} s, single thread as "
                      f"the reference; {model}",
            "seconds": dt, "parity_rel_l2": rel_l2(out.cpu().numpy(), want)}


def cpu_decode(q, cache, out, L, nh, nkv, hd):
    from yllm_amd.attention import kv_to_engine

    O = _oracle()
    from oracle_lib import rel_l2

    ek, ev = kv_to_engine(cache, L)
    kc = ek.view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    vc = ev.view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    qn = q.cpu().numpy()
    reps, t0 = 0, time.perf_counter()
    while True:
        want = O.decode(qn, kc, vc, L - 1, nh, nkv, hd)
        reps += 1
        dt = time.perf_counter() - t0
        if dt > 3.0 or (reps >= 20 and dt > 0.5):
            break
    cores, model = _host_desc(O)
    per = dt / reps
    return {"value": decode_bytes(L, nkv, nh, hd) / per / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{reps} decode step(s) of the same workload, {per:.3f} s each; {model}",
            "seconds": dt, "parity_rel_l2": rel_l2(out.cpu().numpy(), want)}


def cpu_hybrid(g, S_gpu, gout, qkv, gate, aout, dout, T, n_dec, n_gdn, hg, dg, kw, nh, nkv, da):
    """The oracle's restatement of the qwen35 group, token by token as the
    reference runs it (engine.c:723-734 batch -> per token; 786-847 GDN;
    910-960 gated attention), on a bounded sample:
      - one GDN layer over all T + n_dec tokens (conv + silu, gates, l2norm
        + state update, gated RMSNorm; single thread, as gdn_state_update);
        the group has n_gdn such layers, counted n_gdn times;
      - the attention layer's RoPE + KV store of every row, the prefill's
        last 64 query rows (scaled to the whole causal prefill by FLOPs) and
        the last 16 decode steps (scaled to n_dec).
    Parity: that GDN layer's prefill and decode output rows and final state,
    the sampled prefill rows (bf16 output) and the last decode step."""
    O = _oracle()
    from oracle_lib import rel_l2
    from yllm_amd.attention import round_bf16

    L = T + n_dec
    conv = 3 * hg * dg
    kd = hg * dg
    eps = np.float32(1e-6)
    dt0, a0 = np.zeros(hg, np.float32), -np.ones(hg, np.float32)
    # GDN layer, token by token
    t0 = time.perf_counter()
    st = np.zeros((kw, conv), np.float32)
    Sc = np.zeros(hg * dg * dg, np.float32)
    ys = np.empty((L, kd), np.float32)
    for t in range(L):
        st, rows = O.conv_silu(st, g["qkv"][t][None], g["conv_w"], kw)
        beta, gt = O.gdn_gates(g["alpha"][t], g["beta_raw"][t], dt0, a0)
        r = rows[0]
        Sc, o, _, _ = O.gdn_sequence(Sc, r[:kd], r[kd:2 * kd], r[2 * kd:], gt, beta, 1, hg, dg, hg, dg, eps)
        ys[t] = O.rmsnorm_gated(o.reshape(hg, dg), g["norm_w"], g["z"][t].reshape(hg, dg), eps).ravel()
    t_gdn = time.perf_counter() - t0
    # attention: RoPE + store of every row (one pass), then the samples
    qd, kvd = nh * da, nkv * da
    t0 = time.perf_counter()
    q_rot, kc, vc = O.rope_kv_store(qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], 0, nh, nkv, da,
                                    np.float32(1e7), 3, 64)
    t_rope = time.perf_counter() - t0
    S_pre = 64
    p0 = T - S_pre
    q_bf = round_bf16(np.ascontiguousarray(q_rot[p0:T], np.float32).copy())
    t0 = time.perf_counter()
    want_pre = O.prefill(q_bf, kc, vc, p0, S_pre, nh, nkv, da)
    want_pre = O.gate_sigmoid(want_pre.ravel(), gate[p0:T].ravel()).reshape(S_pre, qd)
    t_pre = (time.perf_counter() - t0) * prefill_flops(T, nh, da) / prefill_flops(S_pre, nh, da, p0)
    n_s = 16
    t0 = time.perf_counter()
    for t in range(L - n_s, L):
        want_dec = O.gate_sigmoid(O.decode(q_rot[t], kc[:t + 1], vc[:t + 1], t, nh, nkv, da).ravel(), gate[t])
    t_dec = (time.perf_counter() - t0) * n_dec / n_s
    total = n_gdn * t_gdn + t_rope + t_pre + t_dec
    cores, model = _host_desc(O)
    err_gdn = max(rel_l2(gout[:T], ys[:T]), max(rel_l2(gout[t], ys[t]) for t in range(T, L)))
    return {"value": L / total, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"one GDN layer over all {L} tokens ({t_gdn:.2f} s, single thread, counted {n_gdn}x), the "
                      f"attention layer's RoPE + store of {L} rows ({t_rope:.2f} s), its last {S_pre} prefill rows "
                      f"(scaled by FLOPs to {t_pre:.2f} s) and last {n_s} decode steps (scaled to {n_dec}: "
                      f"{t_dec:.2f} s); OpenMP over heads for attention as the reference; {model}",
            "seconds": total, "parity_rel_l2": max(err_gdn, rel_l2(aout[p0:T], want_pre), rel_l2(dout, want_dec)),
            "parity_detail": {"gdn_out": err_gdn, "gdn_state": rel_l2(S_gpu.ravel(), Sc),
                              "attn_prefill_rows_bf16": rel_l2(aout[p0:T], want_pre),
                              "attn_last_decode": rel_l2(dout, want_dec)}}


def cpu_decode_batch(q, caches, lens, out, nh, nkv, hd):
    """The oracle's decode (the reference runs one engine per sequence,
    OpenMP over heads) on four of the batch's sequences: the shortest, the
    longest and two between; GB/s from their KV bytes, parity per sequence."""
    from yllm_amd.attention import kv_to_engine

    O = _oracle()
    from oracle_lib import rel_l2

    torch = sys.modules["torch"]
    order = np.argsort(lens)
    pick = [int(order[0]), int(order[len(order) // 3]), int(order[2 * len(order) // 3]), int(order[-1])]
    qn, got = q.cpu().numpy(), out.cpu().numpy()
    errs, secs, nbytes = [], 0.0, 0.0
    for i in pick:
        L = int(lens[i])
        ek, ev = kv_to_engine(caches[i], L)
        kc = ek.view(torch.int16).cpu().numpy().view(np.uint16)
        vc = ev.view(torch.int16).cpu().numpy().view(np.uint16)
        t0 = time.perf_counter()
        want = O.decode(qn[i], kc, vc, L - 1, nh, nkv, hd)
        secs += time.perf_counter() - t0
        nbytes += decode_bytes(L, nkv, nh, hd)
        errs.append(rel_l2(got[i], want))
    cores, model = _host_desc(O)
    return {"value": nbytes / secs / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"sequences {pick} ({', '.join(str(int(lens[i])) for i in pick)} keys), one decode step "
                      f"each, {secs:.2f} s; {model}",
            "seconds": secs, "parity_rel_l2": max(errs)}


# -------------------------------------------------------------- traffic

def traffic_of(label: str):
    """HBM bytes per launch of the workload's kernels, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (each scaled by what the counter
    reads for a 1 GiB copy kernel); None when that workload was not counted."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        entry = json.loads(p.read_text()).get(label)
        return None if entry is None else float(entry["bytes"])
    except (OSError, ValueError, KeyError, TypeError):
        return None


# the other configurations' lines in the default run, with their own step counts
SECONDARY = ["decode32k", "prefill8k", "prefill2k_chunked", "decode128k", "decode_batch", "gated4k", "gdn4k", "hybrid",
             "decode512"]
SECONDARY_STEPS = {"decode32k": (200, 20), "prefill8k": (20, 3), "prefill2k_chunked": (30, 3), "decode128k": (50, 5),
                   "decode_batch": (20, 3), "gated4k": (40, 4), "gdn4k": (50, 5), "hybrid": (3, 1),
                   "decode512": (200, 20)}
SECONDARY_METRIC = {"decode32k": "attn decode GB/s", "decode512": "attn decode GB/s", "prefill8k": "prefill attn TFLOP/s",
                    "prefill2k_chunked": "prefill attn TFLOP/s",
                    "decode128k": "attn decode GB/s", "decode_batch": "attn decode GB/s",
                    "gated4k": "prefill attn TFLOP/s", "gdn4k": "GDN prefill tokens/s", "hybrid": "hybrid tokens/s"}
DTYPES = {"gdn4k": "f32 state, gates and accumulation; chunk products in split bf16 (hi*hi + hi*lo + lo*hi on bf16 "
                   "MFMA), the -W operand rounded to bf16, Gram products on f32 MFMA",
          "decode512": "f32 q (f16 hi + lo), f16 K/V MFMA, f32 accumulate/softmax",
          "rope8k": "f32 rotation, f16 stores", "oproj8k": "f16 MFMA, f32 accumulate",
          "oproj1": "f16 weights, f32 activations and accumulate", "kvstore8k": "f32 -> f16 (reference rounding)",
          "gated4k": "bf16 q, f16 K/V MFMA, f32 accumulate/softmax, bf16 out",
          "hybrid": "GDN f32 state and accumulation (chunk products in split bf16); bf16/f16 MFMA attention, "
                    "f32 accumulate"}


def timing_of(w: str, steps: int) -> str:
    how = ("K eager launches" if EAGER else
           "one step captured in a HIP graph, replayed untimed for ~20 ms of GPU work, then replayed K times"
           if w == "hybrid" else
           "K steps captured in one HIP graph; after the W eager warm-up steps the graph is replayed untimed for "
           "~20 ms of GPU work (at most 50 replays) so the clocks are back at steady state after the capture, "
           "then one replay of the K steps is timed")
    return how + ", timed with HIP events on the launch stream"


def run_workload(w: str, steps: int, warmup: int, cpu: bool):
    if w == "prefill2k":
        return run_prefill(2048, 28, 4, 128, 2, steps, warmup, cpu)
    if w == "prefill8k":
        return run_prefill(8192, 32, 8, 128, 4, steps, warmup, cpu)
    if w == "prefill2k_chunked":
        return run_prefill_chunked(2048, 28, 4, 128, 64, 2, steps, warmup, cpu)
    if w == "prefill8k_chunked":
        return run_prefill_chunked(8192, 32, 8, 128, 64, 4, steps, warmup, cpu)
    if w == "decode512":  # the reference's CPU-runnable case: 14 / 2 heads, d 64, 512 keys, fp32 q
        return run_decode(512, 14, 2, 64, 1, 64, steps, warmup, cpu, "decode512", q_f32=True)
    if w == "decode32k":
        return run_decode(32768, 32, 8, 128, 4, 6, steps, warmup, cpu, "decode32k")
    if w == "decode128k":
        return run_decode(131072, 32, 8, 128, 4, 2, steps, warmup, cpu, "decode128k")
    if w == "decode4k_d256":  # the hybrid group's gated-attention decode step at the end of its 256 steps
        return run_decode(4352, 16, 2, 256, 5, 64, steps, warmup, cpu, "decode4k_d256")
    if w == "decode_batch":
        return run_decode_batch(32, 8, 128, 64, steps, warmup, cpu)
    if w == "gdn4k":
        return run_gdn(4096, 16, 128, steps, warmup, cpu)
    if w == "rope8k":
        return run_rope(8192, 32, 8, 128, 500000.0, steps, warmup, cpu)
    if w == "oproj8k":
        return run_oproj(8192, 4096, 4096, steps, warmup, cpu)
    if w == "oproj1":
        return run_oproj(1, 4096, 4096, steps, warmup, cpu)
    if w == "oproj64":
        return run_oproj(64, 4096, 4096, steps, warmup, cpu)
    if w == "kvstore8k":
        return run_kvstore(8192, 8, 128, steps, warmup, cpu)
    if w == "gated4k":
        return run_gated_prefill(4096, 16, 2, 256, steps, warmup, cpu)
    if w == "hybrid":
        return run_hybrid(steps, warmup, cpu)
    raise ValueError(w)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="prefill2k",
                    choices=["prefill2k", "prefill8k", "prefill2k_chunked", "prefill8k_chunked", "decode512", "decode32k",
                             "decode4k_d256", "decode128k", "decode_batch", "gdn4k", "rope8k", "oproj8k", "oproj64",
                             "oproj1", "kvstore8k", "gated4k", "hybrid"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other configurations' secondary lines (" + ", ".join(SECONDARY) + ")")
    ap.add_argument("--gdn-tokenwise", action="store_true",
                    help="gdn4k: time the token-by-token recurrence instead of the chunked form")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step from the host instead of replaying a HIP graph (profiling)")
    args = ap.parse_args()
    global EAGER, CHUNKED_GDN
    EAGER = args.eager
    CHUNKED_GDN = not args.gdn_tokenwise

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): the attention "
              "path is built and measured per GPU; multi-GPU sharding is a design note, not a run.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    from yllm_amd import lib

    lib()  # fails loudly when the HIP library is missing
    cpu = not args.no_cpu
    w = args.workload
    t0 = time.perf_counter()
    res = run_workload(w, args.steps, args.warmup, cpu)
    print(f"bench: {w} {res['value']:.4g} {res['unit']} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr,
          flush=True)
    line = {"metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": DTYPES.get(w, "f16 MFMA, f32 accumulate/softmax"), "data": "synthetic",
            "config": res["config"], "tokens_per_s": res["tokens_per_s"], "roofline": res["roofline"],
            "timing": timing_of(w, args.steps), "measured_copy_GBps": copy_ceiling_gbps()}
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
    if w == "prefill2k" and not args.no_secondary:
        sec = []
        for name in SECONDARY:
            steps, warmup = SECONDARY_STEPS.get(name, (args.steps, args.warmup))
            # each line allocates as it would in a process of its own, not out
            # of the blocks the previous line left in torch's cache
            torch.cuda.empty_cache()
            t0 = time.perf_counter()
            r = run_workload(name, steps, warmup, cpu)
            print(f"bench: {name} {r['value']:.4g} {r['unit']} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr,
                  flush=True)
            sec.append({"workload": name, "metric": SECONDARY_METRIC[name],
                        "dtype": DTYPES.get(name, "f16 MFMA, f32 accumulate/softmax"), "steps": steps,
                        "warmup": warmup, "timing": timing_of(name, steps), **r})
        line["secondary"] = sec
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
