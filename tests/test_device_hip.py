"""The HIP device backend inside the reference engine (end to end).

The engine is the reference's own C (inference/core, device_cpu.c) compiled
from its sources with yllm_amd/device/device_hip.c and a driver
(oracle/e2e_driver.c) into oracle/_ref/libyref_e2e.so.  A synthetic model
(llama, qwen with q/k/v biases, or the qwen35 hybrid of Gated-DeltaNet and
gated attention layers) is written with the reference's LLF writer
(llf_emit, convert.c:31).
Each case runs the same prompt (batched prefill, engine.c:590-709) and greedy
decode steps (engine_forward, engine.c:1248) on the engine bound to the CPU
device and bound to the HIP backend, and compares logits (max relative L2
<= 1e-3 per step) and the chosen tokens (identical).  The backend's failure
path (-1, CPU recompute, CPU for the rest) must give the CPU result.
"""
from __future__ import annotations

import ctypes
import re
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_uint32
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
E2E_LIB = ROOT / "oracle" / "_ref" / "libyref_e2e.so"
HEADER = ROOT / "include" / "yllm_device_hip.h"
TOL = 1e-3


@pytest.fixture(scope="module")
def e2e():
    if not E2E_LIB.exists():
        pytest.skip("oracle/_ref/libyref_e2e.so is not built (needs the reference sources: make -C oracle e2e)")
    lib = ctypes.CDLL(str(E2E_LIB))
    lib.ye_make_model.restype = c_int
    lib.ye_make_model.argtypes = [c_char_p] + [c_uint32] * 9 + [c_char_p, c_size_t]
    lib.ye_make_model_q35.restype = c_int
    lib.ye_make_model_q35.argtypes = [c_char_p] + [c_uint32] * 12 + [c_char_p, c_size_t]
    lib.ye_resume.restype = c_int
    lib.ye_resume.argtypes = [c_char_p, c_int, c_int, POINTER(c_uint32), c_int, c_int, c_int, c_char_p,
                              POINTER(c_float), POINTER(c_uint32), POINTER(c_int), c_char_p, c_size_t]
    lib.device_hip_fail_mode.restype = None
    lib.ye_run.restype = c_int
    lib.ye_run.argtypes = [c_char_p, c_int, c_int, c_int, c_int, POINTER(c_uint32), c_int, c_int, POINTER(c_float),
                           POINTER(c_uint32), POINTER(c_int), POINTER(c_float), c_size_t, c_char_p, c_size_t]
    return lib


ARCH_LLAMA, ARCH_QWEN = 0, 1  # llf.h:22-23


def make_model(lib, path, blocks, hidden, heads, kv_heads, vocab=512, seq=256, seed=7, arch=ARCH_LLAMA, ffn=0):
    err = ctypes.create_string_buffer(256)
    rc = lib.ye_make_model(str(path).encode(), arch, blocks, hidden, heads, kv_heads, vocab, seq, seed, ffn, err,
                           256)
    assert rc == 0, err.value.decode()
    return path


def make_q35(lib, path, blocks, hidden, heads, kv_heads, head_dim, n_k, n_v, hvd, vocab=512, seq=256, seed=11,
             ffn=0):
    """Block b is gated attention when b % 4 == 0, a GDN layer otherwise."""
    err = ctypes.create_string_buffer(256)
    rc = lib.ye_make_model_q35(str(path).encode(), blocks, hidden, heads, kv_heads, head_dim, n_k, n_v, hvd, vocab,
                               seq, seed, ffn, err, 256)
    assert rc == 0, err.value.decode()
    return path


FAIL_BEFORE, FAIL_AFTER, FAIL_LOST = 0, 1, 2  # device_hip_fail_mode


def run(lib, path, prompt, n_decode, use_hip, fail_after=-1, vocab=512, fail_mode=FAIL_BEFORE, gdn_cap=0):
    """logits [(n_decode+1), vocab], tokens, status [bind, KV rows differing, GDN floats], message; with
    gdn_cap > 0 also the engine's GDN delay lines then states at the end (status[2] floats)."""
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    logits = np.zeros((n_decode + 1, vocab), dtype=np.float32)
    tokens = np.zeros(max(n_decode, 1), dtype=np.uint32)
    status = np.zeros(3, dtype=np.int32)
    gdn = np.zeros(max(gdn_cap, 1), dtype=np.float32)
    err = ctypes.create_string_buffer(256)
    rc = lib.ye_run(str(path).encode(), int(use_hip), 0, fail_after, fail_mode,
                    prompt.ctypes.data_as(POINTER(c_uint32)), len(prompt), n_decode,
                    logits.ctypes.data_as(POINTER(c_float)), tokens.ctypes.data_as(POINTER(c_uint32)),
                    status.ctypes.data_as(POINTER(c_int)), gdn.ctypes.data_as(POINTER(c_float)) if gdn_cap else None,
                    gdn_cap, err, 256)
    assert rc == 0, err.value.decode()
    if gdn_cap:
        return logits, tokens[:n_decode], status, err.value.decode(), gdn[: status[2]]
    return logits, tokens[:n_decode], status, err.value.decode()


def resume(lib, path, prompt, n_before, n_after, use_hip, sess_path, vocab=512):
    """Save after n_before decode steps (sess_kv_save), resume in a fresh
    engine (sess_kv_load [+ device_hip_kv_from_host]) for n_after steps."""
    prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
    logits = np.zeros((n_after, vocab), dtype=np.float32)
    tokens = np.zeros(n_before + n_after, dtype=np.uint32)
    status = np.zeros(2, dtype=np.int32)
    err = ctypes.create_string_buffer(256)
    rc = lib.ye_resume(str(path).encode(), int(use_hip), 0, prompt.ctypes.data_as(POINTER(c_uint32)), len(prompt),
                       n_before, n_after, str(sess_path).encode(), logits.ctypes.data_as(POINTER(c_float)),
                       tokens.ctypes.data_as(POINTER(c_uint32)), status.ctypes.data_as(POINTER(c_int)), err, 256)
    assert rc == 0, err.value.decode()
    return logits, tokens, status, err.value.decode()


def read_session(path):
    """A YLLMSKV01 file (cache.c:174-196): 8 magic bytes, n_blocks, kv_dim,
    max_seq, pos (u32), then per layer 1..n_blocks K rows 0..pos-1 and V rows
    0..pos-1 (f16 bits)."""
    raw = Path(path).read_bytes()
    assert raw[:8] == b"YLLMSKV0"
    nb, kvd, max_seq, pos = np.frombuffer(raw[8:24], dtype=np.uint32)
    rows = np.frombuffer(raw[24:], dtype=np.uint16)
    assert rows.size == nb * 2 * pos * kvd
    return (int(nb), int(kvd), int(max_seq), int(pos)), rows.reshape(nb, 2, pos, kvd)


def rel_l2(a, b):
    return float(np.linalg.norm((a - b).ravel()) / max(np.linalg.norm(b.ravel()), 1e-30))


def prompt_of(n, vocab=512, seed=3):
    return np.random.default_rng(seed).integers(1, vocab, size=n, dtype=np.uint32)


# ------------------------------------------------------------------ CPU only

def test_session_resume_on_the_cpu_engine_is_exact(e2e, tmp_path):
    """The driver's save / resume on the CPU engine continues exactly as an
    uninterrupted run (the file holds every KV row the decode reads)."""
    path = make_model(e2e, tmp_path / "m.llf", 2, 512, 8, 2)
    prompt = prompt_of(37)
    nb, na = 3, 4
    want, wt, _, _ = run(e2e, path, prompt, nb + na, use_hip=False)
    got, gt, status, _ = resume(e2e, path, prompt, nb, na, False, tmp_path / "s.kv")
    assert status[1] == len(prompt) + nb
    assert np.array_equal(gt, wt)
    assert np.array_equal(got.view(np.uint32), want[nb + 1:].view(np.uint32))
    (n_blocks, kvd, max_seq, pos), rows = read_session(tmp_path / "s.kv")
    assert (n_blocks, kvd, pos) == (2, 128, len(prompt) + nb)


def test_plugin_exports_every_declared_symbol(e2e):
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"\b(device_\w+)\s*\(", text)
    assert set(names) == {"device_create_hip", "device_hip_kv_from_host", "device_hip_kv_to_host",
                          "device_hip_fail_after", "device_hip_fail_mode"}
    for n in names:
        assert hasattr(e2e, n), n


def test_bind_without_usable_gpu_falls_back_to_cpu(e2e, tmp_path):
    """With no gfx950 device the factory fails with a message, the CPU device
    is bound again and the outputs are the CPU engine's, bit for bit."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU tests cover the bound backend")
    path = make_model(e2e, tmp_path / "m.llf", 2, 256, 4, 2)
    prompt = prompt_of(20)
    want, wt, _, _ = run(e2e, path, prompt, 3, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, 3, use_hip=True)
    assert status[0] == -1 and msg.startswith("hip:"), (status, msg)
    assert np.array_equal(got, want) and np.array_equal(gt, wt)


def test_qwen35_model_runs_on_the_cpu_engine(e2e, tmp_path):
    """The synthetic qwen35 model is one the reference engine runs: batched
    prefill (chunks of >= 16 tokens: smaller ones take the engine's
    per-token DEV_MODE_CPU branch, which calls the llama block) and decode
    through fwd_block_qwen35.  Without a GPU the HIP bind falls back and
    gives the same bits."""
    import torch

    path = make_q35(e2e, tmp_path / "q.llf", 4, 256, 4, 2, 256, 2, 4, 64)
    prompt = prompt_of(40)
    want, wt, _, _ = run(e2e, path, prompt, 3, use_hip=False)
    assert np.isfinite(want).all() and np.std(want[-1]) > 0.1
    if torch.cuda.is_available():
        return
    got, gt, status, msg = run(e2e, path, prompt, 3, use_hip=True)
    assert status[0] == -1 and msg.startswith("hip:"), (status, msg)
    assert np.array_equal(got, want) and np.array_equal(gt, wt)


# ------------------------------------------------------------------------ GPU

@pytest.mark.gpu
@pytest.mark.parametrize("arch,hidden,heads,kv_heads,n_prompt", [
    (ARCH_LLAMA, 512, 8, 2, 83),    # head_dim 64, GQA 4:1; prefill chunks 64 + 19, both batched
    (ARCH_LLAMA, 1024, 8, 2, 70),   # head_dim 128; chunk 64 batched, the 6-token tail on the CPU
    (ARCH_QWEN, 512, 4, 4, 40),     # head_dim 128, no GQA, qwen RoPE and q/k/v biases
    (ARCH_LLAMA, 1024, 4, 1, 33),   # head_dim 256, GQA 4:1
])
def test_engine_end_to_end_matches_cpu(e2e, cuda, tmp_path, arch, hidden, heads, kv_heads, n_prompt):
    path = make_model(e2e, tmp_path / "m.llf", 2, hidden, heads, kv_heads, arch=arch)
    prompt = prompt_of(n_prompt)
    n_dec = 8
    want, wt, _, _ = run(e2e, path, prompt, n_dec, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, n_dec, use_hip=True)
    assert status[0] == 0, msg
    errs = [rel_l2(got[i], want[i]) for i in range(n_dec + 1)]
    print(f"e2e hidden={hidden} heads={heads}/{kv_heads} prompt={n_prompt}: max rel_l2 {max(errs):.3e}, "
          f"tokens {gt.tolist()}")
    assert max(errs) <= TOL
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1))
    assert np.array_equal(gt, wt)
    # the HBM cache holds exactly the engine's KV rows
    assert status[1] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("hidden,heads,kv_heads,max_seq,n_prompt,n_dec", [
    # the second configuration's head shape (28 / 4, head_dim 128) with a
    # prompt of several of the engine's 64-token prefill chunks
    (3584, 28, 4, 1024, 600, 6),
    # a decode workspace sized for max_seq 4352 at 8 kv heads serves the
    # shorter positions too (4352 keys split 17 ways, 2241 keys 18 ways);
    # a short workspace would make the backend fall back to the CPU, and
    # device_hip_kv_to_host at the end of the run would then fail
    (2048, 16, 8, 4352, 2240, 4),
])
def test_engine_end_to_end_real_head_shapes(e2e, cuda, tmp_path, hidden, heads, kv_heads, max_seq, n_prompt, n_dec):
    path = make_model(e2e, tmp_path / "m.llf", 1, hidden, heads, kv_heads, seq=max_seq, ffn=64)
    prompt = prompt_of(n_prompt)
    want, wt, _, _ = run(e2e, path, prompt, n_dec, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, n_dec, use_hip=True)
    assert status[0] == 0, msg
    errs = [rel_l2(got[i], want[i]) for i in range(n_dec + 1)]
    print(f"e2e {heads}/{kv_heads} d={hidden // heads} prompt {n_prompt} max_seq {max_seq}: max rel_l2 "
          f"{max(errs):.3e}, tokens {gt.tolist()}")
    assert max(errs) <= TOL
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1))
    assert np.array_equal(gt, wt)
    assert status[1] == 0  # still bound at the end: the HBM cache equals the host KV


@pytest.mark.gpu
def test_engine_failure_hook_first_call_gives_cpu_result(e2e, cuda, tmp_path):
    path = make_model(e2e, tmp_path / "m.llf", 2, 512, 8, 2)
    prompt = prompt_of(40)
    want, wt, _, _ = run(e2e, path, prompt, 4, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, 4, use_hip=True, fail_after=0)
    assert status[0] == 0, msg
    assert np.array_equal(got, want) and np.array_equal(gt, wt)


@pytest.mark.gpu
def test_engine_failure_hook_mid_run_stays_within_tolerance(e2e, cuda, tmp_path):
    """GPU for the prefill and two decode blocks, then the CPU: the CPU path
    reads the host KV that the backend mirrored."""
    path = make_model(e2e, tmp_path / "m.llf", 2, 512, 8, 2)
    prompt = prompt_of(40)
    want, wt, _, _ = run(e2e, path, prompt, 6, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, 6, use_hip=True, fail_after=4)
    assert status[0] == 0, msg
    assert max(rel_l2(got[i], want[i]) for i in range(7)) <= TOL
    assert np.array_equal(gt, wt)


Q35_CASES = [
    # blocks, hidden, heads, kv, head_dim, n_k, n_v, hvd, prompt
    (4, 256, 4, 2, 256, 2, 4, 64, 83),     # d 256 gated attention; GDN d 64; prefill 64 (chunked) + 19
    (8, 512, 8, 2, 128, 4, 8, 128, 40),    # two groups; GDN d 128, 8 v heads on 4 k heads
]


@pytest.mark.gpu
@pytest.mark.parametrize("blocks,hidden,heads,kv_heads,head_dim,n_k,n_v,hvd,n_prompt", Q35_CASES)
def test_qwen35_end_to_end_matches_cpu(e2e, cuda, tmp_path, blocks, hidden, heads, kv_heads, head_dim, n_k, n_v,
                                       hvd, n_prompt):
    """qwen35 hybrid blocks on the backend: GDN state in HBM (chunked prefill,
    one-token steps), gated attention with the fused gate, against the
    engine's own fwd_block_qwen35 on the CPU."""
    path = make_q35(e2e, tmp_path / "q.llf", blocks, hidden, heads, kv_heads, head_dim, n_k, n_v, hvd)
    prompt = prompt_of(n_prompt)
    n_dec = 8
    want, wt, _, _ = run(e2e, path, prompt, n_dec, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, n_dec, use_hip=True)
    assert status[0] == 0, msg
    errs = [rel_l2(got[i], want[i]) for i in range(n_dec + 1)]
    print(f"e2e qwen35 blocks={blocks} hidden={hidden} attn {heads}/{kv_heads}x{head_dim} gdn {n_k}/{n_v}x{hvd} "
          f"prompt={n_prompt}: max rel_l2 {max(errs):.3e}, tokens {gt.tolist()}")
    assert max(errs) <= TOL
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1))
    assert np.array_equal(gt, wt)
    assert status[1] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("fail_after,fail_mode", [
    (0, FAIL_BEFORE),   # every block on the CPU
    (5, FAIL_BEFORE),   # prefill (4 blocks) and one decode block on the GPU, then the CPU
    # after the kernels ran: the prefill's second GDN layer (its state and delay line were
    # sent up from the host), the first decode token's second GDN layer (state in HBM only,
    # the fused one-launch token) and its attention layer
    (1, FAIL_AFTER),
    (5, FAIL_AFTER),
    (7, FAIL_AFTER),
])
def test_qwen35_failure_hook(e2e, cuda, tmp_path, fail_after, fail_mode):
    """The CPU continues from the GDN state and KV the backend holds: after a
    failed block the HBM state is the one from before that block (the block
    wrote the other buffer of the pair), so the CPU recompute applies the
    block's tokens once."""
    path = make_q35(e2e, tmp_path / "q.llf", 4, 256, 4, 2, 256, 2, 4, 64)
    prompt = prompt_of(40)
    want, wt, _, _ = run(e2e, path, prompt, 4, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, 4, use_hip=True, fail_after=fail_after, fail_mode=fail_mode)
    assert status[0] == 0, msg
    if fail_after == 0:
        assert np.array_equal(got, want) and np.array_equal(gt, wt)
    else:
        errs = [rel_l2(got[i], want[i]) for i in range(5)]
        print(f"qwen35 fail_after={fail_after} mode={fail_mode}: max rel_l2 {max(errs):.3e}")
        assert max(errs) <= TOL
        assert np.array_equal(gt, wt)


@pytest.mark.gpu
def test_qwen35_lost_state_is_reported(e2e, cuda, tmp_path, capfd):
    """A device that fails and then cannot give the HBM-resident GDN state
    back: the block must not continue on the stale host state.  The failing
    block (the first decode token's second GDN layer) reports the loss and
    every later logit is NaN, while the prefill's logits are the CPU's."""
    path = make_q35(e2e, tmp_path / "q.llf", 4, 256, 4, 2, 256, 2, 4, 64)
    prompt = prompt_of(40)
    want, _, _, _ = run(e2e, path, prompt, 3, use_hip=False)
    got, _, status, msg = run(e2e, path, prompt, 3, use_hip=True, fail_after=5, fail_mode=FAIL_LOST)
    assert status[0] == 0, msg
    assert rel_l2(got[0], want[0]) <= TOL
    assert np.isnan(got[1:]).all()
    assert "recurrent state of layer 2 is lost" in capfd.readouterr().err


@pytest.mark.gpu
@pytest.mark.parametrize("fail_after", [1, 3])
def test_engine_failure_after_launch_gives_cpu_result(e2e, cuda, tmp_path, fail_after):
    """llama blocks failing after their kernels ran (the prefill's second
    block, a decode block): the CPU recompute from the host KV is exact for
    that block and the run stays within the tolerance."""
    path = make_model(e2e, tmp_path / "m.llf", 2, 512, 8, 2)
    prompt = prompt_of(40)
    want, wt, _, _ = run(e2e, path, prompt, 4, use_hip=False)
    got, gt, status, msg = run(e2e, path, prompt, 4, use_hip=True, fail_after=fail_after, fail_mode=FAIL_AFTER)
    assert status[0] == 0, msg
    assert max(rel_l2(got[i], want[i]) for i in range(5)) <= TOL
    assert np.array_equal(gt, wt)


@pytest.mark.gpu
def test_qwen35_end_to_end_fifth_config_shapes(e2e, cuda, tmp_path):
    """The hybrid group at its real head shapes through the engine: three
    GDN layers of 16 heads (d_k = d_v = 128, conv width 4) and a gated
    attention layer of 16 / 2 heads of 256, a 1040-token prompt (batched
    prefill in the engine's 64-token chunks) and 16 greedy decode steps,
    against the engine's own fwd_block_qwen35 on the CPU.  The FFN is narrow
    (it is not on the path).  Beyond logits and tokens: the HBM KV equals the
    host KV, the first GDN layer's conv delay line (its inputs are embedding
    rows, the same bits on both engines) equals the CPU engine's bit for bit,
    and every GDN state stays within the tolerance."""
    blocks, hidden, heads, kv, hd, n_k, n_v, hvd = 4, 2048, 16, 2, 256, 16, 16, 128
    path = make_q35(e2e, tmp_path / "q5.llf", blocks, hidden, heads, kv, hd, n_k, n_v, hvd, seq=1152, ffn=128)
    prompt = prompt_of(1040)
    n_dec = 16
    conv_n, state_n, n_gdn = 4 * (2 * n_k + n_v) * hvd, n_v * hvd * hvd, 3
    cap = n_gdn * (conv_n + state_n)
    want, wt, _, _, gw = run(e2e, path, prompt, n_dec, use_hip=False, gdn_cap=cap)
    got, gt, status, msg, gg = run(e2e, path, prompt, n_dec, use_hip=True, gdn_cap=cap)
    assert status[0] == 0, msg
    errs = [rel_l2(got[i], want[i]) for i in range(n_dec + 1)]
    print(f"e2e qwen35 fifth-config shapes, prompt 1040: max rel_l2 {max(errs):.3e}, tokens {gt.tolist()}")
    assert max(errs) <= TOL
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(want, axis=1))
    assert np.array_equal(gt, wt)
    assert status[1] == 0
    assert gw.size == cap and gg.size == cap
    conv_w, conv_g = gw[: n_gdn * conv_n].reshape(n_gdn, conv_n), gg[: n_gdn * conv_n].reshape(n_gdn, conv_n)
    st_w, st_g = gw[n_gdn * conv_n:].reshape(n_gdn, state_n), gg[n_gdn * conv_n:].reshape(n_gdn, state_n)
    assert np.array_equal(conv_g[0].view(np.uint32), conv_w[0].view(np.uint32))
    for i in range(n_gdn):
        assert rel_l2(conv_g[i], conv_w[i]) <= TOL
        assert rel_l2(st_g[i], st_w[i]) <= TOL, i


@pytest.mark.gpu
@pytest.mark.parametrize("arch,hidden,heads,kv_heads", [(ARCH_LLAMA, 512, 8, 2), (ARCH_QWEN, 1024, 8, 2)])
def test_session_save_resume_with_hbm_cache(e2e, cuda, tmp_path, arch, hidden, heads, kv_heads):
    """KV persistence (YLLMSKV01, cache.c:174-247) with an HBM-resident cache:
    a HIP-bound engine saves its session; a fresh HIP-bound engine loads it,
    sends the rows to HBM (device_hip_kv_from_host) and continues exactly as
    the uninterrupted HIP run, bit for bit.  The file carries the same rows
    as the CPU engine's file (first layer bit-equal, later layers within the
    attention tolerance of the residual stream they come from)."""
    path = make_model(e2e, tmp_path / "m.llf", 3, hidden, heads, kv_heads, arch=arch)
    prompt = prompt_of(70)
    nb, na = 3, 5
    want, wt, st_u, msg = run(e2e, path, prompt, nb + na, use_hip=True)
    assert st_u[0] == 0, msg
    got, gt, status, msg = resume(e2e, path, prompt, nb, na, True, tmp_path / "hip.kv")
    assert status[0] == 0, msg
    assert status[1] == len(prompt) + nb
    assert np.array_equal(gt, wt)
    assert np.array_equal(got.view(np.uint32), want[nb + 1:].view(np.uint32))
    _, _, _, _ = resume(e2e, path, prompt, nb, 1, False, tmp_path / "cpu.kv")
    h_hip, rows_hip = read_session(tmp_path / "hip.kv")
    h_cpu, rows_cpu = read_session(tmp_path / "cpu.kv")
    assert h_hip == h_cpu
    assert np.array_equal(rows_hip[0], rows_cpu[0])
    f16 = lambda r: r.view(np.float16).astype(np.float32)
    for layer in range(1, h_hip[0]):
        assert rel_l2(f16(rows_hip[layer]), f16(rows_cpu[layer])) <= TOL
