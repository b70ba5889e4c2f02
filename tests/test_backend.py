"""The engine-side backend (nexus::hip::HipAttnBackend) through its reference signatures.

The reference's engine calls VulkanBackend::attention_flash_gpu / attention_batch_gpu /
attention_stream_gpu / attention_gpu with host pointers and falls back to its CPU
attention when they return false (src/model/transformer.h:8478-8500, :11052-11070).
These tests call the same member functions on HipAttnBackend (through the test shim in
tests/cpp) with host arrays and compare with the CPU oracle, as the reference's
NEXUS_GPU_VERIFY check does (transformer.h:7942-7970).
"""
import ctypes
import os
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O
from nexus_amd.inputs import make_case

ROOT = Path(__file__).resolve().parent.parent
SHIM = ROOT / "tests" / "cpp" / "libbackend_shim.so"

MAX_ABS = 2e-3
REL_L2 = 1e-3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i, _f = ctypes.c_int, ctypes.c_float


def shim():
    if not SHIM.exists():
        pytest.fail(f"{SHIM} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(SHIM))
    lib.shim_ready.restype = _i
    lib.shim_attention_gpu.argtypes = [_f32p, _f32p, _i, _i, _i, _i, _i, _u16p, _u16p, ctypes.c_size_t]
    lib.shim_attention_batch_gpu.argtypes = [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _f, _f, _u16p, _u16p,
                                             ctypes.c_size_t]
    lib.shim_attention_stream_gpu.argtypes = [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _f, _f, _u16p, _u16p, _i]
    lib.shim_attention_flash_gpu.argtypes = [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _f, _f, _u16p, _u16p]
    vp = ctypes.c_void_p
    lib.shim_prefill_device.argtypes = [vp, vp, vp, vp, vp, vp]
    lib.shim_decode_device.argtypes = [vp, vp, vp, vp, vp, _i, vp]
    lib.shim_calls_run.restype = ctypes.c_longlong
    lib.shim_calls_declined.restype = ctypes.c_longlong
    lib.shim_last_decline.restype = ctypes.c_char_p
    return lib


def assert_close(got, ref, what):
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[parity] backend {what} max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma < MAX_ABS and rl < REL_L2, f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}"


# ---------------------------------------------------------------------------- CPU

def test_backend_declines_without_device_and_leaves_output_untouched():
    import torch

    if torch.cuda.is_available():
        pytest.skip("host has a GPU: the no-device decline is tested on CPU hosts")
    lib = shim()
    assert lib.shim_ready() == 0
    q, k, v = make_case(n_q_heads=4, n_kv_heads=2, head_dim=64, n_query=3, n_ctx=10)
    out = np.full(q.shape, 7.0, np.float32)
    assert lib.shim_attention_flash_gpu(q, out, 4, 2, 64, 10, 3, 7, 0, 0.0, 0.0, k, v) == 0
    assert lib.shim_attention_gpu(np.ascontiguousarray(q[0]), out[0], 4, 2, 64, 0, 10, k, v, k.nbytes) == 0
    assert np.all(out == 7.0)
    assert lib.shim_calls_run() == 0 and lib.shim_calls_declined() >= 2
    assert b"no HIP device" in lib.shim_last_decline()


# ---------------------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv,hd,nq,base,sw,cap", [
    (8, 2, 128, 150, 100, 0, 0.0),       # chunk after cache, f32 Q (prefill kernel)
    (40, 8, 128, 3, 900, 0, 0.0),        # a few queries (split-KV kernel)
    (16, 2, 256, 4, 600, 0, 0.0),        # verify shape, hd 256
    (8, 8, 64, 90, 0, 40, 0.0),          # sliding window, cold
    (8, 4, 128, 70, 30, 0, 25.0),        # softcap
])
def test_flash_matches_cpu_attention(hip, hq, hkv, hd, nq, base, sw, cap):
    lib = shim()
    assert lib.shim_ready() == 1
    n_ctx = base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=31)
    out = np.zeros(q.shape, np.float32)
    before = lib.shim_calls_run()
    assert lib.shim_attention_flash_gpu(q, out, hq, hkv, hd, n_ctx, nq, base, sw, 0.0, cap, k, v) == 1, \
        lib.shim_last_decline()
    assert lib.shim_calls_run() == before + 1
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw, softcap=cap,
                       n_threads=8)
    assert_close(out, ref, f"flash hq={hq} hkv={hkv} hd={hd} nq={nq} base={base} sw={sw} cap={cap}")


@pytest.mark.gpu
@pytest.mark.parametrize("q_std", [4.0, 8.0])
@pytest.mark.parametrize("hq,hkv,hd,nq,base,n_rows", [
    (40, 8, 128, 512, 4096, 1536),       # cfg2's shape (sampled rows checked)
    (16, 2, 256, 256, 1000, 0),          # head dim 256 (one wave per SIMD, AGPR operands)
    (8, 2, 128, 150, 100, 0),            # 64-row blocks with two key groups
    (12, 4, 192, 130, 40, 0),            # head dim 192
    (8, 2, 64, 200, 300, 0),             # head dim 64
])
def test_flash_precision_at_large_query_magnitudes(hip, q_std, hq, hkv, hd, nq, base, n_rows):
    """The engine hands attention_flash_gpu f32 queries (transformer.h:8478-8494, as
    attn_batch_cpu takes them, :8653).  With queries of std 4 and 8 the softmax is sharp and
    an f16 rounding of q (or of q * scale) alone moves the output past 2e-3; the kernels keep
    f32 queries as an f16 high part plus its f16 residual."""
    lib = shim()
    assert lib.shim_ready() == 1
    n_ctx = base + nq
    print(f"[case] flash q_std={q_std} hq={hq} hkv={hkv} hd={hd} nq={nq} base={base}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=41,
                        q_scale=q_std)
    out = np.zeros(q.shape, np.float32)
    assert lib.shim_attention_flash_gpu(q, out, hq, hkv, hd, n_ctx, nq, base, 0, 0.0, 0.0, k, v) == 1, \
        lib.shim_last_decline()
    if n_rows:
        rng = np.random.default_rng(7)
        total = nq * hq
        rows = np.unique(np.concatenate([[0, total - 1], rng.choice(total, n_rows, replace=False)])).astype(np.int32)
        ref = O.attn_batch_rows(q, k, v, rows, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base,
                                n_threads=8).reshape(total, hd)[rows]
        got = out.reshape(total, hd)[rows]
    else:
        ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
        got = out
    assert_close(got, ref, f"flash q_std={q_std} hq={hq} hd={hd} nq={nq} base={base}")


@pytest.mark.gpu
def test_batch_and_stream_match_flash(hip):
    lib = shim()
    hq, hkv, hd, nq, base = 10, 2, 128, 60, 200
    n_ctx = base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=32)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    ob = np.zeros(q.shape, np.float32)
    os_ = np.zeros(q.shape, np.float32)
    assert lib.shim_attention_batch_gpu(q, ob, hq, hkv, hd, n_ctx, nq, base, 0, 0.0, 0.0, k, v, k.nbytes) == 1
    assert lib.shim_attention_stream_gpu(q, os_, hq, hkv, hd, n_ctx, nq, base, 0.0, 0.0, k, v, 0) == 1
    assert_close(ob, ref, "batch")
    assert_close(os_, ref, "stream")
    assert np.array_equal(ob, os_)


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv,hd,n_ctx", [(16, 4, 128, 4096), (40, 8, 128, 777), (8, 1, 64, 1)])
def test_attention_gpu_matches_forward_cached_scores(hip, hq, hkv, hd, n_ctx):
    lib = shim()
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=n_ctx, seed=33)
    q0 = np.ascontiguousarray(q[0])
    out = np.zeros_like(q0)
    assert lib.shim_attention_gpu(q0, out, hq, hkv, hd, 3, n_ctx, k, v, k.nbytes) == 1, lib.shim_last_decline()
    ref = O.cached_scores(q0, k, v, n_kv_heads=hkv, pos=n_ctx - 1, n_threads=8)
    assert_close(out, ref, f"attention_gpu hq={hq} hkv={hkv} n_ctx={n_ctx}")


@pytest.mark.gpu
def test_backend_declines_like_the_reference(hip):
    lib = shim()
    q, k, v = make_case(n_q_heads=8, n_kv_heads=2, head_dim=64, n_query=5, n_ctx=20, seed=34)
    out = np.full(q.shape, 3.0, np.float32)
    # head_dim 96 is not a multiple of 64 (vulkan_backend.h:4270)
    q96 = np.zeros((5, 8, 96), np.float32)
    k96 = np.zeros((2, 20, 96), np.uint16)
    o96 = np.full((5, 8, 96), 3.0, np.float32)
    assert lib.shim_attention_flash_gpu(q96, o96, 8, 2, 96, 20, 5, 15, 0, 0.0, 0.0, k96, k96) == 0
    assert np.all(o96 == 3.0)
    # Hq not a multiple of Hkv
    assert lib.shim_attention_flash_gpu(q, out, 8, 3, 64, 20, 5, 15, 0, 0.0, 0.0, k, v) == 0
    # kv_bytes too small for the declared cache
    assert lib.shim_attention_batch_gpu(q, out, 8, 2, 64, 20, 5, 15, 0, 0.0, 0.0, k, v, 16) == 0
    assert np.all(out == 3.0)
    # K+V above the NEXUS_FLASH_KV_MB budget (read per call)
    os.environ["NEXUS_FLASH_KV_MB"] = "1"
    try:
        qb, kb, vb = make_case(n_q_heads=8, n_kv_heads=2, head_dim=128, n_query=2, n_ctx=4096, seed=35)
        ob = np.full(qb.shape, 3.0, np.float32)
        assert lib.shim_attention_flash_gpu(qb, ob, 8, 2, 128, 4096, 2, 4094, 0, 0.0, 0.0, kb, vb) == 0
        assert np.all(ob == 3.0)
        assert b"NEXUS_FLASH_KV_MB" in lib.shim_last_decline()
    finally:
        del os.environ["NEXUS_FLASH_KV_MB"]
    assert lib.shim_attention_flash_gpu(q, out, 8, 2, 64, 20, 5, 15, 0, 0.0, 0.0, k, v) == 1


@pytest.mark.gpu
def test_device_forms_on_two_streams_take_turns_on_the_workspace(hip):
    """prefill_device and decode_device share the backend's split workspace.  Launched back to
    back on two different streams with no synchronisation between them, the second call's
    partials must not overwrite the first call's while its combine still reads them: every
    output matches the oracle."""
    import torch

    from nexus_amd import capi

    lib = shim()
    assert lib.shim_ready() == 1

    def dev(x):
        if x.dtype == np.uint16:
            return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
        return torch.from_numpy(np.ascontiguousarray(x)).cuda()

    # a short chunk over a long cache (split prefill + combine) and a 64-split decode
    pq, pk, pv = make_case(n_q_heads=8, n_kv_heads=2, head_dim=128, n_query=64, n_ctx=8064, seed=61)
    pdesc = capi.make_desc(n_q_heads=8, n_kv_heads=2, head_dim=128, n_query=64, q_base_pos=8000, n_ctx=8064)
    dq, dk, dv = make_case(n_q_heads=40, n_kv_heads=8, head_dim=128, n_query=1, n_ctx=20000, seed=62)
    ddesc = capi.make_desc(n_q_heads=40, n_kv_heads=8, head_dim=128, n_query=1, q_base_pos=19999, n_ctx=20000)
    assert capi.prefill_ws_bytes(pdesc) > 0
    pref = O.attn_batch(pq, pk, pv, n_kv_heads=2, n_ctx=8064, q_base_pos=8000, n_threads=8)
    dref = O.attn_batch(dq, dk, dv, n_kv_heads=8, n_ctx=20000, q_base_pos=19999, n_threads=8)
    pqd, pkd, pvd, dqd, dkd, dvd = map(dev, (pq, pk, pv, dq, dk, dv))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    # size the backend's workspace for the larger of the two calls first
    pout = torch.empty(pq.shape, device="cuda")
    dout = torch.empty(dq.shape, device="cuda")
    for d, call in ((pdesc, lambda st: lib.shim_prefill_device(ctypes.byref(pdesc), pqd.data_ptr(), pkd.data_ptr(),
                                                                pvd.data_ptr(), pout.data_ptr(), st.cuda_stream)),
                    (ddesc, lambda st: lib.shim_decode_device(ctypes.byref(ddesc), dqd.data_ptr(), dkd.data_ptr(),
                                                               dvd.data_ptr(), dout.data_ptr(), 64, st.cuda_stream))):
        assert call(s1) == 1, lib.shim_last_decline()
    torch.cuda.synchronize()
    for it in range(8):
        pout.fill_(float("nan"))
        dout.fill_(float("nan"))
        torch.cuda.synchronize()
        assert lib.shim_prefill_device(ctypes.byref(pdesc), pqd.data_ptr(), pkd.data_ptr(), pvd.data_ptr(),
                                       pout.data_ptr(), s1.cuda_stream) == 1
        assert lib.shim_decode_device(ctypes.byref(ddesc), dqd.data_ptr(), dkd.data_ptr(), dvd.data_ptr(),
                                      dout.data_ptr(), 64, s2.cuda_stream) == 1
        torch.cuda.synchronize()
        assert_close(pout.cpu().numpy(), pref, f"prefill_device on stream 1, round {it}")
        assert_close(dout.cpu().numpy(), dref, f"decode_device on stream 2, round {it}")
