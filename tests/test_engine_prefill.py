"""The engine's prompt attention sequence around the kept boundary, one layer at a time.

tests/cpp/engine_prefill.cpp drives HipAttnBackend the way the reference's engine does
(src/model/transformer.h:8443-8515 per call, :8551-8651 for the tiling): each tile stores its
tokens' K/V into a host cache with the KV cache's truncating conversion, packs rows [0, n_ctx),
calls attention_flash_gpu, falls back to the batch/stream GPU members and then to the CPU
attention, and applies the sigmoid output gate.  The oracle is attn_batch_cpu over the whole
prompt (transformer.h:8653-8685) on the same truncated K/V, times the gate.
"""
import ctypes
import os
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O
from nexus_amd.inputs import f32_to_f16_trunc, normal

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "tests" / "cpp" / "libengine_prefill.so"

MAX_ABS = 2e-3
REL_L2 = 1e-3
GATED, NO_GPU_FALLBACK, BATCHED = 1, 2, 4


class Layer(ctypes.Structure):
    _fields_ = [("n_heads", ctypes.c_int), ("n_kv", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("scale", ctypes.c_float), ("softcap", ctypes.c_float), ("tile", ctypes.c_int),
                ("flags", ctypes.c_int), ("cpu_threads", ctypes.c_int)]


_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def harness():
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB))
    lib.eh_cache_new.restype = ctypes.c_void_p
    lib.eh_cache_new.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.eh_cache_free.argtypes = [ctypes.c_void_p]
    lib.eh_cache_capacity.restype = ctypes.c_long
    lib.eh_cache_capacity.argtypes = [ctypes.c_void_p]
    lib.eh_cache_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u16p, _u16p]
    lib.eh_prefill_layer.argtypes = [ctypes.POINTER(Layer), ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     _f32p, _f32p, _f32p, ctypes.c_void_p, _f32p, _i32p, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int)]
    return lib


class Prompt:
    """Post-RoPE Q/K/V (f32) and gate logits of n tokens of one layer, seeded."""

    def __init__(self, hq, hkv, hd, n, seed, q_std=1.0):
        self.hq, self.hkv, self.hd, self.n = hq, hkv, hd, n
        self.q = (normal(seed, n * hq * hd) * q_std).reshape(n, hq * hd).astype(np.float32)
        self.k = normal(seed + 1, n * hkv * hd).reshape(n, hkv * hd)
        self.v = normal(seed + 2, n * hkv * hd).reshape(n, hkv * hd)
        self.gate = (normal(seed + 3, n * hq * hd) * 3).reshape(n, hq * hd).astype(np.float32)

    def kv_f16(self, n_ctx):
        """K/V of tokens [0, n_ctx) as the cache stores them, packed [Hkv][n_ctx][hd]."""
        k = f32_to_f16_trunc(self.k[:n_ctx].reshape(n_ctx, self.hkv, self.hd).transpose(1, 0, 2).copy())
        v = f32_to_f16_trunc(self.v[:n_ctx].reshape(n_ctx, self.hkv, self.hd).transpose(1, 0, 2).copy())
        return np.ascontiguousarray(k), np.ascontiguousarray(v)

    def reference(self, start, n, gated, rows=None):
        """attn_batch_cpu for tokens [start, start + n) over keys [0, start + n), gated."""
        k, v = self.kv_f16(start + n)
        q = self.q[start:start + n].reshape(n, self.hq, self.hd)
        if rows is None:
            out = O.attn_batch(q, k, v, n_kv_heads=self.hkv, n_ctx=start + n, q_base_pos=start, n_threads=8)
        else:
            out = O.attn_batch_rows(q, k, v, rows, n_kv_heads=self.hkv, n_ctx=start + n, q_base_pos=start,
                                    n_threads=8)
        out = out.reshape(n, self.hq * self.hd)
        return O.gate_mul(out, self.gate[start:start + n]) if gated else out


def run(lib, cache, p, start, n, *, tile, flags, max_tiles=64):
    layer = Layer(p.hq, p.hkv, p.hd, 0.0, 0.0, tile, flags, 8)
    out = np.zeros((n, p.hq * p.hd), np.float32)
    path = np.full(max_tiles, -1, np.int32)
    clean = ctypes.c_int(0)
    gate = p.gate[start:start + n] if flags & GATED else None
    tiles = lib.eh_prefill_layer(ctypes.byref(layer), cache, start, n, np.ascontiguousarray(p.q[start:start + n]),
                                 np.ascontiguousarray(p.k[start:start + n]), np.ascontiguousarray(p.v[start:start + n]),
                                 None if gate is None else np.ascontiguousarray(gate).ctypes.data, out, path,
                                 max_tiles, ctypes.byref(clean))
    return out, list(path[:tiles]), clean.value


def check(got, ref, what):
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[parity] engine {what} max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma < MAX_ABS and rl < REL_L2, f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}"


def tile_sizes(n, t):
    """The engine's tiling (transformer.h:8599-8637): even tiles, never a lone last token."""
    if t <= 0 or n <= t:
        return [n]
    tiles = -(-n // t)
    tile = -(-n // tiles)
    out, t0 = [], 0
    while t0 < n:
        cnt = min(tile, n - t0)
        if n - t0 - cnt == 1:
            cnt += 1
        out.append(cnt)
        t0 += cnt
    return out


# ---------------------------------------------------------------------------- CPU

def test_tiling_rule_matches_the_engine():
    assert tile_sizes(8192, 1024) == [1024] * 8
    assert tile_sizes(1000, 1024) == [1000]
    assert tile_sizes(2049, 1024) == [683, 683, 683]
    assert tile_sizes(1025, 512) == [342, 342, 341]
    assert tile_sizes(17, 8) == [6, 6, 5]
    assert sum(tile_sizes(4097, 1024)) == 4097 and all(s > 1 for s in tile_sizes(4097, 1024))


def test_without_a_device_every_tile_runs_the_cpu_attention():
    """On a host without a GPU every GPU member declines before touching the output, so each
    tile falls back to the CPU attention: the caller sequence (store, pack, gate, tiling, the
    cache handoff between calls) is exercised on CPU."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("host has a GPU: the no-device path is tested on CPU hosts")
    lib = harness()
    p = Prompt(4, 2, 64, 300, seed=11)
    cache = lib.eh_cache_new(2, 64)
    try:
        out, path, clean = run(lib, cache, p, 0, 200, tile=64, flags=GATED)
        assert path == [2] * len(tile_sizes(200, 64)) and clean == 1
        check(out, p.reference(0, 200, True), "cpu cold 200 in tiles of 64")
        out2, path2, clean2 = run(lib, cache, p, 200, 100, tile=0, flags=GATED)   # a chunk onto the cache
        assert path2 == [2] and clean2 == 1
        check(out2, p.reference(200, 100, True), "cpu chunk of 100 after 200")
        # the cache holds exactly the truncating conversion of every stored row
        k_ref, v_ref = p.kv_f16(300)
        kk, vv = np.zeros((300, 64), np.uint16), np.zeros((300, 64), np.uint16)
        for h in range(2):
            assert lib.eh_cache_read(cache, h, 0, 300, kk, vv) == 1
            np.testing.assert_array_equal(kk, k_ref[h])
            np.testing.assert_array_equal(vv, v_ref[h])
        assert lib.eh_cache_capacity(cache) == 512          # 512 tokens at first (kvcache.h:715)
    finally:
        lib.eh_cache_free(cache)


def test_cache_capacity_grows_like_kvcache():
    """512, doubled up to 8192, then +4096 (kvcache.h:856-873), as the tiles store rows."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("exercised through the GPU tests on a GPU host")
    lib = harness()
    p = Prompt(1, 1, 64, 9000, seed=12)
    cache = lib.eh_cache_new(1, 64)
    try:
        caps = []
        for start, n in ((0, 513), (513, 1600), (2113, 6200), (8313, 687)):
            layer = Layer(1, 1, 64, 0.0, 0.0, 0, NO_GPU_FALLBACK, 8)
            out = np.zeros((n, 64), np.float32)
            path = np.zeros(4, np.int32)
            clean = ctypes.c_int(0)
            lib.eh_prefill_layer(ctypes.byref(layer), cache, start, n, np.ascontiguousarray(p.q[start:start + n]),
                                 np.ascontiguousarray(p.k[start:start + n]), np.ascontiguousarray(p.v[start:start + n]),
                                 None, out, path, 4, ctypes.byref(clean))
            caps.append(lib.eh_cache_capacity(cache))
        assert caps == [1024, 4096, 12288, 12288]
    finally:
        lib.eh_cache_free(cache)


# ---------------------------------------------------------------------------- GPU

@pytest.mark.gpu
def test_cold_prompt_in_engine_tiles_matches_one_call_and_the_oracle(hip):
    """A cold 8192-token prompt driven as 8 tiles of 1024 (the engine's default tiling):
    every tile on attention_flash_gpu, the result equal to one call over the whole prompt
    and to the CPU attention, gate included."""
    lib = harness()
    p = Prompt(8, 2, 128, 8192, seed=21)
    print("[case] engine cold 8192 in 8 tiles, gated", flush=True)
    c1, c2 = lib.eh_cache_new(2, 128), lib.eh_cache_new(2, 128)
    try:
        tiled, path, clean = run(lib, c1, p, 0, 8192, tile=1024, flags=GATED)
        assert path == [0] * 8 and clean == 1
        whole, path1, _ = run(lib, c2, p, 0, 8192, tile=0, flags=GATED)
        assert path1 == [0]
        check(tiled, whole, "8 tiles vs one call")
        rng = np.random.default_rng(3)
        rows = np.unique(np.concatenate([[0, 8192 * 8 - 1], rng.choice(8192 * 8, 1024, replace=False)])).astype(np.int32)
        ref = p.reference(0, 8192, True, rows=rows).reshape(8192 * 8, 128)[rows]
        check(tiled.reshape(8192 * 8, 128)[rows], ref, "8 tiles vs oracle (sampled rows)")
    finally:
        lib.eh_cache_free(c1)
        lib.eh_cache_free(c2)


@pytest.mark.gpu
@pytest.mark.parametrize("gpu_fallback", [False, True])
def test_decline_mid_prompt_falls_back_without_touching_outputs(hip, gpu_fallback):
    """NEXUS_FLASH_KV_MB (read per call, vulkan_backend.h:4274-4277) makes
    attention_flash_gpu decline once the packed K/V outgrows it, part-way through the prompt.
    A declined call leaves its tile's output untouched; the tile then runs on the stream
    member (GPU) or on the CPU attention, and the whole prompt still matches the oracle."""
    lib = harness()
    p = Prompt(8, 2, 128, 2048, seed=22)
    # K+V of n_ctx tokens = 2 * 2 heads * n_ctx * 128 * 2 B: 1 MB from n_ctx = 1024 on
    old = os.environ.get("NEXUS_FLASH_KV_MB")
    os.environ["NEXUS_FLASH_KV_MB"] = "1"
    cache = lib.eh_cache_new(2, 128)
    try:
        print(f"[case] engine decline mid-prompt gpu_fallback={gpu_fallback}", flush=True)
        out, path, clean = run(lib, cache, p, 0, 2048, tile=256, flags=GATED | (0 if gpu_fallback else NO_GPU_FALLBACK))
        later = 1 if gpu_fallback else 2
        assert path == [0, 0, 0, 0, later, later, later, later], path
        assert clean == 1
        check(out, p.reference(0, 2048, True), f"decline mid-prompt, fallback {'stream' if gpu_fallback else 'cpu'}")
    finally:
        lib.eh_cache_free(cache)
        if old is None:
            os.environ.pop("NEXUS_FLASH_KV_MB", None)
        else:
            os.environ["NEXUS_FLASH_KV_MB"] = old


@pytest.mark.gpu
def test_chunks_onto_an_existing_cache(hip):
    """Prompt chunks appended after cached tokens (the second user turn of a chat): the
    cache written by the first call is what the second call packs and attends over, and a
    chunk too short for the GPU (< 16 tokens) runs on the CPU attention."""
    lib = harness()
    p = Prompt(16, 2, 256, 1700, seed=23)
    cache = lib.eh_cache_new(2, 256)
    try:
        print("[case] engine chunks 1000 + 690 + 10, hd 256", flush=True)
        a, pa, _ = run(lib, cache, p, 0, 1000, tile=512, flags=GATED | BATCHED)
        b, pb, _ = run(lib, cache, p, 1000, 690, tile=1024, flags=GATED | BATCHED)
        c, pc, _ = run(lib, cache, p, 1690, 10, tile=1024, flags=GATED | BATCHED)
        assert pa == [0, 0] and pb == [0] and pc == [2]
        check(a, p.reference(0, 1000, True), "first chunk")
        check(b, p.reference(1000, 690, True), "second chunk after 1000 cached")
        check(c, p.reference(1690, 10, True), "10-token chunk on the CPU")
    finally:
        lib.eh_cache_free(cache)
