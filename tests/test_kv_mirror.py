"""Device-resident KV cache (HipAttnBackend::q35_attention): the attention half of the
reference's q35_full_layer (src/gpu/vulkan_backend.h:5272-5483) driven the way the engine
drives it (src/model/transformer.h:9440-9461): the host cache is the source of truth, the
call gets host_synced = min(mirror_valid, pos), the host stores the returned K/V with its
own conversion (KVCache::store) and records mirror_valid.

Every step is checked against the CPU oracle: oracle_decode_prep for q/gate/K/V, then
attention of the prepped q over the HOST cache rows [0, pos], times sigmoid(gate) --
max-abs 2e-3 and rel-L2 1e-3 -- and the mirror's rows are compared bit-exactly with the
host cache (the mirror stores with the host's truncating conversion).
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O

ROOT = Path(__file__).resolve().parent.parent
SHIM = ROOT / "tests" / "cpp" / "libbackend_shim.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i, _f, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
_lib = None


def shim():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(SHIM))
        lib.shim_ready.restype = _i
        lib.shim_q35_attention.argtypes = [_vp, _i, _i, _i, _i, _i, _i, _f, _f, _i, _i, _vp, _vp, _i, _i, _vp,
                                           _u16p, _u16p, ctypes.c_longlong, _i, _i, _vp, _vp, _vp, _vp, _f32p,
                                           ctypes.POINTER(ctypes.c_uint), _vp]
        lib.shim_q35_attention.restype = _i
        slot_args = list(lib.shim_q35_attention.argtypes)
        slot_args[25] = _vp                             # kv_out: unused (null) in the chained form
        lib.shim_q35_attention_slot.argtypes = slot_args + [_i]
        lib.shim_q35_attention_slot.restype = _i
        lib.shim_chain_end.restype = _i
        lib.shim_chain_is_open.restype = _i
        lib.shim_chain_kv.argtypes = [_i, _f32p, _i]
        lib.shim_chain_kv.restype = _i
        lib.shim_q35_kv_drop.argtypes = [_vp, _i]
        lib.shim_set_gpu_kv_mb.argtypes = [_i]
        lib.shim_kv_mirror_used.restype = ctypes.c_size_t
        lib.shim_set_mirror_store_rne.argtypes = [_i]
        lib.shim_kv_mirror_info.argtypes = [_vp, _i, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        lib.shim_kv_mirror_read.argtypes = [_vp, _i, _i, _i, _i, _u16p, _u16p]
        lib.shim_last_decline.restype = ctypes.c_char_p
        lib.shim_calls_declined.restype = ctypes.c_longlong
        _lib = lib
    return _lib


def trunc16(x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_trunc_n(x, out, x.size)
    return out


def rne16(x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_rne_n(x, out, x.size)
    return out


class HostLayer:
    """One layer of the host KVCache: f16 [n_kv][cap][hd] plus its mirror_valid
    (src/model/kvcache.h:148-178, 224-241, 276-285)."""

    def __init__(self, n_kv, hd, cap, rne=False):
        self.k = np.zeros((n_kv, cap, hd), np.uint16)
        self.v = np.zeros((n_kv, cap, hd), np.uint16)
        self.n_tokens = 0
        self.mirror_valid = 0
        self.conv = rne16 if rne else trunc16           # KVCache::store truncates (kvcache.h:903-911)

    def store(self, pos, kv_out):
        n_kv, _, hd = self.k.shape
        self.k[:, pos] = self.conv(kv_out[0]).reshape(n_kv, hd)
        self.v[:, pos] = self.conv(kv_out[1]).reshape(n_kv, hd)
        self.mirror_valid = min(self.mirror_valid, pos)
        self.n_tokens = max(self.n_tokens, pos + 1)

    def write_raw(self, pos0, k, v):                   # context editing: rows change under the mirror
        self.k[:, pos0:pos0 + k.shape[1]] = k
        self.v[:, pos0:pos0 + v.shape[1]] = v
        self.mirror_valid = min(self.mirror_valid, pos0)
        self.n_tokens = max(self.n_tokens, pos0 + k.shape[1])


class Layer:
    """Weights and shape of one gated full-attention layer (Qwen3.5 style by default)."""

    def __init__(self, rng, n_heads=16, n_kv=2, hd=256, rot=64, gated=True, q_zc=True, k_zc=True,
                 interleaved=False, host_cap=4096):
        self.n_heads, self.n_kv, self.hd, self.rot, self.gated = n_heads, n_kv, hd, rot, gated
        self.q_zc, self.k_zc, self.interleaved = q_zc, k_zc, interleaved
        self.qnw = (0.1 * rng.standard_normal(hd)).astype(np.float32)
        self.knw = (0.1 * rng.standard_normal(hd)).astype(np.float32)
        self.host = HostLayer(n_kv, hd, host_cap)

    def flags(self):
        return ((O.PREP_Q_ZC if self.q_zc else 0) | (O.PREP_K_ZC if self.k_zc else 0)
                | (0 if self.gated else O.PREP_NO_GATE) | (O.PREP_INTERLEAVED if self.interleaved else 0))

    def table(self, pos):
        i = np.arange(self.rot // 2)
        ang = pos / np.power(1e7, 2.0 * i / self.rot)
        return np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32)


def fill_prompt(layer, rng, n):
    """Rows [0, n) as the CPU prefill would leave them (random f16 of unit scale)."""
    vals = lambda: trunc16(rng.standard_normal((layer.n_kv, n, layer.hd)).astype(np.float32)).reshape(layer.n_kv, n, layer.hd)
    layer.host.write_raw(0, vals(), vals())


def step(layer, rng, pos, owner, layer_id=0, expect_ok=True):
    """One decode token through the backend; returns (device output, returned K/V), both
    checked, when it ran."""
    import torch

    lib = shim()
    hq, nkv, hd = layer.n_heads, layer.n_kv, layer.hd
    qg = (rng.standard_normal((hq, (2 if layer.gated else 1) * hd)) * 2).astype(np.float32)
    kraw = (rng.standard_normal((nkv, hd)) * 2).astype(np.float32)
    vraw = rng.standard_normal((nkv, hd)).astype(np.float32)
    tab = layer.table(pos)
    t = lambda x: torch.from_numpy(x).cuda()
    qg_d, k_d, v_d = t(qg), t(kraw), t(vraw)
    out_d = torch.full((hq, hd), 7.0, dtype=torch.float32, device="cuda")
    kv_out = np.full((2, nkv, hd), 7.0, np.float32)
    mv = ctypes.c_uint(12345)
    h = layer.host
    stream = torch.cuda.current_stream().cuda_stream
    ok = lib.shim_q35_attention(owner, layer_id, hq, nkv, hd, layer.rot, pos, 1e-6, 0.0, int(layer.gated),
                                int(layer.interleaved), layer.qnw.ctypes.data, layer.knw.ctypes.data, int(layer.q_zc),
                                int(layer.k_zc), tab.ctypes.data, h.k.reshape(-1), h.v.reshape(-1), h.k.shape[1],
                                h.n_tokens, min(h.mirror_valid, pos), qg_d.data_ptr(), k_d.data_ptr(), v_d.data_ptr(),
                                out_d.data_ptr(), kv_out, ctypes.byref(mv), stream)
    torch.cuda.synchronize()
    if not expect_ok:
        assert ok == 0
        assert np.all(kv_out == 7.0) and mv.value == 12345
        assert torch.all(out_d == 7.0).item()
        return None
    assert ok == 1, lib.shim_last_decline()
    assert mv.value == pos + 1
    # reference: prep on the CPU, then attention over the host cache with the host's own store
    r_q, r_gate, _, _, r_kv = O.decode_prep(qg, kraw, vraw, layer.qnw, layer.knw, tab, n_heads=hq, n_kv=nkv, hd=hd,
                                            rot=layer.rot, flags=layer.flags(), eps=1e-6, pos=0, cap=1)
    np.testing.assert_allclose(kv_out, r_kv, rtol=1e-5, atol=2e-5)
    h.store(pos, kv_out)
    h.mirror_valid = mv.value                           # KVCache::set_mirror_valid
    ref = O.attn_batch(r_q[None], np.ascontiguousarray(h.k[:, :pos + 1]), np.ascontiguousarray(h.v[:, :pos + 1]),
                       n_kv_heads=nkv, n_ctx=pos + 1, q_base_pos=pos, n_threads=8)[0]
    if layer.gated:
        ref = O.gate_mul(ref, r_gate)
    got = out_d.cpu().numpy()
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[mirror] pos={pos} max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma < 2e-3 and rl < 1e-3, (ma, rl)
    return got, kv_out


def mirror_info(owner, layer_id=0):
    cap, valid = ctypes.c_size_t(), ctypes.c_size_t()
    if not shim().shim_kv_mirror_info(owner, layer_id, ctypes.byref(cap), ctypes.byref(valid)):
        return None
    return cap.value, valid.value


def assert_mirror_equals_host(layer, owner, n, layer_id=0):
    for h in range(layer.n_kv):
        k = np.zeros((n, layer.hd), np.uint16)
        v = np.zeros((n, layer.hd), np.uint16)
        assert shim().shim_kv_mirror_read(owner, layer_id, h, 0, n, k.reshape(-1), v.reshape(-1)) == 1
        np.testing.assert_array_equal(k, layer.host.k[h, :n])
        np.testing.assert_array_equal(v, layer.host.v[h, :n])


# ---------------------------------------------------------------------------- CPU

def test_q35_attention_declines_without_device():
    if not SHIM.exists():
        pytest.skip("tests/cpp/libbackend_shim.so not built")
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a HIP device is present")
    except ImportError:
        pass
    lib = shim()
    z = np.zeros(16, np.uint16)
    kv = np.full((2, 1, 64), 7.0, np.float32)
    mv = ctypes.c_uint(5)
    f = np.zeros(64, np.float32).ctypes.data
    assert lib.shim_q35_attention(1, 0, 1, 1, 64, 0, 0, 1e-6, 0.0, 0, 0, None, None, 0, 0, None, z, z, 0, 0, 0,
                                  f, f, f, f, kv, ctypes.byref(mv), None) == 0
    assert np.all(kv == 7.0) and mv.value == 5
    assert mirror_info(1) is None


# ---------------------------------------------------------------------------- GPU

@pytest.mark.gpu
def test_decode_sequence_fill_grow_and_rewind(hip):
    """Prompt rows filled from the host on the first call, then per-token appends; a jump
    past the 2048-row capacity grows the mirror (rows kept by a device copy, the rest
    filled); an edit of old host rows (rewind) is re-filled from the edited host copy."""
    rng = np.random.default_rng(101)
    lib = shim()
    lib.shim_set_gpu_kv_mb(-1)
    owner = 0x5001
    L = Layer(rng, host_cap=4096)
    fill_prompt(L, rng, 300)                            # CPU prefill: mirror knows nothing yet
    used0 = lib.shim_kv_mirror_used()
    for pos in range(300, 304):
        step(L, rng, pos, owner)
    assert mirror_info(owner) == (2048, 304)            # max(round256(301 * 5/4), 2048)
    assert lib.shim_kv_mirror_used() - used0 == 2048 * 2 * 256 * 2 * 2
    assert_mirror_equals_host(L, owner, 304)

    # host catches up to 2100 tokens on the CPU (e.g. a long chunk), then decodes on the GPU
    more = lambda n: trunc16(rng.standard_normal((L.n_kv, n, L.hd)).astype(np.float32)).reshape(L.n_kv, n, L.hd)
    L.host.write_raw(304, more(2100 - 304), more(2100 - 304))
    step(L, rng, 2100, owner)
    cap, valid = mirror_info(owner)
    assert (cap, valid) == (((2101 * 5 // 4 + 255) // 256) * 256, 2101)
    assert_mirror_equals_host(L, owner, 2101)

    # rewind: rows 50..59 edited on the host (context editing), the next token re-syncs them
    L.host.write_raw(50, more(10), more(10))
    assert L.host.mirror_valid == 50
    step(L, rng, 2101, owner)
    assert_mirror_equals_host(L, owner, 2102)

    lib.shim_q35_kv_drop(owner, -1)
    assert mirror_info(owner) is None
    assert lib.shim_kv_mirror_used() == used0


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [
    dict(n_heads=40, n_kv=8, hd=128, rot=128, gated=False, q_zc=False, k_zc=False),              # plain q/k-norm layer
    dict(n_heads=8, n_kv=8, hd=64, rot=64, gated=False, q_zc=False, k_zc=False, interleaved=True),
    dict(n_heads=12, n_kv=2, hd=192, rot=48, gated=True),
])
def test_layer_variants(hip, cfg):
    rng = np.random.default_rng(7)
    owner = 0x6001
    L = Layer(rng, host_cap=512, **cfg)
    fill_prompt(L, rng, 37)
    for pos in (37, 38, 39):
        step(L, rng, pos, owner, layer_id=3)
    assert_mirror_equals_host(L, owner, 40, layer_id=3)
    shim().shim_q35_kv_drop(owner, -1)


@pytest.mark.gpu
def test_budget_refusal_and_shape_change(hip):
    """A mirror that would exceed the budget is refused (nothing touched) and the refused
    size is remembered; a shape change for the same (owner, layer) starts a new mirror."""
    rng = np.random.default_rng(9)
    lib = shim()
    owner = 0x7001
    L = Layer(rng, host_cap=2048)
    fill_prompt(L, rng, 1700)
    try:
        lib.shim_set_gpu_kv_mb(1)                       # 1 MiB: 256 rows of 2 x 256 x (K+V) f16 fit, 768 do not
        step(L, rng, 10, owner)
        assert mirror_info(owner) == (256, 11)          # the exact-size fallback (round256(need))
        declined = lib.shim_calls_declined()
        step(L, rng, 600, owner, expect_ok=False)
        assert b"budget" in lib.shim_last_decline()
        assert mirror_info(owner) is None               # the too-small mirror was dropped
        step(L, rng, 650, owner, expect_ok=False)       # below the refused size + 1024: declined at once
        assert b"refused" in lib.shim_last_decline()
        assert lib.shim_calls_declined() == declined + 2
        lib.shim_set_gpu_kv_mb(-1)
        step(L, rng, 1700, owner)                       # beyond the remembered size: tried again, runs
        assert mirror_info(owner)[1] == 1701
    finally:
        lib.shim_set_gpu_kv_mb(-1)
    M = Layer(rng, n_heads=8, n_kv=4, hd=128, rot=32, host_cap=64)
    step(M, rng, 0, owner)                              # same owner/layer, other shape
    assert mirror_info(owner) == (2048, 1)
    lib.shim_q35_kv_drop(owner, 0)
    assert mirror_info(owner) is None


@pytest.mark.gpu
def test_mirror_rne_store(hip):
    """With the shader's round-to-nearest-even store each new mirror row is the RNE
    conversion of the returned K/V: a host that stores with RNE too sees its own rows in the
    mirror, and they differ from the truncating store by at most one unit in the last place."""
    rng = np.random.default_rng(11)
    lib = shim()
    owner = 0x8001
    L = Layer(rng, host_cap=64)
    L.host = HostLayer(L.n_kv, L.hd, 64, rne=True)
    fill_prompt(L, rng, 5)
    try:
        lib.shim_set_mirror_store_rne(1)
        for pos in range(5, 8):
            _, kv_out = step(L, rng, pos, owner)
        assert_mirror_equals_host(L, owner, 8)
        rne = rne16(kv_out).astype(np.int32)
        diff = np.abs(rne - trunc16(kv_out).astype(np.int32))
        assert diff.max() <= 1 and diff.sum() > 0
    finally:
        lib.shim_set_mirror_store_rne(0)
        lib.shim_q35_kv_drop(owner, -1)


@pytest.mark.gpu
def test_chained_layers_join_like_q35_chain_flush(hip):
    """Layers chained without waiting (async_kv_slot = layer), as Transformer::forward runs
    consecutive GPU layers, then one join that stores every slot's K/V into its host cache
    (q35_chain_flush, transformer.h:10083-10100).  Every output and slot matches the CPU path;
    the next token, synchronous, sees the rows the chained calls stored in the mirrors."""
    import torch

    rng = np.random.default_rng(55)
    lib = shim()
    lib.shim_set_gpu_kv_mb(-1)
    owner = 0x7001
    layers = [Layer(rng, host_cap=2048) for _ in range(4)]
    for L in layers:
        fill_prompt(L, rng, 900)
    for pos in (900, 901):                              # two tokens of four chained layers each
        pending = []
        for li, L in enumerate(layers):
            hq, nkv, hd = L.n_heads, L.n_kv, L.hd
            qg = (rng.standard_normal((hq, 2 * hd)) * 2).astype(np.float32)
            kraw = (rng.standard_normal((nkv, hd)) * 2).astype(np.float32)
            vraw = rng.standard_normal((nkv, hd)).astype(np.float32)
            tab = L.table(pos)
            t = lambda x: torch.from_numpy(x).cuda()
            qg_d, k_d, v_d = t(qg), t(kraw), t(vraw)
            out_d = torch.full((hq, hd), 7.0, dtype=torch.float32, device="cuda")
            mv = ctypes.c_uint(0)
            h = L.host
            ok = lib.shim_q35_attention_slot(owner, li, hq, nkv, hd, L.rot, pos, 1e-6, 0.0, 1, 0, L.qnw.ctypes.data,
                                             L.knw.ctypes.data, 1, 1, tab.ctypes.data, h.k.reshape(-1),
                                             h.v.reshape(-1), h.k.shape[1], h.n_tokens, min(h.mirror_valid, pos),
                                             qg_d.data_ptr(), k_d.data_ptr(), v_d.data_ptr(), out_d.data_ptr(), None,
                                             ctypes.byref(mv), torch.cuda.current_stream().cuda_stream, li)
            assert ok == 1, lib.shim_last_decline()
            assert mv.value == pos + 1
            pending.append((L, li, qg, kraw, vraw, tab, out_d, (qg_d, k_d, v_d), mv.value))
        assert lib.shim_chain_is_open() == 1
        assert lib.shim_chain_end() == 1                # the join
        assert lib.shim_chain_is_open() == 0
        for L, li, qg, kraw, vraw, tab, out_d, _, mvv in pending:
            hq, nkv, hd = L.n_heads, L.n_kv, L.hd
            kv = np.zeros((2, nkv, hd), np.float32)
            assert lib.shim_chain_kv(li, kv.reshape(-1), kv.size) == 1
            r_q, r_gate, _, _, r_kv = O.decode_prep(qg, kraw, vraw, L.qnw, L.knw, tab, n_heads=hq, n_kv=nkv, hd=hd,
                                                    rot=L.rot, flags=L.flags(), eps=1e-6, pos=0, cap=1)
            np.testing.assert_allclose(kv, r_kv, rtol=1e-5, atol=2e-5)
            L.host.store(pos, kv)                       # kvcache_.store + set_mirror_valid at the flush
            L.host.mirror_valid = mvv
            ref = O.attn_batch(r_q[None], np.ascontiguousarray(L.host.k[:, :pos + 1]),
                               np.ascontiguousarray(L.host.v[:, :pos + 1]), n_kv_heads=nkv, n_ctx=pos + 1,
                               q_base_pos=pos, n_threads=8)[0]
            ref = O.gate_mul(ref, r_gate)
            got = out_d.cpu().numpy()
            ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
            print(f"[chain] pos={pos} layer={li} max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
            assert ma < 2e-3 and rl < 1e-3
    for li, L in enumerate(layers):
        step(L, rng, 902, owner, layer_id=li)           # synchronous, over the rows the chain stored
        assert_mirror_equals_host(L, owner, 903, layer_id=li)
    lib.shim_q35_kv_drop(owner, -1)
