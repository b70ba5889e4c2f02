"""Test-side access to the CPU oracle (oracle/libattn_oracle.so) and, when it was built,
to the reference's own decode code (oracle/_ref/libnexus_ref_attn.so).

Only tests, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this module.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "libattn_oracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libnexus_ref_attn.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i, _l, _f, _d = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double
_vp = ctypes.c_void_p
_vpp = ctypes.POINTER(ctypes.c_void_p)

_oracle = None
_ref = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle` (or __graft_entry__.build())")
        lib = ctypes.CDLL(str(ORACLE_SO))
        lib.nx_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        lib.nx_f16_bits_to_f32.restype = _f
        lib.nx_f32_to_f16_trunc.argtypes = [_f]
        lib.nx_f32_to_f16_trunc.restype = ctypes.c_uint16
        lib.nx_f32_to_f16_rne.argtypes = [_f]
        lib.nx_f32_to_f16_rne.restype = ctypes.c_uint16
        lib.nx_f32_to_f16_trunc_n.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        lib.nx_f32_to_f16_rne_n.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        lib.nx_f16_to_f32_n.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        lib.oracle_attn_batch.argtypes = [_f32p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _l, _i, _i, _i, _f, _f, _i]
        lib.oracle_attn_batch_rows.argtypes = [_f32p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _l, _i, _i, _i,
                                               _f, _f, _i32p, _i, _i]
        lib.oracle_cached_scores.argtypes = [_f32p, _f32p, _u16p, _u16p, _l, _i, _i, _i, _i, _f, _f, _i]
        lib.oracle_split_partials.argtypes = [_f32p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _l, _i, _i, _f, _i, _i]
        lib.oracle_split_combine.argtypes = [_f32p, _f32p, _i, _i, _i]
        lib.oracle_naive_f64.argtypes = [_f32p, _u16p, _u16p, _f64p, _i, _i, _i, _i, _l, _i, _i, _i, _d, _d]
        lib.oracle_gate_mul.argtypes = [_f32p, _f32p, ctypes.c_size_t]
        lib.oracle_decode_prep.argtypes = [_i, _i, _i, _i, _i, _f, _i, _l, _f32p, _f32p, _f32p, _f32p, _f32p,
                                           _f32p, _f32p, _f32p, _u16p, _u16p, _f32p, _i]
        lib.oracle_kv_cache_save.argtypes = [_i, _i32p, _i32p, _vpp, _vpp, _l, _i, _u8p, _l, _i]
        lib.oracle_kv_cache_save.restype = _l
        lib.oracle_kv_layer_save.argtypes = [_i, _i, _i, _vp, _vp, _l, _i, _u8p, _l]
        lib.oracle_kv_layer_save.restype = _l
        lib.oracle_kv_cache_load.argtypes = [_i, _i32p, _i32p, _u8p, _l, _vpp, _vpp, _l]
        lib.oracle_kv_cache_load.restype = _i
        lib.oracle_kv_layer_load.argtypes = [_i, _i32p, _i32p, _u8p, _l, _vpp, _vpp, _l, ctypes.POINTER(_i)]
        lib.oracle_kv_layer_load.restype = _i
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return REF_SO.exists()


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            raise RuntimeError(f"{REF_SO} missing: it is built from /root/reference by `make -C oracle ref`")
        lib = ctypes.CDLL(str(REF_SO))
        lib.ref_forward_cached_scores.argtypes = [_f32p, _f32p, _u16p, _u16p, _l, _i, _i, _i, _i, _f, _f, _i]
        lib.ref_forward_cached_scores.restype = _i
        lib.ref_time_cached_scores.argtypes = [_f32p, _f32p, _u16p, _u16p, _l, _i, _i, _i, _i, _f, _f, _i, _i]
        lib.ref_time_cached_scores.restype = ctypes.c_double
        lib.ref_kv_store_pack.argtypes = [_f32p, _f32p, _i, _i, _i, _u16p, _u16p]
        lib.ref_kv_store_pack.restype = _i
        lib.ref_kv_capacity_after.argtypes = [_i, _i]
        lib.ref_kv_capacity_after.restype = _l
        lib.ref_f32_to_f16_rne.argtypes = [_f]
        lib.ref_f32_to_f16_rne.restype = ctypes.c_uint16
        lib.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.ref_f16_to_f32.restype = _f
        lib.ref_rms_norm.argtypes = [_f32p, _f32p, _f32p, _l, _f]
        lib.ref_rope_apply.argtypes = [_f32p, _i, _i, _f, _i]
        lib.ref_kv_save_cache.argtypes = [_i, _i32p, _i32p, _i, _vpp, _vpp, _l, _i, _u8p, _l]
        lib.ref_kv_save_cache.restype = _l
        lib.ref_kv_save_file.argtypes = [ctypes.c_char_p, _i, _i32p, _i32p, _i, _vpp, _vpp, _l, _i]
        lib.ref_kv_save_file.restype = _i
        lib.ref_kv_save_layer.argtypes = [_i, _i32p, _i32p, _i, _vpp, _vpp, _l, _i, _i, _u8p, _l]
        lib.ref_kv_save_layer.restype = _l
        lib.ref_kv_load_cache.argtypes = [_i, _i32p, _i32p, _i, _u8p, _l, _vpp, _vpp, _l]
        lib.ref_kv_load_cache.restype = _i
        lib.ref_kv_load_layer.argtypes = [_i, _i32p, _i32p, _i, _u8p, _l, _vpp, _vpp, _l]
        lib.ref_kv_load_layer.restype = _i
        _ref = lib
    return _ref


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def attn_batch(q, k, v, *, n_kv_heads, n_ctx, q_base_pos, sliding_window=0, scale=0.0,
               softcap=0.0, n_threads=1):
    """Transformer::attn_batch_cpu restated.  q [nq, Hq, hd] f32; k, v [Hkv, stride, hd] u16."""
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    nq, hq, hd = q.shape
    sc = scale if scale > 0 else 1.0 / np.sqrt(hd)
    out = np.zeros_like(q)
    oracle().oracle_attn_batch(q, k, v, out, hq, n_kv_heads, hd, n_ctx, k.shape[1], nq, q_base_pos,
                               sliding_window, sc, softcap, n_threads)
    return out


def attn_batch_rows(q, k, v, rows, *, n_kv_heads, n_ctx, q_base_pos, scale=0.0, sliding_window=0, softcap=0.0,
                    n_threads=1):
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    nq, hq, hd = q.shape
    sc = scale if scale > 0 else 1.0 / np.sqrt(hd)
    out = np.zeros_like(q)
    rows = _c(rows, np.int32)
    oracle().oracle_attn_batch_rows(q, k, v, out, hq, n_kv_heads, hd, n_ctx, k.shape[1], nq, q_base_pos,
                                    sliding_window, sc, softcap, rows, len(rows), n_threads)
    return out


def cached_scores(q, k, v, *, n_kv_heads, pos, scale=0.0, softcap=0.0, n_threads=1):
    """AttentionLayer::forward_cached_scores restated.  q [Hq, hd]."""
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    hq, hd = q.shape
    out = np.zeros_like(q)
    oracle().oracle_cached_scores(q, out, k, v, k.shape[1], hq, n_kv_heads, hd, pos, scale, softcap, n_threads)
    return out


def ref_cached_scores(q, k, v, *, n_kv_heads, pos, scale=0.0, softcap=0.0, n_threads=1):
    """The reference's own forward_cached_scores (compiled from its sources)."""
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    hq, hd = q.shape
    out = np.zeros_like(q)
    rc = ref().ref_forward_cached_scores(q, out, k, v, k.shape[1], hq, n_kv_heads, hd, pos, scale,
                                         softcap, n_threads)
    assert rc == 0
    return out


def ref_time_cached_scores(q, k, v, *, n_kv_heads, pos, n_threads, reps, scale=0.0, softcap=0.0):
    """Seconds per call of the reference's own forward_cached_scores over a cache filled once."""
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    hq, hd = q.shape
    out = np.zeros_like(q)
    sec = ref().ref_time_cached_scores(q, out, k, v, k.shape[1], hq, n_kv_heads, hd, pos, scale, softcap,
                                       n_threads, reps)
    assert sec > 0
    return sec


def split_partials(q, k, v, *, n_kv_heads, n_ctx, q_base_pos, n_chunks, chunk, scale=0.0):
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    nq, hq, hd = q.shape
    sc = scale if scale > 0 else 1.0 / np.sqrt(hd)
    part = np.zeros((nq * hq, n_chunks, hd + 2), np.float32)
    oracle().oracle_split_partials(q, k, v, part, hq, n_kv_heads, hd, n_ctx, k.shape[1], nq, q_base_pos,
                                   sc, n_chunks, chunk)
    return part


def split_combine(part):
    part = _c(part, np.float32)
    rows, n_chunks, hd2 = part.shape
    out = np.zeros((rows, hd2 - 2), np.float32)
    oracle().oracle_split_combine(part, out, rows, hd2 - 2, n_chunks)
    return out


def gate_mul(out, gate):
    """out * sigmoid(gate) with the reference's clamp (oracle_gate_mul)."""
    out = _c(out, np.float32).copy()
    gate = _c(gate, np.float32)
    assert out.shape == gate.shape
    oracle().oracle_gate_mul(out.reshape(-1), gate.reshape(-1), out.size)
    return out


# decode-prep flags (qwen35_attn_prep.comp:7-8)
PREP_Q_ZC, PREP_K_ZC, PREP_NO_GATE, PREP_NO_QNORM, PREP_NO_KNORM, PREP_INTERLEAVED = 1, 2, 4, 8, 16, 32


def decode_prep(qg, kraw, vraw, qnw, knw, tab, *, n_heads, n_kv, hd, rot, flags, eps, pos, cap,
                kc=None, vc=None, rne=False):
    """One token of the decode prep (oracle_decode_prep).  Returns (q_out, gate_out, kc, vc,
    kv_out); kc/vc are [n_kv][cap][hd] f16 bit arrays (updated copies when given)."""
    assert 0 <= pos < cap, "the K/V row `pos` must lie inside the cap rows"
    qg, kraw, vraw = _c(qg, np.float32).reshape(-1), _c(kraw, np.float32).reshape(-1), _c(vraw, np.float32).reshape(-1)
    qnw = _c(qnw if qnw is not None else np.zeros(hd), np.float32)
    knw = _c(knw if knw is not None else np.zeros(hd), np.float32)
    tab = _c(tab, np.float32)
    q_out = np.zeros(n_heads * hd, np.float32)
    gate_out = np.zeros(n_heads * hd, np.float32)
    kc = np.zeros(n_kv * cap * hd, np.uint16) if kc is None else _c(kc, np.uint16).reshape(-1).copy()
    vc = np.zeros(n_kv * cap * hd, np.uint16) if vc is None else _c(vc, np.uint16).reshape(-1).copy()
    kv_out = np.zeros(2 * n_kv * hd, np.float32)
    oracle().oracle_decode_prep(n_heads, n_kv, hd, rot, flags, eps, pos, cap, qg, kraw, vraw, qnw, knw, tab,
                                q_out, gate_out, kc, vc, kv_out, 1 if rne else 0)
    return (q_out.reshape(n_heads, hd), gate_out.reshape(n_heads, hd), kc.reshape(n_kv, cap, hd),
            vc.reshape(n_kv, cap, hd), kv_out.reshape(2, n_kv, hd))


def ref_rms_norm(x, w, eps):
    x, w = _c(x, np.float32), _c(w, np.float32)
    y = np.zeros_like(x)
    ref().ref_rms_norm(x, w, y, x.size, eps)
    return y


def ref_rope(x, pos, head_dim, base, layout):
    x = _c(x, np.float32).copy()
    ref().ref_rope_apply(x, pos, head_dim, base, layout)
    return x


def naive_f64(q, k, v, *, n_kv_heads, n_ctx, q_base_pos, sliding_window=0, scale=0.0, softcap=0.0):
    q, k, v = _c(q, np.float32), _c(k, np.uint16), _c(v, np.uint16)
    nq, hq, hd = q.shape
    sc = scale if scale > 0 else 1.0 / np.sqrt(hd)
    out = np.zeros(q.shape, np.float64)
    oracle().oracle_naive_f64(q, k, v, out, hq, n_kv_heads, hd, n_ctx, k.shape[1], nq, q_base_pos,
                              sliding_window, sc, softcap)
    return out


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.sqrt(np.sum(b * b))
    return float(np.sqrt(np.sum((a - b) ** 2)) / max(den, 1e-30))


# ------------------------------------------------------------------ KV session formats

class KvCache:
    """A host-side multi-layer cache for the session-format checks: layer l holds K and V
    as uint16 [nh_l, stride, hd_l] (None for a layer without KV, or an empty slot)."""

    def __init__(self, geom, stride, k=None, v=None):
        self.geom = [(int(h), int(d)) for h, d in geom]
        self.stride = int(stride)
        n = len(self.geom)
        self.k = list(k) if k is not None else [None] * n
        self.v = list(v) if v is not None else [None] * n

    @classmethod
    def random(cls, geom, stride, seed, empty=()):
        rng = np.random.default_rng(seed)
        c = cls(geom, stride)
        for l, (h, d) in enumerate(c.geom):
            if h and l not in empty:
                c.k[l] = rng.integers(0, 1 << 16, (h, stride, d), dtype=np.uint16)
                c.v[l] = rng.integers(0, 1 << 16, (h, stride, d), dtype=np.uint16)
        return c

    @classmethod
    def zeros(cls, geom, stride):
        c = cls(geom, stride)
        for l, (h, d) in enumerate(c.geom):
            if h:
                c.k[l] = np.zeros((h, stride, d), np.uint16)
                c.v[l] = np.zeros((h, stride, d), np.uint16)
        return c

    def nh(self):
        return np.array([g[0] for g in self.geom], np.int32)

    def hd(self):
        return np.array([g[1] for g in self.geom], np.int32)

    def ptrs(self, which):
        arr = self.k if which == "k" else self.v
        out = (ctypes.c_void_p * len(arr))()
        for i, a in enumerate(arr):
            out[i] = None if a is None else a.ctypes.data
        return out


def kv_cache_save(c: KvCache, n_tok, legacy=False) -> bytes:
    lib = oracle()
    args = (len(c.geom), c.nh(), c.hd(), c.ptrs("k"), c.ptrs("v"), c.stride, n_tok)
    size = lib.oracle_kv_cache_save(*args, np.zeros(1, np.uint8), 0, int(legacy))
    out = np.zeros(size, np.uint8)
    assert lib.oracle_kv_cache_save(*args, out, size, int(legacy)) == size
    return out.tobytes()


def kv_layer_save(c: KvCache, layer, n_tok) -> bytes:
    lib = oracle()
    h, d = c.geom[layer]
    k = None if c.k[layer] is None else c.k[layer].ctypes.data
    v = None if c.v[layer] is None else c.v[layer].ctypes.data
    size = lib.oracle_kv_layer_save(layer, h, d, k, v, c.stride, n_tok, np.zeros(1, np.uint8), 0)
    out = np.zeros(max(size, 1), np.uint8)
    assert lib.oracle_kv_layer_save(layer, h, d, k, v, c.stride, n_tok, out, size) == size
    return out[:size].tobytes()


def kv_cache_load(data: bytes, geom, stride):
    """Returns (n_tok, KvCache) or (-1, None)."""
    c = KvCache.zeros(geom, stride)
    buf = np.frombuffer(data, np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    n = oracle().oracle_kv_cache_load(len(c.geom), c.nh(), c.hd(), buf, len(data), c.ptrs("k"), c.ptrs("v"), stride)
    return (n, c) if n >= 0 else (-1, None)


def kv_layer_load(data: bytes, geom, stride):
    """Returns (n_tok, layer, KvCache) or (-1, -1, None)."""
    c = KvCache.zeros(geom, stride)
    buf = np.frombuffer(data, np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    layer = ctypes.c_int(-1)
    n = oracle().oracle_kv_layer_load(len(c.geom), c.nh(), c.hd(), buf, len(data), c.ptrs("k"), c.ptrs("v"),
                                      stride, ctypes.byref(layer))
    return (n, layer.value, c) if n >= 0 else (-1, -1, None)


def ref_kv_save_cache(c: KvCache, n_tok, per_layer) -> bytes:
    lib = ref()
    args = (len(c.geom), c.nh(), c.hd(), int(per_layer), c.ptrs("k"), c.ptrs("v"), c.stride, n_tok)
    size = lib.ref_kv_save_cache(*args, np.zeros(1, np.uint8), 0)
    assert size >= 0
    out = np.zeros(size, np.uint8)
    assert lib.ref_kv_save_cache(*args, out, size) == size
    return out.tobytes()


def ref_kv_save_file(path, c: KvCache, n_tok, per_layer):
    assert ref().ref_kv_save_file(str(path).encode(), len(c.geom), c.nh(), c.hd(), int(per_layer), c.ptrs("k"),
                                  c.ptrs("v"), c.stride, n_tok) == 0


def ref_kv_save_layer(c: KvCache, layer, n_tok, per_layer) -> bytes:
    lib = ref()
    args = (len(c.geom), c.nh(), c.hd(), int(per_layer), c.ptrs("k"), c.ptrs("v"), c.stride, n_tok, layer)
    size = lib.ref_kv_save_layer(*args, np.zeros(1, np.uint8), 0)
    assert size >= 0
    out = np.zeros(max(size, 1), np.uint8)
    assert lib.ref_kv_save_layer(*args, out, size) == size
    return out[:size].tobytes()


def ref_kv_load_cache(data: bytes, geom, stride, per_layer):
    c = KvCache.zeros(geom, stride)
    buf = np.frombuffer(data, np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    n = ref().ref_kv_load_cache(len(c.geom), c.nh(), c.hd(), int(per_layer), buf, len(data), c.ptrs("k"),
                                c.ptrs("v"), stride)
    return (n, c) if n >= 0 else (-1, None)


def ref_kv_load_layer(data: bytes, geom, stride, per_layer):
    c = KvCache.zeros(geom, stride)
    buf = np.frombuffer(data, np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    n = ref().ref_kv_load_layer(len(c.geom), c.nh(), c.hd(), int(per_layer), buf, len(data), c.ptrs("k"),
                                c.ptrs("v"), stride)
    return (n, c) if n >= 0 else (-1, None)
