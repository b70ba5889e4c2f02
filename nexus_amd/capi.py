"""ctypes binding of the C ABI in include/nexus_hip_attn.h.

This is the Python side of the drop-in boundary: it loads the in-tree
libnexus_hip_attn.so and exposes the two entry points with device pointers.  There is
no fallback: if the library is missing, or a call is declined, an exception is raised.
torch is only used (in nexus_amd.ops) to own device memory and the stream.
"""
from __future__ import annotations

import ctypes
import math
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libnexus_hip_attn.so"

NEXUS_DT_F32 = 0
NEXUS_DT_F16 = 1

NEXUS_OK = 0
NEXUS_E_UNSUPPORTED = -1
NEXUS_E_INVALID = -2
NEXUS_E_WORKSPACE = -3
NEXUS_E_LAUNCH = -4
NEXUS_E_IO = -5

NEXUS_PLAN_PREFILL = 0
NEXUS_PLAN_DECODE = 1

# Every symbol include/*.h declares (checked by tests/test_capi.py).
EXPORTED_SYMBOLS = (
    "nexus_hip_attn_prefill",
    "nexus_hip_attn_prefill_ws_bytes",
    "nexus_hip_attn_prefill_plan",
    "nexus_hip_attn_decode",
    "nexus_hip_attn_decode_ws_bytes",
    "nexus_hip_attn_decode_default_splits",
    "nexus_hip_attn_prefill_gated",
    "nexus_hip_attn_decode_gated",
    "nexus_hip_attn_decode_prep",
    "nexus_hip_attn_decode_noalloc",
    "nexus_hip_attn_decode_layer",
    "nexus_hip_attn_decode_layer_ws_bytes",
    "nexus_hip_attn_decode_layer_default_splits",
    "nexus_hip_kv_layer_bytes",
    "nexus_hip_kv_cache_bytes",
    "nexus_hip_kv_layer_save",
    "nexus_hip_kv_layer_load",
    "nexus_hip_kv_cache_save",
    "nexus_hip_kv_cache_load",
    "nexus_hip_kv_cache_save_file",
    "nexus_hip_kv_cache_load_file",
    "nexus_hip_attn_last_error",
    "nexus_hip_attn_version",
)


class AttnDesc(ctypes.Structure):
    """struct nexus_attn_desc (include/nexus_hip_attn.h)."""

    _fields_ = [
        ("n_q_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("n_query", ctypes.c_int32),
        ("q_base_pos", ctypes.c_int32),
        ("n_ctx", ctypes.c_int32),
        ("kv_row_stride", ctypes.c_int64),
        ("sliding_window", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("q_dtype", ctypes.c_int32),
        ("o_dtype", ctypes.c_int32),
    ]


def make_desc(*, n_q_heads: int, n_kv_heads: int, head_dim: int, n_query: int, q_base_pos: int,
              n_ctx: int, kv_row_stride: int | None = None, sliding_window: int = 0,
              scale: float = 0.0, softcap: float = 0.0, q_dtype: int = NEXUS_DT_F32,
              o_dtype: int = NEXUS_DT_F32) -> AttnDesc:
    return AttnDesc(n_q_heads, n_kv_heads, head_dim, n_query, q_base_pos, n_ctx,
                    n_ctx if kv_row_stride is None else kv_row_stride, sliding_window,
                    scale, softcap, q_dtype, o_dtype)


# enum nexus_prep_flags
PREP_Q_NORM_ADD_ONE = 1
PREP_K_NORM_ADD_ONE = 2
PREP_NO_GATE = 4
PREP_NO_Q_NORM = 8
PREP_NO_K_NORM = 16
PREP_ROPE_INTERLEAVED = 32
PREP_TRUNC_STORE = 64


class PrefillPlan(ctypes.Structure):
    """struct nexus_attn_prefill_plan (include/nexus_hip_attn.h)."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("block_rows", ctypes.c_int32),
        ("splits", ctypes.c_int32),
        ("packed", ctypes.c_int32),
        ("workgroups", ctypes.c_int32),
    ]


class PrepDesc(ctypes.Structure):
    """struct nexus_attn_prep_desc (include/nexus_hip_attn.h)."""

    _fields_ = [
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rot_dims", ctypes.c_int32),
        ("pos", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("cap", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class KvLayerView(ctypes.Structure):
    """struct nexus_kv_layer_view (include/nexus_hip_kv.h)."""

    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("row_stride", ctypes.c_int64),
    ]


class NexusAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"nexus_hip_attn status {code}: {msg}")
        self.code = code


_lib = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the native library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"native library {p} is missing: run __graft_entry__.build() "
                           "(python -m nexus_amd.build) first")
    lib = ctypes.CDLL(str(p))
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    dp = ctypes.POINTER(AttnDesc)
    lib.nexus_hip_attn_prefill.argtypes = [dp, vp, vp, vp, vp, vp, sz, vp]
    lib.nexus_hip_attn_prefill.restype = ctypes.c_int
    lib.nexus_hip_attn_prefill_ws_bytes.argtypes = [dp]
    lib.nexus_hip_attn_prefill_ws_bytes.restype = sz
    lib.nexus_hip_attn_prefill_plan.argtypes = [dp, ctypes.POINTER(PrefillPlan)]
    lib.nexus_hip_attn_prefill_plan.restype = ctypes.c_int
    lib.nexus_hip_attn_decode.argtypes = [dp, vp, vp, vp, vp, vp, ctypes.c_int, vp]
    lib.nexus_hip_attn_decode.restype = ctypes.c_int
    lib.nexus_hip_attn_decode_ws_bytes.argtypes = [dp, ctypes.c_int]
    lib.nexus_hip_attn_decode_ws_bytes.restype = sz
    lib.nexus_hip_attn_decode_default_splits.argtypes = [dp]
    lib.nexus_hip_attn_decode_default_splits.restype = ctypes.c_int
    lib.nexus_hip_attn_prefill_gated.argtypes = [dp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.nexus_hip_attn_prefill_gated.restype = ctypes.c_int
    lib.nexus_hip_attn_decode_gated.argtypes = [dp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp]
    lib.nexus_hip_attn_decode_gated.restype = ctypes.c_int
    lib.nexus_hip_attn_decode_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, ctypes.c_int, vp]
    lib.nexus_hip_attn_decode_noalloc.restype = ctypes.c_int
    lib.nexus_hip_attn_decode_prep.argtypes = [ctypes.POINTER(PrepDesc)] + [vp] * 12
    lib.nexus_hip_attn_decode_prep.restype = ctypes.c_int
    pdp = ctypes.POINTER(PrepDesc)
    lib.nexus_hip_attn_decode_layer.argtypes = [pdp, ctypes.c_float] + [vp] * 11 + [ctypes.c_int, vp]
    lib.nexus_hip_attn_decode_layer.restype = ctypes.c_int
    lib.nexus_hip_attn_decode_layer_ws_bytes.argtypes = [pdp, ctypes.c_int]
    lib.nexus_hip_attn_decode_layer_ws_bytes.restype = sz
    lib.nexus_hip_attn_decode_layer_default_splits.argtypes = [pdp]
    lib.nexus_hip_attn_decode_layer_default_splits.restype = ctypes.c_int
    kvp = ctypes.POINTER(KvLayerView)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.nexus_hip_kv_layer_bytes.argtypes = [kvp, ctypes.c_int]
    lib.nexus_hip_kv_layer_bytes.restype = sz
    lib.nexus_hip_kv_cache_bytes.argtypes = [kvp, ctypes.c_int, ctypes.c_int]
    lib.nexus_hip_kv_cache_bytes.restype = sz
    lib.nexus_hip_kv_layer_save.argtypes = [ctypes.c_int, kvp, ctypes.c_int, vp, sz, vp]
    lib.nexus_hip_kv_layer_load.argtypes = [vp, sz, kvp, ctypes.c_int, ip, ip, vp]
    lib.nexus_hip_kv_cache_save.argtypes = [kvp, ctypes.c_int, ctypes.c_int, vp, sz, vp]
    lib.nexus_hip_kv_cache_load.argtypes = [vp, sz, kvp, ctypes.c_int, ip, vp]
    lib.nexus_hip_kv_cache_save_file.argtypes = [ctypes.c_char_p, kvp, ctypes.c_int, ctypes.c_int, vp]
    lib.nexus_hip_kv_cache_load_file.argtypes = [ctypes.c_char_p, kvp, ctypes.c_int, ip, vp]
    for name in ("nexus_hip_kv_layer_save", "nexus_hip_kv_layer_load", "nexus_hip_kv_cache_save",
                 "nexus_hip_kv_cache_load", "nexus_hip_kv_cache_save_file", "nexus_hip_kv_cache_load_file"):
        getattr(lib, name).restype = ctypes.c_int
    lib.nexus_hip_attn_last_error.argtypes = []
    lib.nexus_hip_attn_last_error.restype = ctypes.c_char_p
    lib.nexus_hip_attn_version.argtypes = []
    lib.nexus_hip_attn_version.restype = ctypes.c_char_p
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    return load().nexus_hip_attn_last_error().decode()


def version() -> str:
    return load().nexus_hip_attn_version().decode()


def _check(rc: int) -> int:
    if rc != NEXUS_OK:
        raise NexusAttnError(rc, last_error())
    return rc


def prefill_ws_bytes(desc: AttnDesc) -> int:
    return int(load().nexus_hip_attn_prefill_ws_bytes(ctypes.byref(desc)))


def prefill_plan(desc: AttnDesc) -> dict:
    """The launch plan of nexus_hip_attn_prefill for `desc` (with its full workspace) on the
    current device, 256 compute units without one: kernel ("prefill" or "decode"), block_rows,
    splits, packed, workgroups."""
    p = PrefillPlan()
    _check(load().nexus_hip_attn_prefill_plan(ctypes.byref(desc), ctypes.byref(p)))
    return {"kernel": "decode" if p.kernel == NEXUS_PLAN_DECODE else "prefill", "block_rows": p.block_rows,
            "splits": p.splits, "packed": bool(p.packed), "workgroups": p.workgroups}


def decode_ws_bytes(desc: AttnDesc, n_splits: int = 0) -> int:
    return int(load().nexus_hip_attn_decode_ws_bytes(ctypes.byref(desc), int(n_splits)))


def unpack_partials(ws, n_rows: int, n_splits: int, head_dim: int):
    """The split partials in a decode workspace (a flat float32 array) as
    [n_rows][n_splits][head_dim + 2] = (acc, m, l) per row and split, the reference's
    partial (qwen35_attn_part.comp:3).  The library stores acc as [split][row][head_dim]
    followed by (m, l) as [split][row][2]."""
    import numpy as np

    ws = np.asarray(ws, dtype=np.float32).reshape(-1)
    n_acc = n_splits * n_rows * head_dim
    acc = ws[:n_acc].reshape(n_splits, n_rows, head_dim)
    ml = ws[n_acc:n_acc + 2 * n_splits * n_rows].reshape(n_splits, n_rows, 2)
    return np.concatenate([acc, ml], axis=2).transpose(1, 0, 2).copy()


def decode_default_splits(desc: AttnDesc) -> int:
    return int(load().nexus_hip_attn_decode_default_splits(ctypes.byref(desc)))


def prefill_raw(desc: AttnDesc, q: int, k: int, v: int, out: int, ws: int, ws_bytes: int,
                stream: int, check: bool = True, gate: int = 0) -> int:
    lib = load()
    if gate:
        rc = lib.nexus_hip_attn_prefill_gated(ctypes.byref(desc), q, k, v, gate, out, ws, ws_bytes, stream)
    else:
        rc = lib.nexus_hip_attn_prefill(ctypes.byref(desc), q, k, v, out, ws, ws_bytes, stream)
    return _check(rc) if check else rc


def decode_raw(desc: AttnDesc, q: int, k: int, v: int, out: int, ws: int, n_splits: int,
               stream: int, check: bool = True, gate: int = 0) -> int:
    lib = load()
    if gate:
        rc = lib.nexus_hip_attn_decode_gated(ctypes.byref(desc), q, k, v, gate, out, ws, int(n_splits), stream)
    else:
        rc = lib.nexus_hip_attn_decode(ctypes.byref(desc), q, k, v, out, ws, int(n_splits), stream)
    return _check(rc) if check else rc


# Size of the device array behind nexus_hip_attn_decode_noalloc (include/nexus_hip_attn.h).
DECODE_NOALLOC_SCRATCH_BYTES = 8 << 20


def decode_noalloc_raw(desc: AttnDesc, q: int, k: int, v: int, out: int, n_splits: int, stream: int,
                       check: bool = True, gate: int = 0) -> int:
    """nexus_hip_attn_decode_noalloc: the gated decode with the library's fixed partial array."""
    rc = load().nexus_hip_attn_decode_noalloc(ctypes.byref(desc), q, k, v, gate or None, out, int(n_splits), stream)
    return _check(rc) if check else rc


def decode_prep_raw(desc: PrepDesc, qg: int, k_raw: int, v_raw: int, q_norm_w: int, k_norm_w: int,
                    rope_tab: int, q_out: int, gate_out: int, k_cache: int, v_cache: int, kv_out: int,
                    stream: int, check: bool = True) -> int:
    rc = load().nexus_hip_attn_decode_prep(ctypes.byref(desc), qg, k_raw, v_raw, q_norm_w, k_norm_w, rope_tab,
                                           q_out, gate_out, k_cache, v_cache, kv_out, stream)
    return _check(rc) if check else rc


def decode_layer_raw(desc: PrepDesc, scale: float, qg: int, k_raw: int, v_raw: int, q_norm_w: int, k_norm_w: int,
                     rope_tab: int, k_cache: int, v_cache: int, kv_out: int, out: int, ws: int, n_splits: int,
                     stream: int, check: bool = True) -> int:
    """nexus_hip_attn_decode_layer: prep and gated split-KV decode of one token in two launches."""
    rc = load().nexus_hip_attn_decode_layer(ctypes.byref(desc), float(scale), qg, k_raw, v_raw, q_norm_w, k_norm_w,
                                            rope_tab, k_cache, v_cache, kv_out, out, ws, int(n_splits), stream)
    return _check(rc) if check else rc


def decode_layer_ws_bytes(desc: PrepDesc, n_splits: int = 0) -> int:
    return int(load().nexus_hip_attn_decode_layer_ws_bytes(ctypes.byref(desc), int(n_splits)))


def decode_layer_default_splits(desc: PrepDesc) -> int:
    return int(load().nexus_hip_attn_decode_layer_default_splits(ctypes.byref(desc)))


def prefill_flops(n_q_heads: int, head_dim: int, n_query: int, q_base_pos: int, n_ctx: int,
                  sliding_window: int = 0) -> float:
    """Algorithmic FLOPs of a causal prefill: 4*hd per visible (query, key) pair per head."""
    pairs = 0
    for i in range(n_query):
        qpos = q_base_pos + i
        last = min(qpos, n_ctx - 1)
        start = qpos + 1 - sliding_window if (sliding_window > 0 and qpos + 1 > sliding_window) else 0
        pairs += max(0, last - start + 1)
    return 4.0 * head_dim * n_q_heads * pairs


def decode_bytes(n_kv_heads: int, head_dim: int, n_keys: int, n_q_heads: int, n_query: int,
                 q_bytes: int = 4, o_bytes: int = 4) -> float:
    """Algorithmic HBM bytes of a decode: K and V of every visible key once, plus Q and O."""
    return (2.0 * n_kv_heads * n_keys * head_dim * 2
            + n_query * n_q_heads * head_dim * (q_bytes + o_bytes))


def decode_prep_bytes(n_heads: int, n_kv_heads: int, head_dim: int, gated: bool, q_norm: bool,
                      k_norm: bool, rot_dims: int) -> float:
    """Algorithmic HBM bytes of one decode prep: every input read once, every output written
    once (q/gate/k/v in f32, the two f16 cache rows, the f32 K/V echo, weights and table)."""
    q_in = n_heads * head_dim * 4 * (2 if gated else 1)
    kv_in = 2 * n_kv_heads * head_dim * 4
    w = head_dim * 4 * (int(q_norm) + int(k_norm)) + rot_dims * 4
    q_out = n_heads * head_dim * 4 * (2 if gated else 1)
    kv_out = 2 * n_kv_heads * head_dim * (2 + 4)
    return float(q_in + kv_in + w + q_out + kv_out)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
