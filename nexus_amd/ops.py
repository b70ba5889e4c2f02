"""torch-facing wrappers over the C ABI (device memory and the stream come from torch).

    out = attn_prefill(q, k, v, n_kv_heads=..., q_base_pos=..., n_ctx=...)
    out = attn_decode(q, k, v, n_kv_heads=..., q_base_pos=..., n_ctx=..., n_splits=64)

Tensors:  q [n_query, n_q_heads, head_dim] f32 or f16;  k, v [n_kv_heads, stride, head_dim]
f16 (the KV cache layout); out [n_query, n_q_heads, head_dim] f32 or f16.  Everything must
live on a HIP device: there is no CPU path here, a declined call raises NexusAttnError.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import capi

_DT = {torch.float32: capi.NEXUS_DT_F32, torch.float16: capi.NEXUS_DT_F16}


def _kv_view(x: torch.Tensor) -> torch.Tensor:
    if x.dtype in (torch.int16, torch.uint16):
        return x
    if x.dtype != torch.float16:
        raise TypeError(f"K/V must be float16 (f16 bit patterns), got {x.dtype}")
    return x


def _check_tensors(q, k, v, n_kv_heads):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a device tensor (no CPU path)")
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be [n_query, Hq, hd], k/v [Hkv, stride, hd]")
    if q.dtype not in _DT:
        raise TypeError(f"q dtype {q.dtype} not supported")
    if k.shape != v.shape or k.shape[0] != n_kv_heads or k.shape[2] != q.shape[2]:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match Hkv={n_kv_heads}, hd={q.shape[2]}")
    _kv_view(k), _kv_view(v)


def make_desc_for(q: torch.Tensor, k: torch.Tensor, *, n_kv_heads: int, q_base_pos: int, n_ctx: int,
                  sliding_window: int = 0, scale: float = 0.0, softcap: float = 0.0,
                  out_dtype: torch.dtype | None = None) -> capi.AttnDesc:
    od = out_dtype if out_dtype is not None else q.dtype
    return capi.make_desc(n_q_heads=q.shape[1], n_kv_heads=n_kv_heads, head_dim=q.shape[2],
                          n_query=q.shape[0], q_base_pos=q_base_pos, n_ctx=n_ctx,
                          kv_row_stride=k.shape[1], sliding_window=sliding_window, scale=scale,
                          softcap=softcap, q_dtype=_DT[q.dtype], o_dtype=_DT[od])


def _check_out(out: torch.Tensor, q: torch.Tensor) -> None:
    """A caller-supplied output must be exactly what the kernels write: a contiguous tensor
    shaped like q on q's device, f32 or f16 (the kernels store n_query * Hq * hd elements)."""
    if not isinstance(out, torch.Tensor) or not out.is_cuda or out.device != q.device:
        raise ValueError("out must be a device tensor on q's device")
    if out.dtype not in _DT:
        raise ValueError(f"out dtype {out.dtype} not supported (float32 or float16)")
    if tuple(out.shape) != tuple(q.shape) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous and shaped like q {tuple(q.shape)}, got {tuple(out.shape)}")


def _gate_ptr(gate: torch.Tensor | None, q: torch.Tensor) -> int:
    if gate is None:
        return 0
    if gate.dtype != torch.float32 or gate.shape != q.shape or not gate.is_contiguous() or gate.device != q.device:
        raise ValueError("gate must be a contiguous float32 tensor shaped like q on q's device")
    return gate.data_ptr()


def attn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, n_kv_heads: int,
                 q_base_pos: int, n_ctx: int, sliding_window: int = 0, scale: float = 0.0,
                 softcap: float = 0.0, out: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None,
                 workspace: torch.Tensor | None = None, split: bool = True,
                 gate: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA prefill (nexus_hip_attn_prefill); `gate` (f32, q's shape) multiplies the
    output by sigmoid(gate) clamped at +-80 (nexus_hip_attn_prefill_gated)."""
    _check_tensors(q, k, v, n_kv_heads)
    gate_ptr = _gate_ptr(gate, q)
    if out is not None:
        _check_out(out, q)
    desc = make_desc_for(q, k, n_kv_heads=n_kv_heads, q_base_pos=q_base_pos, n_ctx=n_ctx,
                         sliding_window=sliding_window, scale=scale, softcap=softcap,
                         out_dtype=out_dtype if out is None else out.dtype)
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    ws_ptr, ws_bytes = 0, 0
    if split:
        need = capi.prefill_ws_bytes(desc)
        if need > 0:
            if workspace is None or workspace.numel() * workspace.element_size() < need:
                workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    capi.prefill_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws_ptr,
                     ws_bytes, stream, gate=gate_ptr)
    return out


def attn_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, n_kv_heads: int,
                q_base_pos: int, n_ctx: int, n_splits: int = 0, sliding_window: int = 0,
                scale: float = 0.0, softcap: float = 0.0, out: torch.Tensor | None = None,
                out_dtype: torch.dtype | None = None,
                partial_ws: torch.Tensor | None = None,
                gate: torch.Tensor | None = None) -> torch.Tensor:
    """Split-KV decode / verify (nexus_hip_attn_decode); `gate` as in attn_prefill."""
    _check_tensors(q, k, v, n_kv_heads)
    gate_ptr = _gate_ptr(gate, q)
    if out is not None:
        _check_out(out, q)
    desc = make_desc_for(q, k, n_kv_heads=n_kv_heads, q_base_pos=q_base_pos, n_ctx=n_ctx,
                         sliding_window=sliding_window, scale=scale, softcap=softcap,
                         out_dtype=out.dtype if out is not None else (out_dtype or torch.float32))
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or torch.float32, device=q.device)
    need = capi.decode_ws_bytes(desc, n_splits)
    if need <= 0:
        raise capi.NexusAttnError(capi.NEXUS_E_UNSUPPORTED, capi.last_error() or "bad shape")
    if partial_ws is None or partial_ws.numel() * partial_ws.element_size() < need:
        partial_ws = torch.empty(need // 4, dtype=torch.float32, device=q.device)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    capi.decode_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                    partial_ws.data_ptr(), n_splits, stream, gate=gate_ptr)
    return out


def decode_prep(qg: torch.Tensor, k_raw: torch.Tensor, v_raw: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, *, pos: int, rope_tab: torch.Tensor | None,
                q_norm_w: torch.Tensor | None = None, k_norm_w: torch.Tensor | None = None,
                gated: bool = True, q_norm_add_one: bool = False, k_norm_add_one: bool = False,
                rope_interleaved: bool = False, eps: float = 1e-6, trunc_store: bool = False,
                q_out: torch.Tensor | None = None, gate_out: torch.Tensor | None = None,
                kv_out: torch.Tensor | None = None):
    """One token's decode prep (nexus_hip_attn_decode_prep): q/k head norms (a weight of None
    turns that norm off), RoPE over rope_tab.numel() dims, K/V stored into row `pos` of
    k_cache/v_cache [n_kv, cap, hd] (f16).  qg is [n_heads, 2*hd] (q | gate) when gated,
    else [n_heads, hd]; k_raw/v_raw [n_kv, hd]; all f32.  Returns (q_out [n_heads, hd],
    gate_out [n_heads, hd] or None, kv_out [2, n_kv, hd])."""
    desc = _prep_desc(qg, k_raw, v_raw, k_cache, v_cache, pos=pos, rope_tab=rope_tab, q_norm_w=q_norm_w,
                      k_norm_w=k_norm_w, gated=gated, q_norm_add_one=q_norm_add_one, k_norm_add_one=k_norm_add_one,
                      rope_interleaved=rope_interleaved, eps=eps, trunc_store=trunc_store)
    n_heads, n_kv, hd = desc.n_heads, desc.n_kv_heads, desc.head_dim
    dev = qg.device
    q_out = torch.empty(n_heads, hd, dtype=torch.float32, device=dev) if q_out is None else q_out
    if gated and gate_out is None:
        gate_out = torch.empty(n_heads, hd, dtype=torch.float32, device=dev)
    kv_out = torch.empty(2, n_kv, hd, dtype=torch.float32, device=dev) if kv_out is None else kv_out
    ptr = lambda t: 0 if t is None else t.data_ptr()
    capi.decode_prep_raw(desc, qg.data_ptr(), k_raw.data_ptr(), v_raw.data_ptr(), ptr(q_norm_w), ptr(k_norm_w),
                         ptr(rope_tab), q_out.data_ptr(), ptr(gate_out if gated else None), k_cache.data_ptr(),
                         v_cache.data_ptr(), kv_out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return q_out, (gate_out if gated else None), kv_out


def _prep_desc(qg, k_raw, v_raw, k_cache, v_cache, *, pos, rope_tab, q_norm_w, k_norm_w, gated, q_norm_add_one,
               k_norm_add_one, rope_interleaved, eps, trunc_store):
    n_kv, cap, hd = k_cache.shape
    n_heads = qg.shape[0]
    f32 = [("qg", qg), ("k_raw", k_raw), ("v_raw", v_raw)]
    f32 += [(n, t) for n, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("rope_tab", rope_tab)) if t is not None]
    for name, t in f32 + [("k_cache", k_cache), ("v_cache", v_cache)]:
        if not t.is_cuda or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous device tensor (no CPU path)")
    for name, t in f32:
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32, got {t.dtype}")
    _kv_view(k_cache), _kv_view(v_cache)
    if qg.shape != (n_heads, (2 if gated else 1) * hd) or k_raw.shape != (n_kv, hd) or v_raw.shape != (n_kv, hd):
        raise ValueError(f"qg {tuple(qg.shape)} / k_raw {tuple(k_raw.shape)} do not match n_kv={n_kv} hd={hd}")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache differ in shape")
    flags = ((capi.PREP_Q_NORM_ADD_ONE if q_norm_add_one else 0) | (capi.PREP_K_NORM_ADD_ONE if k_norm_add_one else 0)
             | (0 if gated else capi.PREP_NO_GATE) | (capi.PREP_NO_Q_NORM if q_norm_w is None else 0)
             | (capi.PREP_NO_K_NORM if k_norm_w is None else 0)
             | (capi.PREP_ROPE_INTERLEAVED if rope_interleaved else 0) | (capi.PREP_TRUNC_STORE if trunc_store else 0))
    rot = 0 if rope_tab is None else rope_tab.numel()
    return capi.PrepDesc(n_heads, n_kv, hd, rot, pos, flags, cap, eps, 0)


def decode_layer(qg: torch.Tensor, k_raw: torch.Tensor, v_raw: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, *, pos: int, rope_tab: torch.Tensor | None,
                 q_norm_w: torch.Tensor | None = None, k_norm_w: torch.Tensor | None = None,
                 gated: bool = True, q_norm_add_one: bool = False, k_norm_add_one: bool = False,
                 rope_interleaved: bool = False, eps: float = 1e-6, trunc_store: bool = False,
                 scale: float = 0.0, n_splits: int = 0, out: torch.Tensor | None = None,
                 kv_out: torch.Tensor | None = None, partial_ws: torch.Tensor | None = None):
    """The attention of one decode token with its prep (nexus_hip_attn_decode_layer): the
    arguments of decode_prep, plus the scale (0: 1/sqrt(hd)) and the split count (0: the
    library's choice).  Row `pos` of the caches is written; rows [0, pos] are attended.
    Returns (out [n_heads, hd] gated attention output, kv_out [2, n_kv, hd])."""
    desc = _prep_desc(qg, k_raw, v_raw, k_cache, v_cache, pos=pos, rope_tab=rope_tab, q_norm_w=q_norm_w,
                      k_norm_w=k_norm_w, gated=gated, q_norm_add_one=q_norm_add_one, k_norm_add_one=k_norm_add_one,
                      rope_interleaved=rope_interleaved, eps=eps, trunc_store=trunc_store)
    n_heads, n_kv, hd = desc.n_heads, desc.n_kv_heads, desc.head_dim
    dev = qg.device
    for name, t, shape in (("out", out, (n_heads, hd)), ("kv_out", kv_out, (2, n_kv, hd))):
        if t is not None and (t.device != dev or t.dtype != torch.float32 or not t.is_contiguous()
                              or tuple(t.shape) != shape):
            raise ValueError(f"{name} must be a contiguous float32 {shape} tensor on {dev}")
    out = torch.empty(n_heads, hd, dtype=torch.float32, device=dev) if out is None else out
    kv_out = torch.empty(2, n_kv, hd, dtype=torch.float32, device=dev) if kv_out is None else kv_out
    splits = n_splits if n_splits > 0 else capi.decode_layer_default_splits(desc)
    need = capi.decode_layer_ws_bytes(desc, splits)
    if need == 0:
        raise ValueError(capi.last_error() or "unsupported decode layer shape")
    if partial_ws is None or partial_ws.numel() * partial_ws.element_size() < need:
        partial_ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
    ptr = lambda t: 0 if t is None else t.data_ptr()
    capi.decode_layer_raw(desc, scale, qg.data_ptr(), k_raw.data_ptr(), v_raw.data_ptr(), ptr(q_norm_w),
                          ptr(k_norm_w), ptr(rope_tab), k_cache.data_ptr(), v_cache.data_ptr(), kv_out.data_ptr(),
                          out.data_ptr(), partial_ws.data_ptr(), splits, torch.cuda.current_stream(dev).cuda_stream)
    return out, kv_out


# ------------------------------------------------------------------ KV session files

def _kv_views(layers):
    """layers: per model layer, (k, v) device tensors [n_kv, row_stride, hd] of f16 bits, or
    None for a layer without KV."""
    arr = (capi.KvLayerView * len(layers))()
    dev = None
    for i, lv in enumerate(layers):
        if lv is None:
            arr[i] = capi.KvLayerView(None, None, 0, 0, 0)
            continue
        k, v = lv
        for name, t in (("k", k), ("v", v)):
            if not t.is_cuda or not t.is_contiguous() or t.dim() != 3:
                raise RuntimeError(f"layer {i} {name}: a contiguous [n_kv, row_stride, hd] device tensor is needed")
            _kv_view(t)
        if k.shape != v.shape:
            raise ValueError(f"layer {i}: k {tuple(k.shape)} and v {tuple(v.shape)} differ")
        dev = k.device
        arr[i] = capi.KvLayerView(k.data_ptr(), v.data_ptr(), k.shape[0], k.shape[2], k.shape[1])
    return arr, dev


def _kv_stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream if dev is not None else None


def kv_cache_bytes(layers, n_tokens: int) -> int:
    views, _ = _kv_views(layers)
    return int(capi.load().nexus_hip_kv_cache_bytes(views, len(layers), n_tokens))


def kv_cache_save(layers, n_tokens: int):
    """NXKVCACH image of rows [0, n_tokens) (KVCache::save_to_buffer) as a uint8 numpy array."""
    views, dev = _kv_views(layers)
    lib = capi.load()
    buf = np.empty(lib.nexus_hip_kv_cache_bytes(views, len(layers), n_tokens), np.uint8)
    capi._check(lib.nexus_hip_kv_cache_save(views, len(layers), n_tokens, buf.ctypes.data, buf.nbytes,
                                            _kv_stream(dev)))
    return buf


def kv_cache_load(data, layers) -> int:
    """Apply an NXKVCACH image (KVCache::load_from_buffer); returns its token count."""
    buf = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, np.uint8)
    views, dev = _kv_views(layers)
    n = ctypes.c_int(0)
    capi._check(capi.load().nexus_hip_kv_cache_load(buf.ctypes.data, buf.nbytes, views, len(layers), n,
                                                    _kv_stream(dev)))
    return n.value


def kv_layer_save(layer: int, k: torch.Tensor, v: torch.Tensor, n_tokens: int):
    """NXKVLYR1 record of one layer (KVCache::save_layer_to_buffer) as a uint8 numpy array."""
    views, dev = _kv_views([(k, v)])
    lib = capi.load()
    size = lib.nexus_hip_kv_layer_bytes(views, n_tokens)
    buf = np.empty(max(1, size), np.uint8)
    capi._check(lib.nexus_hip_kv_layer_save(layer, views, n_tokens, buf.ctypes.data, size, _kv_stream(dev)))
    return buf[:size]


def kv_layer_load(data, layers) -> tuple[int, int]:
    """Apply an NXKVLYR1 record (KVCache::load_layer_from_buffer); returns (layer, n_tokens)."""
    buf = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, np.uint8)
    views, dev = _kv_views(layers)
    layer, n = ctypes.c_int(0), ctypes.c_int(0)
    capi._check(capi.load().nexus_hip_kv_layer_load(buf.ctypes.data, buf.nbytes, views, len(layers), layer, n,
                                                    _kv_stream(dev)))
    return layer.value, n.value


def kv_cache_save_file(path, layers, n_tokens: int) -> None:
    """KVCache::save(path) from device memory, streamed through pinned staging."""
    views, dev = _kv_views(layers)
    capi._check(capi.load().nexus_hip_kv_cache_save_file(str(path).encode(), views, len(layers), n_tokens,
                                                         _kv_stream(dev)))


def kv_cache_load_file(path, layers) -> int:
    """KVCache::load(path) straight into device memory; returns the token count."""
    views, dev = _kv_views(layers)
    n = ctypes.c_int(0)
    capi._check(capi.load().nexus_hip_kv_cache_load_file(str(path).encode(), views, len(layers), n,
                                                         _kv_stream(dev)))
    return n.value
