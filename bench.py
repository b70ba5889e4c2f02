#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline: chunked causal GQA prefill, 512 queries appended
after 4096 cached tokens, 40 q / 8 kv heads, head_dim 128, f16 Q/K/V/O, f32 accumulate.
A step is one call of nexus_hip_attn_prefill over that batch with inputs resident in HBM.
value = algorithmic TFLOP/s (4*hd per visible (query, key) pair per head).

The other BASELINE configs are reported under "extra" with their own roofline: cold 8192
prefill (MFMA), decode at 4096 and 61440 keys (HBM), and 4-draft speculative verify (HBM).
Decode inputs rotate over enough K/V copies to exceed the 256 MB Infinity Cache.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only cfgN] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20
WARM_S = 0.03                    # minimum warm-up time per measured config

METRIC = "attn prefill TFLOP/s (% MFMA peak) + decode KV GB/s (% HBM peak), 1 MI355X"

CONFIGS = {
    "cfg1": dict(kind="decode", hq=16, hkv=4, hd=128, nq=1, base=4095, n_ctx=4096, q="f32", o="f32", splits=0,
                 desc="decode 1 token, 16q/4kv, hd128, 4096 keys, f32 Q/O, f16 KV"),
    "cfg2": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=512, base=4096, n_ctx=4608, q="f16", o="f16",
                 desc="chunked prefill 512 queries after 4096 cached tokens, 40q/8kv, hd128, f16 Q/K/V/O, f32 accumulate"),
    "cfg3": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=8192, base=0, n_ctx=8192, q="f16", o="f16",
                 desc="cold prefill 8192 tokens, 40q/8kv, hd128, f16 Q/K/V/O, f32 softmax stats"),
    "cfg4": dict(kind="decode", hq=40, hkv=8, hd=128, nq=1, base=61439, n_ctx=61440, q="f32", o="f32", splits=64,
                 desc="decode 1 token, 40q/8kv, hd128, 61440 keys, 64 splits, f32 LSE combine"),
    "q35p": dict(kind="prefill", hq=16, hkv=2, hd=256, nq=8192, base=0, n_ctx=8192, q="f16", o="f16",
                 desc="cold prefill 8192 tokens, 16q/2kv, hd256 (the Qwen3.5 full-attention layer's shape)"),
    "cfg2q32": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=512, base=4096, n_ctx=4608, q="f32", o="f32",
                    desc="cfg2's shape with f32 Q and f32 out (the engine's attention_flash_gpu form: Q as an f16 high "
                         "part plus its f16 residual)"),
    "cap2": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=512, base=4096, n_ctx=4608, q="f16", o="f16", cap=30.0,
                 desc="cfg2's shape with logit softcap 30 (Gemma-style), f16 Q/K/V/O"),
    "swa3": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=8192, base=0, n_ctx=8192, q="f16", o="f16", sw=4096,
                 desc="cfg3's shape with a 4096-token sliding window (work counted over visible pairs)"),
    "q35c": dict(kind="prefill", hq=16, hkv=2, hd=256, nq=512, base=32768, n_ctx=33280, q="f16", o="f16",
                 desc="chunked prefill 512 queries after 32768 cached tokens, 16q/2kv, hd256 (key splits + combine)"),
    "tile3": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=1024, base=3072, n_ctx=4096, q="f16", o="f16",
                  desc="the engine's 1024-token prompt tile (transformer.h:8551-8560) after 3072 cached tokens, "
                       "40q/8kv, hd128"),
    "q35t3": dict(kind="prefill", hq=16, hkv=2, hd=256, nq=1024, base=3072, n_ctx=4096, q="f16", o="f16",
                  desc="the engine's 1024-token prompt tile after 3072 cached tokens, 16q/2kv, hd256 (key splits)"),
    # short chunks behind a long cache read more K/V than they compute on: timed with the K/V
    # rotated past the Infinity Cache like the decode configs
    "c64": dict(kind="prefill", hq=40, hkv=8, hd=128, nq=64, base=32768, n_ctx=32832, q="f16", o="f16", kvrot=True,
                desc="a 64-query chunk after 32768 cached tokens, 40q/8kv, hd128 (64-row blocks in key splits)"),
    "q35s": dict(kind="prefill", hq=16, hkv=2, hd=256, nq=160, base=32768, n_ctx=32928, q="f16", o="f16", kvrot=True,
                 desc="a 160-query chunk after 32768 cached tokens, 16q/2kv, hd256 (packed rows in key splits)"),
    "cfg5": dict(kind="verify", hq=16, hkv=2, hd=256, nq=4, base=32768, n_ctx=32772, q="f32", o="f32", splits=0,
                 desc="MTP verify 4 drafts at 32768 cached tokens, 16q/2kv, hd256, causal among drafts"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def work_of(c: dict) -> tuple[float, str]:
    from nexus_amd import capi

    if c["kind"] == "prefill":
        return capi.prefill_flops(c["hq"], c["hd"], c["nq"], c["base"], c["n_ctx"], c.get("sw", 0)), "flop"
    n_keys = min(c["base"] + c["nq"] - 1, c["n_ctx"] - 1) + 1
    return capi.decode_bytes(c["hkv"], c["hd"], n_keys, c["hq"], c["nq"]), "byte"


def warm_up(call, warmup: int, min_s: float = WARM_S) -> None:
    """At least `warmup` untimed calls, and more until `min_s` seconds of back-to-back work have
    passed: the GPU's clocks settle under sustained load of the kind timed next (measured on
    MI355X: cfg2 launches take ~70 us in the first milliseconds after idle, ~62-66 us later)."""
    import torch

    t_end = time.perf_counter() + min_s
    i = 0
    while i < warmup or time.perf_counter() < t_end:
        call(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def measure(name: str, steps: int, warmup: int, graph: bool = False, rotate: bool = True,
            check: bool = False) -> dict:
    import torch

    from nexus_amd import capi

    c = CONFIGS[name]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    qdt = torch.float16 if c["q"] == "f16" else torch.float32
    odt = torch.float16 if c["o"] == "f16" else torch.float32
    q = torch.randn(c["nq"], c["hq"], c["hd"], generator=g, device=dev).to(qdt)
    kv_bytes = 2 * c["hkv"] * c["n_ctx"] * c["hd"] * 2
    # memory-bound configs rotate over distinct K/V copies so reads come from HBM
    n_sets = 1 if (c["kind"] == "prefill" and not c.get("kvrot")) or not rotate else \
        max(2, min(64, -(-2 * MALL_BYTES // kv_bytes)))
    kvs = []
    for _ in range(n_sets):
        k = torch.randn(c["hkv"], c["n_ctx"], c["hd"], generator=g, device=dev).half()
        v = torch.randn(c["hkv"], c["n_ctx"], c["hd"], generator=g, device=dev).half()
        kvs.append((k, v))
    out = torch.empty(c["nq"], c["hq"], c["hd"], dtype=odt, device=dev)
    desc = capi.make_desc(n_q_heads=c["hq"], n_kv_heads=c["hkv"], head_dim=c["hd"], n_query=c["nq"],
                          q_base_pos=c["base"], n_ctx=c["n_ctx"], softcap=c.get("cap", 0.0),
                          sliding_window=c.get("sw", 0),
                          q_dtype=capi.NEXUS_DT_F16 if qdt == torch.float16 else capi.NEXUS_DT_F32,
                          o_dtype=capi.NEXUS_DT_F16 if odt == torch.float16 else capi.NEXUS_DT_F32)
    if c["kind"] == "decode":
        splits = c["splits"] or capi.decode_default_splits(desc)
        ws_bytes = capi.decode_ws_bytes(desc, splits)
    else:
        splits = 0
        ws_bytes = capi.prefill_ws_bytes(desc)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)

    def call(i: int) -> None:
        k, v = kvs[i % n_sets]
        stream = torch.cuda.current_stream(dev).cuda_stream
        if c["kind"] == "decode":
            capi.decode_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr(),
                            splits, stream)
        else:
            capi.prefill_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr(),
                             ws_bytes, stream)

    warm_up(call, warmup)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(steps):
                call(i)
        gr.replay()
        torch.cuda.synchronize()
        s0.record()
        gr.replay()
        s1.record()
    else:
        s0.record()
        for i in range(steps):
            call(i)
        s1.record()
    s1.synchronize()
    ms = s0.elapsed_time(s1) / steps
    work, unit = work_of(c)
    res = {"config": name, "desc": c["desc"], "ms": ms, "kv_sets": n_sets, "launch": "graph" if graph else "stream"}
    if unit == "flop":
        tf = work / (ms * 1e-3) / 1e12
        res.update(tflops=tf, frac_mfma=tf / MFMA_F16_PEAK_TFLOPS, gflop=work / 1e9)
    else:
        gbs = work / (ms * 1e-3) / 1e9
        res.update(gbs=gbs, frac_hbm=gbs / HBM_PEAK_GBS, mbytes=work / 1e6, splits=splits)
    if c["kind"] == "prefill":
        res["splits"] = (ws_bytes // (c["nq"] * c["hq"] * (c["hd"] + 2) * 4)) if ws_bytes else 1
    if check:
        call(0)
        torch.cuda.synchronize()
        res["parity"] = parity(name, c, q, kvs[0][0], kvs[0][1], out)
    tag = " (1 K/V copy)" if c["kind"] != "prefill" and n_sets == 1 else ""
    log(f"[bench] {name}{tag}: {ms * 1e3:.1f} us/step  " +
        (f"{res['tflops']:.1f} TFLOP/s ({100 * res['frac_mfma']:.1f}% MFMA)" if unit == "flop"
         else f"{res['gbs']:.0f} GB/s ({100 * res['frac_hbm']:.1f}% HBM)"))
    return res


def measure_decode_layer(steps: int, warmup: int) -> dict:
    """The attention half of a gated full-attention decode layer over a device KV cache
    (q35_full_layer's prep + part + comb), one token at 32768 cached tokens, 16 q / 2 kv
    heads, head_dim 256, RoPE over 64 dims: nexus_hip_attn_decode_layer (q/k head norms,
    partial RoPE and the f16 store of the new row inside the split-KV kernel, then the gated
    combine; two launches).  Beside it, the same step as prep kernel + gated decode (three
    launches) and the prep alone.  Timed with HIP events on the stream the work runs on."""
    import torch

    from nexus_amd import capi, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    nh, nkv, hd, rot, pos = 16, 2, 256, 64, 32768
    cap = ((pos + 1) * 5 // 4 + 255) // 256 * 256
    kv_bytes = 2 * nkv * cap * hd * 2
    n_sets = max(2, min(64, -(-2 * MALL_BYTES // kv_bytes)))
    caches = [(torch.randn(nkv, cap, hd, generator=g, device=dev).half(),
               torch.randn(nkv, cap, hd, generator=g, device=dev).half()) for _ in range(n_sets)]
    qg = torch.randn(nh, 2 * hd, generator=g, device=dev)
    kraw = torch.randn(nkv, hd, generator=g, device=dev)
    vraw = torch.randn(nkv, hd, generator=g, device=dev)
    qnw = 0.1 * torch.randn(hd, generator=g, device=dev)
    knw = 0.1 * torch.randn(hd, generator=g, device=dev)
    ang = pos / torch.pow(torch.tensor(1e7, device=dev), torch.arange(rot // 2, device=dev) * 2.0 / rot)
    tab = torch.cat([torch.cos(ang), torch.sin(ang)]).float()
    q_out = torch.empty(nh, hd, device=dev)
    gate = torch.empty(nh, hd, device=dev)
    kvo = torch.empty(2, nkv, hd, device=dev)
    out = torch.empty(1, nh, hd, device=dev)
    desc = capi.make_desc(n_q_heads=nh, n_kv_heads=nkv, head_dim=hd, n_query=1, q_base_pos=pos, n_ctx=pos + 1,
                          kv_row_stride=cap)
    splits = capi.decode_default_splits(desc)
    ws = torch.empty(capi.decode_ws_bytes(desc, splits) // 4, device=dev)
    pdesc = capi.PrepDesc(nh, nkv, hd, rot, pos, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE
                          | capi.PREP_TRUNC_STORE, cap, 1e-6, 0)
    # a warm call through the checked wrapper, then raw C-ABI calls captured in a HIP graph:
    # the step is a few microseconds of GPU work, so host-side launch cost must stay out
    ops.decode_prep(qg, kraw, vraw, caches[0][0], caches[0][1], pos=pos, rope_tab=tab, q_norm_w=qnw, k_norm_w=knw,
                    q_norm_add_one=True, k_norm_add_one=True, trunc_store=True, q_out=q_out, gate_out=gate, kv_out=kvo)

    def prep(i, stream):
        k, v = caches[i % n_sets]
        capi.decode_prep_raw(pdesc, qg.data_ptr(), kraw.data_ptr(), vraw.data_ptr(), qnw.data_ptr(), knw.data_ptr(),
                             tab.data_ptr(), q_out.data_ptr(), gate.data_ptr(), k.data_ptr(), v.data_ptr(),
                             kvo.data_ptr(), stream)

    def two_step(i, stream):
        prep(i, stream)
        k, v = caches[i % n_sets]
        capi.decode_raw(desc, q_out.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr(), splits,
                        stream, gate=gate.data_ptr())

    assert capi.decode_layer_default_splits(pdesc) == splits
    assert capi.decode_layer_ws_bytes(pdesc, splits) <= ws.numel() * 4

    def step(i, stream):
        k, v = caches[i % n_sets]
        capi.decode_layer_raw(pdesc, 0.0, qg.data_ptr(), kraw.data_ptr(), vraw.data_ptr(), qnw.data_ptr(),
                              knw.data_ptr(), tab.data_ptr(), k.data_ptr(), v.data_ptr(), kvo.data_ptr(),
                              out.data_ptr(), ws.data_ptr(), splits, stream)

    def timed(fn):
        stream = torch.cuda.current_stream(dev).cuda_stream
        warm_up(lambda i: fn(i, stream), warmup)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            cap_stream = torch.cuda.current_stream(dev).cuda_stream
            for i in range(steps):
                fn(i, cap_stream)
        gr.replay()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        gr.replay()
        s1.record()
        s1.synchronize()
        return s0.elapsed_time(s1) / steps

    ms_prep, ms_two, ms_step = timed(prep), timed(two_step), timed(step)
    kv_read = 2.0 * nkv * (pos + 1) * hd * 2
    res = {"config": "decode_layer", "desc": "gated decode layer attention over a device KV cache: "
           "nexus_hip_attn_decode_layer (prep folded into the split-KV kernel, gated combine; two launches), "
           "1 token at 32768 cached tokens, 16q/2kv, hd256, rot 64",
           "ms": ms_step, "two_step_ms": ms_two, "prep_ms": ms_prep, "splits": splits, "kv_sets": n_sets,
           "launch": "graph", "launches_per_step": 2,
           "gbs": kv_read / (ms_step * 1e-3) / 1e9, "frac_hbm": kv_read / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS}
    log(f"[bench] decode_layer: {ms_step * 1e3:.1f} us/step fused (prep + decode as three launches "
        f"{ms_two * 1e3:.1f} us, prep alone {ms_prep * 1e3:.1f} us)  "
        f"{res['gbs']:.0f} GB/s of K/V ({100 * res['frac_hbm']:.1f}% HBM)")
    return res


def copy_calibration(steps: int, warmup: int, nbytes: int = 256 << 20) -> None:
    """A plain elementwise copy of known size (torch.mul by 1 over float32: each launch reads
    and writes nbytes): the reference point that scales the rocprofv3 FETCH_SIZE /
    WRITE_SIZE counters."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(warmup):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(steps):
        torch.mul(src, 1.0, out=dst)
    s1.record()
    s1.synchronize()
    ms = s0.elapsed_time(s1) / steps
    log(f"[bench] copy {nbytes >> 20} MiB: {ms * 1e3:.1f} us/launch, {2 * nbytes / (ms * 1e-3) / 1e9:.0f} GB/s "
        f"(read+write), {nbytes / 1024:.0f} KiB read and written per launch")


def gemm_ceiling(steps: int, warmup: int, n: int = 8192) -> dict:
    """A plain library f16 GEMM (torch.matmul, n x n x n, f32 accumulate) on N(0,1) operands and
    on all-zero operands: the matrix-core rate this GPU sustains under full load for data like the
    attention inputs, beside the published dense peak.  The clock follows the power limit and the
    matrix cores' power follows their operand data, so the two rates differ."""
    import torch

    res = {"shape": [n, n, n], "dtype": "f16"}
    for tag, fill in (("normal", lambda t: t.normal_()), ("zeros", lambda t: t.zero_())):
        a = fill(torch.empty(n, n, dtype=torch.float16, device="cuda"))
        b = fill(torch.empty(n, n, dtype=torch.float16, device="cuda"))
        c = torch.empty(n, n, dtype=torch.float16, device="cuda")
        warm_up(lambda i: torch.matmul(a, b, out=c), warmup)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(steps):
            torch.matmul(a, b, out=c)
        s1.record()
        s1.synchronize()
        ms = s0.elapsed_time(s1) / steps
        res[f"{tag}_tflops"] = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        res[f"{tag}_ms"] = ms
        del a, b, c
    res["normal_frac_of_peak"] = res["normal_tflops"] / MFMA_F16_PEAK_TFLOPS
    log(f"[bench] f16 GEMM {n}^3: N(0,1) operands {res['normal_tflops']:.0f} TFLOP/s, zeros "
        f"{res['zeros_tflops']:.0f} TFLOP/s ({100 * res['normal_frac_of_peak']:.1f}% / "
        f"{100 * res['zeros_tflops'] / MFMA_F16_PEAK_TFLOPS:.1f}% of the dense peak)")
    return res


def read_reference(steps: int, warmup: int) -> dict:
    """A plain library read for the decode sizes: torch's int64 max over 64 MiB of f16 data (the
    K/V of the hd-256 decode at 32k keys; eight distinct buffers rotated past the Infinity Cache)
    and over 1 GiB, each timed with HIP events.  The rate a library reduction reaches at 64 MiB,
    with its launch and ramp, against the split-KV decode that reads the same bytes and computes."""
    import torch

    res = {"op": "torch int64 max over f16 data (read only)"}
    for tag, mib, n_sets in (("64MiB", 64, 8), ("1GiB", 1024, 1)):
        n = mib << 20
        sets = [torch.randn(n // 2, device="cuda").half().view(torch.int64) for _ in range(n_sets)]
        warm_up(lambda i: sets[i % n_sets].max(), warmup)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for i in range(steps):
            sets[i % n_sets].max()
        s1.record()
        s1.synchronize()
        us = s0.elapsed_time(s1) / steps * 1e3
        res[f"{tag}_us"] = us
        res[f"{tag}_tbs"] = n / (us * 1e-6) / 1e12
        del sets
    log(f"[bench] library read (torch int64 max): 64 MiB {res['64MiB_us']:.1f} us = {res['64MiB_tbs']:.2f} TB/s, "
        f"1 GiB {res['1GiB_tbs']:.2f} TB/s")
    return res


TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def measured_traffic(name: str):
    """HBM bytes per launch of a config's dominant kernel, from the rocprofv3 FETCH_SIZE and
    WRITE_SIZE runs recorded in profiles/traffic.json (each counter scaled by its reading
    for the calibration copy).  None when no measurement is recorded."""
    import json

    try:
        rec = json.loads(TRAFFIC_FILE.read_text())[name]
        return float(rec["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def cpu_info() -> dict:
    """The host's CPU: the model string, the logical CPUs the OS reports (nproc) and the ones
    this process may run on (its affinity set, the share a container or job scheduler gives it)."""
    model, ids = "unknown", {}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "model name" and model == "unknown":
                model = val.strip()
            elif key in ("cpu family", "model", "stepping", "vendor_id") and key not in ids:
                ids[key] = val.strip()
            elif key == "flags" and "avx512" not in ids:
                ids["avx512"] = "avx512f" in val.split()
            if line.strip() == "":
                break                                    # the first processor's block is enough
    except OSError:
        pass
    if ids:
        model = f"{model} (vendor {ids.get('vendor_id', '?')}, family {ids.get('cpu family', '?')}, " \
                f"model {ids.get('model', '?')}, stepping {ids.get('stepping', '?')}, " \
                f"avx512 {'yes' if ids.get('avx512') else 'no'})"
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": model, "nproc": os.cpu_count() or 1, "usable": usable}


def _timed(fn, target_s: float) -> tuple[float, int]:
    """Seconds per call of fn, repeated until about target_s have passed (at least once)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            return el / n, n


def cpu_baseline(target_s: float = 10.0) -> dict:
    """The reference's CPU attention, restated in oracle/ (the parity checker), timed on this
    host on bounded samples of the BASELINE workloads:
      * prefill (cfg2, the headline): attn_batch_cpu (transformer.h:8653-8685) on a uniform
        sample of (query, head) rows -- single thread, as the reference runs it (:8666), and
        over every usable core (rows in parallel);
      * decode (cfg1, cfg4): forward_cached_scores (attention.h:1201-1259) for one token --
        with the reference's threading (heads in parallel on a pool of every usable core,
        :1255-1257) and on one thread."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    from nexus_amd import capi
    from nexus_amd.inputs import make_case

    info = cpu_info()
    cores = info["usable"]
    c = CONFIGS["cfg2"]
    q, k, v = make_case(n_q_heads=c["hq"], n_kv_heads=c["hkv"], head_dim=c["hd"], n_query=c["nq"],
                        n_ctx=c["n_ctx"], seed=2024, q_f16=True)
    n_rows_total = c["nq"] * c["hq"]
    rng = np.random.default_rng(0)
    order = rng.permutation(n_rows_total).astype(np.int32)

    def run(rows, threads):
        t0 = time.perf_counter()
        O.attn_batch_rows(q, k, v, rows, n_kv_heads=c["hkv"], n_ctx=c["n_ctx"], q_base_pos=c["base"],
                          n_threads=threads)
        return time.perf_counter() - t0

    def flops(rows):
        keys = np.minimum(c["base"] + rows // c["hq"], c["n_ctx"] - 1) + 1
        return float(4.0 * c["hd"] * keys.sum())

    probe = order[:16]
    per_row = run(probe, 1) / len(probe)
    n = int(min(n_rows_total, max(16, target_s / max(per_row, 1e-6))))
    rows = order[:n]
    t1 = run(rows, 1)
    rows_mt = order[: min(n_rows_total, max(16, int(target_s / 2 / max(per_row, 1e-6)) * cores))]
    tm = run(rows_mt, cores)

    # the other attn_batch_cpu workloads: cfg3 on a row sample (a full single-thread run takes
    # most of an hour), cfg5 whole (64 rows)
    prefill_more = {}
    for name, n_sample in (("cfg3", 1024), ("cfg5", 0)):
        d = CONFIGS[name]
        pq, pk, pv = make_case(n_q_heads=d["hq"], n_kv_heads=d["hkv"], head_dim=d["hd"], n_query=d["nq"],
                               n_ctx=d["n_ctx"], seed=9, q_f16=d["q"] == "f16")
        tot = d["nq"] * d["hq"]
        prow = (np.arange(tot) if n_sample == 0 else rng.choice(tot, n_sample, replace=False)).astype(np.int32)
        keys = np.minimum(d["base"] + prow // d["hq"], d["n_ctx"] - 1) + 1
        pfl = float(4.0 * d["hd"] * keys.sum())
        res = {}
        for label, threads in (("one_thread", 1), ("all_cores", cores)):
            t0 = time.perf_counter()
            O.attn_batch_rows(pq, pk, pv, prow, n_kv_heads=d["hkv"], n_ctx=d["n_ctx"], q_base_pos=d["base"],
                              n_threads=threads)
            sec = time.perf_counter() - t0
            res[label] = {"value": pfl / sec / 1e12, "unit": "TFLOP/s", "threads": threads, "seconds": sec}
        res["sample"] = f"{len(prow)} of {tot} (query, head) rows"
        prefill_more[name] = res

    # decode: the reference's own forward_cached_scores, compiled from its sources into
    # oracle/_ref (kind "reference"); the C restatement (kind "port") where that build is absent
    decode = {}
    use_ref = O.ref_available()
    for name in ("cfg1", "cfg4"):
        d = CONFIGS[name]
        dq, dk, dv = make_case(n_q_heads=d["hq"], n_kv_heads=d["hkv"], head_dim=d["hd"], n_query=1, n_ctx=d["n_ctx"],
                               seed=7)
        nbytes = capi.decode_bytes(d["hkv"], d["hd"], d["n_ctx"], d["hq"], 1)
        res = {"kind": "reference" if use_ref else "port",
               "code": "oracle/_ref: forward_cached_scores (attention.h:1201-1259) built from the reference's sources"
                       if use_ref else "oracle/attn_oracle.c restating attention.h:1201-1259"}
        for label, threads in (("reference_threads", cores), ("one_thread", 1)):
            if use_ref:
                probe = O.ref_time_cached_scores(dq[0], dk, dv, n_kv_heads=d["hkv"], pos=d["base"], n_threads=threads,
                                                 reps=1)
                reps = max(1, min(200, int(target_s / 8 / max(probe, 1e-6))))
                sec = O.ref_time_cached_scores(dq[0], dk, dv, n_kv_heads=d["hkv"], pos=d["base"], n_threads=threads,
                                               reps=reps)
            else:
                sec, reps = _timed(lambda: O.cached_scores(dq[0], dk, dv, n_kv_heads=d["hkv"], pos=d["base"],
                                                          n_threads=threads), target_s / 8)
            res[label] = {"value": nbytes / sec / 1e9, "unit": "GB/s", "us_per_token": sec * 1e6, "threads": threads,
                          "calls": reps}
        decode[name] = res
    return {
        "value": flops(rows) / t1 / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} of {n_rows_total} (query, head) rows of cfg2 drawn uniformly, single thread "
                  f"({t1:.1f} s), oracle/attn_oracle.c restating transformer.h:8653-8685",
        "all_cores": {"value": flops(rows_mt) / tm / 1e12, "cores": cores, "rows": int(len(rows_mt)),
                      "seconds": tm},
        "prefill": prefill_more,
        "decode": decode,
        "cpu": info,
    }


def parity(name: str, c: dict, q, k, v, out, n_rows: int = 256) -> dict:
    """The checker: max-abs and rel-L2 of the timed kernels' output against the CPU oracle
    (attn_batch_cpu, transformer.h:8653-8685) on the inputs the bench timed -- every row for
    decode and verify, a uniform sample of (query, head) rows (first and last included) for
    prefill."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O

    qn = q.float().cpu().numpy()
    kn = k.cpu().numpy().view(np.uint16)
    vn = v.cpu().numpy().view(np.uint16)
    got = out.float().cpu().numpy()
    total = c["nq"] * c["hq"]
    kw = dict(n_kv_heads=c["hkv"], n_ctx=c["n_ctx"], q_base_pos=c["base"], sliding_window=c.get("sw", 0),
              softcap=c.get("cap", 0.0), n_threads=min(16, os.cpu_count() or 1))
    if c["kind"] == "prefill":
        rng = np.random.default_rng(11)
        rows = np.unique(np.concatenate([[0, total - 1], rng.choice(total, min(n_rows, total), replace=False)]))
        rows = rows.astype(np.int32)
        ref = O.attn_batch_rows(qn, kn, vn, rows, **kw)
        g = got.reshape(total, -1)[rows]
        r = ref.reshape(total, -1)[rows]
    else:
        rows = np.arange(total)
        g, r = got.reshape(total, -1), O.attn_batch(qn, kn, vn, **kw).reshape(total, -1)
    res = {"max_abs": float(O.max_abs(g, r)), "rel_l2": float(O.rel_l2(g, r)), "rows_checked": int(len(rows)),
           "rows_total": int(total), "tolerance": {"max_abs": 2e-3, "rel_l2": 1e-3}}
    res["ok"] = res["max_abs"] < 2e-3 and res["rel_l2"] < 1e-3
    log(f"[bench] {name} parity: max_abs={res['max_abs']:.2e} rel_l2={res['rel_l2']:.2e} "
        f"({res['rows_checked']} of {total} rows) {'ok' if res['ok'] else 'FAILED'}")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=sorted(CONFIGS) + ["copy", "decode_layer", "gemm", "read"], default=None,
                    help="measure one config only (for profiling runs); 'copy' runs a plain "
                         "device copy of 256 MiB that calibrates the FETCH_SIZE/WRITE_SIZE counters; "
                         "'gemm' a library f16 GEMM on N(0,1) and on zero operands (the attainable "
                         "matrix-core rate); 'read' a library read of 64 MiB and 1 GiB")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's attention path runs on a single MI355X "
              "(sharding over several GPUs is not built in this tier); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from nexus_amd import capi

    capi.load()
    props = torch.cuda.get_device_properties(0)
    log(f"[bench] device {props.name} CUs={props.multi_processor_count} lib={capi.version()}")

    if args.only == "copy":
        copy_calibration(args.steps, args.warmup)
        return 0
    if args.only == "decode_layer":
        measure_decode_layer(args.steps, args.warmup)
        return 0
    if args.only == "gemm":
        gemm_ceiling(args.steps, args.warmup)
        return 0
    if args.only == "read":
        read_reference(args.steps, args.warmup)
        return 0
    if args.only:
        measure(args.only, args.steps, args.warmup)
        return 0

    extra = {"cfg3": measure("cfg3", max(5, args.steps // 5), max(args.warmup, 20), check=True)}
    head = measure("cfg2", args.steps, args.warmup, check=True)
    for name in ("cfg4", "cfg1", "cfg5"):
        extra[name] = measure(name, args.steps, args.warmup, check=True)
    extra["cfg1_graph"] = measure("cfg1", args.steps, args.warmup, graph=True)
    # the same decode calls with one K/V copy (resident in the 256 MB Infinity Cache)
    extra["cfg4_warm"] = measure("cfg4", args.steps, args.warmup, rotate=False)
    extra["cfg5_warm"] = measure("cfg5", args.steps, args.warmup, rotate=False)
    extra["q35p"] = measure("q35p", max(5, args.steps // 5), args.warmup, check=True)
    extra["q35c"] = measure("q35c", args.steps, args.warmup, check=True)
    extra["cfg2q32"] = measure("cfg2q32", args.steps, args.warmup, check=True)
    extra["tile3"] = measure("tile3", args.steps, args.warmup, check=True)
    extra["q35t3"] = measure("q35t3", args.steps, args.warmup, check=True)
    extra["c64"] = measure("c64", args.steps, args.warmup, check=True)
    extra["q35s"] = measure("q35s", args.steps, args.warmup, check=True)
    extra["cap2"] = measure("cap2", args.steps, args.warmup, check=True)
    extra["swa3"] = measure("swa3", max(5, args.steps // 5), args.warmup, check=True)
    extra["decode_layer"] = measure_decode_layer(args.steps, args.warmup)
    extra["gemm_ceiling"] = gemm_ceiling(max(5, args.steps // 5), args.warmup)
    extra["read_reference"] = read_reference(args.steps, args.warmup)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle, bounded sample) ...")
        cpu = cpu_baseline()
        log(f"[bench] CPU baseline: {cpu['value'] * 1e3:.2f} GFLOP/s single thread")

    c2 = CONFIGS["cfg2"]
    line = {
        "metric": METRIC,
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1), torch RNG on device)",
        "config": {"workload": "cfg2: " + c2["desc"], "n_q_heads": c2["hq"], "n_kv_heads": c2["hkv"],
                   "head_dim": c2["hd"], "n_query": c2["nq"], "q_base_pos": c2["base"], "n_ctx": c2["n_ctx"],
                   "kv_splits": head["splits"], "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": head["tflops"] / MFMA_F16_PEAK_TFLOPS,
                     "traffic": measured_traffic("cfg2"),
                     "kernel": "nxa::prefill_wide_kernel<128, KS=2, f16 Q, f16 O> (64-row blocks, key range "
                               "over two waves; one launch per call, timed with HIP events on its stream)",
                     "algorithmic_gflop_per_call": head["gflop"]},
        "cpu_baseline": cpu,
        "parity": head.get("parity"),
        "extra": extra,
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
