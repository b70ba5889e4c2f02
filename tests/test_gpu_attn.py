"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Tolerance: max-abs 2e-3 and rel-L2 1e-3 of the fp32-accumulated
output against the reference's CPU attention on the same seeded inputs; f16 outputs are
upcast before comparing.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from nexus_amd import capi, ops
from nexus_amd.inputs import make_case

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
REL_L2 = 1e-3


def dev(x):
    if x.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def assert_close(got, ref, what=""):
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[parity] {what} max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma < MAX_ABS and rl < REL_L2, f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}"


def run_prefill(q, k, v, *, hkv, n_ctx, q_base, q_f16=False, o_f16=False, sw=0, cap=0.0, split=True, gate=None):
    qt = dev(q)
    if q_f16:
        qt = qt.half()
    out = ops.attn_prefill(qt, dev(k), dev(v), n_kv_heads=hkv, q_base_pos=q_base, n_ctx=n_ctx,
                           sliding_window=sw, softcap=cap, out_dtype=torch.float16 if o_f16 else torch.float32,
                           split=split, gate=None if gate is None else dev(gate))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def run_decode(q, k, v, *, hkv, n_ctx, q_base, n_splits=0, sw=0, cap=0.0, ws=None, gate=None, o_f16=False,
               scale=0.0):
    out = ops.attn_decode(dev(q), dev(k), dev(v), n_kv_heads=hkv, q_base_pos=q_base, n_ctx=n_ctx,
                          n_splits=n_splits, sliding_window=sw, softcap=cap, partial_ws=ws, scale=scale,
                          gate=None if gate is None else dev(gate),
                          out_dtype=torch.float16 if o_f16 else torch.float32)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def make_gate(shape, seed):
    """Gate logits over the sigmoid's whole range plus entries beyond the +-80 clamps."""
    rng = np.random.default_rng(seed)
    z = (rng.standard_normal(shape) * 4).astype(np.float32)
    flat = z.reshape(-1)
    idx = rng.choice(flat.size, size=max(1, flat.size // 50), replace=False)
    flat[idx] = rng.choice(np.array([-1e4, -81.0, 81.0, 1e4], np.float32), size=idx.size)
    return z


# ------------------------------------------------------------------------ prefill

PREFILL_CASES = [
    # (Hq, Hkv, hd, n_query, q_base, extra_stride, q_f16, o_f16, sw, cap)
    (8, 2, 128, 128, 0, 0, True, True, 0, 0.0),        # one full block, cold
    (8, 2, 128, 200, 0, 0, True, True, 0, 0.0),        # ragged second block
    (10, 2, 128, 77, 300, 5, True, False, 0, 0.0),     # chunk after cache, padded stride
    (4, 4, 64, 150, 17, 0, False, False, 0, 0.0),      # MHA, hd 64, f32 q/o
    (16, 2, 256, 96, 40, 3, True, True, 0, 0.0),       # hd 256, G=8
    (6, 2, 192, 70, 10, 0, True, True, 0, 0.0),        # hd 192
    (8, 8, 128, 130, 0, 0, True, True, 50, 0.0),       # sliding window
    (8, 4, 128, 100, 60, 0, False, False, 0, 30.0),    # softcap
    (8, 2, 128, 64, 2000, 0, True, True, 0, 0.0),      # long cache, short chunk: pipelined kernel in 8 key splits
    (40, 8, 128, 33, 1000, 0, True, True, 0, 0.0),     # cfg-2 head layout, small
    # pipelined kernel with 128-row blocks (>= one block per CU of a 256-CU MI355X)
    (64, 8, 128, 520, 37, 3, False, False, 0, 0.0),    # ragged last block, unaligned base, f32 q/o
    (64, 16, 64, 512, 0, 0, True, True, 0, 0.0),       # hd 64
    # pipelined kernel, 64-row blocks, odd tile count: key group 1 runs one tile past the end
    (8, 2, 128, 80, 0, 0, True, False, 0, 0.0),
    # pipelined kernel at head dim 256 (one wave per SIMD, O and Q^T in AGPRs): >= 256 blocks
    (64, 8, 256, 512, 0, 0, True, True, 0, 0.0),      # cold
    (32, 4, 256, 1030, 17, 5, False, False, 0, 0.0),  # f32 q/o, ragged last block, padded stride
    (32, 4, 256, 1024, 300, 0, True, False, 0, 0.0),  # chunk after a cache, f32 out
    # head dim 256 with fewer blocks than CUs: 128-row blocks, unsplit or in key splits
    (16, 2, 256, 1030, 0, 0, True, True, 0, 0.0),
    (16, 4, 256, 64, 500, 0, True, False, 0, 0.0),
    # key splits merged by the one-wave-per-row combine (>= 256 rows); hd 192 in AGPRs
    (4, 4, 64, 100, 3000, 0, False, False, 0, 0.0),    # 12 splits: a partial second merge batch
    (8, 1, 256, 64, 4000, 0, True, True, 0, 0.0),      # 16 splits: two full merge batches
    (6, 2, 192, 70, 2000, 0, True, False, 0, 0.0),
    # pipelined kernel with softcap / sliding window (raw MFMA scores, VALU softcap; window
    # tiles skipped below the block's first row, masked above)
    (16, 4, 128, 520, 100, 0, True, True, 300, 0.0),     # window, 64-row blocks, ragged
    (64, 8, 128, 512, 2000, 0, False, False, 200, 20.0), # window + softcap, 128-row blocks, f32 q/o
    (16, 2, 256, 300, 1000, 0, True, True, 0, 50.0),     # hd 256 softcap in key splits
    (8, 2, 64, 200, 5000, 0, True, False, 1000, 0.0),    # hd 64 window in key splits
    (8, 2, 256, 256, 0, 0, False, True, 100, 30.0),      # hd 256 window + softcap, cold
    # a window without softcap takes the plain form (accumulators seeded with -m, masking only)
    (16, 2, 256, 300, 40, 0, True, True, 150, 0.0),      # hd 256 window, AGPR form
    (12, 4, 192, 200, 100, 0, False, False, 90, 0.0),    # hd 192 window, f32 q/o
    (64, 8, 128, 512, 300, 0, False, True, 256, 0.0),    # window, 128-row blocks, f32 q (residual MFMA)
    # 64-row blocks at one to one and a half per CU (cfg2's regime)
    (32, 8, 128, 512, 100, 0, True, True, 0, 0.0),       # exactly one block per CU
    (40, 8, 128, 520, 300, 0, False, False, 0, 0.0),     # 360 blocks, ragged last block
    (36, 4, 64, 512, 700, 0, True, False, 200, 10.0),    # hd 64, window + softcap
    # kv head counts that do not divide 8: XCD groups of several kv heads (work order only)
    (24, 12, 128, 700, 0, 0, True, True, 0, 0.0),        # 12 kv heads: 4 groups of 3 on 2 XCDs each
    (18, 6, 64, 1000, 50, 0, True, True, 0, 0.0),        # 6 kv heads: 2 groups of 3 on 4 XCDs each
    (15, 3, 256, 600, 0, 0, True, False, 0, 0.0),        # 3 kv heads, hd 256: one group on 8 XCDs
    (16, 2, 256, 1024, 1024, 0, True, True, 0, 0.0),     # the engine's 1024-token tile at hd 256: 128 blocks in 2 splits
    (40, 8, 128, 1024, 1024, 0, True, True, 0, 0.0),     # its second tile at 40 heads: 320 blocks, paired CUs rotated
    # short chunks over long caches through the split-KV decode kernel (several 32-row groups)
    (16, 2, 256, 16, 9000, 0, True, True, 0, 0.0),       # 4 row groups (2R <= G behind >= 8k keys)
    (40, 8, 128, 12, 17000, 3, False, False, 0, 0.0),    # 2 row groups at hd 128 behind >= 16k: packed, f32 q/o
    (64, 8, 128, 8, 12000, 0, True, True, 0, 0.0),       # 2R <= G = 8 behind 8k-16k keys: packed
    (16, 2, 256, 8, 17000, 0, False, False, 0, 0.0),     # 2 row groups that cannot pack: decode kernel, f32 q/o
    (48, 8, 128, 16, 9000, 0, True, True, 0, 0.0),       # R = 3, 2R <= G: packed rather than the decode kernel
    (16, 2, 256, 12, 20000, 0, True, False, 300, 20.0),  # window + softcap on that path
    # chunks of <= 128 queries behind >= 16k keys with packed (query, head-in-group) rows
    (40, 8, 128, 32, 20000, 0, True, True, 0, 0.0),      # 64-row blocks of 12.8 queries x 5 heads
    (40, 8, 128, 47, 16500, 2, False, False, 5000, 30.0),  # window + softcap, f32 q/o, ragged last block
    (16, 2, 256, 96, 17000, 0, True, False, 0, 0.0),     # hd 256: 12 packed 128-row blocks of 16 queries x 8 heads
    (64, 8, 128, 20, 12000, 0, True, True, 0, 0.0),      # packed behind 8k-16k keys
    (16, 2, 256, 32, 17000, 0, True, True, 0, 0.0),      # 4 packed blocks in 64 key splits
    (4, 4, 128, 64, 20000, 0, False, False, 0, 0.0),     # MHA, 4 blocks in 64 key splits, f32 q/o
    (40, 8, 128, 200, 12000, 0, True, True, 0, 0.0),     # 200 queries behind 12k keys, packed
    (16, 2, 256, 160, 17000, 0, True, False, 0, 0.0),    # 160 queries packed at hd 256
    (32, 8, 64, 24, 17000, 0, True, True, 0, 0.0),       # packed at hd 64 behind >= 16k keys
    (8, 1, 128, 32, 20000, 0, True, False, 0, 0.0),      # one kv head: packed, 64 splits
    (24, 4, 192, 16, 20000, 0, True, True, 0, 0.0),      # R = 3 < G = 6: packed rather than the decode kernel
    (8, 1, 256, 16, 20000, 0, False, False, 0, 0.0),     # R = 4 < G = 8 that cannot pack: decode kernel
    (24, 4, 192, 100, 16384, 0, False, True, 0, 0.0),    # hd 192, f32 q
    (40, 8, 128, 24, 17000, 3, False, False, 0, 0.0),    # 4 row groups at hd 128: packed, f32 q/o
    (64, 8, 128, 20, 17000, 0, True, True, 0, 0.0),      # G = 8: 240 packed workgroups against 256 plain
]


@pytest.mark.parametrize("hq,hkv,hd,nq,base,extra,qf16,of16,sw,cap", PREFILL_CASES)
def test_prefill_vs_oracle(hip, hq, hkv, hd, nq, base, extra, qf16, of16, sw, cap):
    n_ctx = base + nq
    print(f"[case] prefill hq={hq} hkv={hkv} hd={hd} nq={nq} base={base} sw={sw} cap={cap}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx,
                        kv_stride=n_ctx + extra, seed=nq + base, q_f16=qf16)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=qf16, o_f16=of16, sw=sw, cap=cap)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw,
                       softcap=cap, n_threads=8)
    assert_close(got, ref, f"prefill {hq}/{hkv} hd{hd} nq{nq}@{base}")


def test_prefill_queries_past_cache_and_short_cache(hip):
    """n_ctx < q_base + n_query: late queries see [0, n_ctx-1] (transformer.h:8670)."""
    hq, hkv, hd, nq, base, n_ctx = 8, 2, 128, 150, 40, 100
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=3, q_f16=True)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=True)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    assert_close(got, ref, "past-cache")


def test_prefill_golden(hip, golden):
    hq, hkv, hd, q_base, nq, n_ctx = (int(x) for x in golden["pre_a_meta"])
    got = run_prefill(golden["pre_a_q"], golden["pre_a_k"], golden["pre_a_v"], hkv=hkv, n_ctx=n_ctx, q_base=q_base)
    assert_close(got, golden["pre_a_out"], "golden pre_a")


@pytest.mark.parametrize("hq,hkv,hd,nq,base,sw,cap", [
    (8, 2, 128, 1, 500, 0, 0.0),        # one row of a 64-row block
    (16, 2, 256, 3, 900, 0, 0.0),       # AGPR form, three rows
    (12, 4, 192, 5, 300, 64, 25.0),     # head dim 192, window + softcap
    (4, 4, 64, 2, 0, 0, 0.0),           # cold, two queries
])
def test_prefill_tiny_chunks_without_workspace(hip, hq, hkv, hd, nq, base, sw, cap):
    """A handful of queries and no workspace: the pipelined kernel runs blocks that are almost
    all padding rows (the split-KV path needs the workspace)."""
    n_ctx = base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=nq + hd, q_f16=True)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=True, sw=sw, cap=cap, split=False)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw, softcap=cap,
                       n_threads=8)
    assert_close(got, ref, f"tiny {hq}/{hkv} hd{hd} nq{nq}@{base}")


@pytest.mark.parametrize("cap", [0.0, 30.0])
def test_prefill_split_equals_unsplit(hip, cap):
    """With a workspace the pipelined kernel splits this short chunk's key range over
    workgroups (plain and softcapped); the result must not depend on it."""
    hq, hkv, hd, nq, base = 8, 2, 128, 256, 3000
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=4, q_f16=True)
    a = run_prefill(q, k, v, hkv=hkv, n_ctx=base + nq, q_base=base, q_f16=True, cap=cap, split=True)
    b = run_prefill(q, k, v, hkv=hkv, n_ctx=base + nq, q_base=base, q_f16=True, cap=cap, split=False)
    assert O.max_abs(a, b) < 1e-3 and O.rel_l2(a, b) < 5e-4


def test_prefill_chunked_equals_cold_rows(hip):
    """Rows of a chunk appended after a cache == the same rows of a cold prefill."""
    hq, hkv, hd, base, nq = 8, 2, 128, 384, 256
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=base + nq, n_ctx=base + nq, seed=5, q_f16=True)
    cold = run_prefill(q, k, v, hkv=hkv, n_ctx=base + nq, q_base=0, q_f16=True, split=False)
    chunk = run_prefill(q[base:], k, v, hkv=hkv, n_ctx=base + nq, q_base=base, q_f16=True, split=False)
    assert O.max_abs(chunk, cold[base:]) < 1e-3


GATED_PREFILL_CASES = [
    # (Hq, Hkv, hd, n_query, q_base, q_f16, o_f16, sw, cap, split) -- one per epilogue
    (64, 8, 128, 520, 37, False, False, 0, 0.0, True),     # pipelined kernel, 128-row blocks, f32 out
    (8, 2, 128, 80, 0, True, True, 0, 0.0, True),          # pipelined kernel, 64-row blocks (key-group merge)
    (16, 2, 256, 96, 40, True, True, 0, 0.0, True),        # pipelined kernel, hd 256
    (8, 2, 128, 64, 2000, True, False, 0, 0.0, True),      # pipelined kernel's key split + row combine
    (6, 2, 192, 70, 10, True, True, 0, 0.0, True),         # pipelined kernel, hd 192 (AGPR form)
    (8, 1, 256, 64, 4000, True, False, 0, 0.0, True),      # hd 256 in 16 key splits: gate in the row combine
    (6, 2, 192, 70, 2000, False, True, 300, 20.0, True),   # hd 192 key splits, window + softcap
    (8, 2, 128, 80, 0, True, True, 40, 0.0, True),         # window without softcap, 64-row blocks
    (40, 8, 128, 40, 17000, True, False, 0, 0.0, True),    # packed rows behind a long cache, gated
    (8, 4, 128, 100, 60, False, False, 0, 30.0, True),     # pipelined kernel, softcap
    (8, 2, 128, 256, 3000, True, True, 0, 30.0, True),     # softcapped key split + combine
    (40, 8, 128, 520, 300, True, True, 0, 0.0, True),      # pipelined kernel, 360 64-row blocks
]


@pytest.mark.parametrize("hq,hkv,hd,nq,base,qf16,of16,sw,cap,split", GATED_PREFILL_CASES)
def test_prefill_gated(hip, hq, hkv, hd, nq, base, qf16, of16, sw, cap, split):
    """out * sigmoid(gate) fused into every prefill epilogue (qwen35_attn_comb.comp:34-38)."""
    n_ctx = base + nq
    print(f"[case] prefill gated hq={hq} hkv={hkv} hd={hd} nq={nq} base={base} cap={cap}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=nq + 7, q_f16=qf16)
    gate = make_gate(q.shape, nq)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=qf16, o_f16=of16, sw=sw, cap=cap,
                      split=split, gate=gate)
    ref = O.gate_mul(O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw,
                                  softcap=cap, n_threads=8), gate)
    assert_close(got, ref, f"prefill gated {hq}/{hkv} hd{hd} nq{nq}@{base}")


# ------------------------------------------------------------------------ decode

DECODE_CASES = [
    # (Hq, Hkv, hd, n_query, q_base, n_ctx, n_splits, extra_stride)
    (16, 4, 128, 1, 4095, 4096, 0, 0),          # cfg 1
    (16, 4, 128, 1, 4095, 4096, 1, 0),
    (40, 8, 128, 1, 3000, 3001, 64, 7),         # cfg 4 layout, short
    (40, 8, 128, 1, 777, 778, 13, 0),           # ragged splits
    (16, 2, 256, 4, 2000, 2004, 0, 0),          # MTP verify layout (cfg 5), short
    (16, 2, 256, 4, 2000, 2004, 5, 0),
    (8, 8, 64, 1, 0, 1, 0, 0),                  # single key
    (12, 2, 192, 3, 100, 103, 0, 0),            # G=6 x 3 drafts, hd 192
    (64, 1, 128, 1, 500, 501, 0, 0),            # G=64: two row groups
]


@pytest.mark.parametrize("hq,hkv,hd,nq,base,n_ctx,splits,extra", DECODE_CASES)
def test_decode_vs_oracle(hip, hq, hkv, hd, nq, base, n_ctx, splits, extra):
    print(f"[case] decode hq={hq} hkv={hkv} hd={hd} nq={nq} base={base} ctx={n_ctx} splits={splits}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx,
                        kv_stride=n_ctx + extra, seed=n_ctx + hq)
    got = run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, n_splits=splits)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    assert_close(got, ref, f"decode {hq}/{hkv} hd{hd} nq{nq}@{base}")
    if nq == 1:
        dec = O.cached_scores(q[0], k, v, n_kv_heads=hkv, pos=base, n_threads=8)
        assert_close(got[0], dec, "decode vs forward_cached_scores restatement")


@pytest.mark.parametrize("name", ["dec_a", "dec_b", "dec_c", "dec_d"])
@pytest.mark.parametrize("splits", [1, 0])
def test_decode_golden(hip, golden, name, splits):
    """Fixtures written by the reference's own forward_cached_scores (attention.h:1201-1259,
    tests/golden/make_golden.py), with their scale and softcap (dec_c: scale 0.1, softcap 30,
    which the reference computes with its Pade tanh, attention.h:232-245)."""
    hq, hkv, hd, pos = (int(x) for x in golden[f"{name}_meta"])
    scale, cap = (float(x) for x in golden[f"{name}_fmeta"])
    q = golden[f"{name}_q"][None]
    got = run_decode(q, golden[f"{name}_k"], golden[f"{name}_v"], hkv=hkv, n_ctx=pos + 1, q_base=pos,
                     n_splits=splits, scale=scale, cap=cap)
    assert_close(got[0], golden[f"{name}_out"], f"golden {name} scale={scale} softcap={cap} splits={splits}")


def test_decode_sliding_window_and_softcap(hip):
    hq, hkv, hd, nq, base = 8, 2, 128, 2, 900
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=6)
    for sw, cap in ((100, 0.0), (0, 20.0), (33, 10.0)):
        got = run_decode(q, k, v, hkv=hkv, n_ctx=base + nq, q_base=base, sw=sw, cap=cap)
        ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base, sliding_window=sw,
                           softcap=cap, n_threads=8)
        assert_close(got, ref, f"decode sw={sw} cap={cap}")


def test_decode_partials_have_reference_meaning(hip):
    """The partial of every row and split is (sum e^{s-m} v, m, l) over the split's keys, as
    qwen35_attn_part.comp:3 defines them (m is the split's max score)."""
    hq, hkv, hd, base = 8, 2, 128, 1023
    n_ctx = base + 1
    splits = 8
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=n_ctx, seed=7)
    desc = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, q_base_pos=base, n_ctx=n_ctx)
    ws = torch.zeros(capi.decode_ws_bytes(desc, splits) // 4, dtype=torch.float32, device="cuda")
    ws[: hq * splits * (hd + 2)] = float("nan")          # every partial must be written
    run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, n_splits=splits, ws=ws)
    got = capi.unpack_partials(ws.cpu().numpy(), hq, splits, hd)
    chunk = ((n_ctx + splits - 1) // splits + 31) // 32 * 32
    ref = O.split_partials(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_chunks=splits, chunk=chunk)
    assert np.max(np.abs(got[:, :, hd] - ref[:, :, hd])) < 1e-4                     # m
    assert O.rel_l2(got[:, :, hd + 1], ref[:, :, hd + 1]) < 1e-3                    # l
    assert O.rel_l2(got[:, :, :hd], ref[:, :, :hd]) < 1e-3                          # acc


def test_repeated_calls_reuse_workspace(hip):
    """The workspace carries no state between calls: a workspace full of NaN garbage, and
    repeated calls on one workspace, give bit-identical outputs (decode with and without
    row tiles, prefill split path)."""
    import torch

    cases = [("decode", 40, 8, 128, 1, 3000, 16), ("decode", 16, 2, 256, 4, 3000, 200),
             ("prefill", 8, 2, 128, 200, 2500, 0)]
    for kind, hq, hkv, hd, nq, base, splits in cases:
        print(f"[case] workspace reuse {kind} hq={hq} hkv={hkv} hd={hd} nq={nq}", flush=True)
        q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=9)
        qt, kt, vt = dev(q), dev(k), dev(v)
        if kind == "decode":
            d = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, q_base_pos=base, n_ctx=base + nq)
            ws = torch.full((capi.decode_ws_bytes(d, splits) // 4,), float("nan"), dtype=torch.float32, device="cuda")
            outs = [ops.attn_decode(qt, kt, vt, n_kv_heads=hkv, q_base_pos=base, n_ctx=base + nq,
                                    n_splits=splits, partial_ws=ws).cpu().numpy() for _ in range(3)]
        else:
            qt = qt.half()
            d = ops.make_desc_for(qt, kt, n_kv_heads=hkv, q_base_pos=base, n_ctx=base + nq)
            ws = torch.full((max(capi.prefill_ws_bytes(d), 256) // 4,), float("nan"), dtype=torch.float32,
                            device="cuda")
            outs = [ops.attn_prefill(qt, kt, vt, n_kv_heads=hkv, q_base_pos=base, n_ctx=base + nq,
                                     workspace=ws).float().cpu().numpy() for _ in range(3)]
        assert np.all(np.isfinite(outs[0])), kind
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2]), kind


def test_decode_split_count_invariance(hip):
    hq, hkv, hd, base = 16, 4, 128, 5000
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=base + 1, seed=8)
    outs = [run_decode(q, k, v, hkv=hkv, n_ctx=base + 1, q_base=base, n_splits=s) for s in (1, 3, 64, 157)]
    # P is rounded to f16 relative to each split's own max, so split counts agree to the
    # f16 rounding of P (2^-12 relative per term), not bit for bit.
    for o in outs[1:]:
        assert O.max_abs(o, outs[0]) < 1e-4 and O.rel_l2(o, outs[0]) < 3e-4


# ------------------------------------------------------------------ declines (device)

def test_declined_call_leaves_device_output_untouched(hip):
    q = torch.randn(4, 8, 96, device="cuda")
    k = torch.zeros(2, 16, 96, dtype=torch.float16, device="cuda")
    out = torch.full((4, 8, 96), 5.0, device="cuda")
    d = capi.make_desc(n_q_heads=8, n_kv_heads=2, head_dim=96, n_query=4, q_base_pos=12, n_ctx=16)
    rc = capi.prefill_raw(d, q.data_ptr(), k.data_ptr(), k.data_ptr(), out.data_ptr(), 0, 0,
                          torch.cuda.current_stream().cuda_stream, check=False)
    assert rc == capi.NEXUS_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert torch.all(out == 5.0)


# ------------------------------------------------------------------ full-size configs

def _sample_rows(nq, hq, n, seed):
    rng = np.random.default_rng(seed)
    rows = rng.choice(nq * hq, size=min(n, nq * hq), replace=False)
    # always include the first and last query rows (shortest and longest windows)
    return np.unique(np.concatenate([rows, [0, hq - 1, nq * hq - 1, (nq - 1) * hq]])).astype(np.int32)


@pytest.mark.parametrize("cfg", ["cfg2", "cfg3", "q35"])
def test_prefill_full_config_sampled_rows(hip, cfg):
    hq, hkv, hd = (16, 2, 256) if cfg == "q35" else (40, 8, 128)
    nq, base = (512, 4096) if cfg == "cfg2" else (8192, 0)
    n_ctx = base + nq
    print(f"[case] {cfg} full size", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=2024, q_f16=True)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=True, o_f16=True)
    assert np.all(np.isfinite(got))
    rows = _sample_rows(nq, hq, 256, 1)
    ref = O.attn_batch_rows(q, k, v, rows, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    g = got.reshape(nq * hq, hd)[rows]
    r = ref.reshape(nq * hq, hd)[rows]
    assert_close(g, r, f"{cfg} sampled rows")


def test_decode_full_cfg4(hip):
    hq, hkv, hd, n_ctx = 40, 8, 128, 61440
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=n_ctx, seed=4)
    got = run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=n_ctx - 1, n_splits=64)
    ref = O.cached_scores(q[0], k, v, n_kv_heads=hkv, pos=n_ctx - 1, n_threads=8)
    assert_close(got[0], ref, "cfg4 full")


def test_verify_full_cfg5(hip):
    hq, hkv, hd, base, nq = 16, 2, 256, 32768, 4
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=5)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=base + nq, q_base=base)      # routed to split-KV
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base, n_threads=8)
    assert_close(got, ref, "cfg5 full")


GATED_DECODE_CASES = [
    # (Hq, Hkv, hd, n_query, q_base, n_ctx, n_splits, o_f16)
    (40, 8, 128, 1, 3000, 3001, 1, False),      # one split: the kernel writes the output itself
    (40, 8, 128, 1, 3000, 3001, 64, True),      # split-KV: the combine applies the gate, f16 out
    (16, 2, 256, 4, 2000, 2004, 0, False),      # MTP verify layout
    (64, 1, 128, 1, 500, 501, 0, False),        # two row groups
]


@pytest.mark.parametrize("hq,hkv,hd,nq,base,n_ctx,splits,of16", GATED_DECODE_CASES)
def test_decode_gated(hip, hq, hkv, hd, nq, base, n_ctx, splits, of16):
    """Gated decode (transformer.h:8502-8515): the split combine or the single-split epilogue
    multiplies by sigmoid(gate)."""
    print(f"[case] decode gated hq={hq} hkv={hkv} hd={hd} nq={nq} ctx={n_ctx} splits={splits}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=n_ctx + 1)
    gate = make_gate(q.shape, n_ctx)
    got = run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, n_splits=splits, gate=gate, o_f16=of16)
    ref = O.gate_mul(O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8), gate)
    assert_close(got, ref, f"decode gated {hq}/{hkv} hd{hd} nq{nq} splits{splits}")
    plain = run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, n_splits=splits, o_f16=of16)
    sat = np.abs(gate) > 80
    np.testing.assert_array_equal(got[sat & (gate > 0)], plain[sat & (gate > 0)])
    assert not np.any(got[sat & (gate < 0)])


# ------------------------------------------- query magnitudes beyond N(0, 1)

@pytest.mark.parametrize("q_std", [4.0, 8.0])
@pytest.mark.parametrize("hq,hkv,hd,nq,base,qf16", [
    (40, 8, 128, 512, 4096, True),     # cfg2's shape, f16 queries used exactly as given
    (40, 8, 128, 512, 4096, False),    # cfg2's shape, f32 queries (f16 high part + residual)
    (16, 2, 256, 300, 600, True),      # head dim 256, f16 queries
    (8, 2, 128, 64, 3000, False),      # a short chunk in key splits (partials in raw units)
])
def test_prefill_precision_at_large_query_magnitudes(hip, q_std, hq, hkv, hd, nq, base, qf16):
    """Sharp softmaxes (queries of std 4 and 8): the scale is applied to the scores in f32, so
    f16 queries are not rounded a second time and f32 queries keep ~22 mantissa bits."""
    n_ctx = base + nq
    print(f"[case] prefill q_std={q_std} hq={hq} hkv={hkv} hd={hd} nq={nq} base={base} qf16={qf16}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=43,
                        q_f16=qf16, q_scale=q_std)
    got = run_prefill(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, q_f16=qf16)
    rows = _sample_rows(nq, hq, 1024, 3)
    ref = O.attn_batch_rows(q, k, v, rows, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    assert_close(got.reshape(nq * hq, hd)[rows], ref.reshape(nq * hq, hd)[rows],
                 f"prefill q_std={q_std} hd={hd} qf16={qf16}")


@pytest.mark.parametrize("q_std", [4.0, 8.0])
@pytest.mark.parametrize("hq,hkv,hd,nq,base,splits", [
    (40, 8, 128, 1, 20000, 64),        # decode
    (16, 2, 256, 4, 8000, 0),          # MTP verify
])
def test_decode_precision_at_large_query_magnitudes(hip, q_std, hq, hkv, hd, nq, base, splits):
    n_ctx = base + nq
    print(f"[case] decode q_std={q_std} hq={hq} hkv={hkv} hd={hd} nq={nq} base={base}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=44, q_scale=q_std)
    got = run_decode(q, k, v, hkv=hkv, n_ctx=n_ctx, q_base=base, n_splits=splits)
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_threads=8)
    assert_close(got, ref, f"decode q_std={q_std} hd={hd} nq={nq}")
