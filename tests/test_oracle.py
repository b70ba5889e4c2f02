"""Pins for the CPU oracle (oracle/attn_oracle.c) -- CPU only.

Each oracle function is checked against something it does not restate: the reference's
own compiled code (oracle/_ref, when present), committed fixtures that code wrote
(tests/golden/golden_attn.npz), library routines (numpy float16), float64 brute force,
and closed forms chosen so that a dropped term, a wrong sign, an off-by-one in the
causal window or a transposed operand fails at least one of them.
"""
import numpy as np
import pytest

import oracle_lib as O
from nexus_amd.inputs import f32_to_f16_trunc, f16_to_f32, make_case, normal

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")


# ---------------------------------------------------------------- f16 conversions

def test_f16_decode_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    got = np.zeros(65536, np.float32)
    O.oracle().nx_f16_to_f32_n(bits, got, 65536)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@needs_ref
def test_f16_decode_exhaustive_vs_reference():
    r = O.ref()
    bits = np.arange(65536, dtype=np.uint16)
    got = np.zeros(65536, np.float32)
    O.oracle().nx_f16_to_f32_n(bits, got, 65536)
    want = np.array([r.ref_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _rand_f32(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return x[~np.isnan(x)]


def test_f16_rne_vs_numpy_2m_patterns():
    x = _rand_f32(2_000_000, 1)
    got = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_rne_n(x, got, x.size)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
    y = (normal(3, 200_000) * np.float32(1e-5)).astype(np.float32)     # dense in the subnormal range
    got = np.zeros(y.size, np.uint16)
    O.oracle().nx_f32_to_f16_rne_n(y, got, y.size)
    assert np.array_equal(got, y.astype(np.float16).view(np.uint16))


@needs_ref
def test_f16_rne_vs_reference():
    x = _rand_f32(100_000, 2)
    got = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_rne_n(x, got, x.size)
    r = O.ref()
    want = np.array([r.ref_f32_to_f16_rne(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


def test_f16_trunc_is_nearest_toward_zero():
    """Truncating store = the f16 neighbour of x toward zero, in the normal range."""
    x = _rand_f32(400_000, 4)
    ax = np.abs(x)
    x = x[(ax >= 2.0**-14) & (ax < 65504.0)]
    got = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_trunc_n(x, got, x.size)
    h = got.view(np.float16)
    hv = h.astype(np.float64)
    assert np.all(np.abs(hv) <= np.abs(x.astype(np.float64)))
    nxt = np.nextafter(h, np.copysign(np.float16(np.inf), h)).astype(np.float64)
    assert np.all(np.abs(nxt) > np.abs(x.astype(np.float64)))
    assert np.array_equal(np.signbit(hv), np.signbit(x))


def test_f16_trunc_special_cases():
    f = O.oracle().nx_f32_to_f16_trunc
    assert f(0.0) == 0x0000 and f(-0.0) == 0x8000
    assert f(6.0e-5) == 0x0000            # below 2^-14: flushed (no subnormals)
    assert f(-3.0e-5) == 0x8000
    assert f(2.0**-14) == 0x0400
    assert f(65504.0) == 0x7BFF and f(65519.0) == 0x7BFF
    assert f(65536.0) == 0x7C00 and f(-1e9) == 0xFC00
    assert f(float("inf")) == 0x7C00 and f(float("nan")) == 0x7C00
    assert f(1.0 + 2.0**-10 + 2.0**-11) == 0x3C01     # truncation, not rounding


def test_f16_trunc_matches_numpy_restatement():
    x = _rand_f32(300_000, 5)
    got = np.zeros(x.size, np.uint16)
    O.oracle().nx_f32_to_f16_trunc_n(x, got, x.size)
    assert np.array_equal(got, f32_to_f16_trunc(x))


def test_kv_store_golden(golden):
    """KVCache::store + pack_k/pack_v bits written by the reference's own KVCache."""
    hkv, hd, ntok = golden["kv_meta"]
    kf, vf = golden["kv_kf"], golden["kv_vf"]
    for src, packed in ((kf, golden["kv_kpacked"]), (vf, golden["kv_vpacked"])):
        bits = np.zeros(src.size, np.uint16)
        O.oracle().nx_f32_to_f16_trunc_n(np.ascontiguousarray(src.ravel()), bits, src.size)
        mine = bits.reshape(ntok, hkv, hd).transpose(1, 0, 2)     # [tok][h][d] -> packed [h][tok][d]
        assert np.array_equal(mine, packed)
        assert np.array_equal(f32_to_f16_trunc(src).reshape(ntok, hkv, hd).transpose(1, 0, 2), packed)


# ------------------------------------------------------- decode: forward_cached_scores

@pytest.mark.parametrize("name", ["dec_a", "dec_b", "dec_c", "dec_d"])
def test_cached_scores_vs_golden(golden, name):
    hq, hkv, hd, pos = (int(x) for x in golden[f"{name}_meta"])
    scale, cap = (float(x) for x in golden[f"{name}_fmeta"])
    y = O.cached_scores(golden[f"{name}_q"], golden[f"{name}_k"], golden[f"{name}_v"],
                        n_kv_heads=hkv, pos=pos, scale=scale, softcap=cap)
    ref = golden[f"{name}_out"]
    assert O.max_abs(y, ref) < 2e-6 and O.rel_l2(y, ref) < 1e-5


@needs_ref
@pytest.mark.parametrize("hq,hkv,hd,pos,cap", [(16, 4, 128, 1500, 0.0), (40, 8, 128, 700, 0.0),
                                               (6, 3, 64, 2, 0.0), (8, 1, 256, 333, 50.0)])
def test_cached_scores_vs_reference(hq, hkv, hd, pos, cap):
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=pos + 1,
                        kv_stride=pos + 17, seed=pos)
    y = O.cached_scores(q[0], k, v, n_kv_heads=hkv, pos=pos, softcap=cap, n_threads=4)
    r = O.ref_cached_scores(q[0], k, v, n_kv_heads=hkv, pos=pos, softcap=cap, n_threads=4)
    assert O.max_abs(y, r) < 2e-6 and O.rel_l2(y, r) < 1e-5


# ------------------------------------------------------------ prefill: attn_batch_cpu

def test_attn_batch_vs_golden_prefill(golden):
    """Each chunked-prefill row equals the reference's decode at that query's position."""
    hq, hkv, hd, q_base, nq, n_ctx = (int(x) for x in golden["pre_a_meta"])
    y = O.attn_batch(golden["pre_a_q"], golden["pre_a_k"], golden["pre_a_v"], n_kv_heads=hkv,
                     n_ctx=n_ctx, q_base_pos=q_base)
    ref = golden["pre_a_out"]
    assert O.max_abs(y, ref) < 2e-6 and O.rel_l2(y, ref) < 1e-5


@needs_ref
@pytest.mark.parametrize("hq,hkv,hd,q_base,nq,extra", [(8, 2, 128, 200, 33, 0), (5, 1, 64, 0, 40, 7),
                                                        (12, 4, 256, 31, 9, 3)])
def test_attn_batch_rows_vs_reference_decode(hq, hkv, hd, q_base, nq, extra):
    """attn_batch row i == forward_cached_scores at q_base + i; keys past the query
    (n_ctx > q_base + nq would not change it) and the stride padding are ignored."""
    n_ctx = q_base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx,
                        kv_stride=n_ctx + extra, seed=hq * 7 + nq)
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=q_base)
    for i in range(nq):
        r = O.ref_cached_scores(q[i], k, v, n_kv_heads=hkv, pos=q_base + i)
        assert O.max_abs(y[i], r) < 2e-6 and O.rel_l2(y[i], r) < 1e-5, i


# the reference's own batched-attention test shapes (test_attn_batch.cpp:183-204), N scaled down
REF_TEST_CASES = [
    ("qwen_full_hd256", 24, 4, 256, 96, 0, 0, 0.0),
    ("mha_hd128", 32, 32, 128, 64, 0, 0, 0.0),
    ("gqa_hd128", 32, 8, 128, 64, 0, 0, 0.0),
    ("gqa_hd64", 16, 4, 64, 100, 0, 0, 0.0),
    ("continuation", 24, 4, 256, 32, 600, 0, 0.0),
    ("swa_window256", 32, 8, 128, 300, 0, 256, 0.0),
    ("softcap30_hd128", 16, 16, 128, 80, 0, 0, 30.0),
    ("N1_hd256", 24, 4, 256, 1, 0, 0, 0.0),
]


@pytest.mark.parametrize("name,hq,hkv,hd,nq,base,sw,cap", REF_TEST_CASES)
def test_attn_batch_vs_f64_bruteforce(name, hq, hkv, hd, nq, base, sw, cap):
    n_ctx = base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=len(name))
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw,
                     softcap=cap, n_threads=8)
    r = O.naive_f64(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, sliding_window=sw, softcap=cap)
    assert O.max_abs(y, r) < 2e-4          # test_attn_batch.cpp:169


def test_closed_form_single_key():
    q, k, v = make_case(n_q_heads=4, n_kv_heads=2, head_dim=64, n_query=3, n_ctx=1, seed=3)
    y = O.attn_batch(q, k, v, n_kv_heads=2, n_ctx=1, q_base_pos=0)
    vv = f16_to_f32(v[:, 0])                           # [Hkv][hd]
    for h in range(4):
        for i in range(3):
            assert np.array_equal(y[i, h], vv[h * 2 // 4])


def test_closed_form_zero_query_is_mean_of_visible_values():
    hq, hkv, hd, base, nq = 6, 3, 64, 10, 5
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=4)
    q[:] = 0.0
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base)
    vf = f16_to_f32(v)
    for i in range(nq):
        for h in range(hq):
            want = vf[h * hkv // hq, : base + i + 1].mean(axis=0)
            assert np.max(np.abs(y[i, h] - want)) < 1e-5


def test_closed_form_one_hot_key_selects_its_value():
    """K_j = c*q for one key j (large c), others orthogonal-ish: out ~= V_j."""
    hd = 64
    q = np.zeros((1, 1, hd), np.float32)
    q[0, 0, 3] = 1.0
    n_ctx = 9
    kf = np.zeros((1, n_ctx, hd), np.float32)
    kf[0, 5, 3] = 200.0
    k = kf.astype(np.float16).view(np.uint16)
    v = normal(9, n_ctx * hd).reshape(1, n_ctx, hd).astype(np.float16).view(np.uint16)
    y = O.attn_batch(q, k, v, n_kv_heads=1, n_ctx=n_ctx, q_base_pos=n_ctx - 1)
    assert np.max(np.abs(y[0, 0] - f16_to_f32(v[0, 5]))) < 1e-6
    # the same key beyond the query's position is masked: query at position 4 cannot see key 5
    y2 = O.attn_batch(q, k, v, n_kv_heads=1, n_ctx=n_ctx, q_base_pos=4)
    assert np.max(np.abs(y2[0, 0] - f16_to_f32(v[0, :5]).mean(axis=0))) < 1e-5


def test_window_of_one_returns_own_value():
    hq, hkv, hd, base, nq = 4, 2, 64, 20, 6
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=5)
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base, sliding_window=1)
    vf = f16_to_f32(v)
    for i in range(nq):
        for h in range(hq):
            assert np.array_equal(y[i, h], vf[h * hkv // hq, base + i])


def test_softcap_limits():
    hq, hkv, hd, nq = 4, 2, 64, 12
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=nq, seed=6)
    plain = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=nq, q_base_pos=0)
    huge = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=nq, q_base_pos=0, softcap=1e6)
    assert O.max_abs(plain, huge) < 1e-6
    tiny = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=nq, q_base_pos=0, softcap=1e-6)
    vf = f16_to_f32(v)
    for i in range(nq):
        for h in range(hq):
            assert np.max(np.abs(tiny[i, h] - vf[h * hkv // hq, : i + 1].mean(axis=0))) < 1e-4


def test_queries_past_the_cache_see_all_keys():
    """q_base + i >= n_ctx: the window ends at n_ctx - 1 (transformer.h:8670)."""
    hq, hkv, hd = 4, 1, 64
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=3, n_ctx=10, seed=8)
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=10, q_base_pos=20)
    r = O.naive_f64(q, k, v, n_kv_heads=hkv, n_ctx=10, q_base_pos=20)
    assert O.max_abs(y, r) < 1e-6
    y0 = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=10, q_base_pos=9)
    assert O.max_abs(y, y0) < 1e-7


def test_chunked_rows_equal_cold_prefill_rows():
    hq, hkv, hd, base, nq = 8, 2, 128, 48, 16
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=base + nq, n_ctx=base + nq, seed=9)
    cold = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=0)
    chunk = O.attn_batch(q[base:], k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base)
    assert np.array_equal(chunk, cold[base:])


def test_gqa_head_permutation_equivariance():
    hq, hkv, hd, nq = 6, 2, 64, 10
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=nq, seed=10)
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=nq, q_base_pos=0)
    perm_kv = [1, 0]
    perm_q = [3, 4, 5, 0, 1, 2]
    y2 = O.attn_batch(q[:, perm_q], k[perm_kv], v[perm_kv], n_kv_heads=hkv, n_ctx=nq, q_base_pos=0)
    assert np.array_equal(y2, y[:, perm_q])


def test_causality_future_keys_do_not_matter():
    hq, hkv, hd, nq = 4, 2, 64, 8
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=nq + 5, seed=12)
    y = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=nq + 5, q_base_pos=0)
    k2, v2 = k.copy(), v.copy()
    k2[:, nq:] ^= 0x1234
    v2[:, nq:] ^= 0x0F0F
    y2 = O.attn_batch(q, k2, v2, n_kv_heads=hkv, n_ctx=nq + 5, q_base_pos=0)
    assert np.array_equal(y, y2)


# ------------------------------------------------------------ split-K partials/combine

@pytest.mark.parametrize("chunk", [1, 7, 32, 128, 1000])
def test_split_combine_equals_unsplit(chunk):
    hq, hkv, hd, pos = 8, 2, 128, 900
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=pos + 1, seed=13)
    n_chunks = (pos + 1 + chunk - 1) // chunk
    part = O.split_partials(q, k, v, n_kv_heads=hkv, n_ctx=pos + 1, q_base_pos=pos, n_chunks=n_chunks, chunk=chunk)
    y = O.split_combine(part).reshape(1, hq, hd)
    r = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=pos + 1, q_base_pos=pos)
    assert O.max_abs(y, r) < 2e-6 and O.rel_l2(y, r) < 1e-5


@pytest.mark.parametrize("nq,chunk", [(1, 37), (3, 64)])
def test_split_partials_meaning_per_chunk(nq, chunk):
    """Each partial is (acc, m, l) of its chunk alone, as qwen35_attn_part.comp:62-70 writes
    it: m = the chunk's max scaled score (natural-log units), l = sum_k e^{s_k - m},
    acc = sum_k e^{s_k - m} v_k over the chunk's visible keys -- checked in float64 numpy per
    chunk, so a units or offset mistake shared by the partial and the combine is caught."""
    hq, hkv, hd, base = 4, 2, 64, 250
    n_ctx = base + nq
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=17)
    n_chunks = (n_ctx + chunk - 1) // chunk
    scale = 1.0 / np.sqrt(hd)
    part = O.split_partials(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=base, n_chunks=n_chunks, chunk=chunk)
    part = part.reshape(nq * hq, n_chunks, hd + 2)
    kf = k.view(np.float16).astype(np.float64)
    vf = v.view(np.float16).astype(np.float64)
    for qi in range(nq):
        last = min(base + qi, n_ctx - 1)
        for h in range(hq):
            kv = h * hkv // hq
            s = (kf[kv, : last + 1] @ q[qi, h].astype(np.float64)) * scale
            for c in range(n_chunks):
                lo, hi = c * chunk, min((c + 1) * chunk, last + 1)
                pr = part[qi * hq + h, c]
                if lo >= hi:                       # no visible key: l = 0, acc = 0
                    assert pr[hd + 1] == 0.0 and not np.any(pr[:hd])
                    continue
                m = s[lo:hi].max()
                e = np.exp(s[lo:hi] - m)
                assert abs(pr[hd] - m) < 1e-5 * max(1.0, abs(m)), (qi, h, c)
                assert abs(pr[hd + 1] - e.sum()) < 1e-5 * e.sum()
                np.testing.assert_allclose(pr[:hd], e @ vf[kv, lo:hi], rtol=1e-4, atol=1e-5)


def test_split_partials_causal_drafts():
    """Speculative verify rows: drafts at q_base + i see keys <= q_base + i."""
    hq, hkv, hd, base, nq = 8, 1, 256, 500, 4
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=base + nq, seed=14)
    part = O.split_partials(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base, n_chunks=8, chunk=63)
    y = O.split_combine(part).reshape(nq, hq, hd)
    r = O.naive_f64(q, k, v, n_kv_heads=hkv, n_ctx=base + nq, q_base_pos=base)
    assert O.max_abs(y, r) < 1e-5


# ------------------------------------------------------------------ output gate, decode prep

def test_gate_mul_sigmoid_and_clamps():
    """oracle_gate_mul == out * expit(gate) inside (-80, 80); exactly out / 0 beyond."""
    from scipy.special import expit
    rng = np.random.default_rng(11)
    z = rng.uniform(-79.9, 79.9, 4096).astype(np.float32)
    out = rng.standard_normal(4096).astype(np.float32)
    got = O.gate_mul(out, z)
    np.testing.assert_allclose(got, out * expit(z.astype(np.float64)), rtol=2e-6, atol=1e-30)
    z2 = np.array([80.5, 1e3, np.float32(3e38), -80.5, -1e3, 0.0], np.float32)
    o2 = np.array([1.5, -2.0, 3.0, 4.0, -5.0, 6.0], np.float32)
    np.testing.assert_array_equal(O.gate_mul(o2, z2), np.array([1.5, -2.0, 3.0, 0.0, -0.0, 3.0], np.float32))


def _prep_inputs(rng, n_heads, n_kv, hd, rot, gated, pos):
    qg = rng.standard_normal((n_heads, (2 if gated else 1) * hd)).astype(np.float32) * 3
    kraw = rng.standard_normal((n_kv, hd)).astype(np.float32) * 3
    vraw = rng.standard_normal((n_kv, hd)).astype(np.float32)
    qnw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    knw = (0.1 * rng.standard_normal(hd)).astype(np.float32)
    i = np.arange(rot // 2)
    ang = pos / np.power(1e7, 2.0 * i / rot)
    tab = np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32)
    return qg, kraw, vraw, qnw, knw, tab


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("zc", [False, True])
def test_prep_norm_vs_reference_rms_norm(zc):
    """Head norm without RoPE (identity table): the reference's cpu::rms_norm with w, or
    with 1 + w for the zero-centred form (nx_rms_norm_add_one is rms_norm with 1 + w)."""
    rng = np.random.default_rng(5)
    n_heads, n_kv, hd, rot = 4, 2, 128, 32
    qg, kraw, vraw, qnw, knw, _ = _prep_inputs(rng, n_heads, n_kv, hd, rot, False, 0)
    tab = np.concatenate([np.ones(rot // 2), np.zeros(rot // 2)]).astype(np.float32)
    flags = O.PREP_NO_GATE | (O.PREP_Q_ZC | O.PREP_K_ZC if zc else 0)
    q_out, _, _, _, kv_out = O.decode_prep(qg, kraw, vraw, qnw, knw, tab, n_heads=n_heads, n_kv=n_kv, hd=hd,
                                           rot=rot, flags=flags, eps=1e-6, pos=0, cap=1)
    for h in range(n_heads):
        ref = O.ref_rms_norm(qg[h], qnw + 1 if zc else qnw, 1e-6)
        np.testing.assert_allclose(q_out[h], ref, rtol=2e-6, atol=1e-7)
    for h in range(n_kv):
        np.testing.assert_allclose(kv_out[0, h], O.ref_rms_norm(kraw[h], knw + 1 if zc else knw, 1e-6),
                                   rtol=2e-6, atol=1e-7)
        np.testing.assert_array_equal(kv_out[1, h], vraw[h])          # V: no norm, no RoPE


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("layout", [0, 1])
def test_prep_rope_vs_reference_rope_apply(layout):
    """Full-width RoPE with the standard angles (base 1e4): the reference's own rope_apply,
    interleaved (layout 0) and rotate_half (layout 1).  The reference takes cos/sin of a float
    angle near 777 rad in float; the table here rounds the double value, so a few ulp of |x| differ."""
    rng = np.random.default_rng(6)
    hd, pos, base = 64, 777, 10000.0
    x = rng.standard_normal((1, hd)).astype(np.float32)
    i = np.arange(hd // 2)
    theta = (np.float32(pos) * (np.float32(1) / np.power(np.float32(base), (2 * i).astype(np.float32) / np.float32(hd))))
    tab = np.concatenate([np.cos(theta.astype(np.float64)), np.sin(theta.astype(np.float64))]).astype(np.float32)
    flags = O.PREP_NO_GATE | O.PREP_NO_QNORM | O.PREP_NO_KNORM | (O.PREP_INTERLEAVED if layout == 0 else 0)
    q_out, *_ = O.decode_prep(x, x, x, None, None, tab, n_heads=1, n_kv=1, hd=hd, rot=hd, flags=flags,
                              eps=1e-6, pos=0, cap=1)           # the angle is in the table; pos is the store row
    np.testing.assert_allclose(q_out[0], O.ref_rope(x[0], pos, hd, base, layout), rtol=0, atol=6e-5)


def test_prep_rope_invariants():
    """Pair norms are preserved, the unrotated tail is untouched, rotating by a then b equals
    rotating by a+b, and rotate_half equals interleaved under the pair permutation."""
    rng = np.random.default_rng(7)
    n_heads, hd, rot = 3, 128, 32
    x = rng.standard_normal((n_heads, hd)).astype(np.float32)
    a, b = rng.uniform(-3, 3, rot // 2), rng.uniform(-3, 3, rot // 2)
    t = lambda ang: np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32)
    base = dict(n_heads=n_heads, n_kv=1, hd=hd, rot=rot, eps=1e-6, pos=0, cap=1)
    kv = np.zeros((1, hd), np.float32)
    f = O.PREP_NO_GATE | O.PREP_NO_QNORM | O.PREP_NO_KNORM
    ya = O.decode_prep(x, kv, kv, None, None, t(a), flags=f, **base)[0]
    yab = O.decode_prep(ya, kv, kv, None, None, t(b), flags=f, **base)[0]
    y = O.decode_prep(x, kv, kv, None, None, t(a + b), flags=f, **base)[0]
    np.testing.assert_allclose(yab, y, atol=3e-5)
    half = rot // 2
    np.testing.assert_allclose(ya[:, :half] ** 2 + ya[:, half:rot] ** 2, x[:, :half] ** 2 + x[:, half:rot] ** 2, rtol=1e-5)
    np.testing.assert_array_equal(ya[:, rot:], x[:, rot:])
    perm = np.empty(rot, np.int64)
    perm[0::2], perm[1::2] = np.arange(half), np.arange(half) + half     # interleaved slot -> half-split slot
    xi = x.copy()
    xi[:, :rot] = x[:, perm]
    yi = O.decode_prep(xi, kv, kv, None, None, t(a), flags=f | O.PREP_INTERLEAVED, **base)[0]
    np.testing.assert_allclose(yi[:, :rot], ya[:, perm], atol=1e-6)


def test_prep_layout_gate_and_store():
    """Gated layout: q from the first half of each head row, the raw gate from the second;
    K/V land in row `pos` of [n_kv][cap][hd] with the chosen f16 conversion, other rows
    untouched; kv_out holds the f32 values that were stored."""
    rng = np.random.default_rng(8)
    n_heads, n_kv, hd, rot, pos, cap = 4, 2, 64, 16, 5, 9
    qg, kraw, vraw, qnw, knw, tab = _prep_inputs(rng, n_heads, n_kv, hd, rot, True, pos)
    kc0 = rng.integers(0, 1 << 16, (n_kv, cap, hd), dtype=np.uint16)
    vc0 = rng.integers(0, 1 << 16, (n_kv, cap, hd), dtype=np.uint16)
    for rne in (False, True):
        q_out, gate_out, kc, vc, kv_out = O.decode_prep(qg, kraw, vraw, qnw, knw, tab, n_heads=n_heads, n_kv=n_kv,
                                                        hd=hd, rot=rot, flags=0, eps=1e-6, pos=pos, cap=cap,
                                                        kc=kc0, vc=vc0, rne=rne)
        np.testing.assert_array_equal(gate_out, qg[:, hd:])
        plain = O.decode_prep(qg[:, :hd], kraw, vraw, qnw, knw, tab, n_heads=n_heads, n_kv=n_kv, hd=hd, rot=rot,
                              flags=O.PREP_NO_GATE, eps=1e-6, pos=pos, cap=cap, rne=rne)
        np.testing.assert_array_equal(q_out, plain[0])
        conv = O.oracle().nx_f32_to_f16_rne_n if rne else O.oracle().nx_f32_to_f16_trunc_n
        for which, cache, c0 in ((0, kc, kc0), (1, vc, vc0)):
            want = np.zeros(n_kv * hd, np.uint16)
            conv(np.ascontiguousarray(kv_out[which].reshape(-1)), want, want.size)
            np.testing.assert_array_equal(cache[:, pos], want.reshape(n_kv, hd))
            keep = np.ones(cap, bool)
            keep[pos] = False
            np.testing.assert_array_equal(cache[:, keep], c0[:, keep])


# ------------------------------------------------------------------ KV session formats

KV_UNIFORM = ([(2, 64)] * 3, 8, 5, False)                                   # geom, stride, n_tok, per_layer
KV_PER_LAYER = ([(2, 64), (0, 0), (4, 128), (1, 256), (0, 0)], 7, 6, True)   # layers without KV, mixed dims
KV_CASES = {"uniform": KV_UNIFORM, "per_layer": KV_PER_LAYER}


@needs_ref
@pytest.mark.parametrize("name", list(KV_CASES))
@pytest.mark.parametrize("n_tok_delta", [0, -2])
def test_kv_cache_image_matches_reference(name, n_tok_delta, tmp_path):
    """NXKVCACH bytes: the restatement == KVCache::save_to_buffer == KVCache::save(path);
    a layer whose slots were never written is saved as zeros."""
    geom, stride, n_tok, per_layer = KV_CASES[name]
    n_tok += n_tok_delta
    c = O.KvCache.random(geom, stride, seed=1, empty=(2,) if name == "per_layer" else ())
    mine = O.kv_cache_save(c, n_tok)
    ref = O.ref_kv_save_cache(c, n_tok, per_layer)
    assert mine == ref
    O.ref_kv_save_file(tmp_path / "kv.bin", c, n_tok, per_layer)
    assert (tmp_path / "kv.bin").read_bytes() == ref
    hdr = np.frombuffer(ref[8:24], np.int32)
    assert ref[:8] == b"NXKVCACH" and list(hdr) == [len(geom), max(g[0] for g in geom), max(g[1] for g in geom), n_tok]


@needs_ref
@pytest.mark.parametrize("name", list(KV_CASES))
def test_kv_layer_record_matches_reference(name):
    geom, stride, n_tok, per_layer = KV_CASES[name]
    c = O.KvCache.random(geom, stride, seed=2)
    for l in range(len(geom)):
        mine = O.kv_layer_save(c, l, n_tok)
        assert mine == O.ref_kv_save_layer(c, l, n_tok, per_layer), l
        assert (mine == b"") == (geom[l][0] == 0)


def _same_rows(a, b, n_tok):
    for l, (h, _) in enumerate(a.geom):
        if h:
            np.testing.assert_array_equal(a.k[l][:, :n_tok], b.k[l][:, :n_tok])
            np.testing.assert_array_equal(a.v[l][:, :n_tok], b.v[l][:, :n_tok])


@needs_ref
@pytest.mark.parametrize("name", list(KV_CASES))
def test_kv_loaders_agree_with_reference(name):
    """Each loader reads the other's image back to the same rows; a record restores its layer."""
    geom, stride, n_tok, per_layer = KV_CASES[name]
    c = O.KvCache.random(geom, stride, seed=3)
    n, back = O.kv_cache_load(O.ref_kv_save_cache(c, n_tok, per_layer), geom, stride)
    assert n == n_tok
    _same_rows(back, c, n_tok)
    n, back = O.ref_kv_load_cache(O.kv_cache_save(c, n_tok), geom, stride, per_layer)
    assert n == n_tok
    _same_rows(back, c, n_tok)
    l = 2 if name == "per_layer" else 1
    rec = O.kv_layer_save(c, l, n_tok)
    n, layer, mine = O.kv_layer_load(rec, geom, stride)
    nr, theirs = O.ref_kv_load_layer(rec, geom, stride, per_layer)
    assert (n, layer) == (n_tok, l) and nr == n_tok
    for x in (mine, theirs):
        np.testing.assert_array_equal(x.k[l][:, :n_tok], c.k[l][:, :n_tok])
        np.testing.assert_array_equal(x.v[l][:, :n_tok], c.v[l][:, :n_tok])


@needs_ref
def test_kv_legacy_layout_read_like_the_reference():
    """The legacy image (every layer at the header geometry, zero blocks for layers without KV)
    is what the reference's loader still accepts: it reads the restatement's legacy image to
    the same rows as the restatement's own loader."""
    geom, stride, n_tok, _ = KV_PER_LAYER
    geom = [(4, 128), (0, 0), (4, 128), (0, 0)]          # KV layers at the header geometry
    c = O.KvCache.random(geom, stride, seed=4)
    legacy = O.kv_cache_save(c, n_tok, legacy=True)
    assert len(legacy) > len(O.kv_cache_save(c, n_tok))
    n, theirs = O.ref_kv_load_cache(legacy, geom, stride, True)
    assert n == n_tok
    _same_rows(theirs, c, n_tok)
    n, mine = O.kv_cache_load(legacy, geom, stride)
    assert n == n_tok
    _same_rows(mine, c, n_tok)


@needs_ref
def test_kv_refusals_agree_with_reference():
    geom, stride, n_tok, per_layer = KV_PER_LAYER
    c = O.KvCache.random(geom, stride, seed=5)
    img = O.kv_cache_save(c, n_tok)
    bad = [img[:-1], b"NXKVCACX" + img[8:], img[:20]]
    other = [(2, 64), (0, 0), (4, 128), (1, 128), (0, 0)]  # a different model
    for data, g in [(x, geom) for x in bad] + [(img, other)]:
        assert O.kv_cache_load(data, g, stride)[0] == -1
        assert O.ref_kv_load_cache(data, g, stride, per_layer)[0] == -1
    rec = O.kv_layer_save(c, 3, n_tok)
    for data in (rec[:-1], b"NXKVLYR2" + rec[8:]):
        assert O.kv_layer_load(data, geom, stride)[0] == -1
        assert O.ref_kv_load_layer(data, geom, stride, per_layer)[0] == -1


def test_kv_images_vs_golden(golden_kv):
    """The restatement reproduces the images the reference wrote (tests/golden/golden_kv.npz)."""
    g = golden_kv
    for name, (geom, stride, n_tok, _) in KV_CASES.items():
        c = O.KvCache(geom, stride, [g.get(f"{name}_k{l}") for l in range(len(geom))],
                      [g.get(f"{name}_v{l}") for l in range(len(geom))])
        assert O.kv_cache_save(c, n_tok) == g[f"{name}_image"].tobytes()
        for l in range(len(geom)):
            assert O.kv_layer_save(c, l, n_tok) == g[f"{name}_layer{l}"].tobytes()
