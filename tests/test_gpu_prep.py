"""GPU parity of the decode prep (nexus_hip_attn_decode_prep) against the CPU oracle.

The f32 outputs (q, gate, the K/V echo) agree with oracle_decode_prep to rounding (the
norm's sum of squares is reduced in a different order, and the GPU may fuse a multiply-add
in the rotation): max-abs 2e-5 at |x| <= ~4, relative 1e-5.  The f16 cache rows are
checked bit-exactly against the oracle's conversion of the kernel's own f32 echo, and the
conversions themselves bit-exactly on special values where the f32 input passes through
unchanged.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from nexus_amd import capi, ops

pytestmark = pytest.mark.gpu


def dev(x):
    if x.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host_u16(t):
    return t.cpu().numpy().view(np.uint16)


def conv(x, rne):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.uint16)
    (O.oracle().nx_f32_to_f16_rne_n if rne else O.oracle().nx_f32_to_f16_trunc_n)(x, out, x.size)
    return out


def rope_table(rot, pos, base=1e6):
    i = np.arange(rot // 2)
    ang = pos / np.power(base, 2.0 * i / max(rot, 1))
    return np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32)


PREP_CASES = [
    # (n_heads, n_kv, hd, rot, flags, pos, cap)
    (16, 2, 256, 64, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE, 4095, 4608),   # gated, partial RoPE
    (40, 8, 128, 128, capi.PREP_NO_GATE, 0, 2048),                                        # q/k norm, full RoPE
    (32, 8, 128, 128, capi.PREP_NO_GATE | capi.PREP_NO_Q_NORM | capi.PREP_NO_K_NORM, 77, 256),  # no head norm
    (8, 8, 64, 64, capi.PREP_NO_GATE | capi.PREP_NO_Q_NORM | capi.PREP_NO_K_NORM | capi.PREP_ROPE_INTERLEAVED, 9, 16),
    (4, 1, 512, 0, capi.PREP_Q_NORM_ADD_ONE, 3, 4),                                       # widest head, no RoPE
    (6, 3, 80, 32, capi.PREP_NO_GATE, 1, 2),                                             # ragged head (80 dims)
    (16, 2, 256, 64, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE | capi.PREP_TRUNC_STORE, 100, 128),
    (12, 4, 192, 96, capi.PREP_ROPE_INTERLEAVED | capi.PREP_K_NORM_ADD_ONE, 5, 6),       # gated, interleaved
    # rotations whose partners are exchanged through LDS (the others come from registers)
    (12, 4, 192, 96, capi.PREP_K_NORM_ADD_ONE, 5, 6),                                    # rotate_half, rot 96
    (8, 2, 256, 192, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_NO_GATE, 40, 64),              # rot 192
    (4, 2, 64, 48, capi.PREP_NO_GATE, 2, 8),                                              # rot 48, hd 64
]


@pytest.mark.parametrize("n_heads,n_kv,hd,rot,flags,pos,cap", PREP_CASES)
def test_decode_prep_vs_oracle(hip, n_heads, n_kv, hd, rot, flags, pos, cap):
    print(f"[case] prep heads={n_heads} kv={n_kv} hd={hd} rot={rot} flags={flags} pos={pos} cap={cap}", flush=True)
    rng = np.random.default_rng(n_heads * 1000 + hd + flags)
    gated = not flags & capi.PREP_NO_GATE
    qg = (rng.standard_normal((n_heads, (2 if gated else 1) * hd)) * 3).astype(np.float32)
    kraw = (rng.standard_normal((n_kv, hd)) * 3).astype(np.float32)
    vraw = rng.standard_normal((n_kv, hd)).astype(np.float32)
    qnw = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    knw = (0.2 * rng.standard_normal(hd)).astype(np.float32)
    tab = rope_table(rot, pos)
    kc0 = rng.integers(0, 1 << 15, (n_kv, cap, hd), dtype=np.uint16)
    vc0 = rng.integers(0, 1 << 15, (n_kv, cap, hd), dtype=np.uint16)
    rne = not flags & capi.PREP_TRUNC_STORE

    kc_t, vc_t = dev(kc0), dev(vc0)
    q_out, gate_out, kv_out = ops.decode_prep(
        dev(qg), dev(kraw), dev(vraw), kc_t, vc_t, pos=pos, rope_tab=dev(tab) if rot else None,
        q_norm_w=None if flags & capi.PREP_NO_Q_NORM else dev(qnw),
        k_norm_w=None if flags & capi.PREP_NO_K_NORM else dev(knw), gated=gated,
        q_norm_add_one=bool(flags & capi.PREP_Q_NORM_ADD_ONE), k_norm_add_one=bool(flags & capi.PREP_K_NORM_ADD_ONE),
        rope_interleaved=bool(flags & capi.PREP_ROPE_INTERLEAVED), eps=1e-6, trunc_store=not rne)
    torch.cuda.synchronize()
    r_q, r_gate, _, _, r_kv = O.decode_prep(qg, kraw, vraw, qnw, knw, tab if rot else np.zeros(1, np.float32),
                                            n_heads=n_heads, n_kv=n_kv, hd=hd, rot=rot, flags=flags & 63, eps=1e-6,
                                            pos=pos, cap=cap, rne=rne)
    got_q, got_kv = q_out.cpu().numpy(), kv_out.cpu().numpy()
    np.testing.assert_allclose(got_q, r_q, rtol=1e-5, atol=2e-5)
    np.testing.assert_allclose(got_kv, r_kv, rtol=1e-5, atol=2e-5)
    np.testing.assert_array_equal(got_kv[1], vraw)                      # V passes through untouched
    if gated:
        np.testing.assert_array_equal(gate_out.cpu().numpy(), qg[:, hd:])
    else:
        assert gate_out is None
    kc, vc = host_u16(kc_t), host_u16(vc_t)
    np.testing.assert_array_equal(kc[:, pos].reshape(-1), conv(got_kv[0], rne))
    np.testing.assert_array_equal(vc[:, pos].reshape(-1), conv(got_kv[1], rne))
    other = np.arange(cap) != pos
    np.testing.assert_array_equal(kc[:, other], kc0[:, other])
    np.testing.assert_array_equal(vc[:, other], vc0[:, other])


SPECIALS = np.array([
    0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, -65520.0, 1e6, np.inf, -np.inf, np.nan,
    6.1035156e-05, 6.0e-05, 5.9604645e-08, 2.9802322e-08, 2.98023259e-08, 8.9406967e-08, 1e-10, -3.0e-06,
    1.00048828125, 1.000244140625, 1.0007324, 2049.0, 2051.0, -2051.0, 0.33333334, 3.14159274,
], np.float32)


@pytest.mark.parametrize("trunc", [False, True])
def test_decode_prep_store_conversions_bit_exact(hip, trunc):
    """With both norms and RoPE off, K passes through unchanged, so the cache row is the pure
    f32 -> f16 conversion: round-to-nearest-even (ties, f16 subnormals, overflow to inf,
    NaN) or the host store's truncation (flush below the normal range, inf above)."""
    rng = np.random.default_rng(3)
    hd = 256
    vals = np.concatenate([SPECIALS, (rng.standard_normal(hd - SPECIALS.size) * 10.0 ** rng.integers(-9, 5, hd - SPECIALS.size))]).astype(np.float32)
    kraw = np.stack([vals, -vals[::-1]])
    vraw = kraw[::-1].copy()
    qg = np.ones((2, hd), np.float32)
    kc_t = dev(np.zeros((2, 3, hd), np.uint16))
    vc_t = dev(np.zeros((2, 3, hd), np.uint16))
    _, _, kv_out = ops.decode_prep(dev(qg), dev(kraw), dev(vraw), kc_t, vc_t, pos=2, rope_tab=None, gated=False,
                                   trunc_store=trunc)
    torch.cuda.synchronize()
    kv = kv_out.cpu().numpy()
    np.testing.assert_array_equal(kv[0].view(np.uint32), kraw.view(np.uint32))
    np.testing.assert_array_equal(host_u16(kc_t)[:, 2].reshape(-1), conv(kraw, not trunc))
    np.testing.assert_array_equal(host_u16(vc_t)[:, 2].reshape(-1), conv(vraw, not trunc))


LAYER_CASES = [
    # (n_heads, n_kv, hd, rot, flags, pos, cap, n_splits); n_splits 0 = the library's choice
    (16, 2, 256, 64, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE | capi.PREP_TRUNC_STORE, 4095, 4608, 0),
    (16, 2, 256, 64, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE, 100, 128, 7),   # key pos mid-split grid
    (40, 8, 128, 128, capi.PREP_NO_GATE, 0, 2048, 0),                      # the new row is the only key
    (32, 8, 128, 128, capi.PREP_NO_GATE | capi.PREP_NO_Q_NORM | capi.PREP_NO_K_NORM, 77, 256, 4),
    (8, 8, 64, 64, capi.PREP_NO_GATE | capi.PREP_ROPE_INTERLEAVED, 9, 16, 1),  # G = 1, one split
    (12, 4, 192, 96, capi.PREP_ROPE_INTERLEAVED | capi.PREP_K_NORM_ADD_ONE, 300, 320, 3),
    (64, 2, 128, 64, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE, 1000, 1024, 0),   # G = 32: two row tiles
    (64, 1, 64, 0, capi.PREP_TRUNC_STORE, 2500, 2560, 0),                  # G = 64: two row groups, no RoPE
    (12, 4, 192, 96, capi.PREP_K_NORM_ADD_ONE, 300, 320, 3),              # rotate_half rot 96: partners via LDS
    (16, 2, 256, 192, capi.PREP_Q_NORM_ADD_ONE | capi.PREP_K_NORM_ADD_ONE, 700, 768, 0),   # rot 192 via LDS
    (16, 4, 128, 32, capi.PREP_NO_GATE, 50, 64, 2),                       # rot 32: partners lane ^ 16
]


@pytest.mark.parametrize("n_heads,n_kv,hd,rot,flags,pos,cap,n_splits", LAYER_CASES)
def test_decode_layer_fused_vs_prep_then_decode(hip, n_heads, n_kv, hd, rot, flags, pos, cap, n_splits):
    """nexus_hip_attn_decode_layer (prep folded into the split-KV kernel, the new row attended
    from registers) against the two-step path (prep kernel, then the gated decode over the
    cache it wrote) on the same inputs and split count: the same cache rows and K/V echo bit
    for bit, outputs equal to f32 rounding; and the output against the CPU oracle (the
    oracle's prep, then forward_cached_scores over the cache, then the gate)."""
    print(f"[case] decode layer heads={n_heads} kv={n_kv} hd={hd} rot={rot} flags={flags} pos={pos} cap={cap} "
          f"splits={n_splits}", flush=True)
    rng = np.random.default_rng(n_heads * 7 + hd + pos)
    gated = not flags & capi.PREP_NO_GATE
    qg = (rng.standard_normal((n_heads, (2 if gated else 1) * hd)) * 2).astype(np.float32)
    kraw = (rng.standard_normal((n_kv, hd)) * 2).astype(np.float32)
    vraw = rng.standard_normal((n_kv, hd)).astype(np.float32)
    qnw = (0.2 * rng.standard_normal(hd)).astype(np.float32)
    knw = (0.2 * rng.standard_normal(hd)).astype(np.float32)
    tab = rope_table(rot, pos)
    # cache rows: N(0,1) in f16 below pos, garbage (NaN bit patterns included) from pos on
    kc0 = np.concatenate([np.float16(rng.standard_normal((n_kv, pos, hd))).view(np.uint16),
                          rng.integers(0, 1 << 16, (n_kv, cap - pos, hd), dtype=np.uint16)], axis=1)
    vc0 = np.concatenate([np.float16(rng.standard_normal((n_kv, pos, hd))).view(np.uint16),
                          rng.integers(0, 1 << 16, (n_kv, cap - pos, hd), dtype=np.uint16)], axis=1)
    kw = dict(pos=pos, rope_tab=dev(tab) if rot else None,
              q_norm_w=None if flags & capi.PREP_NO_Q_NORM else dev(qnw),
              k_norm_w=None if flags & capi.PREP_NO_K_NORM else dev(knw), gated=gated,
              q_norm_add_one=bool(flags & capi.PREP_Q_NORM_ADD_ONE),
              k_norm_add_one=bool(flags & capi.PREP_K_NORM_ADD_ONE),
              rope_interleaved=bool(flags & capi.PREP_ROPE_INTERLEAVED), eps=1e-6,
              trunc_store=bool(flags & capi.PREP_TRUNC_STORE))
    # two-step path
    kc_a, vc_a = dev(kc0), dev(vc0)
    q_out, gate_out, kv_a = ops.decode_prep(dev(qg), dev(kraw), dev(vraw), kc_a, vc_a, **kw)
    ref2 = ops.attn_decode(q_out[None], kc_a, vc_a, n_kv_heads=n_kv, q_base_pos=pos, n_ctx=pos + 1,
                           n_splits=n_splits, gate=gate_out[None] if gated else None)[0]
    # fused, on a workspace full of NaN (every partial it reads must be written first)
    kc_b, vc_b = dev(kc0), dev(vc0)
    desc = ops._prep_desc(dev(qg), dev(kraw), dev(vraw), kc_b, vc_b, **kw)
    ws = torch.full((max(capi.decode_layer_ws_bytes(desc, n_splits), 4) // 4,), float("nan"), device="cuda")
    out, kv_b = ops.decode_layer(dev(qg), dev(kraw), dev(vraw), kc_b, vc_b, n_splits=n_splits, partial_ws=ws, **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_u16(kc_b), host_u16(kc_a))
    np.testing.assert_array_equal(host_u16(vc_b), host_u16(vc_a))
    np.testing.assert_array_equal(kv_b.cpu().numpy(), kv_a.cpu().numpy())
    got, two = out.cpu().numpy(), ref2.cpu().numpy()
    assert np.all(np.isfinite(got))
    print(f"[parity] fused vs two-step max_abs={O.max_abs(got, two):.3e} rel_l2={O.rel_l2(got, two):.3e}")
    np.testing.assert_allclose(got, two, rtol=1e-5, atol=1e-6)
    # oracle: its own prep, then forward_cached_scores over the cache rows [0, pos], then the gate
    r_q, r_gate, r_kc, r_vc, _ = O.decode_prep(qg, kraw, vraw, qnw, knw, tab if rot else np.zeros(1, np.float32),
                                               n_heads=n_heads, n_kv=n_kv, hd=hd, rot=rot, flags=flags & 63,
                                               eps=1e-6, pos=pos, cap=cap, kc=kc0, vc=vc0,
                                               rne=not flags & capi.PREP_TRUNC_STORE)
    ref = O.cached_scores(r_q, r_kc, r_vc, n_kv_heads=n_kv, pos=pos, n_threads=8)
    if gated:
        ref = O.gate_mul(ref, r_gate)
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[parity] fused vs oracle max_abs={ma:.3e} rel_l2={rl:.3e}")
    assert ma < 2e-3 and rl < 1e-3


def test_decode_layer_declines_before_side_effects(hip):
    """Bad arguments return an error and touch neither the caches nor the outputs."""
    n_heads, n_kv, hd, pos, cap = 16, 2, 96, 5, 8                            # head dim 96: not a decode head dim
    qg = dev(np.ones((n_heads, 2 * hd), np.float32))
    kc = dev(np.zeros((n_kv, cap, hd), np.uint16))
    vc = dev(np.zeros((n_kv, cap, hd), np.uint16))
    x = dev(np.ones((n_kv, hd), np.float32))
    out = torch.full((n_heads, hd), 3.0, device="cuda")
    kvo = torch.full((2, n_kv, hd), 3.0, device="cuda")
    desc = capi.PrepDesc(n_heads, n_kv, hd, 0, pos, capi.PREP_NO_Q_NORM | capi.PREP_NO_K_NORM, cap, 1e-6, 0)
    assert capi.decode_layer_ws_bytes(desc, 0) == 0
    rc = capi.decode_layer_raw(desc, 0.0, qg.data_ptr(), x.data_ptr(), x.data_ptr(), 0, 0, 0, kc.data_ptr(),
                               vc.data_ptr(), kvo.data_ptr(), out.data_ptr(), 0, 1, 0, check=False)
    assert rc == capi.NEXUS_E_UNSUPPORTED
    desc = capi.PrepDesc(n_heads, n_kv, 128, 0, cap, capi.PREP_NO_Q_NORM | capi.PREP_NO_K_NORM, cap, 1e-6, 0)
    rc = capi.decode_layer_raw(desc, 0.0, qg.data_ptr(), x.data_ptr(), x.data_ptr(), 0, 0, 0, kc.data_ptr(),
                               vc.data_ptr(), kvo.data_ptr(), out.data_ptr(), 0, 1, 0, check=False)
    assert rc == capi.NEXUS_E_INVALID                                        # pos outside the cache
    torch.cuda.synchronize()
    assert torch.all(out == 3.0) and torch.all(kvo == 3.0)
    assert torch.all(kc == 0) and torch.all(vc == 0)
