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
