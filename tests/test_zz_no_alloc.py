"""GPU test of nexus_hip_attn_decode_noalloc (the decode entry point that allocates nothing):
through the C ABI its output must equal nexus_hip_attn_decode_gated's on the same inputs and
split count (same kernels, so bit for bit), on two calls in a row, the second one smaller, so
partials left in the library's array by the first call cannot leak into the second.  Both are
also checked against the CPU oracle at the north-star tolerance."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from nexus_amd import capi
from nexus_amd.inputs import make_case

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
REL_L2 = 1e-3


def _dev(x):
    if x.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _run_pair(hq, hkv, hd, nq, pos, n_splits, seed, gated):
    n_ctx = pos + nq
    print(f"[case] noalloc hq={hq} hkv={hkv} hd={hd} nq={nq} pos={pos} splits={n_splits} gated={gated}", flush=True)
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=n_ctx, seed=seed)
    gate = (np.random.default_rng(seed + 1).standard_normal(q.shape) * 3).astype(np.float32) if gated else None
    desc = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, q_base_pos=pos, n_ctx=n_ctx)
    splits = n_splits if n_splits > 0 else capi.decode_default_splits(desc)
    qd, kd, vd = _dev(q), _dev(k), _dev(v)
    gd = _dev(gate) if gated else None
    gptr = gd.data_ptr() if gated else 0
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(capi.decode_ws_bytes(desc, splits) // 4 + 64, device="cuda")
    ref_out = torch.full(q.shape, float("nan"), device="cuda")
    capi.decode_raw(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ref_out.data_ptr(), ws.data_ptr(), splits,
                    stream, gate=gptr)
    out = torch.full(q.shape, float("nan"), device="cuda")
    capi.decode_noalloc_raw(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), splits, stream,
                            gate=gptr)
    torch.cuda.synchronize()
    got, want = out.cpu().numpy(), ref_out.cpu().numpy()
    assert np.array_equal(got, want), f"noalloc differs from decode_gated: max diff {np.nanmax(np.abs(got - want))}"
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=n_ctx, q_base_pos=pos, n_threads=8)
    if gated:
        ref = O.gate_mul(ref, gate)
    ma, rl = O.max_abs(got, ref), O.rel_l2(got, ref)
    print(f"[parity] noalloc max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma < MAX_ABS and rl < REL_L2


@pytest.mark.parametrize("gated", [False, True])
def test_noalloc_matches_workspace_entry_two_calls(hip, gated):
    # first call: 4-draft verify at hd 256 over 8k keys, 64 splits (4.2 MB of partials)
    _run_pair(16, 2, 256, 4, 8192, 64, seed=31, gated=gated)
    # second call, smaller: one token at hd 128 over 3000 keys, library-chosen splits
    _run_pair(8, 2, 128, 1, 2999, 0, seed=32, gated=gated)


def test_noalloc_refuses_partials_beyond_its_array(hip):
    hq, hkv, hd, nq, pos = 32, 1, 256, 4, 20000
    desc = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, q_base_pos=pos, n_ctx=pos + nq)
    splits = 512                                  # 128 rows x 512 x 258 x 4 B = 67 MB > 8 MiB
    assert capi.decode_ws_bytes(desc, splits) > capi.DECODE_NOALLOC_SCRATCH_BYTES
    q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, n_ctx=pos + nq, seed=5)
    qd, kd, vd = _dev(q), _dev(k), _dev(v)
    out = torch.full(q.shape, 7.0, device="cuda")
    rc = capi.decode_noalloc_raw(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), splits,
                                 torch.cuda.current_stream().cuda_stream, check=False)
    torch.cuda.synchronize()
    assert rc == capi.NEXUS_E_WORKSPACE, (rc, capi.last_error())
    assert "partials" in capi.last_error()
    assert bool((out == 7.0).all())
    # the library-chosen split count is lowered to fit and the call runs
    capi.decode_noalloc_raw(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), 0,
                            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = O.attn_batch(q, k, v, n_kv_heads=hkv, n_ctx=pos + nq, q_base_pos=pos, n_threads=8)
    got = out.cpu().numpy()
    assert O.max_abs(got, ref) < MAX_ABS and O.rel_l2(got, ref) < REL_L2
