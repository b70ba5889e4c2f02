"""Write tests/golden/golden_attn.npz: input/output vectors produced by the reference's
OWN code (oracle/_ref/libnexus_ref_attn.so, compiled from the reference sources by
`make -C oracle ref`).  The fixtures pin the CPU oracle wherever the reference is absent.

Cases
  dec_*  AttentionLayer::forward_cached_scores (src/model/attention.h:1201-1259) at `pos`.
  pre_a  a chunked prefill (q_base > 0): row i is forward_cached_scores at q_base + i over
         keys [0, q_base + i], i.e. the causal rule of attn_batch_cpu, written by the
         reference's decode code.
  kv     KVCache::store + pack_k/pack_v (src/model/kvcache.h:148-178, 655-672, 903-911)
         on f32 values chosen to hit truncation, flush-to-zero, overflow and nan.
  cap    KVCache slot capacity after storing n tokens (growth policy kvcache.h:856-873).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

from nexus_amd.inputs import make_case, normal  # noqa: E402
import oracle_lib as O  # noqa: E402

DEC_CASES = {
    # name: (Hq, Hkv, hd, pos, scale, softcap, seed)
    "dec_a": (8, 2, 64, 299, 0.0, 0.0, 11),
    "dec_b": (16, 4, 128, 127, 0.0, 0.0, 12),
    "dec_c": (4, 1, 128, 99, 0.1, 30.0, 13),
    "dec_d": (16, 2, 256, 63, 0.0, 0.0, 14),
}
PRE = dict(Hq=8, Hkv=2, hd=64, q_base=60, nq=20, seed=15)
CAP_TOKENS = [1, 511, 512, 513, 1024, 1025, 4097, 8192, 8193, 12288, 12289, 61440]


def main() -> None:
    if not O.ref_available():
        raise SystemExit(f"{O.REF_SO} is missing; build it with `make -C oracle ref`")
    out = {}
    for name, (hq, hkv, hd, pos, scale, cap, seed) in DEC_CASES.items():
        q, k, v = make_case(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=1, n_ctx=pos + 1, seed=seed)
        y = O.ref_cached_scores(q[0], k, v, n_kv_heads=hkv, pos=pos, scale=scale, softcap=cap)
        out[f"{name}_q"], out[f"{name}_k"], out[f"{name}_v"], out[f"{name}_out"] = q[0], k, v, y
        out[f"{name}_meta"] = np.array([hq, hkv, hd, pos], np.int64)
        out[f"{name}_fmeta"] = np.array([scale, cap], np.float32)

    p = PRE
    n_ctx = p["q_base"] + p["nq"]
    q, k, v = make_case(n_q_heads=p["Hq"], n_kv_heads=p["Hkv"], head_dim=p["hd"], n_query=p["nq"],
                        n_ctx=n_ctx, seed=p["seed"])
    y = np.stack([O.ref_cached_scores(q[i], k, v, n_kv_heads=p["Hkv"], pos=p["q_base"] + i)
                  for i in range(p["nq"])])
    out.update(pre_a_q=q, pre_a_k=k, pre_a_v=v, pre_a_out=y,
               pre_a_meta=np.array([p["Hq"], p["Hkv"], p["hd"], p["q_base"], p["nq"], n_ctx], np.int64))

    # KV store: magnitudes across the f16 range and its edges, both signs, nan, -0.
    hkv, hd, ntok = 2, 64, 6
    vals = np.concatenate([
        normal(21, 200) * 3.0,
        np.array([0.0, -0.0, 1e-5, -3e-5, 6.1e-5, 6.2e-5, 65504.0, 65519.0, 65520.0, 70000.0,
                  -1e9, np.inf, -np.inf, np.nan, 1.0009765625, 1.00146484375, -2.5e-8], np.float32),
        np.exp(normal(22, 300) * 6.0).astype(np.float32) * np.sign(normal(23, 300)),
    ]).astype(np.float32)
    kf = np.resize(vals, ntok * hkv * hd).astype(np.float32).reshape(ntok, hkv * hd)
    vf = np.resize(vals[::-1], ntok * hkv * hd).astype(np.float32).reshape(ntok, hkv * hd)
    kp = np.zeros((hkv, ntok, hd), np.uint16)
    vp = np.zeros((hkv, ntok, hd), np.uint16)
    rc = O.ref().ref_kv_store_pack(np.ascontiguousarray(kf), np.ascontiguousarray(vf), ntok, hkv, hd, kp, vp)
    assert rc == 0
    out.update(kv_kf=kf, kv_vf=vf, kv_kpacked=kp, kv_vpacked=vp, kv_meta=np.array([hkv, hd, ntok], np.int64))

    caps = [O.ref().ref_kv_capacity_after(n, 128) for n in CAP_TOKENS]
    out.update(cap_tokens=np.array(CAP_TOKENS, np.int64), cap_hd128=np.array(caps, np.int64))

    dst = HERE / "golden_attn.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
