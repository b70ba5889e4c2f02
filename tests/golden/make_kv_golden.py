"""Write tests/golden/golden_kv.npz: KV session images written by the reference's OWN
KVCache (oracle/_ref/libnexus_ref_attn.so, compiled from the reference sources by
`make -C oracle ref`): KVCache::save_to_buffer (NXKVCACH) and save_layer_to_buffer
(NXKVLYR1), src/model/kvcache.h:383-449, for a uniform cache and for one with per-layer
geometry (layers without KV, mixed head dims; KVCache::init_per_layer).

    python tests/golden/make_kv_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import oracle_lib as O  # noqa: E402

CASES = {
    # name: (geometry [(kv heads, head dim)] per layer, row stride, tokens, per-layer init)
    "uniform": ([(2, 64)] * 3, 8, 5, False),
    "per_layer": ([(2, 64), (0, 0), (4, 128), (1, 256), (0, 0)], 7, 6, True),
}


def main() -> None:
    out = {}
    for name, (geom, stride, n_tok, per_layer) in CASES.items():
        c = O.KvCache.random(geom, stride, seed=11)
        for l, (h, _) in enumerate(geom):
            if h:
                out[f"{name}_k{l}"] = c.k[l]
                out[f"{name}_v{l}"] = c.v[l]
        out[f"{name}_image"] = np.frombuffer(O.ref_kv_save_cache(c, n_tok, per_layer), np.uint8)
        for l in range(len(geom)):
            out[f"{name}_layer{l}"] = np.frombuffer(O.ref_kv_save_layer(c, l, n_tok, per_layer), np.uint8)
    np.savez_compressed(HERE / "golden_kv.npz", **out)
    print(f"wrote {HERE / 'golden_kv.npz'} ({len(out)} arrays)")


if __name__ == "__main__":
    main()
