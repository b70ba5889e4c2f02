"""Launch plans of the prefill entry, checked without a GPU (the library plans for 256 compute
units when none is visible, MI355X's count).  The GPU parity cases of test_gpu_attn.py are
chosen to exercise these routes; this pins that they do, and pins the routing rules themselves:
which kernel a chunk runs on, rows per block, key splits and packed rows."""
import pytest

from nexus_amd import capi


@pytest.fixture(scope="module", autouse=True)
def plan_for_256_cus():
    try:
        import torch
        if torch.cuda.is_available() and torch.cuda.get_device_properties(0).multi_processor_count != 256:
            pytest.skip("plans below are for 256 compute units")
    except ImportError:
        pass
    capi.load()


def plan(hq, hkv, hd, nq, base, sw=0, cap=0.0):
    d = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, q_base_pos=base, n_ctx=base + nq,
                       sliding_window=sw, softcap=cap)
    return capi.prefill_plan(d)


def P(rows, splits, wgs, packed=False):
    return {"kernel": "prefill", "block_rows": rows, "splits": splits, "packed": packed, "workgroups": wgs}


def D(rows, splits, wgs):
    return {"kernel": "decode", "block_rows": rows, "splits": splits, "packed": False, "workgroups": wgs}


@pytest.mark.parametrize("shape,want", [
    # the BASELINE configs and the bench's extra shapes
    ((40, 8, 128, 512, 4096), P(64, 1, 320)),         # cfg2: 320 64-row blocks, unsplit
    ((40, 8, 128, 8192, 0), P(128, 1, 2560)),         # cfg3
    ((16, 2, 256, 4, 32768), D(32, 128, 256)),        # cfg5 through the prefill entry: one 32-row group
    ((16, 2, 256, 512, 32768), P(128, 4, 256)),       # q35c: 64 blocks in 4 key splits
    ((16, 2, 256, 8192, 0), P(128, 1, 1024)),         # q35p
    ((40, 8, 128, 1024, 3072), P(128, 1, 320)),       # tile3: a long cache before the chunk keeps 128 rows
    ((16, 2, 256, 1024, 3072), P(128, 2, 256)),       # q35t3: 128 blocks at one per CU -> 2 splits
])
def test_bench_shapes(shape, want):
    assert plan(*shape) == want


@pytest.mark.parametrize("shape,kernel", [
    # one 32-row group: the decode kernel at any cache length
    ((16, 4, 128, 8, 100), "decode"),
    ((8, 1, 128, 4, 0), "decode"),
    # 2R <= G behind >= 8k keys (16q/2kv: G = 8)
    ((16, 2, 256, 16, 9000), "decode"),               # R = 4
    ((16, 2, 256, 16, 8000), "prefill"),              # below 8k keys
    ((16, 2, 256, 20, 9000), "prefill"),              # R = 5: 2R > G, and below 16k
    # behind >= 16k keys: R < G and no packed grid that fills the chip
    ((16, 2, 256, 8, 17000), "decode"),               # R = 2, too few packed blocks
    ((16, 2, 256, 16, 17000), "decode"),              # R = 4: one packed block per kv head, too small a grid
    ((16, 2, 256, 24, 17000), "prefill"),             # R = 6 < 8, but 4 packed blocks fill the grid
    ((16, 2, 256, 32, 17000), "prefill"),             # R = 8 = G
    ((24, 4, 192, 24, 32768), "prefill"),             # R = 5 < 6, packed
    ((8, 1, 128, 16, 32768), "decode"),               # R = 4, one kv head: packing cannot fill the grid
    ((40, 8, 128, 12, 17000), "prefill"),             # R = 2 at head dim 128: packed
    ((16, 4, 128, 16, 32768), "prefill"),             # R = 2, G = 4: packed
    ((40, 8, 128, 24, 17000), "prefill"),             # R = 4 at head dim 128: packed rows
    ((64, 8, 128, 16, 32768), "prefill"),             # R = 4 < G = 8 at head dim 128: packed rows
    ((40, 8, 128, 32, 17000), "prefill"),             # R = 5 = G
    ((16, 8, 128, 24, 32768), "prefill"),             # R = 2 = G: nothing shared
    # 2R <= G behind 8k-16k keys, again without a packed grid
    ((64, 8, 128, 8, 12000), "prefill"),              # R = 2: packed
    ((64, 8, 128, 4, 12000), "decode"),               # one group
    ((64, 8, 128, 16, 12000), "prefill"),             # R = 4: packed
    ((16, 2, 256, 16, 9000), "decode"),               # R = 4: too few packed blocks
    ((64, 8, 128, 20, 12000), "prefill"),             # 2R = 10 > 8
    ((40, 8, 128, 12, 4000), "prefill"),              # short cache: the prefill kernel's lower fixed costs
    # window + softcap ride the same rule
    ((16, 2, 256, 12, 20000, 300, 20.0), "decode"),
])
def test_short_chunk_route(shape, kernel):
    assert plan(*shape)["kernel"] == kernel


@pytest.mark.parametrize("shape,packed", [
    ((40, 8, 128, 32, 20000), True),
    ((40, 8, 128, 47, 16500, 5000, 30.0), True),
    ((16, 2, 256, 96, 17000), True),                  # 12 packed 128-row blocks against 16
    ((16, 2, 256, 128, 17000), False),                # 16 blocks either way: nothing saved
    ((24, 4, 192, 100, 16384), True),
    ((40, 8, 128, 40, 17000), True),                  # the gated packed case
    ((64, 8, 128, 20, 17000), True),                  # 240 packed workgroups against 256 plain ones
    ((64, 8, 128, 40, 32768), True),
    ((40, 8, 128, 24, 9000), True),                   # 8k-16k keys at head dim 128
    ((40, 8, 128, 32, 7000), False),                  # below 8k keys
    ((32, 8, 64, 48, 9000), False),                   # head dim 64 below 16k keys
    ((40, 8, 128, 64, 9000), False),                  # 40 blocks either way
    ((16, 2, 256, 32, 8192), False),                  # packing lost there (64 workgroups for 256)
    ((40, 8, 128, 160, 32768), True),                 # 160 queries: 13 packed blocks per kv head against 15
    ((40, 8, 128, 256, 32768), False),                # 256 queries: as many blocks either way
    ((40, 8, 128, 600, 32768), False),                # more than 512 queries
    ((8, 8, 128, 64, 20000), False),                  # no GQA group to pack
])
def test_packed_rows_rule(shape, packed):
    p = plan(*shape)
    assert p["kernel"] == "prefill"
    assert p["packed"] == packed


def test_packed_grid_never_smaller_than_it_needs():
    """Packing is taken only when its grid has at least 3/4 of the workgroups of the plain one
    or of the CUs."""
    for hq, hkv in [(40, 8), (16, 2), (24, 4), (32, 8), (64, 8)]:
        for hd in (64, 128, 192, 256):
            for nq in (33, 48, 64, 96, 100, 128):
                for base in (16384, 32768, 65536):
                    p = plan(hq, hkv, hd, nq, base)
                    if p["packed"]:
                        assert 4 * p["workgroups"] >= 3 * min(256, _plain_wgs(hq, hkv, hd, nq, base)), \
                            (hq, hkv, hd, nq, base, p)


def _plain_wgs(hq, hkv, hd, nq, base):
    """Workgroups of the unpacked grid: what the plan gives with one q head per kv head
    scaled back up (same block rows and splits rule at Hq = Hkv, where packing is off)."""
    p = plan(hq, hq, hd, nq, base)
    return p["workgroups"] if p["kernel"] == "prefill" else 0


@pytest.mark.parametrize("shape,want", [
    ((32, 8, 128, 512, 100), P(64, 1, 256)),          # exactly one 128-row block per CU -> 64 rows
    ((40, 8, 128, 520, 300), P(64, 1, 360)),          # 360 64-row blocks
    ((16, 2, 256, 1024, 1024), P(128, 2, 256)),       # the engine's 1024-token tile at hd 256
    ((8, 2, 128, 256, 3000), P(64, 8, 256)),          # short chunk over a longer cache: key splits
    ((4, 4, 128, 64, 32768), P(64, 64, 256)),         # 4 blocks behind 32k keys: 64 splits
    ((40, 8, 128, 256, 32768), P(128, 6, 480)),       # behind a long cache: 80 128-row blocks in 6 splits
    ((8, 8, 128, 160, 32768), P(64, 21, 504)),        # ... unless 128-row blocks pad more rows
    ((32, 8, 128, 256, 16384), P(128, 8, 512)),       # 64 128-row blocks
    ((64, 8, 128, 512, 8192), P(64, 1, 512)),         # ... or give a smaller grid
    ((40, 8, 128, 64, 32768), P(64, 12, 480)),        # 40 blocks, 43 tiles per split at two per CU
    ((40, 8, 128, 24, 9000), P(64, 16, 256, True)),   # 16 packed blocks, too few tiles for two per CU
    ((16, 2, 256, 32, 32768), P(128, 64, 256, True)), # 4 packed blocks, 64 splits
    ((40, 8, 128, 1024, 0), P(64, 1, 640)),           # the engine's first 1024-token tile: 64 rows
    ((40, 8, 128, 1024, 1024), P(128, 1, 320)),       # its second (cache as long as the chunk): 128 rows
    ((40, 8, 128, 1024, 2048), P(128, 1, 320)),       # a longer cache before the chunk: 128 rows
])
def test_block_rows_and_splits(shape, want):
    assert plan(*shape) == want


@pytest.mark.parametrize("shape", [(40, 8, 128, 512, 4096), (16, 2, 256, 512, 32768), (16, 2, 256, 4, 32768),
                                   (40, 8, 128, 32, 20000)])
def test_workspace_matches_plan(shape):
    """nexus_hip_attn_prefill_ws_bytes sizes exactly the partials of the planned splits."""
    hq, hkv, hd, nq, base = shape
    d = capi.make_desc(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, n_query=nq, q_base_pos=base, n_ctx=base + nq)
    p = capi.prefill_plan(d)
    want = 0 if p["splits"] <= 1 else nq * hq * p["splits"] * (hd + 2) * 4
    assert capi.prefill_ws_bytes(d) == want


def test_plan_declines_like_the_entry():
    d = capi.make_desc(n_q_heads=8, n_kv_heads=3, head_dim=128, n_query=4, q_base_pos=0, n_ctx=4)
    with pytest.raises(capi.NexusAttnError) as e:
        capi.prefill_plan(d)
    assert e.value.code == capi.NEXUS_E_UNSUPPORTED or e.value.code == capi.NEXUS_E_INVALID
