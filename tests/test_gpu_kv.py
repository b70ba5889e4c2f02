"""GPU checks of the KV session formats read into and written from device memory
(include/nexus_hip_kv.h) -- bit-exact: the images and records must equal, byte for byte,
what the reference's own KVCache wrote (tests/golden/golden_kv.npz), and loads must put
exactly those rows in device memory and nothing else.
"""
import time

import numpy as np
import pytest
import torch

import oracle_lib as O
from nexus_amd import capi, ops

pytestmark = pytest.mark.gpu

CASES = {
    "uniform": ([(2, 64)] * 3, 8, 5),
    "per_layer": ([(2, 64), (0, 0), (4, 128), (1, 256), (0, 0)], 7, 6),
}


def dev16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def host16(t):
    return t.cpu().numpy().view(np.uint16)


def device_layers(geom, stride, fill=None, arrays=None):
    """Per layer (k, v) device tensors [nh, stride, hd] (None for layers without KV), filled
    from `arrays` (k list, v list) or with the constant `fill`."""
    out = []
    for l, (h, d) in enumerate(geom):
        if h == 0:
            out.append(None)
        elif arrays is not None:
            out.append((dev16(arrays[0][l]), dev16(arrays[1][l])))
        else:
            out.append((torch.full((h, stride, d), fill, dtype=torch.int16, device="cuda"),
                        torch.full((h, stride, d), fill, dtype=torch.int16, device="cuda")))
    return out


def golden_arrays(g, name, n_layers):
    return ([g.get(f"{name}_k{l}") for l in range(n_layers)], [g.get(f"{name}_v{l}") for l in range(n_layers)])


@pytest.mark.parametrize("name", list(CASES))
def test_save_from_device_equals_reference_images(hip, golden_kv, name):
    geom, stride, n_tok = CASES[name]
    arrays = golden_arrays(golden_kv, name, len(geom))
    layers = device_layers(geom, stride, arrays=arrays)
    img = ops.kv_cache_save(layers, n_tok)
    assert img.tobytes() == golden_kv[f"{name}_image"].tobytes()
    for l, lv in enumerate(layers):
        if lv is None:
            continue
        rec = ops.kv_layer_save(l, lv[0], lv[1], n_tok)
        assert rec.tobytes() == golden_kv[f"{name}_layer{l}"].tobytes()


@pytest.mark.parametrize("name", list(CASES))
def test_load_into_device_puts_exactly_the_rows(hip, golden_kv, name):
    """Rows [0, n_tok) of every head hold the image's data; rows past n_tok keep what they had."""
    geom, stride, n_tok = CASES[name]
    arrays = golden_arrays(golden_kv, name, len(geom))
    layers = device_layers(geom, stride, fill=0x5a5a)
    assert ops.kv_cache_load(golden_kv[f"{name}_image"], layers) == n_tok
    torch.cuda.synchronize()
    for l, lv in enumerate(layers):
        if lv is None:
            continue
        for t, src in ((lv[0], arrays[0][l]), (lv[1], arrays[1][l])):
            got = host16(t)
            np.testing.assert_array_equal(got[:, :n_tok], src[:, :n_tok])
            assert np.all(got[:, n_tok:] == 0x5a5a)
    # one layer record into a fresh cache: only that layer changes
    layers = device_layers(geom, stride, fill=0x1111)
    target = 2 if name == "per_layer" else 1
    assert ops.kv_layer_load(golden_kv[f"{name}_layer{target}"], layers) == (target, n_tok)
    for l, lv in enumerate(layers):
        if lv is None:
            continue
        got = host16(lv[0])
        if l == target:
            np.testing.assert_array_equal(got[:, :n_tok], arrays[0][l][:, :n_tok])
        else:
            assert np.all(got == 0x1111)


def test_legacy_image_loads_into_device(hip):
    geom, stride, n_tok = [(4, 128), (0, 0), (4, 128), (0, 0)], 9, 7
    c = O.KvCache.random(geom, stride, seed=21)
    legacy = np.frombuffer(O.kv_cache_save(c, n_tok, legacy=True), np.uint8)
    layers = device_layers(geom, stride, fill=0)
    assert ops.kv_cache_load(legacy, layers) == n_tok
    for l, lv in enumerate(layers):
        if lv is not None:
            np.testing.assert_array_equal(host16(lv[0])[:, :n_tok], c.k[l][:, :n_tok])
            np.testing.assert_array_equal(host16(lv[1])[:, :n_tok], c.v[l][:, :n_tok])


def test_refused_image_leaves_device_untouched(hip, golden_kv):
    geom, stride, n_tok = CASES["per_layer"]
    layers = device_layers(geom, stride, fill=0x2222)
    with pytest.raises(capi.NexusAttnError):
        ops.kv_cache_load(golden_kv["per_layer_image"][:-2], layers)
    with pytest.raises(capi.NexusAttnError):
        ops.kv_layer_load(golden_kv["per_layer_layer3"][:-1], layers)
    torch.cuda.synchronize()
    for lv in layers:
        if lv is not None:
            assert bool(torch.all(lv[0] == 0x2222)) and bool(torch.all(lv[1] == 0x2222))


def test_large_session_file_round_trip(hip, tmp_path):
    """A 32k-token session of a hybrid model (a KV layer every fourth layer, 2 x 256 heads):
    device -> file -> device through pinned staging, identical to the in-memory image."""
    n_layers, every, h, d, stride, n_tok = 16, 4, 2, 256, 33024, 32768
    geom = [(h, d) if l % every == every - 1 else (0, 0) for l in range(n_layers)]
    g = torch.Generator(device="cuda").manual_seed(5)
    layers = [None if gh == 0 else
              (torch.randint(-32768, 32767, (gh, stride, gd), dtype=torch.int16, device="cuda", generator=g),
               torch.randint(-32768, 32767, (gh, stride, gd), dtype=torch.int16, device="cuda", generator=g))
              for gh, gd in geom]
    path = tmp_path / "session.nxkv"
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ops.kv_cache_save_file(path, layers, n_tok)
    t_save = time.perf_counter() - t0
    size = path.stat().st_size
    assert size == ops.kv_cache_bytes(layers, n_tok) == 24 + 4 * h * n_tok * d * 4
    mem = ops.kv_cache_save(layers, n_tok)
    file_bytes = np.fromfile(path, np.uint8)
    assert np.array_equal(file_bytes, mem)
    fresh = [None if lv is None else (torch.zeros_like(lv[0]), torch.zeros_like(lv[1])) for lv in layers]
    t0 = time.perf_counter()
    assert ops.kv_cache_load_file(path, fresh) == n_tok
    t_load = time.perf_counter() - t0
    for a, b in zip(layers, fresh):
        if a is not None:
            assert torch.equal(a[0][:, :n_tok], b[0][:, :n_tok]) and torch.equal(a[1][:, :n_tok], b[1][:, :n_tok])
            assert not bool(torch.any(b[0][:, n_tok:]))
    print(f"[kv-session] {size / 2**20:.0f} MiB: save_file {size / t_save / 1e9:.2f} GB/s, "
          f"load_file {size / t_load / 1e9:.2f} GB/s", flush=True)
