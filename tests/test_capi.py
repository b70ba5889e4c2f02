"""C ABI checks that need no GPU: the library loads, exports every symbol the header
declares, and declines unsupported or invalid calls before touching any output (the
reference's `return false` before side effects, vulkan_backend.h:4267-4277)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from nexus_amd import capi

HEADER = Path(__file__).resolve().parent.parent / "include" / "nexus_hip_attn.h"
HEADERS = sorted(HEADER.parent.glob("*.h"))


def declared_functions():
    text = "\n".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(nexus_hip_[a-z_0-9]+)\s*\(", text, re.M)))


def test_header_declares_what_the_binding_knows():
    assert declared_functions() == sorted(capi.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert "gfx950" in capi.version()


def test_library_has_no_undefined_kernel_symbols():
    """Every kernel the library launches is defined in it.  (hipcc's host pass can drop a kernel
    template without a diagnostic -- seen when a buffer-load-to-LDS builtin's argument list held an
    array selection -- and the library then references the missing stub.)"""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("no nm on this host")
    res = subprocess.run([nm, "-D", "--undefined-only", str(capi.LIB_PATH)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    missing = [line.split()[-1] for line in res.stdout.splitlines() if "nxa" in line]
    assert not missing, missing[:8]


@pytest.mark.parametrize("cls,cname", [(capi.AttnDesc, "nexus_attn_desc"), (capi.PrepDesc, "nexus_attn_prep_desc"),
                                       (capi.KvLayerView, "nexus_kv_layer_view"),
                                       (capi.PrefillPlan, "nexus_attn_prefill_plan")])
def test_desc_layout_matches_header(tmp_path, cls, cname):
    """The ctypes mirrors of the descriptors have the C compiler's size and offsets."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler on this host")
    fields = [f[0] for f in cls._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "nexus_hip_attn.h"\n#include "nexus_hip_kv.h"\n'
                   'int main(void){'
                   f'printf("%zu", sizeof({cname}));'
                   + "".join(f'printf(" %zu", offsetof({cname}, {f}));' for f in fields)
                   + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(cls)
    assert got[1:] == [getattr(cls, f).offset for f in fields]


def test_prep_flag_values_match_header():
    text = HEADER.read_text()
    for name in ("Q_NORM_ADD_ONE", "K_NORM_ADD_ONE", "NO_GATE", "NO_Q_NORM", "NO_K_NORM", "ROPE_INTERLEAVED", "TRUNC_STORE"):
        m = re.search(rf"NEXUS_PREP_{name}\s*=\s*(\d+)", text)
        assert m and int(m.group(1)) == getattr(capi, f"PREP_{name}"), name


def _desc(**kw):
    base = dict(n_q_heads=8, n_kv_heads=2, head_dim=128, n_query=16, q_base_pos=32, n_ctx=48)
    base.update(kw)
    return capi.make_desc(**base)


BAD = [
    (dict(head_dim=96), capi.NEXUS_E_UNSUPPORTED),
    (dict(head_dim=320), capi.NEXUS_E_UNSUPPORTED),
    (dict(n_q_heads=7, n_kv_heads=2), capi.NEXUS_E_UNSUPPORTED),
    (dict(n_kv_heads=0), capi.NEXUS_E_UNSUPPORTED),
    (dict(n_query=0), capi.NEXUS_E_INVALID),
    (dict(n_ctx=0), capi.NEXUS_E_INVALID),
    (dict(q_base_pos=-1), capi.NEXUS_E_INVALID),
    (dict(kv_row_stride=47), capi.NEXUS_E_INVALID),
    (dict(sliding_window=-3), capi.NEXUS_E_INVALID),
    (dict(scale=float("nan")), capi.NEXUS_E_INVALID),
    (dict(softcap=-1.0), capi.NEXUS_E_INVALID),
    (dict(q_dtype=7), capi.NEXUS_E_UNSUPPORTED),
]


@pytest.mark.parametrize("kw,code", BAD)
def test_declines_before_side_effects(kw, code):
    d = _desc(**kw)
    out = np.full(64, 7.0, np.float32)
    dummy = np.zeros(64, np.float32)
    p = dummy.ctypes.data
    rc = capi.prefill_raw(d, p, p, p, out.ctypes.data, 0, 0, 0, check=False)
    assert rc == code, capi.last_error()
    assert capi.last_error()
    rc = capi.decode_raw(d, p, p, p, out.ctypes.data, p, 4, 0, check=False)
    assert rc == code
    assert np.all(out == 7.0)


def test_null_pointers_declined():
    d = _desc()
    out = np.full(8, 3.0, np.float32)
    rc = capi.prefill_raw(d, 0, 0, 0, out.ctypes.data, 0, 0, 0, check=False)
    assert rc == capi.NEXUS_E_INVALID
    x = np.zeros(4, np.float32).ctypes.data
    rc = capi.decode_raw(d, x, x, x, out.ctypes.data, 0, 4, 0, check=False)
    assert rc == capi.NEXUS_E_WORKSPACE
    rc = capi.decode_raw(d, x, x, x, out.ctypes.data, x, 5000, 0, check=False)
    assert rc == capi.NEXUS_E_UNSUPPORTED
    assert np.all(out == 3.0)


def test_workspace_sizes():
    # decode: f32 partials, (hd + 2) floats per row and split, and nothing else (no state)
    d = capi.make_desc(n_q_heads=40, n_kv_heads=8, head_dim=128, n_query=1, q_base_pos=61439, n_ctx=61440)
    assert capi.decode_ws_bytes(d, 64) == 40 * 64 * 130 * 4
    assert capi.decode_ws_bytes(d, 0) == 40 * capi.decode_default_splits(d) * 130 * 4
    assert capi.decode_ws_bytes(_desc(head_dim=96), 4) == 0
    # a cold 8192 prompt with 40 heads fills the GPU unsplit: no workspace
    cold = capi.make_desc(n_q_heads=40, n_kv_heads=8, head_dim=128, n_query=8192, q_base_pos=0, n_ctx=8192)
    assert capi.prefill_ws_bytes(cold) == 0
    # 4 speculative drafts x G=8 rows run through the split-KV path
    mtp = capi.make_desc(n_q_heads=16, n_kv_heads=2, head_dim=256, n_query=4, q_base_pos=32768, n_ctx=32772)
    assert capi.prefill_ws_bytes(mtp) == capi.decode_ws_bytes(mtp, 0) > 0


def test_algorithmic_work_formulas():
    # cfg2 / cfg3 visible (query, key) pairs per head: 512 queries after 4096 keys, 8192 cold
    assert capi.prefill_flops(40, 128, 512, 4096, 4608) == 4 * 128 * 40 * 2_228_480
    assert capi.prefill_flops(40, 128, 8192, 0, 8192) == 4 * 128 * 40 * 33_558_528
    assert capi.decode_bytes(8, 128, 61440, 40, 1) == 2 * 8 * 61440 * 128 * 2 + 40 * 128 * 8


def _prep_desc(**kw):
    base = dict(n_heads=8, n_kv_heads=2, head_dim=128, rot_dims=32, pos=5, flags=0, cap=16, eps=1e-6, reserved=0)
    base.update(kw)
    return capi.PrepDesc(**base)


PREP_BAD = [
    (dict(n_heads=0), capi.NEXUS_E_INVALID),
    (dict(n_kv_heads=-1), capi.NEXUS_E_INVALID),
    (dict(head_dim=0), capi.NEXUS_E_UNSUPPORTED),
    (dict(head_dim=520, rot_dims=0), capi.NEXUS_E_UNSUPPORTED),
    (dict(rot_dims=31), capi.NEXUS_E_INVALID),
    (dict(rot_dims=130), capi.NEXUS_E_INVALID),
    (dict(pos=16), capi.NEXUS_E_INVALID),
    (dict(pos=-1), capi.NEXUS_E_INVALID),
    (dict(cap=0, pos=0), capi.NEXUS_E_INVALID),
    (dict(flags=128), capi.NEXUS_E_INVALID),
    (dict(eps=float("inf")), capi.NEXUS_E_INVALID),
    (dict(reserved=1), capi.NEXUS_E_INVALID),
]


@pytest.mark.parametrize("kw,code", PREP_BAD)
def test_prep_declines_before_side_effects(kw, code):
    out = np.full(64, 7.0, np.float32)
    p, o = np.zeros(64, np.float32).ctypes.data, out.ctypes.data
    rc = capi.decode_prep_raw(_prep_desc(**kw), p, p, p, p, p, p, o, o, o, o, o, 0, check=False)
    assert rc == code, capi.last_error()
    assert capi.last_error()
    assert np.all(out == 7.0)


def test_prep_null_pointers_declined():
    """Pointers are required exactly where the flags say the kernel reads or writes them."""
    out = np.full(64, 7.0, np.float32)
    p, o = np.zeros(64, np.float32).ctypes.data, out.ctypes.data
    d = _prep_desc()
    assert capi.decode_prep_raw(d, p, p, p, p, p, p, o, 0, o, o, o, 0, check=False) == capi.NEXUS_E_INVALID   # gate_out
    assert capi.decode_prep_raw(d, p, p, p, 0, p, p, o, o, o, o, o, 0, check=False) == capi.NEXUS_E_INVALID   # q norm w
    assert capi.decode_prep_raw(d, p, p, p, p, 0, p, o, o, o, o, o, 0, check=False) == capi.NEXUS_E_INVALID   # k norm w
    assert capi.decode_prep_raw(d, p, p, p, p, p, 0, o, o, o, o, o, 0, check=False) == capi.NEXUS_E_INVALID   # table
    assert capi.decode_prep_raw(d, p, p, p, p, p, p, o, o, 0, o, o, 0, check=False) == capi.NEXUS_E_INVALID   # k cache
    assert np.all(out == 7.0)


# ------------------------------------------------------------------ KV session entry points

def _kv_views(geom, stride, ptr=None):
    arr = (capi.KvLayerView * len(geom))()
    for i, (h, d) in enumerate(geom):
        arr[i] = capi.KvLayerView(ptr if h else None, ptr if h else None, h, d, stride)
    return arr


def test_kv_sizes_match_the_reference_images(golden_kv):
    """nexus_hip_kv_*_bytes agree with the images the reference's KVCache wrote."""
    lib = capi.load()
    for name, geom, stride, n_tok in (("uniform", [(2, 64)] * 3, 8, 5),
                                      ("per_layer", [(2, 64), (0, 0), (4, 128), (1, 256), (0, 0)], 7, 6)):
        views = _kv_views(geom, stride)
        assert lib.nexus_hip_kv_cache_bytes(views, len(geom), n_tok) == golden_kv[f"{name}_image"].size
        for l in range(len(geom)):
            assert lib.nexus_hip_kv_layer_bytes(ctypes.byref(views[l]), n_tok) == golden_kv[f"{name}_layer{l}"].size


def test_kv_declines_before_any_copy(golden_kv):
    """Bad images and impossible requests are refused during validation: no device needed,
    nothing written (the reference's loader can stop part-way; this one checks first)."""
    lib = capi.load()
    geom, stride, n_tok = [(2, 64), (0, 0), (4, 128), (1, 256), (0, 0)], 7, 6
    sentinel = np.full(4096, 7, np.uint16)
    views = _kv_views(geom, stride, sentinel.ctypes.data)
    img = golden_kv["per_layer_image"]
    n = ctypes.c_int(-9)
    bad_images = [img[:-1], img[:20], np.concatenate([np.frombuffer(b"NXKVCACX", np.uint8), img[8:]])]
    for data in bad_images:
        data = np.ascontiguousarray(data)
        assert lib.nexus_hip_kv_cache_load(data.ctypes.data, data.size, views, len(geom), ctypes.byref(n), None) == \
            capi.NEXUS_E_INVALID
    other = _kv_views([(2, 64), (0, 0), (4, 128), (1, 128), (0, 0)], stride, sentinel.ctypes.data)  # other model
    assert lib.nexus_hip_kv_cache_load(img.ctypes.data, img.size, other, len(geom), ctypes.byref(n), None) == \
        capi.NEXUS_E_INVALID
    assert b"model mismatch" in capi.load().nexus_hip_attn_last_error()
    short = _kv_views(geom, n_tok - 1, sentinel.ctypes.data)                 # capacity below the image's tokens
    assert lib.nexus_hip_kv_cache_load(img.ctypes.data, img.size, short, len(geom), ctypes.byref(n), None) == \
        capi.NEXUS_E_INVALID
    rec = golden_kv["per_layer_layer2"]
    wrong = _kv_views([(2, 64), (0, 0), (4, 64), (1, 256), (0, 0)], stride, sentinel.ctypes.data)
    lo = ctypes.c_int(-9)
    for data, v in ((rec[:-1], views), (rec, wrong)):
        data = np.ascontiguousarray(data)
        assert lib.nexus_hip_kv_layer_load(data.ctypes.data, data.size, v, len(geom), ctypes.byref(lo),
                                           ctypes.byref(n), None) == capi.NEXUS_E_INVALID
    out = np.full(64, 5, np.uint8)
    assert lib.nexus_hip_kv_cache_save(views, len(geom), n_tok, out.ctypes.data, out.size, None) == \
        capi.NEXUS_E_INVALID                                              # buffer too small
    assert lib.nexus_hip_kv_cache_save(views, len(geom), stride + 1, out.ctypes.data, 1 << 30, None) == \
        capi.NEXUS_E_INVALID                                              # more tokens than rows
    assert lib.nexus_hip_kv_cache_load_file(b"/nonexistent/kv.bin", views, len(geom), ctypes.byref(n), None) == \
        capi.NEXUS_E_IO
    assert np.all(sentinel == 7) and np.all(out == 5) and n.value == -9 and lo.value == -9
