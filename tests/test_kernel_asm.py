"""CPU checks of the gfx950 assembly the kernels compile to (hipcc cross-compiles here).

The pipelined prefill kernel issues its head-dim-256 MFMAs as inline asm, which the compiler's
hazard recognizer does not see.  These tests compile the kernel source exactly as the library
build does and check, with tests/asm_hazards.py, that no instruction touches a register of an
inline-asm MFMA (its result, or its accumulator input) before enough wait states have passed on
every path.  The checker itself is pinned on small listings with and without such a hazard.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

import asm_hazards as H

ROOT = Path(__file__).resolve().parents[1]

MFMA = "\tv_mfma_f32_32x32x16_f16 a[0:15], v[0:3], v[4:7], a[0:15]"


def listing(body: str) -> str:
    lines = ["_Zkernel:"]
    for l in body.strip("\n").split("\n"):
        l = l.strip()
        if l.startswith("ASM "):
            lines += ["\t;;#ASMSTART", "\t" + l[4:], "\t;;#ASMEND"]
        else:
            lines.append(l if l.endswith(":") else "\t" + l)
    lines += ["\ts_endpgm", ".Lfunc_end0:"]
    return "\n".join(lines)


def hazards(body: str) -> list[str]:
    return H.check_listing(listing(body))["_Zkernel"]


def test_checker_flags_result_read_too_soon():
    assert hazards(f"ASM {MFMA.strip()}\nv_accvgpr_read_b32 v10, a3") != []
    assert hazards(f"ASM {MFMA.strip()}\nv_accvgpr_mov_b32 a20, a15") != []


def test_checker_accepts_settled_result():
    assert hazards(f"ASM {MFMA.strip()}\ns_nop 7\ns_nop 7\ns_nop 3\nv_accvgpr_read_b32 v10, a3") == []
    # registers the MFMA does not touch need no wait
    assert hazards(f"ASM {MFMA.strip()}\nv_accvgpr_read_b32 v10, a16\nv_add_f32 v8, v9, v9") == []


def test_checker_flags_accumulator_input_overwritten():
    body = "ASM v_mfma_f32_32x32x16_f16 v[20:35], v[0:3], a[4:7], v[40:55]\nds_read_b128 v[40:43], v1"
    assert hazards(body) != []
    assert hazards(body.replace("v[40:43]", "v[60:63]")) == []


def test_checker_follows_branches():
    """The short path into a join decides: a settle on one incoming path only is not enough."""
    body = f"""
ASM {MFMA.strip()}
s_cbranch_scc0 .LBB0_2
s_nop 7
s_nop 7
s_nop 3
.LBB0_2:
v_accvgpr_read_b32 v10, a0
"""
    assert hazards(body) != []
    assert hazards(body.replace("s_cbranch_scc0 .LBB0_2\n", "")) == []
    # a loop back edge carries the state around
    loop = f"""
.LBB0_1:
v_accvgpr_read_b32 v10, a0
s_nop 7
s_nop 7
s_nop 3
ASM {MFMA.strip()}
s_cbranch_scc0 .LBB0_1
"""
    assert hazards(loop) != []


def compile_listing(src: Path, out: Path) -> str:
    from nexus_amd import build as B
    if shutil.which(B.HIPCC) is None and not Path(B.HIPCC).exists():
        pytest.skip("hipcc not available")
    flags = [f for f in B.COMMON_FLAGS if f != "-fPIC"]
    cmd = [B.HIPCC, "-x", "hip", *flags, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def test_prefill_wide_inline_mfma_waits(tmp_path):
    asm = compile_listing(ROOT / "nexus_amd" / "csrc" / "attn_prefill_wide.hip", tmp_path / "wide.s")
    found = H.check_listing(asm)
    with_asm_mfma = [k for k, v in found.items() if "prefill_wide_kernelILi256" in k or "prefill_wide_kernelILi192" in k]
    assert len(with_asm_mfma) == 16, sorted(found)      # head dims 192, 256: q f16/f32 x o f16/f32 x ext
    bad = {k: v for k, v in found.items() if v}
    assert not bad, "\n".join(f"{k}:\n  " + "\n  ".join(v[:8]) for k, v in bad.items())
