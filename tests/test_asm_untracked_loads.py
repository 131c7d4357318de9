"""CPU check of the compiled GEMM kernels: no inline-asm load destination is touched before its wait, on
any control-flow path of any instantiation (tests/asm_untracked_loads.py). Includes a self-test on a
hand-written violation so the check cannot silently pass everything."""
import os
import re
import shutil

import pytest

from tests.asm_untracked_loads import (check_function, check_text, compile_to_asm, kernel_spills,
                                       scratch_in_inner_mfma_loop)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "krea_image_amd", "csrc")

BAD = """k:
\t;;#ASMSTART
\tglobal_load_dword v7, v[2:3], off
\t;;#ASMEND
\tv_add_u32_e32 v7, 1, v4
\ts_waitcnt vmcnt(0)
\ts_endpgm
"""
GOOD = """k:
\t;;#ASMSTART
\tglobal_load_dword v7, v[2:3], off
\t;;#ASMEND
\tglobal_load_dword v8, v[2:3], off
\ts_waitcnt vmcnt(1)
\tv_add_u32_e32 v7, 1, v7
\ts_endpgm
"""
LOOP_BAD = """k:
.LBB0_1:
\tv_mov_b32_e32 v7, 0
\t;;#ASMSTART
\tglobal_load_dword v7, v[2:3], off
\t;;#ASMEND
\ts_cbranch_scc1 .LBB0_1
\ts_waitcnt vmcnt(0)
\ts_endpgm
"""


def test_checker_flags_known_violations():
    assert check_function(BAD)
    assert not check_function(GOOD)
    assert check_function(LOOP_BAD)  # the write at the loop head hits the load of the previous iteration


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not available")
@pytest.mark.parametrize("unit", ["kh_gemm_f16.hip", "kh_gemm_bf16.hip"])
def test_gemm_kernels_have_no_untracked_load_hazards(tmp_path, unit):
    text = compile_to_asm(os.path.join(CSRC, unit), str(tmp_path / "gemm.s"), CSRC)
    res = check_text(text)
    assert len(res) >= 80, f"expected every GEMM instantiation, found {len(res)}"
    bad = {k: v[:3] for k, v in res.items() if v}
    assert not bad, f"inline-asm load destinations used before their wait: {bad}"
    # Register budget: no spill traffic inside the K loop (the innermost loop holding MFMAs) of any
    # int8-weight instantiation. Known exceptions: three 16-bit-weight (WF_16) stream-K kernels at 256-wide
    # tiles reload one or two spilled dwords per two K steps; the count is capped so a new one cannot slip in.
    loop_spills = {}
    for f in re.split(r"\n(?=_ZN\S*:)", text):
        name = f.split(":", 1)[0]
        if "gemm_kernel" in name:
            hits = scratch_in_inner_mfma_loop(f[:f.find(".Lfunc_end")])
            if hits:
                loop_spills[name] = hits
    unexpected = [k for k in loop_spills if not re.search(r"gemm_kernelILi\d+ELi0ELi\d+ELi8ELb1ELi256ELb0E", k)]
    assert not unexpected, f"scratch accesses inside a GEMM K loop: {unexpected}"
    assert len(loop_spills) <= 3, f"more 16-bit-weight stream-K kernels spill in the K loop: {sorted(loop_spills)}"


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not available")
def test_attention_kernels_do_not_spill(tmp_path):
    """Every attention instantiation fits its registers (it holds ~250 of the 256 VGPRs a wave has at two
    waves per SIMD): no VGPR spills and no scratch segment."""
    text = compile_to_asm(os.path.join(CSRC, "kh_attention.hip"), str(tmp_path / "attn.s"), CSRC)
    ks = kernel_spills(text, "attn_kernel")
    assert len(ks) == 64, f"expected 64 attention instantiations (32 per address form), found {len(ks)}"
    bad = {k: v for k, v in ks.items() if v != (0, 0)}
    assert not bad, f"attention kernels with spills / scratch: {bad}"
