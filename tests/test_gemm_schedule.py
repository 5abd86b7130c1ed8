"""CPU checks of the fused GEMM's generated main loop (hif8_gemm_dtl.hip).

- hif8_gemm_schedule.inc is what gen_gemm_schedule.py generates;
- compiled for gfx950, the kernel spills nothing, uses the full 160 KB LDS array, and its
  main loop passes the in-flight-register and VALU->MFMA checks of isa_check.py with the
  expected instruction census (256 MFMA, 208 LDS loads, 24 global->LDS loads per 2 k-steps).
"""
import importlib.util
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "osp-next_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def test_schedule_include_is_generated():
    spec = importlib.util.spec_from_file_location("gen_gemm_schedule", os.path.join(CSRC, "gen_gemm_schedule.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    with open(os.path.join(CSRC, "hif8_gemm_schedule.inc")) as f:
        assert f.read() == gen.generate()
    with open(os.path.join(CSRC, "hif8_gemm_schedule_w16.inc")) as f:
        assert f.read() == gen.generate_w16()


@pytest.fixture(scope="module")
def dtl_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "dtl.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", os.path.join(CSRC, "hif8_gemm_dtl.hip"), "-o", str(out),
           "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    # the assembler checks operand ranges (e.g. lgkmcnt <= 15) that -S does not
    obj = subprocess.run(cmd[:-5] + ["-c", os.path.join(CSRC, "hif8_gemm_dtl.hip"), "-o", str(out) + ".o"],
                         capture_output=True, text=True, timeout=600)
    assert obj.returncode == 0, obj.stderr[-2000:]
    return out.read_text(), r.stderr


def test_resources(dtl_asm):
    """Both instantiations (plain and GELU + amax epilogue)."""
    _, remarks = dtl_asm
    spills = re.findall(r"(?:VGPRs|SGPRs) Spill: (\d+)", remarks)
    lds = re.findall(r"LDS Size \[bytes/block\]: (\d+)", remarks)
    scratch = re.findall(r"ScratchSize \[bytes/lane\]: (\d+)", remarks)
    assert len(lds) == 2 and set(lds) == {"163840"}, lds
    assert spills and set(spills) == {"0"}, spills
    assert scratch and set(scratch) == {"0"}, scratch


def test_main_loop_hazards(dtl_asm):
    import isa_check
    loops = isa_check.mfma_loops(dtl_asm[0])
    assert len(loops) == 2
    for body in loops:
        kinds = isa_check.census(body)
        assert kinds.get("mfma") == 256 and kinds.get("lds_load") == 208 and kinds.get("lds_dma") == 24, kinds
        errors = isa_check.check_body(body)
        assert not errors, "\n".join(errors[:20])


def test_load_groups_share_m0(dtl_asm):
    """Global->LDS loads go in groups of four behind one m0 write: in each main loop, every
    `buffer_load_dwordx4 ... lds` without an offset follows an m0 write, the next three carry
    offsets 0x400, 0x800, 0xc00 in order, and nothing else writes m0 in between."""
    loops = _dtl_loop_lines(dtl_asm[0])
    assert len(loops) == 2
    for lines in loops:
        expect, m0_set, groups = None, False, 0
        for ln in lines:
            op = ln.split()[0] if ln.split() else ""
            if "m0" in ln and not op.startswith("buffer_load"):
                assert op == "s_mov_b32" and ln.split()[1].rstrip(",") == "m0", ln
                assert expect in (None, 0x1000), f"m0 written inside a group: {ln}"
                m0_set, expect = True, None
            elif op == "buffer_load_dwordx4" and ln.rstrip().endswith("lds"):
                m = re.search(r"offset:(0x[0-9a-f]+|\d+)", ln)
                off = int(m.group(1), 0) if m else 0
                if off == 0:
                    assert m0_set, f"group load without its m0 write: {ln}"
                    m0_set, expect, groups = False, 0x400, groups + 1
                else:
                    assert off == expect, f"offset {off:#x} where {expect} was due: {ln}"
                    expect = off + 0x400
        assert groups == 6 and expect == 0x1000, (groups, expect)


def _dtl_loop_lines(asm):
    """The instruction lines of each MFMA main loop of the fused kernel's assembly."""
    import isa_check
    return [[text for _, _, text in body] for body in isa_check.mfma_loops(asm)]


def test_checker_catches_planted_mistakes():
    """The checker must flag a read of an in-flight LDS load and a VALU->MFMA gap of 1."""
    import isa_check
    body = isa_check.parse([
        "ds_read_b128 v[4:7], v1 offset:0",
        "v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], a[0:15]",
        "s_waitcnt lgkmcnt(0)",
        "v_perm_b32 v12, v2, v3, s0",
        "v_mfma_f32_32x32x16_bf16 a[16:31], v[12:15], v[8:11], a[16:31]",
    ])
    errs = isa_check.check_body(body)
    assert any("in flight" in e for e in errs)
    assert any("after a VALU write" in e for e in errs)
    merge = isa_check.parse([
        "ds_read_u16 v20, v1 offset:0",
        "ds_read_u16_d16_hi v20, v2 offset:0",
    ])
    assert any("in flight" in e for e in isa_check.check_body(merge))
    ok = isa_check.parse([
        "ds_read_b128 v[4:7], v1 offset:0",
        "s_waitcnt lgkmcnt(0)",
        "v_perm_b32 v12, v2, v3, s0",
        "s_nop 2",
        "v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[12:15], a[0:15]",
    ])
    assert not isa_check.check_body(ok)


@pytest.fixture(scope="module")
def w16_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa16") / "w16.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", os.path.join(CSRC, "hif8_gemm_w16.hip"), "-o", str(out),
           "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    obj = subprocess.run(cmd[:-5] + ["-c", os.path.join(CSRC, "hif8_gemm_w16.hip"), "-o", str(out) + ".o"],
                         capture_output=True, text=True, timeout=600)
    assert obj.returncode == 0, obj.stderr[-2000:]
    return out.read_text(), r.stderr


def test_w16_resources(w16_asm):
    """The decode-free twin: its five instantiations (bf16 epilogue, GELU statistic, fp32 split
    partials; the last and the first also with token-major operands) with the 160 KB LDS ring, the
    split-tail reduce kernel without LDS, no spills."""
    _, remarks = w16_asm
    spills = re.findall(r"(?:VGPRs|SGPRs) Spill: (\d+)", remarks)
    lds = re.findall(r"LDS Size \[bytes/block\]: (\d+)", remarks)
    scratch = re.findall(r"ScratchSize \[bytes/lane\]: (\d+)", remarks)
    assert sorted(lds) == ["0"] + ["163840"] * 5, lds
    assert spills and set(spills) == {"0"}, spills
    assert scratch and set(scratch) == {"0"}, scratch


def test_w16_main_loop_hazards(w16_asm):
    """Per k-step: 128 MFMAs (16x16x32), 16 global->LDS loads, and 32 fragment reads (16 per
    phase), or 64 transposing reads for token-major operands (two per fragment), with no register
    copies of the fragments (each pair of reads lands in its fragment's registers)."""
    import isa_check
    loops = isa_check.mfma_loops(w16_asm[0])
    assert len(loops) == 5
    reads = []
    for body in loops:
        kinds = isa_check.census(body)
        assert kinds.get("mfma") == 128 and kinds.get("lds_dma") == 16, kinds
        reads.append(kinds.get("lds_load"))
        assert not any(ins[0].startswith("v_mov") for ins in body), "fragment copies in the loop"
        errors = isa_check.check_body(body)
        assert not errors, "\n".join(errors[:20])
    assert sorted(reads) == [32, 32, 32, 64, 64], reads
