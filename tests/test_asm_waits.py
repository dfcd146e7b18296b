"""Hand-counted waits on inline-asm loads, checked on the gfx950 assembly of
every kernel source (no GPU needed: hipcc cross-compiles).  The checker is
pinned on small assembly snippets first: a register read before its load is
retired must be flagged; the same read after the wait, or after a partial
wait that retires it, must not be."""

import concurrent.futures as cf
import os
import shutil
import tempfile

import pytest

from tests.asm_wait_check import registers, scan

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _fn(body: str) -> str:
    return "_Zkern:\n" + "\n".join("\t" + l for l in body.strip().split("\n")) + "\n.Lfunc_end0:\n"


def test_registers_parse_ranges_and_singles():
    assert registers("v[4:7], v1 offset:16") == {"v4", "v5", "v6", "v7", "v1"}
    assert registers("a[0:1], s[2:3]") == {"a0", "a1"}


def test_read_before_wait_is_flagged():
    asm = _fn("""
;;#ASMSTART
ds_read_b128 v[8:11], v1 offset:0
;;#ASMEND
v_mov_b32 v20, v9
s_waitcnt lgkmcnt(0)
""")
    hz = scan(asm)
    assert len(hz) == 1 and "v_mov_b32" in hz[0].text


def test_spill_of_pending_destination_is_flagged():
    asm = _fn("""
;;#ASMSTART
ds_read_b64_tr_b16 v[248:249], v1 offset:0
;;#ASMEND
scratch_store_dwordx4 off, v[248:251], off offset:8
s_waitcnt lgkmcnt(0)
""")
    assert len(scan(asm)) == 1


def test_uses_after_the_retiring_wait_are_clean():
    asm = _fn("""
;;#ASMSTART
ds_read_b128 v[8:11], v1 offset:0
;;#ASMEND
;;#ASMSTART
ds_read_b128 v[12:15], v1 offset:512
;;#ASMEND
s_waitcnt lgkmcnt(1)
v_mfma_f32_32x32x16_bf16 v[16:31], v[8:11], v[40:43], v[16:31]
s_waitcnt lgkmcnt(0)
v_mfma_f32_32x32x16_bf16 v[16:31], v[12:15], v[40:43], v[16:31]
""")
    assert scan(asm) == []


def test_partial_wait_keeps_the_younger_load_pending():
    asm = _fn("""
;;#ASMSTART
ds_read_b128 v[8:11], v1 offset:0
;;#ASMEND
;;#ASMSTART
ds_read_b128 v[12:15], v1 offset:512
;;#ASMEND
s_waitcnt lgkmcnt(1)
v_mov_b32 v30, v12
s_waitcnt lgkmcnt(0)
""")
    hz = scan(asm)
    assert len(hz) == 1 and "v12" in hz[0].text


def test_compiler_loads_are_not_tracked_and_functions_reset():
    asm = _fn("""
ds_read_b128 v[8:11], v1
v_mov_b32 v20, v9
""") + _fn("""
;;#ASMSTART
ds_read_b128 v[8:11], v1
;;#ASMEND
""") + _fn("""
v_mov_b32 v20, v9
""")
    assert scan(asm) == []


def _kernel_sources():
    csrc = os.path.join(ROOT, "nano-qwen_amd", "csrc")
    return sorted(os.path.join(csrc, f) for f in os.listdir(csrc) if f.endswith(".hip"))


@pytest.mark.skipif(not (os.path.exists("/opt/rocm/bin/hipcc") or shutil.which("hipcc")),
                    reason="hipcc is needed to produce the gfx950 assembly")
def test_kernel_assembly_has_no_pending_register_use():
    from nano_qwen_amd.build import device_asm
    srcs = _kernel_sources()
    with tempfile.TemporaryDirectory() as tmp:
        outs = [os.path.join(tmp, os.path.basename(s) + ".s") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            list(ex.map(lambda so: device_asm(*so), zip(srcs, outs)))
        asm_loads = 0
        problems = []
        for src, out in zip(srcs, outs):
            text = open(out).read()
            asm_loads += text.count(";;#ASMSTART")
            problems += [f"{os.path.basename(src)}: {h}" for h in scan(text)]
    assert asm_loads > 0, "no inline asm found: the check would be vacuous"
    assert not problems, "\n".join(problems[:20])
