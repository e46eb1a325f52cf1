"""No register of the built library is used while a load into it is in flight.

The GEMM kernels read LDS fragments (and the MX kernel one global word) from
inline asm and wait for them later, so the compiler's own waits do not drain the
direct-to-LDS loads in flight. The compiler does not know those registers are
pending; a copy or reuse it inserts before the wait (a merge of two paths after a
branch, a spill) would compute with stale data silently. This test disassembles
the in-tree library's gfx950 code and checks every kernel for such uses; the
checker itself is pinned on hand-written instruction sequences."""
import os
import shutil

import pytest

from _isa_waits import disassemble, gfx950_code_objects, scan

LIB = os.path.join(os.path.dirname(__file__), "..", "vllm-neuron_amd", "vllm_neuron_amd", "lib",
                   "libmoe_fp8.so")
OBJDUMP = shutil.which("llvm-objdump", path="/opt/rocm/llvm/bin") or shutil.which("llvm-objdump")


def test_checker_flags_use_before_wait():
    # the pattern the compiler produced for a read issued under a branch: a copy of
    # the destination before the wait
    bad = ["0000000000001000 <k>:",
           "\tds_read_b128 v[188:191], v204 offset:0",
           "\tv_mov_b64_e32 v[206:207], v[190:191]",
           "\ts_waitcnt lgkmcnt(0)"]
    assert [v[1] for v in scan(bad)] == ["v_mov_b64_e32 v[206:207], v[190:191]"]
    # an older read retired by lgkmcnt(1) while a newer one is still pending
    mixed = ["0000000000001000 <k>:",
             "\tds_read_b128 v[0:3], v10",
             "\tds_read_b128 v[4:7], v11",
             "\ts_waitcnt lgkmcnt(1)",
             "\tv_add_f32_e32 v20, v0, v1",
             "\tv_add_f32_e32 v21, v4, v1"]
    assert [v[1] for v in scan(mixed)] == ["v_add_f32_e32 v21, v4, v1"]
    # a global load into a register the compiler then overwrites before vmcnt
    vm = ["0000000000001000 <k>:",
          "\tglobal_load_dword v5, v[2:3], off  // 000000001000: DC508000 057F0002",
          "\tv_mov_b32_e32 v5, 0  // 000000001008: 7E0A0280",
          "\ts_waitcnt vmcnt(0)  // 00000000100C: BF8C0F70"]
    assert len(scan(vm)) == 1
    # ... unless it runs only with EXEC = 0 (jumped over when any lane is active);
    # a non-returning atomic has no destination
    skip = ["0000000000001000 <k>:",
            "\tglobal_load_dword v5, v[2:3], off  // 000000001000: DC508000 057F0002",
            "\ts_cbranch_execnz 1  // 000000001008: BF890001",
            "\tv_mov_b32_e32 v5, 0  // 00000000100C: 7E0A0280",
            "\tglobal_atomic_add v3, v2, s[10:11]  // 000000001010: DD088000 000A0203",
            "\tv_mov_b32_e32 v3, 1  // 000000001018: 7E060281",
            "\ts_waitcnt vmcnt(0)  // 00000000101C: BF8C0F70"]
    assert scan(skip) == []
    ret = ["0000000000001000 <k>:",
           "\tglobal_atomic_add v3, v[4:5], v2, off sc0  // 000000001000: DD098000 03000204",
           "\tv_mov_b32_e32 v6, v3  // 000000001008: 7E0C0303"]
    assert len(scan(ret)) == 1
    # direct-to-LDS loads have no register destination; MFMA operands read after the wait
    good = ["0000000000001000 <k>:",
            "\tglobal_load_lds_dwordx4 v134, s[58:59]",
            "\tds_read_b128 v[80:83], v8",
            "\tds_read_b128 v[84:87], v9",
            "\tv_mul_f32_e32 v100, v100, v101",
            "\ts_waitcnt lgkmcnt(0)",
            "\tv_mfma_f32_16x16x128_f8f6f4 v[176:179], v[24:31], v[80:87], v[176:179]",
            "\ts_branch 4",
            "\tds_read_b32 v1, v2",
            "\ts_waitcnt vmcnt(0) lgkmcnt(0)",
            "\tv_mov_b32_e32 v3, v1"]
    assert scan(good) == []


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
@pytest.mark.skipif(OBJDUMP is None, reason="llvm-objdump not available")
def test_library_has_no_use_of_pending_load_registers(tmp_path):
    objs = gfx950_code_objects(LIB)
    assert objs, "no gfx950 code objects in the library"
    found, kernels = [], 0
    for o in objs:
        lines = disassemble(o, OBJDUMP, tmp_path)
        kernels += sum(1 for l in lines if l.strip().endswith(">:"))
        found += scan(lines)
    assert kernels > 20
    assert not found, "\n".join(f"{f}: '{t}' before the wait for '{s}'" for f, t, s in found[:20])
