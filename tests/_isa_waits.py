"""Scan of gfx950 assembly for registers used while a load into them is in flight.

Several kernels issue LDS reads (and one global load) from inline asm and wait
for them later with an explicit s_waitcnt, so that the compiler does not drain
other loads in flight. The compiler does not know such a register is pending: if
it copies, reads or reuses it before the wait (for instance to merge two paths
after a branch), the kernel computes with stale data and no error is raised. This
module finds such uses in disassembled code.

Model: per counter (lgkmcnt for LDS and scalar memory, vmcnt for vector memory),
the loads in flight form a queue in issue order; s_waitcnt <cnt>(N) retires all
but the newest N. An instruction that reads or writes a VGPR or AGPR that is the
destination of a queued load is reported. The scan is linear: after an
unconditional branch the queues are cleared, code reached only through a branch
target is checked with the state the straight-line order gives, and instructions
that s_cbranch_execnz jumps over (they run only with EXEC = 0 and change nothing)
are skipped."""
import re
import struct
import subprocess

_REG = re.compile(r"^([va])(?:\[(\d+):(\d+)\]|(\d+))$")
_WAIT = re.compile(r"(vmcnt|lgkmcnt)\((\d+)\)")
_FUNC = re.compile(r"^[0-9a-fA-F]+ <(.+)>:$")


def _regs(tok):
    m = _REG.match(tok.strip())
    if not m:
        return set()
    kind = m.group(1)
    if m.group(4) is not None:
        return {(kind, int(m.group(4)))}
    return {(kind, i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}


def _operands(text):
    return [a.strip().split()[0] for a in text.split(",") if a.strip()]


def _classify(op, args):
    """(counter, destination registers) of a memory instruction, or None."""
    if op.startswith("ds_"):
        has_dst = (op.startswith(("ds_read", "ds_bpermute", "ds_permute", "ds_swizzle", "ds_consume",
                                  "ds_append")) or "_rtn_" in op)
        return "lgkm", (_regs(args[0]) if has_dst and args else set())
    if op.startswith(("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_getpc", "s_dcache")):
        return "lgkm", set()
    if op.startswith(("global_", "buffer_", "flat_", "scratch_")):
        if "_lds_" in op or op.endswith("_lds") or " lds" in op:
            return "vm", set()
        # atomics return a value only with sc0 (glc before gfx940)
        loads = ("_load" in op) or ("_atomic" in op and (" sc0" in op or " glc" in op))
        return "vm", (_regs(args[0]) if loads and args else set())
    return None


_ADDR = re.compile(r"//\s*([0-9A-Fa-f]+):")


def scan(lines):
    """Violations in disassembly lines (llvm-objdump -d output, whose comments give
    each instruction's address)."""
    out = []
    func = "?"
    q = {"vm": [], "lgkm": []}
    skip_to = -1  # code jumped over by s_cbranch_execnz runs with EXEC = 0: no effect
    for raw in lines:
        m = _FUNC.match(raw.strip())
        if m:
            func = m.group(1)
            q = {"vm": [], "lgkm": []}
            skip_to = -1
            continue
        am = _ADDR.search(raw)
        addr = int(am.group(1), 16) if am else None
        text = raw.split("//")[0].split(";")[0].strip()
        if not text or text.endswith(":") or text.startswith("."):
            continue
        if addr is not None and addr < skip_to:
            continue
        op, _, rest = text.partition(" ")
        if op == "s_cbranch_execnz" and addr is not None:
            try:
                skip_to = addr + 4 + 4 * int(rest.split()[0])
            except ValueError:
                pass
            continue
        if op.startswith(("buffer_", "global_", "flat_")):
            for mod in (" lds", " sc0", " glc"):
                if mod in " " + rest:
                    op = op + mod
        args = _operands(rest)
        if op == "s_waitcnt":
            found = dict((k, int(v)) for k, v in _WAIT.findall(rest))
            if rest.strip() == "0":
                found = {"vmcnt": 0, "lgkmcnt": 0}
            for name, key in (("vmcnt", "vm"), ("lgkmcnt", "lgkm")):
                if name in found:
                    n = found[name]
                    q[key] = q[key][len(q[key]) - n:] if n < len(q[key]) else q[key]
                    if n == 0:
                        q[key] = []
            continue
        if op in ("s_branch", "s_setpc_b64", "s_endpgm"):
            q = {"vm": [], "lgkm": []}
            continue
        if op.startswith("s_"):
            cls = _classify(op, args)
            if cls:
                q[cls[0]].append((set(), text))
            continue
        used = set()
        for a in args:
            used |= _regs(a)
        for key in ("vm", "lgkm"):
            for dst, src in q[key]:
                hit = dst & used
                if hit:
                    out.append((func, text, src))
                    break
        cls = _classify(op, args)
        if cls:
            q[cls[0]].append((cls[1], text))
    return out


def gfx950_code_objects(lib_path):
    """The gfx950 code objects of a hipcc-built shared library (its .hip_fatbin
    section holds one clang offload bundle per translation unit)."""
    data = open(lib_path, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    objs = []
    for m in re.finditer(re.escape(magic), data):
        st = m.start()
        n = struct.unpack_from("<Q", data, st + 24)[0]
        p = st + 32
        for _ in range(n):
            off, size, idl = struct.unpack_from("<QQQ", data, p)
            p += 24
            tid = data[p:p + idl].decode(errors="replace")
            p += idl
            if tid.endswith("gfx950") and size > 0:
                objs.append(data[st + off:st + off + size])
    return objs


def disassemble(obj_bytes, objdump, tmp_path):
    f = tmp_path / "code.o"
    f.write_bytes(obj_bytes)
    r = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(f)], capture_output=True, text=True,
                       check=True)
    return r.stdout.splitlines()
