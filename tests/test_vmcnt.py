"""The hand-counted vector-memory waits of the DMA kernels, checked in the gfx950 code of the built libmbq.so.

gemm_kernel, sgemm_kernel, wsgemm_kernel and kgemm_kernel copy x tiles into LDS with `buffer_load ... lds` (DMA) and
wait for them with `s_waitcnt vmcnt(N)` before a barrier, N counting the vector-memory instructions issued after the
DMA that must have landed (they complete in issue order). The compiler does not track that LDS for other waves, so
the count is right only if it matches the instructions the compiler emitted: a load it drops (nothing reads its
result) or merges with another (the same address) leaves N too high, and the barrier then lets the other waves read
the stage before the DMA has landed. sgemm_kernel had exactly that: its last producer steps loaded weights nobody
read, the compiler dropped them, and now and then the final K step of a tile read stale x rows.

This test disassembles each of those kernels from the library (llvm-objdump of the gfx950 code objects in its
.hip_fatbin section) and walks every path of its control flow, keeping the queue of the wave's outstanding
vector-memory instructions (`s_waitcnt vmcnt(N)` keeps the newest N). At each s_barrier, no DMA issued G or more
barriers earlier may still be outstanding, G being the kernel's pipeline distance (the DMA for the stage read after
barrier b is issued before barrier b - G):
  sgemm_kernel   1       (producer step l issues x(l + 2), and barrier l + 1 needs x(l + 1))
  gemm_kernel    P - 1   (x runs P steps ahead; template argument 4)
  wsgemm_kernel  D - 2   (D = 4 stages; the wait precedes the barrier of the step that reads the stage)
  kgemm_kernel   D - 2   (D = kgm_depth(T, MT, RG) stages)
and no path may reach s_endpgm with a DMA outstanding. An exec-masked if / else (s_and_saveexec ... s_cbranch_execz,
then s_andn2_saveexec ... s_cbranch_execz) runs at least one arm, so the path that skips both is not followed.
What the walk cannot tell apart: two stages issued within one barrier interval (a prologue's first stage, read after
the first barrier, and the next). The first is covered by each prologue's own wait: gemm_kernel waits for every load
(vmcnt(0)), sgemm_kernel for all but the next stage's 8 DMA instructions, wsgemm_kernel and kgemm_kernel by their
first step's count, which the prologue's issue order (and, in wsgemm_kernel, a compiler barrier between its
iterations' loads) keeps exact.

The same walk checks a wave's own LDS writes in every kernel that has a barrier: no `ds_write` may be outstanding at
an s_barrier (the barrier does not wait for them, and the other waves read after it), counting `s_waitcnt lgkmcnt(N)`
as keeping the newest N LDS / scalar-memory operations (none retired while a scalar load, which returns out of order,
is among them). sgemm_kernel once had that race (producers passing the barrier before their dequantized weights
landed in LDS), and the check flags every sgemm_kernel instantiation of that build.
"""
import os
import re
import shutil
import struct
import subprocess
from collections import defaultdict
from concurrent.futures import ProcessPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "mashbox_amd", "libmbq.so")
OBJDUMP = next((p for p in ("/opt/rocm/llvm/bin/llvm-objdump", shutil.which("llvm-objdump") or "") if p and os.path.exists(p)), None)

T_Q40T, T_Q4KT, T_Q5KT, T_Q6KT = -11, -12, -13, -14


def kgm_depth(t, mt, rg):
    """the stages of kgemm_kernel's x ring (kgm_depth / kgm_stage / KGM_LDS_MAX of mbq_kgemm.hip)"""
    cw = 128 if t in (T_Q4KT, T_Q5KT, T_Q6KT, T_Q40T) else 64
    stage = 16 * mt * 2 * cw
    return 2 if rg == 1 else (3 if (8 // rg) * 3 * stage <= 160 * 1024 - 256 else 2)


def template_args(name):
    """the integer and bool template arguments of an Itanium-mangled name (ILi12E, ILin12E, ILb1E)"""
    return [(-1 if m.group(2) else 1) * int(m.group(3)) for m in re.finditer(r"L([ib])(n?)(\d+)E", name)]


def guard(name):
    a = template_args(name)
    if "13wsgemm_kernel" in name:
        return 2
    if "12sgemm_kernel" in name:
        return 1
    if "12kgemm_kernel" in name:
        return kgm_depth(a[0], a[1], a[2]) - 2
    if "11gemm_kernel" in name:
        return a[3] - 1
    return None


def code_objects(path):
    """the gfx950 ELF code objects of the clang offload bundles in the library's .hip_fatbin section"""
    data = open(path, "rb").read()
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    sec = [struct.unpack_from("<IIQQQQ", data, shoff + i * shentsize) for i in range(shnum)]
    strtab = sec[shstrndx][4]
    name = lambda s: data[strtab + s[0]:data.index(b"\0", strtab + s[0])].decode()
    fat = next(s for s in sec if name(s) == ".hip_fatbin")
    blob = data[fat[4]:fat[4] + fat[5]]
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    out, p = [], blob.find(magic)
    while p >= 0:
        n, = struct.unpack_from("<Q", blob, p + 24)
        q = p + 32
        for _ in range(n):
            o, size, tlen = struct.unpack_from("<QQQ", blob, q)
            triple = blob[q + 24:q + 24 + tlen].decode()
            q += 24 + tlen
            if "gfx950" in triple:
                out.append(blob[p + o:p + o + size])
        p = blob.find(magic, p + 1)
    return out


VMEM = re.compile(r"^(buffer_|global_|flat_|scratch_)")
LGKM = re.compile(r"^(ds_|s_load|s_buffer_load|s_memtime|s_memrealtime|s_sendmsg|flat_)")
LDS_WRITE = re.compile(r"^ds_(write|store|add|sub|max|min|and|or|xor|inc|dec|cmpst|wrxchg|append|consume)")
LGKMCNT = re.compile(r"lgkmcnt\((\d+)\)")
VMCNT = re.compile(r"vmcnt\((\d+)\)")
BRANCH = re.compile(r"^s_(c?branch\w*)\s+(L\d+)")


def functions(dis):
    """{mangled name: [("label", L) | ("ins", text)]} from llvm-objdump --symbolize-operands output"""
    funcs, cur = {}, None
    for line in dis.splitlines():
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:", line)
        if m:
            if m.group(1).startswith("_Z"):
                cur = funcs.setdefault(m.group(1), [])
            elif cur is not None:
                cur.append(("label", m.group(1)))
            continue
        s = line.split("//")[0].strip()
        if cur is not None and s and not s.startswith(("Disassembly", ".")):
            cur.append(("ins", s))
    return funcs


def blocks(ins):
    """basic blocks [(label, instructions, successor labels)]: a label or a branch ends a block"""
    bl, label, cur, n = [], "entry", [], 0
    for kind, s in ins:
        if kind == "label":
            if cur or label == "entry":
                bl.append([label, cur, [None]])
            label, cur = s, []
            continue
        cur.append(s)
        m = BRANCH.match(s)
        if m or s.startswith("s_endpgm"):
            succ = [] if s.startswith("s_endpgm") else [m.group(2)] if m.group(1) == "branch" else [m.group(2), None]
            bl.append([label, cur, succ])
            n += 1
            label, cur = f"_{n}", []
    if cur:
        bl.append([label, cur, []])
    for k, b in enumerate(bl):                                   # None: fall through to the next block
        b[2] = [bl[k + 1][0] if s is None else s for s in b[2] if s is not None or k + 1 < len(bl)]
    return {b[0]: b for b in bl}, bl[0][0]


def check(args):
    """[(function, problem)] for one function: barriers a DMA may pass, or an end with a DMA outstanding (G >= 0); or,
    with G = None, barriers an LDS write of the wave may pass"""
    fname, ins, G = args
    lds = G is None
    bmap, entry = blocks(ins)
    seen = defaultdict(set)
    work = [(entry, (), False)]
    bad = set()
    while work:
        lab, st, skipped = work.pop()
        if (st, skipped) in seen[lab]:
            continue
        seen[lab].add((st, skipped))
        if len(seen[lab]) > 20000:
            return [(fname, f"too many queue states at {lab}")]
        q = list(st)
        body = bmap[lab][1]
        for k, s in enumerate(body):
            op = s.split()[0]
            if lds:
                if LGKM.match(op):
                    q.append("W" if LDS_WRITE.match(op) else "S" if op.startswith("s_") else "R")
                    q = q[-32:]
                elif op == "s_waitcnt" and LGKMCNT.search(s):
                    keep = int(LGKMCNT.search(s).group(1))
                    if keep == 0:
                        q = []
                    elif "S" not in q:
                        q = q[-keep:]
                elif op == "s_barrier" and "W" in q:
                    bad.add(f"barrier at {lab}+{k}: an LDS write of the wave may be outstanding")
                continue
            if VMEM.match(op):
                dma = op.startswith(("buffer_load", "global_load")) and re.search(r"\blds\b", s) is not None
                q.append(("D" if dma else "L", 0))
                q = q[-64:]
            elif op == "s_waitcnt" and VMCNT.search(s):
                keep = int(VMCNT.search(s).group(1))
                q = q[-keep:] if keep else []
            elif op == "s_barrier":
                if any(kd == "D" and c >= G for kd, c in q):
                    bad.add(f"barrier at {lab}+{k}: a DMA issued {G} or more barriers earlier may be outstanding")
                q = [(kd, min(c + 1, G + 1)) for kd, c in q]
            elif op == "s_endpgm" and any(kd == "D" for kd, _ in q):
                bad.add(f"s_endpgm at {lab}+{k} with a DMA outstanding")
        term = body[-1] if body else ""
        execz = term.startswith("s_cbranch_execz")
        is_then = execz and any(x.startswith("s_and_saveexec") for x in body)
        is_else = execz and (any(x.startswith("s_andn2_saveexec") for x in body) or
                             (any(x.startswith("s_or_saveexec") for x in body) and any(x.startswith("s_xor_b64 exec") for x in body)))
        for k2, sc in enumerate(bmap[lab][2]):
            if sc not in bmap:
                continue
            taken = term.startswith("s_cbranch") and k2 == 0
            if is_else and skipped and taken:
                continue                                      # the then arm was skipped: every lane runs the else arm
            work.append((sc, tuple(q), taken if is_then else False if is_else else skipped))
    return [(fname, b) for b in sorted(bad)]


_FUNCS = []


def _library_functions():
    """every kernel of the library's gfx950 code objects, disassembled once per session"""
    if OBJDUMP is None or not os.path.exists(LIB):
        pytest.skip("needs the built libmbq.so and llvm-objdump")
    if not _FUNCS:
        for k, co in enumerate(code_objects(LIB)):
            path = os.path.join(os.environ.get("TMPDIR", "/tmp"), f"mbq_vmcnt_{os.getpid()}_{k}.co")
            with open(path, "wb") as f:
                f.write(co)
            try:
                dis = subprocess.run([OBJDUMP, "-d", "--symbolize-operands", "--no-show-raw-insn", "--mcpu=gfx950", path],
                                     capture_output=True, text=True, check=True).stdout
            finally:
                os.remove(path)
            _FUNCS.extend(functions(dis).items())
    return _FUNCS


def _dma_kernels():
    found = []
    for fname, ins in _library_functions():
        G = guard(fname)
        if G is not None and any(kind == "ins" and re.search(r"\blds\b", s) for kind, s in ins):
            found.append((fname, ins, G))
    return found


def test_every_lds_dma_lands_before_the_barrier_that_publishes_it():
    kernels = _dma_kernels()
    names = {f for f, _, _ in kernels}
    for kind in ("11gemm_kernel", "12sgemm_kernel", "13wsgemm_kernel", "12kgemm_kernel"):
        assert any(kind in n for n in names), f"no {kind} with LDS DMA found in {LIB}"
    with ProcessPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        problems = [p for r in ex.map(check, kernels, chunksize=4) for p in r]
    assert not problems, f"{len(problems)} problems in {len({f for f, _ in problems})} kernels, e.g. {problems[:4]}"


def test_every_lds_write_lands_before_the_barrier_that_publishes_it():
    kernels = [(f, ins, None) for f, ins in _library_functions() if any(k == "ins" and s.startswith("s_barrier") for k, s in ins)]
    assert any("12sgemm_kernel" in f for f, _, _ in kernels) and len(kernels) > 100, len(kernels)
    with ProcessPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        problems = [p for r in ex.map(check, kernels, chunksize=8) for p in r]
    assert not problems, f"{len(problems)} problems in {len({f for f, _ in problems})} kernels, e.g. {problems[:4]}"


def test_the_checker_finds_an_uncovered_lds_write():
    w = ("ins", "ds_write_b128 v1, v[2:5]")
    assert check(("waited", [w, ("ins", "s_waitcnt lgkmcnt(0)"), ("ins", "s_barrier"), ("ins", "s_endpgm")], None)) == []
    assert check(("unwaited", [w, ("ins", "s_barrier"), ("ins", "s_endpgm")], None))
    # lgkmcnt(1) after the write and a later LDS read retires the write; with a scalar load in flight it does not
    rd = ("ins", "ds_read_b128 v[6:9], v1")
    assert check(("older", [w, rd, ("ins", "s_waitcnt lgkmcnt(1)"), ("ins", "s_barrier"), ("ins", "s_endpgm")], None)) == []
    assert check(("newest", [rd, w, ("ins", "s_waitcnt lgkmcnt(1)"), ("ins", "s_barrier"), ("ins", "s_endpgm")], None))
    sl = ("ins", "s_load_dwordx2 s[0:1], s[4:5], 0x0")
    assert check(("scalar", [w, sl, ("ins", "s_waitcnt lgkmcnt(1)"), ("ins", "s_barrier"), ("ins", "s_endpgm")], None))


def test_the_checker_finds_an_uncovered_dma():
    """the checker itself on small hand-written sequences: a wait one too high lets a DMA pass the barrier"""
    good = [("ins", "buffer_load_dwordx4 v1, s[0:3], 0 offen lds"), ("ins", "buffer_load_dwordx4 v[2:5], v0, s[4:7], 0 offen"),
            ("ins", "s_waitcnt vmcnt(1)"), ("ins", "s_barrier"), ("ins", "s_waitcnt vmcnt(0)"), ("ins", "s_endpgm")]
    assert check(("good", good, 0)) == []
    loose = [x if x[1] != "s_waitcnt vmcnt(1)" else ("ins", "s_waitcnt vmcnt(2)") for x in good]
    assert check(("loose", loose, 0)) and "barrier" in check(("loose", loose, 0))[0][1]
    # G = 1: the DMA may pass one barrier, not two
    two = good[:2] + [("ins", "s_barrier"), ("ins", "s_barrier")] + good[4:]
    assert check(("one", good[:2] + [("ins", "s_barrier")] + good[4:], 1)) == []
    assert check(("two", two, 1))
    # a skipped load on one path (a conditional branch around it) makes the fixed wait too high on that path
    branchy = [("ins", "buffer_load_dwordx4 v1, s[0:3], 0 offen lds"), ("ins", "s_cbranch_scc1 L1"),
               ("ins", "buffer_load_dwordx4 v[2:5], v0, s[4:7], 0 offen"), ("label", "L1"), ("ins", "s_waitcnt vmcnt(1)"),
               ("ins", "s_barrier"), ("ins", "s_waitcnt vmcnt(0)"), ("ins", "s_endpgm")]
    assert check(("branchy", branchy, 0))
    # an exec-masked if / else with the DMA in both arms: one arm always runs
    ifelse = [("ins", "s_and_saveexec_b64 s[2:3], vcc"), ("ins", "s_cbranch_execz L1"),
              ("ins", "buffer_load_dwordx4 v1, s[0:3], 0 offen lds"), ("label", "L1"), ("ins", "s_andn2_saveexec_b64 s[2:3], s[2:3]"),
              ("ins", "s_cbranch_execz L2"), ("ins", "buffer_load_dwordx4 v1, s[0:3], 0 offen lds"), ("label", "L2"),
              ("ins", "buffer_load_dwordx4 v[2:5], v0, s[4:7], 0 offen"), ("ins", "s_waitcnt vmcnt(1)"), ("ins", "s_barrier"),
              ("ins", "s_waitcnt vmcnt(0)"), ("ins", "s_endpgm")]
    assert check(("ifelse", ifelse, 0)) == []
    assert check(("end", good[:2] + [("ins", "s_endpgm")], 0))
