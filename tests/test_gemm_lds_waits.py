"""CPU check of the GEMMs' hand-counted LDS waits.

The matrix-core GEMMs read LDS with inline-asm ds_read instructions and wait for
them with hand-written `s_waitcnt lgkmcnt(N)` (aeth_gemm_common.hpp): the
compiler cannot see when such a read's destination registers become valid, so
it could schedule a use (or a copy into another register) of a destination
before the wait that covers it, and the result would be silently wrong. This
test compiles the GEMM sources for gfx950 to assembly, as the build does, and
runs a dataflow check over every kernel: for each instruction, no source or
destination register may be the destination of an LDS read that the waits on
every path to it leave in flight.

The model: LDS operations of one wave complete in issue order, so after
`s_waitcnt lgkmcnt(N)` every LDS read that has at least N LDS operations issued
after it is complete (scalar-memory operations also count in lgkmcnt but may
complete early, so they never make a wait stronger and are ignored). At a join
of control flow a register keeps the smallest such age over its predecessors.
Loops are followed to a fixed point.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "aether_amd", "csrc")
# the kernels with inline-asm LDS reads, and aeth_gemm.hip's compiler-scheduled ones (the checker must pass those)
SOURCES = ["aeth_gemm_kq.hip", "aeth_gemm_q6k.hip", "aeth_gemm_q80.hip", "aeth_gemm.hip"]

_REG_RANGE = re.compile(r"\b([va])\[(\d+):(\d+)\]")
_REG_ONE = re.compile(r"\b([va])(\d+)\b")
_LABEL = re.compile(r"^(\.LBB\w+|_Z\w+):")
_BRANCH = re.compile(r"^s_(?:cbranch_\w+|branch)\s+(\.LBB\w+)")
_WAIT = re.compile(r"lgkmcnt\((\d+)\)")
NO_DEST = ("ds_write", "ds_store", "global_store", "buffer_store", "flat_store", "scratch_store", "ds_add_u32",
           "ds_add_f32", "ds_max", "ds_min", "s_waitcnt", "s_nop", "s_barrier", "s_branch", "s_cbranch",
           "s_endpgm", "s_setprio", "s_sleep", "s_sched", "s_dcache", "buffer_wbl2", "buffer_inv")


def regs(text):
    """The VGPRs / AGPRs an operand string names, as ('v', n) / ('a', n)."""
    out = set()
    for kind, lo, hi in _REG_RANGE.findall(text):
        out.update((kind, i) for i in range(int(lo), int(hi) + 1))
    text = _REG_RANGE.sub(" ", text)
    out.update((kind, int(n)) for kind, n in _REG_ONE.findall(text))
    return out


def split_operands(line):
    """(opcode, dest registers, source registers) of one instruction line."""
    body = line.split(";")[0].strip()
    op, _, rest = body.partition(" ")
    ops = [o.strip() for o in rest.split(",")] if rest.strip() else []
    if not ops or op.startswith(NO_DEST):
        return op, set(), regs(rest)
    dest = regs(ops[0])
    return op, dest, regs(",".join(ops[1:]))


def kernels(asm):
    """{name: [instruction or label lines]} for every kernel of an assembly file."""
    out, cur, name = {}, None, None
    for raw in asm.splitlines():
        line = raw.strip()
        if not line or line.startswith(";"):
            continue
        m = _LABEL.match(line)
        if m and m.group(1).startswith("_Z") and raw.startswith("_Z"):
            name, cur = m.group(1), []
            out[name] = cur
            continue
        if cur is None:
            continue
        if line.startswith(".Lfunc_end"):
            cur, name = None, None
            continue
        if m or not line.startswith("."):
            cur.append(line)
    return out


def blocks(lines):
    """Basic blocks: [(label or None, [instructions], [successor labels], falls_through)]."""
    out, cur = [], [None, [], [], True]
    for line in lines:
        m = _LABEL.match(line)
        if m:
            if cur[1] or cur[0] is not None:
                out.append(cur)
            cur = [m.group(1), [], [], True]
            continue
        cur[1].append(line)
        b = _BRANCH.match(line)
        if b:
            cur[2].append(b.group(1))
            if line.startswith("s_branch"):
                cur[3] = False
            out.append(cur)
            cur = [None, [], [], True]
        elif line.startswith("s_endpgm"):
            cur[3] = False
            out.append(cur)
            cur = [None, [], [], True]
    if cur[1] or cur[0] is not None:
        out.append(cur)
    return out


def step(state, line, problems, where):
    """Applies one instruction to state {register: age}; records hazards."""
    op, dest, src = split_operands(line)
    live = set(state)
    bad = (src | dest) & live
    if bad and not op.startswith("s_waitcnt"):
        problems.append("%s: %r uses %s while an LDS read into it may be in flight" %
                        (where, line, sorted(bad)[:4]))
    if op.startswith("s_waitcnt"):
        m = _WAIT.search(line)
        if m is not None or re.fullmatch(r"s_waitcnt\s+0", line.split(";")[0].strip()):
            n = int(m.group(1)) if m else 0
            for r in [r for r, age in state.items() if age >= n]:
                del state[r]
    elif op.startswith("ds_"):
        for r in list(state):
            state[r] += 1
        if not op.startswith(NO_DEST):
            for r in dest:
                state[r] = 0


def check_kernel(lines, name):
    bl = blocks(lines)
    index = {b[0]: i for i, b in enumerate(bl) if b[0] is not None}
    succ = []
    for i, (_, _, targets, falls) in enumerate(bl):
        s = [index[t] for t in targets if t in index]
        if falls and i + 1 < len(bl):
            s.append(i + 1)
        succ.append(s)
    entry = [None] * len(bl)
    entry[0] = {}
    work = [0]
    problems = []
    seen_msgs = set()
    while work:
        i = work.pop()
        state = dict(entry[i])
        local = []
        for k, line in enumerate(bl[i][1]):
            step(state, line, local, "%s block %s+%d" % (name, bl[i][0], k))
        for p in local:
            if p not in seen_msgs:
                seen_msgs.add(p)
                problems.append(p)
        for j in succ[i]:
            if entry[j] is None:
                entry[j] = dict(state)
                work.append(j)
                continue
            merged = dict(entry[j])
            changed = False
            for r, age in state.items():
                if r not in merged or age < merged[r]:
                    merged[r] = age
                    changed = True
            if changed:
                entry[j] = merged
                work.append(j)
    return problems


def compile_asm(src, out):
    from aether_amd import build as B

    cmd = B.compile_command(src, out)
    cmd = [c for c in cmd if c not in ("-c",)]
    cmd.insert(cmd.index("-o"), "--cuda-device-only")
    cmd.insert(cmd.index("-o"), "-S")
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]


@pytest.fixture(scope="module")
def assembly():
    if not shutil.which("hipcc") and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    tmp = tempfile.mkdtemp(prefix="aeth_lds_")
    out = {}
    try:
        paths = [os.path.join(tmp, s + ".s") for s in SOURCES]
        with concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as ex:
            list(ex.map(compile_asm, SOURCES, paths))
        for s, path in zip(SOURCES, paths):
            out[s] = open(path).read()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return out


def test_checker_finds_a_planted_early_use():
    """The checker itself: a use of a read's destination before its wait is
    reported, after the wait it is not, and a loop carries a read across its
    back edge."""
    early = ["ds_read_b128 v[4:7], v1 offset:0", "ds_read_b64 v[8:9], v1 offset:16", "s_waitcnt lgkmcnt(1)",
             "v_add_u32_e32 v10, v4, v5", "v_add_u32_e32 v11, v8, v5", "s_waitcnt lgkmcnt(0)",
             "v_add_u32_e32 v11, v8, v9", "s_endpgm"]
    probs = check_kernel(early, "planted")
    assert len(probs) == 1 and "v_add_u32_e32 v11, v8, v5" in probs[0]
    loop = [".LBB0_1:", "v_mov_b32_e32 v20, v4", "ds_read_b32 v4, v1 offset:0", "s_cbranch_scc1 .LBB0_1",
            "s_waitcnt lgkmcnt(0)", "s_endpgm"]
    probs = check_kernel(loop, "loop")
    assert any("v_mov_b32_e32 v20, v4" in p for p in probs)
    copy = ["ds_read_b128 v[4:7], v1 offset:0", "v_accvgpr_write_b32 a0, v5", "s_waitcnt lgkmcnt(0)", "s_endpgm"]
    assert check_kernel(copy, "copy")


@pytest.mark.parametrize("src", SOURCES)
def test_no_lds_destination_used_before_its_wait(assembly, src):
    ks = kernels(assembly[src])
    assert ks, "no kernels found in %s" % src
    n_reads = sum(1 for lines in ks.values() for l in lines if l.startswith("ds_read"))
    assert n_reads > 0
    problems = []
    for name, lines in ks.items():
        problems += check_kernel(lines, name)
    assert not problems, "\n".join(problems[:20])
