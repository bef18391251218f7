"""CPU checks of the drop-in boundary: the C-ABI library loads without a GPU
and exports every function include/*.h declares (no compute calls)."""
import ctypes
import os
import subprocess

import aether_amd as A


def test_library_exports_every_declared_symbol():
    names = A.header_symbols()
    assert len(names) >= 50
    L = A.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_exports_are_exactly_the_declared_ones():
    out = subprocess.run(["nm", "-D", "--defined-only", A.LIB_PATH], stdout=subprocess.PIPE, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-2] in ("T", "W")}
    ours = {n for n in exported if n.startswith(("aeth_", "aether_"))}
    assert ours == set(A.header_symbols())


def test_block_geometry_and_errors_without_gpu():
    L = A.lib()
    e, b = ctypes.c_int(), ctypes.c_int()
    for dt, geo in ((8, (32, 34)), (12, (256, 144)), (13, (256, 176)), (14, (256, 210))):
        assert L.aeth_block_geometry(dt, ctypes.byref(e), ctypes.byref(b)) == 0
        assert (e.value, b.value) == geo
    assert L.aeth_block_geometry(2, ctypes.byref(e), ctypes.byref(b)) == -4  # Q4_0 is not on this path
    assert "unsupported" in A.last_error()
    # NULL arguments are refused before any device work
    assert L.aeth_weight_create(12, 4, 256, None, 0, None, None) == -1
    assert L.aeth_dequant(12, None, 256, None, None) == -1
    assert L.aether_load(b"/nonexistent/model.gguf") is None


def test_header_is_plain_c():
    """The headers compile as C (no torch or C++ types in the signatures)."""
    inc = os.path.join(os.path.dirname(A.HERE), "include")
    src = '#include "aether_hip.h"\n#include "aether.h"\nint main(void){return 0;}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", inc, "-x", "c", "-", "-o", "/dev/null"],
                       input=src, text=True, stderr=subprocess.PIPE)
    assert r.returncode == 0, r.stderr


def test_weight_fingerprint_sees_every_byte():
    """The content check of the host-slice weight cache (CPU only): the same bytes
    give the same fingerprint from any thread; one byte changed at the start, in
    the middle or at the end of a 40 MiB buffer (hashed in 1 MiB chunks by the
    library's persistent host thread pool) or of a small one changes it."""
    import threading

    import numpy as np

    L = A.lib()

    def fp(buf):
        out = ctypes.c_uint64()
        assert L.aeth_weight_fingerprint(buf.ctypes.data, buf.nbytes, ctypes.byref(out)) == 0
        return out.value

    for size in (40 << 20, 4096 + 7):
        buf = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8)
        base = fp(buf)
        seen = []
        th = [threading.Thread(target=lambda: seen.append(fp(buf))) for _ in range(4)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        assert seen == [base] * 4
        for pos in (0, size // 2, size - 1, (1 << 20) + 3 if size > (1 << 21) else 1):
            buf[pos] ^= 1
            assert fp(buf) != base, pos
            buf[pos] ^= 1
        assert fp(buf) == base
        assert fp(buf[:-1]) != base  # the length enters the fingerprint
