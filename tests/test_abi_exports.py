"""The C-ABI library loads and exports what include/*.h declare (no GPU
needed: nothing here launches work)."""
import ctypes as C
import os
import re
import subprocess

import pytest

import ctbind as cb

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:backend|hipb)_[A-Za-z0-9_]+)\s*\(", text))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], check=True,
                         capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_backend_abi_exports():
    """The reference's 40 functions, plus the one allocation-free variant
    declared after them."""
    names = declared("backend.h")
    assert names - set(cb.ABI_SIGS) == set(cb.ABI_EXT_SIGS)
    assert len(names - set(cb.ABI_EXT_SIGS)) == 40
    assert set(cb.ABI_SIGS) <= names
    syms = exported(cb.HIP_LIB)
    assert names <= syms
    lib = C.CDLL(cb.HIP_LIB)
    for n in names:
        assert getattr(lib, n)


def test_engine_exports():
    path = os.path.join(REPO, "include", "hipb.h")
    if not os.path.exists(path):
        return
    names = declared("hipb.h")
    assert names and names <= exported(cb.HIP_LIB)


def test_product_does_not_link_the_oracle():
    syms = subprocess.run(["nm", "-D", cb.HIP_LIB], check=True, capture_output=True, text=True).stdout
    assert "orc_" not in syms
    deps = subprocess.run(["ldd", cb.HIP_LIB], capture_output=True, text=True).stdout
    assert "oracle" not in deps and "ref_cpu" not in deps


def test_kernel_struct_mirrors_match():
    """The tests' ctypes mirrors of CtGemv, CtWarmSet and CtGemm have the C structs' sizes."""
    from structs import CtGemm, CtGemv, CtWarmSet
    lib = C.CDLL(cb.HIP_LIB)
    lib.ctk_gemv_sizeof.restype = C.c_int
    lib.ctk_warmset_sizeof.restype = C.c_int
    lib.ctk_gemm_sizeof.restype = C.c_int
    assert C.sizeof(CtGemv) == lib.ctk_gemv_sizeof()
    assert C.sizeof(CtWarmSet) == lib.ctk_warmset_sizeof()
    assert C.sizeof(CtGemm) == lib.ctk_gemm_sizeof()


def test_gemv_read_ahead_descriptor_covers_each_tile_once():
    """ctk_gemv_warm (host code) describes the tiles each decode-GEMM
    workgroup reads: workgroup i (K-slice i % gy, column position i / gy)
    reads cb column blocks x per K-steps.  For every decoder shape and row
    count the workgroups' tiles together are each weight tile exactly once,
    the split matches ctk_gemv_ksplit, and a QKV launch's head-h tiles sit on
    XCD h."""
    import numpy as np
    from structs import CtGemv, CtWarm
    lib = C.CDLL(cb.HIP_LIB)
    lib.ctk_gemv_warm.argtypes = [C.POINTER(CtGemv), C.POINTER(CtWarm)]
    lib.ctk_gemv_ksplit.argtypes = [C.c_int, C.c_int]
    lib.ctk_gemv_ksplit.restype = C.c_int
    def qkv_col(p, cb):      # ct_qkv_col: head-by-head positions of a QKV launch
        j, bph = p >> 3, 8 // cb
        return (j // bph) * (64 // cb) + (p & 7) * bph + j % bph
    widths = set()
    for M in (8, 24, 64, 80):
        for N, K, partial, out in ((3072, 1024, False, 3), (3072, 1024, False, 1), (1024, 1024, True, 0),
                                   (4096, 1024, False, 2), (1024, 4096, True, 0), (16384, 1024, False, 1),
                                   (1024, 1024, False, 4), (1024, 4096, False, 4), (1024, 1024, False, 1)):
            ks = lib.ctk_gemv_ksplit(N, K) if partial else 1
            g = CtGemv(W=1 << 20, M=M, N=N, K=K, ksplit=ks, wtile=1, out=out)
            w = CtWarm()
            lib.ctk_gemv_warm(C.byref(g), C.byref(w))
            assert (w.gy, w.nsteps, w.per * w.gy, w.gx * w.cb * 16) == (ks, K // 32, K // 32, N), (N, K)
            assert (w.gx * w.gy) % 8 == 0    # later row groups land on the same XCDs
            widths.add((N, K, w.cb))
            seen = np.zeros((N // 16) * (K // 32), np.int32)
            assert w.heads == (out == 3)
            for i in range(w.gx * w.gy):
                cx, k = (qkv_col(i // w.gy, w.cb) if w.heads else i // w.gy), i % w.gy
                if w.heads:   # the attention's head h runs on XCD h
                    assert (cx * w.cb * 16 % 1024) // 128 == i % 8
                for c in range(w.cb):
                    t0 = (cx * w.cb + c) * w.nsteps + k * w.per
                    seen[t0:t0 + w.per] += 1
            assert np.all(seen == 1), (M, N, K)
            # the read-ahead's dealing (ct_warm_tiles, 32 rows per XCD): unit u = k*cb + c of
            # XCD x is GEMM workgroup x + 8k's column block c; every tile once, on the GEMM
            # workgroup's XCD, and each read-ahead workgroup's share set by N, K alone
            rows, seen[:] = 32, 0
            for x in range(8):
                U = (w.gx * w.gy - x + 7) // 8 * w.cb
                share = [len(range(j, U, rows)) for j in range(rows)]
                assert max(share) == -(-(N // 16) * ks // 8 // rows), (M, N, K)
                for u in range(U):
                    i, c = x + 8 * (u // w.cb), u % w.cb
                    cx, k = (qkv_col(i // w.gy, w.cb) if w.heads else i // w.gy), i % w.gy
                    t0 = (cx * w.cb + c) * w.nsteps + k * w.per
                    seen[t0:t0 + w.per] += 1
            assert np.all(seen == 1), (M, N, K)
            g.wtile = 0
            lib.ctk_gemv_warm(C.byref(g), C.byref(w))
            assert w.gx == 0
    # every tile width of the QKV launch is covered
    assert {(3072, 1024, 1), (3072, 1024, 2), (3072, 1024, 4)} <= widths


def test_noalloc_variant_rejects_long_clips():
    """backend_rel_pos_mhsa_noalloc refuses clips beyond its 376-frame scratch
    with a clear error before touching any device (checked in a child
    process: the backend exits like the reference's fatal errors)."""
    import sys
    code = ("import ctypes as C; L = C.CDLL(%r); "
            "L.backend_rel_pos_mhsa_noalloc(None, None, 377, None)" % cb.HIP_LIB)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
    assert "T=377 outside [1, 376]" in r.stderr


FATAL_CASES = {
    # weight pointer translated before the blob was uploaded (abi.c ct_dev_w)
    "weight_before_upload": ("L.backend_device_ptr(C.c_void_p(4096))",
                             "weight pointer used before backend_weights_upload_blob"),
    # S beyond MAX_SEQ (the reference's token buffer size)
    "embed_long": ("L.backend_embed(None, None, 1025, 0, None, None, None, None)",
                   "embed: S outside [0, MAX_SEQ]"),
    "upload_tokens_long": ("L.backend_upload_tokens(None, 1025)", "upload_tokens: S outside [0, MAX_SEQ]"),
    # batch beyond the 256 slots the batched entry points stage
    "batch_257": ("L.backend_embed_decode_batch(None, None, None, None, 257, None, None, None, None)",
                  "batch size outside [0, 256]"),
    "batch_negative": ("L.backend_argmax_batch(None, None, None, -1)", "batch size outside [0, 256]"),
    # arena request no device can hold (and whose byte count would overflow)
    "arena_huge": ("L.backend_arena_alloc(C.c_size_t(1 << 62))", "request above 2^40 floats"),
}


@pytest.mark.parametrize("case", sorted(FATAL_CASES))
def test_fatal_paths_before_device_work(case):
    """The backend's error convention is the reference's: print what went
    wrong and exit(1) (backends/cuda/backend.cu:26-33, backends/cpu/
    backend.c:43-46).  Argument checks run before any device work, so each
    of these fires on a host without a GPU: run in a child process, the call
    exits with status 1 and names the problem on stderr."""
    import sys
    call, msg = FATAL_CASES[case]
    code = f"import ctypes as C; L = C.CDLL({cb.HIP_LIB!r}); {call}; print('returned')"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert msg in r.stderr, r.stderr
    assert "returned" not in r.stdout


TRANSCRIBE_HIP = os.path.join(REPO, "oracle", "_ref", "transcribe_hip")


@pytest.mark.skipif(not os.path.exists(TRANSCRIBE_HIP),
                    reason="oracle/_ref/transcribe_hip is built only where the reference sources are")
def test_reference_transcribe_links_against_hip_backend():
    """The reference's CLI host (transcribe.c), unchanged, links against
    libct_hip.so with the link line of the build.sh binding: every backend_*
    symbol it needs is undefined in the binary and defined by the library,
    the loader finds the library, and the program runs to its argument check
    (usage and status 1, transcribe.c:1283-1293) without touching a device."""
    und = subprocess.run(["nm", "-D", "--undefined-only", TRANSCRIBE_HIP], check=True,
                         capture_output=True, text=True).stdout
    needed = {ln.split()[-1] for ln in und.splitlines() if ln.split()[-1].startswith("backend_")}
    assert len(needed) >= 20
    assert needed <= exported(cb.HIP_LIB)
    deps = subprocess.run(["ldd", TRANSCRIBE_HIP], capture_output=True, text=True).stdout
    line = next(ln for ln in deps.splitlines() if "libct_hip.so" in ln)
    assert os.path.realpath(line.split("=>")[1].split()[0]) == os.path.realpath(cb.HIP_LIB)
    r = subprocess.run([TRANSCRIBE_HIP], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Usage:" in r.stderr
