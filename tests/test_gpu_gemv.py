"""GPU checks of the decode step's GEMM (ctk_gemv) and residual LayerNorm
(ctk_ln_frag), called through libct_hip.so's C entry points.

The activations are given directly as (hi, lo) bf16 pairs in the frag layout,
so the exact operand is x = hi + lo and the float64 product x W^T is the
reference; fp32 accumulation over K <= 4096 terms stays within 1e-5 of it
(relative to the largest output).  Each row's result must not depend on how
many rows the launch has, or where the row sits: bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

import ctbind as cb
import kernel_suite as ks
from structs import CtGemv, CtWarm, CtWarmSet

pytestmark = pytest.mark.gpu

PARTIAL, DENSE, FRAG, QKV = 0, 1, 2, 3
TOL = 1e-5




def frag_index(M, K):
    """uint16 offset of the hi plane of element (m, k) of an [M][K] frag
    buffer: rows in 64-row blocks, K-steps of 32, 16-row groups of 1024
    entries (hi plane then lo plane), lane 16*(k%32//8) + m%16, 8 entries per
    lane."""
    m = np.arange(M)[:, None]
    k = np.arange(K)[None, :]
    grp = ((m >> 6) * (K >> 5) + (k >> 5)) * 4 + ((m >> 4) & 3)
    lane = (((k >> 3) & 3) << 4) + (m & 15)
    return (grp << 10) + (lane << 3) + (k & 7)


def frag_elems(M, K):
    return (M + 63) // 64 * 64 * K * 2


def to_frag(hi, lo):
    M, K = hi.shape
    buf = np.zeros(frag_elems(M, K), np.uint16)
    idx = frag_index(M, K)
    buf[idx] = hi
    buf[idx + 512] = lo
    return buf


def from_frag(buf, M, K):
    idx = frag_index(M, K)
    return buf[idx], buf[idx + 512]


def bf16_to_f32(u):
    return (np.asarray(u, np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def split(x):
    hi = f32_to_bf16(x)
    lo = f32_to_bf16(np.asarray(x, np.float32) - bf16_to_f32(hi))
    return hi, lo


@pytest.fixture(scope="module")
def lib(hip):
    L = C.CDLL(cb.HIP_LIB)
    L.ctk_gemv_sizeof.restype = C.c_int
    L.ctk_warmset_sizeof.restype = C.c_int
    # the mirrors must match the C structs before any kernel reads them
    assert C.sizeof(CtGemv) == L.ctk_gemv_sizeof()
    assert C.sizeof(CtWarmSet) == L.ctk_warmset_sizeof()
    L.ctk_gemv_warm.argtypes = [C.POINTER(CtGemv), C.POINTER(CtWarm)]
    L.ctk_ln_frag_warm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                   C.c_void_p, C.c_void_p, C.c_int, C.POINTER(CtWarmSet),
                                   C.c_void_p]
    L.ctk_gemv.argtypes = [C.POINTER(CtGemv), C.c_void_p]
    L.ctk_gemv_ksplit.argtypes = [C.c_int, C.c_int]
    L.ctk_gemv_ksplit.restype = C.c_int
    L.ctk_tile_w.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    L.ctk_ln_frag.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                              C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
    return L


class Dev:
    """Arena-backed device buffers of raw bytes."""

    def __init__(self, hip):
        self.hip = hip
        self.ar = ks.ArenaDev(hip, floats=1 << 25)
        self.ev = cb.HipEvents()

    def put(self, a):
        a = np.ascontiguousarray(a)
        f = a.view(np.uint8)
        pad = (-f.size) % 4
        f = np.concatenate([f, np.zeros(pad, np.uint8)]) if pad else f
        return self.ar.put(f.view(np.float32))[0]

    def zeros(self, nbytes):
        return self.put(np.zeros(nbytes, np.uint8))

    def get(self, p, dtype, n):
        self.ev.sync()
        nb = np.dtype(dtype).itemsize * n
        out = np.empty((nb + 3) // 4, np.float32)
        self.hip.backend_dtoh(out.ctypes.data, p, out.nbytes)   # bytes (backend.h:46)
        return out.view(np.uint8)[:nb].view(dtype).copy()


def run_gemv(lib, dev, A_f32, pw, N, pb, out, relu=0, ksplit=1, wtile=0):
    """pw / pb: device pointers of the bf16 weight [N][K] (tiled if wtile)
    and bias (or None)."""
    M, K = A_f32.shape
    hi, lo = split(A_f32)
    pa = dev.put(to_frag(hi, lo))
    g = CtGemv(A=pa, W=pw, bias=pb, M=M, N=N, K=K, ksplit=ksplit, out=out, relu=relu, wtile=wtile)
    if out == PARTIAL:
        g.Y = dev.zeros(ksplit * M * N * 4)
    elif out == DENSE:
        g.Y = dev.zeros(M * N * 4)
        g.ldy = N
    elif out == FRAG:
        g.F = dev.zeros(frag_elems(M, N) * 2)
    dev.ev.sync()
    lib.ctk_gemv(C.byref(g), None)
    if out == PARTIAL:
        return dev.get(g.Y, np.float32, ksplit * M * N).reshape(ksplit, M, N)
    if out == DENSE:
        return dev.get(g.Y, np.float32, M * N).reshape(M, N)
    buf = dev.get(g.F, np.uint16, frag_elems(M, N))
    h, l = from_frag(buf, M, N)
    return h, l


def exact_ref(A_f32, W_bf, bias_bf):
    hi, lo = split(A_f32)
    x = bf16_to_f32(hi).astype(np.float64) + bf16_to_f32(lo)
    y = x @ bf16_to_f32(W_bf).astype(np.float64).T
    if bias_bf is not None:
        y = y + bf16_to_f32(bias_bf)
    return y


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


SHAPES = [(1024, 1024), (1024, 4096), (4096, 1024), (16384, 1024)]


@pytest.mark.parametrize("N,K", SHAPES)
def test_gemv_matches_float64(lib, hip, N, K):
    dev = Dev(hip)
    rng = np.random.default_rng(N + K)
    W = f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.03)
    b = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1)
    pw, pb = dev.put(W), dev.put(b)
    ksplit = lib.ctk_gemv_ksplit(N, K)
    for M in (1, 5, 64, 70, 130):
        print(f"case: gemv N={N} K={K} M={M} ksplit={ksplit}", flush=True)
        A = rng.standard_normal((M, K)).astype(np.float32)
        ref = exact_ref(A, W, b)
        tol = TOL
        if ksplit > 1:
            parts = run_gemv(lib, dev, A, pw, N, None, PARTIAL, ksplit=ksplit)
            got = parts.astype(np.float64).sum(0) + bf16_to_f32(b)
        elif N >= 8192:
            got = run_gemv(lib, dev, A, pw, N, pb, DENSE)
        else:
            h, l = run_gemv(lib, dev, A, pw, N, pb, FRAG, relu=1)
            ref = np.maximum(ref, 0.0)
            got = bf16_to_f32(h).astype(np.float64) + bf16_to_f32(l)
            tol = 2e-5          # plus the hi/lo split of the output (2^-17)
        e = rel(got, ref)
        print(f"  relerr {e:.2e}")
        assert e <= tol, (M, e)


@pytest.mark.parametrize("N,K,rows", [(1024, 1024, 130), (1024, 4096, 130), (4096, 1024, 130),
                                      (16384, 1024, 130), (3072, 1024, 80), (1024, 4096, 80)])
def test_gemv_rows_independent_of_batch(lib, hip, N, K, rows):
    """Row r of a 130-row launch (64-row blocks) or an 80-row launch (one
    80-row block: a step's slots plus its prompt rows) equals the same row
    launched alone, bit for bit."""
    dev = Dev(hip)
    rng = np.random.default_rng(7)
    W = f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.03)
    b = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1)
    A = rng.standard_normal((rows, K)).astype(np.float32)
    ksplit = lib.ctk_gemv_ksplit(N, K)
    out = PARTIAL if ksplit > 1 else DENSE
    pw = dev.put(W)
    pb = dev.put(b) if out == DENSE else None
    full = run_gemv(lib, dev, A, pw, N, pb, out, ksplit=ksplit)
    for r in (0, 17, 63, 64, rows - 1):
        print(f"case: gemv row {r} of {rows} alone N={N} K={K}", flush=True)
        one = run_gemv(lib, dev, A[r:r + 1], pw, N, pb, out, ksplit=ksplit)
        if out == PARTIAL:
            assert np.array_equal(full[:, r].view(np.uint32), one[:, 0].view(np.uint32))
        else:
            assert np.array_equal(full[r].view(np.uint32), one[0].view(np.uint32))


def test_gemv_qkv_scatter(lib, hip):
    """QKV output: query rows dense, key/value rows into head-major caches at
    rowoff[m] (bf16); rows with rowoff < 0 leave the caches untouched."""
    dev = Dev(hip)
    rng = np.random.default_rng(3)
    M, K, N = 6, 1024, 3072
    smax = 16
    W = f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.03)
    b = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1)
    A = rng.standard_normal((M, K)).astype(np.float32)
    hi, lo = split(A)
    cache_el = M * 8 * smax * 128
    sentinel = np.full(cache_el, 0x3F80, np.uint16)      # 1.0 in bf16
    kc, vc = dev.put(sentinel), dev.put(sentinel)
    pos = np.array([3, -1, 0, 15, -1, 7])
    rowoff = np.where(pos >= 0, (np.arange(M) * 8 * smax + pos) * 128, -1).astype(np.int64)
    g = CtGemv(A=dev.put(to_frag(hi, lo)), W=dev.put(W), bias=dev.put(b), M=M, N=N, K=K, ksplit=1,
               out=QKV, relu=0, Y=dev.zeros(M * 1024 * 4), ldy=1024, kc=kc, vc=vc,
               rowoff=dev.put(rowoff), hstride=smax * 128, kv_bf16=1)
    dev.ev.sync()
    lib.ctk_gemv(C.byref(g), None)
    q = dev.get(g.Y, np.float32, M * 1024).reshape(M, 1024)
    kk = dev.get(kc, np.uint16, cache_el).reshape(M, 8, smax, 128)
    vv = dev.get(vc, np.uint16, cache_el).reshape(M, 8, smax, 128)
    ref = exact_ref(A, W, b)
    assert rel(q, ref[:, :1024]) <= TOL
    for m in range(M):
        for name, cache, lo_c in (("k", kk, 1024), ("v", vv, 2048)):
            if pos[m] < 0:
                assert np.all(cache[m] == 0x3F80), (name, m)
                continue
            got = bf16_to_f32(cache[m, :, pos[m], :]).reshape(1024)
            want = ref[m, lo_c:lo_c + 1024]
            assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6, (name, m)
            others = np.delete(cache[m], pos[m], axis=1)
            assert np.all(others == 0x3F80), (name, m)


def test_ln_frag(lib, hip):
    """h += ((p0 + p1) + ...) + bias in that order, then LayerNorm (two-pass
    mean / variance, eps 1e-5, backends/cpu/backend.c:109-122) split into frag."""
    dev = Dev(hip)
    rng = np.random.default_rng(5)
    D = 1024
    for M, nparts in ((1, 0), (64, 4), (70, 8)):
        print(f"case: ln_frag M={M} nparts={nparts}", flush=True)
        h = rng.standard_normal((M, D)).astype(np.float32)
        parts = rng.standard_normal((max(nparts, 1), M, D)).astype(np.float32)
        pb = f32_to_bf16(rng.standard_normal(D).astype(np.float32) * 0.1)
        w = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
        bb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
        ph = dev.put(h)
        pf = dev.zeros(frag_elems(M, D) * 2)
        pp = dev.put(parts)
        dev.ev.sync()
        lib.ctk_ln_frag(ph, pf, pp, nparts, dev.put(pb), dev.put(w), dev.put(bb), M, None)
        h_new = dev.get(ph, np.float32, M * D).reshape(M, D)
        if nparts:
            acc = parts[0].copy()
            for p in range(1, nparts):
                acc = acc + parts[p]
            want_h = h + (acc + bf16_to_f32(pb))
            assert np.array_equal(h_new.view(np.uint32), want_h.astype(np.float32).view(np.uint32))
        else:
            assert np.array_equal(h_new, h)
        x = h_new.astype(np.float64)
        mu = x.mean(1, keepdims=True)
        var = ((x - mu) ** 2).mean(1, keepdims=True)
        ref = (x - mu) / np.sqrt(var + 1e-5) * bf16_to_f32(w) + bf16_to_f32(bb)
        hi, lo = from_frag(dev.get(pf, np.uint16, frag_elems(M, D)), M, D)
        got = bf16_to_f32(hi).astype(np.float64) + bf16_to_f32(lo)
        assert rel(got, ref) <= 1e-5


def test_ln_frag_read_ahead_leaves_results(lib, hip):
    """Read-ahead workgroups appended to the LayerNorm launch (the tiles of a
    QKV-shaped and an FFN-down-shaped decode GEMM) change nothing it writes:
    h and the frag output are bit-identical to the plain launch, and the GEMM
    that follows on those weights gives the same bits as without."""
    dev = Dev(hip)
    rng = np.random.default_rng(11)
    D, M, nparts = 1024, 80, 4
    h = rng.standard_normal((M, D)).astype(np.float32)
    parts = rng.standard_normal((nparts, M, D)).astype(np.float32)
    pb = f32_to_bf16(rng.standard_normal(D).astype(np.float32) * 0.1)
    w = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    bb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    pp, ppb, pw, pbb = dev.put(parts), dev.put(pb), dev.put(w), dev.put(bb)
    shapes = ((3 * D, D, 1), (D, 4 * D, lib.ctk_gemv_ksplit(D, 4 * D)))
    ws = CtWarmSet()
    tiled = []
    for t, (N, K, ksplit) in enumerate(shapes):
        wt = f32_to_bf16(0.05 * rng.standard_normal((N, K)).astype(np.float32))
        praw, ptile = dev.put(wt), dev.zeros(N * K * 2)
        lib.ctk_tile_w(praw, ptile, N, K, None)
        g = CtGemv(W=ptile, N=N, K=K, ksplit=ksplit, wtile=1)
        lib.ctk_gemv_warm(C.byref(g), C.byref(ws.t[t]))
        assert (ws.t[t].gx * ws.t[t].gy, ws.t[t].per * ws.t[t].gy) == (256 if t else 192, K // 32)
        tiled.append((ptile, N, K))
    ws.n, ws.rows, ws.magic, ws.sink = 2, 32, 0x5BD1E995, dev.zeros(1024)
    outs = []
    for warm in (None, C.byref(ws)):
        print(f"case: ln_frag M={M} read-ahead={warm is not None}", flush=True)
        ph, pf = dev.put(h), dev.zeros(frag_elems(M, D) * 2)
        dev.ev.sync()
        lib.ctk_ln_frag_warm(ph, pf, pp, nparts, ppb, pw, pbb, M, warm, None)
        ptile, N, K = tiled[0]
        py = dev.zeros(M * N * 4)
        g = CtGemv(A=pf, W=ptile, M=M, N=N, K=K, ksplit=1, out=1, Y=py, ldy=N, wtile=1)
        lib.ctk_gemv(C.byref(g), None)
        outs.append((dev.get(ph, np.uint32, M * D), dev.get(pf, np.uint16, frag_elems(M, D)),
                     dev.get(py, np.uint32, M * N)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def wtile_index(N, K):
    """uint16 offset of W[n][k] in the tile layout: one 1024-entry tile per
    (16 rows, K-step of 32), row-block major; lane 16*(k%32//8) + n%16 holds
    8 consecutive k."""
    n = np.arange(N)[:, None]
    k = np.arange(K)[None, :]
    tile = (n >> 4) * (K >> 5) + (k >> 5)
    lane = (((k >> 3) & 3) << 4) + (n & 15)
    return (tile << 9) + (lane << 3) + (k & 7)


@pytest.mark.parametrize("N,K,out", [(1024, 1024, PARTIAL), (3072, 1024, DENSE), (4096, 1024, FRAG),
                                     (1024, 4096, PARTIAL), (16384, 1024, DENSE)])
def test_gemv_tiled_weights(lib, hip, N, K, out):
    """ctk_tile_w writes the tile layout (checked element by element against
    the index formula), and the GEMM on tiled weights gives the same bits as
    on row-major ones."""
    dev = Dev(hip)
    rng = np.random.default_rng(N * 3 + K)
    W = f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.03)
    b = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1)
    pw, pb = dev.put(W), dev.put(b)
    pt = dev.zeros(N * K * 2)
    dev.ev.sync()
    lib.ctk_tile_w(pw, pt, N, K, None)
    tiled = dev.get(pt, np.uint16, N * K)
    want = np.zeros(N * K, np.uint16)
    want[wtile_index(N, K)] = W
    assert np.array_equal(tiled, want)
    ksplit = lib.ctk_gemv_ksplit(N, K) if out == PARTIAL else 1
    for M in (1, 37, 64, 130):
        print(f"case: tiled gemv N={N} K={K} out={out} M={M}", flush=True)
        A = rng.standard_normal((M, K)).astype(np.float32)
        bias = None if out == PARTIAL else pb
        a = run_gemv(lib, dev, A, pw, N, bias, out, relu=int(out == FRAG), ksplit=ksplit)
        t = run_gemv(lib, dev, A, pt, N, bias, out, relu=int(out == FRAG), ksplit=ksplit, wtile=1)
        if out == FRAG:
            assert np.array_equal(a[0], t[0]) and np.array_equal(a[1], t[1]), M
        else:
            assert np.array_equal(a.view(np.uint32), t.view(np.uint32)), M


def test_gemv_residual_stats_and_layernorm_input(lib, hip):
    """The residual projection (out CT_GV_RESID): h += x W^T + b on the
    residual rows, leaving each row's (mean, squared deviations) per 32-column
    block, against float64; then a GEMM whose A is LayerNorm(h) normalised in
    the kernel from those statistics (CtGemv.X), against the float64 LayerNorm
    (backends/cpu/backend.c layernorm, eps 1e-5) and product.  Rows must not
    depend on the launch's row count or on the tile width it takes (M = 8, 24,
    64 and 80 use 16-, 32- and 64-column tiles): bit-exact; rows past M stay
    untouched."""
    rng = np.random.default_rng(11)
    dev = Dev(hip)
    D, M, N2 = 1024, 80, 4096
    h0 = (2.0 + rng.standard_normal((M, D))).astype(np.float32)      # rows with a nonzero mean
    hi, lo = split(rng.standard_normal((M, D)).astype(np.float32))
    Wo = f32_to_bf16(rng.standard_normal((D, D)).astype(np.float32) / 32)
    bo = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    lnw = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    lnb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    W2 = f32_to_bf16(rng.standard_normal((N2, D)).astype(np.float32) / 32)
    b2 = f32_to_bf16(0.1 * rng.standard_normal(N2).astype(np.float32))

    def tiled(W):
        N, K = W.shape
        praw, pt = dev.put(W), dev.zeros(N * K * 2)
        lib.ctk_tile_w(praw, pt, N, K, None)
        return pt

    pWo, pW2 = tiled(Wo), tiled(W2)
    pa, pbo = dev.put(to_frag(hi, lo)), dev.put(bo)
    plnw, plnb, pb2 = dev.put(lnw), dev.put(lnb), dev.put(b2)
    res = {}
    for m in (80, 64, 24, 8):
        print(f"case: residual projection + LayerNorm-input GEMM, M={m}", flush=True)
        ph, pst, py = dev.put(h0), dev.zeros(M * 32 * 8), dev.zeros(M * N2 * 4)
        dev.ev.sync()
        g = CtGemv(A=pa, W=pWo, bias=pbo, M=m, N=D, K=D, ksplit=1, out=4, Y=ph, ldy=D, wtile=1,
                   lnstat=pst)
        lib.ctk_gemv(C.byref(g), None)
        g2 = CtGemv(X=ph, ldx=D, lnstat=pst, lnw=plnw, lnb=plnb, W=pW2, bias=pb2, M=m, N=N2, K=D,
                    ksplit=1, out=DENSE, Y=py, ldy=N2, wtile=1)
        lib.ctk_gemv(C.byref(g2), None)
        res[m] = (dev.get(ph, np.float32, M * D).reshape(M, D),
                  dev.get(pst, np.float32, M * 64).reshape(M, 32, 2),
                  dev.get(py, np.float32, M * N2).reshape(M, N2))
    h, st, y = res[M]
    x64 = bf16_to_f32(hi).astype(np.float64) + bf16_to_f32(lo)
    href = h0 + x64 @ bf16_to_f32(Wo).astype(np.float64).T + bf16_to_f32(bo)
    e = np.abs(h - href).max() / np.abs(href).max()
    print(f"  residual relerr {e:.2e}")
    assert e <= TOL
    blk = h.astype(np.float64).reshape(M, 32, 32)
    mean = blk.mean(2)
    m2 = ((blk - mean[:, :, None]) ** 2).sum(2)
    assert np.abs(st[:, :, 0] - mean).max() <= 1e-6 * np.abs(mean).max()
    assert np.all(np.abs(st[:, :, 1] - m2) <= 1e-5 * m2 + 1e-6 * m2.max())
    hd = h.astype(np.float64)
    mu = hd.mean(1, keepdims=True)
    var = ((hd - mu) ** 2).mean(1, keepdims=True)
    ln = (hd - mu) / np.sqrt(var + 1e-5) * bf16_to_f32(lnw) + bf16_to_f32(lnb)
    yref = ln @ bf16_to_f32(W2).astype(np.float64).T + bf16_to_f32(b2)
    e = np.abs(y - yref).max() / np.abs(yref).max()
    print(f"  LayerNorm-input GEMM relerr {e:.2e}")
    assert e <= TOL
    for m in (64, 24, 8):
        hm, sm, ym = res[m]
        assert np.array_equal(hm[:m].view(np.uint32), h[:m].view(np.uint32)), m
        assert np.array_equal(sm[:m].view(np.uint32), st[:m].view(np.uint32)), m
        assert np.array_equal(ym[:m].view(np.uint32), y[:m].view(np.uint32)), m
        assert np.array_equal(hm[m:].view(np.uint32), h0[m:].view(np.uint32)), m
        assert not sm[m:].any() and not ym[m:].any(), m
