"""GPU checks of the decode step's GEMM (ctk_gemv), its folded LayerNorms
(residual projections leaving frag(h * w) and block statistics, GEMMs that
correct each row in the epilogue) and the step's embedding launch, called
through libct_hip.so's C entry points.

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

PARTIAL, DENSE, FRAG, QKV, RESID = 0, 1, 2, 3, 4
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
    L.ctk_embed_fold.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                 C.POINTER(CtWarmSet), C.c_void_p]
    L.ctk_resid_fold.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_int, C.POINTER(CtWarmSet), C.c_void_p]
    L.ctk_fold_cols.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                C.c_void_p, C.c_void_p, C.c_void_p]
    L.ctk_gemv.argtypes = [C.POINTER(CtGemv), C.c_void_p]
    L.ctk_gemv_ksplit.argtypes = [C.c_int, C.c_int]
    L.ctk_gemv_ksplit.restype = C.c_int
    L.ctk_tile_w.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    return L


class Dev:
    """Arena-backed device buffers of raw bytes."""

    def __init__(self, hip, floats=1 << 25):
        self.hip = hip
        self.ar = ks.ArenaDev(hip, floats=floats)
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


def tiled(lib, dev, W):
    N, K = W.shape
    praw, pt = dev.put(W), dev.zeros(N * K * 2)
    lib.ctk_tile_w(praw, pt, N, K, None)
    return pt


def ln64(h, w, b):
    """The reference LayerNorm (backends/cpu/backend.c:109-122: two-pass
    mean and variance, eps 1e-5) in float64."""
    x = np.asarray(h, np.float64)
    mu = x.mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * bf16_to_f32(w) + bf16_to_f32(b)


def block_stats64(h):
    x = np.asarray(h, np.float64).reshape(h.shape[0], 32, 32)
    mean = x.mean(2)
    return mean, ((x - mean[..., None]) ** 2).sum(2)


def check_fold_input(dev, h, pst, pf, w, rows, what):
    """lnstat holds each row's (mean, squared deviations) per 32-column block
    of h (float64, 1e-5), and the frag buffer frag(h * w): the fp32 product,
    split hi/lo, bit for bit."""
    M, D = h.shape
    st = dev.get(pst, np.float32, M * 64).reshape(M, 32, 2)[:rows]
    mean, m2 = block_stats64(h[:rows])
    assert np.abs(st[..., 0] - mean).max() <= 1e-5 * max(np.abs(mean).max(), 1.0), what
    assert np.abs(st[..., 1] - m2).max() <= 1e-5 * m2.max(), what
    hi, lo = from_frag(dev.get(pf, np.uint16, frag_elems(M, D)), M, D)
    x = h[:rows] * bf16_to_f32(w)
    whi, wlo = split(x)
    bad = np.argwhere((hi[:rows] != whi) | (lo[:rows] != wlo))
    for m, k in bad[:6]:
        print(f"  {what}: row {m} col {k}: x {x[m, k]!r} got hi/lo {hi[m, k]:#06x}/{lo[m, k]:#06x} "
              f"want {whi[m, k]:#06x}/{wlo[m, k]:#06x}")
    assert len(bad) == 0, (what, len(bad))


def test_folded_layernorm_gemms(lib, hip):
    """The decode step's LayerNorms run inside GEMMs.  A residual projection
    (out CT_GV_RESID, the attention outputs' projections, K = 1024):
    h += x W^T + b on the residual rows against float64, leaving each row's
    block statistics and frag(h * w) of the next LayerNorm's gain.  Then the
    GEMMs with that LayerNorm folded in (fold_c1 / fold_c2 from ctk_fold_cols,
    checked against float64 sums): the cross-query and QKV shapes (dense)
    and FFN up (frag, ReLU) against the float64
    LayerNorm of h (backends/cpu/backend.c layernorm) times W plus bias,
    within 2e-5 of the largest output: the rows here have mean 2 and unit
    spread, so the subtraction of mu * c1 doubles the split's 2^-18 relative
    error.  Every row's bits are independent of the launch's row count
    (M = 80, 64, 24, 8: 16-, 32- and 64-column tiles); rows past M stay
    untouched."""
    rng = np.random.default_rng(11)
    dev = Dev(hip, floats=1 << 27)
    D, M = 1024, 80
    h0 = (2.0 + rng.standard_normal((M, D))).astype(np.float32)      # rows with a nonzero mean
    lnw = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    lnb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    plnw, plnb = dev.put(lnw), dev.put(lnb)
    for K in (1024,):
        hi, lo = split(rng.standard_normal((M, K)).astype(np.float32))
        Wo = f32_to_bf16(rng.standard_normal((D, K)).astype(np.float32) / np.sqrt(K))
        bo = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
        pWo, pa, pbo = tiled(lib, dev, Wo), dev.put(to_frag(hi, lo)), dev.put(bo)
        res = {}
        for m in (80, 64, 24, 8):
            print(f"case: residual projection K={K} M={m} with the folded next input", flush=True)
            ph, pst, pf = dev.put(h0), dev.zeros(M * 32 * 8), dev.zeros(frag_elems(M, D) * 2)
            dev.ev.sync()
            g = CtGemv(A=pa, W=pWo, bias=pbo, M=m, N=D, K=K, ksplit=1, out=RESID, Y=ph, ldy=D, wtile=1,
                       lnstat=pst, F=pf, fold_w=plnw)
            lib.ctk_gemv(C.byref(g), None)
            res[m] = (dev.get(ph, np.uint32, M * D).reshape(M, D),
                      dev.get(pst, np.uint32, M * 64).reshape(M, 64),
                      dev.get(pf, np.uint16, frag_elems(M, D)), (ph, pst, pf))
            if m == M:
                h = res[m][0].view(np.float32)
                x64 = bf16_to_f32(hi).astype(np.float64) + bf16_to_f32(lo)
                href = h0 + x64 @ bf16_to_f32(Wo).astype(np.float64).T + bf16_to_f32(bo)
                e = rel(h, href)
                print(f"  residual relerr {e:.2e}")
                assert e <= TOL
                check_fold_input(dev, h, pst, pf, lnw, M, f"resid K={K}")
        hM, sM, fM, ptrs = res[M]
        for m in (64, 24, 8):
            h, st, fr, _ = res[m]
            assert np.array_equal(h[:m], hM[:m]) and np.array_equal(h[m:], h0[m:].view(np.uint32)), (K, m)
            assert np.array_equal(st[:m], sM[:m]) and not st[m:].any(), (K, m)
            fi = frag_index(M, D)
            assert np.array_equal(fr[fi[:m]], fM[fi[:m]]) and np.array_equal(fr[fi[:m] + 512], fM[fi[:m] + 512])
    # the GEMMs consuming the projection's output
    h = hM.view(np.float32)
    ph, pst, pf = ptrs
    ln = ln64(h, lnw, lnb)
    for N, out, relu in ((1024, DENSE, 0), (3072, DENSE, 0), (4096, FRAG, 1)):
        W2 = f32_to_bf16(rng.standard_normal((N, D)).astype(np.float32) / 32)
        b2 = f32_to_bf16(0.1 * rng.standard_normal(N).astype(np.float32))
        praw, pb2 = dev.put(W2), dev.put(b2)
        pc1, pc2 = dev.zeros(N * 4), dev.zeros(N * 4)
        dev.ev.sync()
        lib.ctk_fold_cols(praw, plnw, plnb, pb2, N, D, pc1, pc2, None)
        W64 = bf16_to_f32(W2).astype(np.float64)
        c1 = dev.get(pc1, np.float32, N)
        c2 = dev.get(pc2, np.float32, N)
        assert np.abs(c1 - W64 @ bf16_to_f32(lnw)).max() <= 2 ** -23 * np.abs(c1).max()
        assert np.abs(c2 - (W64 @ bf16_to_f32(lnb) + bf16_to_f32(b2))).max() <= 2 ** -23 * np.abs(c2).max()
        pW2 = tiled(lib, dev, W2)
        ref = ln @ W64.T + bf16_to_f32(b2)
        if relu:
            ref = np.maximum(ref, 0.0)
        outs = {}
        for m in (80, 64, 24, 8):
            print(f"case: folded LayerNorm GEMM N={N} out={out} M={m}", flush=True)
            g = CtGemv(A=pf, W=pW2, M=m, N=N, K=D, ksplit=1, out=out, relu=relu, wtile=1, lnstat=pst,
                       fold_c1=pc1, fold_c2=pc2)
            if out == DENSE:
                g.Y, g.ldy = dev.zeros(M * N * 4), N
            else:
                g.F = dev.zeros(frag_elems(M, N) * 2)
            dev.ev.sync()
            lib.ctk_gemv(C.byref(g), None)
            if out == DENSE:
                y = dev.get(g.Y, np.float32, M * N).reshape(M, N)
                assert not y[m:].any(), (N, m)
                y = y[:m]
            else:
                yh, yl = from_frag(dev.get(g.F, np.uint16, frag_elems(M, N)), M, N)
                y = (bf16_to_f32(yh).astype(np.float64) + bf16_to_f32(yl))[:m]
            outs[m] = y
            e = rel(y, ref[:m])
            print(f"  relerr {e:.2e}")
            assert e <= 2e-5, (N, m, e)
        m0 = max(outs)
        for m, y in outs.items():
            assert np.array_equal(np.asarray(y).view(np.uint64 if y.dtype == np.float64 else np.uint32),
                                  np.asarray(outs[m0][:m]).view(np.uint64 if y.dtype == np.float64 else np.uint32)), (N, m)


def test_embed_fold_and_read_ahead(lib, hip):
    """The step's embedding launch: h = LN_e(etw[token] + epw[pos - 1]) for
    active rows (float64, 1e-5; inactive rows keep their h), then each row's
    block statistics and frag(h * w) for the first layer's folded LayerNorm.
    Read-ahead workgroups appended to it (the tiles of a QKV-shaped and an
    FFN-down-shaped decode GEMM) change nothing it writes, bit for bit, nor
    the bits of the GEMM that follows on those weights."""
    dev = Dev(hip)
    rng = np.random.default_rng(12)
    D, M, V, P = 1024, 80, 40, 30
    etw = f32_to_bf16(rng.standard_normal((V, D)).astype(np.float32))
    epw = f32_to_bf16(0.5 * rng.standard_normal((P, D)).astype(np.float32))
    elnw = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    elnb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    w = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    tok = rng.integers(0, V, M).astype(np.int32)
    pos = rng.integers(1, P + 1, M).astype(np.int32)
    act = (rng.random(M) < 0.8).astype(np.int32)
    h0 = rng.standard_normal((M, D)).astype(np.float32)
    ptr = [dev.put(a) for a in (tok, pos, act, etw, epw, elnw, elnb, w)]
    shapes = ((3 * D, D, QKV), (D, 4 * D, RESID))
    ws = CtWarmSet()
    tiles = []
    for t, (N, K, out) in enumerate(shapes):
        wt = f32_to_bf16(0.05 * rng.standard_normal((N, K)).astype(np.float32))
        ptile = tiled(lib, dev, wt)
        g = CtGemv(W=ptile, N=N, K=K, M=M, ksplit=1, out=out, wtile=1)
        lib.ctk_gemv_warm(C.byref(g), C.byref(ws.t[t]))
        tiles.append((ptile, N, K))
    ws.n, ws.rows, ws.magic, ws.sink = 2, 32, 0x5BD1E995, dev.zeros(1024)
    outs = []
    for warm in (None, C.byref(ws)):
        print(f"case: embedding fold M={M} read-ahead={warm is not None}", flush=True)
        ph, pst, pf = dev.put(h0), dev.zeros(M * 32 * 8), dev.zeros(frag_elems(M, D) * 2)
        dev.ev.sync()
        lib.ctk_embed_fold(ph, pst, pf, *ptr, M, warm, None)
        ptile, N, K = tiles[1]
        py = dev.zeros(M * 4 * D * 4)
        g = CtGemv(A=pf, W=tiles[0][0], M=M, N=D, K=D, ksplit=1, out=DENSE, Y=py, ldy=D, wtile=1)
        lib.ctk_gemv(C.byref(g), None)
        outs.append((dev.get(ph, np.uint32, M * D), dev.get(pst, np.uint32, M * 64),
                     dev.get(pf, np.uint16, frag_elems(M, D)), dev.get(py, np.uint32, M * D)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    h = outs[0][0].view(np.float32).reshape(M, D)
    e = bf16_to_f32(etw)[tok].astype(np.float64) + bf16_to_f32(epw)[pos - 1]
    want = ln64(e, elnw, elnb)
    on = act != 0
    assert rel(h[on], want[on]) <= 1e-5
    assert np.array_equal(h[~on], h0[~on])
    check_fold_input(dev, h, pst, pf, w, M, "embedding")


def test_resid_fold_after_k_split(lib, hip):
    """The residual update after the K-split FFN down projection:
    h += ((p0 + p1) + ... + p7) + bias, the slices in order then the bias,
    bit for bit against the same fp32 sums, then the next LayerNorm's folded
    input (block statistics, frag(h * w)); rows independent of M."""
    dev = Dev(hip)
    rng = np.random.default_rng(13)
    D, M, NP = 1024, 80, 8
    h0 = (1.5 + rng.standard_normal((M, D))).astype(np.float32)
    parts = (0.3 * rng.standard_normal((NP, M, D))).astype(np.float32)
    pb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    w = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    pp, ppb, pw = dev.put(parts), dev.put(pb), dev.put(w)
    res = {}
    for m in (80, 37):
        print(f"case: residual update after a K split, M={m}", flush=True)
        ph, pst, pf = dev.put(h0), dev.zeros(M * 32 * 8), dev.zeros(frag_elems(M, D) * 2)
        dev.ev.sync()
        pparts = pp if m == M else dev.put(np.ascontiguousarray(parts[:, :m]))
        lib.ctk_resid_fold(ph, pst, pf, pparts, NP, ppb, pw, None, m, None, None)
        res[m] = (dev.get(ph, np.uint32, M * D).reshape(M, D), dev.get(pst, np.uint32, M * 64).reshape(M, 64))
        if m == M:
            acc = parts[0].copy()
            for p in range(1, NP):
                acc = acc + parts[p]
            want = h0 + (acc + bf16_to_f32(pb))
            h = res[m][0].view(np.float32)
            assert np.array_equal(h.view(np.uint32), want.astype(np.float32).view(np.uint32))
            check_fold_input(dev, h, pst, pf, w, M, "resid fold")
    assert np.array_equal(res[37][0][:37], res[M][0][:37]) and np.array_equal(res[37][0][37:], h0[37:].view(np.uint32))
    assert np.array_equal(res[37][1][:37], res[M][1][:37])


def test_resid_fold_final_layernorm(lib, hip):
    """The residual update after the last FFN normalises the rows itself: h +=
    ((p0 + ... + p7) + b2) bit for bit, then frag(LayerNorm(h)) with the final
    gain and bias against the float64 LayerNorm (1e-5), the input of the LM
    head; rows independent of M."""
    dev = Dev(hip)
    rng = np.random.default_rng(19)
    D, M, NP = 1024, 80, 8
    h0 = (2.0 + rng.standard_normal((M, D))).astype(np.float32)
    parts = (0.3 * rng.standard_normal((NP, M, D))).astype(np.float32)
    b2 = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    lnw = f32_to_bf16(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32))
    lnb = f32_to_bf16(0.1 * rng.standard_normal(D).astype(np.float32))
    acc = parts[0].copy()
    for p in range(1, NP):
        acc = acc + parts[p]
    want = (h0 + (acc + bf16_to_f32(b2))).astype(np.float32)
    outs = {}
    for m in (80, 37):
        print(f"case: residual update with the final LayerNorm, M={m}", flush=True)
        ph, pf = dev.put(h0), dev.zeros(frag_elems(M, D) * 2)
        pp = dev.put(np.ascontiguousarray(parts[:, :m]))
        dev.ev.sync()
        lib.ctk_resid_fold(ph, dev.zeros(M * 32 * 8), pf, pp, NP, dev.put(b2), dev.put(lnw), dev.put(lnb), m,
                           None, None)
        h = dev.get(ph, np.float32, M * D).reshape(M, D)
        assert np.array_equal(h[:m].view(np.uint32), want[:m].view(np.uint32))
        assert np.array_equal(h[m:].view(np.uint32), h0[m:].view(np.uint32))
        hi, lo = from_frag(dev.get(pf, np.uint16, frag_elems(M, D)), M, D)
        outs[m] = (hi[:m], lo[:m])
        y = bf16_to_f32(hi[:m]).astype(np.float64) + bf16_to_f32(lo[:m])
        e = rel(y, ln64(want[:m], lnw, lnb))
        print(f"  final LayerNorm relerr {e:.2e}")
        assert e <= 1e-5
    assert np.array_equal(outs[37][0], outs[80][0][:37]) and np.array_equal(outs[37][1], outs[80][1][:37])
