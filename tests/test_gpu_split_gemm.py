"""GPU checks of the encoder's pre-split GEMM kernels (ctk_gemm with Ahi set:
the 256-row hi + lo and single-pass kernels and the 128-row kernel) through
every output mode the encoder and the cross K/V projection use, called
through libct_hip.so's C entry point.

* The 128-row and 256-row tiles run the same per-element MFMA sequence, so
  forcing either (ctk_gemm_force_tile) gives the same bits.
* hi + lo: the activation is x = hi + lo exactly, and the fp32-activation
  kernel (A set instead of Ahi) splits x in registers the same way, so it
  gives the same bits too; against float64 the sums agree to 1e-5.
* Single-pass (no lo plane): the activation is the bf16 hi alone; against the
  float64 product of those values the fp32 sums agree to 1e-5, and an output
  rounded to bf16 lies within one bf16 step of the float64 value.
* A row's bits do not depend on how many rows the launch has.
* GLU (the conv module's first pointwise projection): value column j times
  the sigmoid of gate column j + N/2, both with their bias.

Semantics per output: backends/cpu/backend.c:124-182, 309 (y = x W^T + b, SiLU, GLU,
ReLU, fmadd), with the encoder's output layouts (split planes, three dense
segments, head-major cache rows with skipped rows).
"""
import ctypes as C

import numpy as np
import pytest

import ctbind as cb
from structs import CtGemm, CtSeg
from test_gpu_gemv import Dev, bf16_to_f32, f32_to_bf16, split

pytestmark = pytest.mark.gpu

EPI_STORE, EPI_SILU, EPI_RELU, EPI_FMADD, EPI_GLU = 0, 1, 2, 3, 4
OUT_DENSE, OUT_HEADS_BF16, OUT_SPLIT = 0, 2, 3
M_FULL, M_PART = 1100, 300          # 4 full 256-row tiles and a partial one; a prefix of it
KV_HSTRIDE = 64 * 128                # head stride of the head-major cache rows


@pytest.fixture(scope="module")
def lib(hip):
    L = C.CDLL(cb.HIP_LIB)
    L.ctk_gemm_sizeof.restype = C.c_int
    assert C.sizeof(CtGemm) == L.ctk_gemm_sizeof()
    L.ctk_gemm.argtypes = [C.POINTER(CtGemm), C.c_void_p]
    L.ctk_gemm_force_tile.argtypes = [C.c_int]
    yield L
    L.ctk_gemm_force_tile(0)


def kv_rowoff(M):
    """Cache row offsets of a head-major layout; every 7th row skipped (-1)."""
    m = np.arange(M)
    ro = ((m // 64) * 8 * 64 + m % 64) * 128
    return np.where(m % 7 == 3, -1, ro).astype(np.int64)


class Case:
    """One GEMM launch: operands on the device and the output buffers it writes."""

    def __init__(self, dev, mode, N, K, lo, seed):
        self.dev, self.mode, self.N, self.K, self.lo = dev, mode, N, K, lo
        rng = np.random.default_rng(seed)
        self.x = rng.standard_normal((M_FULL, K)).astype(np.float32)
        self.hi, self.lo_bits = split(self.x)
        W = f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * (2.0 / np.sqrt(K)))
        b = f32_to_bf16(rng.standard_normal(N).astype(np.float32) * 0.1)
        self.W, self.b = W, b
        self.pA, self.pAh, self.pAl = dev.put(self.x), dev.put(self.hi), dev.put(self.lo_bits)
        self.pW, self.pb = dev.put(W), dev.put(b)
        self.y0 = rng.standard_normal((M_FULL, N)).astype(np.float32)   # FMADD input
        self.ro = kv_rowoff(M_FULL)
        self.pro = dev.put(self.ro)
        if mode == "heads":
            self.kv_elems = int(((M_FULL // 64 + 1) * 8 * 64) * 128 + 8 * KV_HSTRIDE)
            self.pout = [dev.zeros(self.kv_elems * 2), dev.zeros(self.kv_elems * 2)]
        elif mode == "split":
            self.pout = [dev.zeros(M_FULL * N * 2), dev.zeros(M_FULL * N * 2)]
        elif mode == "glu":
            self.pout = [dev.zeros(M_FULL * (N // 2) * 4)]
        else:
            self.pout = [dev.zeros(M_FULL * N * 4)]

    def gemm(self, M, fp32_a=False):
        g = CtGemm(lda=self.K, W=self.pW, bias=self.pb, M=M, N=self.N, K=self.K, scale=0.5)
        if fp32_a:
            g.A = self.pA
        else:
            g.Ahi = self.pAh
            g.Alo = self.pAl if self.lo else None
        if self.mode == "split":
            g.epi, g.nseg, g.seg_w = EPI_SILU, 1, self.N
            g.seg[0] = CtSeg(mode=OUT_SPLIT, base=self.pout[0], ld=self.N,
                             base_lo=self.pout[1] if self.lo else None)
        elif self.mode == "qkv":
            w = self.N // 3
            g.epi, g.nseg, g.seg_w = EPI_STORE, 3, w
            for i in range(3):
                g.seg[i] = CtSeg(mode=OUT_DENSE, base=self.pout[0] + i * M_FULL * w * 4, ld=w)
        elif self.mode == "heads":
            w = self.N // 2
            g.epi, g.nseg, g.seg_w = EPI_STORE, 2, w
            for i in range(2):
                g.seg[i] = CtSeg(mode=OUT_HEADS_BF16, base=self.pout[i], rowoff=self.pro,
                                 hstride=KV_HSTRIDE)
        elif self.mode == "fmadd":
            g.epi, g.Y, g.ldy = EPI_FMADD, self.pout[0], self.N
        elif self.mode == "glu":
            g.epi, g.glu_half, g.Y, g.ldy = EPI_GLU, self.N // 2, self.pout[0], self.N // 2
        else:
            g.epi, g.Y, g.ldy = EPI_RELU, self.pout[0], self.N
        return g

    def run(self, lib, M, tile=0, fp32_a=False):
        """Clears (or, for FMADD, re-seeds) the outputs, launches, returns the output bytes."""
        d = self.dev
        for p in self.pout:
            nb = (self.kv_elems * 2 if self.mode == "heads" else M_FULL * self.N * 2 if self.mode in ("split", "glu")
                  else M_FULL * self.N * 4)
            # the host array must outlive the copy (a temporary's buffer is freed at once)
            src = self.y0 if self.mode == "fmadd" else np.full(nb // 4, -7.0, np.float32)
            d.hip.backend_htod(p, src.ctypes.data, src.size)
            del src
        lib.ctk_gemm_force_tile(tile)
        g = self.gemm(M, fp32_a)
        d.ev.sync()
        lib.ctk_gemm(C.byref(g), None)
        outs = []
        for p in self.pout:
            if self.mode == "heads":
                outs.append(d.get(p, np.uint16, self.kv_elems))
            elif self.mode == "split":
                outs.append(d.get(p, np.uint16, M_FULL * self.N).reshape(M_FULL, self.N))
            elif self.mode == "glu":
                outs.append(d.get(p, np.float32, M_FULL * self.N // 2).reshape(M_FULL, self.N // 2))
            elif self.mode == "qkv":
                # three [M][N/3] segments back to back -> the logical [M][N] rows
                w = self.N // 3
                y = d.get(p, np.float32, M_FULL * self.N).reshape(3, M_FULL, w)
                outs.append(np.concatenate(list(y), 1))
            else:
                outs.append(d.get(p, np.float32, M_FULL * self.N).reshape(M_FULL, self.N))
        return outs

    def ref_sums(self, rows):
        a = bf16_to_f32(self.hi[rows]).astype(np.float64)
        if self.lo:
            a = a + bf16_to_f32(self.lo_bits[rows])
        return a @ bf16_to_f32(self.W).astype(np.float64).T + bf16_to_f32(self.b)


MODES = [("split", 5120, 1280), ("qkv", 3840, 1280), ("heads", 2048, 1024), ("fmadd", 1280, 2560),
         ("relu", 1000, 1312), ("glu", 2560, 1280)]


@pytest.mark.parametrize("lo", [True, False], ids=["hilo", "single"])
@pytest.mark.parametrize("mode,N,K", MODES, ids=[m[0] for m in MODES])
def test_split_gemm_tiles_modes_and_float64(lib, hip, mode, N, K, lo):
    dev = Dev(hip)
    case = Case(dev, mode, N, K, lo, seed=N + K + lo)
    print(f"case: split GEMM {mode} M={M_FULL} N={N} K={K} {'hi+lo' if lo else 'single-pass'}", flush=True)
    o128 = case.run(lib, M_FULL, tile=128)
    o256 = case.run(lib, M_FULL, tile=256)
    for a, b in zip(o128, o256):
        assert np.array_equal(a, b), "128- and 256-row tiles differ"
    if lo and K != 1024:
        # (K == 1024 routes fp32 activations to the decoder-shaped kernel, which
        # splits K over waves: a different summation order)
        of = case.run(lib, M_FULL, fp32_a=True)
        for a, b in zip(o256, of):
            assert np.array_equal(a, b), "pre-split and fp32-activation kernels differ"
    # prefix rows launched alone: the same bits (both tiles)
    for tile in (128, 256):
        op = case.run(lib, M_PART, tile=tile)
        for a, b in zip(o256, op):
            if mode == "heads":
                rows_ok = case.ro[:M_PART] >= 0
                for hh in range(8):
                    for m in np.nonzero(rows_ok)[0][:40]:
                        o = case.ro[m] + hh * KV_HSTRIDE
                        assert np.array_equal(a[o:o + 128], b[o:o + 128])
            else:
                assert np.array_equal(a[:M_PART], b[:M_PART]), f"rows depend on M (tile {tile})"
                # rows >= M untouched
                rest = b[M_PART:]
                if mode == "fmadd":
                    assert np.array_equal(rest, case.y0[M_PART:])
                else:
                    assert np.all(np.ascontiguousarray(rest).view(np.float32) == -7.0)
    # float64 on a sample of rows, the partial tile's rows among them
    rng = np.random.default_rng(K)
    rows = np.unique(np.concatenate([rng.choice(M_FULL, 48, replace=False), np.arange(M_FULL - 20, M_FULL)]))
    s = case.ref_sums(rows)
    scale = np.abs(s).max()
    if mode == "split":
        v = s / (1.0 + np.exp(-s))
        hi = bf16_to_f32(o256[0][rows]).astype(np.float64)
        if lo:
            got = hi + bf16_to_f32(o256[1][rows])
            e = np.abs(got - v).max() / np.abs(v).max()
            print(f"  relerr {e:.2e}")
            assert e <= 2e-5
        else:
            # one bf16 step (2^-8 relative) plus the fp32 sums' own error
            assert np.all(np.abs(hi - v) <= np.abs(v) * 2.0 ** -8 + 1e-5 * scale)
            assert np.all(o256[1].view(np.float32) == -7.0)   # lo plane untouched
    elif mode == "qkv":
        e = np.abs(o256[0][rows] - s).max() / scale
        print(f"  relerr {e:.2e}")
        assert e <= 1e-5
    elif mode == "heads":
        w = N // 2
        for seg in range(2):
            for j, m in enumerate(rows):
                if case.ro[m] < 0:
                    continue
                for hh in range(w // 128):
                    o = case.ro[m] + hh * KV_HSTRIDE
                    got = bf16_to_f32(o256[seg][o:o + 128]).astype(np.float64)
                    ref = s[j, seg * w + hh * 128:seg * w + (hh + 1) * 128]
                    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-5 * scale)
        # skipped rows' cache entries untouched (still the fill pattern)
        m = np.nonzero(case.ro < 0)[0][0]
        o = ((m // 64) * 8 * 64 + m % 64) * 128
        fill = np.tile(np.full(1, -7.0, np.float32).view(np.uint16), 64)
        for seg in range(2):
            for hh in range(8):
                assert np.array_equal(o256[seg][o + hh * KV_HSTRIDE:o + hh * KV_HSTRIDE + 128], fill)
    elif mode == "glu":
        h = N // 2
        v = s[:, :h] / (1.0 + np.exp(-s[:, h:]))
        e = np.abs(o256[0][rows].astype(np.float64) - v).max() / np.abs(v).max()
        print(f"  relerr {e:.2e}")
        assert e <= 2e-5
    elif mode == "fmadd":
        got = o256[0][rows].astype(np.float64)
        ref = case.y0[rows].astype(np.float64) + 0.5 * s
        e = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"  relerr {e:.2e}")
        assert e <= 1e-5
    else:
        got = o256[0][rows].astype(np.float64)
        e = np.abs(got - np.maximum(s, 0.0)).max() / scale
        print(f"  relerr {e:.2e}")
        assert e <= 1e-5
