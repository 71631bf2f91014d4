"""GPU check of the encoder's fused LayerNorm pair (ctk_layernorm_pair_split),
called through libct_hip.so's C entry point: one layer's output norm
x = LN1(x), in place, and the next layer's first FFN norm LN2(x), written as
hi/lo bf16 planes, in one launch.

* It gives the bits of the two launches it replaces (ctk_layernorm, then
  ctk_layernorm_split on the updated rows), at both model widths, with and
  without the lo plane (the single-pass FFN writes none, and the plane's
  memory stays untouched).
* Against float64 (backends/cpu/backend.c:109-122, applied twice): LN1's
  rows within 1e-5, and hi + lo of LN2 within 1e-5 of the float64 norm of
  LN1's fp32 rows; the hi plane alone is LN2 rounded to bf16 (within one
  bf16 step).
"""
import ctypes as C

import numpy as np
import pytest

import ctbind as cb
from test_gpu_gemv import Dev, bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

T = 37   # rows: 9 full workgroups of 4 and a partial one


@pytest.fixture(scope="module")
def lib(hip):
    L = C.CDLL(cb.HIP_LIB)
    P = C.c_void_p
    L.ctk_layernorm.argtypes = [P, P, P, P, C.c_int, C.c_int, P]
    L.ctk_layernorm_split.argtypes = [P, P, P, P, P, C.c_int, C.c_int, P]
    L.ctk_layernorm_pair_split.argtypes = [P, P, P, P, P, P, P, C.c_int, C.c_int, P]
    return L


def ln64(x, w, b):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * w + b


@pytest.mark.parametrize("D", [1024, 1280])
@pytest.mark.parametrize("with_lo", [True, False])
def test_layernorm_pair_matches_two_launches(lib, hip, D, with_lo):
    rng = np.random.default_rng(D + 7 * with_lo)
    # rows with their own offsets and spreads
    x = (rng.standard_normal((T, D)) * rng.uniform(0.5, 4.0, (T, 1)) + rng.standard_normal((T, 1)) * 2)
    x = x.astype(np.float32)
    w1, w2 = (f32_to_bf16(1.0 + 0.3 * rng.standard_normal(D)) for _ in range(2))
    b1, b2 = (f32_to_bf16(0.2 * rng.standard_normal(D)) for _ in range(2))
    dev = Dev(hip, floats=1 << 20)
    pw1, pb1, pw2, pb2 = (dev.put(a) for a in (w1, b1, w2, b2))
    xa, xb = dev.put(x), dev.put(x)
    ha, la, hb, lb = (dev.zeros(T * D * 2) for _ in range(4))
    print(f"case: D={D} lo={with_lo} rows={T}", flush=True)
    lib.ctk_layernorm(xa, xa, pw1, pb1, T, D, None)
    lib.ctk_layernorm_split(ha, la if with_lo else None, xa, pw2, pb2, T, D, None)
    lib.ctk_layernorm_pair_split(xb, hb, lb if with_lo else None, pw1, pb1, pw2, pb2, T, D, None)
    ya, yb = dev.get(xa, np.float32, T * D), dev.get(xb, np.float32, T * D)
    got_h = {k: dev.get(p, np.uint16, T * D) for k, p in (("ha", ha), ("la", la), ("hb", hb), ("lb", lb))}
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
    assert np.array_equal(got_h["ha"], got_h["hb"])
    assert np.array_equal(got_h["la"], got_h["lb"])
    if not with_lo:
        assert not got_h["lb"].any()
    # against float64
    y = yb.reshape(T, D)
    want1 = ln64(x, bf16_to_f32(w1), bf16_to_f32(b1))
    assert np.abs(y - want1).max() <= 1e-5 * np.abs(want1).max()
    want2 = ln64(y, bf16_to_f32(w2), bf16_to_f32(b2))
    hi = bf16_to_f32(got_h["hb"]).reshape(T, D).astype(np.float64)
    if with_lo:
        z = hi + bf16_to_f32(got_h["lb"]).reshape(T, D)
        assert np.abs(z - want2).max() <= 1e-5 * np.abs(want2).max()
    # RNE to bf16 is within half a step (2^-8 relative) of the fp32 value, itself within 1e-5
    assert np.all(np.abs(hi - want2) <= np.abs(want2) * 2.0 ** -8 * 1.001 + 1e-5 * np.abs(want2).max())
