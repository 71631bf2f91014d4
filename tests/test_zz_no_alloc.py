"""The allocation-free entry point — needs an MI355X.

backend_rel_pos_mhsa_noalloc runs the same kernels as backend_rel_pos_mhsa
with its scratch in a static device array instead of the caller's workspace.
Two calls in a row through the C ABI, the second with a shorter clip (the
array keeps the first call's contents), each compared bit for bit with the
workspace entry point on the same input, and with the oracle at 1e-4.
"""
import numpy as np
import pytest

import ctbind as cb
import kernel_suite as ks
import oracle_bind as ob

pytestmark = pytest.mark.gpu


def test_rel_pos_mhsa_noalloc_matches_workspace_entry(hip, kernel_model):
    hip.backend_weights_upload_blob(kernel_model.data_ptr, kernel_model.data_bytes)
    dev = ks.ArenaDev(hip)
    D, TM = cb.ENC_D, 376
    pe_max = dev.zeros(2 * TM - 1, D)
    hip.backend_make_rel_pos_emb(pe_max[0], TM)
    o = ob.oracle()
    for T, layer in ((376, 3), (37, 11)):
        rng = np.random.default_rng(T)
        x0 = rng.standard_normal((T, D)).astype(np.float32)
        pe = pe_max[0] + (TM - T) * D * 4          # the batch form's shifted table
        work = dev.zeros((5 * T - 1) * D + max(T * (3 * T - 1), 2 * T * D))
        xa = dev.put(x0)
        hip.backend_rel_pos_mhsa(xa[0], pe, T, kernel_model.elayer_ptr(layer), work[0])
        xb = dev.put(x0)
        print(f"case: rel_pos_mhsa_noalloc T={T} layer {layer}", flush=True)
        hip.backend_rel_pos_mhsa_noalloc(xb[0], pe, T, kernel_model.elayer_ptr(layer))
        a, b = dev.get(xa), dev.get(xb)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), T
        pe_ref = np.zeros((2 * T - 1, D), np.float32)
        o.orc_make_rel_pos_emb(pe_ref.ctypes.data, T)
        want = x0.copy()
        o.orc_rel_pos_mhsa(want.ctypes.data, pe_ref.ctypes.data, T, kernel_model.elayer_ptr(layer), None)
        err = float(np.abs(b.astype(np.float64) - want).max() / np.abs(want).max())
        print(f"  bit-equal to the workspace entry point; vs oracle {err:.2e}", flush=True)
        assert err <= 1e-4
