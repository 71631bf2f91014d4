"""Kernel-boundary suite over the backend ABI.

run_suite(abi, dev, model) drives every compute function of the 40-function
ABI on seeded inputs and returns {case: output array}.  The same code runs
against the reference CPU backend (to write golden fixtures, in this
container) and against the HIP backend (GPU parity tests), so both see
identical inputs and call sequences.

Inputs come from numpy's PCG64 with fixed seeds; weights from the synthetic
model (perturbed variant, so biases and gains are non-trivial).
"""
import ctypes as C

import numpy as np

import oracle_bind as ob  # noqa: F401  (puts the package dir on sys.path)
import ctbind as cb

D, DD, FF = cb.ENC_D, cb.DEC_D, cb.DEC_FF


class HostDev:
    """'Device' memory for a CPU backend: plain numpy arrays."""

    def __init__(self):
        self.keep = []

    def put(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32).copy()
        self.keep.append(a)
        return (a.ctypes.data, a.shape)

    def zeros(self, *shape):
        return self.put(np.zeros(shape, np.float32))

    def get(self, h):
        ptr, shape = h
        n = int(np.prod(shape))
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(n,)).reshape(shape).copy()


class ArenaDev:
    """Device memory carved from the backend's own arena (backend_arena_alloc),
    filled with backend_htod and read with backend_dtoh — the way the
    reference host uses the ABI."""

    def __init__(self, abi, floats=1 << 26):
        self.abi = abi
        self.base = abi.backend_arena_alloc(floats)
        if not self.base:
            raise RuntimeError("backend_arena_alloc returned NULL")
        self.cap = floats
        self.off = 0

    def _take(self, n):
        n_al = (n + 63) // 64 * 64
        if self.off + n_al > self.cap:
            raise RuntimeError("suite arena exhausted")
        p = self.base + self.off * 4
        self.off += n_al
        return p

    def put(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        p = self._take(a.size)
        self.abi.backend_htod(p, a.ctypes.data, a.size)
        return (p, a.shape)

    def zeros(self, *shape):
        return self.put(np.zeros(shape, np.float32))

    def get(self, h):
        ptr, shape = h
        out = np.empty(shape, np.float32)
        self.abi.backend_dtoh(out.ctypes.data, ptr, out.nbytes)
        return out


def _ints(vals):
    return np.ascontiguousarray(vals, dtype=np.int32)


def make_inputs(seed=2024):
    r = np.random.default_rng(seed)
    n = lambda *s: r.standard_normal(s).astype(np.float32)  # noqa: E731
    inp = {
        "ln_x": n(5, D), "ln2_x": n(3, DD),
        "lin_x": n(3, D), "linnb_x": n(4, D), "silu_x": n(3, D), "relu_x": n(2, DD),
        "fm_x": n(3, cb.ENC_FF) * 0.5, "fm_acc": n(3, D), "fm2_x": n(2, DD), "fm2_acc": n(2, DD),
        "add_dst": n(1000), "add_src": n(1000),
        "sub_mel": n(cb.N_MELS, 20),
        "mhsa_x": n(5, D), "mhsa8_x": n(5, D), "conv_x": n(6, D),
        "sdp_q": n(4, DD) * 0.3, "sdp_k": n(4, DD) * 0.3, "sdp_v": n(4, DD),
        "sdc_q": n(2, DD) * 0.3, "sdc_k": n(7, DD) * 0.3, "sdc_v": n(7, DD),
        "lm_last": n(DD),
        "dv_cache_k": n(8, DD) * 0.3, "dv_cache_v": n(8, DD), "dv_x": n(DD), "dv_q": n(DD) * 0.3,
        "bt_h": np.full((4, DD), 7.5, np.float32), "bt_x": n(4, DD),
        "bt_cache": n(4, 10, DD) * 0.3, "bt_cache_v": n(4, 10, DD), "bt_q": n(4, DD) * 0.3,
        "bt_ck": n(4, 6, DD) * 0.3, "bt_cv": n(4, 6, DD),
        "bt_lg_init": np.full((4, cb.VOCAB), -3.25, np.float32),
        "am_logits": n(4, cb.VOCAB),
    }
    # argmax edge cases: row 0 max at index 0, row 3 an exact tie (20 and 50).
    inp["am_logits"][0, 0] = 9.0
    inp["am_logits"][3, 20] = 11.0
    inp["am_logits"][3, 50] = 11.0
    return inp


def run_suite(abi, dev, model, inp):
    """Returns {case: np.ndarray} for every compute function of the ABI."""
    A = abi
    out = {}
    p = model.ptr

    # layernorm (out of place, and in place as model.h:741 uses it)
    x = dev.put(inp["ln_x"]); y = dev.zeros(5, D)
    A.backend_layernorm(y[0], x[0], p("enc0.ff1_lnw"), p("enc0.ff1_lnb"), 5, D)
    out["layernorm"] = dev.get(y)
    x = dev.put(inp["ln2_x"])
    A.backend_layernorm(x[0], x[0], p("dec0.sa_lnw"), p("dec0.sa_lnb"), 3, DD)
    out["layernorm_inplace"] = dev.get(x)

    # linear family
    x = dev.put(inp["lin_x"]); y = dev.zeros(3, D)
    A.backend_linear(y[0], x[0], p("enc0.sa_qw"), p("enc0.sa_qb"), 3, D, D)
    out["linear"] = dev.get(y)
    x = dev.put(inp["linnb_x"]); y = dev.zeros(4, D)
    A.backend_linear(y[0], x[0], p("enc0.sa_pw"), None, 4, D, D)
    out["linear_nobias"] = dev.get(y)
    x = dev.put(inp["silu_x"]); y = dev.zeros(3, cb.ENC_FF)
    A.backend_linear_silu(y[0], x[0], p("enc0.ff1_w1"), p("enc0.ff1_b1"), 3, D, cb.ENC_FF)
    out["linear_silu"] = dev.get(y)
    x = dev.put(inp["relu_x"]); y = dev.zeros(2, FF)
    A.backend_linear_relu(y[0], x[0], p("dec0.ffn_w1"), p("dec0.ffn_b1"), 2, DD, FF)
    out["linear_relu"] = dev.get(y)
    x = dev.put(inp["fm_x"]); acc = dev.put(inp["fm_acc"])
    A.backend_linear_fmadd(acc[0], 0.5, x[0], p("enc0.ff1_w2"), p("enc0.ff1_b2"), 3, cb.ENC_FF, D)
    out["linear_fmadd"] = dev.get(acc)
    x = dev.put(inp["fm2_x"]); acc = dev.put(inp["fm2_acc"])
    A.backend_linear_fmadd(acc[0], 1.0, x[0], p("dec0.sa_ow"), None, 2, DD, DD)
    out["linear_fmadd_nobias"] = dev.get(acc)

    d = dev.put(inp["add_dst"]); s = dev.put(inp["add_src"])
    A.backend_add_inplace(d[0], s[0], 1000)
    out["add_inplace"] = dev.get(d)

    # encoder subsampling: T_mel 17 read from a buffer padded to stride 20
    T_mel, stride = 17, 20
    Te = cb.t_enc(T_mel)
    mel = dev.put(inp["sub_mel"]); xe = dev.zeros(Te, D)
    T1 = (T_mel + 1) // 2
    T2 = (T1 + 1) // 2
    work = dev.zeros(cb.SUB_CH * (T1 * 64 + T2 * 32))
    A.backend_encoder_subsampling(mel[0], T_mel, stride, xe[0], Te, work[0], model.weights_ref())
    out["subsampling"] = dev.get(xe)

    # relative positional table (T=5 and the degenerate T=1)
    pe5 = dev.zeros(9, D)
    A.backend_make_rel_pos_emb(pe5[0], 5)
    out["rel_pos_emb5"] = dev.get(pe5)
    pe1 = dev.zeros(1, D)
    A.backend_make_rel_pos_emb(pe1[0], 1)
    out["rel_pos_emb1"] = dev.get(pe1)

    # rel-pos MHSA, T=5: own table, and the batch form (table built for
    # T_max=8, pointer shifted by (8-5) rows, model.h:586-592)
    T = 5
    def mhsa_work(T):
        return dev.zeros((5 * T - 1) * D + max(T * (3 * T - 1), 2 * T * D))
    x = dev.put(inp["mhsa_x"])
    A.backend_rel_pos_mhsa(x[0], pe5[0], T, model.elayer_ptr(0), mhsa_work(T)[0])
    out["rel_pos_mhsa"] = dev.get(x)
    pe8 = dev.zeros(15, D)
    A.backend_make_rel_pos_emb(pe8[0], 8)
    x = dev.put(inp["mhsa8_x"])
    A.backend_rel_pos_mhsa(x[0], pe8[0] + (8 - T) * D * 4, T, model.elayer_ptr(0), mhsa_work(T)[0])
    out["rel_pos_mhsa_shifted"] = dev.get(x)

    # conformer conv module, T=6 (layer 1 weights)
    x = dev.put(inp["conv_x"])
    A.backend_conformer_conv(x[0], 6, model.elayer_ptr(1), dev.zeros(3 * 6 * D)[0])
    out["conformer_conv"] = dev.get(x)

    # sdp attention: causal 4x4 (prefill) and unmasked 2x7 (cross)
    m = dev.zeros(4, 4)
    A.backend_fill_causal_mask(m[0], 4)
    out["causal_mask"] = dev.get(m)
    q, k, v, o = dev.put(inp["sdp_q"]), dev.put(inp["sdp_k"]), dev.put(inp["sdp_v"]), dev.zeros(4, DD)
    A.backend_sdp_attn(o[0], q[0], k[0], v[0], m[0], 4, 4, dev.zeros(16)[0])
    out["sdp_attn_causal"] = dev.get(o)
    q, k, v, o = dev.put(inp["sdc_q"]), dev.put(inp["sdc_k"]), dev.put(inp["sdc_v"]), dev.zeros(2, DD)
    A.backend_sdp_attn(o[0], q[0], k[0], v[0], None, 2, 7, dev.zeros(14)[0])
    out["sdp_attn_cross"] = dev.get(o)

    # embedding (+LN) at positions 2..4; tokens staged first as model.h:466 does
    toks = _ints([5, 100, 16383])
    A.backend_upload_tokens(toks.ctypes.data, 3)
    h = dev.zeros(3, DD)
    A.backend_embed(h[0], toks.ctypes.data, 3, 2, p("etw"), p("epw"), p("elnw"), p("elnb"))
    out["embed"] = dev.get(h)

    last = dev.put(inp["lm_last"]); lg = dev.zeros(cb.VOCAB)
    A.backend_lm_head(lg[0], last[0], p("etw"), p("hdb"))
    out["lm_head"] = dev.get(lg)

    # device-counter path (B = 1): S set to 4, incremented to 5
    A.backend_decode_set_S(4)
    A.backend_decode_inc_S()
    tk = _ints([77])
    A.backend_upload_tokens(tk.ctypes.data, 1)
    h = dev.zeros(DD)
    A.backend_embed_decode(h[0], p("etw"), p("epw"), p("elnw"), p("elnb"))
    out["embed_decode"] = dev.get(h)
    ck, cvv = dev.put(inp["dv_cache_k"]), dev.put(inp["dv_cache_v"])
    x = dev.put(inp["dv_x"])
    A.backend_linear_to_kvcache(ck[0], x[0], p("dec1.sa_kw"), p("dec1.sa_kb"), DD, DD)
    A.backend_linear_to_kvcache(cvv[0], x[0], p("dec1.sa_vw"), p("dec1.sa_vb"), DD, DD)
    out["kvcache_k"] = dev.get(ck)
    out["kvcache_v"] = dev.get(cvv)
    q = dev.put(inp["dv_q"]); o = dev.zeros(DD)
    A.backend_sdp_attn_devS(o[0], q[0], ck[0], cvv[0], dev.zeros(cb.MAX_SEQ)[0])
    out["sdp_devS"] = dev.get(o)

    # batched decode helpers: B=4, item 1 inactive
    B = 4
    active = _ints([1, 0, 1, 1])
    btok = _ints([9, 1000, 3, 16000])
    S_dev = _ints([3, 5, 1, 8])
    h = dev.put(inp["bt_h"])
    A.backend_embed_decode_batch(h[0], btok.ctypes.data, S_dev.ctypes.data, active.ctypes.data,
                                 B, p("etw"), p("epw"), p("elnw"), p("elnb"))
    out["embed_decode_batch"] = dev.get(h)
    x = dev.put(inp["bt_x"]); kc = dev.put(inp["bt_cache"]); vc = dev.put(inp["bt_cache_v"])
    A.backend_linear_to_kvcache_batch(kc[0], x[0], p("dec2.sa_kw"), p("dec2.sa_kb"), B, 10, DD, DD)
    A.backend_linear_to_kvcache_batch(vc[0], x[0], p("dec2.sa_vw"), p("dec2.sa_vb"), B, 10, DD, DD)
    out["kvcache_batch_k"] = dev.get(kc)
    out["kvcache_batch_v"] = dev.get(vc)
    q = dev.put(inp["bt_q"]); o = dev.zeros(B, DD)
    A.backend_sdp_attn_batch_decode_sa(o[0], q[0], kc[0], vc[0], 10, B, dev.zeros(B * 8 * 10)[0])
    out["sdp_batch_sa"] = dev.get(o)
    Tenc = _ints([4, 2, 6, 1])
    A.backend_upload_T_enc(Tenc.ctypes.data, B)
    kk, vv, o = dev.put(inp["bt_ck"]), dev.put(inp["bt_cv"]), dev.zeros(B, DD)
    A.backend_sdp_attn_batch_decode_ca(o[0], q[0], kk[0], vv[0], 6, B, dev.zeros(B * 8 * 6)[0])
    out["sdp_batch_ca"] = dev.get(o)
    lg = dev.put(inp["bt_lg_init"])
    A.backend_lm_head_batch(lg[0], h[0], p("etw"), p("hdb"), active.ctypes.data, B)
    out["lm_head_batch"] = dev.get(lg)
    lgi = dev.put(inp["am_logits"])
    am = _ints([-7, -7, -7, -7])
    A.backend_argmax_batch(am.ctypes.data, lgi[0], active.ctypes.data, B)
    out["argmax_batch"] = am.astype(np.float32)
    return out


# Cases whose reference result is exact (bit-identical on any correct backend).
EXACT_CASES = {"causal_mask", "argmax_batch", "add_inplace"}
