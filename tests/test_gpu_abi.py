"""GPU parity of the drop-in ABI (libct_hip.so) — needs an MI355X.

Every check calls the HIP backend through the C ABI and compares with the
reference (golden fixtures written from the compiled reference CPU backend and
host graph) or with the oracle on the same seeded inputs.  Tolerance for fp32
outputs: ||got - ref||_inf / ||ref||_inf <= 1e-4 per tensor (the activations
enter bf16 MFMA as hi+lo pairs, ~2^-17 relative), far inside the 1e-2 the
path is specified to; integer results and untouched rows are exact.
Batch-vs-single checks are bit-exact.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import ctbind as cb
import kernel_suite as ks
import oracle_bind as ob

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_DIR = ob.REF_DIR
TOL = 1e-4


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def kmodel(hip, kernel_model):
    hip.backend_weights_upload_blob(kernel_model.data_ptr, kernel_model.data_bytes)
    return kernel_model


def test_kernel_suite_matches_reference(hip, kmodel):
    print("case: kernel suite (seed 11, perturbed weights)", flush=True)
    g = np.load(os.path.join(GOLD, "kernels_ext.npz"))
    out = ks.run_suite(hip, ks.ArenaDev(hip), kmodel, ks.make_inputs())
    bad = []
    for k, v in out.items():
        ref = g["out_" + k]
        if k in ks.EXACT_CASES:
            ok = bits_equal(v, ref)
        else:
            ok = relerr(v, ref) <= TOL
        print(f"  {k:24s} relerr={relerr(v, ref):.2e} exact={bits_equal(v, ref)}")
        if not ok:
            bad.append(k)
    assert not bad, bad


def test_untouched_rows_and_argmax(hip, kmodel):
    g = np.load(os.path.join(GOLD, "kernels_ext.npz"))
    out = ks.run_suite(hip, ks.ArenaDev(hip), kmodel, ks.make_inputs())
    # inactive item 1 keeps its sentinel rows exactly
    assert np.all(out["embed_decode_batch"][1] == 7.5)
    assert np.all(out["lm_head_batch"][1] == -3.25)
    assert np.array_equal(out["argmax_batch"], g["out_argmax_batch"])


def test_reference_kernel_test_binary(hip, tmp_path):
    """The reference's own tests/test_kernels.c, linked against libct_hip.so,
    judged by its own criterion (abs 1e-4, tests/run_tests.sh:12)."""
    exe = os.path.join(REF_DIR, "test_kernels_hip")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_kernels_hip not built")
    out = tmp_path / "hip.bin"
    print("case: reference tests/test_kernels.c on HIP", flush=True)
    subprocess.run([exe, str(out)], check=True, timeout=120)
    got = np.fromfile(out, np.float32)
    ref = np.fromfile(os.path.join(GOLD, "test_kernels_ref_cpu.bin"), np.float32)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 1e-4


def test_gemm_shapes_and_batch_invariance(hip, kmodel):
    o = ob.oracle()
    dev = ks.ArenaDev(hip, 1 << 26)
    rng = np.random.default_rng(10)
    cases = [(1, 1024, "dec0.sa_qw", 1024, "dec0.sa_qb"),
             (200, 4096, "dec1.ffn_w1", 1024, "dec1.ffn_b1"),
             (65, 1024, "dec1.ffn_w2", 4096, "dec1.ffn_b2"),
             (37, 1280, "enc0.ff1_w2", 5120, "enc0.ff1_b2")]
    for M, N, wf, K, bfield in cases:
        print(f"case: linear M={M} N={N} K={K}", flush=True)
        x = rng.standard_normal((M, K)).astype(np.float32)
        xd = dev.put(x)
        y = dev.zeros(M, N)
        hip.backend_linear(y[0], xd[0], kmodel.ptr(wf), kmodel.ptr(bfield), M, K, N)
        got = dev.get(y)
        ref = np.zeros((M, N), np.float32)
        o.orc_linear(ref.ctypes.data, x.ctypes.data, kmodel.ptr(wf), kmodel.ptr(bfield), M, K, N)
        assert relerr(got, ref) <= TOL, (M, N, K, relerr(got, ref))
        # every row equals the same row computed alone (M = 1)
        for r in sorted({0, M // 2, M - 1}):
            y1 = dev.zeros(1, N)
            hip.backend_linear(y1[0], xd[0] + r * K * 4, kmodel.ptr(wf), kmodel.ptr(bfield), 1, K, N)
            assert bits_equal(dev.get(y1)[0], got[r]), (M, r)


def test_gemm_unaligned_k(hip):
    """K not a multiple of 8 takes the scalar-load path (test_kernels.c uses
    K = 64; here K = 45 with an unaligned activation pointer)."""
    o = ob.oracle()
    rng = np.random.default_rng(11)
    M, K, N = 3, 45, 50
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)
    b = (rng.standard_normal(N) * 0.05).astype(np.float32)
    bb = (b.view(np.uint32) >> 16).astype(np.uint16)
    blob = np.concatenate([wb, bb])
    hip.backend_weights_upload_blob(blob.ctypes.data, blob.nbytes)
    dev = ks.ArenaDev(hip, 1 << 20)
    x = rng.standard_normal((M, K)).astype(np.float32)
    # one leading float makes the activation pointer 4-byte (not 16-byte) aligned
    xd = dev.put(np.concatenate([np.zeros(1, np.float32), x.ravel()]))
    y = dev.zeros(M, N)
    hip.backend_linear_relu(y[0], xd[0] + 4, blob.ctypes.data, blob.ctypes.data + wb.nbytes, M, K, N)
    ref = np.zeros((M, N), np.float32)
    o.orc_linear_relu(ref.ctypes.data, x.ctypes.data, blob.ctypes.data, blob.ctypes.data + wb.nbytes, M, K, N)
    assert relerr(dev.get(y), ref) <= TOL


def test_ragged_attention_batch_invariance(hip, kmodel):
    o = ob.oracle()
    hip.backend_weights_upload_blob(kmodel.data_ptr, kmodel.data_bytes)
    dev = ks.ArenaDev(hip, 1 << 26)
    rng = np.random.default_rng(12)
    B, stride = 9, 300
    lens = np.array([1, 2, 17, 64, 65, 130, 257, 299, 300], np.int32)
    Q = (rng.standard_normal((B, 1024)) * 0.3).astype(np.float32)
    K = (rng.standard_normal((B, stride, 1024)) * 0.3).astype(np.float32)
    V = rng.standard_normal((B, stride, 1024)).astype(np.float32)
    qd, kd, vd, od = dev.put(Q), dev.put(K), dev.put(V), dev.zeros(B, 1024)
    hip.backend_upload_T_enc(lens.ctypes.data, B)
    print("case: ragged cross attention B=9", flush=True)
    hip.backend_sdp_attn_batch_decode_ca(od[0], qd[0], kd[0], vd[0], stride, B, None)
    got = dev.get(od)
    for b in range(B):
        ref = np.zeros(1024, np.float32)
        o.orc_sdp_attn(ref.ctypes.data, Q[b].ctypes.data, K[b].ctypes.data, V[b].ctypes.data,
                       None, 1, int(lens[b]), None)
        assert relerr(got[b], ref) <= TOL, b
    # item b alone (B = 1) gives the same bits
    for b in (0, 4, 8):
        one = np.array([lens[b]], np.int32)
        hip.backend_upload_T_enc(one.ctypes.data, 1)
        o1 = dev.zeros(1, 1024)
        hip.backend_sdp_attn_batch_decode_ca(o1[0], qd[0] + b * 4096, kd[0] + b * stride * 4096,
                                             vd[0] + b * stride * 4096, stride, 1, None)
        assert bits_equal(dev.get(o1)[0], got[b]), b
    # the devS form with the same length gives the same bits too
    hip.backend_decode_set_S(int(lens[5]))
    o2 = dev.zeros(1024)
    hip.backend_sdp_attn_devS(o2[0], qd[0] + 5 * 4096, kd[0] + 5 * stride * 4096,
                              vd[0] + 5 * stride * 4096, None)
    assert bits_equal(dev.get(o2), got[5])


def test_empty_batches_and_edge_lengths(hip, kmodel):
    """Edge cases of the batched ABI as the reference's loops treat them
    (backends/cpu/backend.c:425-500): a batch of 0 items writes nothing; an
    item of zero keys gets a zero attention row (a sum over no keys); and
    the longest lengths, MAX_SEQ self keys and 1024 encoder frames, match
    the oracle, ragged beside short items, with the item alone giving the
    same bits."""
    o = ob.oracle()
    dev = ks.ArenaDev(hip, 1 << 26)
    rng = np.random.default_rng(44)
    DD, V = 1024, cb.VOCAB
    ints = ks._ints
    # B = 0: every output untouched
    print("case: batch of 0 items", flush=True)
    h0 = np.full((2, DD), 2.5, np.float32)
    lg0 = np.full((2, V), -1.5, np.float32)
    h, lg, od = dev.put(h0), dev.put(lg0), dev.put(h0)
    kc = dev.put(np.full((2, 4, DD), 0.75, np.float32))
    hip.backend_embed_decode_batch(h[0], ints([3, 4]).ctypes.data, ints([1, 1]).ctypes.data,
                                   ints([1, 1]).ctypes.data, 0, kmodel.ptr("etw"), kmodel.ptr("epw"),
                                   kmodel.ptr("elnw"), kmodel.ptr("elnb"))
    hip.backend_lm_head_batch(lg[0], h[0], kmodel.ptr("etw"), kmodel.ptr("hdb"), ints([1, 1]).ctypes.data, 0)
    am = ints([-7, -7])
    hip.backend_argmax_batch(am.ctypes.data, lg[0], ints([1, 1]).ctypes.data, 0)
    hip.backend_linear_to_kvcache_batch(kc[0], h[0], kmodel.ptr("dec2.sa_kw"), kmodel.ptr("dec2.sa_kb"),
                                        0, 4, DD, DD)
    hip.backend_upload_T_enc(ints([3, 3]).ctypes.data, 0)
    hip.backend_sdp_attn_batch_decode_sa(od[0], h[0], kc[0], kc[0], 4, 0, dev.zeros(2 * 8 * 4)[0])
    hip.backend_sdp_attn_batch_decode_ca(od[0], h[0], kc[0], kc[0], 4, 0, dev.zeros(2 * 8 * 4)[0])
    assert bits_equal(dev.get(h), h0) and bits_equal(dev.get(lg), lg0) and bits_equal(dev.get(od), h0)
    assert np.all(dev.get(kc) == 0.75) and np.all(am == -7)
    # cross attention: 0, 1, 1024 and 517 frames in one ragged batch
    stride = 1024
    lens = np.array([0, 1, 1024, 517], np.int32)
    B = len(lens)
    print(f"case: ragged cross attention, lengths {lens.tolist()}", flush=True)
    Q = (rng.standard_normal((B, DD)) * 0.3).astype(np.float32)
    K = (rng.standard_normal((B, stride, DD)) * 0.3).astype(np.float32)
    Vv = rng.standard_normal((B, stride, DD)).astype(np.float32)
    qd, kd, vd, out = dev.put(Q), dev.put(K), dev.put(Vv), dev.put(np.full((B, DD), 9.0, np.float32))
    hip.backend_upload_T_enc(lens.ctypes.data, B)
    hip.backend_sdp_attn_batch_decode_ca(out[0], qd[0], kd[0], vd[0], stride, B, dev.zeros(B * 8 * stride)[0])
    got = dev.get(out)
    assert np.all(got[0] == 0.0)
    for b in range(1, B):
        ref = np.zeros(DD, np.float32)
        o.orc_sdp_attn(ref.ctypes.data, Q[b].ctypes.data, K[b].ctypes.data, Vv[b].ctypes.data,
                       None, 1, int(lens[b]), None)
        assert relerr(got[b], ref) <= TOL, b
    one = lens[2:3].copy()
    hip.backend_upload_T_enc(one.ctypes.data, 1)
    o1 = dev.zeros(1, DD)
    hip.backend_sdp_attn_batch_decode_ca(o1[0], qd[0] + 2 * DD * 4, kd[0] + 2 * stride * DD * 4,
                                         vd[0] + 2 * stride * DD * 4, stride, 1, dev.zeros(8 * stride)[0])
    assert bits_equal(dev.get(o1)[0], got[2])
    # self attention at S = MAX_SEQ beside S = 1, the lengths latched by the batched embedding
    print("case: self attention at S = MAX_SEQ and S = 1", flush=True)
    S = np.array([cb.MAX_SEQ, 1], np.int32)
    B = len(S)
    hs = dev.zeros(B, DD)
    hip.backend_embed_decode_batch(hs[0], ints([11, 12]).ctypes.data, S.ctypes.data, ints([1, 1]).ctypes.data,
                                   B, kmodel.ptr("etw"), kmodel.ptr("epw"), kmodel.ptr("elnw"), kmodel.ptr("elnb"))
    stride = cb.MAX_SEQ
    Ks = (rng.standard_normal((B, stride, DD)) * 0.3).astype(np.float32)
    Vs = rng.standard_normal((B, stride, DD)).astype(np.float32)
    Qs = (rng.standard_normal((B, DD)) * 0.3).astype(np.float32)
    qd, kd, vd, out = dev.put(Qs), dev.put(Ks), dev.put(Vs), dev.zeros(B, DD)
    hip.backend_sdp_attn_batch_decode_sa(out[0], qd[0], kd[0], vd[0], stride, B, dev.zeros(B * 8 * stride)[0])
    got = dev.get(out)
    for b in range(B):
        ref = np.zeros(DD, np.float32)
        o.orc_sdp_attn(ref.ctypes.data, Qs[b].ctypes.data, Ks[b].ctypes.data, Vs[b].ctypes.data,
                       None, 1, int(S[b]), None)
        assert relerr(got[b], ref) <= TOL, b


def test_graph_capture_replay(hip, kmodel):
    """A captured region replays to the eager result, several times, with
    eager work and synchronisation in between."""
    hip.backend_weights_upload_blob(kmodel.data_ptr, kmodel.data_bytes)
    dev = ks.ArenaDev(hip, 1 << 22)
    rng = np.random.default_rng(13)
    x = dev.put(rng.standard_normal((4, 1024)).astype(np.float32))
    y = dev.zeros(4, 1024)
    z = dev.zeros(4, 4096)
    p = kmodel.ptr

    def region():
        hip.backend_layernorm(y[0], x[0], p("dec3.sa_lnw"), p("dec3.sa_lnb"), 4, 1024)
        hip.backend_linear_relu(z[0], y[0], p("dec3.ffn_w1"), p("dec3.ffn_b1"), 4, 1024, 4096)
        hip.backend_linear_fmadd(y[0], 1.0, z[0], p("dec3.ffn_w2"), p("dec3.ffn_b2"), 4, 4096, 1024)

    region()
    eager = dev.get(y)
    assert hip.backend_graph_replay(7, 1, 2, 3) == 0
    hip.backend_graph_begin_capture(7)
    region()
    hip.backend_graph_end_capture(7, 1, 2, 3)
    assert bits_equal(dev.get(y), eager)
    for i in range(3):
        hip.backend_layernorm(y[0], y[0], p("dec4.sa_lnw"), p("dec4.sa_lnb"), 4, 1024)  # eager noise
        assert hip.backend_graph_replay(7, 1, 2, 3) == 1
        assert bits_equal(dev.get(y), eager), i


# --------------------------------------------------------------------------
# the reference host graph (model.h) driving the HIP backend
# --------------------------------------------------------------------------
def ref_model_hip():
    path = os.path.join(REF_DIR, "libref_model_hip.so")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref/libref_model_hip.so not built")
    lib = C.CDLL(path)
    P, I = C.c_void_p, C.c_int
    lib.ref_set_weights.argtypes = [P]
    lib.ref_transcribe_single.argtypes = [P, I, P, I, I, I, I, P, P, P]
    lib.ref_transcribe_single.restype = I
    lib.ref_transcribe_batch.argtypes = [P, I, P, I, P, I, P, I, I, I, P, P, P]
    return lib


@pytest.mark.parametrize("variant,fname", [(0, "model_small.npz"), (2, "model_small_hot.npz")])
def test_reference_host_on_hip(hip, variant, fname):
    from golden.make_golden import CLIPS, SINGLE_LIMIT, BATCH_LIMITS, MODEL_SEED
    path = os.path.join(GOLD, fname)
    if not os.path.exists(path):
        pytest.skip("model fixture not generated")
    g = np.load(path)
    lib = ref_model_hip()
    m = cb.SynthModel(seed=MODEL_SEED, variant=variant)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    lib.ref_set_weights(m.weights_ref())
    prompt = np.asarray(cb.PROMPT, np.int32)
    mel0 = g["mel0"]
    print(f"case: model.h single path on HIP, variant {variant}", flush=True)
    toks = np.zeros(SINGLE_LIMIT, np.int32)
    lg = np.zeros((SINGLE_LIMIT, cb.VOCAB), np.float32)
    eh = np.zeros((cb.t_enc(mel0.shape[1]), cb.DEC_D), np.float32)
    n = lib.ref_transcribe_single(mel0.ctypes.data, mel0.shape[1], prompt.ctypes.data, len(prompt),
                                  SINGLE_LIMIT, 1, 0, toks.ctypes.data, lg.ctypes.data, eh.ctypes.data)
    print("  enc_h relerr", relerr(eh, g["enc_h0"]), "logits relerr", relerr(lg[:2], g["single_logits"]))
    assert relerr(eh, g["enc_h0"]) <= 1e-3
    assert relerr(lg[:2], g["single_logits"]) <= 1e-3
    assert np.array_equal(toks[:n], g["single_tokens"])
    print(f"case: model.h batch path on HIP, variant {variant}", flush=True)
    mels = [g["mel0"], g["mel1"]]
    B = 2
    Tm = np.asarray([mm.shape[1] for mm in mels], np.int32)
    Tmax = int(Tm.max())
    mb = np.zeros((B, cb.N_MELS, Tmax), np.float32)
    for b, mm in enumerate(mels):
        mb[b, :, :mm.shape[1]] = mm
    lim = np.asarray(BATCH_LIMITS, np.int32)
    bt = np.zeros((B, max(BATCH_LIMITS)), np.int32)
    nb = np.zeros(B, np.int32)
    lib.ref_transcribe_batch(mb.ctypes.data, B, Tm.ctypes.data, Tmax, prompt.ctypes.data, len(prompt),
                             lim.ctypes.data, 1, 1, max(BATCH_LIMITS), bt.ctypes.data, nb.ctypes.data, None)
    assert np.array_equal(nb, g["batch_n"])
    assert np.array_equal(bt, g["batch_tokens"])



def test_reference_host_threads_on_hip(hip):
    """transcribe.c's worker pattern (transcribe.c:849-943): each thread calls
    backend_init, runs the model.h single path on its own clip through its own
    thread-local state (stream, arena, device S counter, graphs), then
    backend_thread_cleanup.  Three threads at once give each clip the tokens
    and logits bits of a run on the main thread."""
    import threading
    from golden.make_golden import SINGLE_LIMIT, MODEL_SEED
    path = os.path.join(GOLD, "model_small_hot.npz")
    if not os.path.exists(path):
        pytest.skip("model fixture not generated")
    g = np.load(path)
    lib = ref_model_hip()
    m = cb.SynthModel(seed=MODEL_SEED, variant=2)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    lib.ref_set_weights(m.weights_ref())
    prompt = np.asarray(cb.PROMPT, np.int32)
    mels = [np.ascontiguousarray(g["mel0"]), np.ascontiguousarray(g["mel1"])]

    def run(mel):
        toks = np.zeros(SINGLE_LIMIT, np.int32)
        lg = np.zeros((SINGLE_LIMIT, cb.VOCAB), np.float32)
        n = lib.ref_transcribe_single(mel.ctypes.data, mel.shape[1], prompt.ctypes.data, len(prompt),
                                      SINGLE_LIMIT, 1, 0, toks.ctypes.data, lg.ctypes.data, None)
        return toks[:n], lg[:n]

    print("case: model.h single path, main thread, clips 0 and 1", flush=True)
    want = [run(mm) for mm in mels]
    got, errs = [None] * 3, []

    def worker(i):
        try:
            hip.backend_init(0)
            got[i] = run(mels[i % 2])
            hip.backend_thread_cleanup()
        except BaseException as ex:   # surfaced below
            errs.append(ex)

    print("case: three worker threads, clips 0, 1, 0", flush=True)
    ts = [threading.Thread(target=worker, args=(i,)) for i in range(3)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=240)
    assert not errs and all(not t.is_alive() for t in ts)
    for i in range(3):
        wt, wl = want[i % 2]
        assert np.array_equal(got[i][0], wt), i
        assert bits_equal(got[i][1], wl), i


ENC_T = [17, 37, 101, 376, 751, 2048]


@pytest.mark.parametrize("T", ENC_T)
def test_encoder_ops_long_T_vs_oracle(hip, kmodel, T):
    """Rel-pos MHSA and the conformer conv module at encoder lengths of 1.3 s
    to the supported maximum (T = 17, 37, 101, 376, 751 and 2048 frames:
    several 16-query blocks, multi-tile score loops, the 32-key PV loop, score
    rows up to the 131 KB LDS bound), through the ABI against the oracle
    (backends/cpu/backend.c:244-337): own position table and the batch form
    whose table is built for the longest clip (376, or T beyond it) and read
    from row T_max - T (model.h:586-592).  <= 1e-4 relative per tensor."""
    hip.backend_weights_upload_blob(kmodel.data_ptr, kmodel.data_bytes)
    dev = ks.ArenaDev(hip)
    o = ob.oracle()
    rng = np.random.default_rng(1000 + T)
    x0 = rng.standard_normal((T, cb.ENC_D)).astype(np.float32)
    D = cb.ENC_D
    work = dev.zeros((5 * T - 1) * D + max(T * (3 * T - 1), 2 * T * D))
    pe_own = dev.zeros(2 * T - 1, D)
    hip.backend_make_rel_pos_emb(pe_own[0], T)
    TM = max(376, T)
    pe_max = dev.zeros(2 * TM - 1, D)
    hip.backend_make_rel_pos_emb(pe_max[0], TM)
    pe_ref = np.zeros((2 * T - 1, D), np.float32)
    o.orc_make_rel_pos_emb(pe_ref.ctypes.data, T)
    assert relerr(dev.get(pe_own), pe_ref) <= 1e-6
    x = dev.zeros(T, D)
    conv_work = dev.zeros(3 * T * D)
    for layer in (0, 7):
        want = x0.copy()
        o.orc_rel_pos_mhsa(want.ctypes.data, pe_ref.ctypes.data, T, kmodel.elayer_ptr(layer), None)
        for form, pe_ptr in (("own", pe_own[0]), ("shifted", pe_max[0] + (TM - T) * D * 4)):
            hip.backend_htod(x[0], x0.ctypes.data, x0.size)
            hip.backend_rel_pos_mhsa(x[0], pe_ptr, T, kmodel.elayer_ptr(layer), work[0])
            e = relerr(dev.get(x), want)
            print(f"case: rel_pos_mhsa T={T} layer {layer} {form} table: relerr {e:.2e}", flush=True)
            assert e <= TOL, (T, layer, form, e)
        want = x0.copy()
        o.orc_conformer_conv(want.ctypes.data, T, kmodel.elayer_ptr(layer), None)
        hip.backend_htod(x[0], x0.ctypes.data, x0.size)
        hip.backend_conformer_conv(x[0], T, kmodel.elayer_ptr(layer), conv_work[0])
        e = relerr(dev.get(x), want)
        print(f"case: conformer_conv T={T} layer {layer}: relerr {e:.2e}", flush=True)
        assert e <= TOL, (T, layer, e)


@pytest.mark.parametrize("case", ["weight_outside_blob", "arena_beyond_device"])
def test_fatal_paths_after_init(case):
    """Fatal exits that need an uploaded blob and an initialised device, in
    a child process (the reference's convention: print and exit(1),
    backends/cuda/backend.cu:26-33): a weight pointer past the end of the
    uploaded blob, and an arena larger than the device's memory (1 TiB: the
    allocation fails and the backend exits instead of returning NULL).  No
    kernel is launched in either case."""
    import sys
    calls = {"weight_outside_blob": ("L.backend_device_ptr(C.c_void_p(C.addressof(b) + 8192))",
                                     "weight pointer outside the uploaded blob"),
             "arena_beyond_device": ("L.backend_arena_alloc(C.c_size_t(1 << 38))", "HIP error")}
    call, msg = calls[case]
    code = (f"import ctypes as C; L = C.CDLL({cb.HIP_LIB!r}); b = (C.c_char * 4096)(); "
            "L.backend_weights_upload_blob(b, C.c_size_t(4096)); L.backend_init(0); "
            f"print('case {case}', flush=True); {call}; print('returned')")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert f"case {case}" in r.stdout, r.stderr
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert msg in r.stderr, r.stderr
    assert "returned" not in r.stdout
