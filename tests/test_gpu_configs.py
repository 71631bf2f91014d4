"""The benchmark configurations on the engine — needs an MI355X.

  * single clip (8 s, 48 tokens) and uniform batch (10 s clips, 96 tokens):
    the engine (bf16 and fp32 KV caches) against fixtures written by the
    reference itself (model.h single-sequence path on the reference CPU
    backend, fp32 KV: tests/golden/config_c0c1_v*.npz).  Encoder output and
    logits within 1e-2 max relative error (||.||_inf per row) — the specified
    bound — and within a regression bound near the measured error (one
    documented exception below); greedy tokens identical up to the first
    step whose reference top-1/top-2 gap is below twice the logit bound
    (relative), where a correct backend may pick either;
  * the same fixtures with the encoder FFN projections in single-pass bf16
    (their inputs rounded to bf16, fp32 accumulation): encoder output within
    the specified 1e-2, logits of the specified weights within 5e-3; and the
    HIP single-pass path against the oracle's emulation of that rounding
    (one rounding layer, short clip) by the size and direction of the error
    each makes against fp32;
  * ragged batch of 32 (clips 2-30 s, limits 16-224, one packed step loop):
    tokens, the chosen logit of every token, and every step's logits of
    sampled requests bit-identical to the same request run alone;
  * the continuous-batching stream (256 requests, <= 64 in flight, encoding
    overlapped with decoding): every request produces exactly its limit, and
    sampled requests are bit-identical to runs alone.
"""
import ctypes as C
import os

import numpy as np
import pytest

import ctbind as cb
import oracle_bind as ob

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SPEC_TOL = 1e-2
# encoder regression bound per FFN mode: fp32-accurate (hi+lo split) or
# single-pass bf16 (the rounding of the FFN inputs alone moves the encoder
# output by 3.8e-3 in the oracle)
ENC_REG = {False: 3e-5, True: 5e-3}
# logits of the specified weights in single-pass FFN mode
FFN_LOGIT_SPEC = 5e-3
# Logits bound per (weight variant, bf16 KV): the specified 1e-2, or a
# regression bound near the measured error when tighter.  The exception is
# bf16 KV on the decoder-hot test weights (linears N(0, 0.12) instead of the
# specified N(0, 0.02)): their large activations make the bf16 rounding of
# K/V alone move the fp32 logits by 1-1.7% (the oracle in both KV modes
# against each other, the reference's own arithmetic otherwise), so that
# case is held to 2.5e-2.  The decoder-warm weights (linears N(0, 0.08)) keep
# greedy decoding input-dependent with bf16 K/V inside the specified 1e-2.
# The benchmark runs the specified weights.
LOGIT_TOL = {(0, True): 1e-3, (0, False): 1e-5, (2, True): 2.5e-2, (2, False): 2e-4,
             (3, True): SPEC_TOL, (3, False): 2e-4}
# single-pass FFN mode: the encoder's bf16 rounding reaches the logits
# (oracle emulation: 6e-4 on the specified weights, 4.7e-3 on the hot ones)
LOGIT_TOL_FFN = {(0, True): 2e-3, (0, False): 2e-3, (2, True): 2.5e-2, (2, False): 1e-2,
                 (3, True): SPEC_TOL, (3, False): SPEC_TOL}


def row_relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


_models = {}


def model(hip, variant):
    """Synthetic weights (seed 5) of the given variant, uploaded as the
    current blob."""
    if variant not in _models:
        _models.clear()
        _models[variant] = cb.SynthModel(seed=5, variant=variant)
    m = _models[variant]
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    return m


def fixture_requests(g):
    keys = sorted({k.rsplit("_", 1)[0] for k in g.files if k.endswith("_tokens")})
    out = []
    for key in keys:
        x = cb.synth_audio(int(g[f"{key}_samples"]), int(g[f"{key}_seed"]))
        mel = ob.compute_mel(x)
        s = float(np.asarray(mel, np.float64).sum())
        assert abs(s - float(g[f"{key}_mel_sum"])) <= 1e-9 * max(1.0, abs(s)), key
        out.append((key, mel))
    return out


@pytest.mark.parametrize("ffn_bf16", [False, True])
@pytest.mark.parametrize("variant", [0, 2, 3])
@pytest.mark.parametrize("kv_bf16", [True, False])
def test_single_and_uniform_configs_vs_reference(hip, variant, kv_bf16, ffn_bf16):
    path = os.path.join(GOLD, f"config_c0c1_v{variant}.npz")
    g = np.load(path)
    m = model(hip, variant)
    reqs = fixture_requests(g)
    limits = [len(g[f"{k}_tokens"]) for k, _ in reqs]
    npr = len(cb.PROMPT)
    eng = cb.Engine(m, slots=len(reqs), max_requests=len(reqs), max_frames=128, kv_bf16=kv_bf16,
                    max_tokens=npr + max(limits), prefill_rows=0, enc_ffn_bf16=int(ffn_bf16))
    try:
        for (key, mel), lim in zip(reqs, limits):
            eng.submit(mel, lim, cb.HIPB_SUPPRESS_EOS)
        eng.encode()
        rows = {i: {} for i in range(len(reqs))}
        want_rows = {i: set(int(j) for j in g[f"{k}_rows"]) for i, (k, _) in enumerate(reqs)}
        for step in range(npr + max(limits)):
            eng.step()
            if step == 0:
                assert [eng.slot_of(i) for i in range(len(reqs))] == list(range(len(reqs)))
            j = step - (npr - 1)
            for i in range(len(reqs)):
                if j in want_rows[i]:
                    rows[i][j] = eng.logits(i)
            if eng.finished() == len(reqs):
                break
        assert eng.finished() == len(reqs)
        worst_enc = worst_lg = 0.0
        for i, (key, _) in enumerate(reqs):
            enc_err = row_relerr(eng.enc_out(i), g[f"{key}_enc_h"])
            worst_enc = max(worst_enc, enc_err)
            toks, ref = eng.tokens(i), g[f"{key}_tokens"]
            assert len(toks) == len(ref)
            gap = g[f"{key}_margin"]
            # tokens must agree while every reference top-1/top-2 gap so far
            # exceeds twice the logit bound (a smaller gap may flip)
            tol = (LOGIT_TOL_FFN if ffn_bf16 else LOGIT_TOL)[(variant, kv_bf16)]
            n_cmp = int(np.argmax(gap < 2 * tol)) if (gap < 2 * tol).any() else len(ref)
            same = int(np.argmax(toks != ref)) if (toks != ref).any() else len(ref)
            print(f"case: v{variant} kv_bf16={kv_bf16} ffn_bf16={ffn_bf16} {key} T_enc={g[f'{key}_enc_h'].shape[0]} "
                  f"enc relerr {enc_err:.2e}, tokens agree {same}/{len(ref)} "
                  f"(clear-gap prefix {n_cmp})", flush=True)
            assert same >= n_cmp, (key, same, n_cmp)
            for r, j in enumerate(g[f"{key}_rows"]):
                j = int(j)
                if j > same:      # conditioned on a different earlier token
                    continue
                e = row_relerr(rows[i][j], g[f"{key}_logits"][r])
                worst_lg = max(worst_lg, e)
                print(f"    logits row {j}: relerr {e:.2e}", flush=True)
                assert e <= tol, (key, j, e)
            assert enc_err <= SPEC_TOL, (key, enc_err)
        print(f"  worst: encoder {worst_enc:.2e}, logits {worst_lg:.2e}", flush=True)
        assert worst_enc <= ENC_REG[ffn_bf16], worst_enc
        if variant == 0:
            assert worst_lg <= (FFN_LOGIT_SPEC if ffn_bf16 else SPEC_TOL)
        if variant == 3:
            # input-dependent tokens and the specified bound in every mode,
            # the benchmark's (bf16 K/V, single-pass FFN) included
            assert worst_lg <= SPEC_TOL
            assert max(len(set(g[f"{k}_tokens"].tolist())) for k, _ in reqs) >= 10
    finally:
        eng.close()


def one_layer_model(variant):
    """Weights of the given variant (seed 5) whose encoder layers 1..23 pass
    their input through their final LayerNorm only: zero FFN output
    projections, MHSA output projection and conv pointwise-2, unit final LN
    scale and zero shift.  The encoder's single-pass FFN rounding then acts
    in layer 0 alone."""
    m = cb.SynthModel(seed=5, variant=variant)
    D, FF = cb.ENC_D, cb.ENC_FF
    zero = {"ff1_w2": D * FF, "ff1_b2": D, "ff2_w2": D * FF, "ff2_b2": D, "sa_ow": D * D,
            "sa_ob": D, "cv_pw2w": D * D, "cv_pw2b": D, "out_lnb": D}
    for layer in range(1, cb.ENC_N):
        for f, n in zero.items():
            C.memset(m.ptr(f"enc{layer}.{f}"), 0, 2 * n)
        one = np.full(D, 0x3F80, np.uint16)
        C.memmove(m.ptr(f"enc{layer}.out_lnw"), one.ctypes.data, 2 * D)
    return m


def err_signature(got, emu, fp32):
    """(|got - fp32| / |emu - fp32|, cosine of the two error vectors), L2."""
    d_got = np.asarray(got, np.float64) - fp32
    d_emu = np.asarray(emu, np.float64) - fp32
    n_got, n_emu = np.linalg.norm(d_got), np.linalg.norm(d_emu)
    return float(n_got / n_emu), float((d_got * d_emu).sum() / (n_got * n_emu))


@pytest.mark.parametrize("variant", [0, 2])
def test_single_pass_ffn_vs_oracle_mode(hip, variant):
    """The single-pass FFN path against the oracle's emulation of its bf16
    rounding of the FFN inputs, on a model whose rounding happens in one
    encoder layer.  The rounding is chaotic in its inputs' last bits (an
    input within the two computations' fp32 noise of a bf16 boundary rounds
    one ulp apart; noise of 5e-6 on the oracle's own layer input moves its
    output by half the mode's error), so the two are compared by the error
    each makes against the fp32 oracle: equal size (ratio 1.00 measured,
    where rounding only the LayerNorm output or only the SiLU output gives
    0.70 and truncation 2.6) and aligned (cosine 0.76 for the encoder, 0.9
    for the logits; 0.21 for SiLU-only rounding, -0.06 for truncation).
    2.2 s clip, fp32 KV, 6 tokens, identical to the emulation's."""
    _models.clear()
    m = one_layer_model(variant)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    mel = ob.compute_mel(cb.synth_audio(int(2.2 * cb.SR), 77))
    limit = 6
    with ob.enc_ffn_bf16():
        emu_toks, emu_lg, emu_enc = ob.transcribe(m, mel, limit, want_logits=True)
    _, fp_lg, fp_enc = ob.transcribe(m, mel, limit, want_logits=True)
    npr = len(cb.PROMPT)
    eng = cb.Engine(m, slots=1, max_requests=1, max_frames=64, kv_bf16=False,
                    max_tokens=npr + limit, prefill_rows=0, enc_ffn_bf16=1)
    try:
        eng.submit(mel, limit, cb.HIPB_SUPPRESS_EOS)
        eng.encode()
        lg = []
        for step in range(npr + limit):
            eng.step()
            if step >= npr - 1 and eng.finished() == 0:
                lg.append(eng.logits(0))
            if eng.finished() == 1:
                break
        assert eng.finished() == 1
        enc = eng.enc_out(0)
        toks = eng.tokens(0)
    finally:
        eng.close()
    k = limit - 1
    assert len(lg) == k
    e_ratio, e_cos = err_signature(enc, emu_enc, fp_enc)
    l_ratio, l_cos = err_signature(np.stack(lg), emu_lg[:k], fp_lg[:k])
    print(f"case: v{variant} T_enc={emu_enc.shape[0]}: encoder error vs emulation's: ratio "
          f"{e_ratio:.3f} cos {e_cos:.3f}; logits ratio {l_ratio:.3f} cos {l_cos:.3f}; "
          f"tokens {toks.tolist()}", flush=True)
    assert np.array_equal(toks, emu_toks)
    assert 0.9 <= e_ratio <= 1.1 and e_cos >= 0.5, (e_ratio, e_cos)
    assert 0.8 <= l_ratio <= 1.25 and l_cos >= 0.7, (l_ratio, l_cos)


def run_collect(eng, n_req, watch):
    """Steps until all n_req requests finished; returns, per watched request,
    the logits row of each step it held a slot after."""
    hist = {r: [] for r in watch}
    n = 0
    while eng.finished() < n_req:
        eng.step()
        n += 1
        assert n < 4 * cb.MAX_SEQ
        for r in watch:
            s = eng.slot_of(r)
            if s >= 0:
                hist[r].append(eng.logits(s))
    return hist


def compare_alone(m, pcm, limit, prompt_rows, packed_tokens, packed_scores, packed_hist, max_frames,
                  label, ffn_bf16=0):
    alone = cb.Engine(m, slots=1, max_requests=1, max_frames=max_frames, kv_bf16=True,
                      max_tokens=len(cb.PROMPT) + limit, prefill_rows=prompt_rows,
                      enc_ffn_bf16=ffn_bf16)
    try:
        alone.submit_pcm(pcm, limit, cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS)
        alone.encode()
        ha = run_collect(alone, 1, [0]) if packed_hist is not None else None
        if ha is None:
            alone.run(chunk=8)
        toks, sc = alone.tokens(0), alone.scores(0)
    finally:
        alone.close()
    print(f"case: {label}: {len(toks)} tokens", flush=True)
    assert np.array_equal(toks, packed_tokens), label
    assert np.array_equal(bits(sc), bits(packed_scores)), label
    if packed_hist is not None:
        # the rows that produced tokens 0 .. limit-2 (the last step's row is
        # read after the slot is freed, in neither run)
        k = limit - 1
        a, p = ha[0][len(ha[0]) - k:], packed_hist[len(packed_hist) - k:]
        assert len(a) == len(p) == k
        for j in range(k):
            assert np.array_equal(bits(a[j]), bits(p[j])), (label, j)


def test_ragged_batch32_vs_single(hip):
    """32 requests, clips U(2,30) s (a 30 s clip among them), limits U(16,224),
    EOS suppressed and forced at the limit, all in one packed step loop with
    16 spare prompt rows; four requests (the 30 s clip, the longest limit, two
    more) rerun alone on one slot with no spare rows."""
    m = model(hip, 2)
    rng = np.random.default_rng(32)
    secs = rng.uniform(2.0, 30.0, 32)
    secs[5] = 30.0
    limits = rng.integers(16, 225, 32)
    pcms = [cb.synth_audio(int(s * cb.SR), 3200 + i) for i, s in enumerate(secs)]
    sample = sorted({5, int(np.argmax(limits)), 0, 17})
    eng = cb.Engine(m, slots=32, max_requests=32, max_frames=376, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 224, prefill_rows=16)
    try:
        for p, lim in zip(pcms, limits):
            eng.submit_pcm(p, int(lim), cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS)
        eng.encode()
        hist = run_collect(eng, 32, sample)
        assert eng.finished() == 32
        toks = {r: eng.tokens(r) for r in range(32)}
        scores = {r: eng.scores(r) for r in sample}
    finally:
        eng.close()
    for r in range(32):
        assert len(toks[r]) == limits[r] and toks[r][-1] == cb.EOS, r
    for r in sample:
        compare_alone(m, pcms[r], int(limits[r]), 0, toks[r], scores[r], hist[r], 376,
                      f"request {r} ({secs[r]:.1f} s, {limits[r]} tokens) alone vs batch of 32")


@pytest.mark.parametrize("admit_order,ffn_bf16,batch_frames", [(0, 0, 6144), (1, 1, 13056)])
def test_stream256_counts_and_samples_alone(hip, admit_order, ffn_bf16, batch_frames):
    """The continuous-batching stream: 256 requests (clips lognormal, median
    6 s, in [1, 30] s; limits U[8, 256]), 64 slots, 16 spare prompt rows,
    encoding overlapped with decoding in batches of 6144 or 13056 frames.  Every
    request yields exactly its limit; four requests (the longest clip, the
    longest limit, the last submitted, one more) rerun alone give the same
    tokens and chosen-logit bits.  In submission order with the fp32-accurate
    encoder, and with the benchmark's own settings: largest token budget
    first, the single-pass FFN encoder, batches of 13056 frames (51 row tiles
    of 256)."""
    m = model(hip, 2)
    rng = np.random.default_rng(3)
    secs = np.clip(np.exp(rng.normal(np.log(6.0), 0.5, 256)), 1.0, 30.0)
    samples = (secs * cb.SR).astype(np.int64)
    limits = rng.integers(8, 257, 256)
    pcms = [cb.synth_audio(int(n), 1000 + i) for i, n in enumerate(samples)]
    eng = cb.Engine(m, slots=64, max_requests=256, max_frames=376, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 256, prefill_rows=16, admit_order=admit_order,
                    enc_ffn_bf16=ffn_bf16)
    try:
        for p, lim in zip(pcms, limits):
            eng.submit_pcm(p, int(lim), cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS)
        steps = eng.process(max_batch_frames=batch_frames, chunk=8)
        assert eng.finished() == 256
        toks = [eng.tokens(r) for r in range(256)]
        sample = sorted({int(np.argmax(samples)), int(np.argmax(limits)), 255, 100})
        scores = {r: eng.scores(r) for r in sample}
        print(f"case: stream of 256, admit_order {admit_order}, ffn_bf16 {ffn_bf16}: {steps} steps",
              flush=True)
    finally:
        eng.close()
    assert [len(t) for t in toks] == [int(x) for x in limits]
    assert all(t[-1] == cb.EOS for t in toks)
    for r in sample:
        compare_alone(m, pcms[r], int(limits[r]), 16, toks[r], scores[r], None, 376,
                      f"stream request {r} ({secs[r]:.1f} s, {limits[r]} tokens) alone", ffn_bf16)
