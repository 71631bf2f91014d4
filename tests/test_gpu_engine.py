"""GPU parity of the decode engine (include/hipb.h) — needs an MI355X.

The engine feeds the prompt one token per step through the decode kernels,
keeps KV caches head-major on the device and admits requests into freed
slots by itself.  Checks:
  * token ids identical to the oracle's greedy decode under the forced-length
    policy, with fp32 KV and with bf16 KV (the oracle rounds its K/V to bf16
    the same way); the decoder-hot weight variant makes the ids
    input-dependent with near-ties;
  * encoder output within 1e-4 (||.||_inf relative) of the oracle;
  * every step's logits of a request bit-identical whether it runs alone
    (1 slot) or packed with others;
  * continuous batching: more requests than slots, all finish, same tokens.
"""
import numpy as np
import pytest

import ctbind as cb
import oracle_bind as ob

pytestmark = pytest.mark.gpu

CLIPS = [(4000, 101), (7200, 102), (5600, 103)]
LIMITS = [6, 9, 4]
FLAGS = cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.fixture(scope="module")
def hot(hip):
    m = cb.SynthModel(seed=5, variant=2)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    return m


@pytest.fixture(scope="module")
def mels():
    return [ob.compute_mel(cb.synth_audio(n, s)) for n, s in CLIPS]


@pytest.fixture(scope="module")
def oracle_runs(hot, mels):
    out = {}
    for kvb in (False, True):
        for i, mel in enumerate(mels):
            out[(kvb, i)] = ob.transcribe(hot, mel, LIMITS[i], suppress=True, force=True,
                                          kv_bf16=kvb)
    return out


@pytest.mark.parametrize("kv_bf16", [False, True])
def test_engine_matches_oracle(hip, hot, mels, oracle_runs, kv_bf16):
    print(f"case: engine vs oracle, kv_bf16={kv_bf16}", flush=True)
    eng = cb.Engine(hot, slots=4, max_requests=8, max_frames=64, kv_bf16=kv_bf16)
    try:
        ids = [eng.submit(mel, LIMITS[i], FLAGS) for i, mel in enumerate(mels)]
        eng.encode()
        steps = eng.run(chunk=4)
        assert eng.finished() == len(ids)
        for i, r in enumerate(ids):
            toks, _, enc_h = oracle_runs[(kv_bf16, i)]
            got = eng.tokens(r)
            print(f"  req {i}: engine {got.tolist()} oracle {toks.tolist()}")
            assert np.array_equal(got, toks), i
            assert relerr(eng.enc_out(r), enc_h) <= 1e-4, i
        assert steps >= len(cb.PROMPT) + max(LIMITS) - 1
    finally:
        eng.close()


def run_stepwise(eng, n_req, max_steps=64):
    """Steps an engine whose requests all fit in slots; returns per request
    the list of logits rows (one per step while it is in a slot)."""
    hist = {r: [] for r in range(n_req)}
    for _ in range(max_steps):
        eng.step()
        for r in range(n_req):
            s = eng.slot_of(r)
            if s >= 0:
                hist[r].append(eng.logits(s))
        if eng.finished() == n_req:
            break
    return hist


@pytest.mark.parametrize("admit_order", [0, 1])
def test_engine_admission_order(hip, hot, mels, admit_order):
    """Admission follows the policy step by step: before each step the free
    slots, in slot order, take the waiting requests in submission order (or,
    with admit_order 1, largest token budget first, ties in submission
    order); a request then holds its slot for len(prompt) + limit - 1 steps
    (one prompt id a step, the last one yielding the first token) and frees
    it after the step that generates its limit-th token.  Checked against a
    host model of that policy after every step, with more requests than
    slots."""
    limits = [3, 7, 2, 5, 4, 1, 6, 7]
    n, S, npr = len(limits), 3, len(cb.PROMPT)
    eng = cb.Engine(hot, slots=S, max_requests=n, max_frames=64, kv_bf16=True, prefill_rows=0,
                    admit_order=admit_order)
    try:
        for i, lim in enumerate(limits):
            eng.submit(mels[i % len(mels)], lim, FLAGS)
        eng.encode()
        waiting = sorted(range(n), key=lambda r: (-limits[r], r)) if admit_order else list(range(n))
        slots, left = [None] * S, {}
        for step in range(200):
            for s in range(S):
                if slots[s] is None and waiting:
                    r = waiting.pop(0)
                    slots[s], left[r] = r, npr + limits[r] - 1
            for s in range(S):
                if slots[s] is not None:
                    left[slots[s]] -= 1
                    if left[slots[s]] == 0:
                        slots[s] = None
            want = {r: s for s, r in enumerate(slots) if r is not None}
            eng.step()
            got = {r: eng.slot_of(r) for r in range(n)}
            print(f"case: step {step} slots {slots}", flush=True)
            for r in range(n):
                assert got[r] == want.get(r, -1), (step, r, got[r], want.get(r, -1))
            if not waiting and all(x is None for x in slots):
                break
        assert eng.finished() == n
        for r, lim in enumerate(limits):
            assert len(eng.tokens(r)) == lim, r
    finally:
        eng.close()


@pytest.mark.parametrize("slots,max_tokens", [(128, 512), (256, 1024)])
def test_engine_scheduling_knobs_keep_bits(hip, hot, monkeypatch, slots, max_tokens):
    """Dealing attention items to compute units by length rank (steps of at
    least HIPB_RANK_MIN_ROWS rows) and the weight read-ahead workgroups change
    only where work runs: one step over 128 slots at the microbench's shapes
    (S ~ U(1,448), T_enc ~ U(25,375), seeded bf16 caches), and over the
    largest engine (256 slots, 1024-token caches, S up to 960), gives the
    same logits bits with each of them off.  A rank table that skipped or
    repeated an item would leave some slot's attention output stale."""
    rng = np.random.default_rng(21)
    S, T = rng.integers(1, max_tokens - 63, slots), rng.integers(25, 376, slots)
    outs = []
    for rank_min, read_ahead in (("96", "1"), ("100000", "1"), ("96", "0")):
        print(f"case: {slots} slots, rank from {rank_min} rows, read-ahead {read_ahead}", flush=True)
        monkeypatch.setenv("HIPB_RANK_MIN_ROWS", rank_min)
        monkeypatch.setenv("HIPB_READ_AHEAD", read_ahead)
        eng = cb.Engine(hot, slots=slots, max_requests=slots, max_frames=376, kv_bf16=True,
                        max_tokens=max_tokens)
        try:
            eng.bench_fill(S, T, seed=9)
            eng.step()
            outs.append(np.stack([eng.logits(s) for s in range(slots)]))
        finally:
            eng.close()
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))


def test_engine_eager_launches_equal_graph_replay(hip, hot, mels, monkeypatch):
    """HIPB_EAGER=1 (the mode every profile is taken in) launches each step's
    kernels one by one instead of replaying the captured graphs; a run of
    three requests on 2 slots with 2 spare prompt rows (the narrow and the
    wide step both) gives the same tokens and chosen-logit bits either way."""
    runs = []
    for eager in ("0", "1"):
        print(f"case: HIPB_EAGER={eager}", flush=True)
        monkeypatch.setenv("HIPB_EAGER", eager)
        eng = cb.Engine(hot, slots=2, max_requests=4, max_frames=64, kv_bf16=True,
                        max_tokens=len(cb.PROMPT) + max(LIMITS), prefill_rows=2)
        try:
            for i, mel in enumerate(mels):
                eng.submit(mel, LIMITS[i], FLAGS)
            eng.encode()
            eng.run(chunk=2)
            assert eng.finished() == len(mels)
            runs.append([(eng.tokens(r), eng.scores(r)) for r in range(len(mels))])
        finally:
            eng.close()
    for (ta, sa), (tb, sb) in zip(*runs):
        assert np.array_equal(ta, tb)
        assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))


def test_engine_128_slot_step_rows_independent(hip, hot):
    """The decode-step microbench shape: 128 slots, self lengths U(1, 448),
    encoder lengths U(25, 375), bf16 K/V filled from a seeded hash of each
    element's index (hipb_bench_fill), one step.  A slot's logits are the same
    bits whatever lengths the other 127 slots have.  At 128 rows the
    attention deals its items by length rank, so the launch position of the
    probed items moves between the two runs.  The logits are finite and
    differ from slot to slot."""
    rng = np.random.default_rng(31)
    B = 128
    S, T = rng.integers(1, 449, B), rng.integers(25, 376, B)
    S2, T2 = rng.integers(1, 449, B), rng.integers(25, 376, B)
    probe = [0, 5, 63, 64, 100, 127]
    S2[probe], T2[probe] = S[probe], T[probe]
    runs = []
    for run, (s_, t_) in enumerate(((S, T), (S2, T2))):
        print(f"case: 128-slot step, lengths set {run}", flush=True)
        eng = cb.Engine(hot, slots=B, max_requests=B, max_frames=376, kv_bf16=True, max_tokens=512)
        try:
            eng.bench_fill(s_, t_, seed=9)
            eng.step()
            runs.append(np.stack([eng.logits(slot) for slot in range(B)]))
        finally:
            eng.close()
    a, b = runs
    assert np.isfinite(a).all() and np.isfinite(b).all()
    assert np.abs(a - a[0]).max() > 0.0
    def rank(L):
        # position in the device's ranking: descending length, ties by row
        rows = np.arange(B)
        return np.array([np.sum((L > L[r]) | ((L == L[r]) & (rows < r))) for r in rows])
    moved = [p for p in probe if rank(S)[p] != rank(S2)[p]]
    print(f"  probed slots {probe}, self-length rank moved for {moved}")
    assert moved
    for p in probe:
        assert np.array_equal(a[p].view(np.uint32), b[p].view(np.uint32)), p


def test_engine_batch_vs_single_bitexact(hip, hot, mels):
    packed = cb.Engine(hot, slots=4, max_requests=8, max_frames=64, kv_bf16=True)
    try:
        for i, mel in enumerate(mels):
            packed.submit(mel, LIMITS[i], FLAGS)
        packed.encode()
        hp = run_stepwise(packed, len(mels))
        tp = [packed.tokens(r) for r in range(len(mels))]
    finally:
        packed.close()
    for i, mel in enumerate(mels):
        print(f"case: request {i} alone vs packed", flush=True)
        alone = cb.Engine(hot, slots=1, max_requests=1, max_frames=64, kv_bf16=True)
        try:
            alone.submit(mel, LIMITS[i], FLAGS)
            alone.encode()
            ha = run_stepwise(alone, 1)
            assert np.array_equal(alone.tokens(0), tp[i])
        finally:
            alone.close()
        # the packed run reports the last step's logits after the slot is
        # freed; compare the steps both runs observed
        n = min(len(ha[0]), len(hp[i]))
        assert n >= len(cb.PROMPT)
        for k in range(n):
            assert np.array_equal(ha[0][k].view(np.uint32), hp[i][k].view(np.uint32)), (i, k)


@pytest.mark.parametrize("kv_bf16", [False, True])
def test_engine_logits_match_oracle(hip, hot, mels, kv_bf16):
    """Logits behind every generated token, engine (4 slots, ragged) vs the
    oracle in the same KV mode: max relative error per row within the
    specified 1e-2, and with fp32 KV within a regression bound of 1e-4
    (measured 4e-5: split-bf16 activations, fp32 accumulation).  With bf16
    KV two correct implementations differ by ~4e-3 on these decoder-hot
    weights: an element whose fp32 value lies within rounding noise of a bf16
    rounding boundary rounds the other way, and the flips cascade."""
    eng = cb.Engine(hot, slots=4, max_requests=8, max_frames=64, kv_bf16=kv_bf16)
    try:
        for i, mel in enumerate(mels):
            eng.submit(mel, LIMITS[i], FLAGS)
        eng.encode()
        hist = run_stepwise(eng, len(mels))
    finally:
        eng.close()
    npr = len(cb.PROMPT)
    worst = 0.0
    for i, mel in enumerate(mels):
        print(f"case: logits of request {i}, kv_bf16={kv_bf16}", flush=True)
        toks, lg, _ = ob.transcribe(hot, mel, LIMITS[i], suppress=True, force=True, kv_bf16=kv_bf16,
                                    want_logits=True)
        # step npr-1+j produced generated token j; the last one is read after
        # the slot was freed, so it is not in the history
        n = min(len(hist[i]) - (npr - 1), len(toks))
        assert n >= len(toks) - 1 >= 1
        for j in range(n):
            e = relerr(hist[i][npr - 1 + j], lg[j])
            worst = max(worst, e)
            assert e <= 1e-2, (i, j, e)
    print(f"  worst logits relerr {worst:.2e}")
    if not kv_bf16:
        assert worst <= 1e-4


def test_engine_continuous_batching(hip, hot, mels, oracle_runs):
    """Six requests through two slots: freed slots are refilled on device."""
    # self caches sized to the longest request (max_tokens)
    eng = cb.Engine(hot, slots=2, max_requests=8, max_frames=64, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + max(LIMITS))
    order = [0, 1, 2, 2, 0, 1]
    try:
        for i in order:
            eng.submit(mels[i], LIMITS[i], FLAGS)
        eng.encode(max_batch_frames=8)       # several encoder batches
        eng.run(chunk=3)
        assert eng.finished() == len(order)
        for r, i in enumerate(order):
            assert np.array_equal(eng.tokens(r), oracle_runs[(True, i)][0]), (r, i)
    finally:
        eng.close()


def test_gpu_mel_matches_oracle(hip, hot):
    """GPU log-mel (exact twiddles, one FFT per workgroup) vs the oracle's
    restatement of transcribe.c:177-214 (recurrence twiddles)."""
    eng = cb.Engine(hot, slots=1, max_requests=2, max_frames=400, kv_bf16=True)
    try:
        for n, seed in ((16000 + 37, 9), (160 * 7, 10), (8 * 16000, 11)):
            x = cb.synth_audio(n, seed)
            got = eng.mel(x)
            ref = ob.compute_mel(x)
            print(f"case: mel n={n} max abs err {np.abs(got - ref).max():.2e}", flush=True)
            assert got.shape == ref.shape
            assert np.abs(got - ref).max() < 2e-3
    finally:
        eng.close()


def test_engine_pcm_path(hip, hot, oracle_runs):
    """PCM submitted (host and device-resident) -> GPU mel -> same tokens as
    the oracle fed the oracle's mel."""
    eng = cb.Engine(hot, slots=2, max_requests=4, max_frames=64, kv_bf16=True)
    try:
        for i, (n, s) in enumerate(CLIPS):
            eng.submit_pcm(cb.synth_audio(n, s), LIMITS[i], FLAGS)
        eng.encode()
        eng.run(chunk=2)
        for i in range(len(CLIPS)):
            assert np.array_equal(eng.tokens(i), oracle_runs[(True, i)][0]), i
    finally:
        eng.close()


# four short clips packed into ~300 rows, and 23 clips of ~20 s plus one of
# 30 s (the longest, 376 encoder frames) packed into ~6100 rows, where the FFN
# projections take the 256-row tile kernel while each clip alone (<= 376
# rows) takes the 128-row one
# "long": recordings of 60 s and 2 min left unchunked (751 and 1501 encoder
# frames) beside a 5 s clip, in an engine sized for 2048 frames
ENC_CLIPS = {"small": [(4000, 101), (33000, 104), (7200, 102), (161 * 160, 105)],
             "large": [(320000 + 1600 * i, 200 + i) for i in range(23)] + [(480000, 230)],
             "long": [(960000, 301), (1920000, 302), (80000, 303)]}


@pytest.mark.parametrize("batch", ["small", "large", "long"])
def test_packed_encoder_bitexact_vs_abi_encoder(hip, hot, batch):
    """The engine's packed encoder (pre-split activations, DMA-fed GEMM,
    ragged attention/conv kernels) gives the same bits per request as the
    reference host graph (model.h encoder_forward) driving the ABI one clip
    at a time: every kernel pair runs the same per-element arithmetic."""
    import ctypes as C
    import os
    path = os.path.join(ob.REF_DIR, "libref_model_hip.so")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref/libref_model_hip.so not built")
    ref = C.CDLL(path)
    ref.ref_set_weights.argtypes = [C.c_void_p]
    ref.ref_encoder.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    ref.ref_set_weights(hot.weights_ref())
    mels = [ob.compute_mel(cb.synth_audio(n, s)) for n, s in ENC_CLIPS[batch]]
    eng = cb.Engine(hot, slots=2, max_requests=len(mels), max_frames=2048 if batch == "long" else 400,
                    kv_bf16=True)
    try:
        for m in mels:
            eng.submit(m, 2, FLAGS)
        eng.encode(max_batch_frames=8192)     # one packed batch
        for i, m in enumerate(mels):
            want = np.zeros((cb.t_enc(m.shape[1]), cb.DEC_D), np.float32)
            ref.ref_encoder(m.ctypes.data, m.shape[1], want.ctypes.data)
            got = eng.enc_out(i)
            print(f"case: clip {i} T_enc={got.shape[0]} max diff {np.abs(got - want).max():.3g}", flush=True)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
    finally:
        eng.close()


def long_recording(seed, n_seg=4, seg=5600, gap=1600):
    """Speech-like segments (cb.synth_audio) separated by 0.1 s of low noise."""
    rng = np.random.default_rng(seed)
    parts = []
    for i in range(n_seg):
        parts.append(cb.synth_audio(seg + 160 * i, seed * 10 + i))
        parts.append((rng.standard_normal(gap) * 0.002).astype(np.float32))
    return np.concatenate(parts[:-1])


SPLIT = dict(silence_db=-40.0, silence_dur=0.05, target_sec=0.2)
CHUNK_LIMIT = 5
# Recordings whose chunk decodes have no near-tie: the oracle's best and
# second-best logit differ by > 1e-3 relative at every chosen token (ties
# closer than the engine-vs-oracle logit error, ~1e-4, may go either way).
REC_SEEDS = (2, 14)


@pytest.fixture(scope="module")
def chunked_oracle(hot):
    out = {}
    for s in REC_SEEDS:
        runs = ob.transcribe_chunked(hot, long_recording(s), CHUNK_LIMIT, suppress=True, force=True,
                                     kv_bf16=True, want_logits=True, **SPLIT)
        for _, _, toks, lg in runs:
            for i in range(len(toks) - 1):          # the last token is the forced EOS
                l = lg[i].astype(np.float64)
                l[3] = -np.inf                      # EOS suppressed
                top = np.sort(l)[::-1]
                assert (top[0] - top[1]) / abs(top[0]) > 1e-3, (s, i)
        out[s] = [r[:3] for r in runs]
    return out


@pytest.mark.parametrize("prefill_rows", [0, 8])
def test_engine_chunked_carry_matches_oracle(hip, hot, mels, oracle_runs, chunked_oracle, prefill_rows):
    """Two long recordings queued as chained chunks plus one plain request on
    two slots: every chunk waits for its predecessor, gets the carried ids in
    its prompt on the device, and decodes to the oracle's tokens (with and
    without spare prompt rows)."""
    eng = cb.Engine(hot, slots=2, max_requests=16, max_frames=64, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 64 + CHUNK_LIMIT, prefill_rows=prefill_rows)
    try:
        a, b = REC_SEEDS
        ids = {}
        ids[a] = eng.submit_pcm_chunked(long_recording(a), CHUNK_LIMIT, FLAGS, **SPLIT)
        plain = eng.submit(mels[0], LIMITS[0], FLAGS)
        ids[b] = eng.submit_pcm_chunked(long_recording(b), CHUNK_LIMIT, FLAGS, **SPLIT)
        eng.encode(max_batch_frames=64)
        eng.run(chunk=4)
        assert eng.finished() == len(ids[a]) + len(ids[b]) + 1
        assert np.array_equal(eng.tokens(plain), oracle_runs[(True, 0)][0])
        for s in REC_SEEDS:
            ref = chunked_oracle[s]
            print(f"case: recording {s}: {len(ref)} chunks, prompts "
                  f"{[len(p) for _, p, _ in ref]}", flush=True)
            assert len(ids[s]) == len(ref) >= 3
            for r, (_, _, toks) in zip(ids[s], ref):
                assert np.array_equal(eng.tokens(r), toks), (s, r)
    finally:
        eng.close()


def test_engine_chunk_equals_request_with_carried_prompt(hip, hot, chunked_oracle):
    """A chained chunk gives the same tokens as the same audio submitted on
    its own with the carried prompt written out on the host."""
    rec = long_recording(REC_SEEDS[0])
    ref = chunked_oracle[REC_SEEDS[0]]
    eng = cb.Engine(hot, slots=3, max_requests=8, max_frames=64, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 64 + CHUNK_LIMIT)
    try:
        rids = [eng.submit_pcm(rec[a:b], CHUNK_LIMIT, FLAGS, prompt=np.asarray(p, np.int32))
                for (a, b), p, _ in ref[1:]]
        eng.encode()
        eng.run(chunk=2)
        for r, (_, _, toks) in zip(rids, ref[1:]):
            assert np.array_equal(eng.tokens(r), toks), r
    finally:
        eng.close()


def test_engine_prefill_rows_bitexact(hip, hot, mels):
    """Spare prompt rows feed a 16-id prompt in 1 step (16 rows) or 4 steps
    (3 rows: 4 ids a step) instead of 16: the generated ids and the logits
    of the last step are the same bits as with one prompt id per step."""
    prompt = np.asarray(list(cb.PROMPT) + [20, 21, 22, 23, 24, 25], np.int32)
    limit = 6
    res = {}
    for P in (0, 3, 16):
        eng = cb.Engine(hot, slots=1, max_requests=1, max_frames=64, kv_bf16=True,
                        max_tokens=len(prompt) + limit, prefill_rows=P)
        try:
            eng.submit(mels[1], limit, FLAGS, prompt=prompt)
            eng.encode()
            steps = 0
            while eng.finished() < 1:
                eng.step()
                steps += 1
                assert steps < 64
            res[P] = (eng.tokens(0), eng.logits(0), steps)
        finally:
            eng.close()
        print(f"case: prefill_rows={P}: {res[P][2]} steps", flush=True)
    assert [res[P][2] for P in (0, 3, 16)] == [16 + limit - 1, 4 + limit - 1, 1 + limit - 1]
    for P in (3, 16):
        assert np.array_equal(res[P][0], res[0][0]), P
        assert np.array_equal(res[P][1].view(np.uint32), res[0][1].view(np.uint32)), P


def test_engine_prefill_rows_continuous_batching(hip, hot, mels, oracle_runs):
    """Six requests through two slots with 5 spare prompt rows (two slots
    compete for them when both admit at once): the oracle's tokens."""
    eng = cb.Engine(hot, slots=2, max_requests=8, max_frames=64, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + max(LIMITS), prefill_rows=5)
    order = [0, 1, 2, 2, 0, 1]
    try:
        for i in order:
            eng.submit(mels[i], LIMITS[i], FLAGS)
        eng.encode()
        steps = eng.run(chunk=1)
        assert eng.finished() == len(order)
        for r, i in enumerate(order):
            assert np.array_equal(eng.tokens(r), oracle_runs[(True, i)][0]), (r, i)
        print(f"case: 6 requests, 2 slots, 5 spare rows: {steps} steps", flush=True)
    finally:
        eng.close()


def test_engine_process_overlapped(hip, hot, mels, oracle_runs, chunked_oracle):
    """hipb_process: encoding (several batches, on its own stream and
    thread) overlapped with decoding; plain and chained requests give the
    oracle's tokens, and a second round on the same engine too."""
    eng = cb.Engine(hot, slots=2, max_requests=24, max_frames=64, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 64 + CHUNK_LIMIT, prefill_rows=4)
    try:
        for rnd in range(2):
            eng.reset()
            order = [0, 1, 2, 2, 0, 1]
            plain = [eng.submit(mels[i], LIMITS[i], FLAGS) for i in order]
            chunks = eng.submit_pcm_chunked(long_recording(REC_SEEDS[1]), CHUNK_LIMIT, FLAGS, **SPLIT)
            steps = eng.process(max_batch_frames=64, chunk=2)
            print(f"case: process round {rnd}: {len(plain)} + {len(chunks)} requests, {steps} steps",
                  flush=True)
            assert eng.finished() == len(plain) + len(chunks)
            for r, i in zip(plain, order):
                assert np.array_equal(eng.tokens(r), oracle_runs[(True, i)][0]), (rnd, r, i)
            for r, (_, _, toks) in zip(chunks, chunked_oracle[REC_SEEDS[1]]):
                assert np.array_equal(eng.tokens(r), toks), (rnd, r)
    finally:
        eng.close()


def test_engine_process_chain_waits_for_its_encoding(hip, hot, mels):
    """A chained chunk whose predecessor retires before the chunk's encoder
    batch is published waits for that batch: a long plain request and the
    first chunk of a recording form encoder batch 0, the second chunk starts
    batch 1, and the encoder thread is held after batch 0 until the first
    chunk has finished.  Tokens equal hipb_encode + hipb_run bit for bit
    (admitting the chunk early would attend over cross K/V not written yet)."""
    rec = long_recording(REC_SEEDS[0])
    bounds = cb.chunk_bounds(rec, **SPLIT)
    assert len(bounds) >= 2
    frames = [cb.t_enc(cb.t_mel(b - a)) for a, b in bounds]
    long_mel = mels[1]
    t_long = cb.t_enc(long_mel.shape[1])
    batch0 = t_long + frames[0]
    assert batch0 + frames[1] > batch0 >= max([t_long] + frames)
    limit_chain, limit_long = 3, 40
    max_frames = max([t_long] + frames)            # tmax <= batch0 keeps the batch cut there

    def submit_all(eng):
        plain = eng.submit(long_mel, limit_long, FLAGS)
        chain = eng.submit_pcm_chunked(rec, limit_chain, FLAGS, **SPLIT)
        return plain, chain

    kw = dict(slots=2, max_requests=16, max_frames=max_frames, kv_bf16=True,
              max_tokens=len(cb.PROMPT) + 64 + limit_long)
    ref = cb.Engine(hot, **kw)
    try:
        plain, chain = submit_all(ref)
        ref.encode()
        ref.run(chunk=1)
        want = [ref.tokens(r) for r in [plain] + chain]
    finally:
        ref.close()
    eng = cb.Engine(hot, **kw)
    try:
        plain, chain = submit_all(eng)
        eng.hold_encoder(1, 1)
        print(f"case: chain {frames} frames, batch 0 = {batch0} frames, hold after batch 0", flush=True)
        eng.process(max_batch_frames=batch0, chunk=1)
        assert not eng.hold_expired()
        assert eng.finished() == 1 + len(chain)
        for r, w in zip([plain] + chain, want):
            assert np.array_equal(eng.tokens(r), w), r
    finally:
        eng.close()


def test_engine_entry_pool_recycles(hip, hot):
    """max_requests bounds the encoder state held at once, not the requests
    that flow through: 8 entries serve 32 requests (4x), among them a long
    recording's chained chunks, on 3 slots, both overlapped (hipb_process)
    and encode-then-run (hipb_run encoding the rest as entries come back).
    Every request yields its limit, and sampled requests, including two
    chunks, give the tokens and chosen-logit bits of the same audio alone."""
    rng = np.random.default_rng(88)
    n_plain, P = 28, 8
    pcms = [cb.synth_audio(int(rng.integers(2400, 12000)), 4000 + i) for i in range(n_plain)]
    limits = [int(x) for x in rng.integers(2, 14, n_plain)]
    rec = long_recording(REC_SEEDS[1])
    kw = dict(slots=3, max_requests=P, max_frames=80, kv_bf16=True,
              max_tokens=len(cb.PROMPT) + 64 + CHUNK_LIMIT + 14, prefill_rows=2)
    runs = {}
    for mode in ("process", "run"):
        eng = cb.Engine(hot, **kw)
        try:
            plain = [eng.submit_pcm(p, lim, FLAGS) for p, lim in zip(pcms[:14], limits[:14])]
            chain = eng.submit_pcm_chunked(rec, CHUNK_LIMIT, FLAGS, **SPLIT)
            plain += [eng.submit_pcm(p, lim, FLAGS) for p, lim in zip(pcms[14:], limits[14:])]
            n = len(plain) + len(chain)
            assert n >= 4 * P
            print(f"case: {n} requests through {P} encoder entries, {mode}", flush=True)
            if mode == "process":
                eng.process(max_batch_frames=40, chunk=2)
            else:
                eng.encode(max_batch_frames=40)
                eng.run(chunk=2)
            assert eng.finished() == n
            runs[mode] = ([eng.tokens(r) for r in plain], [eng.scores(r) for r in plain],
                          [eng.tokens(r) for r in chain], [eng.scores(r) for r in chain])
        finally:
            eng.close()
        toks = runs[mode][0]
        assert [len(t) for t in toks] == limits, mode
        assert all(len(t) == CHUNK_LIMIT for t in runs[mode][2]), mode
    for a, b in zip(runs["process"], runs["run"]):
        for x, y in zip(a, b):
            assert np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32))
    ref = cb.chunk_bounds(rec, **SPLIT)
    for i in (0, 9, 27):
        alone = cb.Engine(hot, slots=1, max_requests=1, max_frames=80, kv_bf16=True,
                          max_tokens=len(cb.PROMPT) + 14)
        try:
            alone.submit_pcm(pcms[i], limits[i], FLAGS)
            alone.encode()
            alone.run(chunk=4)
            assert np.array_equal(alone.tokens(0), runs["process"][0][i]), i
            assert np.array_equal(alone.scores(0).view(np.uint32), runs["process"][1][i].view(np.uint32)), i
        finally:
            alone.close()
    # a chunk alone: its audio with the prompt its predecessor's tokens made
    for c in (1, len(ref) - 1):
        prev = runs["process"][2][c - 1]
        nc = min(len(prev) - 1, 64)
        prompt = list(cb.PROMPT[:2]) + [int(t) for t in prev[len(prev) - 1 - nc:len(prev) - 1]] + list(cb.PROMPT[2:])
        a, b = ref[c]
        alone = cb.Engine(hot, slots=1, max_requests=1, max_frames=80, kv_bf16=True,
                          max_tokens=len(prompt) + CHUNK_LIMIT)
        try:
            alone.submit_pcm(rec[a:b], CHUNK_LIMIT, FLAGS, prompt=np.asarray(prompt, np.int32))
            alone.encode()
            alone.run(chunk=4)
            assert np.array_equal(alone.tokens(0), runs["process"][2][c]), c
            assert np.array_equal(alone.scores(0).view(np.uint32), runs["process"][3][c].view(np.uint32)), c
        finally:
            alone.close()


def test_engine_request_ring_wraps(hip, hot, monkeypatch):
    """The request ring (per-request device fields indexed by id & mask)
    wraps around: with HIPB_RING_MIN=16 the ring of a 2-slot engine holds
    64 requests, and 120 requests flow through it in three waves, so ids
    64..119 reuse the slots of 0..55, whose results move to the host first.
    Every request yields its limit; sampled requests (results collected to
    the host, and still in their slot) give the tokens and chosen-logit bits
    of the same audio alone; a request submitted but not yet uploaded reports
    no tokens (its slot still holds request id - 64's)."""
    monkeypatch.setenv("HIPB_RING_MIN", "16")
    rng = np.random.default_rng(91)
    n, wave = 120, 40
    pcms = [cb.synth_audio(int(rng.integers(2400, 6000)), 7000 + i) for i in range(n)]
    limits = [int(x) for x in rng.integers(2, 7, n)]
    kw = dict(slots=2, max_requests=4, max_frames=40, kv_bf16=True,
              max_tokens=len(cb.PROMPT) + 6, prefill_rows=2)
    eng = cb.Engine(hot, **kw)
    try:
        for w0 in range(0, n, wave):
            ids = [eng.submit_pcm(p, lim, FLAGS) for p, lim in zip(pcms[w0:w0 + wave], limits[w0:w0 + wave])]
            assert ids == list(range(w0, w0 + wave))
            print(f"case: request ring of 64, wave of ids {w0}..{w0 + wave - 1}", flush=True)
            eng.encode(max_batch_frames=64)
            eng.run(chunk=2)
            assert eng.finished() == w0 + wave
        toks = [eng.tokens(r) for r in range(n)]
        sample = (3, 50, 60, 70, 119)
        scores = {r: eng.scores(r) for r in sample}
        extra = eng.submit_pcm(pcms[0], limits[0], FLAGS)
        assert extra == n
        assert len(eng.tokens(extra)) == 0
        assert np.array_equal(eng.tokens(n - 64), toks[n - 64])
    finally:
        eng.close()
    assert [len(t) for t in toks] == limits
    assert all(t[-1] == cb.EOS for t in toks)
    monkeypatch.delenv("HIPB_RING_MIN")
    for r in sample:
        alone = cb.Engine(hot, slots=1, max_requests=1, max_frames=40, kv_bf16=True,
                          max_tokens=len(cb.PROMPT) + 6)
        try:
            alone.submit_pcm(pcms[r], limits[r], FLAGS)
            alone.encode()
            alone.run(chunk=4)
            assert np.array_equal(alone.tokens(0), toks[r]), r
            assert np.array_equal(alone.scores(0).view(np.uint32), scores[r].view(np.uint32)), r
        finally:
            alone.close()


def test_engine_from_c_host_matches_binding(hip):
    """The engine driven from a plain C program (examples/engine_demo.c: its
    own synthetic weights, backend_weights_upload_blob, backend_init,
    hipb_create / hipb_submit_pcm / hipb_encode / hipb_run / hipb_tokens)
    gives every request the tokens the same calls give through this binding
    in this process."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(cb.HIP_LIB), "_build", "engine_demo")
    if not os.path.exists(exe):
        pytest.skip("cohere-transcribe_amd/_build/engine_demo not built")
    seed, variant, n, slots = 4321, 3, 6, 3
    print(f"case: C host, weights seed {seed} variant {variant}, {n} clips on {slots} slots", flush=True)
    r = subprocess.run([exe, str(seed), str(variant), str(n), str(slots)], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    got = {}
    for line in r.stdout.splitlines():
        head, rest = line.split(":")
        vals = [int(v) for v in rest.split()]
        got[int(head.split()[1])] = vals[1:1 + vals[0]]
    assert sorted(got) == list(range(n))
    m = cb.SynthModel(seed=seed, variant=variant)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    eng = cb.Engine(m, slots=slots, max_requests=n, max_frames=376, kv_bf16=True, max_tokens=32,
                    admit_order=1, enc_ffn_bf16=1)
    try:
        flags = cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS
        for i in range(n):
            eng.submit_pcm(cb.synth_audio(8000 + 3000 * i, 500 + i), 4 + 3 * (i % 5), flags)
        eng.encode(max_batch_frames=4096)
        eng.run(chunk=4)
        for i in range(n):
            want = list(eng.tokens(i))
            assert len(want) == 4 + 3 * (i % 5), i
            assert got[i] == want, i
    finally:
        eng.close()
