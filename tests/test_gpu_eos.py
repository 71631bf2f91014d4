"""Retirement under the reference's own rules — needs an MI355X.

transcribe.c:789 retires a sequence when it emits EOS (id 3) or reaches its
length cap; the chunk loop (transcribe.c:375-387, 510-529) carries the last
<= 64 generated ids of a chunk, without its final one, into the next chunk's
prompt.  Here no request suppresses EOS (flags 0), on the decoder-hot
weights with the LM head's EOS bias raised to 2.375, which makes greedy
decoding stop by itself after 1 to 9 tokens on these clips.  The engine uses
fp32 KV caches so the oracle it is compared with is the reference CPU path's
own arithmetic (the closest top-1/top-2 logit gap on these decodes is 1.4%,
the engine's logit error ~1e-5).
"""
import numpy as np
import pytest

import ctbind as cb
import oracle_bind as ob
from test_gpu_engine import CLIPS, SPLIT, long_recording

pytestmark = pytest.mark.gpu

EOS_BIAS = 2.375
NATURAL = 0          # no suppression, no forced EOS


@pytest.fixture(scope="module")
def eos_model(hip):
    m = cb.SynthModel(seed=5, variant=2)
    m.set_bf16("hdb", cb.EOS, EOS_BIAS)
    hip.backend_weights_upload_blob(m.data_ptr, m.data_bytes)
    return m


@pytest.fixture(scope="module")
def eos_mels():
    return [ob.compute_mel(cb.synth_audio(n, s)) for n, s in CLIPS]


def test_natural_eos_and_cap_retirement(hip, eos_model, eos_mels):
    """Four requests through two slots: one whose first token is EOS, two
    that stop on EOS after 4 and 8 tokens, one that reaches its limit of 3
    first.  Tokens equal the oracle's; each request leaves its slot right
    after the step that produced its last token and the freed slot takes the
    next request at the next step (checked step by step)."""
    reqs = [(0, 12), (1, 12), (2, 12), (2, 3)]          # (clip, limit)
    want = [ob.transcribe(eos_model, eos_mels[c], lim, suppress=False, force=False)[0]
            for c, lim in reqs]
    print("case: oracle tokens", [w.tolist() for w in want], flush=True)
    assert len(want[0]) == 1 and want[0][0] == cb.EOS           # EOS first
    assert want[1][-1] == cb.EOS and want[2][-1] == cb.EOS      # natural stops
    assert len(want[3]) == 3 and cb.EOS not in want[3]          # limit reached first
    npr, S = len(cb.PROMPT), 2
    eng = cb.Engine(eos_model, slots=S, max_requests=8, max_frames=64, kv_bf16=False, prefill_rows=0)
    try:
        for c, lim in reqs:
            eng.submit(eos_mels[c], lim, NATURAL)
        eng.encode()
        slots, left, waiting = [None] * S, {}, list(range(len(reqs)))
        for step in range(100):
            for s in range(S):
                if slots[s] is None and waiting:
                    r = waiting.pop(0)
                    slots[s], left[r] = r, npr + len(want[r]) - 1
            for s in range(S):
                if slots[s] is not None:
                    left[slots[s]] -= 1
                    if left[slots[s]] == 0:
                        slots[s] = None
            eng.step()
            for r in range(len(reqs)):
                exp = slots.index(r) if r in slots else -1
                assert eng.slot_of(r) == exp, (step, r)
            if not waiting and all(x is None for x in slots):
                break
        assert eng.finished() == len(reqs)
        for r, w in enumerate(want):
            assert np.array_equal(eng.tokens(r), w), (r, eng.tokens(r), w)
    finally:
        eng.close()


REC_SEED = 7
CHAIN_LIMIT = 8


@pytest.mark.parametrize("prefill_rows", [0, 8])
def test_chained_chunks_with_natural_eos(hip, eos_model, eos_mels, prefill_rows):
    """A recording's chunks stop on EOS by themselves (one after its first
    token); each successor's prompt carries its predecessor's ids without the
    final EOS.  With a plain request beside them on two slots, the engine's
    tokens equal the oracle's chunk-by-chunk decode."""
    rec = long_recording(REC_SEED)
    ref = ob.transcribe_chunked(eos_model, rec, CHAIN_LIMIT, suppress=False, force=False, **SPLIT)
    print("case: oracle chunks", [(len(p), t.tolist()) for _, p, t in ref], flush=True)
    assert len(ref) >= 3
    assert all(t[-1] == cb.EOS and len(t) < CHAIN_LIMIT for _, _, t in ref)
    assert any(len(t) > 1 for _, _, t in ref) and any(len(t) == 1 for _, _, t in ref)
    plain_want = ob.transcribe(eos_model, eos_mels[2], 12, suppress=False, force=False)[0]
    eng = cb.Engine(eos_model, slots=2, max_requests=16, max_frames=64, kv_bf16=False,
                    max_tokens=len(cb.PROMPT) + 64 + 12, prefill_rows=prefill_rows)
    try:
        ids = eng.submit_pcm_chunked(rec, CHAIN_LIMIT, NATURAL, **SPLIT)
        plain = eng.submit(eos_mels[2], 12, NATURAL)
        eng.encode(max_batch_frames=64)
        eng.run(chunk=2)
        assert eng.finished() == len(ids) + 1
        assert np.array_equal(eng.tokens(plain), plain_want)
        assert len(ids) == len(ref)
        for r, (_, _, toks) in zip(ids, ref):
            assert np.array_equal(eng.tokens(r), toks), (r, eng.tokens(r), toks)
    finally:
        eng.close()
