"""Long-audio chunking (transcribe.c:397-535) on the host — no GPU needed.

The oracle's splitter is pinned by closed forms: recordings built from 10 ms
frames of known RMS (zeros, constants, one full period of a 100 Hz sine per
frame) whose quiet runs sit at chosen frames, so the cut points (midpoints
of qualifying runs, in samples), the target merging and the automatic
threshold ((5th-percentile bucket / 1024) * 10) follow by hand.  The
engine's splitter (hipb_chunk_bounds in libct_hip.so, host code) must then
give the same boundaries as the oracle on randomized recordings, bit for
bit (integer sample indices).
"""
import numpy as np
import pytest

import ctbind as cb
import oracle_bind as ob

HOP = 160
NAN = float("nan")


def frames(spec):
    """spec: list of (kind, n_frames); kind 'loud' = one 100 Hz period per
    frame at amplitude 0.3 (RMS 0.212), 'zero', or a float constant."""
    t = np.arange(HOP, dtype=np.float64)
    loud = (0.3 * np.sin(2 * np.pi * t / HOP)).astype(np.float32)
    parts = []
    for kind, n in spec:
        if kind == "loud":
            f = loud
        elif kind == "zero":
            f = np.zeros(HOP, np.float32)
        else:
            f = np.full(HOP, kind, np.float32)
        parts.append(np.tile(f, n))
    return np.concatenate(parts)


LAYOUT = [("loud", 50), ("zero", 30), ("loud", 50), ("zero", 5), ("loud", 65), ("zero", 60),
          ("loud", 40), ("zero", 20)]          # 320 frames; the last quiet run reaches the end


@pytest.mark.parametrize("target,expect", [
    (0.0, [65 * HOP, 230 * HOP]),     # both qualifying runs (30 and 60 frames >= 20) cut
    (1.0, [230 * HOP]),               # 10400 - 0 < 16000: merged into the next chunk
    (3.0, []),                        # no cut 48000 samples past the start
])
def test_oracle_cuts_closed_form(target, expect):
    x = frames(LAYOUT)
    b = ob.chunk_bounds(x, silence_db=-30.0, silence_dur=0.2, target_sec=target)
    edges = [0] + expect + [len(x)]
    assert b == list(zip(edges[:-1], edges[1:]))


def test_oracle_min_run_and_trailing_partial_frame():
    # runs of exactly 20 frames qualify, 19 do not (dur 0.2 s); 100 extra
    # samples past the last whole frame belong to the last chunk
    x = np.concatenate([frames([("loud", 30), ("zero", 20), ("loud", 30), ("zero", 19), ("loud", 30)]),
                        np.zeros(100, np.float32)])
    b = ob.chunk_bounds(x, silence_db=-30.0, silence_dur=0.2, target_sec=0.0)
    assert b == [(0, 40 * HOP), (40 * HOP, len(x))]


def test_oracle_auto_threshold_closed_form():
    # quiet frames of constant 0.01 (RMS 0.01 -> bucket 10) make up 90 of 320
    # frames (> 5%): threshold (10/1024)*10 = 0.0977 separates them from the
    # sine frames (RMS 0.212), so the cuts equal the explicit-threshold ones
    lay = [(0.01 if k == "zero" else k, n) for k, n in LAYOUT]
    x = frames(lay)
    assert ob.chunk_bounds(x, silence_db=NAN, silence_dur=0.2, target_sec=0.0) == \
        ob.chunk_bounds(frames(LAYOUT), silence_db=-30.0, silence_dur=0.2, target_sec=0.0)
    # quiet frames under 5%: the 5th percentile falls in the sine frames'
    # bucket (217), threshold 2.12 > every RMS, one quiet run to the end, no cut
    y = frames([("loud", 150), (0.01, 5), ("loud", 150)])
    assert ob.chunk_bounds(y, silence_db=NAN, silence_dur=0.2, target_sec=0.0) == [(0, len(y))]
    # a 0 dB threshold is 1.0: everything is quiet, again a single chunk
    assert ob.chunk_bounds(x, silence_db=0.0, silence_dur=0.2, target_sec=0.0) == [(0, len(x))]


def test_oracle_short_inputs():
    assert ob.chunk_bounds(np.zeros(100, np.float32)) == [(0, 100)]
    assert ob.chunk_bounds(np.zeros(0, np.float32)) == []


def _random_recording(rng):
    segs = []
    for _ in range(rng.integers(3, 12)):
        n = int(rng.integers(1, 400))
        if rng.random() < 0.5:
            segs.append((rng.standard_normal(n * HOP) * rng.uniform(0.05, 0.4)).astype(np.float32))
        else:
            segs.append((rng.standard_normal(n * HOP) * rng.uniform(0.0, 0.01)).astype(np.float32))
    x = np.concatenate(segs + [np.zeros(int(rng.integers(0, HOP)), np.float32)])
    return x


def test_engine_splitter_matches_oracle():
    rng = np.random.default_rng(31)
    cases = 0
    for i in range(40):
        x = _random_recording(rng)
        db = NAN if i % 3 == 0 else float(rng.uniform(-60, -15))
        dur = float(rng.choice([0.05, 0.1, 0.2, 0.5]))
        target = float(rng.choice([0.0, 0.5, 1.0, 2.0, 20.0]))
        got = cb.chunk_bounds(x, silence_db=db, silence_dur=dur, target_sec=target)
        ref = ob.chunk_bounds(x, silence_db=db, silence_dur=dur, target_sec=target)
        assert got == ref, (i, db, dur, target)
        cases += len(ref) > 1
    assert cases >= 10          # most recordings do get cut
    # chunks tile the recording
    x = _random_recording(rng)
    b = cb.chunk_bounds(x, silence_db=-30.0, silence_dur=0.1, target_sec=0.0)
    assert b[0][0] == 0 and b[-1][1] == len(x)
    assert all(b[i][1] == b[i + 1][0] for i in range(len(b) - 1))
