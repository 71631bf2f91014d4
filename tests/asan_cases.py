"""Checks of the host C run by tests/test_sanitize.py in a child process
whose host libraries are the AddressSanitizer + UndefinedBehaviorSanitizer
builds (CT_HOST_LIB, CT_CHUNK_LIB).  Not collected by the default run: the
parent names this file explicitly.  Expected digests come from the normal
builds, computed by the parent (CT_ASAN_EXPECT, JSON)."""
import hashlib
import json
import os

import numpy as np

import ctbind as cb

EXPECT = json.loads(os.environ.get("CT_ASAN_EXPECT", "{}"))


def digests():
    """Digests of what the synthetic-workload generator writes: the weight
    image of variant 1 (perturbed affine terms), its bound Weights struct's
    offsets, three clips and the counter-based generator."""
    m = cb.SynthModel(seed=77, variant=1, nthreads=8)
    out = {"image": hashlib.blake2b(memoryview(m.image), digest_size=16).hexdigest()}
    base = m.image.ctypes.data
    raw = bytes(m.W)
    ptrs = np.frombuffer(raw[:len(raw) // 8 * 8], np.uint64).astype(np.int64)
    inside = ptrs[(ptrs >= base) & (ptrs < base + m.image.nbytes)]
    out["weights_bound"] = int(inside.size)
    out["weights_offsets"] = hashlib.blake2b((inside - base).tobytes(), digest_size=16).hexdigest()
    del m
    clips = [cb.synth_audio(n, s) for n, s in ((160, 1), (16000, 2), (123457, 3))]
    out["audio"] = hashlib.blake2b(b"".join(c.tobytes() for c in clips), digest_size=16).hexdigest()
    L = cb.host()
    hv = [L.ct_hash64(k, i) for k in (0, 1, 2**63 + 5) for i in (0, 1, 999, 2**40)]
    out["hash64"] = hashlib.blake2b(np.asarray(hv, np.uint64).tobytes(), digest_size=16).hexdigest()
    nv = [L.ct_normal16(h) for h in hv]
    out["normal16"] = hashlib.blake2b(np.asarray(nv, np.float32).tobytes(), digest_size=16).hexdigest()
    return out


def test_synth_matches_normal_build():
    got = digests()
    assert got == EXPECT, (got, EXPECT)
    assert got["weights_bound"] > 100


def test_sanitizer_builds_are_loaded():
    """The child really runs the instrumented libraries: the ASan runtime and
    both sanitizer builds are mapped into this process once used."""
    cb.host()
    cb.chunk_bounds(np.zeros(3200, np.float32))
    maps = open("/proc/self/maps").read()
    assert "libasan" in maps
    assert os.environ["CT_HOST_LIB"] in maps and cb.HOST_LIB == os.environ["CT_HOST_LIB"]
    assert os.environ["CT_CHUNK_LIB"] in maps
