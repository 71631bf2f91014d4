"""Benchmark: continuous-batching transcription on one MI355X.

Workload (one "step"): the continuous-batching stream of 256 requests —
clip lengths log-normal (median 6 s, sigma 0.5) clipped to [1, 30] s, forced
decode lengths uniform in [8, 256] (EOS suppressed until the limit, then
EOS), at most 64 requests in flight; a freed KV slot is refilled from the
queue on the device, the waiting requests taken largest token budget first
(--admit-order 0: in submission order).  The PCM of all clips is resident in HBM when the timed
region starts; a step runs the GPU log-mel front-end, the packed Conformer
encoder, cross-attention K/V and the decode loop until every request has
finished.  value = audio seconds transcribed per wall second (RTFx).

Random-init weights at the model's dimensions (seeded, the converter's
safetensors layout), seeded synthetic audio; nothing is downloaded.

Also reported, measured live with HIP events on the engine's stream, each
for one kernel family at a fixed shape (launched on its own, so a profiler's
per-kernel averages of `bench.py --roofline-only` can be set beside them):
  rooflines.attention     decode attention (self + cross, bf16 KV) at the
                          128-slot ragged microbench shape (S ~ U(1,448),
                          T_enc ~ U(25,375)): algorithmic K+V bytes per
                          launch / average launch time, against 8 TB/s;
  rooflines.attention_64  the same lengths over 64 slots (a ragged batch
                          of 64);
  rooflines.attention_b64 the same at the stream's own step shape: 64 slots
                          and 16 prompt rows, lengths drawn from the stream's
                          requests;
  rooflines.decode_step_b64  whole decode steps at the stream's shape (64
                          slots, 16 idle spare rows) replayed from the
                          captured graph: weight + K/V bytes per step / step
                          time, against 8 TB/s;
  rooflines.decode_gemm   the 49 decode GEMMs of one step at the stream's 64
                          slots: weight + activation-in + output bytes per
                          launch / average launch time, against 8 TB/s; with
                          the same launches reading their weights alone
                          (read_floor) beside it;
  rooflines.encoder_gemm  the packed encoder's FFN up-projection (M = 16384
                          frames, 1280 -> 5120) in the stream's precision mode
                          (encoder_gemm_split: the fp32-accurate form): 2*M*N*K
                          per launch / time, against the bf16 dense MFMA peak;
  roofline                the one of them whose kernels take the largest
                          share of the stream's GPU time;
  config_runs             the single-clip and uniform-batch configurations
                          end to end on the engine (wall seconds);
  stream_other_ffn_precision  the same stream with the other encoder FFN
                          precision (fp32-accurate hi+lo when the line runs
                          single-pass bf16), one timed pass;
  cpu_baseline            the reference CPU path (its model.h on its CPU
                          backend, compiled from its sources) on the host's
                          cores (one process alone, then one per core of
                          the host's one-GPU share, 16), on a bounded sample
                          extrapolated to this workload's audio/token mix.
HBM traffic per launch (`traffic`) comes from rocprofv3 FETCH_SIZE and
WRITE_SIZE counter runs recorded in profiles/traffic.json, when present.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "cohere-transcribe_amd"))
import ctbind as cb  # noqa: E402

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")
# The kernel family with the largest share of the stream's GPU time (from the
# eager rocprofv3 profile of the stream, encoding not overlapped: decode GEMMs
# 33.8%, the encoder's pre-split GEMMs 25.4%, decode attention 22.2%).
DOMINANT = "decode_gemm"
BF16_PEAK_TFLOPS = 2500.0
# Encoder frames per batch of the overlapped encode/decode (0: encode all,
# then decode).  51 row tiles of 256 frames: every encoder GEMM's width is a
# multiple of 1280 = 5 column tiles of 256, so a batch of 51 row tiles gives
# 255, 510, 765 or 1020 tiles, each just under a whole number of rounds on
# 256 CUs (52 row tiles would start a fifth round of the FFN-up GEMM for 16
# of its 1040 tiles).  Measured on the stream: 10240 -> 4209 RTFx, 11264 ->
# 4295, 12288 -> 4306, 12800 -> 4361, 13056 -> 4364, 13312 -> 4108, 14336 ->
# 4130, 16384 -> 4134, 22528 (one batch) -> 4174.
OVERLAP_BATCH_FRAMES = int(os.environ.get("CT_BENCH_OVERLAP", str(51 * 256)))
METRIC = "audio-sec/sec (RTFx) + decode tokens/s at ragged batch 64; % HBM/MFMA peak"


def make_stream(n_req, seed):
    rng = np.random.default_rng(seed)
    secs = np.clip(np.exp(rng.normal(np.log(6.0), 0.5, n_req)), 1.0, 30.0)
    samples = (secs * cb.SR).astype(np.int64)
    limits = rng.integers(8, 257, n_req)
    return samples, limits


def run_stream(hip, eng, ev, dev_pcm, offs, samples, limits, overlap=OVERLAP_BATCH_FRAMES):
    """One pass of the workload; returns (seconds, decode seconds, steps).
    Overlapped (encoder batches of `overlap` frames beside the decode steps),
    the decode seconds span the whole encode + decode phase."""
    stream = eng.stream()
    eng.reset()
    flags = cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS
    prompt = np.asarray(cb.PROMPT, np.int32)
    ev.sync()
    t0 = time.perf_counter()
    for i in range(len(samples)):
        eng.L.hipb_submit_pcm_device(eng.e, dev_pcm + int(offs[i]) * 4, int(samples[i]),
                                     prompt.ctypes.data, len(prompt), int(limits[i]), flags)
    if overlap:
        # encoder batches on their own stream, published while decoding runs
        t1 = time.perf_counter()
        steps = eng.process(max_batch_frames=overlap, chunk=8)
    else:
        eng.encode(max_batch_frames=24576)
        t1 = time.perf_counter()
        steps = eng.run(chunk=8)
    ev.sync()
    t2 = time.perf_counter()
    del stream
    return t2 - t0, t2 - t1, steps


def config_latency(hip, model, ev, ffn_bf16, reps=3):
    """The single-clip (one 8 s clip, 48 tokens) and uniform-batch (8 x 10 s,
    96 tokens) configurations end to end on the engine, PCM resident in HBM:
    mel, encoder, cross K/V, prompt, decode, one slot per request.  Wall
    seconds per run (mean of `reps` after one warm run), for comparison with
    the reference CPU path's full runs of the same configurations."""
    out = {}
    prompt = np.asarray(cb.PROMPT, np.int32)
    flags = cb.HIPB_SUPPRESS_EOS | cb.HIPB_FORCE_EOS
    for name, secs, n, limit in (("single clip (8 s, 48 tokens)", 8, 1, 48),
                                 ("uniform batch (8 x 10 s, 96 tokens)", 10, 8, 96)):
        pcm = np.concatenate([cb.synth_audio(secs * cb.SR, 800 + i) for i in range(n)])
        dev = hip.backend_arena_alloc(pcm.size)
        hip.backend_htod(dev, pcm.ctypes.data, pcm.size)
        eng = cb.Engine(model, slots=n, max_requests=n, max_frames=376, kv_bf16=True,
                        max_tokens=len(prompt) + limit, prefill_rows=16, enc_ffn_bf16=ffn_bf16)
        try:
            times = []
            for rep in range(reps + 1):
                eng.reset()
                ev.sync()
                t0 = time.perf_counter()
                for i in range(n):
                    eng.L.hipb_submit_pcm_device(eng.e, dev + i * secs * cb.SR * 4, secs * cb.SR,
                                                 prompt.ctypes.data, len(prompt), limit, flags)
                eng.encode(max_batch_frames=24576)
                eng.run(chunk=8)
                ev.sync()
                if rep:
                    times.append(time.perf_counter() - t0)
                if [len(eng.tokens(r)) for r in range(n)] != [limit] * n:
                    raise RuntimeError(f"{name}: a request did not produce {limit} tokens")
        finally:
            eng.close()
            hip.backend_arena_free(dev)
        t = float(np.mean(times))
        out[name] = {"seconds": round(t, 5), "audio_sec_per_sec": round(secs * n / t, 1),
                     "tokens_per_s": round(limit * n / t, 1)}
    return out


def attention_roofline(hip, model, ev, reps=20, step_reps=0, B=128):
    """Decode-attention kernel at the microbench's ragged lengths (S ~
    U(1,448), T_enc ~ U(25,375)) over B slots; with step_reps > 0 also the
    whole decode step at that shape (eager steps)."""
    rng = np.random.default_rng(4)
    S = rng.integers(1, 449, B)
    T = rng.integers(25, 376, B)
    eng = cb.Engine(model, slots=B, max_requests=B, max_frames=376, kv_bf16=True, max_tokens=512)
    step_ms = None
    try:
        eng.bench_fill(S, T, seed=9)
        eng.step()                     # sets per-slot lengths (S after append)
        s = eng.stream()
        a, b = ev.event(), ev.event()
        eng.attention_only()           # warm
        ev.record(a, s)
        for _ in range(reps):
            eng.attention_only()
        ev.record(b, s)
        ms = ev.ms(a, b)
        per_launch_us = ms * 1e3 / (reps * 16)
        S_now = S + 1
        bytes_step = 8 * float(np.sum(2 * (S_now + T) * cb.DEC_D * 2))
        bytes_launch = bytes_step / 16
        if step_reps:
            a2, b2 = ev.event(), ev.event()
            ev.record(a2, s)
            for _ in range(step_reps):
                eng.step()
            ev.record(b2, s)
            step_ms = ev.ms(a2, b2) / step_reps
    finally:
        eng.close()
    achieved = bytes_launch / (per_launch_us * 1e-6) / 1e9
    micro = {"slots": B, "attention_ms_per_step": round(per_launch_us * 16 / 1e3, 3),
             "attention_GBs": round(bytes_step / (per_launch_us * 16e-6) / 1e9, 1)}
    if step_ms is not None:
        micro["step_ms"] = round(step_ms, 3)
    return {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
        "kernel": "attn_kernel<true, true> (decode self + cross attention, bf16 KV)",
        "avg_launch_us": round(per_launch_us, 3), "bytes_per_launch": int(bytes_launch),
        "workload": f"{B} slots, S~U(1,448)+1, T_enc~U(25,375), bf16 KV, 8 layers x (self, cross)",
    }, micro


def stream_rows(samples, limits, n_slots, n_prompt, seed):
    """Self and cross lengths of the rows of one decode step of the stream:
    n_slots slots each holding a random request of the stream part-way
    through its decode (the 10 prompt ids fed, U[0, limit) tokens generated),
    and n_prompt spare rows each feeding a prompt id (position U[1, 10]) of a
    random request.  Returns (S, T_enc): keys before this step's append, and
    encoder frames."""
    rng = np.random.default_rng(seed)
    T_all = np.asarray([cb.t_enc(cb.t_mel(int(n))) for n in samples], np.int64)
    r = rng.integers(0, len(samples), n_slots + n_prompt)
    S = np.empty(n_slots + n_prompt, np.int64)
    S[:n_slots] = len(cb.PROMPT) + rng.integers(0, limits[r[:n_slots]])
    S[n_slots:] = rng.integers(1, len(cb.PROMPT) + 1, n_prompt)
    return S, T_all[r]


def decode_b64(model, ev, samples, limits, reps=20):
    """The decode step at the stream's shape (64 slots, 16 spare prompt
    rows, bf16 K/V, lengths drawn from the stream's requests):
      attention_b64    the 16 decode-attention launches of a step over the
                       64 slots' rows plus 16 prompt rows (80 items, the
                       widest step of the stream), algorithmic K+V bytes per
                       launch / average launch time;
      decode_step_b64  whole decode steps as the stream launches them (the
                       captured wide-step graph, spare rows idle) over the
                       64 slots: weight bytes + K/V bytes per step / step
                       time, against 8 TB/s."""
    smax = len(cb.PROMPT) + 256 + 64           # lengths up to 266 plus the timed steps
    S, T = stream_rows(samples, limits, 64, 16, seed=21)
    eng = cb.Engine(model, slots=80, max_requests=80, max_frames=376, kv_bf16=True, max_tokens=smax)
    try:
        eng.bench_fill(S, T, seed=9)
        eng.step()                             # lengths now S + 1
        s = eng.stream()
        eng.attention_only()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for _ in range(reps):
            eng.attention_only()
        ev.record(b, s)
        att_us = ev.ms(a, b) * 1e3 / (reps * 16)
    finally:
        eng.close()
    # K+V bytes per launch: a layer's self (S + 1 keys) and cross (T_enc) launches
    att_bytes = float(np.sum(2 * (S + 1 + T) * cb.DEC_D * 2)) / 2
    att_gbs = att_bytes / (att_us * 1e-6) / 1e9
    attention = {"bound": "hbm", "achieved": round(att_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                 "frac": round(att_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                 "kernel": "attn_kernel<true, true> (decode self + cross attention, bf16 KV)",
                 "avg_launch_us": round(att_us, 3), "bytes_per_launch": int(att_bytes),
                 "workload": "80 items = 64 slots (S = 10 + U[0, limit) of a random stream request) "
                             "+ 16 prompt rows (S ~ U[1,10]), T_enc of random stream requests "
                             f"(mean S {np.mean(S + 1):.1f}, mean T_enc {np.mean(T):.1f}), bf16 KV, "
                             "8 layers x (self, cross)"}
    S, T = S[:64], T[:64]
    warm = 3
    eng = cb.Engine(model, slots=64, max_requests=64, max_frames=376, kv_bf16=True, max_tokens=smax,
                    prefill_rows=16)
    try:
        eng.bench_fill(S, T, seed=9)
        s = eng.stream()
        eng.bench_steps(warm)
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        eng.bench_steps(reps)
        ev.record(b, s)
        step_us = ev.ms(a, b) * 1e3 / reps
    finally:
        eng.close()
    w_bytes = float(sum(N * K * 2 for N, K in DEC_GEMMS))
    # step i (0-based, counting the warm steps) attends over S + 1 + i self keys
    s_mean = np.mean(S) + 1 + warm + (reps - 1) / 2.0
    kv_bytes = cb.DEC_N * float(np.sum(2 * (s_mean + T) * cb.DEC_D * 2))
    gbs = (w_bytes + kv_bytes) / (step_us * 1e-6) / 1e9
    step = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "whole decode step (captured graph of the wide step)",
            "step_us": round(step_us, 2), "bytes_per_step": int(w_bytes + kv_bytes),
            "weight_bytes": int(w_bytes), "kv_bytes": int(kv_bytes),
            "workload": "64 slots (S = 10 + U[0, limit) of a random stream request, T_enc of that "
                        "request), 16 spare prompt rows idle, bf16 KV"}
    return attention, step


# The decode step's weights (N, K): per layer QKV, out, cross Q, cross out,
# FFN up, FFN down, then the LM head.
DEC_GEMMS = ([(3 * cb.DEC_D, cb.DEC_D), (cb.DEC_D, cb.DEC_D), (cb.DEC_D, cb.DEC_D), (cb.DEC_D, cb.DEC_D),
              (cb.DEC_FF, cb.DEC_D), (cb.DEC_D, cb.DEC_FF)] * cb.DEC_N + [(cb.VOCAB, cb.DEC_D)])


def dec_gemm_launch_bytes(slots):
    """Algorithmic bytes of the step's 49 GEMM launches: weights, input rows
    (fp32-equivalent hi+lo) and output rows (fp32)."""
    return [N * K * 2 + slots * K * 4 + slots * N * 4 for N, K in DEC_GEMMS]


def decode_gemm_roofline(model, ev, slots=64, reps=20):
    """The decode step's GEMM launches alone (8 x QKV, out, cross Q, cross
    out, FFN up, FFN down; LM head: 49 launches) at the stream's slot count."""
    rng = np.random.default_rng(6)
    S = rng.integers(1, 201, slots)
    T = rng.integers(26, 377, slots)
    eng = cb.Engine(model, slots=slots, max_requests=slots, max_frames=376, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 256)
    try:
        eng.bench_fill(S, T, seed=5)
        eng.step()
        s = eng.stream()
        eng.decode_gemms_only()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for _ in range(reps):
            eng.decode_gemms_only()
        ev.record(b, s)
        step_us = ev.ms(a, b) * 1e3 / reps
        # the same launches reading their weight tiles alone
        eng.decode_gemm_read_floor()
        a2, b2 = ev.event(), ev.event()
        ev.record(a2, s)
        for _ in range(reps):
            eng.decode_gemm_read_floor()
        ev.record(b2, s)
        floor_us = ev.ms(a2, b2) * 1e3 / reps
    finally:
        eng.close()
    per = dec_gemm_launch_bytes(slots)
    n = len(per)
    w_bytes = float(sum(N * K * 2 for N, K in DEC_GEMMS))
    bytes_step = float(sum(per))
    per_launch_us = step_us / n
    achieved = bytes_step / (step_us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "gemv_kernel (decode GEMMs, all instances)",
            "avg_launch_us": round(per_launch_us, 3),
            "bytes_per_launch": int(bytes_step / n), "launches_per_step": n, "step_us": round(step_us, 2),
            "workload": f"{slots} slots, one step's {n} GEMM launches (268.4 MB of bf16 weights)",
            "read_floor": {"step_us": round(floor_us, 2),
                           "weight_GBs": round(w_bytes / (floor_us * 1e-6) / 1e9, 1),
                           "gemm_over_floor": round(step_us / floor_us, 3),
                           "what": "the same 49 launches (grids, weight tiles per workgroup) reading "
                                   "their weights alone: no activations, no MFMAs, no outputs"}}


def encoder_gemm_roofline(model, ev, ffn_bf16, M=16384, reps=10):
    K, N = cb.ENC_D, cb.ENC_FF
    eng = cb.Engine(model, slots=1, max_requests=1, max_frames=8, kv_bf16=True,
                    enc_ffn_bf16=ffn_bf16)
    try:
        s = eng.stream()
        eng.encoder_gemm(M)
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for _ in range(reps):
            eng.encoder_gemm(M)
        ev.record(b, s)
        ms = ev.ms(a, b) / reps
    finally:
        eng.close()
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    out = {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
           "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None,
           "avg_launch_us": round(ms * 1e3, 1), "flops_per_launch": 2 * M * N * K,
           "workload": f"M={M} N={N} K={K}"}
    if ffn_bf16:
        out.update(kernel="gemm_split256_sp_kernel (encoder FFN up, SiLU, single-pass bf16 "
                          "in/out)",
                   note="bf16 activations (rounded by the producer) against bf16 weights, fp32 "
                        "accumulation: the MFMA pipe runs the algorithmic flops counted here")
    else:
        out.update(kernel="gemm_split256_kernel (encoder FFN up, SiLU, pre-split in/out)",
                   note="activations as hi+lo bf16 against exact bf16 weights: the MFMA pipe "
                        "runs 2x the algorithmic flops counted here")
    return out


def copy_calibration(ev, stream, mib=256):
    """A plain device-to-device copy of known size on the engine stream, the
    scale for FETCH_SIZE / WRITE_SIZE counter runs."""
    rt = ev.rt
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    rt.hipFree.argtypes = [C.c_void_p]
    n = mib << 20
    src, dst = C.c_void_p(), C.c_void_p()
    if rt.hipMalloc(C.byref(src), n) or rt.hipMalloc(C.byref(dst), n):
        raise RuntimeError("hipMalloc failed")
    try:
        for _ in range(3):
            if rt.hipMemcpyAsync(dst, src, n, 3, stream):
                raise RuntimeError("hipMemcpyAsync failed")
        ev.sync()
    finally:
        rt.hipFree(src)
        rt.hipFree(dst)
    return {"bytes": n}


MFMA_FILE = os.path.join(REPO, "profiles", "mfma.json")


def with_traffic(rooflines):
    """Fills `traffic` (HBM bytes per launch) from the FETCH_SIZE/WRITE_SIZE
    counter runs and, for the encoder GEMM, the counter-derived MFMA
    utilisation (SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_VALU_MFMA_BUSY_CYCLES,
    GRBM_GUI_ACTIVE), when those runs are recorded under profiles/."""
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            tr = json.load(f)
        for k, r in rooflines.items():
            if k in tr.get("per_launch_bytes", {}) and tr.get("kernels", {}).get(k) == r.get("kernel"):
                r["traffic"] = tr["per_launch_bytes"][k]
    if os.path.exists(MFMA_FILE):
        with open(MFMA_FILE) as f:
            mf = json.load(f)
        for k, r in rooflines.items():
            if k in mf and mf[k].get("kernel") == r.get("kernel"):
                r["mfma_counters"] = dict(mf[k], source=mf["source"])
    return rooflines


REF_MODEL_LIB = os.path.join(REPO, "oracle", "_ref", "libref_model.so")
# The CPU baseline's sample: per process, one Conformer layer over the
# frames of an 8 s clip and a few decode steps at the stream's median shape.
CPU_LAYER_T = 101
CPU_DEC_T, CPU_DEC_S0, CPU_DEC_STEPS = 76, 74, 4


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _ref_worker(args):
    """One process of the CPU baseline: the reference host graph (model.h)
    on the reference CPU backend (backends/cpu/backend.c), both compiled from
    the reference's sources into oracle/_ref/libref_model.so.  Runs on the
    weight image inherited from the parent.  Returns (layer s, decode s)."""
    what, T, n_layers, dec_T, dec_S0, dec_steps = args
    lib = C.CDLL(REF_MODEL_LIB)
    lib.ref_set_weights.argtypes = [C.c_void_p]
    lib.ref_encoder_layers.argtypes = [C.c_void_p, C.c_int, C.c_int]
    lib.ref_decode_steps.argtypes = [C.c_int, C.c_int, C.c_int]
    lib.ref_decode_steps.restype = C.c_int
    lib.ref_set_weights(C.byref(_CPU_MODEL.W))
    x = np.random.default_rng(T).standard_normal((T, cb.ENC_D)).astype(np.float32)
    t0 = time.perf_counter()
    lib.ref_encoder_layers(x.ctypes.data, T, n_layers)
    t1 = time.perf_counter()
    lib.ref_decode_steps(dec_T, dec_S0, dec_steps)
    t2 = time.perf_counter()
    return t1 - t0, t2 - t1


_CPU_MODEL = None


def cpu_baseline(samples, limits, procs=None):
    """The reference CPU backend timed on this host's cores, before the GPU
    is touched.  The reference runs one sequence per thread, with as many
    CPU "devices" as cores (transcribe.c:947-984, backends/cpu/backend.c:
    21-24); here one process per core, each timing a bounded sample of the
    reference's own host graph: one Conformer layer over 101 frames (an 8 s
    clip) and 4 decode steps (self length 74, 76 encoder frames).  The
    per-frame and per-token costs are extrapolated to the stream's audio and
    token rows (prompt rows are prefilled, so each costs about a decode
    step); the aggregate is the per-process rate times the process count,
    all processes running at once.  Falls back to the oracle (kind "port")
    where the reference library is not built."""
    global _CPU_MODEL
    import multiprocessing as mp
    affine = len(os.sched_getaffinity(0))
    # at most 16 processes: a one-GPU share of the host's cores
    procs = procs or min(16, affine)
    audio = float(np.sum(samples)) / cb.SR
    T_enc = np.asarray([cb.t_enc(cb.t_mel(int(n))) for n in samples], np.float64)
    rows = float(np.sum(limits)) + len(cb.PROMPT) * len(limits)
    if not os.path.exists(REF_MODEL_LIB):
        return cpu_baseline_port(samples, limits)
    _CPU_MODEL = cb.SynthModel(seed=1234, variant=0)
    job = ("sample", CPU_LAYER_T, 1, CPU_DEC_T, CPU_DEC_S0, CPU_DEC_STEPS)

    def rate(res):
        t_layer = float(np.mean([r[0] for r in res]))
        t_step = float(np.mean([r[1] for r in res])) / CPU_DEC_STEPS
        per_frame = t_layer * cb.ENC_N / CPU_LAYER_T          # s of one process per encoder frame
        return audio / (float(np.sum(T_enc)) * per_frame + rows * t_step), t_layer, t_step

    # one process alone (the 1-thread figure), then one per core at once
    with mp.get_context("fork").Pool(1) as pool:
        alone, _, _ = rate(pool.map(_ref_worker, [job]))
    t0 = time.perf_counter()
    with mp.get_context("fork").Pool(procs) as pool:
        res = pool.map(_ref_worker, [job] * procs)
    wall = time.perf_counter() - t0
    _CPU_MODEL = None
    per_proc, t_layer, t_step = rate(res)
    return {"value": round(per_proc * procs, 4), "unit": "audio-sec/sec", "cores": procs,
            "kind": "reference", "one_thread_value": round(alone, 5),
            "nproc": os.cpu_count(), "affinity_cores": affine,
            "sample": f"{procs} processes at once, one per core (the reference's thread-per-device "
                      f"pool), each running the reference's model.h on its CPU backend: one "
                      f"Conformer layer over {CPU_LAYER_T} frames ({t_layer:.2f} s) and "
                      f"{CPU_DEC_STEPS} decode steps at S={CPU_DEC_S0}, T_enc={CPU_DEC_T} "
                      f"({t_step:.3f} s/step); extrapolated to the stream's {audio:.0f} audio-s "
                      f"({int(np.sum(T_enc))} encoder frames) and {int(rows)} token rows: "
                      f"{per_proc:.4f} audio-s/s per process; {wall:.1f} s wall; one process "
                      f"alone {alone:.4f} audio-s/s (one_thread_value). {procs} of the "
                      f"{affine} cores this process may run on (nproc {os.cpu_count()}): a "
                      f"one-GPU share of the host",
            "cpu_model": cpu_model_name(), "extrapolated": True}


def cpu_baseline_port(samples, limits):
    """The oracle (C fp32 restatement of the reference CPU backend, OpenMP),
    used when the reference library is not built: one 2 s clip through mel +
    encoder, then 16 decode steps, extrapolated to the stream's mix."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle_bind as ob
    threads = min(16, os.cpu_count() or 1)
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    model = cb.SynthModel(seed=1234, variant=0)
    o = ob.oracle()
    x = cb.synth_audio(2 * cb.SR, 77)
    t0 = time.perf_counter()
    mel = ob.compute_mel(x)
    eh = np.zeros((cb.t_enc(mel.shape[1]), cb.DEC_D), np.float32)
    o.orc_encoder_forward(mel.ctypes.data, mel.shape[1], mel.shape[1], model.weights_ref(), None,
                          eh.ctypes.data)
    t_enc = time.perf_counter() - t0
    t1 = time.perf_counter()
    toks, _, _ = ob.transcribe(model, mel, 16, suppress=True)   # includes a second encoder pass
    t_all = time.perf_counter() - t1
    t_dec = max(t_all - t_enc, 1e-6)
    n_dec = len(cb.PROMPT) + 16                                  # prompt rows + generated
    enc_rate = 2.0 / t_enc                                       # audio s per s
    dec_rate = n_dec / t_dec                                     # tokens per s (1 sequence)
    audio = float(np.sum(samples)) / cb.SR
    tokens = float(np.sum(limits)) + len(cb.PROMPT) * len(limits)
    t_est = audio / enc_rate + tokens / dec_rate
    return {"value": round(audio / t_est, 4), "unit": "audio-sec/sec", "cores": threads, "kind": "port",
            "sample": "one 2 s clip: mel + 48-layer encoder, then prompt + 16 greedy tokens; "
                      f"encoder {enc_rate:.3f} audio-s/s, decode {dec_rate:.2f} tok/s, "
                      "extrapolated to the stream's audio/token mix",
            "cpu_model": cpu_model_name(), "extrapolated": True}


def cpu_configs_full(procs):
    """The single-clip and uniform-batch configurations in full on the
    reference CPU path (its model.h on its CPU backend), one sequence per
    process as the reference's thread-per-device pool runs them:
      * single clip: an 8 s clip, 48 tokens, EOS suppressed; alone, then
        `procs` copies at once (the CPU's aggregate);
      * uniform batch: 8 clips of 10 s, 96 tokens each, 8 processes at once.
    Minutes of CPU time: run on request only.  The reference prints each
    finished encoder layer (its `verbose` flag) as progress."""
    global _CPU_MODEL
    import multiprocessing as mp
    _CPU_MODEL = cb.SynthModel(seed=1234, variant=0)
    out = {}
    for name, jobs in (("single clip alone", [(8, 48, 800)]),
                       (f"single clip x {procs}", [(8, 48, 800 + i) for i in range(procs)]),
                       ("uniform batch (8 x 10 s, 96 tokens)", [(10, 96, 900 + i) for i in range(8)])):
        t0 = time.perf_counter()
        with mp.get_context("fork").Pool(len(jobs)) as pool:
            res = pool.map(_ref_clip, jobs)
        wall = time.perf_counter() - t0
        audio = float(sum(j[0] for j in jobs))
        toks = sum(j[1] for j in jobs)
        out[name] = {"processes": len(jobs), "wall_s": round(wall, 1),
                     "per_clip_s": [round(r, 1) for r in res],
                     "audio_sec_per_sec": round(audio / wall, 4),
                     "tokens_per_s": round(toks / wall, 2)}
        print(f"{name}: {out[name]['wall_s']} s", file=sys.stderr, flush=True)
    _CPU_MODEL = None
    return {"path": "reference model.h + backends/cpu/backend.c (oracle/_ref/libref_model.so)",
            "cpu_model": cpu_model_name(), "runs": out}


def _ref_clip(job):
    secs, limit, seed = job
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle_bind as ob
    lib = C.CDLL(REF_MODEL_LIB)
    lib.ref_set_weights.argtypes = [C.c_void_p]
    lib.ref_transcribe_single.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                          C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.ref_transcribe_single.restype = C.c_int
    C.c_int.in_dll(lib, "verbose").value = 1
    lib.ref_set_weights(C.byref(_CPU_MODEL.W))
    mel = ob.compute_mel(cb.synth_audio(secs * cb.SR, seed))
    prompt = np.asarray(cb.PROMPT, np.int32)
    toks = np.zeros(limit, np.int32)
    t0 = time.perf_counter()
    n = lib.ref_transcribe_single(mel.ctypes.data, mel.shape[1], prompt.ctypes.data, len(prompt), limit,
                                  1, 0, toks.ctypes.data, None, None)
    if n != limit:
        raise RuntimeError(f"reference produced {n} of {limit} tokens")
    return time.perf_counter() - t0


def measure_rooflines(hip, model, ev, ffn_bf16, samples, limits, step_reps=5):
    """Per-kernel rooflines; encoder_gemm is the FFN GEMM in the stream's
    precision mode, encoder_gemm_split the fp32-accurate form beside it
    when the stream runs the single-pass one; attention_b64 and
    decode_step_b64 at the stream's own step shape."""
    att, micro = attention_roofline(hip, model, ev, step_reps=step_reps)
    att_64, _ = attention_roofline(hip, model, ev, B=64)
    att64, step64 = decode_b64(model, ev, samples, limits)
    roofs = {"attention": att, "attention_64": att_64, "attention_b64": att64, "decode_step_b64": step64,
             "decode_gemm": decode_gemm_roofline(model, ev),
             "encoder_gemm": encoder_gemm_roofline(model, ev, ffn_bf16)}
    if ffn_bf16:
        roofs["encoder_gemm_split"] = encoder_gemm_roofline(model, ev, 0)
    tmp = cb.Engine(model, slots=1, max_requests=1, max_frames=8, kv_bf16=True)
    try:
        copy_calibration(ev, tmp.stream())
    finally:
        tmp.close()
    return with_traffic(roofs), micro


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--requests", type=int, default=256)
    ap.add_argument("--slots", type=int, default=64)
    ap.add_argument("--prefill-rows", type=int, default=16,
                    help="spare step rows that feed prompts several tokens a step")
    ap.add_argument("--admit-order", type=int, default=1,
                    help="0: encode and admit in submission order; 1: largest token budget first")
    ap.add_argument("--enc-ffn-bf16", type=int, default=1,
                    help="1: the encoder's FFN projections in single-pass bf16 (inputs rounded "
                         "to bf16, fp32 accumulation); 0: fp32-accurate hi+lo split")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the per-kernel roofline microbenchmarks (for profiling)")
    ap.add_argument("--no-rooflines", action="store_true",
                    help="run only the stream (for profiling its kernel mix)")
    ap.add_argument("--cpu-configs", type=int, default=0, metavar="PROCS",
                    help="only time the single-clip (alone and PROCS at once) and uniform-batch "
                         "configurations in full on the reference CPU path (minutes), and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (requests shard "
              "across GPUs with no exchange, see the design notes).", file=sys.stderr)
        sys.exit(2)
    if args.cpu_configs:
        print(json.dumps(cpu_configs_full(args.cpu_configs)))
        return

    samples, limits = make_stream(args.requests, seed=3)
    # the CPU baseline runs first, in forked processes, before this process
    # touches the GPU
    cpu = None
    if not (args.no_cpu_baseline or args.roofline_only):
        cpu = cpu_baseline(samples, limits)

    hip = cb.hip()
    model = cb.SynthModel(seed=1234, variant=0)
    hip.backend_weights_upload_blob(model.data_ptr, model.data_bytes)
    hip.backend_init(0)
    ev = cb.HipEvents()

    if args.roofline_only:
        roofs, micro = measure_rooflines(hip, model, ev, args.enc_ffn_bf16, samples, limits, step_reps=0)
        print(json.dumps({"rooflines": roofs, "decode_microbench": micro}))
        return

    offs = np.concatenate([[0], np.cumsum(samples)[:-1]])
    total = int(np.sum(samples))
    pcm = np.concatenate([cb.synth_audio(int(n), 1000 + i) for i, n in enumerate(samples)])
    # self caches sized for the longest request (prompt + 256 tokens)
    eng = cb.Engine(model, slots=args.slots, max_requests=args.requests, max_frames=376, kv_bf16=True,
                    max_tokens=len(cb.PROMPT) + 256, prefill_rows=args.prefill_rows,
                    admit_order=args.admit_order, enc_ffn_bf16=args.enc_ffn_bf16)
    # device-resident input: the PCM buffer lives in a second engine-independent
    # allocation (the backend arena)
    dev_pcm = hip.backend_arena_alloc(total)
    hip.backend_htod(dev_pcm, pcm.ctypes.data, total)

    for _ in range(args.warmup):
        run_stream(hip, eng, ev, dev_pcm, offs, samples, limits)
    times, dec_times, steps = [], [], []
    for _ in range(args.steps):
        t, td, st = run_stream(hip, eng, ev, dev_pcm, offs, samples, limits)
        times.append(t); dec_times.append(td); steps.append(st)
    # all requests produced exactly their forced length
    got = [len(eng.tokens(r)) for r in range(len(limits))]
    if got != [int(x) for x in limits]:
        raise RuntimeError("a request did not produce its forced number of tokens")
    audio = total / cb.SR
    t_step = float(np.sum(times)) / args.steps
    rtfx = audio / t_step
    gen_tokens = int(np.sum(limits))
    if OVERLAP_BATCH_FRAMES:
        # decode alone: one more pass that encodes everything first (not part
        # of the timed steps)
        _, td, _ = run_stream(hip, eng, ev, dev_pcm, offs, samples, limits, overlap=0)
        dec_tps = gen_tokens / td
    else:
        dec_tps = gen_tokens / (float(np.sum(dec_times)) / args.steps)
    eng.close()

    # the same stream with the other encoder FFN precision (one warm and one
    # timed pass on an engine of its own), so the precision trade is visible
    other = None
    if not args.no_rooflines:
        eng2 = cb.Engine(model, slots=args.slots, max_requests=args.requests, max_frames=376,
                         kv_bf16=True, max_tokens=len(cb.PROMPT) + 256, prefill_rows=args.prefill_rows,
                         admit_order=args.admit_order, enc_ffn_bf16=1 - args.enc_ffn_bf16)
        try:
            run_stream(hip, eng2, ev, dev_pcm, offs, samples, limits)
            t2, _, st2 = run_stream(hip, eng2, ev, dev_pcm, offs, samples, limits)
            if [len(eng2.tokens(r)) for r in range(len(limits))] != [int(x) for x in limits]:
                raise RuntimeError("a request did not produce its forced number of tokens")
        finally:
            eng2.close()
        other = {"encoder_ffn": "hi+lo split" if args.enc_ffn_bf16 else "single-pass bf16",
                 "value": round(audio / t2, 2), "unit": "audio-sec/sec", "ms_per_pass": round(t2 * 1e3, 2),
                 "decode_steps": int(st2), "passes": 1, "warmup": 1}
    roofs, micro = ({}, {}) if args.no_rooflines else measure_rooflines(hip, model, ev,
                                                                         args.enc_ffn_bf16, samples, limits)
    configs = None if args.no_rooflines else config_latency(hip, model, ev, args.enc_ffn_bf16)

    out = {
        "metric": METRIC, "value": round(rtfx, 2), "unit": "audio-sec/sec", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t_step * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32+bf16",
        "data": "synthetic (seeded audio, random-init weights at model dims)",
        "config": {"workload": "continuous-batching stream: 256 requests, clips lognormal(median 6 s) "
                               "in [1,30] s, forced decode lengths U[8,256], <= 64 in flight",
                   "requests": args.requests, "slots": args.slots,
                   "prefill_rows": args.prefill_rows, "audio_sec": round(audio, 1),
                   "encoder_batch_frames": OVERLAP_BATCH_FRAMES or 24576,
                   "encode_decode_overlap": bool(OVERLAP_BATCH_FRAMES),
                   "generated_tokens": gen_tokens, "kv": "bf16", "parallelism": "single GPU",
                   "admission": "largest token budget first" if args.admit_order else "submission order",
                   "encoder_ffn": "single-pass bf16" if args.enc_ffn_bf16 else "hi+lo split"},
        "decode_tokens_per_s": round(dec_tps, 1),
        "decode_steps": int(np.mean(steps)),
        "roofline": dict(roofs[DOMINANT], name=DOMINANT) if roofs else None, "rooflines": roofs,
        "decode_microbench": micro,
        "stream_other_ffn_precision": other,
        "config_runs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
