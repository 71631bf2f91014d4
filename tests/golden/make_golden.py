"""Writes the golden fixtures under tests/golden/ from the reference itself.

Run in the container that holds the reference sources, after
`make -C oracle` has compiled them into oracle/_ref/:

  test_kernels_ref_cpu.bin  output of the reference's tests/test_kernels.c on
                            its CPU backend (9 functions, LCG inputs).
  kernels_ext.npz           every compute function of the backend ABI on the
                            reference CPU backend (tests/kernel_suite.py
                            inputs, synthetic weights seed 11, perturbed).
  model_small.npz           the reference host graph (model.h) on the CPU
                            backend: encoder outputs, first-step logits and
                            forced-length token ids for two short clips, single
                            and batched (weights seed 5, spec init).
  model_small_hot.npz       the same with the decoder-hot weight variant, where
                            greedy decoding is input-dependent.
  config_c0c1_v{0,2,3}.npz  `configs`: the single-sequence path at benchmark
                            lengths (one 8 s clip with 48 tokens, two 10 s
                            clips with 96 tokens), fp32 KV, EOS suppressed:
                            encoder outputs, token ids, three logits rows per
                            clip and every step's top-1/top-2 margin.

Only data is written (inputs are regenerated from the stated seeds; their
checksums are stored to detect drift).
"""
import ctypes as C
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_bind as ob  # noqa: E402
import ctbind as cb  # noqa: E402
import kernel_suite as ks  # noqa: E402

REF = ob.REF_DIR

# model-level fixture definition (shared with the tests)
MODEL_SEED = 5
MODEL_FIXTURES = {0: "model_small.npz", 2: "model_small_hot.npz"}   # variant -> file
CLIPS = [(4000, 101), (7200, 102)]          # (samples, audio seed): T_enc 4 and 6
SINGLE_LIMIT = 6
BATCH_LIMITS = [5, 3]
KERNEL_SEED, KERNEL_VARIANT = 11, 1


def checksum(a):
    return float(np.float64(np.asarray(a, np.float64).sum()))


def kernels_bin():
    out = os.path.join(HERE, "test_kernels_ref_cpu.bin")
    subprocess.run([os.path.join(REF, "test_kernels_cpu"), out], check=True)


def kernels_ext():
    ref = cb.bind_abi(C.CDLL(os.path.join(REF, "libref_cpu.so")))
    model = cb.SynthModel(seed=KERNEL_SEED, variant=KERNEL_VARIANT)
    inp = ks.make_inputs()
    ref.backend_weights_upload_blob(model.data_ptr, model.data_bytes)
    ref.backend_init(0)
    out = ks.run_suite(ref, ks.HostDev(), model, inp)
    np.savez_compressed(os.path.join(HERE, "kernels_ext.npz"),
                        **{"out_" + k: v for k, v in out.items()},
                        **{"sum_" + k: np.float64(checksum(v)) for k, v in inp.items()})


def model_small(variant, fname):
    lib = C.CDLL(os.path.join(REF, "libref_model.so"))
    P, I = C.c_void_p, C.c_int
    lib.ref_set_weights.argtypes = [P]
    lib.ref_encoder.argtypes = [P, I, P]
    lib.ref_transcribe_single.argtypes = [P, I, P, I, I, I, I, P, P, P]
    lib.ref_transcribe_single.restype = I
    lib.ref_transcribe_batch.argtypes = [P, I, P, I, P, I, P, I, I, I, P, P, P]
    model = cb.SynthModel(seed=MODEL_SEED, variant=variant)
    lib.ref_set_weights(model.weights_ref())
    mels = [ob.compute_mel(cb.synth_audio(n, s)) for n, s in CLIPS]
    prompt = np.asarray(cb.PROMPT, np.int32)
    res = {}
    for i, mel in enumerate(mels):
        res[f"mel{i}"] = mel
    # single path, EOS suppressed
    t0 = time.time()
    toks = np.zeros(SINGLE_LIMIT, np.int32)
    lg = np.zeros((SINGLE_LIMIT, cb.VOCAB), np.float32)
    eh = np.zeros((cb.t_enc(mels[0].shape[1]), cb.DEC_D), np.float32)
    n = lib.ref_transcribe_single(mels[0].ctypes.data, mels[0].shape[1], prompt.ctypes.data,
                                  len(prompt), SINGLE_LIMIT, 1, 0, toks.ctypes.data,
                                  lg.ctypes.data, eh.ctypes.data)
    res["single_tokens"] = toks[:n]
    res["single_logits"] = lg[:2]
    res["enc_h0"] = eh
    print("single", toks[:n], f"{time.time() - t0:.1f}s", flush=True)
    # natural stop (no suppression), short limit
    toks2 = np.zeros(4, np.int32)
    n2 = lib.ref_transcribe_single(mels[1].ctypes.data, mels[1].shape[1], prompt.ctypes.data,
                                   len(prompt), 4, 0, 0, toks2.ctypes.data, None, None)
    res["natural_tokens"] = toks2[:n2]
    print("natural", toks2[:n2], flush=True)
    # batched ragged path, suppressed with EOS forced at each item's limit
    B = len(mels)
    Tm = np.asarray([m.shape[1] for m in mels], np.int32)
    Tmax = int(Tm.max())
    mb = np.zeros((B, cb.N_MELS, Tmax), np.float32)
    for b, m in enumerate(mels):
        mb[b, :, :m.shape[1]] = m
    lim = np.asarray(BATCH_LIMITS, np.int32)
    bt = np.zeros((B, max(BATCH_LIMITS)), np.int32)
    nb = np.zeros(B, np.int32)
    ehb = np.zeros((B, cb.t_enc(Tmax), cb.DEC_D), np.float32)
    lib.ref_transcribe_batch(mb.ctypes.data, B, Tm.ctypes.data, Tmax, prompt.ctypes.data,
                             len(prompt), lim.ctypes.data, 1, 1, max(BATCH_LIMITS),
                             bt.ctypes.data, nb.ctypes.data, ehb.ctypes.data)
    res["batch_tokens"] = bt
    res["batch_n"] = nb
    res["enc_h1"] = ehb[1, :cb.t_enc(mels[1].shape[1])]
    res["enc_h0_batch"] = ehb[0, :cb.t_enc(mels[0].shape[1])]
    print("batch", bt, nb, flush=True)
    np.savez_compressed(os.path.join(HERE, fname), **res)


# Benchmark-configuration fixtures: the reference host graph (model.h
# transcribe_chunk path, transcribe.c:264-390) on the reference CPU backend,
# fp32 KV, greedy with EOS suppressed, at the lengths of the single-clip
# configuration (one 8 s clip, 48 tokens) and two clips of the uniform batch
# configuration (10 s, 96 tokens).  Spec weights (variant 0: greedy repeats one
# token), decoder-hot weights (variant 2: input-dependent tokens) and
# decoder-warm weights (variant 3: input-dependent tokens, bf16 K/V within the
# specified 1e-2 of the fp32 logits).
CONFIG_SEED = MODEL_SEED
CONFIG_JOBS = {"c0": [(8 * 16000, 800, 48)],
               "c1": [(10 * 16000, 1000, 96), (10 * 16000, 1001, 96)]}
CONFIG_VARIANTS = (0, 2, 3)


def config_fname(variant):
    return f"config_c0c1_v{variant}.npz"


def margins(lg):
    """(top1 - top2) / |top1| of each logits row with EOS excluded, the
    row's gap between the chosen token and the runner-up."""
    x = np.asarray(lg, np.float64).copy()
    x[:, cb.EOS] = -np.inf
    top = -np.sort(-x, axis=1)[:, :2]
    return (top[:, 0] - top[:, 1]) / np.abs(top[:, 0])


def config_job(args):
    variant, name, idx, n, seed, limit = args
    lib = C.CDLL(os.path.join(REF, "libref_model.so"))
    P, I = C.c_void_p, C.c_int
    lib.ref_set_weights.argtypes = [P]
    lib.ref_transcribe_single.argtypes = [P, I, P, I, I, I, I, P, P, P]
    lib.ref_transcribe_single.restype = I
    model = cb.SynthModel(seed=CONFIG_SEED, variant=variant, nthreads=2)
    lib.ref_set_weights(model.weights_ref())
    mel = ob.compute_mel(cb.synth_audio(n, seed))
    prompt = np.asarray(cb.PROMPT, np.int32)
    toks = np.zeros(limit, np.int32)
    lg = np.zeros((limit, cb.VOCAB), np.float32)
    eh = np.zeros((cb.t_enc(mel.shape[1]), cb.DEC_D), np.float32)
    t0 = time.time()
    got = lib.ref_transcribe_single(mel.ctypes.data, mel.shape[1], prompt.ctypes.data, len(prompt),
                                    limit, 1, 0, toks.ctypes.data, lg.ctypes.data, eh.ctypes.data)
    assert got == limit
    # logits rows kept: first, middle, last; for the decoder-warm weights also
    # the first 12, which precede the first near-tie under bf16 K/V
    first = list(range(12)) if variant == 3 else [0]
    rows = np.asarray(sorted(set(first + [limit // 2, limit - 1])), np.int32)
    key = f"{name}_{idx}"
    print(f"v{variant} {key}: T_enc {eh.shape[0]}, {time.time() - t0:.0f} s, tokens {toks[:8]}...",
          flush=True)
    return variant, {f"{key}_samples": np.int64(n), f"{key}_seed": np.int64(seed),
                     f"{key}_mel_sum": np.float64(checksum(mel)), f"{key}_tokens": toks,
                     f"{key}_enc_h": eh, f"{key}_rows": rows, f"{key}_logits": lg[rows],
                     f"{key}_margin": margins(lg).astype(np.float32),
                     f"{key}_logit_absmax": np.abs(lg).max(axis=1).astype(np.float32)}


def configs(variants=CONFIG_VARIANTS):
    import multiprocessing as mp
    jobs = [(v, name, i, n, s, lim) for v in variants for name, js in CONFIG_JOBS.items()
            for i, (n, s, lim) in enumerate(js)]
    with mp.get_context("fork").Pool(len(jobs)) as pool:
        res = pool.map(config_job, jobs)
    for v in variants:
        out = {"weight_seed": np.int64(CONFIG_SEED), "variant": np.int64(v)}
        for vv, d in res:
            if vv == v:
                out.update(d)
        np.savez_compressed(os.path.join(HERE, config_fname(v)), **out)


if __name__ == "__main__":
    which = sys.argv[1:] or ["bin", "ext", "model"]
    if "bin" in which:
        kernels_bin()
    if "ext" in which:
        kernels_ext()
    if "model" in which:
        for var, fname in MODEL_FIXTURES.items():
            model_small(var, fname)
    if "configs" in which:
        configs()
    for v in CONFIG_VARIANTS:
        if f"configs{v}" in which:         # one variant's file alone
            configs((v,))
