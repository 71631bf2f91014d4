"""ctypes bindings for the MI355X backend libraries built in this directory.

libct_hip.so exports the 40-function backend ABI (include/backend.h) and the
hipb_* decode engine (include/hipb.h); libct_host.so holds the seeded
synthetic workload (weights in the converter's safetensors layout, audio).

Nothing here falls back to a CPU path: if a library is missing the loader
raises, so a test or benchmark that runs has run the HIP code.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# CT_HOST_LIB / CT_CHUNK_LIB name sanitizer builds of the host C to load
# instead (tests/test_sanitize.py)
HOST_LIB = os.environ.get("CT_HOST_LIB") or os.path.join(PKG_DIR, "libct_host.so")
HIP_LIB = os.path.join(PKG_DIR, "libct_hip.so")

# Model constants (include/model_types.h).
ENC_D, ENC_FF, ENC_H, ENC_DK, ENC_N, ENC_CK, SUB_CH = 1280, 5120, 8, 160, 48, 9, 256
DEC_D, DEC_FF, DEC_H, DEC_DK, DEC_N = 1024, 4096, 8, 128, 8
VOCAB, MAX_SEQ = 16384, 1024
N_MELS, HOP_LEN, SR = 128, 160, 16000
EOS = 3
# Prompt built by transcribe.c:1320-1330 with pnc/itn/timestamps/diarize off;
# the language id is a fixed placeholder (the vocabulary is not available).
PROMPT = [13764, 7, 4, 16, 62, 62, 6, 9, 11, 13]

# Field order of the Weights struct (include/model_types.h), flattened.
_FIXED_A = ["s0w", "s0b", "s2w", "s2b", "s3w", "s3b", "s5w", "s5b", "s6w", "s6b", "sow", "sob"]
ELAYER_FIELDS = ["ff1_lnw", "ff1_lnb", "ff1_w1", "ff1_b1", "ff1_w2", "ff1_b2",
                 "sa_lnw", "sa_lnb", "sa_qw", "sa_qb", "sa_kw", "sa_kb",
                 "sa_vw", "sa_vb", "sa_pw", "sa_ow", "sa_ob", "sa_pbu", "sa_pbv",
                 "cv_lnw", "cv_lnb", "cv_pw1w", "cv_pw1b", "cv_dww", "cv_dwb",
                 "cv_bnw", "cv_bnb", "cv_bnmean", "cv_bnvar", "cv_pw2w", "cv_pw2b",
                 "ff2_lnw", "ff2_lnb", "ff2_w1", "ff2_b1", "ff2_w2", "ff2_b2",
                 "out_lnw", "out_lnb"]
DLAYER_FIELDS = ["sa_lnw", "sa_lnb", "sa_qw", "sa_qb", "sa_kw", "sa_kb",
                 "sa_vw", "sa_vb", "sa_ow", "sa_ob",
                 "ca_lnw", "ca_lnb", "ca_qw", "ca_qb", "ca_kw", "ca_kb",
                 "ca_vw", "ca_vb", "ca_ow", "ca_ob",
                 "ffn_lnw", "ffn_lnb", "ffn_w1", "ffn_b1", "ffn_w2", "ffn_b2"]
FIELDS = (_FIXED_A
          + [f"enc{i}.{f}" for i in range(ENC_N) for f in ELAYER_FIELDS]
          + ["prw", "prb", "etw", "epw", "elnw", "elnb"]
          + [f"dec{i}.{f}" for i in range(DEC_N) for f in DLAYER_FIELDS]
          + ["dlnw", "dlnb", "hdb"])
FIELD_INDEX = {n: i for i, n in enumerate(FIELDS)}
N_PTRS = len(FIELDS)                     # 2101
WeightsT = C.c_void_p * N_PTRS
ELAYER_BYTES = len(ELAYER_FIELDS) * 8
DLAYER_BYTES = len(DLAYER_FIELDS) * 8
ENC_OFF = len(_FIXED_A)                  # index of enc[0] inside Weights


def t_mel(n_samples):
    return 1 + n_samples // HOP_LEN


def t_enc(T_mel):
    a = (T_mel + 1) // 2
    b = (a + 1) // 2
    return (b + 1) // 2


_host = None


def host():
    """libct_host.so (synthetic workload)."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB):
            raise RuntimeError(f"{HOST_LIB} is not built (run __graft_entry__.build())")
        L = C.CDLL(HOST_LIB)
        L.ct_synth_file_bytes.restype = C.c_size_t
        L.ct_synth_weights.argtypes = [C.c_void_p, C.c_size_t, C.c_uint64, C.c_int, C.c_int]
        L.ct_synth_weights.restype = C.c_int
        L.ct_weights_bind.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p,
                                      C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
        L.ct_weights_bind.restype = C.c_int
        L.ct_synth_audio.argtypes = [C.c_void_p, C.c_int, C.c_uint64]
        L.ct_hash64.argtypes = [C.c_uint64, C.c_uint64]
        L.ct_hash64.restype = C.c_uint64
        L.ct_normal16.argtypes = [C.c_uint64]
        L.ct_normal16.restype = C.c_float
        _host = L
    return _host


class SynthModel:
    """Seeded synthetic weights at model dimensions, bound to a Weights struct.

    `image` is the full safetensors file image; `data_ptr`/`data_bytes` is its
    data section (what the host hands to backend_weights_upload_blob)."""

    def __init__(self, seed=1234, variant=0, nthreads=0):
        L = host()
        n = L.ct_synth_file_bytes()
        self.image = np.empty(n, dtype=np.uint8)
        rc = L.ct_synth_weights(self.image.ctypes.data, n, seed, variant, nthreads)
        if rc != 0:
            raise RuntimeError("ct_synth_weights failed")
        self.W = WeightsT()
        data = C.c_void_p()
        nbytes = C.c_size_t()
        rc = L.ct_weights_bind(self.image.ctypes.data, n, C.byref(self.W),
                               C.byref(data), C.byref(nbytes))
        if rc != 0:
            raise RuntimeError("ct_weights_bind failed")
        self.data_ptr = data.value
        self.data_bytes = nbytes.value
        self.seed, self.variant = seed, variant

    def ptr(self, field):
        return self.W[FIELD_INDEX[field]]

    def tensor(self, field, n):
        """First n bf16 values of a tensor, widened to float32."""
        raw = np.ctypeslib.as_array(C.cast(self.ptr(field), C.POINTER(C.c_uint16)), shape=(n,))
        return (raw.astype(np.uint32) << 16).view(np.float32)

    def set_bf16(self, field, index, value):
        """Overwrites one bf16 value of a tensor in the host image (value must
        be exactly representable); upload the blob again afterwards."""
        f = np.float32(value)
        raw = int(f.view(np.uint32))
        if raw & 0xFFFF:
            raise ValueError(f"{value} is not a bf16 value")
        C.cast(self.ptr(field), C.POINTER(C.c_uint16))[index] = raw >> 16

    def weights_ref(self):
        return C.byref(self.W)

    def elayer_ptr(self, i):
        return C.addressof(self.W) + (ENC_OFF + i * len(ELAYER_FIELDS)) * 8


def synth_audio(n_samples, seed):
    out = np.empty(n_samples, dtype=np.float32)
    host().ct_synth_audio(out.ctypes.data, n_samples, seed)
    return out


# ---------------------------------------------------------------------------
# The 40-function backend ABI (include/backend.h).  Any library exporting it
# (this backend, or the reference CPU backend when it is built for fixtures)
# can be bound with bind_abi().
# ---------------------------------------------------------------------------
_P, _I, _F, _Z = C.c_void_p, C.c_int, C.c_float, C.c_size_t
ABI_SIGS = {
    "backend_init": ([_I], None),
    "backend_destroy": ([], None),
    "backend_num_devices": ([], _I),
    "backend_thread_cleanup": ([], None),
    "backend_weights_upload_blob": ([_P, _Z], None),
    "backend_device_ptr": ([_P], _P),
    "backend_arena_alloc": ([_Z], _P),
    "backend_arena_free": ([_P], None),
    "backend_htod": ([_P, _P, _Z], None),
    "backend_dtoh": ([_P, _P, _Z], None),
    "backend_layernorm": ([_P, _P, _P, _P, _I, _I], None),
    "backend_linear": ([_P, _P, _P, _P, _I, _I, _I], None),
    "backend_linear_silu": ([_P, _P, _P, _P, _I, _I, _I], None),
    "backend_linear_relu": ([_P, _P, _P, _P, _I, _I, _I], None),
    "backend_linear_fmadd": ([_P, _F, _P, _P, _P, _I, _I, _I], None),
    "backend_add_inplace": ([_P, _P, _I], None),
    "backend_encoder_subsampling": ([_P, _I, _I, _P, _I, _P, _P], None),
    "backend_make_rel_pos_emb": ([_P, _I], None),
    "backend_rel_pos_mhsa": ([_P, _P, _I, _P, _P], None),
    "backend_conformer_conv": ([_P, _I, _P, _P], None),
    "backend_sdp_attn": ([_P, _P, _P, _P, _P, _I, _I, _P], None),
    "backend_embed": ([_P, _P, _I, _I, _P, _P, _P, _P], None),
    "backend_fill_causal_mask": ([_P, _I], None),
    "backend_lm_head": ([_P, _P, _P, _P], None),
    "backend_upload_tokens": ([_P, _I], None),
    "backend_graph_replay": ([_I, _I, _I, _I], _I),
    "backend_graph_begin_capture": ([_I], None),
    "backend_graph_end_capture": ([_I, _I, _I, _I], None),
    "backend_decode_set_S": ([_I], None),
    "backend_decode_inc_S": ([], None),
    "backend_linear_to_kvcache": ([_P, _P, _P, _P, _I, _I], None),
    "backend_sdp_attn_devS": ([_P, _P, _P, _P, _P], None),
    "backend_embed_decode": ([_P, _P, _P, _P, _P], None),
    "backend_embed_decode_batch": ([_P, _P, _P, _P, _I, _P, _P, _P, _P], None),
    "backend_lm_head_batch": ([_P, _P, _P, _P, _P, _I], None),
    "backend_argmax_batch": ([_P, _P, _P, _I], None),
    "backend_upload_T_enc": ([_P, _I], None),
    "backend_linear_to_kvcache_batch": ([_P, _P, _P, _P, _I, _I, _I, _I], None),
    "backend_sdp_attn_batch_decode_sa": ([_P, _P, _P, _P, _I, _I, _P], None),
    "backend_sdp_attn_batch_decode_ca": ([_P, _P, _P, _P, _I, _I, _P], None),
}
assert len(ABI_SIGS) == 40
# This backend's addition to the ABI (include/backend.h, after the 40).
ABI_EXT_SIGS = {
    "backend_rel_pos_mhsa_noalloc": ([_P, _P, _I, _P], None),
}


def bind_abi(lib):
    for name, (args, ret) in ABI_SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ret
    for name, (args, ret) in ABI_EXT_SIGS.items():
        fn = getattr(lib, name, None)
        if fn is not None:
            fn.argtypes = args
            fn.restype = ret
    return lib


_hip = None


def hip():
    """libct_hip.so with the ABI bound.  Raises if the library is missing:
    there is no CPU fallback behind this binding."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB):
            raise RuntimeError(f"{HIP_LIB} is not built (run __graft_entry__.build())")
        _hip = bind_abi(C.CDLL(HIP_LIB))
    return _hip


# ---------------------------------------------------------------------------
# The decode engine (include/hipb.h)
# ---------------------------------------------------------------------------
HIPB_SUPPRESS_EOS = 1
HIPB_FORCE_EOS = 2


class HipbConfig(C.Structure):
    _fields_ = [("slots", C.c_int), ("max_requests", C.c_int),
                ("max_frames", C.c_int), ("kv_bf16", C.c_int), ("max_tokens", C.c_int),
                ("prefill_rows", C.c_int), ("admit_order", C.c_int), ("enc_ffn_bf16", C.c_int)]


_ENGINE_SIGS = {
    "hipb_create": ([C.POINTER(HipbConfig), C.c_void_p], C.c_void_p),
    "hipb_destroy": ([C.c_void_p], None),
    "hipb_submit": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int], C.c_int),
    "hipb_encode": ([C.c_void_p, C.c_int], None),
    "hipb_step": ([C.c_void_p], None),
    "hipb_run": ([C.c_void_p, C.c_int], C.c_long),
    "hipb_process": ([C.c_void_p, C.c_int, C.c_int], C.c_long),
    "hipb_finished": ([C.c_void_p], C.c_int),
    "hipb_tokens": ([C.c_void_p, C.c_int, C.c_void_p, C.c_int], C.c_int),
    "hipb_token_scores": ([C.c_void_p, C.c_int, C.c_void_p, C.c_int], C.c_int),
    "hipb_slot_of": ([C.c_void_p, C.c_int], C.c_int),
    "hipb_logits": ([C.c_void_p, C.c_int, C.c_void_p], None),
    "hipb_enc_out": ([C.c_void_p, C.c_int, C.c_void_p], None),
    "hipb_req_frames": ([C.c_void_p, C.c_int], C.c_int),
    "hipb_bench_fill": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64], None),
    "hipb_attention_only": ([C.c_void_p], None),
    "hipb_bench_decode_gemms": ([C.c_void_p], None),
    "hipb_bench_read_floor": ([C.c_void_p], None),
    "hipb_bench_encoder_gemm": ([C.c_void_p, C.c_int], None),
    "hipb_bench_steps": ([C.c_void_p, C.c_int], None),
    "hipb_stream": ([C.c_void_p], C.c_void_p),
}


def engine_lib():
    lib = hip()
    if not getattr(lib, "_hipb_bound", False):
        for n, (a, r) in _ENGINE_SIGS.items():
            fn = getattr(lib, n)
            fn.argtypes = a
            fn.restype = r
        lib._hipb_bound = True
    return lib


class Engine:
    """Thin owner of a HipbEngine* (the calling thread must have run
    backend_init and uploaded the model's blob)."""

    def __init__(self, model, slots, max_requests, max_frames, kv_bf16=True, max_tokens=0,
                 prefill_rows=0, admit_order=0, enc_ffn_bf16=0):
        self.L = engine_lib()
        self.model = model
        cfg = HipbConfig(slots, max_requests, max_frames, int(kv_bf16), int(max_tokens),
                         int(prefill_rows), int(admit_order), int(enc_ffn_bf16))
        self.e = self.L.hipb_create(C.byref(cfg), model.weights_ref())
        self.slots = slots

    def submit(self, mel, limit, flags=HIPB_SUPPRESS_EOS, prompt=None):
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        p = np.ascontiguousarray(prompt if prompt is not None else PROMPT, dtype=np.int32)
        return self.L.hipb_submit(self.e, mel.ctypes.data, mel.shape[1], p.ctypes.data, len(p),
                                  limit, flags)

    def encode(self, max_batch_frames=32768):
        self.L.hipb_encode(self.e, max_batch_frames)

    def step(self):
        self.L.hipb_step(self.e)

    def run(self, chunk=8):
        return self.L.hipb_run(self.e, chunk)

    def process(self, max_batch_frames=8192, chunk=8):
        """Encode and decode overlapped (hipb_process)."""
        return self.L.hipb_process(self.e, max_batch_frames, chunk)

    def finished(self):
        return self.L.hipb_finished(self.e)

    def tokens(self, req):
        out = np.zeros(MAX_SEQ, np.int32)
        n = self.L.hipb_tokens(self.e, req, out.ctypes.data, MAX_SEQ)
        return out[:n].copy()

    def scores(self, req):
        """Per generated token, the largest logit the argmax weighed."""
        out = np.zeros(MAX_SEQ, np.float32)
        n = self.L.hipb_token_scores(self.e, req, out.ctypes.data, MAX_SEQ)
        return out[:n].copy()

    def slot_of(self, req):
        return self.L.hipb_slot_of(self.e, req)

    def logits(self, slot):
        out = np.zeros(VOCAB, np.float32)
        self.L.hipb_logits(self.e, slot, out.ctypes.data)
        return out

    def enc_out(self, req):
        T = self.L.hipb_req_frames(self.e, req)
        out = np.zeros((T, DEC_D), np.float32)
        self.L.hipb_enc_out(self.e, req, out.ctypes.data)
        return out

    def bench_fill(self, S, T_enc, seed=1):
        S = np.ascontiguousarray(S, np.int32)
        T = np.ascontiguousarray(T_enc, np.int32)
        self.L.hipb_bench_fill(self.e, S.ctypes.data, T.ctypes.data, seed)

    def attention_only(self):
        self.L.hipb_attention_only(self.e)

    def decode_gemms_only(self):
        self.L.hipb_bench_decode_gemms(self.e)

    def decode_gemm_read_floor(self):
        self.L.hipb_bench_read_floor(self.e)

    def encoder_gemm(self, M):
        self.L.hipb_bench_encoder_gemm(self.e, M)

    def bench_steps(self, n):
        self.L.hipb_bench_steps(self.e, n)

    def stream(self):
        return self.L.hipb_stream(self.e)

    def close(self):
        if self.e:
            self.L.hipb_destroy(self.e)
            self.e = None


_ENGINE_SIGS.update({
    "hipb_submit_pcm": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int], C.c_int),
    "hipb_mel": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p], None),
    "hipb_reset": ([C.c_void_p], None),
    "hipb_submit_pcm_device": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int], C.c_int),
    "hipb_submit_pcm_chunked": ([C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                 C.c_float, C.c_float, C.c_float, C.POINTER(C.c_int)], C.c_int),
    "hipb_chunk_bounds": ([C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_float, C.c_void_p, C.c_int],
                          C.c_int),
    "hipb_test_hold_encoder": ([C.c_void_p, C.c_int, C.c_int], None),
    "hipb_test_hold_expired": ([C.c_void_p], C.c_int),
})


def chunk_bounds(samples, silence_db=float("nan"), silence_dur=0.2, target_sec=20.0):
    """Chunk boundaries of a long recording, [(start, end), ...] in samples
    (hipb_chunk_bounds, host code of libct_hip.so)."""
    if os.environ.get("CT_CHUNK_LIB"):
        lib = C.CDLL(os.environ["CT_CHUNK_LIB"])
        lib.hipb_chunk_bounds.argtypes, lib.hipb_chunk_bounds.restype = _ENGINE_SIGS["hipb_chunk_bounds"]
    else:
        lib = engine_lib()
    samples = np.ascontiguousarray(samples, np.float32)
    cap = len(samples) // HOP_LEN + 1
    b = np.zeros(2 * cap, np.int32)
    n = lib.hipb_chunk_bounds(samples.ctypes.data, len(samples), silence_db, silence_dur, target_sec,
                              b.ctypes.data, cap)
    if n < 0:
        raise MemoryError("hipb_chunk_bounds: out of host memory")
    return [(int(b[2 * i]), int(b[2 * i + 1])) for i in range(n)]


def _engine_chunked(self, pcm, limit, flags=HIPB_SUPPRESS_EOS, prompt=None, silence_db=float("nan"),
                    silence_dur=0.2, target_sec=20.0):
    """Queues a long recording as chained chunk requests; returns their ids."""
    pcm = np.ascontiguousarray(pcm, np.float32)
    p = np.ascontiguousarray(prompt if prompt is not None else PROMPT, dtype=np.int32)
    first = C.c_int(-1)
    n = self.L.hipb_submit_pcm_chunked(self.e, pcm.ctypes.data, len(pcm), p.ctypes.data, len(p), limit,
                                       flags, silence_db, silence_dur, target_sec, C.byref(first))
    return list(range(first.value, first.value + n))


Engine.submit_pcm_chunked = _engine_chunked


def _engine_extra(self, pcm, limit, flags=HIPB_SUPPRESS_EOS, prompt=None):
    pcm = np.ascontiguousarray(pcm, dtype=np.float32)
    p = np.ascontiguousarray(prompt if prompt is not None else PROMPT, dtype=np.int32)
    return self.L.hipb_submit_pcm(self.e, pcm.ctypes.data, len(pcm), p.ctypes.data, len(p), limit, flags)


def _engine_mel(self, pcm):
    pcm = np.ascontiguousarray(pcm, dtype=np.float32)
    out = np.zeros((N_MELS, t_mel(len(pcm))), np.float32)
    self.L.hipb_mel(self.e, pcm.ctypes.data, len(pcm), out.ctypes.data)
    return out


Engine.submit_pcm = _engine_extra
Engine.hold_encoder = lambda self, batches, finished: self.L.hipb_test_hold_encoder(self.e, batches, finished)
Engine.hold_expired = lambda self: bool(self.L.hipb_test_hold_expired(self.e))
Engine.mel = _engine_mel
Engine.reset = lambda self: self.L.hipb_reset(self.e)


class HipEvents:
    """hipEvent timing on a given stream (libamdhip64 through ctypes)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [C.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.rt.hipDeviceSynchronize.argtypes = []

    def event(self):
        ev = C.c_void_p()
        if self.rt.hipEventCreate(C.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev

    def record(self, ev, stream):
        if self.rt.hipEventRecord(ev, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def ms(self, a, b):
        self.rt.hipEventSynchronize(b)
        out = C.c_float()
        self.rt.hipEventElapsedTime(C.byref(out), a, b)
        return out.value

    def sync(self):
        if self.rt.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")
