"""ctypes bindings to the oracle (oracle/liboracle.so) — the checker.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
this; the HIP product path never does.
"""
import ctypes as C
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "cohere-transcribe_amd"))
import ctbind as cb  # noqa: E402

ORACLE_LIB = os.path.join(REPO, "oracle", "liboracle.so")
REF_DIR = os.path.join(REPO, "oracle", "_ref")

_P = C.c_void_p
_I = C.c_int
_F = C.c_float

_SIGS = {
    "orc_layernorm": [_P, _P, _P, _P, _I, _I],
    "orc_linear": [_P, _P, _P, _P, _I, _I, _I],
    "orc_linear_silu": [_P, _P, _P, _P, _I, _I, _I],
    "orc_linear_relu": [_P, _P, _P, _P, _I, _I, _I],
    "orc_linear_fmadd": [_P, _F, _P, _P, _P, _I, _I, _I],
    "orc_add_inplace": [_P, _P, _I],
    "orc_encoder_subsampling": [_P, _I, _I, _P, _I, _P, _P],
    "orc_make_rel_pos_emb": [_P, _I],
    "orc_rel_pos_mhsa": [_P, _P, _I, _P, _P],
    "orc_conformer_conv": [_P, _I, _P, _P],
    "orc_sdp_attn": [_P, _P, _P, _P, _P, _I, _I, _P],
    "orc_embed": [_P, _P, _I, _I, _P, _P, _P, _P],
    "orc_fill_causal_mask": [_P, _I],
    "orc_lm_head": [_P, _P, _P, _P],
    "orc_argmax": [_P, _I, _I],
    "orc_T_enc": [_I],
    "orc_T_mel": [_I],
    "orc_conformer_layer": [_P, _P, _I, _P, _P],
    "orc_encoder_forward": [_P, _I, _I, _P, _P, _P],
    "orc_cross_kv": [_P, _I, _P, _P, _P],
    "orc_transcribe": [_P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P],
    "orc_compute_mel": [_P, _I, _P],
    "orc_mel_filterbank": [_P],
    "orc_chunk_bounds": [_P, _I, _F, _F, _F, _P, _I],
    "orc_round_bf16_n": [_P, C.c_long],
    "orc_set_enc_ffn_bf16": [_I],
}
_RET = {"orc_argmax": _I, "orc_T_enc": _I, "orc_T_mel": _I, "orc_transcribe": _I,
        "orc_chunk_bounds": _I}


def _bind(lib, sigs, rets):
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = rets.get(name, None)
    return lib


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} is not built")
        _oracle = _bind(C.CDLL(ORACLE_LIB), _SIGS, _RET)
    return _oracle


class enc_ffn_bf16:
    """Context: the oracle's encoder FFN linears take bf16-rounded inputs
    (the HIP encoder's single-pass FFN mode) inside the block."""

    def __init__(self, on=True):
        self.on = bool(on)

    def __enter__(self):
        oracle().orc_set_enc_ffn_bf16(int(self.on))
        return self

    def __exit__(self, *exc):
        oracle().orc_set_enc_ffn_bf16(0)
        return False


def ptr(a):
    return a.ctypes.data if a is not None else None


def f32(*shape):
    return np.zeros(shape, dtype=np.float32)


def transcribe(model, mel, limit, suppress=True, force=False, kv_bf16=False,
               prompt=None, want_logits=False):
    """Oracle request: returns (tokens, logits or None, enc_h)."""
    prompt = np.asarray(prompt if prompt is not None else cb.PROMPT, dtype=np.int32)
    T_mel = mel.shape[1]
    toks = np.zeros(limit, dtype=np.int32)
    lg = f32(limit, cb.VOCAB) if want_logits else None
    eh = f32(cb.t_enc(T_mel), cb.DEC_D)
    n = oracle().orc_transcribe(model.weights_ref(), ptr(mel), T_mel, mel.shape[1],
                                ptr(prompt), len(prompt), limit, int(suppress), int(force),
                                int(kv_bf16), ptr(toks), ptr(lg), ptr(eh))
    return toks[:n], (lg[:n] if lg is not None else None), eh


def chunk_bounds(samples, silence_db=float("nan"), silence_dur=0.2, target_sec=20.0):
    """Oracle chunking of a long recording: [(start, end), ...] in samples."""
    samples = np.ascontiguousarray(samples, np.float32)
    cap = len(samples) // 160 + 1
    b = np.zeros(2 * cap, np.int32)
    n = oracle().orc_chunk_bounds(ptr(samples), len(samples), silence_db, silence_dur, target_sec,
                                  ptr(b), cap)
    return [(int(b[2 * i]), int(b[2 * i + 1])) for i in range(n)]


CARRY_MAX = 64


def transcribe_chunked(model, samples, limit, prompt=None, suppress=True, force=False,
                       kv_bf16=False, want_logits=False, **split):
    """Oracle long-audio transcription (transcribe.c:480-533): chunks in
    order, each prompt = prompt[:2] + carry + prompt[2:], carry = the last
    <= 64 generated ids of the previous chunk without its final one
    (transcribe.c:382-387).  Returns [(bounds, prompt, tokens), ...], with
    each chunk's per-token logits appended when want_logits."""
    prompt = list(prompt if prompt is not None else cb.PROMPT)
    out, carry = [], []
    for (a, b) in chunk_bounds(samples, **split):
        p = prompt[:2] + carry + prompt[2:]
        toks, lg, _ = transcribe(model, compute_mel(samples[a:b]), limit, suppress=suppress,
                                 force=force, kv_bf16=kv_bf16, prompt=p, want_logits=want_logits)
        out.append(((a, b), p, toks) + ((lg,) if want_logits else ()))
        n = min(max(len(toks) - 1, 0), CARRY_MAX)
        carry = [int(t) for t in toks[len(toks) - 1 - n:len(toks) - 1]]
    return out


def compute_mel(samples):
    T = cb.t_mel(len(samples))
    mel = f32(cb.N_MELS, T)
    oracle().orc_compute_mel(ptr(samples), len(samples), ptr(mel))
    return mel


class OracleABI:
    """The oracle behind the backend ABI's names, for kernel_suite.run_suite.

    Stateless functions map to orc_*; the stateful ones keep the reference
    CPU backend's thread-local latches (backends/cpu/backend.c:27-33, 393-396)
    in Python and loop over items as backends/cpu/backend.c:425-500 do."""

    def __init__(self):
        self.o = oracle()
        self.S = 0
        self.tokens = np.zeros(cb.MAX_SEQ, np.int32)
        self.S_batch = np.zeros(256, np.int32)
        self.T_enc = np.zeros(256, np.int32)
        for n in ("layernorm", "linear", "linear_silu", "linear_relu", "linear_fmadd",
                  "add_inplace", "encoder_subsampling", "make_rel_pos_emb", "rel_pos_mhsa",
                  "conformer_conv", "sdp_attn", "embed", "fill_causal_mask", "lm_head"):
            setattr(self, "backend_" + n, getattr(self.o, "orc_" + n))

    @staticmethod
    def _ints(p, n):
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_int)), shape=(n,)).copy()

    def backend_upload_tokens(self, p, S):
        self.tokens[:S] = self._ints(p, S)

    def backend_decode_set_S(self, n):
        self.S = n

    def backend_decode_inc_S(self):
        self.S += 1

    def backend_linear_to_kvcache(self, cache, x, W, b, in_d, out_d):
        self.o.orc_linear(cache + (self.S - 1) * out_d * 4, x, W, b, 1, in_d, out_d)

    def backend_sdp_attn_devS(self, out, q, k, v, work):
        self.o.orc_sdp_attn(out, q, k, v, None, 1, self.S, work)

    def backend_embed_decode(self, h, etw, epw, elnw, elnb):
        self.o.orc_embed(h, self.tokens.ctypes.data, 1, self.S - 1, etw, epw, elnw, elnb)

    def backend_embed_decode_batch(self, h, tokens, S_dev, active, B, etw, epw, elnw, elnb):
        S = self._ints(S_dev, B)
        act = self._ints(active, B)
        tk = self._ints(tokens, B)
        self.S_batch[:B] = S
        for b in range(B):
            if act[b]:
                t1 = np.array([tk[b]], np.int32)
                self.o.orc_embed(h + b * cb.DEC_D * 4, t1.ctypes.data, 1, int(S[b]) - 1,
                                 etw, epw, elnw, elnb)

    def backend_upload_T_enc(self, p, B):
        self.T_enc[:B] = self._ints(p, B)

    def backend_linear_to_kvcache_batch(self, cache, x, W, b, B, stride, in_d, out_d):
        for i in range(B):
            dst = cache + ((i * stride) + int(self.S_batch[i]) - 1) * out_d * 4
            self.o.orc_linear(dst, x + i * in_d * 4, W, b, 1, in_d, out_d)

    def _batch_attn(self, out, Q, K, V, stride, B, lens):
        for i in range(B):
            self.o.orc_sdp_attn(out + i * cb.DEC_D * 4, Q + i * cb.DEC_D * 4,
                                K + i * stride * cb.DEC_D * 4, V + i * stride * cb.DEC_D * 4,
                                None, 1, int(lens[i]), None)

    def backend_sdp_attn_batch_decode_sa(self, out, Q, K, V, stride, B, work):
        self._batch_attn(out, Q, K, V, stride, B, self.S_batch)

    def backend_sdp_attn_batch_decode_ca(self, out, Q, K, V, stride, B, work):
        self._batch_attn(out, Q, K, V, stride, B, self.T_enc)

    def backend_lm_head_batch(self, logits, h, etw, hdb, active, B):
        act = self._ints(active, B)
        for b in range(B):
            if act[b]:
                self.o.orc_lm_head(logits + b * cb.VOCAB * 4, h + b * cb.DEC_D * 4, etw, hdb)

    def backend_argmax_batch(self, out, logits, active, B):
        act = self._ints(active, B)
        res = np.ctypeslib.as_array(C.cast(out, C.POINTER(C.c_int)), shape=(B,))
        for b in range(B):
            if act[b]:
                res[b] = self.o.orc_argmax(logits + b * cb.VOCAB * 4, cb.VOCAB, -1)
