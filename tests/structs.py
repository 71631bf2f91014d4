"""ctypes mirrors of the C structs the tests pass to libct_hip.so's kernel
entry points (cohere-transcribe_amd/csrc/ct_launch.h).  The library reports
each struct's size (ctk_gemv_sizeof, ctk_warmset_sizeof, ctk_gemm_sizeof), and tests/test_abi_exports.py checks
the mirror against it on the CPU, so a field added on one side only fails
there before any kernel reads past a mirror."""
import ctypes as C


class CtGemv(C.Structure):
    _fields_ = [("A", C.c_void_p), ("W", C.c_void_p), ("bias", C.c_void_p),
                ("M", C.c_int), ("N", C.c_int), ("K", C.c_int), ("ksplit", C.c_int),
                ("out", C.c_int), ("relu", C.c_int),
                ("Y", C.c_void_p), ("ldy", C.c_long), ("F", C.c_void_p),
                ("kc", C.c_void_p), ("vc", C.c_void_p), ("rowoff", C.c_void_p),
                ("hstride", C.c_long), ("kv_bf16", C.c_int), ("wtile", C.c_int),
                ("m_active", C.c_void_p), ("lnstat", C.c_void_p), ("fold_w", C.c_void_p),
                ("fold_c1", C.c_void_p), ("fold_c2", C.c_void_p)]


class CtWarm(C.Structure):
    _fields_ = [("W", C.c_void_p), ("gx", C.c_int), ("gy", C.c_int), ("cb", C.c_int),
                ("per", C.c_int), ("nsteps", C.c_int), ("heads", C.c_int)]


class CtWarmSet(C.Structure):
    _fields_ = [("t", CtWarm * 4), ("n", C.c_int), ("rows", C.c_int), ("magic", C.c_uint),
                ("sink", C.c_void_p)]


class CtSeg(C.Structure):
    _fields_ = [("mode", C.c_int), ("base", C.c_void_p), ("ld", C.c_long), ("base_lo", C.c_void_p),
                ("rowoff", C.c_void_p), ("hstride", C.c_long)]


class CtGemm(C.Structure):
    _fields_ = [("A", C.c_void_p), ("lda", C.c_long), ("Ahi", C.c_void_p), ("Alo", C.c_void_p),
                ("W", C.c_void_p), ("bias", C.c_void_p), ("Y", C.c_void_p), ("ldy", C.c_long),
                ("M", C.c_int), ("N", C.c_int), ("K", C.c_int), ("epi", C.c_int), ("scale", C.c_float),
                ("row_len", C.c_void_p), ("row_len_step", C.c_int), ("row_stride", C.c_long),
                ("glu_half", C.c_int), ("row_mask", C.c_void_p), ("nseg", C.c_int), ("seg_w", C.c_int),
                ("seg", CtSeg * 3)]

