"""ctypes loader for the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  It wraps oracle/liboracle.so (the C restatement in
swiftkv_oracle.c) and, when built, oracle/_ref/libswiftkv_ref*.so (the
reference emulator's attention stage, compiled from the reference sources).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
HD, PAIRS, G32, NGROUPS = 128, 64, 32, 4

_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i16p = np.ctypeslib.ndpointer(np.int16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def _load(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
    return C.CDLL(path)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    L = _load(os.path.join(_HERE, "liboracle.so"))
    L.oracle_f2q17.restype = C.c_int32
    L.oracle_f2q17.argtypes = [C.c_float]
    L.oracle_f2q17_array.argtypes = [_f32p, _i32p, C.c_int64]
    L.oracle_reduce_partials.argtypes = [_f32p, C.c_int, C.c_int64, _f32p, C.c_int64]
    L.oracle_finalize_partials.argtypes = [_f32p, C.c_int, C.c_int64, _i32p, C.c_int64]
    L.oracle_f2q17_digest.restype = C.c_uint64
    L.oracle_f2q17_digest.argtypes = [C.c_uint64, C.c_uint64]
    L.oracle_rne_shift.restype = C.c_int64
    L.oracle_rne_shift.argtypes = [C.c_int64, C.c_uint]
    L.oracle_wrap.restype = C.c_int64
    L.oracle_wrap.argtypes = [C.c_int64, C.c_uint]
    L.oracle_rope_values.argtypes = [C.c_int, C.c_int, C.c_double, _i32p, _i32p]
    L.oracle_rope_pack.argtypes = [C.c_int, _i32p, _i32p, _u8p]
    L.oracle_rope_unpack.argtypes = [C.c_int, _u8p, _i32p, _i32p]
    L.oracle_rope_rotate.argtypes = [_i32p, _i32p, _i32p]
    L.oracle_g32_shift.restype = C.c_uint8
    L.oracle_g32_shift.argtypes = [_i32p]
    L.oracle_g32_code.restype = C.c_int8
    L.oracle_g32_code.argtypes = [C.c_int32, C.c_uint8]
    L.oracle_quantize_row.argtypes = [_i32p, _i8p, _u8p]
    L.oracle_quantize_rows.argtypes = [_i32p, C.c_int64, _i8p, _u8p]
    L.oracle_rope_rotate_rows.argtypes = [_i32p, C.c_int64, _i32p, _i32p]
    L.oracle_shift_scale.restype = C.c_float
    L.oracle_shift_scale.argtypes = [C.c_uint8]
    L.oracle_pack_record.argtypes = [_i8p, _u8p, _i8p, _u8p, _u8p]
    L.oracle_unpack_record.argtypes = [_u8p, _i8p, _u8p, _i8p, _u8p]
    L.oracle_exp_neg_q17.restype = C.c_uint32
    L.oracle_exp_neg_q17.argtypes = [C.c_int32]
    L.oracle_attend_head_int.argtypes = [_i32p, _i8p, _u8p, _i8p, _u8p, C.c_int, _i32p]
    L.oracle_attend_head_fp.argtypes = [_i32p, _i8p, _u8p, _i8p, _u8p, C.c_int, _f64p]
    L.oracle_a14_group.argtypes = [_f32p, _i16p, _u8p]
    L.oracle_a14_group_q17.argtypes = [_i32p, _i16p, _u8p]
    L.oracle_pack_a14.argtypes = [_i16p, _u8p]
    L.oracle_step_q17.argtypes = [
        C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p, _i32p, C.c_int,
        _i8p, _u8p, _i8p, _u8p, C.c_void_p, C.c_void_p, C.c_void_p]
    L.oracle_fill_q17.argtypes = [
        C.c_int, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p,
        _i8p, _u8p, _i8p, _u8p]
    L.oracle_kat_pe0.argtypes = [_i32p, _i32p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- primitives
def f2q17(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.int32)
    lib().oracle_f2q17_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def reduce_partials(parts: np.ndarray) -> np.ndarray:
    """FP32 split-K partials [P][...] (P = 1, 2 or 4) reduced as the linear
    stage does (int4_linear_controller.cpp:1039-1054, 1655-1667, 1100-1118)."""
    p = np.ascontiguousarray(parts, dtype=np.float32)
    n = p[0].size
    out = np.empty(p.shape[1:], np.float32)
    lib().oracle_reduce_partials(p.reshape(-1), p.shape[0], n, out.reshape(-1), n)
    return out


def finalize_partials(parts: np.ndarray) -> np.ndarray:
    """Q15.17 of reduce_partials(parts): the Q/K/V finalize (:1100-1118)."""
    p = np.ascontiguousarray(parts, dtype=np.float32)
    n = p[0].size
    out = np.empty(p.shape[1:], np.int32)
    lib().oracle_finalize_partials(p.reshape(-1), p.shape[0], n, out.reshape(-1), n)
    return out


def f2q17_digest(lo: int, hi: int) -> int:
    return int(lib().oracle_f2q17_digest(lo, hi))


def rope_values(npos: int, pos0: int = 0, theta: float = 10000.0):
    c = np.empty((npos, PAIRS), np.int32)
    s = np.empty((npos, PAIRS), np.int32)
    lib().oracle_rope_values(pos0, npos, theta, c.reshape(-1), s.reshape(-1))
    return c, s


def rope_pack(cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    npos = cos.shape[0]
    out = np.empty(npos * 512, np.uint8)
    lib().oracle_rope_pack(npos, np.ascontiguousarray(cos, np.int32).reshape(-1),
                           np.ascontiguousarray(sin, np.int32).reshape(-1), out)
    return out


def rope_unpack(buf: np.ndarray):
    buf = np.ascontiguousarray(buf, np.uint8)
    npos = buf.size // 512
    c = np.empty((npos, PAIRS), np.int32)
    s = np.empty((npos, PAIRS), np.int32)
    lib().oracle_rope_unpack(npos, buf, c.reshape(-1), s.reshape(-1))
    return c, s


def rope_rotate(x: np.ndarray, cos64: np.ndarray, sin64: np.ndarray) -> np.ndarray:
    """Rotate every 128-channel head row of x (int32, [..., 128]).  cos64/sin64
    are one table row [64] for all rows, or one per row [..., 64]."""
    x = np.array(x, dtype=np.int32, copy=True)
    rows = np.ascontiguousarray(x.reshape(-1, HD))
    n = rows.shape[0]
    c = np.ascontiguousarray(np.broadcast_to(np.asarray(cos64, np.int32).reshape(-1, PAIRS), (n, PAIRS)))
    s = np.ascontiguousarray(np.broadcast_to(np.asarray(sin64, np.int32).reshape(-1, PAIRS), (n, PAIRS)))
    lib().oracle_rope_rotate_rows(rows.reshape(-1), n, c.reshape(-1), s.reshape(-1))
    return rows.reshape(x.shape)


def quantize_rows(x: np.ndarray):
    """G32-quantize int32 rows [..., 128] -> (codes int8 [...,128], shifts uint8 [...,4])."""
    x = np.ascontiguousarray(x, np.int32)
    rows = x.reshape(-1, HD)
    codes = np.empty(rows.shape, np.int8)
    shifts = np.empty((rows.shape[0], NGROUPS), np.uint8)
    lib().oracle_quantize_rows(rows.reshape(-1), rows.shape[0], codes.reshape(-1), shifts.reshape(-1))
    return codes.reshape(x.shape), shifts.reshape(x.shape[:-1] + (NGROUPS,))


def shift_scale_bits(shifts: np.ndarray) -> np.ndarray:
    """FP32 bit pattern of 2^(s-17) for each shift (exactly representable)."""
    return ((shifts.astype(np.uint32) + np.uint32(110)) << np.uint32(23)).astype(np.uint32)


def exp_neg_q17(x: int) -> int:
    return int(lib().oracle_exp_neg_q17(int(x)))


def attend_head_fp(q, kc, ks, vc, vs) -> np.ndarray:
    out = np.empty(HD, np.float64)
    n = kc.shape[0]
    lib().oracle_attend_head_fp(np.ascontiguousarray(q, np.int32), np.ascontiguousarray(kc, np.int8),
                                np.ascontiguousarray(ks, np.uint8), np.ascontiguousarray(vc, np.int8),
                                np.ascontiguousarray(vs, np.uint8), n, out)
    return out


def attend_head_int(q, kc, ks, vc, vs) -> np.ndarray:
    out = np.empty(HD, np.int32)
    n = kc.shape[0]
    lib().oracle_attend_head_int(np.ascontiguousarray(q, np.int32), np.ascontiguousarray(kc, np.int8),
                                 np.ascontiguousarray(ks, np.uint8), np.ascontiguousarray(vc, np.int8),
                                 np.ascontiguousarray(vs, np.uint8), n, out)
    return out


def a14(x: np.ndarray):
    """A14/E8M0 of float values [..., 32] -> (int16 [..., 32], uint8 [...])."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.reshape(-1, G32)
    q = np.empty(rows.shape, np.int16)
    e = np.empty(rows.shape[0], np.uint8)
    for r in range(rows.shape[0]):
        qr = np.empty(G32, np.int16)
        er = np.empty(1, np.uint8)
        lib().oracle_a14_group(np.ascontiguousarray(rows[r]), qr, er)
        q[r] = qr
        e[r] = er[0]
    return q.reshape(x.shape), e.reshape(x.shape[:-1])


def a14_q17(raw: np.ndarray):
    """Integer-path A14/E8M0 of Q15.17 values [..., 32] -> (int16 [..., 32], uint8 [...])."""
    raw = np.ascontiguousarray(raw, np.int32)
    rows = raw.reshape(-1, G32)
    q = np.empty(rows.shape, np.int16)
    e = np.empty(rows.shape[0], np.uint8)
    for r in range(rows.shape[0]):
        qr = np.empty(G32, np.int16)
        er = np.empty(1, np.uint8)
        lib().oracle_a14_group_q17(np.ascontiguousarray(rows[r]), qr, er)
        q[r] = qr
        e[r] = er[0]
    return q.reshape(raw.shape), e.reshape(raw.shape[:-1])


def pack_a14(q14: np.ndarray) -> np.ndarray:
    rows = np.ascontiguousarray(q14, np.int16).reshape(-1, G32)
    out = np.empty((rows.shape[0], 56), np.uint8)
    for r in range(rows.shape[0]):
        w = np.empty(56, np.uint8)
        lib().oracle_pack_a14(np.ascontiguousarray(rows[r]), w)
        out[r] = w
    return out.reshape(q14.shape[:-1] + (56,))


def pack_record(kc, ks, vc, vs) -> np.ndarray:
    rec = np.empty(320, np.uint8)
    lib().oracle_pack_record(np.ascontiguousarray(kc, np.int8), np.ascontiguousarray(ks, np.uint8),
                             np.ascontiguousarray(vc, np.int8), np.ascontiguousarray(vs, np.uint8), rec)
    return rec


def unpack_record(rec):
    kc = np.empty(HD, np.int8)
    vc = np.empty(HD, np.int8)
    ks = np.empty(NGROUPS, np.uint8)
    vs = np.empty(NGROUPS, np.uint8)
    lib().oracle_unpack_record(np.ascontiguousarray(rec, np.uint8), kc, ks, vc, vs)
    return kc, ks, vc, vs


def kat_pe0(cos: np.ndarray, sin: np.ndarray):
    h0 = C.c_uint64()
    h1 = C.c_uint64()
    lib().oracle_kat_pe0(np.ascontiguousarray(cos, np.int32).reshape(-1),
                         np.ascontiguousarray(sin, np.int32).reshape(-1), C.byref(h0), C.byref(h1))
    return int(h0.value), int(h1.value)


class SequenceCache:
    """Host cache of one sequence, one layer: codes [heads][cap][128], shifts [heads][cap][4]."""

    def __init__(self, heads: int, cap: int):
        self.heads, self.cap = heads, cap
        self.kc = np.zeros((heads, cap, HD), np.int8)
        self.vc = np.zeros((heads, cap, HD), np.int8)
        self.ks = np.zeros((heads, cap, NGROUPS), np.uint8)
        self.vs = np.zeros((heads, cap, NGROUPS), np.uint8)

    def fill_q17(self, k_q17: np.ndarray, v_q17: np.ndarray, pos0: int, cos_tab, sin_tab):
        """Append rule for tokens [pos0, pos0+n): k/v int32 [n][heads*128]."""
        n = k_q17.shape[0]
        lib().oracle_fill_q17(self.heads, self.cap, n, pos0,
                              np.ascontiguousarray(k_q17, np.int32).reshape(-1),
                              np.ascontiguousarray(v_q17, np.int32).reshape(-1),
                              np.ascontiguousarray(cos_tab, np.int32).reshape(-1),
                              np.ascontiguousarray(sin_tab, np.int32).reshape(-1),
                              self.kc.reshape(-1), self.ks.reshape(-1), self.vc.reshape(-1), self.vs.reshape(-1))

    def step_q17(self, q, k, v, pos: int, cos64, sin64, fp: bool = True, integer: bool = False):
        """One decode step: returns dict with qrot [heads,128], fp [heads,128] float64, int."""
        H = self.heads
        qrot = np.empty((H, HD), np.int32)
        fp_out = np.empty((H, HD), np.float64) if fp else None
        int_out = np.empty((H, HD), np.int32) if integer else None
        lib().oracle_step_q17(H, self.cap,
                              np.ascontiguousarray(q, np.int32).reshape(-1),
                              np.ascontiguousarray(k, np.int32).reshape(-1),
                              np.ascontiguousarray(v, np.int32).reshape(-1),
                              np.ascontiguousarray(cos64, np.int32).reshape(-1),
                              np.ascontiguousarray(sin64, np.int32).reshape(-1), pos,
                              self.kc.reshape(-1), self.ks.reshape(-1), self.vc.reshape(-1), self.vs.reshape(-1),
                              _ptr(qrot), _ptr(fp_out), _ptr(int_out))
        return {"qrot": qrot, "fp": fp_out, "int": int_out}


# ------------------------------------------------------------- reference build
class Reference:
    """The reference emulator's attention stage compiled from its own source."""

    def __init__(self, omp: bool = False):
        name = "libswiftkv_ref_omp.so" if omp else "libswiftkv_ref.so"
        L = _load(os.path.join(_HERE, "_ref", name))
        L.ref_float_to_q17.restype = C.c_int32
        L.ref_float_to_q17.argtypes = [C.c_float]
        L.ref_float_to_q17_array.argtypes = [_f32p, _i32p, C.c_int64]
        L.ref_exp_negative_q17.restype = C.c_uint32
        L.ref_exp_negative_q17.argtypes = [C.c_int32]
        L.ref_shift_for_group.restype = C.c_uint8
        L.ref_shift_for_group.argtypes = [_i32p]
        L.ref_quantize_raw.restype = C.c_int8
        L.ref_quantize_raw.argtypes = [C.c_int32, C.c_uint8]
        L.ref_set_rope.argtypes = [_i32p, _i32p, C.c_int]
        L.ref_apply_rope.argtypes = [_i32p, C.c_int]
        L.ref_cache_create.restype = C.c_void_p
        L.ref_cache_create.argtypes = [C.c_int]
        L.ref_cache_destroy.argtypes = [C.c_void_p]
        L.ref_cache_row.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, _i8p, _u8p, _i8p, _u8p]
        L.ref_cache_rows.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, _i8p, _u8p, _i8p, _u8p]
        L.ref_attention.argtypes = [C.c_void_p, _i32p, _i32p, _i32p, C.c_int, _i16p, _f32p]
        L.ref_omp_threads.restype = C.c_int
        self.L = L

    @staticmethod
    def available(omp: bool = False) -> bool:
        name = "libswiftkv_ref_omp.so" if omp else "libswiftkv_ref.so"
        return os.path.exists(os.path.join(_HERE, "_ref", name))

    def f2q17(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.int32)
        self.L.ref_float_to_q17_array(x.reshape(-1), out.reshape(-1), x.size)
        return out

    def set_rope(self, cos, sin):
        self.L.ref_set_rope(np.ascontiguousarray(cos, np.int32).reshape(-1),
                            np.ascontiguousarray(sin, np.int32).reshape(-1), cos.shape[0])

    def apply_rope(self, vec4096: np.ndarray, pos: int) -> np.ndarray:
        x = np.array(vec4096, np.int32, copy=True)
        self.L.ref_apply_rope(x, pos)
        return x

    def cache(self, seq_len: int):
        return _RefCache(self.L, seq_len)


class _RefCache:
    def __init__(self, L, seq_len):
        self.L = L
        self.h = L.ref_cache_create(seq_len)
        self.seq_len = seq_len

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_cache_destroy(self.h)
            self.h = None

    def load_from(self, sc: SequenceCache, ntok: int):
        for h in range(sc.heads):
            self.L.ref_cache_rows(self.h, h, 0, ntok, np.ascontiguousarray(sc.kc[h, :ntok]),
                                  np.ascontiguousarray(sc.ks[h, :ntok]), np.ascontiguousarray(sc.vc[h, :ntok]),
                                  np.ascontiguousarray(sc.vs[h, :ntok]))

    def row(self, head: int, token: int):
        kc = np.empty(HD, np.int8)
        vc = np.empty(HD, np.int8)
        ks = np.empty(NGROUPS, np.uint8)
        vs = np.empty(NGROUPS, np.uint8)
        self.L.ref_cache_row(self.h, 1, head, token, kc, ks, vc, vs)
        return kc, ks, vc, vs

    def attention(self, qrot, krot, v, pos):
        aq = np.empty(4096, np.int16)
        asc = np.empty(128, np.float32)
        self.L.ref_attention(self.h, np.ascontiguousarray(qrot, np.int32).reshape(-1),
                             np.ascontiguousarray(krot, np.int32).reshape(-1),
                             np.ascontiguousarray(v, np.int32).reshape(-1), pos, aq, asc)
        return aq, asc
