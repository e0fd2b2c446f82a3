"""Python host mirror of the SwiftKV decode-attention stage (ctypes over libswiftkv.so).

Mirrors the reference's local-PE attention entry
    int4_swiftkv_attention_pe{0..3}(q, k, v, kv_cache, rope_lut_ddr,
                                    activation_q, activation_scale,
                                    layer_index, position)
(kernel_HLS/swiftkv_attention.hpp:167-209) with the same argument meaning: the
KV cache and the RoPE table are persistent device objects owned by the caller,
`position` is the cached-token count (the step writes that token and attends
[0, position]), and the outputs are the FP32 attention result plus the optional
A14/E8M0 activation words for the O projection.  All 32 heads of a layer run on
one GPU; a batch of sequences runs in one call.

Follows the repo precedent of reaching native code through ctypes
(run_autoround.py:5-21).  There is no CPU fallback: importing this module
without the built library raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from typing import Optional, Sequence

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libswiftkv.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "swiftkv.h")

HEADS = 32
HEAD_DIM = 128
MODEL_DIM = HEADS * HEAD_DIM
GROUP = 32
GROUPS_PER_HEAD = HEAD_DIM // GROUP
REFERENCE_MAX_SEQ = 4096
MAX_SEQ = 32768
ROPE_LUT_BYTES_PER_POSITION = 512
RECORD_BYTES = 320
A14_WORD_BYTES = 56
TOKEN_BYTES = 288          # algorithmic bytes per cached token-head: 2 x 128 codes + 8 FP32 scales

OK, EINVAL, ERANGE, EHIP, ENOMEM, ESTATE = 0, -1, -2, -3, -4, -5
DIST_NORMAL, DIST_STUDENT_T3 = 0, 1
KERNEL_APPEND, KERNEL_STEP, KERNEL_EXACT = 0, 1, 2
KERNEL_KINDS = 3
_STATUS_NAMES = {EINVAL: "EINVAL", ERANGE: "ERANGE", EHIP: "EHIP", ENOMEM: "ENOMEM", ESTATE: "ESTATE"}


class SwiftKVError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"swiftkv error {code} ({_STATUS_NAMES.get(code, '?')}): {message}")
        self.code = code


_vp = C.c_void_p
_i32 = C.c_int32
_sz = C.c_size_t

# name -> (restype, argtypes); every declaration of include/swiftkv.h.
_SIGNATURES = {
    "swiftkv_last_error": (C.c_char_p, []),
    "swiftkv_version": (C.c_char_p, []),
    "swiftkv_context_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "swiftkv_context_destroy": (C.c_int, [_vp]),
    "swiftkv_synchronize": (C.c_int, [_vp]),
    "swiftkv_set_split_tokens": (C.c_int, [_vp, _i32]),
    "swiftkv_debug_set_split_generation": (C.c_int, [_vp, C.c_uint32, _i32]),
    "swiftkv_debug_force_merge_timeout": (C.c_int, [_vp, _i32]),
    "swiftkv_debug_set_step_shape": (C.c_int, [_vp, _i32, _i32]),
    "swiftkv_debug_step_plan": (C.c_int, [_i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "swiftkv_rope_lut_load": (C.c_int, [_vp, _vp, _sz, C.POINTER(_vp)]),
    "swiftkv_rope_lut_generate": (C.c_int, [_vp, _i32, C.c_double, C.POINTER(_vp)]),
    "swiftkv_rope_lut_destroy": (C.c_int, [_vp]),
    "swiftkv_rope_lut_positions": (_i32, [_vp]),
    "swiftkv_rope_lut_export": (C.c_int, [_vp, _i32, _i32, _vp]),
    "swiftkv_kv_cache_create": (C.c_int, [_vp, _i32, _i32, _i32, C.POINTER(_vp)]),
    "swiftkv_kv_cache_destroy": (C.c_int, [_vp]),
    "swiftkv_kv_cache_zero": (C.c_int, [_vp, _vp]),
    "swiftkv_kv_cache_bytes": (_sz, [_vp]),
    "swiftkv_kv_cache_read": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "swiftkv_kv_cache_export_records": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "swiftkv_kv_cache_import_records": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "swiftkv_attention_f32": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp]),
    "swiftkv_attention_q17": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp]),
    "swiftkv_attention_f32_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp]),
    "swiftkv_attention_partials": (C.c_int, [_vp, _vp, _vp, _vp, _i32, C.c_int64, _vp, _vp, _vp, _vp, _i32, _vp,
                                             _i32, _vp]),
    "swiftkv_set_host_io": (C.c_int, [_vp, _i32]),
    "swiftkv_attention_exact": (C.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp]),
    "swiftkv_append_tokens": (C.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32]),
    "swiftkv_fill_synthetic_f32": (C.c_int, [_vp, _vp, _sz, C.c_uint64, C.c_uint64, C.c_uint64, _i32, _i32]),
    "swiftkv_kv_cache_fill_synthetic": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, C.c_uint64,
                                                  _i32, _i32]),
    "swiftkv_device_alloc": (C.c_int, [_vp, _sz, C.POINTER(_vp)]),
    "swiftkv_device_free": (C.c_int, [_vp, _vp]),
    "swiftkv_memcpy_h2d": (C.c_int, [_vp, _vp, _vp, _sz]),
    "swiftkv_memcpy_d2h": (C.c_int, [_vp, _vp, _vp, _sz]),
    "swiftkv_memset_d": (C.c_int, [_vp, _vp, C.c_int, _sz]),
    "swiftkv_convert_f32_q17": (C.c_int, [_vp, _vp, _vp, _sz]),
    "swiftkv_convert_partials_q17": (C.c_int, [_vp, _vp, _i32, C.c_int64, _vp, _sz]),
    "swiftkv_a14_unpack": (C.c_int, [_vp, _sz, _vp]),
    "swiftkv_a14_decode": (C.c_int, [_vp, _vp, _sz, _vp]),
    "swiftkv_capture_begin": (C.c_int, [_vp]),
    "swiftkv_capture_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "swiftkv_graph_launch": (C.c_int, [_vp, _vp]),
    "swiftkv_graph_destroy": (C.c_int, [_vp]),
    "swiftkv_timer_record": (C.c_int, [_vp, _i32]),
    "swiftkv_timer_elapsed": (C.c_int, [_vp, _i32, _i32, C.POINTER(C.c_float)]),
    "swiftkv_profile_enable": (C.c_int, [_vp, _i32]),
    "swiftkv_profile_collect": (C.c_int, [_vp, C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
}

_lib: Optional[C.CDLL] = None


def header_symbols() -> list:
    """Function names declared in include/swiftkv.h."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(swiftkv_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    """Load libswiftkv.so; raises if it has not been built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python 4pe_u250_amd/build.py` "
                          "(or __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != OK:
        msg = lib().swiftkv_last_error()
        raise SwiftKVError(rc, msg.decode() if msg else "")


def _host_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


_INT32_MIN, _INT32_MAX = -(1 << 31), (1 << 31) - 1


def _positions(ctx: "Context", position):
    """(address, count, owner) of a step's positions as int32, `owner` keeping
    the memory alive across the call.  A single position (the latency-bound
    batch-1 step) goes through the context's one-element buffer: building a
    numpy array and its ctypes view cost several microseconds per call, more
    than a short step takes on the GPU."""
    if isinstance(position, (int, np.integer)) and _INT32_MIN <= position <= _INT32_MAX:
        buf = ctx._one_position
        buf[0] = int(position)
        return C.addressof(buf), 1, buf
    pos = np.ascontiguousarray(np.atleast_1d(np.asarray(position, dtype=np.int32)))
    return pos.ctypes.data, int(pos.size), pos


class DeviceBuffer:
    """A device allocation with numpy-style upload/download (no framework needed)."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        # The C context outlives Context.close() while this buffer exists, so
        # the buffer keeps the raw handle to free itself later.
        self._ctx_handle = ctx.handle
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib().swiftkv_device_alloc(ctx.handle, self.nbytes, C.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, ctx: "Context", a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(ctx, a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload exceeds the buffer")
        _check(lib().swiftkv_memcpy_h2d(self.ctx.handle, C.c_void_p(self.ptr + offset), _host_ptr(a), a.nbytes))

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds the buffer")
        _check(lib().swiftkv_memcpy_d2h(self.ctx.handle, _host_ptr(out), C.c_void_p(self.ptr + offset), out.nbytes))
        return out

    def zero(self) -> None:
        _check(lib().swiftkv_memset_d(self.ctx.handle, C.c_void_p(self.ptr), 0, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            ptr, self.ptr = self.ptr, None
            _check(lib().swiftkv_device_free(self._ctx_handle, C.c_void_p(ptr)))

    def __del__(self):
        try:
            if self.ptr:
                lib().swiftkv_device_free(self._ctx_handle, C.c_void_p(self.ptr))
        except Exception:
            pass


class Context:
    """Device, HIP stream and workspace (one per GPU, not thread-safe)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().swiftkv_context_create(device, C.byref(h)))
        self.handle = h.value
        self.device = device
        self.host_io = False
        self._one_position = (C.c_int32 * 1)()

    def close(self) -> None:
        if self.handle:
            _check(lib().swiftkv_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self) -> None:
        _check(lib().swiftkv_synchronize(self.handle))

    def set_split_tokens(self, n: int) -> None:
        _check(lib().swiftkv_set_split_tokens(self.handle, int(n)))

    def debug_set_split_generation(self, generation: int, noalloc: bool = False) -> None:
        """Testing aid: set every generation of the split workspace (the
        context's, or with noalloc this device's allocation-free one) and zero
        its partial words, so launches can be run across the tag wrap."""
        _check(lib().swiftkv_debug_set_split_generation(self.handle, int(generation), 1 if noalloc else 0))

    def debug_force_merge_timeout(self, enable: bool) -> None:
        """Testing aid: while enabled, every split merge of this context's step
        launches gives up after one poll (NaN in the merged heads' outputs,
        SwiftKVError EHIP from the next synchronize, step or graph launch)."""
        _check(lib().swiftkv_debug_force_merge_timeout(self.handle, 1 if enable else 0))

    def debug_set_step_shape(self, waves: int = 0, block_tokens: int = 0) -> None:
        """Testing aid: force the step kernel's shape (waves per workgroup,
        tokens per block: (4, 64), (8, 32) or (8, 64)) for later step launches;
        waves = 0 returns to the launch plan's choice."""
        _check(lib().swiftkv_debug_set_step_shape(self.handle, int(waves), int(block_tokens)))

    def set_host_io(self, enable: bool) -> None:
        """Host-memory I/O: step and append tensors are numpy arrays, staged
        through the device by the library; each call returns with its outputs
        written back."""
        _check(lib().swiftkv_set_host_io(self.handle, 1 if enable else 0))
        self.host_io = bool(enable)

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        return DeviceBuffer.from_array(self, a)

    def capture_begin(self) -> None:
        _check(lib().swiftkv_capture_begin(self.handle))

    def capture_end(self) -> "Graph":
        g = C.c_void_p()
        _check(lib().swiftkv_capture_end(self.handle, C.byref(g)))
        return Graph(self, g.value)

    def timer_record(self, slot: int) -> None:
        _check(lib().swiftkv_timer_record(self.handle, slot))

    def timer_elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        _check(lib().swiftkv_timer_elapsed(self.handle, a, b, C.byref(ms)))
        return float(ms.value)

    def profile(self, on: bool) -> None:
        _check(lib().swiftkv_profile_enable(self.handle, 1 if on else 0))

    def profile_collect(self):
        counts = (C.c_int64 * KERNEL_KINDS)()
        ms = (C.c_double * KERNEL_KINDS)()
        _check(lib().swiftkv_profile_collect(self.handle, counts, ms))
        return list(counts), list(ms)

    def fill_synthetic(self, dst: DeviceBuffer, n: int, seed: int, stream: int, dist: int = DIST_NORMAL,
                       outliers: bool = False, first: int = 0) -> None:
        """Elements [first, first+n) of the synthetic stream (seed, stream) as FP32 into dst."""
        _check(lib().swiftkv_fill_synthetic_f32(self.handle, C.c_void_p(dst.ptr), n, first, seed, stream, dist,
                                                1 if outliers else 0))

    def convert_f32_q17(self, src: DeviceBuffer, dst: DeviceBuffer, n: int) -> None:
        _check(lib().swiftkv_convert_f32_q17(self.handle, C.c_void_p(src.ptr), C.c_void_p(dst.ptr), n))

    def convert_partials_q17(self, src: DeviceBuffer, dst: DeviceBuffer, n: int, parts: int,
                             part_stride: Optional[int] = None) -> None:
        """The linear stage's finalize: Q15.17 of `parts` FP32 partials reduced
        in the reference's order; part p of element i at src[i + p * part_stride]
        (default part_stride = n)."""
        stride = n if part_stride is None else int(part_stride)
        _check(lib().swiftkv_convert_partials_q17(self.handle, C.c_void_p(src.ptr), int(parts), stride,
                                                  C.c_void_p(dst.ptr), n))


class Graph:
    """A recorded sequence of asynchronous calls, replayed with one launch."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self) -> None:
        _check(lib().swiftkv_graph_launch(self.ctx.handle, self.handle))

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            _check(lib().swiftkv_graph_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RopeLut:
    """Device RoPE table (rope_lut.bin format: 512 bytes per position)."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle

    @classmethod
    def load(cls, ctx: Context, image: bytes) -> "RopeLut":
        buf = np.frombuffer(image, np.uint8)
        h = C.c_void_p()
        _check(lib().swiftkv_rope_lut_load(ctx.handle, _host_ptr(buf), buf.nbytes, C.byref(h)))
        return cls(ctx, h.value)

    @classmethod
    def generate(cls, ctx: Context, positions: int = REFERENCE_MAX_SEQ, theta: float = 10000.0) -> "RopeLut":
        h = C.c_void_p()
        _check(lib().swiftkv_rope_lut_generate(ctx.handle, positions, theta, C.byref(h)))
        return cls(ctx, h.value)

    @property
    def positions(self) -> int:
        return int(lib().swiftkv_rope_lut_positions(self.handle))

    def export(self, pos0: int = 0, n: Optional[int] = None) -> bytes:
        n = self.positions - pos0 if n is None else n
        out = np.zeros(n * ROPE_LUT_BYTES_PER_POSITION, np.uint8)
        _check(lib().swiftkv_rope_lut_export(self.handle, pos0, n, _host_ptr(out)))
        return out.tobytes()

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            _check(lib().swiftkv_rope_lut_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """GPU-resident INT8/G32 KV cache for `max_batch` sequences x `layers` x 32 heads."""

    def __init__(self, ctx: Context, layers: int, max_batch: int, max_seq_len: int):
        h = C.c_void_p()
        _check(lib().swiftkv_kv_cache_create(ctx.handle, layers, max_batch, max_seq_len, C.byref(h)))
        self.ctx = ctx
        self.handle = h.value
        self.layers, self.max_batch, self.max_seq_len = layers, max_batch, max_seq_len

    @property
    def nbytes(self) -> int:
        return int(lib().swiftkv_kv_cache_bytes(self.handle))

    def zero(self) -> None:
        _check(lib().swiftkv_kv_cache_zero(self.ctx.handle, self.handle))

    def read(self, seq: int, layer: int, head: int, tok0: int, n: int):
        """-> (k_codes int8 [n,128], v_codes int8 [n,128], k_scales f32 [n,4], v_scales f32 [n,4])."""
        kc = np.empty((n, HEAD_DIM), np.int8)
        vc = np.empty((n, HEAD_DIM), np.int8)
        ks = np.empty((n, GROUPS_PER_HEAD), np.float32)
        vs = np.empty((n, GROUPS_PER_HEAD), np.float32)
        _check(lib().swiftkv_kv_cache_read(self.ctx.handle, self.handle, seq, layer, head, tok0, n,
                                           _host_ptr(kc), _host_ptr(vc), _host_ptr(ks), _host_ptr(vs)))
        return kc, vc, ks, vs

    def export_records(self, seq: int, layer: int, head: int, tok0: int, n: int) -> np.ndarray:
        out = np.empty((n, RECORD_BYTES), np.uint8)
        _check(lib().swiftkv_kv_cache_export_records(self.ctx.handle, self.handle, seq, layer, head, tok0, n,
                                                     _host_ptr(out)))
        return out

    def import_records(self, seq: int, layer: int, head: int, tok0: int, records: np.ndarray) -> None:
        rec = np.ascontiguousarray(records, np.uint8).reshape(-1, RECORD_BYTES)
        _check(lib().swiftkv_kv_cache_import_records(self.ctx.handle, self.handle, seq, layer, head, tok0,
                                                     rec.shape[0], _host_ptr(rec)))

    def fill_synthetic(self, rope_lut: "RopeLut", ntok: int, seed: int, layer0: int = 0, nlayers: Optional[int] = None,
                       seq0: int = 0, nseq: Optional[int] = None, dist: int = DIST_NORMAL,
                       k_outliers: bool = False) -> None:
        """Fill tokens [0, ntok) from synthetic streams through the append rule."""
        nlayers = self.layers - layer0 if nlayers is None else nlayers
        nseq = self.max_batch - seq0 if nseq is None else nseq
        _check(lib().swiftkv_kv_cache_fill_synthetic(self.ctx.handle, self.handle, rope_lut.handle, layer0, nlayers,
                                                     seq0, nseq, ntok, seed, dist, 1 if k_outliers else 0))

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            _check(lib().swiftkv_kv_cache_destroy(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, np.ndarray):
        raise TypeError("a numpy array is host memory: pass a DeviceBuffer, or enable ctx.set_host_io(True)")
    return int(x)


def _io_ptr(ctx: "Context", x, dtype=None, writable: bool = False) -> Optional[int]:
    """Pointer for a step/append tensor: device memory normally, C-contiguous
    numpy arrays (of `dtype`) in host-memory I/O mode."""
    if x is None:
        return None
    if not ctx.host_io:
        return _ptr(x)
    if not isinstance(x, np.ndarray):
        raise TypeError("host-memory I/O mode takes numpy arrays")
    if not x.flags["C_CONTIGUOUS"] or (writable and not x.flags["WRITEABLE"]):
        raise ValueError("host arrays must be C-contiguous (and writable for outputs)")
    if dtype is not None and x.dtype != np.dtype(dtype):
        raise TypeError(f"expected {np.dtype(dtype)}, got {x.dtype}")
    return x.ctypes.data


def _check_io_sizes(ctx: Context, batch: int, q, k, v, out, aq, asc, in_elems: Optional[int] = None) -> None:
    """In host-memory I/O mode the library copies whole [batch][...] rows (and
    for split-K partials `in_elems` elements per input): refuse host arrays
    too small for them."""
    if not ctx.host_io:
        return
    n_in = batch * 4096 if in_elems is None else in_elems
    need = [(q, n_in), (k, n_in), (v, n_in), (out, batch * 4096),
            (aq, batch * 128 * 56), (asc, batch * 128)]
    for x, n in need:
        if isinstance(x, np.ndarray) and x.size < n:
            raise ValueError(f"host array holds {x.size} values, the step needs {n}")


def swiftkv_attention(ctx: Context, q, k, v, kv_cache: KVCache, rope_lut: RopeLut,
                      activation_q, activation_scale, layer_index: int, position,
                      out, q17: bool = False) -> None:
    """One decode-attention step (the drop-in for int4_swiftkv_attention_peN).

    q, k, v: device [batch][4096] (FP32, or Q15.17 int32 when q17=True);
    position: int (batch 1) or a sequence of cached-token counts, one per
    sequence; out: device [batch][4096] FP32; activation_q/activation_scale:
    device [batch][128][56] bytes and [batch][128] E8M0 codes, or None.
    Asynchronous on the context stream.
    """
    pos, batch, _keep = _positions(ctx, position)
    fn = lib().swiftkv_attention_q17 if q17 else lib().swiftkv_attention_f32
    _check_io_sizes(ctx, batch, q, k, v, out, activation_q, activation_scale)
    it = np.int32 if q17 else np.float32
    _check(fn(ctx.handle, _io_ptr(ctx, q, it), _io_ptr(ctx, k, it), _io_ptr(ctx, v, it), kv_cache.handle,
              rope_lut.handle, _io_ptr(ctx, activation_q, np.uint8, True),
              _io_ptr(ctx, activation_scale, np.uint8, True), int(layer_index), pos, batch,
              _io_ptr(ctx, out, np.float32, True)))


NOALLOC_WORKSPACE_BYTES = 8650752   # 128 KiB of arrival words + 8 splits x 32 sequences x 32 heads of partials


def step_plan(positions, cus: int = 256, workgroups_per_cu: int = 3, split_tokens: int = 0):
    """The launch plan of one step launch (host-only, no device needed):
    (tokens per split, splits of the longest sequence, waves per workgroup,
    tokens per block, sequence index per grid row)."""
    pos = np.ascontiguousarray(np.atleast_1d(np.asarray(positions, dtype=np.int32)))
    split, grid, waves, block = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
    rows = np.zeros(pos.size, np.int32)
    _check(lib().swiftkv_debug_step_plan(int(cus), int(workgroups_per_cu), int(split_tokens), _host_ptr(pos),
                                         int(pos.size), C.byref(split), C.byref(grid), C.byref(waves),
                                         C.byref(block), _host_ptr(rows)))
    return split.value, grid.value, waves.value, block.value, rows


def swiftkv_attention_noalloc(ctx: Context, q, k, v, kv_cache: KVCache, rope_lut: RopeLut,
                              activation_q, activation_scale, layer_index: int, position, out) -> None:
    """swiftkv_attention (FP32 inputs) through the allocation-free entry: the
    split workspace is the library's fixed per-GPU array, so the call never
    allocates device memory.  Calls that overlap in time on one GPU race.
    Device pointers only (host-memory I/O mode is refused)."""
    pos, batch, _keep = _positions(ctx, position)
    _check(lib().swiftkv_attention_f32_noalloc(ctx.handle, _ptr(q), _ptr(k), _ptr(v), kv_cache.handle,
                                               rope_lut.handle, _ptr(activation_q), _ptr(activation_scale),
                                               int(layer_index), pos, batch, _ptr(out)))


def swiftkv_attention_partials(ctx: Context, q, k, v, parts: int, kv_cache: KVCache, rope_lut: RopeLut,
                               activation_q, activation_scale, layer_index: int, position, out,
                               part_stride: Optional[int] = None) -> None:
    """The decode step fed by a split-K Q/K/V projection.

    q, k, v each hold `parts` (1, 2 or 4) FP32 partial sums, part p at element
    offset p * part_stride (default batch * 4096), each [batch][4096].  The
    step reduces them as the reference's linear stage does -- fl(p0 + p1), or
    fl(fl(p0 + p1) + fl(p2 + p3)) (int4_linear_controller.cpp:1039-1054,
    1655-1667, 1089-1118) -- then converts to Q15.17 and proceeds as
    swiftkv_attention.  Asynchronous on the context stream.
    """
    pos, batch, _keep = _positions(ctx, position)
    stride = batch * 4096 if part_stride is None else int(part_stride)
    _check_io_sizes(ctx, batch, q, k, v, out, activation_q, activation_scale,
                    in_elems=(int(parts) - 1) * stride + batch * 4096 if int(parts) > 1 else None)
    f = np.float32
    _check(lib().swiftkv_attention_partials(ctx.handle, _io_ptr(ctx, q, f), _io_ptr(ctx, k, f), _io_ptr(ctx, v, f),
                                            int(parts), stride, kv_cache.handle, rope_lut.handle,
                                            _io_ptr(ctx, activation_q, np.uint8, True),
                                            _io_ptr(ctx, activation_scale, np.uint8, True), int(layer_index),
                                            pos, batch, _io_ptr(ctx, out, np.float32, True)))


def swiftkv_attention_exact(ctx: Context, q, k, v, kv_cache: KVCache, rope_lut: RopeLut,
                            activation_q, activation_scale, layer_index: int, position,
                            out_q17, q17: bool = False) -> None:
    """The decode step in the reference's own Q15.17 integer arithmetic.

    Same append and arguments as swiftkv_attention, but the attention is the
    single-pass (max, Z, Y) recurrence of int4_swiftkv_attention_peN
    (swiftkv_attention.cpp:934-1880), so activation_q / activation_scale are
    bit-identical to the reference's.  out_q17: device [batch][4096] int32,
    the normalized Q15.17 state.  A verification path: one to four
    workgroups per (sequence, head), sequential in the token index.  Every
    position must be below 4096, the reference's bound (SwiftKVError ERANGE
    otherwise, with nothing enqueued).
    """
    pos, batch, _keep = _positions(ctx, position)
    _check_io_sizes(ctx, batch, q, k, v, out_q17, activation_q, activation_scale)
    it = np.int32 if q17 else np.float32
    _check(lib().swiftkv_attention_exact(ctx.handle, _io_ptr(ctx, q, it), _io_ptr(ctx, k, it),
                                         _io_ptr(ctx, v, it), 1 if q17 else 0, kv_cache.handle, rope_lut.handle,
                                         _io_ptr(ctx, activation_q, np.uint8, True),
                                         _io_ptr(ctx, activation_scale, np.uint8, True), int(layer_index),
                                         pos, batch, _io_ptr(ctx, out_q17, np.int32, True)))


def swiftkv_append_tokens(ctx: Context, k, v, kv_cache: KVCache, rope_lut: RopeLut, layer_index: int,
                          seq: int, pos0: int, n: int, q17: bool = False) -> None:
    """Bulk append (prefill) of n tokens [pos0, pos0+n) of one sequence."""
    it = np.int32 if q17 else np.float32
    if ctx.host_io:
        for x in (k, v):
            if isinstance(x, np.ndarray) and x.size < n * 4096:
                raise ValueError(f"host array holds {x.size} values, need {n} x 4096")
    _check(lib().swiftkv_append_tokens(ctx.handle, _io_ptr(ctx, k, it), _io_ptr(ctx, v, it), 1 if q17 else 0,
                                       kv_cache.handle, rope_lut.handle, int(layer_index), int(seq), int(pos0),
                                       int(n)))


def a14_unpack(words: np.ndarray) -> np.ndarray:
    """Packed A14 words [..., 56] bytes -> int16 lanes [..., 32] through the C ABI."""
    w = np.ascontiguousarray(words, dtype=np.uint8)
    if w.shape[-1] != 56:
        raise ValueError("A14 words are 56 bytes")
    groups = w.size // 56
    out = np.empty(w.shape[:-1] + (32,), np.int16)
    _check(lib().swiftkv_a14_unpack(w.ctypes.data, groups, out.ctypes.data))
    return out


def a14_decode(words: np.ndarray, e8m0: np.ndarray) -> np.ndarray:
    """Packed A14 words [..., 56] and their E8M0 bytes [...] -> the float values
    lane * 2^(code - 140) [..., 32] the O projection multiplies (C ABI)."""
    w = np.ascontiguousarray(words, dtype=np.uint8)
    e = np.ascontiguousarray(e8m0, dtype=np.uint8)
    if w.shape[-1] != 56 or e.shape != w.shape[:-1]:
        raise ValueError("words must be [..., 56] bytes and e8m0 [...] bytes")
    groups = w.size // 56
    out = np.empty(w.shape[:-1] + (32,), np.float32)
    _check(lib().swiftkv_a14_decode(w.ctypes.data, e.ctypes.data, groups, out.ctypes.data))
    return out


def unpack_a14(words: np.ndarray) -> np.ndarray:
    """[..., 56] bytes of packed 14-bit lanes -> int16 [..., 32] (lane 0 = bits [13:0])."""
    w = np.ascontiguousarray(words, np.uint8)
    bits = np.unpackbits(w, axis=-1, bitorder="little")[..., :32 * 14]
    bits = bits.reshape(w.shape[:-1] + (32, 14)).astype(np.int32)
    vals = (bits << np.arange(14, dtype=np.int32)).sum(-1)
    vals = np.where(vals >= 8192, vals - 16384, vals)
    return vals.astype(np.int16)


def scale_bits(shifts: np.ndarray) -> np.ndarray:
    """FP32 bit pattern of the G32 scale 2^(s-17)."""
    return ((np.asarray(shifts, np.uint32) + np.uint32(110)) << np.uint32(23)).astype(np.uint32)


def version() -> str:
    return lib().swiftkv_version().decode()
