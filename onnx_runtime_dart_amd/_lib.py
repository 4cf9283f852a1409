"""ctypes binding of libmmnb.so (the C ABI declared in include/mmnb.h).

This is the Python counterpart of the dart:ffi binding a Dart host would
use: plain pointers, sizes and int status codes.  Loading fails loudly when
the library has not been built; there is no CPU fallback.
"""
import ctypes
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libmmnb.so"

MMNB_OK = 0
MMNB_ERR_ARG = -1
MMNB_ERR_UNSUPPORTED = -2
MMNB_ERR_DEVICE = -3
MMNB_ERR_OOM = -4

# Every symbol include/mmnb.h declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_P = ctypes.POINTER
SIGNATURES = {
    "mmnb_abi_version": (_int, []),
    "mmnb_last_error": (ctypes.c_char_p, []),
    "mmnb_init": (_int, [_int, _P(_vp)]),
    "mmnb_shutdown": (_int, [_vp]),
    "mmnb_device_info": (_int, [_vp, ctypes.c_char_p, _sz, _P(_int), _P(_i64)]),
    "mmnb_pack_nbits": (_int, [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                               _i64, _P(_vp)]),
    "mmnb_matmul_nbits": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "mmnb_matmul_nbits_dev": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "mmnb_matmul_nbits_dev_noalloc": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "mmnb_noalloc_workspace_bytes": (_i64, []),
    "mmnb_dynamic_quantize_linear": (_int, [_vp, _vp, _i64, _vp, _P(ctypes.c_float),
                                            _P(_i64)]),
    "mmnb_dynamic_quantize_linear_dev": (_int, [_vp, _vp, _i64, _vp, _vp, _vp]),
    "mmnb_pack_integer": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _vp, _i64, _P(_vp)]),
    "mmnb_matmul_integer": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _i64, _vp]),
    "mmnb_matmul_integer_dev": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _i64, _vp]),
    "mmnb_dynamic_matmul_dev": (_int, [_vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                       _vp, _vp]),
    "mmnb_pack_nbits_ex": (_int, [_vp, _vp, _P(_vp)]),
    "mmnb_model_load": (_int, [_vp, ctypes.c_char_p, _P(_vp)]),
    "mmnb_model_pack_count": (_i64, [_vp]),
    "mmnb_model_pack_info": (_int, [_vp, _i64, _P(ctypes.c_char_p), _P(ctypes.c_char_p),
                                    _P(_vp)]),
    "mmnb_model_find": (_int, [_vp, ctypes.c_char_p, _P(_vp)]),
    "mmnb_model_free": (_int, [_vp]),
    "mmnb_check_external_ref": (_int, [ctypes.c_char_p, _i64, _i64, _i64]),
    "mmnb_qlinear_matmul": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _i64, ctypes.c_float,
                                   ctypes.c_float, ctypes.c_float, _i64, _int, _vp]),
    "mmnb_qlinear_matmul_dev": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _i64,
                                       ctypes.c_float, ctypes.c_float, ctypes.c_float, _i64,
                                       _int, _vp]),
    "mmnb_pack_conv": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                              _P(_vp)]),
    "mmnb_conv_output_shape": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _P(_i64), _P(_i64)]),
    "mmnb_conv_integer": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "mmnb_conv_integer_dev": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _vp,
                                     _vp]),
    "mmnb_qlinear_conv": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                                 ctypes.c_float, _vp, _i64, ctypes.c_float, _i64, _int, _vp, _vp,
                                 _vp]),
    "mmnb_qlinear_conv_dev": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                                     ctypes.c_float, _vp, _i64, ctypes.c_float, _i64, _int, _vp,
                                     _vp, _vp]),
    "mmnb_pack_free": (_int, [_vp]),
    "mmnb_pack_device_bytes": (_i64, [_vp]),
    "mmnb_pack_dims": (_int, [_vp, _P(_i64), _P(_i64), _P(_i64)]),
    "mmnb_device_alloc": (_int, [_vp, _sz, _P(_vp)]),
    "mmnb_device_free": (_int, [_vp, _vp]),
    "mmnb_memcpy_h2d": (_int, [_vp, _vp, _vp, _sz]),
    "mmnb_memcpy_d2h": (_int, [_vp, _vp, _vp, _sz]),
    "mmnb_memset_dev": (_int, [_vp, _vp, _int, _sz]),
    "mmnb_memcpy_d2d": (_int, [_vp, _vp, _vp, _sz]),
    "mmnb_synchronize": (_int, [_vp]),
    "mmnb_event_record": (_int, [_vp, _int]),
    "mmnb_event_elapsed_ms": (_int, [_vp, _int, _int, _P(ctypes.c_float)]),
    "mmnb_kernel_timing": (_int, [_vp, _int, _int]),
    "mmnb_kernel_timing_read": (_int, [_vp, _int, _P(_i64), _P(ctypes.c_double),
                                       _P(ctypes.c_double), _P(ctypes.c_double)]),
    "mmnb_kernel_timing_samples": (_int, [_vp, _int, _P(ctypes.c_float), _i64, _P(_i64)]),
    "mmnb_kernel_name": (ctypes.c_char_p, [_int]),
    "mmnb_probe_empty": (_int, [_vp, _int]),
    "mmnb_probe_stream_read": (_int, [_vp, _vp, _sz]),
    "mmnb_graph_begin": (_int, [_vp]),
    "mmnb_graph_end": (_int, [_vp, _P(_vp)]),
    "mmnb_graph_launch": (_int, [_vp, _vp]),
    "mmnb_graph_destroy": (_int, [_vp, _vp]),
    "mmnb_rmsnorm_dev": (_int, [_vp, _vp, _i64, _i64, _vp, ctypes.c_float, _vp]),
    "mmnb_rotary_dev": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64,
                               _int, _vp]),
    "mmnb_gqa_dev": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                            _vp, _vp, _i64, _vp, _vp, _i64, _int, _int, _vp, _i64, _vp, _vp,
                            _vp]),
    "mmnb_decoder_create": (_int, [_vp, _vp, _vp, _vp, _vp, _P(_vp)]),
    "mmnb_decoder_set_layer": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mmnb_decoder_prefill": (_int, [_vp, _vp, _i64, _P(ctypes.c_int32)]),
    "mmnb_decoder_decode": (_int, [_vp, _i64, _vp]),
    "mmnb_decoder_logits": (_int, [_vp, _vp]),
    "mmnb_decoder_position": (_int, [_vp, _P(_i64)]),
    "mmnb_decoder_reset": (_int, [_vp]),
    "mmnb_decoder_set_graph": (_int, [_vp, _int]),
    "mmnb_decoder_free": (_int, [_vp]),
}


class DecoderConfig(ctypes.Structure):
    """mmnb_decoder_config (include/mmnb.h)."""
    _fields_ = [("layers", _i64), ("hidden", _i64), ("heads", _i64), ("kv_heads", _i64),
                ("head_dim", _i64), ("intermediate", _i64), ("vocab", _i64),
                ("max_len", _i64), ("eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]

DT_F32, DT_U8, DT_F16 = 1, 2, 10
ZP_FLAT, ZP_PER_COLUMN = 0, 1


class NBitsDesc(ctypes.Structure):
    """mmnb_nbits_desc (include/mmnb.h)."""
    _fields_ = [("k", _i64), ("n", _i64), ("bits", _i64), ("block_size", _i64),
                ("b_q", _vp), ("b_q_len", _i64),
                ("scales", _vp), ("scales_len", _i64), ("scales_type", _int),
                ("zero_points", _vp), ("zero_points_len", _i64), ("zero_points_type", _int),
                ("zero_points_layout", _int),
                ("g_idx", _vp), ("g_idx_len", _i64),
                ("bias", _vp), ("bias_len", _i64), ("bias_type", _int)]


class ConvParams(ctypes.Structure):
    """mmnb_conv_params (include/mmnb.h)."""
    _fields_ = [("strides", _i64 * 2), ("pads", _i64 * 4), ("dilations", _i64 * 2)]


_lib = None
_lock = threading.RLock()


class MmnbError(RuntimeError):
    """Device or allocation failure (no reference counterpart)."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


def load():
    """Load libmmnb.so; raises if it is missing (build it first)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built: run `python -m onnx_runtime_dart_amd.build` "
                    "(the HIP extension is required; there is no CPU fallback)")
            L = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def check(rc):
    """Map a status code to the reference's exception types:
    ArgumentError -> ValueError, UnsupportedError -> NotImplementedError."""
    if rc == MMNB_OK:
        return
    msg = load().mmnb_last_error().decode(errors="replace")
    if rc == MMNB_ERR_ARG:
        raise ValueError(msg)
    if rc == MMNB_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == MMNB_ERR_OOM:
        raise MemoryError(msg)
    raise MmnbError(rc, msg)


def ptr(a):
    """Raw data pointer of a C-contiguous numpy array (None for None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


class Context:
    """One HIP device context (one stream) of libmmnb."""

    def __init__(self, device=0):
        self.lib = load()
        h = ctypes.c_void_p()
        check(self.lib.mmnb_init(int(device), ctypes.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            check(self.lib.mmnb_shutdown(self.handle))
            self.handle = None

    def info(self):
        name = ctypes.create_string_buffer(256)
        cus = ctypes.c_int()
        hbm = ctypes.c_int64()
        check(self.lib.mmnb_device_info(self.handle, name, 256, ctypes.byref(cus),
                                        ctypes.byref(hbm)))
        return {"name": name.value.decode(), "compute_units": cus.value,
                "hbm_bytes": hbm.value}

    def synchronize(self):
        check(self.lib.mmnb_synchronize(self.handle))

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr):
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, arr.nbytes, dtype=arr.dtype, shape=arr.shape)
        if arr.nbytes:
            check(self.lib.mmnb_memcpy_h2d(self.handle, buf.ptr, ptr(arr), arr.nbytes))
        return buf

    def event_record(self, slot):
        check(self.lib.mmnb_event_record(self.handle, int(slot)))

    def kernel_timing(self, enable, max_launches=4096):
        check(self.lib.mmnb_kernel_timing(self.handle, int(bool(enable)), int(max_launches)))

    def kernel_timing_read(self):
        """{kernel name: (count, total_ms, min_ms, max_ms)} of recorded launches."""
        out = {}
        kid = 0
        while True:
            name = self.lib.mmnb_kernel_name(kid)
            if name is None:
                break
            c = ctypes.c_int64()
            t, lo, hi = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
            check(self.lib.mmnb_kernel_timing_read(self.handle, kid, ctypes.byref(c),
                                                   ctypes.byref(t), ctypes.byref(lo),
                                                   ctypes.byref(hi)))
            if c.value:
                out[name.decode()] = (c.value, t.value, lo.value, hi.value)
            kid += 1
        return out

    def kernel_timing_samples(self, name):
        """Every recorded duration (ms) of kernel `name`, in launch order, as a
        float32 array (empty if it was not launched while timing was on)."""
        kid = 0
        while True:
            kn = self.lib.mmnb_kernel_name(kid)
            if kn is None:
                raise KeyError(name)
            if kn.decode() == name:
                break
            kid += 1
        c = ctypes.c_int64()
        check(self.lib.mmnb_kernel_timing_samples(self.handle, kid, None, 0, ctypes.byref(c)))
        out = np.zeros(c.value, np.float32)
        if c.value:
            check(self.lib.mmnb_kernel_timing_samples(
                self.handle, kid, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), c.value,
                ctypes.byref(c)))
        return out

    def graph_begin(self):
        check(self.lib.mmnb_graph_begin(self.handle))

    def graph_end(self):
        g = ctypes.c_void_p()
        check(self.lib.mmnb_graph_end(self.handle, ctypes.byref(g)))
        return g

    def graph_launch(self, g):
        check(self.lib.mmnb_graph_launch(self.handle, g))

    def graph_destroy(self, g):
        check(self.lib.mmnb_graph_destroy(self.handle, g))

    def event_elapsed_ms(self, s0, s1):
        ms = ctypes.c_float()
        check(self.lib.mmnb_event_elapsed_ms(self.handle, int(s0), int(s1), ctypes.byref(ms)))
        return float(ms.value)


class DeviceBuffer:
    """A device allocation made through the C ABI."""

    def __init__(self, ctx, nbytes, dtype=np.uint8, shape=None):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = ctypes.c_void_p()
        check(ctx.lib.mmnb_device_alloc(ctx.handle, max(1, self.nbytes), ctypes.byref(p)))
        self.ptr = p

    def numpy(self, dtype=None, shape=None):
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        sh = shape if shape is not None else (self.shape if dtype is None else
                                              (self.nbytes // dt.itemsize,))
        out = np.empty(sh, dtype=dt)
        if out.nbytes:
            check(self.ctx.lib.mmnb_memcpy_d2h(self.ctx.handle, ptr(out), self.ptr,
                                               out.nbytes))
        return out

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        if arr.nbytes:
            check(self.ctx.lib.mmnb_memcpy_h2d(self.ctx.handle, self.ptr, ptr(arr),
                                               arr.nbytes))

    def free(self):
        if self.ptr:
            check(self.ctx.lib.mmnb_device_free(self.ctx.handle, self.ptr))
            self.ptr = None


_default_ctx = None


def default_context():
    """Process-wide context on device 0 (what the Dart binding opens once)."""
    global _default_ctx
    with _lock:
        if _default_ctx is None:
            _default_ctx = Context(0)
    return _default_ctx
