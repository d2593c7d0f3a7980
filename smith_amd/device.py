"""ctypes wrapper around libsmith.so -- the Python mirror of src/device.js.

The reference binds its Objective-C Metal bridge with bun:ffi at import
(src/device.js:10-50) and initialises the device immediately
(src/device.js:57-58).  Here the symbol table is bound at import (no GPU
needed) and the HIP context is created on first use, so CPU-only processes can
import the package; any GPU operation without a device raises RuntimeError
instead of falling back to the CPU.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libsmith.so")
CODE_OBJECT_PATH = os.path.join(_HERE, "lib", "smith_kernels.hsaco")
LLAMA_CODE_OBJECT_PATH = os.path.join(_HERE, "lib", "smith_llama.hsaco")
GEMM_CODE_OBJECT_PATH = os.path.join(_HERE, "lib", "smith_gemm.hsaco")

SHARED = 0
PRIVATE = 1

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_STR = ctypes.c_char_p


class SmithTiming(ctypes.Structure):
    _fields_ = [("gpu_start", ctypes.c_double), ("gpu_end", ctypes.c_double), ("gpu_ms", ctypes.c_double)]


# name -> (restype, argtypes); mirrors the dlopen table of src/device.js:10-50
# plus the explicit-copy, op-level and timing entry points of include/smith.h.
SYMBOLS = {
    "smith_init": (_P, []),
    "smith_destroy": (None, [_P]),
    "smith_device_name": (_P, [_P]),
    "smith_max_threadgroup_memory": (_U64, [_P]),
    "smith_max_threads_per_threadgroup": (_U64, [_P]),
    "smith_alloc": (_P, [_P, _U64, _U32]),
    "smith_buffer_contents": (_P, [_P]),
    "smith_buffer_length": (_U64, [_P]),
    "smith_release_buffer": (None, [_P]),
    "smith_test_release": (_I64, [_P]),
    "smith_test_release_after_use": (_I64, [_P]),
    "smith_buffer_retain_count": (_I64, [_P]),
    "smith_allocated_size": (_U64, [_P]),
    "smith_copy_h2d": (_INT, [_P, _P, _U64, _P, _U64]),
    "smith_copy_d2h": (_INT, [_P, _P, _P, _U64, _U64]),
    "smith_copy_d2d": (_INT, [_P, _P, _U64, _P, _U64, _U64]),
    "smith_fill_zero": (_INT, [_P, _P, _U64]),
    "smith_prep_next": (_INT, [_P, _P, ctypes.c_float]),
    "smith_sync": (_INT, [_P]),
    "smith_free": (None, [_P]),
    "smith_last_error": (_STR, [_P]),
    "smith_load_library": (_P, [_P, _STR]),
    "smith_compile_source": (_P, [_P, _STR, ctypes.POINTER(_P)]),
    "smith_create_pipeline": (_P, [_P, _P, _STR]),
    "smith_begin": (_P, [_P]),
    "smith_set_buffer": (None, [_P, _P, _U32]),
    "smith_set_bytes": (None, [_P, _P, _U32, _U32]),
    "smith_set_pipeline": (None, [_P, _P]),
    "smith_set_threadgroup_memory": (None, [_P, _U64, _U32]),
    "smith_dispatch": (None, [_P, _U64, _U64, _U64, _U64, _U64, _U64]),
    "smith_end_sync": (None, [_P]),
    "smith_end_async": (_P, [_P]),
    "smith_wait": (None, [_P]),
    "smith_end_timed": (ctypes.POINTER(SmithTiming), [_P]),
    "smith_dispatch_sync": (None, [_P, _P, ctypes.POINTER(_P), ctypes.POINTER(_U32), _U32, _P, _U32, _U32,
                                   _U64, _U64, _U64, _U64, _U64, _U64]),
    "smith_quantize_q4": (_INT, [_P, _P, _P, _U32, _U32]),
    "smith_quantize_q8": (_INT, [_P, _P, _P, _U32, _U32]),
    "smith_matmul_q4": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "smith_matmul_q4_noalloc": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "smith_matmul_q8": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "smith_repack_q4_0": (_INT, [_P, _P, _P, _P, _U32, _U32]),
    "smith_matmul_q4_0": (_INT, [_P, _P, _P, _P, _P, _U32, _U32, _U32]),
    "smith_quantize_q4_0": (_INT, [_P, _P, _P, _U32, _U32]),
    "smith_repack_q4_0_into": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "smith_repack_q8_0_into": (_INT, [_P, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "smith_linear_q4_0": (_INT, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, ctypes.c_float, _P, _U32]),
    "smith_repack_q4_0_t_into": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "smith_linear_q4_0_t": (_INT, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, ctypes.c_float, _P, _U32]),
    "smith_attention_parts": (_INT, [_P, _P, _P, _U32, _U32, _U32, _P, _P, _U32, _P, _P, _P, _U32, _P]),
    "smith_linear_q4_0_t_attn": (_INT, [_P, _P, _P, _U32, _P, _P, _P, _U32, _U32, _P, _U32, _P, _P]),
    "smith_linear_q4_0_t_act": (_INT, [_P, _P, ctypes.c_int, ctypes.c_float, _P, _P, _P, _U32, _U32, _P, _U32, _P,
                                       _P]),
    "smith_gguf_tiles_bytes": (_U64, [_U32, _U32, _U32]),
    "smith_lmhead_q6_k_bytes": (_U64, [_U32, _U32]),
    "smith_repack_lmhead_q6_k": (_INT, [_P, _P, _P, _U32, _U32]),
    "smith_lmhead_q6_k_nb": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _U32, _U32]),
    "smith_lmhead_q6_k_greedy": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _U32, _U32, _P, _P, _P, _P, _P, _P, _P,
                                        _P, _P, _U32, _U32, _U32, _P]),
    "smith_copy_2d": (_INT, [_P, _P, _U64, _P, _U64, _U64, _U64]),
    "smith_repack_gguf_tiles_into": (_INT, [_P, _U32, _P, _P, _U32, _U32, _U32, _U32, _U32]),
    "smith_linear_gguf_tiles": (_INT, [_P, _U32, _P, _P, _P, _U32, _U32, _U32, _P, ctypes.c_float, _P, _U32]),
    "smith_linear_gguf_tiles_act": (_INT, [_P, _U32, _P, ctypes.c_int, ctypes.c_float, _P, _P, _U32, _U32, _P,
                                           _U32, _P, _P]),
    "smith_linear_gguf_tiles_attn": (_INT, [_P, _U32, _P, _P, _U32, _P, _P, _U32, _U32, _P, _U32, _P, _P]),
    "smith_dequantize_gguf": (_INT, [_P, _U32, _P, _P, _U64]),
    "smith_gguf_tiles_pair_ok": (_INT, [_U32, _U32]),
    "smith_linear_gguf_tiles_pair_act": (_INT, [_P, _U32, _P, _U32, _U32, _P, _U32, _P, ctypes.c_int, ctypes.c_float,
                                                _P, _U32]),
    "smith_linear_q8": (_INT, [_P, _P, _P, _P, _U32, _U32, _U32, _P, ctypes.c_float, _P, _U32]),
    "smith_rmsnorm": (_INT, [_P, _P, _P, _P, _U32, _U32, ctypes.c_float]),
    "smith_embed": (_INT, [_P, _P, _P, _P, _U32, _U32, _P, _P]),
    "smith_attention": (_INT, [_P, _P, _U32, _P, _U32, _U32, _U32, _U32, _P, _P, _U32, _P, _P, _U32, _P, _P]),
    "smith_repack_lmhead_q4_0": (_INT, [_P, _P, _P, _P, _U32, _U32]),
    "smith_lmhead_q4_0_nb": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _P, _U32, _U32]),
    "smith_lmhead_q4_0_greedy": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _P, _U32, _U32, _P, _P, _P, _P, _P, _P,
                                        _P, _P, _P, _U32, _U32, _U32, _P]),
    "smith_gemv_f32": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _U32, _U32, _INT]),
    "smith_argmax_embed": (_INT, [_P, _P, _U32, _P, _U32, _P, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _P]),
    "smith_set_i32": (_INT, [_P, _P, ctypes.c_int32]),
    "smith_randn": (_INT, [_P, _P, _U64, _U64, _U64, ctypes.c_float, ctypes.c_float]),
    "smith_graph_begin": (_INT, [_P]),
    "smith_graph_end": (_P, [_P]),
    "smith_graph_launch": (_INT, [_P, _P]),
    "smith_graph_destroy": (None, [_P]),
    "smith_profile_kernels": (_INT, [_P, _INT]),
    "smith_profile_read": (_INT, [_P, _STR, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_U64)]),
    "smith_timer_start": (_INT, [_P]),
    "smith_timer_stop": (ctypes.c_double, [_P]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "smith: %s is missing -- build it with `python -m smith_amd.build` "
            "(there is no CPU fallback)" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SYMBOLS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


class _LazyLib:
    """dlopen libsmith.so on first use, so importing the package (and
    `python -m smith_amd.build`) never needs a built library."""
    _L = None

    def __getattr__(self, name):
        if _LazyLib._L is None:
            _LazyLib._L = _load()
        return getattr(_LazyLib._L, name)


lib = _LazyLib()

_ctx = None
_library = None
_pipelines = {}


def ctx():
    """The process-wide HIP context (created on first use)."""
    global _ctx
    if _ctx is None:
        c = lib.smith_init()
        if not c:
            raise RuntimeError("smith: failed to initialize HIP device. An AMD GPU (gfx950) is required.")
        _ctx = c
    return _ctx


def check(rc, what="smith"):
    if rc != 0:
        msg = lib.smith_last_error(ctx())
        raise RuntimeError("%s: %s" % (what, msg.decode() if msg else "unknown error"))
    return rc


def shader_lib():
    """The gfx950 code object (src/device.js:71-79 loads the metallib lazily)."""
    global _library
    if _library is None:
        c = ctx()
        lp = lib.smith_load_library(c, CODE_OBJECT_PATH.encode())
        if not lp:
            raise RuntimeError("smith: failed to load code object at %s: %s"
                               % (CODE_OBJECT_PATH, lib.smith_last_error(c).decode()))
        _library = lp
        for path in (LLAMA_CODE_OBJECT_PATH, GEMM_CODE_OBJECT_PATH):
            if not lib.smith_load_library(c, path.encode()):
                raise RuntimeError("smith: failed to load code object at %s: %s"
                                   % (path, lib.smith_last_error(c).decode()))
    return _library


def pipeline(kernel_name):
    p = _pipelines.get(kernel_name)
    if p is None:
        p = lib.smith_create_pipeline(ctx(), shader_lib(), kernel_name.encode())
        if not p:
            raise RuntimeError("smith: kernel '%s' not found in code object" % kernel_name)
        _pipelines[kernel_name] = p
    return p


def ops_ctx():
    """Context with the code object loaded, for the op-level entry points."""
    shader_lib()
    return _ctx


def device_name():
    p = lib.smith_device_name(ctx())
    if not p:
        return ""
    s = ctypes.cast(p, ctypes.c_char_p).value.decode()
    lib.smith_free(p)
    return s


def max_threadgroup_memory():
    return int(lib.smith_max_threadgroup_memory(ctx()))


def max_threads_per_threadgroup():
    return int(lib.smith_max_threads_per_threadgroup(ctx()))


def alloc(nbytes, mode=SHARED):
    buf = lib.smith_alloc(ctx(), int(nbytes), mode)
    if not buf:
        raise RuntimeError("smith: failed to allocate %d bytes (mode=%d)" % (nbytes, mode))
    return buf


def buffer_length(buf):
    return int(lib.smith_buffer_length(buf))


def release_buffer(buf):
    lib.smith_release_buffer(buf)


def allocated_size():
    return int(lib.smith_allocated_size(ctx()))


def upload(buf, host_array, offset=0):
    """Host -> device copy of a contiguous numpy array."""
    import numpy as np
    a = np.ascontiguousarray(host_array)
    check(lib.smith_copy_h2d(ctx(), buf, offset, a.ctypes.data_as(_P), a.nbytes), "smith_copy_h2d")


def download(buf, nbytes, dtype, offset=0):
    """Device -> host copy into a new numpy array (waits for the stream)."""
    import numpy as np
    out = np.empty(int(nbytes) // np.dtype(dtype).itemsize, dtype=dtype)
    check(lib.smith_copy_d2h(ctx(), out.ctypes.data_as(_P), buf, offset, out.nbytes), "smith_copy_d2h")
    return out


def sync():
    check(lib.smith_sync(ctx()), "smith_sync")


# --- encoded dispatch (src/device.js:144-193) ---

def begin():
    return lib.smith_begin(ctx())


def set_buffer(enc, buf, index):
    lib.smith_set_buffer(enc, buf, index)


def set_bytes(enc, data, index):
    b = bytes(data)
    lib.smith_set_bytes(enc, b, len(b), index)


def set_threadgroup_memory(enc, length, index):
    lib.smith_set_threadgroup_memory(enc, length, index)


def set_pipeline(enc, p):
    lib.smith_set_pipeline(enc, p)


def dispatch(enc, gx, gy, gz, bx, by, bz):
    lib.smith_dispatch(enc, gx, gy, gz, bx, by, bz)


def end_sync(enc):
    lib.smith_end_sync(enc)
    err = lib.smith_last_error(ctx())
    return err


def end_async(enc):
    return lib.smith_end_async(enc)


def wait(token):
    lib.smith_wait(token)


def end_timed(enc):
    t = lib.smith_end_timed(enc)
    if not t:
        return {"gpuStart": 0.0, "gpuEnd": 0.0, "gpuMs": 0.0}
    r = {"gpuStart": t.contents.gpu_start, "gpuEnd": t.contents.gpu_end, "gpuMs": t.contents.gpu_ms}
    lib.smith_free(ctypes.cast(t, _P))  # the reference leaks this struct (src/device.js:189-191)
    return r


def compile_source(source):
    err = _P()
    lp = lib.smith_compile_source(ctx(), source.encode(), ctypes.byref(err))
    if not lp:
        msg = ctypes.cast(err, ctypes.c_char_p).value.decode() if err.value else "unknown error"
        if err.value:
            lib.smith_free(err)
        raise RuntimeError("smith: shader compilation failed: %s" % msg)
    return lp


def create_pipeline(library, fn_name):
    p = lib.smith_create_pipeline(ctx(), library, fn_name.encode())
    if not p:
        raise RuntimeError("smith: kernel '%s' not found" % fn_name)
    return p


def timer_start():
    check(lib.smith_timer_start(ctx()), "smith_timer_start")


def timer_stop():
    ms = lib.smith_timer_stop(ctx())
    if ms < 0:
        check(-1, "smith_timer_stop")
    return ms


def profile_kernels(enable=True):
    check(lib.smith_profile_kernels(ctx(), 1 if enable else 0), "smith_profile_kernels")


def profile_read(prefix=""):
    """(total_ms, count) of recorded op-kernel launches named prefix*."""
    tot = ctypes.c_double()
    n = _U64()
    check(lib.smith_profile_read(ctx(), prefix.encode(), ctypes.byref(tot), ctypes.byref(n)), "smith_profile_read")
    return tot.value, int(n.value)
