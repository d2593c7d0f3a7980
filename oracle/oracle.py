"""ctypes front end of the CPU oracle (oracle/smith_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Each wrapper
names the reference file:line its C function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

Q4S_BYTES = 24
Q8_BYTES = 34
Q4_0_BYTES = 18
GGML_F32 = 0
GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q4_1 = 3
GGML_Q5_0 = 6
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14
GGML_BF16 = 30
# (elements, bytes) per block, src/gguf.js:30-41
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_BF16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q4_1: (32, 20),
         GGML_Q5_0: (32, 22), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210)}


def build():
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        for name, args, res in [
            ("oracle_from_f16", [ctypes.c_uint16], ctypes.c_double),
            ("oracle_to_f16_trunc", [ctypes.c_float], ctypes.c_uint16),
            ("oracle_f32_to_f16_rne", [ctypes.c_float], ctypes.c_uint16),
            ("oracle_quantize_q4s", [P, I, I, P], None),
            ("oracle_dequant_q4s", [P, I, I, P], None),
            ("oracle_quantize_q8", [P, I, I, P], None),
            ("oracle_dequant_q8", [P, I, I, P], None),
            ("oracle_dequant_q4_0_block", [P, P], None),
            ("oracle_dequant_q8_0_block", [P, P], None),
            ("oracle_dequant_q4_1_block", [P, P], None),
            ("oracle_dequant_q5_0_block", [P, P], None),
            ("oracle_dequant_q4_k_block", [P, P], None),
            ("oracle_dequant_q6_k_block", [P, P], None),
            ("oracle_dequantize_tensor", [ctypes.c_int, P, I, P], ctypes.c_int),
            ("oracle_quantize_rows", [ctypes.c_int, P, I, I, P], ctypes.c_int),
            ("oracle_matmul_f64acc", [P, P, I, I, I, P], None),
            ("oracle_matmul_f32", [P, P, I, I, I, P], None),
            ("oracle_matmul_q4s", [P, P, I, I, I, P], None),
            ("oracle_matmul_q8", [P, P, I, I, I, P], None),
            ("oracle_matmul_gguf", [ctypes.c_int, P, P, I, I, I, P], ctypes.c_int),
        ]:
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def from_f16(h):
    """fromFloat16, src/gguf.js:398-408."""
    return lib().oracle_from_f16(int(h))


def to_f16_trunc(x):
    """toFloat16, src/dtype.js:29-58 (truncating)."""
    return lib().oracle_to_f16_trunc(float(x))


def f32_to_f16_rne(x):
    return lib().oracle_f32_to_f16_rne(float(x))


def _out_f32(out, K, N):
    if out is None:
        return np.empty((K, N), dtype=np.float32)
    if out.dtype != np.float32 or out.shape != (K, N) or not out.flags.c_contiguous:
        raise ValueError("out must be a C-contiguous float32 [%d, %d] array" % (K, N))
    return out


def quantize_q4s(w):
    """quantizeQ4, src/ops/quantize.js:14-68 -> Q4S bytes."""
    w = _f32(w)
    K, N = w.shape
    groups = (K + 31) // 32
    out = np.zeros(groups * N * Q4S_BYTES, dtype=np.uint8)
    lib().oracle_quantize_q4s(_p(w), K, N, _p(out))
    return out


def dequant_q4s(q, K, N, out=None):
    """dequant_q4, shaders/matmul_q4.metal:24-28 -> f32 [K,N] (into `out`
    when given: a reused C-contiguous f32 [K,N] array)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    w = _out_f32(out, K, N)
    lib().oracle_dequant_q4s(_p(q), K, N, _p(w))
    return w


def quantize_q8(w):
    """Q8 blocks in matmul_q8.metal's layout (ggml q8_0 rounding)."""
    w = _f32(w)
    K, N = w.shape
    groups = (K + 31) // 32
    out = np.zeros(groups * N * Q8_BYTES, dtype=np.uint8)
    lib().oracle_quantize_q8(_p(w), K, N, _p(out))
    return out


def dequant_q8(q, K, N, out=None):
    """shaders/matmul_q8.metal:44-52 -> f32 [K,N] (into `out` when given)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    w = _out_f32(out, K, N)
    lib().oracle_dequant_q8(_p(q), K, N, _p(w))
    return w


def dequant_q4_0_block(blk):
    """dequantQ4_0, src/gguf.js:187-197."""
    blk = np.ascontiguousarray(blk, dtype=np.uint8)
    out = np.empty(32, dtype=np.float32)
    lib().oracle_dequant_q4_0_block(_p(blk), _p(out))
    return out


def dequant_q8_0_block(blk):
    """dequantQ8_0, src/gguf.js:221-231."""
    blk = np.ascontiguousarray(blk, dtype=np.uint8)
    out = np.empty(32, dtype=np.float32)
    lib().oracle_dequant_q8_0_block(_p(blk), _p(out))
    return out


def _block(fn, n, blk):
    blk = np.ascontiguousarray(blk, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    getattr(lib(), fn)(_p(blk), _p(out))
    return out


def dequant_q4_1_block(blk):
    """dequantQ4_1, src/gguf.js:203-215."""
    return _block("oracle_dequant_q4_1_block", 32, blk)


def dequant_q5_0_block(blk):
    """dequantQ5_0, src/gguf.js:238-259."""
    return _block("oracle_dequant_q5_0_block", 32, blk)


def dequant_q4_k_block(blk):
    """dequantQ4_K, src/gguf.js:264-305."""
    return _block("oracle_dequant_q4_k_block", 256, blk)


def dequant_q6_k_block(blk):
    """dequantQ6_K, src/gguf.js:309-339."""
    return _block("oracle_dequant_q6_k_block", 256, blk)


def dequantize_tensor(ggml_type, data, numel, out=None):
    """dequantizeTensor, src/gguf.js:343-394 (F32, F16, BF16, Q4_0, Q4_1,
    Q5_0, Q8_0, Q4_K, Q6_K).  `out`: an optional f32 array of numel
    elements to decode into."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    if out is None:
        out = np.empty(numel, dtype=np.float32)
    assert out.dtype == np.float32 and out.size == numel and out.flags.c_contiguous
    if lib().oracle_dequantize_tensor(ggml_type, _p(data), numel, _p(out)):
        raise ValueError("unsupported type %d" % ggml_type)
    return out


def quantize_rows(ggml_type, x):
    """GGUF block encoder for this build's synthetic files, row by row
    (Q4_0/Q8_0/Q4_1/Q5_0: ggml reference rounding; Q4_K/Q6_K: this build's
    rounding), packed in the order the reference's decoders read."""
    x = _f32(x)
    rows, cols = x.shape
    be, bpb = BLOCK[ggml_type]
    out = np.zeros(rows * ((cols + be - 1) // be) * bpb, dtype=np.uint8)
    if lib().oracle_quantize_rows(ggml_type, _p(x), rows, cols, _p(out)):
        raise ValueError("unsupported type %d" % ggml_type)
    return out


def matmul_f64acc(a, w):
    a, w = _f32(a), _f32(w)
    M, K = a.shape
    N = w.shape[1]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_f64acc(_p(a), _p(w), M, N, K, _p(c))
    return c


def matmul_f32(a, w):
    a, w = _f32(a), _f32(w)
    M, K = a.shape
    N = w.shape[1]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_f32(_p(a), _p(w), M, N, K, _p(c))
    return c


def matmul_q4s(a, q, K, N):
    """matmulQ4 reference: dequant (matmul_q4.metal:24-28) then matmul."""
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.uint8)
    M = a.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_q4s(_p(a), _p(q), M, N, K, _p(c))
    return c


def matmul_q8(a, q, K, N):
    """matmulQ8 reference: dequant (matmul_q8.metal:44-52) then matmul."""
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.uint8)
    M = a.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_q8(_p(a), _p(q), M, N, K, _p(c))
    return c


def matmul_gguf(ggml_type, a, q, K, N):
    """y = a . W^T for a GGUF weight listed [out=N, in=K]."""
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.uint8)
    M = a.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    if lib().oracle_matmul_gguf(ggml_type, _p(a), _p(q), M, N, K, _p(c)):
        raise ValueError("unsupported type %d" % ggml_type)
    return c


def normwise_rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))


def elementwise_rel_err(y, ref, atol_frac=1e-3):
    """max |y - ref| / (|ref| + atol) over all elements, atol = atol_frac *
    rms(ref): the per-element relative error, kept finite where an output
    crosses zero."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    atol = atol_frac * float(np.sqrt(np.mean(ref * ref)))
    if atol <= 0:
        atol = 1.0
    return float(np.max(np.abs(y - ref) / (np.abs(ref) + atol)))
