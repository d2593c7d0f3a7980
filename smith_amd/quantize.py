"""Quantized matmul ops -- mirror of src/ops/quantize.js.

Same names, arguments, return shapes and error messages as the reference:
  quantizeQ4(weight[K,N]) -> {buffer, K, N, groups, totalBytes}   (quantize.js:14-68)
  matmulQ4(a[M,K], wq)    -> Tensor[M,N]                          (quantize.js:71-90)
  matmulQ8(a[M,K], wq)    -> Tensor[M,N]                          (quantize.js:99-118)
plus quantizeQ8, which the reference lacks (its matmulQ8 consumes a
caller-built buffer).  Each op is one call into libsmith.so; the packed
bytes are produced on the GPU and are byte-exact with the reference layout.
"""
import numpy as np

from . import device
from . import tensor as T

GROUP_SIZE = 32
GROUP_BYTES = 24  # 16 nibble bytes + f32 scale + f32 zero
Q8_BLOCK_SIZE = 32
Q8_BLOCK_BYTES = 34  # f16 scale + 32 x int8


class QuantizedWeight(dict):
    """{buffer, K, N, groups, totalBytes} with attribute access."""

    def __getattr__(self, k):
        try:
            return self[k]
        except KeyError:
            raise AttributeError(k)


def _as_device_weight(weight):
    if isinstance(weight, T.Tensor):
        return weight, None
    w = np.ascontiguousarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("quantize: weight must be 2-D [K, N]")
    t = T.tensor(w)
    return t, t


def _quantize(weight, block_bytes, entry, what):
    w, tmp = _as_device_weight(weight)
    K, N = w.shape
    groups = -(-K // GROUP_SIZE)
    total = groups * N * block_bytes
    ctx = device.ops_ctx()
    buf = device.alloc(total, device.SHARED)
    device.check(entry(ctx, w.buffer, buf, K, N), what)
    if tmp is not None:
        device.sync()
        tmp.release()
    return QuantizedWeight(buffer=buf, K=K, N=N, groups=groups, totalBytes=total)


def quantizeQ4(weight):
    """Pack f32 [K,N] to the reference's Q4 records (scale, zero point per 32)."""
    return _quantize(weight, GROUP_BYTES, device.lib.smith_quantize_q4, "quantizeQ4")


def quantizeQ8(weight):
    """Pack f32 [K,N] to matmulQ8's blocks (f16 scale + 32 x int8 per 32)."""
    return _quantize(weight, Q8_BLOCK_BYTES, device.lib.smith_quantize_q8, "quantizeQ8")


def _matmul(a, bq, entry, what):
    M = a.shape[0]
    N, K, groups = bq["N"], bq["K"], bq["groups"]
    if a.shape[1] != K:
        raise ValueError("%s: inner dims don't match: %d vs %d" % (what, a.shape[1], K))
    out = T.create([M, N], a.dtype)
    device.check(entry(device.ops_ctx(), a.buffer, bq["buffer"], out.buffer, M, N, K, groups), what)
    return out


def matmulQ4(a, bQuant):
    """C[M,N] = A[M,K](f32) @ B[K,N](q4)."""
    return _matmul(a, bQuant, device.lib.smith_matmul_q4, "matmulQ4")


def matmulQ8(a, bQuant):
    """C[M,N] = A[M,K](f32) @ B[K,N](q8)."""
    return _matmul(a, bQuant, device.lib.smith_matmul_q8, "matmulQ8")


def matmul_reference_dispatch(kernel, a, bQuant):
    """The reference's own dispatch of matmul_q4 / matmul_q8
    (src/ops/quantize.js:79-87): one thread per output, grid {x:N, y:M},
    group {min(N,16), min(M,16)}, params u32[M,N,K,groups] at slot 3 --
    through the generic encoder API of the bridge."""
    import struct
    from .dispatch import run
    M = a.shape[0]
    N, K, groups = bQuant["N"], bQuant["K"], bQuant["groups"]
    if a.shape[1] != K:
        raise ValueError("%s: inner dims don't match: %d vs %d"
                         % ("matmulQ4" if kernel == "matmul_q4" else "matmulQ8", a.shape[1], K))
    out = T.create([M, N], a.dtype)
    run(kernel, [{"buffer": a.buffer, "index": 0}, {"buffer": bQuant["buffer"], "index": 1},
                 {"buffer": out.buffer, "index": 2}],
        {"x": N, "y": M}, {"x": min(N, 16), "y": min(M, 16)},
        {"data": struct.pack("<4I", M, N, K, groups), "index": 3})
    return out
