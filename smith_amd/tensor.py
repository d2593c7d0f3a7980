"""Minimal device tensor -- the part of src/tensor.js the path needs.

The reference's T.create (src/tensor.js:55-74) returns a pooled SHARED Metal
buffer with a typed-array view (zero copy).  On MI355X the buffer is device
memory: `.data` downloads a host copy and `set_data` uploads, both explicit.
Row-major and contiguous only (the reference's matmulQ4 also passes
a.buffer with no offset or strides, src/ops/quantize.js:83).
"""
import numpy as np

from . import device, prng

_DTYPES = {"f32": np.float32, "i32": np.int32, "u8": np.uint8}


class Tensor:
    __slots__ = ("shape", "dtype", "buffer", "size", "strides", "offset", "_owner")

    def __init__(self, shape, dtype="f32", buffer=None):
        self.shape = [int(s) for s in shape]
        self.dtype = dtype
        self.size = int(np.prod(self.shape)) if self.shape else 1
        st, acc = [], 1
        for s in reversed(self.shape):
            st.append(acc)
            acc *= s
        self.strides = list(reversed(st))
        self.offset = 0
        self._owner = buffer is None
        self.buffer = buffer if buffer is not None else device.alloc(self.nbytes)

    @property
    def nbytes(self):
        return self.size * np.dtype(_DTYPES[self.dtype]).itemsize

    @property
    def data(self):
        """Host copy of the contents (device -> host, waits for the stream)."""
        return device.download(self.buffer, self.nbytes, _DTYPES[self.dtype]).reshape(self.shape)

    def set_data(self, arr):
        a = np.ascontiguousarray(arr, dtype=_DTYPES[self.dtype])
        if a.size != self.size:
            raise ValueError("set_data: %d elements for a tensor of %d" % (a.size, self.size))
        device.upload(self.buffer, a)
        return self

    def release(self):
        if self._owner and self.buffer:
            device.release_buffer(self.buffer)
        self.buffer = None

    def __repr__(self):
        return "Tensor(shape=%s, dtype=%s)" % (self.shape, self.dtype)


def create(shape, dtype="f32"):
    return Tensor(shape, dtype)


def tensor(data, shape=None, dtype="f32"):
    a = np.asarray(data, dtype=_DTYPES[dtype])
    t = Tensor(list(a.shape) if shape is None else shape, dtype)
    return t.set_data(a)


def zeros(shape, dtype="f32"):
    return tensor(np.zeros(shape, dtype=_DTYPES[dtype]), dtype=dtype)


def ones(shape, dtype="f32"):
    return tensor(np.ones(shape, dtype=_DTYPES[dtype]), dtype=dtype)


def randn(shape, seed=0, std=1.0, mean=0.0):
    """Seeded N(mean, std) -- src/tensor.js:127-146 with a reproducible source."""
    return tensor(prng.randn(shape, seed, std=std, mean=mean))


def to_array(t):
    """toArray: nested host values of a tensor."""
    return t.data.tolist()
