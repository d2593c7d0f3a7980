"""GGUF reader and writer -- mirror of src/gguf.js (parseGGUF, type tables,
extractConfig) plus a writer for synthetic model files.

The reader memory-maps the file: tensor data is never copied on the host
before it is uploaded.  Only the block types the decode path consumes are
decoded here (F32, F16; Q4_0 / Q8_0 blocks are uploaded as bytes and
repacked on the GPU).
"""
import struct

import numpy as np

# GGUF metadata value types (src/gguf.js:7-12)
GGUF_TYPE = dict(UINT8=0, INT8=1, UINT16=2, INT16=3, UINT32=4, INT32=5, FLOAT32=6, BOOL=7, STRING=8, ARRAY=9,
                 UINT64=10, INT64=11, FLOAT64=12)

# GGML tensor types (src/gguf.js:15-25)
GGML_TYPE = dict(F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, Q8_1=9, Q2_K=10, Q3_K=11, Q4_K=12,
                 Q5_K=13, Q6_K=14, IQ2_XXS=16, IQ2_XS=17, IQ3_XXS=18, IQ1_S=19, IQ4_NL=20, IQ3_S=21, IQ2_S=22,
                 IQ4_XS=23, I8=24, I16=25, I32=26, I64=27, F64=28, IQ1_M=29, BF16=30)
GGML_TYPE_NAME = {v: k for k, v in GGML_TYPE.items()}

# block size / bytes per block (src/gguf.js:30-41)
GGML_TYPE_INFO = {
    GGML_TYPE["F32"]: (1, 4), GGML_TYPE["F16"]: (1, 2), GGML_TYPE["Q4_0"]: (32, 18), GGML_TYPE["Q4_1"]: (32, 20),
    GGML_TYPE["Q8_0"]: (32, 34), GGML_TYPE["Q8_1"]: (32, 36), GGML_TYPE["Q5_0"]: (32, 22),
    GGML_TYPE["Q4_K"]: (256, 144), GGML_TYPE["Q6_K"]: (256, 210), GGML_TYPE["BF16"]: (1, 2),
}

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}


class _Reader:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def scalar(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.scalar("<Q")
        # invalid UTF-8 becomes U+FFFD, as TextDecoder does (gguf.js:74)
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def value(self, t):
        if t in _SCALAR:
            return self.scalar(_SCALAR[t])
        if t == GGUF_TYPE["BOOL"]:
            return self.scalar("<B") != 0
        if t == GGUF_TYPE["STRING"]:
            return self.string()
        if t == GGUF_TYPE["ARRAY"]:
            et = self.scalar("<I")
            n = self.scalar("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError("Unknown GGUF value type: %d" % t)


def parseGGUF(buffer):
    """src/gguf.js:127-165: header, metadata, tensor infos, aligned data offset."""
    r = _Reader(buffer)
    magic = r.scalar("<I")
    if magic != 0x46554747:
        raise ValueError("Not a GGUF file (magic: 0x%x)" % magic)
    version = r.scalar("<I")
    if version < 2 or version > 3:
        raise ValueError("Unsupported GGUF version: %d" % version)
    n_tensors = r.scalar("<Q")
    n_kv = r.scalar("<Q")
    metadata = {}
    for _ in range(n_kv):
        key = r.string()
        t = r.scalar("<I")
        metadata[key] = r.value(t)
    tensors = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.scalar("<I")
        shape = [r.scalar("<Q") for _ in range(nd)]
        t = r.scalar("<I")
        off = r.scalar("<Q")
        tensors.append({"name": name, "shape": shape, "type": t, "offset": off})
    align = metadata.get("general.alignment", 32)
    data_offset = -(-r.pos // align) * align
    return {"version": version, "metadata": metadata, "tensors": tensors, "dataOffset": data_offset,
            "buffer": buffer}


def loadGGUFFile(path):
    """Memory-map a GGUF file and parse it."""
    buf = np.memmap(path, dtype=np.uint8, mode="r")
    return parseGGUF(buf)


def tensorBytes(info):
    """src/gguf.js:169-175."""
    ti = GGML_TYPE_INFO.get(info["type"])
    if ti is None:
        raise ValueError("Unsupported tensor type: %s" % GGML_TYPE_NAME.get(info["type"], info["type"]))
    numel = int(np.prod(info["shape"])) if info["shape"] else 1
    return -(-numel // ti[0]) * ti[1]


def readTensorData(parsed, info):
    """src/gguf.js:177-181: a view of the tensor's bytes (no copy)."""
    start = parsed["dataOffset"] + info["offset"]
    return parsed["buffer"][start:start + tensorBytes(info)]


def dense_f32(parsed, info):
    """F32 / F16 tensor as f32 (dequantizeTensor, src/gguf.js:343-362)."""
    data = readTensorData(parsed, info)
    numel = int(np.prod(info["shape"]))
    if info["type"] == GGML_TYPE["F32"]:
        return np.frombuffer(data, dtype=np.float32, count=numel)
    if info["type"] == GGML_TYPE["F16"]:
        return np.frombuffer(data, dtype=np.float16, count=numel).astype(np.float32)
    raise ValueError("not a dense tensor: %s" % GGML_TYPE_NAME.get(info["type"], info["type"]))


def getArch(metadata):
    return metadata.get("general.architecture", "unknown")


def extractConfig(metadata):
    """src/gguf.js:421-439 (same keys and defaults)."""
    arch = getArch(metadata)

    def get(key):
        v = metadata.get("%s.%s" % (arch, key))
        return v if v is not None else metadata.get("general.%s" % key)

    def first(*vals):
        for v in vals:
            if v is not None:
                return v
        return None

    return {
        "arch": arch,
        "name": metadata.get("general.name", "unknown"),
        "vocabSize": first(get("vocab_size"), 32000),
        "dim": first(get("embedding_length"), get("hidden_size")),
        "numLayers": first(get("block_count"), get("num_hidden_layers")),
        "numHeads": first(get("attention.head_count"), get("num_attention_heads")),
        "numKVHeads": first(get("attention.head_count_kv"), get("num_key_value_heads")),
        "maxSeqLen": first(get("context_length"), 2048),
        "ffnDim": get("feed_forward_length"),
        "ropeFreqBase": first(get("rope.freq_base"), 10000),
        "ropeScaling": get("rope.scaling.type"),
        "normEps": first(get("attention.layer_norm_rms_epsilon"), get("attention.layer_norm_epsilon"), 1e-5),
    }


# ---------------------------------------------------------------------------
# Writer (the format buildGGUF in tests/gguf.test.js:22-112 emits).
# ---------------------------------------------------------------------------

def _w_string(parts, s):
    b = s.encode("utf-8")
    parts.append(struct.pack("<Q", len(b)))
    parts.append(b)


def _w_value(parts, t, v):
    if t in _SCALAR:
        parts.append(struct.pack(_SCALAR[t], v))
    elif t == GGUF_TYPE["BOOL"]:
        parts.append(struct.pack("<B", 1 if v else 0))
    elif t == GGUF_TYPE["STRING"]:
        _w_string(parts, v)
    elif t == GGUF_TYPE["ARRAY"]:
        et, items = v
        parts.append(struct.pack("<IQ", et, len(items)))
        for it in items:
            _w_value(parts, et, it)
    else:
        raise ValueError("unknown GGUF value type %d" % t)


def write_gguf(path, metadata, tensors, version=3, alignment=32):
    """metadata: {key: (gguf_type, value)}; tensors: [(name, shape, ggml_type,
    nbytes, producer)] where producer() returns the bytes (called once, in
    order, so large tensors can be generated on the fly)."""
    parts = [struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))]
    for k, (t, v) in metadata.items():
        _w_string(parts, k)
        parts.append(struct.pack("<I", t))
        _w_value(parts, t, v)
    off = 0
    offsets = []
    for name, shape, gt, nbytes, _ in tensors:
        _w_string(parts, name)
        parts.append(struct.pack("<I", len(shape)))
        for d in shape:
            parts.append(struct.pack("<Q", d))
        parts.append(struct.pack("<IQ", gt, off))
        offsets.append(off)
        off += -(-nbytes // alignment) * alignment
    header = b"".join(parts)
    pad = -len(header) % alignment
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * pad)
        pos = 0
        for (name, shape, gt, nbytes, producer), o in zip(tensors, offsets):
            if pos < o:
                f.write(b"\0" * (o - pos))
                pos = o
            data = producer()
            b = memoryview(np.ascontiguousarray(data)).cast("B") if not isinstance(data, (bytes, bytearray)) else data
            if len(b) != nbytes:
                raise ValueError("%s: %d bytes produced, %d declared" % (name, len(b), nbytes))
            f.write(b)
            pos += nbytes
    return path
