"""GGUF header parsing edge cases (src/gguf.js:60-165), CPU only."""
import struct

import numpy as np

from smith_amd import gguf as G


def _header_with_string(key, raw):
    out = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
    out += struct.pack("<Q", len(key)) + key
    out += struct.pack("<I", G.GGUF_TYPE["STRING"]) + struct.pack("<Q", len(raw)) + raw
    return out + b"\0" * (-len(out) % 32)


def test_invalid_utf8_string_is_replaced_like_textdecoder():
    # TextDecoder (gguf.js:74) turns each invalid byte into U+FFFD instead of throwing
    raw = b"ab\xff\xfecd\xc3"
    parsed = G.parseGGUF(np.frombuffer(_header_with_string(b"tokenizer.x", raw), np.uint8))
    assert parsed["metadata"]["tokenizer.x"] == "ab��cd�"


def test_valid_utf8_string_round_trip():
    s = "smith é中"
    parsed = G.parseGGUF(np.frombuffer(_header_with_string(b"general.name", s.encode()), np.uint8))
    assert parsed["metadata"]["general.name"] == s


def _kv(key, t, payload):
    return struct.pack("<Q", len(key)) + key + struct.pack("<I", t) + payload


def test_int8_values_advance_one_byte():
    """An INT8 value takes one byte.  Deliberate divergence: the reference's
    readValue returns getInt8 at the cursor without advancing it
    (src/gguf.js:93), so after an INT8 scalar, or inside an array of INT8
    (readValue per element, :108), it misreads every following field; this
    parser advances, so the keys after them parse."""
    T = G.GGUF_TYPE
    kvs = [_kv(b"a.int8", T["INT8"], struct.pack("<b", -3)),
           _kv(b"a.int8s", T["ARRAY"], struct.pack("<IQ", T["INT8"], 4) + struct.pack("<4b", -1, 2, -128, 127)),
           _kv(b"a.after", T["UINT32"], struct.pack("<I", 0xC0FFEE))]
    out = struct.pack("<IIQQ", 0x46554747, 3, 0, len(kvs)) + b"".join(kvs)
    out += b"\0" * (-len(out) % 32)
    md = G.parseGGUF(np.frombuffer(out, np.uint8))["metadata"]
    assert md["a.int8"] == -3
    assert md["a.int8s"] == [-1, 2, -128, 127]
    assert md["a.after"] == 0xC0FFEE
