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
