"""Pins the oracle's other GGUF block decoders -- CPU only.

The reference's only tests of these decoders need a real model file that is
not here (tests/gguf_model.test.js:238-362: finite values, |v| < 10, mostly
nonzero).  They are pinned instead by:

  * blocks assembled by an independent packer (a bit-position table written
    from the reference's field description, filled through Python integers)
    from chosen integer fields, decoded and compared with the values those
    fields define -- nibble order, fifth/sixth bits, the packed 6-bit
    scale/min pairs (all 64 x 64 values at every sub-block index), int8 scale
    signs, the f16 fields' byte order;
  * closed forms with unit scales (the decoded block IS the integer field);
  * the reference tests' own criteria on realistic encoded weights;
  * encoder round trips (error bounds) and dequantize_tensor == the block
    decoders back to back (ragged last block cut).
"""
import numpy as np
import pytest

from oracle import oracle as O
from smith_amd import prng

F16 = {1.0: 0x3C00, 0.5: 0x3800, 2.0: 0x4000, 0.25: 0x3400, -3.0: 0xC200, 0.0: 0x0000}


def f16bits(x):
    return int(np.array(x, np.float16).view(np.uint16))


def f16val(x):
    return float(np.array(x, np.float16).astype(np.float64))


class Bits:
    """A little-endian bit string of n bytes written field by field."""

    def __init__(self, nbytes):
        self.v = 0
        self.n = nbytes

    def put(self, bitpos, width, value):
        assert 0 <= value < (1 << width)
        self.v |= value << bitpos

    def bytes(self):
        return np.frombuffer(self.v.to_bytes(self.n, "little"), np.uint8).copy()


# --- layouts from the reference's decoders, as bit positions -----------------

def pack_q4_1(d16, m16, q):
    b = Bits(20)
    b.put(0, 16, d16)
    b.put(16, 16, m16)
    for i, v in enumerate(q):  # element i: byte 4 + i//2, low nibble when i even
        b.put(8 * (4 + i // 2) + 4 * (i % 2), 4, v)
    return b.bytes()


def pack_q5_0(d16, q):
    b = Bits(22)
    b.put(0, 16, d16)
    for i, v in enumerate(q):
        b.put(16 + i, 1, v >> 4)  # bit i of the 32-bit word at byte 2
        b.put(8 * (6 + i // 2) + 4 * (i % 2), 4, v & 15)
    return b.bytes()


def pack_q4_k(d16, dmin16, sc, mn, q):
    b = Bits(144)
    b.put(0, 16, d16)
    b.put(16, 16, dmin16)
    base = 32  # the 12 scale bytes
    for i in range(8):
        if i < 4:
            b.put(base + 8 * i, 6, sc[i])
            b.put(base + 8 * (i + 4), 6, mn[i])
        else:
            b.put(base + 8 * (i - 4) + 6, 2, sc[i] & 3)       # low 2 bits: top of byte i-4
            b.put(base + 8 * (i + 4), 4, sc[i] >> 2)          # high 4 bits: low nibble of byte i+4
            b.put(base + 8 * i + 6, 2, mn[i] & 3)             # low 2 bits: top of byte i
            b.put(base + 8 * (i + 4) + 4, 4, mn[i] >> 2)      # high 4 bits: high nibble of byte i+4
    for j, v in enumerate(q):
        b.put(8 * (16 + j // 2) + 4 * (j % 2), 4, v)
    return b.bytes()


def pack_q6_k(d16, sc, q):
    b = Bits(210)
    for j, v in enumerate(q):
        b.put(8 * (j // 2) + 4 * (j % 2), 4, v & 15)          # ql
        b.put(8 * (128 + j // 4) + 2 * (j % 4), 2, v >> 4)    # qh
    for i, s in enumerate(sc):
        b.put(8 * (192 + i), 8, s & 0xFF)
    b.put(8 * 208, 16, d16)
    return b.bytes()


# --- closed forms -------------------------------------------------------------

def test_q4_1_unit_scale_is_the_nibbles():
    q = [(7 * i + 3) % 16 for i in range(32)]
    got = O.dequant_q4_1_block(pack_q4_1(F16[1.0], F16[0.0], q))
    assert np.array_equal(got, np.array(q, np.float32))
    got = O.dequant_q4_1_block(pack_q4_1(F16[0.5], F16[-3.0], q))
    assert np.array_equal(got, np.array(q, np.float32) * 0.5 - 3.0)


def test_q5_0_fifth_bit_per_element():
    q = list(range(32))  # elements >= 16 carry the fifth bit
    got = O.dequant_q5_0_block(pack_q5_0(F16[1.0], q))
    assert np.array_equal(got, np.arange(32, dtype=np.float32) - 16)
    q = [(13 * i + 5) % 32 for i in range(32)]
    got = O.dequant_q5_0_block(pack_q5_0(F16[0.25], q))
    assert np.array_equal(got, (np.array(q, np.float32) - 16) * 0.25)


def test_q4_k_unit_scales_are_the_nibbles():
    q = [(5 * j + j // 32) % 16 for j in range(256)]
    got = O.dequant_q4_k_block(pack_q4_k(F16[1.0], F16[0.0], [1] * 8, [0] * 8, q))
    assert np.array_equal(got, np.array(q, np.float32))


@pytest.mark.parametrize("i", range(8))
def test_q4_k_every_scale_min_pair_at_every_index(i):
    """All 64 x 64 (scale, min) values of sub-block i (the other sub-blocks
    hold distinct fixed pairs that must not move): value = scale*q - min."""
    q = [(j * 3) % 16 for j in range(256)]
    other_sc = [(11 * k + 7) % 64 for k in range(8)]
    other_mn = [(29 * k + 3) % 64 for k in range(8)]
    for s in range(64):
        sc = list(other_sc)
        sc[i] = s
        for m in (0, 1, 2, 3, 4, 17, 42, 63) if s % 8 else range(64):
            mn = list(other_mn)
            mn[i] = m
            got = O.dequant_q4_k_block(pack_q4_k(F16[1.0], F16[1.0], sc, mn, q))
            want = np.array([sc[j // 32] * q[j] - mn[j // 32] for j in range(256)], np.float32)
            assert np.array_equal(got, want), (i, s, m)


def test_q4_k_f32_scale_products_and_rounding():
    """sc = f32(d*scale) and mn = f32(dmin*min) are exact (11 x 6 bits); the
    value sc*q - mn is rounded once, from f64, to f32."""
    d, dmin = f16val(0.0123), f16val(0.00457)
    sc = [63, 1, 37, 50, 2, 61, 19, 44]
    mn = [5, 63, 0, 22, 41, 7, 60, 33]
    q = [(j * 7) % 16 for j in range(256)]
    got = O.dequant_q4_k_block(pack_q4_k(f16bits(d), f16bits(dmin), sc, mn, q))
    want = np.array([np.float64(np.float32(d * sc[j // 32])) * q[j] - np.float64(np.float32(dmin * mn[j // 32]))
                     for j in range(256)]).astype(np.float32)
    assert np.array_equal(got, want)


def test_q6_k_unit_scale_is_q_minus_32():
    q = [(j * 37) % 64 for j in range(256)]
    got = O.dequant_q6_k_block(pack_q6_k(F16[1.0], [1] * 16, q))
    assert np.array_equal(got, np.array(q, np.float32) - 32)


def test_q6_k_signed_scales_per_16():
    q = [63 if (j // 16) % 2 else 0 for j in range(256)]  # +31 / -32
    sc = [-128, 127, -1, 1, -77, 90, 0, 5, -5, 64, -64, 33, -33, 100, -100, 2]
    got = O.dequant_q6_k_block(pack_q6_k(F16[0.5], sc, q))
    want = np.array([0.5 * sc[j // 16] * (q[j] - 32) for j in range(256)], np.float32)
    assert np.array_equal(got, want)


def test_bf16_and_f16_tensors():
    raw = np.array([0x3F80, 0xC000, 0x0000, 0x7F80], np.uint16).view(np.uint8)
    assert np.array_equal(O.dequantize_tensor(O.GGML_BF16, raw, 4), np.array([1.0, -2.0, 0.0, np.inf], np.float32))
    raw = np.array([0x3C00, 0xC200, 0x3400], np.uint16).view(np.uint8)
    assert np.array_equal(O.dequantize_tensor(O.GGML_F16, raw, 3), np.array([1.0, -3.0, 0.25], np.float32))


# --- tensor decode and encoders ------------------------------------------------

BLOCK_FN = {O.GGML_Q4_0: O.dequant_q4_0_block, O.GGML_Q4_1: O.dequant_q4_1_block,
            O.GGML_Q5_0: O.dequant_q5_0_block, O.GGML_Q8_0: O.dequant_q8_0_block,
            O.GGML_Q4_K: O.dequant_q4_k_block, O.GGML_Q6_K: O.dequant_q6_k_block}
KQ = [O.GGML_Q4_1, O.GGML_Q5_0, O.GGML_Q4_K, O.GGML_Q6_K]


@pytest.mark.parametrize("t", list(BLOCK_FN))
def test_dequantize_tensor_is_blocks_back_to_back(t):
    be, bb = O.BLOCK[t]
    w = prng.randn((3, 2 * be), 40 + t, std=0.05)
    raw = O.quantize_rows(t, w)
    numel = 6 * be - 7  # ragged: the last block is cut
    got = O.dequantize_tensor(t, raw, numel)
    want = np.concatenate([BLOCK_FN[t](raw[k * bb:(k + 1) * bb]) for k in range(6)])[:numel]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t", KQ)
def test_encoders_meet_reference_test_criteria(t):
    """tests/gguf_model.test.js:256-362 on encoded N(0, 0.02) weights: finite,
    |v| < 10, more than 100 of 256 nonzero."""
    be, _ = O.BLOCK[t]
    w = prng.randn((4, 1024), 50 + t, std=0.02)
    v = O.dequantize_tensor(t, O.quantize_rows(t, w), w.size).reshape(-1, 256)
    assert np.all(np.isfinite(v)) and np.all(np.abs(v) < 10)
    assert np.all((v != 0).sum(1) > 100)


@pytest.mark.parametrize("t,bound", [(O.GGML_Q4_1, 0.6 / 15), (O.GGML_Q5_0, 0.6 / 16), (O.GGML_Q4_K, 1.2 / 15),
                                     (O.GGML_Q6_K, 1.2 / 32)])
def test_encoder_round_trip_error(t, bound):
    """Per block, |x - decode(encode(x))| <= bound * (block range): half a
    quantization step (4 / 5 / 6 bits), with slack for the 6-bit / int8
    scale rounding of the super-block formats."""
    be, _ = O.BLOCK[t]
    w = prng.randn((8, 512), 60 + t, std=0.02)
    v = O.dequantize_tensor(t, O.quantize_rows(t, w), w.size).reshape(-1, be)
    x = w.reshape(-1, be).astype(np.float64)
    rng = np.maximum(x.max(1) - np.minimum(x.min(1), 0), np.abs(x).max(1))
    assert np.all(np.abs(v - x).max(1) <= bound * rng * 1.0001 + 1e-7)


def test_matmul_gguf_kquant_vs_numpy():
    K, N, M = 512, 24, 3
    a = prng.randn((M, K), 70)
    for t in KQ:
        w = prng.randn((N, K), 71 + t, std=0.02)
        raw = O.quantize_rows(t, w)
        wd = O.dequantize_tensor(t, raw, N * K).reshape(N, K).astype(np.float64)
        got = O.matmul_gguf(t, a, raw, K, N)
        assert O.normwise_rel_err(got, a.astype(np.float64) @ wd.T) < 1e-6
