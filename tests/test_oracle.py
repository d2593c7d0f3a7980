"""Pins the CPU oracle (oracle/smith_oracle.c) -- CPU only.

How each oracle function is pinned (no reference test can run here: the
reference needs Bun + Metal; it has no golden-vector files):

  from_f16            all 65536 bit patterns vs numpy's IEEE half decoder
  to_f16_trunc        truncation property on 200k values + known answers
  f32_to_f16_rne      bit-exact vs numpy's IEEE RNE conversion (all ranges)
  quantize_q4s        known answers derived from src/ops/quantize.js semantics
                      (identity group, -0 zero point, constant group, JS
                      Math.round ties, ragged K padding, NaN/Inf), the
                      per-element error bound, and the reference's own test
                      criteria (tests/inference.test.js:94-135)
  dequant_q4s         exact reconstruction on the identity/integer groups
  quantize_q8         known answers (amax 127 -> d=1, half-away rounding,
                      all-zero block) + error bound
  dequant_q4_0/q8_0   the reference's known answers (tests/gguf.test.js:208-245)
  quantize_rows       integer round trip through the reference decoder
  matmul_*            vs numpy float64 matmul of the dequantized weights
"""
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O
from smith_amd import prng


def f32bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def rec_fields(q, idx):
    r = q[idx * 24:(idx + 1) * 24]
    nib = []
    for b in r[:16]:
        nib += [b & 15, b >> 4]
    scale = struct.unpack("<f", bytes(r[16:20]))[0]
    zero = struct.unpack("<f", bytes(r[20:24]))[0]
    return nib, scale, zero, bytes(r[16:20]), bytes(r[20:24])


# ---------------- f16 helpers ----------------

def test_from_f16_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float64)
    got = np.array([O.from_f16(int(x)) for x in h])
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # signed zero kept
    assert np.signbit(O.from_f16(0x8000)) and O.from_f16(0x8000) == 0.0


def test_to_f16_trunc_known_answers():
    assert O.to_f16_trunc(1.0) == 0x3C00
    assert O.to_f16_trunc(0.5) == 0x3800
    assert O.to_f16_trunc(-2.0) == 0xC000
    assert O.to_f16_trunc(65504.0) == 0x7BFF
    assert O.to_f16_trunc(65535.0) == 0x7BFF  # exp 15: truncated, not rounded
    assert O.to_f16_trunc(65536.0) == 0x7C00  # exp 16: overflow
    assert O.to_f16_trunc(float("inf")) == 0x7C00
    assert O.to_f16_trunc(float("-inf")) == 0xFC00
    assert O.to_f16_trunc(float("nan")) & 0x7E00 == 0x7E00
    # 1 + 2^-10 + 2^-11 truncates to 1 + 2^-10 (RNE would round to 1+2^-9)
    assert O.to_f16_trunc(1.0 + 2 ** -10 + 2 ** -11) == 0x3C01
    # subnormal results: src/dtype.js:48-54 shifts the 24-bit significand by
    # (-1 - exp) and then by 13 more, i.e. 2^13 too far -- restated as is
    assert O.to_f16_trunc(2.0 ** -24) == 0x0000
    assert O.to_f16_trunc(2.0 ** -15) == 0x0000
    assert O.to_f16_trunc(-(2.0 ** -15) * 1.5) == 0x8000
    assert O.to_f16_trunc(2.0 ** -25) == 0x0000


def test_to_f16_trunc_is_truncation():
    rng = np.random.default_rng(1)
    mag = np.exp2(rng.uniform(-14, 16.5, 200000)).astype(np.float32)  # normal f16 range
    x = mag * rng.choice([-1.0, 1.0], mag.size).astype(np.float32)
    for v in x[:20000]:
        h = O.to_f16_trunc(float(v))
        a = abs(float(v))
        hv = abs(O.from_f16(h))
        if a >= 65536.0:
            assert h & 0x7FFF == 0x7C00
            continue
        assert hv <= a
        nxt = O.from_f16((h & 0x7FFF) + 1)
        assert nxt > a
        assert (h >> 15) == (1 if v < 0 and h & 0x7FFF else h >> 15)


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2 ** 32, 300000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # add the interesting ranges densely: subnormal results, ties, overflow edge
    extra = np.concatenate([
        np.exp2(rng.uniform(-26, -13, 50000)), np.exp2(rng.uniform(14, 17, 50000)),
        np.array([65504, 65519.99, 65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 1 + 2 ** -11, 1 + 3 * 2 ** -11]),
    ]).astype(np.float32)
    x = np.concatenate([x, extra, -extra])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_rne(float(v)) for v in x], dtype=np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


# ---------------- Q4S (quantizeQ4) ----------------

def test_q4s_identity_group_and_negative_zero():
    w = (np.arange(32) % 16).astype(np.float32).reshape(32, 1)
    q = O.quantize_q4s(w)
    assert q.size == 24
    nib, scale, zero, sb, zb = rec_fields(q, 0)
    assert nib == list(range(16)) * 2
    assert scale == 1.0
    assert struct.unpack("<I", zb)[0] == 0x80000000  # -minVal/scale with minVal = 0 -> -0
    # packing: element k -> byte k>>1, even k low nibble
    assert list(q[:8]) == [(2 * j) | ((2 * j + 1) << 4) for j in range(8)]
    assert np.array_equal(O.dequant_q4s(q, 32, 1)[:, 0], w[:, 0])


def test_q4s_constant_group_and_round_half_up():
    w = np.full((32, 3), 0.3, dtype=np.float32)
    w[:, 1] = -3.5  # 8 - 3.5 = 4.5 -> Math.round -> 5
    w[:, 2] = 7.6   # 15.6 clamps to 15
    q = O.quantize_q4s(w)
    for col, expect in [(0, 8), (1, 5), (2, 15)]:
        nib, scale, zero, _, _ = rec_fields(q, col)
        assert scale == 1.0 and zero == 8.0
        assert nib == [expect] * 32


def test_q4s_ties_round_toward_plus_infinity():
    v = np.array([0, 15, 0.5, 1.5, 2.5, 14.5, 7.5, 3.25] + [0] * 24, dtype=np.float32).reshape(32, 1)
    q = O.quantize_q4s(v)
    nib, scale, zero, _, _ = rec_fields(q, 0)
    assert scale == 1.0
    assert nib[:8] == [0, 15, 1, 2, 3, 15, 8, 3]  # JS Math.round: ties up (banker's would give 0,2,2,14,8)


def test_q4s_ragged_k_padding():
    K, N = 100, 2
    w = prng.randn((K, N), 5, std=0.02)
    w[96:, 1] = [-1.5, 13.5, 0.0, 5.0]  # last group of column 1: scale 1, zero 1.5
    q = O.quantize_q4s(w)
    assert q.size == 4 * N * 24
    nib, scale, zero, _, _ = rec_fields(q, 3 * N + 1)
    assert scale == 1.0 and zero == 1.5
    assert nib[:4] == [0, 15, 2, 7]
    assert nib[4:] == [2] * 28  # padded k quantizes v = 0: round(0 + 1.5) = 2


def test_q4s_nan_and_inf():
    w = np.zeros((32, 3), dtype=np.float32)
    w[:, 0] = np.arange(32) % 16
    w[3, 0] = np.nan  # ignored by min/max; its nibble is ToUint8(NaN) = 0
    w[:, 1] = np.nan  # min=+inf, max=-inf -> range -inf -> scale 1, zero 8, all nibbles 0
    w[:, 2] = 1.0
    w[0, 2] = np.inf  # range inf -> scale inf, zero -0, finite v -> 0, inf -> NaN -> 0
    q = O.quantize_q4s(w)
    nib, scale, zero, _, _ = rec_fields(q, 0)
    assert nib[3] == 0 and nib[2] == 2 and scale == 1.0
    nib, scale, zero, _, _ = rec_fields(q, 1)
    assert nib == [0] * 32 and scale == 1.0 and zero == 8.0
    nib, scale, zero, sb, zb = rec_fields(q, 2)
    assert nib == [0] * 32 and scale == float("inf") and struct.unpack("<I", zb)[0] == 0x80000000


def test_q4s_error_bound_random():
    K, N = 256, 64
    w = prng.randn((K, N), 7, std=0.02)
    q = O.quantize_q4s(w)
    d = O.dequant_q4s(q, K, N)
    scale = np.array([[struct.unpack("<f", bytes(q[(g * N + n) * 24 + 16:(g * N + n) * 24 + 20]))[0]
                       for n in range(N)] for g in range(K // 32)], dtype=np.float64)
    bound = np.repeat(scale, 32, axis=0) * (0.5 + 1e-5) + 1e-9
    assert np.all(np.abs(d.astype(np.float64) - w) <= bound)


def test_q4s_reference_test_criteria():
    # tests/inference.test.js:94-123: rand [64,32], ones activation, column sums within 15%
    K, N = 64, 32
    w = prng.uniform(11, 0, K * N).astype(np.float32).reshape(K, N)
    q = O.quantize_q4s(w)
    assert q.size == 2 * N * 24
    out = O.matmul_q4s(np.ones((1, K), np.float32), q, K, N)[0]
    exp = w.sum(axis=0)
    assert np.all(np.abs(out - exp) / (np.abs(exp) + 1e-6) < 0.15)
    # tests/inference.test.js:125-135
    assert (256 // 32) * 256 * 24 / (256 * 256 * 4) < 0.35


# ---------------- Q8 ----------------

def test_q8_known_answers():
    w = np.zeros((32, 2), dtype=np.float32)
    w[:8, 0] = [127, -127, 63.5, -63.5, 0.5, -0.5, 1.49, -1.51]
    q = O.quantize_q8(w)
    b = q[:34]
    assert int(b[0]) | (int(b[1]) << 8) == 0x3C00  # d = 127/127 = 1
    vals = b[2:10].astype(np.int8).tolist()
    assert vals == [127, -127, 64, -64, 1, -1, 1, -2]  # roundf: half away from zero
    b = q[34:68]  # all-zero block: d = 0, id = 0
    assert b[0] == 0 and b[1] == 0 and not np.any(b[2:])
    assert np.array_equal(O.dequant_q8(q, 32, 2)[:, 0], w[:, 0].round() * 0 + np.array(
        [127, -127, 64, -64, 1, -1, 1, -2] + [0] * 24, dtype=np.float32))


def test_q8_error_bound():
    K, N = 96, 40
    w = prng.randn((K, N), 8, std=0.02)
    q = O.quantize_q8(w)
    d = O.dequant_q8(q, K, N)
    amax = np.abs(w.reshape(K // 32, 32, N)).max(axis=1)
    # |f16(d)*q - x| <= d/2 + |q|*|f16(d)-d| <= d*(0.5 + 127*2^-11)
    bound = np.repeat(amax / 127.0, 32, axis=0) * (0.5 + 127 * 2.0 ** -11) * 1.0001 + 1e-9
    assert np.all(np.abs(d - w) <= bound)


# ---------------- GGUF blocks ----------------

def test_q4_0_block_known_answers():
    # tests/gguf.test.js:208-226
    blk = np.zeros(18, dtype=np.uint8)
    blk[0], blk[1] = 0x00, 0x38
    blk[2:] = 0x88
    assert np.allclose(O.dequant_q4_0_block(blk), 0.0)
    blk[2:] = 0xFF
    assert O.dequant_q4_0_block(blk)[0] == 3.5
    # interleaved order: element 1 is the HIGH nibble of byte 0 (src/gguf.js:192-193)
    blk[2:] = 0
    blk[2] = 0x9F  # low = 15 -> element 0, high = 9 -> element 1
    v = O.dequant_q4_0_block(blk)
    assert v[0] == 0.5 * 7 and v[1] == 0.5 * 1 and v[2] == 0.5 * -8


def test_q8_0_block_known_answers():
    # tests/gguf.test.js:228-245
    blk = np.zeros(34, dtype=np.uint8)
    blk[0], blk[1] = 0x00, 0x3C
    blk[2:] = [1 if i % 2 == 0 else 255 for i in range(32)]
    v = O.dequant_q8_0_block(blk)
    assert v[0] == 1.0 and v[1] == -1.0 and v[2] == 1.0


def test_q4_0_encoder_round_trip():
    x = np.array(list(range(-8, 8)) * 2, dtype=np.float32).reshape(1, 32)
    q = O.quantize_rows(O.GGML_Q4_0, x)
    assert int(q[0]) | (int(q[1]) << 8) == 0x3C00  # max-magnitude element -8 -> d = -8/-8 = 1
    qs = [int(v) + 8 for v in x[0]]
    assert list(q[2:18]) == [qs[2 * j] | (qs[2 * j + 1] << 4) for j in range(16)]
    assert np.array_equal(O.dequantize_tensor(O.GGML_Q4_0, q, 32), x[0])
    # random rows: error <= d/2 except at the +8 clamp (q = 16 -> 15), where it is <= d;
    # the f16 scale adds |q - 8| * |f16(d) - d| <= 8 * 2^-11 * d
    x = prng.randn((4, 96), 9, std=0.02)
    q = O.quantize_rows(O.GGML_Q4_0, x)
    d = O.dequantize_tensor(O.GGML_Q4_0, q, x.size).reshape(x.shape)
    amax = np.abs(x.reshape(4, 3, 32)).max(axis=2)
    assert np.all(np.abs(d - x).reshape(4, 3, 32) <= (amax / 8 * (1 + 8 * 2.0 ** -11) * 1.0001 + 1e-9)[..., None])


def test_q8_0_encoder_round_trip():
    x = np.array(list(range(-127, 128, 8)), dtype=np.float32)[:32].reshape(1, 32)
    x[0, 0] = -127
    q = O.quantize_rows(O.GGML_Q8_0, x)
    assert np.array_equal(O.dequantize_tensor(O.GGML_Q8_0, q, 32), x[0])


# ---------------- matmul references ----------------

@pytest.mark.parametrize("M,K,N", [(1, 64, 32), (3, 100, 17), (5, 256, 48)])
def test_matmul_refs_vs_numpy(M, K, N):
    a = prng.randn((M, K), 1)
    w = prng.randn((K, N), 2, std=0.02)
    ref = a.astype(np.float64) @ w.astype(np.float64)
    assert O.normwise_rel_err(O.matmul_f64acc(a, w), ref) < 1e-6
    assert O.normwise_rel_err(O.matmul_f32(a, w), ref) < 1e-5
    q = O.quantize_q4s(w)
    dq = O.dequant_q4s(q, K, N).astype(np.float64)
    assert O.normwise_rel_err(O.matmul_q4s(a, q, K, N), a.astype(np.float64) @ dq) < 1e-6
    q8 = O.quantize_q8(w)
    dq8 = O.dequant_q8(q8, K, N).astype(np.float64)
    assert O.normwise_rel_err(O.matmul_q8(a, q8, K, N), a.astype(np.float64) @ dq8) < 1e-6


def test_matmul_gguf_vs_numpy():
    M, N, K = 3, 24, 96
    a = prng.randn((M, K), 3)
    w = prng.randn((N, K), 4, std=0.02)  # GGUF listing [out, in]
    for t in (O.GGML_Q4_0, O.GGML_Q8_0):
        q = O.quantize_rows(t, w)
        wd = O.dequantize_tensor(t, q, N * K).reshape(N, K).astype(np.float64)
        assert O.normwise_rel_err(O.matmul_gguf(t, a, q, K, N), a.astype(np.float64) @ wd.T) < 1e-6


# ---------------- committed fixtures ----------------

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


def test_golden_fixtures():
    g = np.load(GOLDEN)
    assert np.array_equal(prng.splitmix64(0, 0, 8), g["splitmix_seed0"])
    assert np.allclose(prng.randn((16,), 0), g["randn_seed0"], rtol=1e-6, atol=0)
    w = prng.randn((70, 24), 3, std=0.02)
    assert np.array_equal(w, g["w_q4s"])
    assert np.array_equal(O.quantize_q4s(g["w_q4s"]), g["q4s_bytes"])
    assert np.array_equal(O.quantize_q8(g["w_q8"]), g["q8_bytes"])
    assert np.array_equal(O.quantize_rows(O.GGML_Q4_0, g["w_q4_0"]), g["q4_0_bytes"])


def test_splitmix64_published_vectors():
    # first outputs of the reference SplitMix64 (Steele/Lea/Flood; Vigna's splitmix64.c) for seed 0
    assert [int(x) for x in prng.splitmix64(0, 0, 3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                                         0x06C45D188009454F]
    u = prng.uniform(0, 0, 1000)
    assert np.all((u > 0) & (u <= 1))
