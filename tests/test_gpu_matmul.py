"""GPU parity: the HIP path (libsmith.so + gfx950 code object) against the CPU
oracle on the same seeded inputs.

Bars (stated by the path's spec):
  * packed bytes (quantizeQ4, quantizeQ8, Q4_0 encoder, Q4_0 repack):
    bit-exact with the oracle;
  * matmul outputs: normwise max|y - ref| / max|ref| <= 1e-3 against the f32
    dequantize-then-matmul result (accumulated in f64).  The hi/lo
    activation split (M <= 8) is additionally held to 2e-5;
  * configs 1-3 also report and bound the elementwise
    max|y - ref| / (|ref| + 1e-3 rms(ref)) (bars at ELEM_* below).
"""
import numpy as np
import pytest

import smith_amd as S
from oracle import oracle as O
from smith_amd import device, prng

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_HILO = 2e-5
TOL_GEMM = 1e-2  # f16 activations and f16 dequantized weights on MFMA (M >= 64)
# Elementwise max|y - ref| / (|ref| + 1e-3 rms(ref)) of the GEMVs (configs
# 1-3), per path (observed maxima on MI355X in brackets):
#   M <= 2, single-row kernels: hi/lo activations, the MFMA sums a * (offset +
#     q) and the offset term C1 comes off in f32 afterwards, which costs ~7
#     bits near zero outputs: 5e-2 [Q4S 1.8e-2, Q4_0 9.7e-3, Q8 1.5e-3];
#   3 <= M <= 8: hi/lo activations and exact q operands (offsets removed in
#     f16 before the MFMA): 1e-3 [2.4e-4];
#   9 <= M <= 32: plain f16 activations (2^-11 relative rounding per
#     element; normwise ~2e-4): near-zero outputs carry errors of the order
#     of atol, bar 1.0 [0.57].
ELEM_M2 = 5e-2
ELEM_HILO = 1e-3
ELEM_F16 = 1.0


def elem(y, ref, what):
    e = O.elementwise_rel_err(y, ref)
    print("elementwise", what, "%.3e" % e, flush=True)
    return e


def elem_bar(M):
    return ELEM_M2 if M <= 2 else ELEM_HILO if M <= 8 else ELEM_F16


def dev_bytes(q):
    return device.download(q["buffer"], q["totalBytes"], np.uint8)


def err(y, ref):
    return O.normwise_rel_err(y, ref)


# ---------------- quantizers: bit-exact ----------------

def edge_weight():
    K, N = 96, 8
    w = prng.randn((K, N), 21, std=0.02)
    w[:32, 0] = np.arange(32) % 16            # identity group, zero = -0
    w[:, 1] = 0.3                              # constant groups
    w[:32, 2] = [0, 15, 0.5, 1.5, 2.5, 14.5, 7.5, 3.25] + [0] * 24  # ties
    w[3, 3] = np.nan                           # NaN element
    w[32:64, 4] = np.nan                       # all-NaN group
    w[64, 5] = np.inf                          # infinite element
    w[65, 6] = -np.inf
    w[:, 7] = -0.0
    return w


@pytest.mark.parametrize("K,N,seed", [(32, 1, 1), (64, 32, 2), (100, 3, 3), (70, 24, 4), (4096, 256, 5),
                                      (33, 300, 6)])
def test_quantize_q4_bit_exact(K, N, seed):
    w = prng.randn((K, N), seed, std=0.02)
    q = S.quantizeQ4(S.tensor(w))
    assert (q.K, q.N, q.groups, q.totalBytes) == (K, N, -(-K // 32), -(-K // 32) * N * 24)
    assert np.array_equal(dev_bytes(q), O.quantize_q4s(w))


def test_quantize_q4_edge_values_bit_exact():
    w = edge_weight()
    assert np.array_equal(dev_bytes(S.quantizeQ4(w)), O.quantize_q4s(w))


def test_quantize_q4_golden_fixture():
    g = np.load(__file__.replace("test_gpu_matmul.py", "golden/golden.npz"))
    assert np.array_equal(dev_bytes(S.quantizeQ4(g["w_q4s"])), g["q4s_bytes"])
    assert np.array_equal(dev_bytes(S.quantizeQ8(g["w_q8"])), g["q8_bytes"])


@pytest.mark.parametrize("K,N,seed", [(32, 2, 1), (100, 17, 2), (4096, 128, 3)])
def test_quantize_q8_bit_exact(K, N, seed):
    w = prng.randn((K, N), seed, std=0.02)
    w[0, 0] = 0.0
    assert np.array_equal(dev_bytes(S.quantizeQ8(w)), O.quantize_q8(w))


def test_quantize_q4_0_rows_bit_exact():
    rows, cols = 48, 256
    x = prng.randn((rows, cols), 31, std=0.02)
    x[0, :32] = np.arange(-8, 24) % 16 - 8
    xt = S.tensor(x)
    out = device.alloc(rows * cols // 32 * 18)
    device.check(device.lib.smith_quantize_q4_0(device.ops_ctx(), xt.buffer, out, rows, cols))
    got = device.download(out, rows * cols // 32 * 18, np.uint8)
    assert np.array_equal(got, O.quantize_rows(O.GGML_Q4_0, x))


# ---------------- matmul parity ----------------

MS = [1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 70]
SHAPES = [(32, 1), (100, 17), (256, 64), (1024, 300)]


@pytest.mark.parametrize("K,N", SHAPES)
def test_matmul_q4_parity(K, N):
    w = prng.randn((K, N), 41, std=0.02)
    q = S.quantizeQ4(w)
    qb = dev_bytes(q)
    dq = O.dequant_q4s(qb, K, N).astype(np.float64)
    for M in MS:
        a = prng.randn((M, K), 100 + M)
        y = S.matmulQ4(S.tensor(a), q).data
        assert y.shape == (M, N)
        ref = a.astype(np.float64) @ dq
        e = err(y, ref)
        assert e <= tol_for(M, K), (M, K, N, e)


def tol_for(M, K):
    if M >= 64 and K % 32 == 0:
        return TOL_GEMM
    return TOL_HILO if M <= 8 else TOL


@pytest.mark.parametrize("K,N", SHAPES)
def test_matmul_q8_parity(K, N):
    w = prng.randn((K, N), 42, std=0.02)
    q = S.quantizeQ8(w)
    dq = O.dequant_q8(dev_bytes(q), K, N).astype(np.float64)
    for M in MS:
        a = prng.randn((M, K), 200 + M)
        y = S.matmulQ8(S.tensor(a), q).data
        ref = a.astype(np.float64) @ dq
        e = err(y, ref)
        assert e <= tol_for(M, K), (M, K, N, e)


def test_matmul_q4_oracle_matmul_small():
    # the oracle's own quantize -> dequant -> matmul chain end to end
    K, N, M = 100, 24, 3
    w = prng.randn((K, N), 43, std=0.02)
    a = prng.randn((M, K), 44)
    y = S.matmulQ4(S.tensor(a), S.quantizeQ4(w)).data
    assert err(y, O.matmul_q4s(a, O.quantize_q4s(w), K, N)) <= TOL_HILO


def test_reference_dispatch_kernels():
    """matmul_q4 / matmul_q8 bound exactly as src/ops/quantize.js:82-87 binds them."""
    from smith_amd.quantize import matmul_reference_dispatch
    K, N, M = 100, 40, 5
    w = prng.randn((K, N), 45, std=0.02)
    a = prng.randn((M, K), 46)
    at = S.tensor(a)
    q4, q8 = S.quantizeQ4(w), S.quantizeQ8(w)
    y4 = matmul_reference_dispatch("matmul_q4", at, q4).data
    y8 = matmul_reference_dispatch("matmul_q8", at, q8).data
    assert err(y4, O.matmul_q4s(a, O.quantize_q4s(w), K, N)) <= 1e-6
    assert err(y8, O.matmul_q8(a, O.quantize_q8(w), K, N)) <= 1e-6


def test_matmul_deterministic_and_k_mismatch():
    K, N = 4096, 512
    q = S.quantizeQ4(prng.randn((K, N), 47, std=0.02))
    a = S.tensor(prng.randn((1, K), 48))
    y1 = S.matmulQ4(a, q).data
    y2 = S.matmulQ4(a, q).data
    assert np.array_equal(y1, y2)  # split-K reduction order is fixed
    with pytest.raises(ValueError, match="inner dims don't match: 100 vs 4096"):
        S.matmulQ4(S.tensor(np.zeros((1, 100), np.float32)), q)


# ---------------- GGUF Q4_0 ----------------

@pytest.mark.parametrize("N,K", [(16, 32), (40, 96), (300, 1024)])
def test_q4_0_repack_and_matmul(N, K):
    w = prng.randn((N, K), 51, std=0.02)  # GGUF listing [out, in]
    blocks = O.quantize_rows(O.GGML_Q4_0, w)
    G = K // 32
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    nib = device.alloc(N * G * 16)
    dsc = device.alloc(N * G * 2)
    ctx = device.ops_ctx()
    device.check(device.lib.smith_repack_q4_0(ctx, src, nib, dsc, N, K))
    got_nib = device.download(nib, N * G * 16, np.uint8).reshape(G, N, 16)
    got_d = device.download(dsc, N * G * 2, np.uint8).reshape(G, N, 2)
    b = blocks.reshape(N, G, 18)
    assert np.array_equal(got_nib, b[:, :, 2:].transpose(1, 0, 2))
    assert np.array_equal(got_d, b[:, :, :2].transpose(1, 0, 2))
    wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N * K).reshape(N, K).astype(np.float64)
    for M in MS:
        a = prng.randn((M, K), 300 + M)
        at = S.tensor(a)
        out = S.create([M, N])
        device.check(device.lib.smith_matmul_q4_0(ctx, at.buffer, nib, dsc, out.buffer, M, N, K))
        e = err(out.data, a.astype(np.float64) @ wd.T)
        assert e <= tol_for(M, K), (M, N, K, e)


# ---------------- the benchmark configurations at full size ----------------

def test_config1_q4_gemv_4096():
    K = N = 4096
    w = prng.randn((K, N), 1, std=0.02)
    a = prng.randn((1, K), 0)
    q = S.quantizeQ4(w)
    qb = dev_bytes(q)
    assert np.array_equal(qb, O.quantize_q4s(w))
    y = S.matmulQ4(S.tensor(a), q).data
    ref = O.matmul_q4s(a, qb, K, N)
    assert err(y, ref) <= TOL_HILO
    assert elem(y, ref, "cfg1 q4s") <= ELEM_M2


@pytest.mark.parametrize("M", [1, 4, 32])
def test_config1_q4_0_tile_planes_gemv(M):
    """Config 1 on GGUF Q4_0 blocks in the tile-major planes the GGUF loader
    holds (bench.py's headline_q4_0 kernel at M = 1): repacked from the
    oracle's encoder bytes, against the float64 product of the decoded
    weights."""
    K = N = 4096
    w = prng.randn((N, K), 1, std=0.02)  # GGUF listing [out, in]
    blocks = O.quantize_rows(O.GGML_Q4_0, w)
    G = K // 32
    ctx = device.ops_ctx()
    src, nib, dsc = device.alloc(blocks.size), device.alloc(N * G * 16), device.alloc(N * G * 2)
    device.upload(src, blocks)
    device.check(device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N, K, 0, 1, N))
    wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N * K).reshape(N, K).astype(np.float64)
    a = prng.randn((M, K), 0)
    at = S.tensor(a)
    out = S.create([M, N])
    device.check(device.lib.smith_linear_q4_0_t(ctx, at.buffer, nib, dsc, out.buffer, M, N, K, None, 0.0, None, 0))
    ref = a.astype(np.float64) @ wd.T
    assert err(out.data, ref) <= (TOL_HILO if M <= 8 else TOL)
    assert elem(out.data, ref, "cfg1 q4_0 tiles M=%d" % M) <= elem_bar(M)
    for b in (src, nib, dsc):
        device.release_buffer(b)


@pytest.mark.parametrize("N,K", [(4096, 14336), (4004, 9248), (3600, 12288)])
def test_single_row_long_k_one_block(N, K):
    """M = 1 with 288 < K/32 <= 448 and 225-320 column tiles: one 16-wave
    block covers all of K (no split-K finish); ragged N and a K whose last
    waves hold no groups, Q4S records and Q4_0 tile planes against the
    float64 product of the decoded weights."""
    w = prng.randn((K, N), 71, std=0.02)
    q = S.quantizeQ4(w)
    dq = O.dequant_q4s(dev_bytes(q), K, N).astype(np.float64)
    a = prng.randn((1, K), 72)
    y = S.matmulQ4(S.tensor(a), q).data
    ref = a.astype(np.float64) @ dq
    assert err(y, ref) <= TOL_HILO
    assert elem(y, ref, "q4s M=1 N=%d K=%d" % (N, K)) <= ELEM_M2
    if N % 16 == 0:
        wt = prng.randn((N, K), 73, std=0.02)
        blocks = O.quantize_rows(O.GGML_Q4_0, wt)
        G = K // 32
        ctx = device.ops_ctx()
        src, nib, dsc = device.alloc(blocks.size), device.alloc(N * G * 16), device.alloc(N * G * 2)
        device.upload(src, blocks)
        device.check(device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N, K, 0, 1, N))
        wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N * K).reshape(N, K).astype(np.float64)
        at = S.tensor(a)
        out = S.create([1, N])
        device.check(device.lib.smith_linear_q4_0_t(ctx, at.buffer, nib, dsc, out.buffer, 1, N, K, None, 0.0, None, 0))
        ref = a.astype(np.float64) @ wd.T
        assert err(out.data, ref) <= TOL_HILO
        assert elem(out.data, ref, "q4_0 tiles M=1 N=%d K=%d" % (N, K)) <= ELEM_M2
        for b in (src, nib, dsc):
            device.release_buffer(b)


def test_gemv_activations_beyond_f16_range():
    """The GEMVs (M <= 32, K % 32 == 0) feed f16 operands to the MFMAs but
    keep the reference's f32 range: rows with entries up to 1e6 / 3e30 next
    to rows of ordinary size (every row bucket, Q4S, Q8 and Q4_0 tile
    planes) match the float64 product of the decoded weights row by row at
    the usual bars (a wave whose f16 sums overflow recomputes its part in
    f32)."""
    N, K = 512, 1024
    w = prng.randn((K, N), 81, std=0.02)
    q4, q8 = S.quantizeQ4(w), S.quantizeQ8(w)
    dq4 = O.dequant_q4s(dev_bytes(q4), K, N).astype(np.float64)
    dq8 = O.dequant_q8(dev_bytes(q8), K, N).astype(np.float64)
    wt = prng.randn((N, K), 82, std=0.02)
    blocks = O.quantize_rows(O.GGML_Q4_0, wt)
    G = K // 32
    ctx = device.ops_ctx()
    src, nib, dsc = device.alloc(blocks.size), device.alloc(N * G * 16), device.alloc(N * G * 2)
    device.upload(src, blocks)
    device.check(device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N, K, 0, 1, N))
    wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N * K).reshape(N, K).astype(np.float64)
    for M in (1, 2, 4, 8, 16, 32):
        a = prng.randn((M, K), 83 + M)
        a[0, 5] = 1.0e6                  # one huge entry, the rest ordinary
        if M > 1:
            a[1] *= 3.0e4                # a whole row near the f16 limit
            a[M - 1, 700:710] = -3.0e30  # far beyond it, beside ordinary rows
        at = S.tensor(a)
        out = S.create([M, N])
        device.check(device.lib.smith_linear_q4_0_t(ctx, at.buffer, nib, dsc, out.buffer, M, N, K, None, 0.0, None, 0))
        bar = TOL_HILO if M <= 8 else TOL
        for name, y, ref in (("q4s", S.matmulQ4(at, q4).data, a.astype(np.float64) @ dq4),
                             ("q8", S.matmulQ8(at, q8).data, a.astype(np.float64) @ dq8),
                             ("q4_0 tiles", out.data, a.astype(np.float64) @ wd.T)):
            assert np.isfinite(y).all(), (name, M)
            for m in range(M):
                e = err(y[m], ref[m])
                assert e <= bar, (name, M, m, e)
    for b in (src, nib, dsc):
        device.release_buffer(b)


def test_gemv_beyond_f16_range_ragged_k():
    """K % 32 != 0 (the prepared-activation batched GEMV, M > 2, and the
    fused single-row one) with rows beyond the f16 range: the same f32
    results as the reference, Q4S and Q8, per row at the usual bars."""
    N, K = 200, 1000
    w = prng.randn((K, N), 95, std=0.02)
    q4, q8 = S.quantizeQ4(w), S.quantizeQ8(w)
    dq4 = O.dequant_q4s(dev_bytes(q4), K, N).astype(np.float64)
    dq8 = O.dequant_q8(dev_bytes(q8), K, N).astype(np.float64)
    for M in (1, 4, 16, 32):
        a = prng.randn((M, K), 96 + M)
        a[0, 999] = 2.0e5
        if M > 1:
            a[M - 1, :40] = -7.0e4
        at = S.tensor(a)
        for name, y, ref in (("q4s", S.matmulQ4(at, q4).data, a.astype(np.float64) @ dq4),
                             ("q8", S.matmulQ8(at, q8).data, a.astype(np.float64) @ dq8)):
            assert np.isfinite(y).all(), (name, M)
            for m in range(M):
                assert err(y[m], ref[m]) <= (TOL_HILO if M <= 8 else TOL), (name, M, m)


def test_gemv_infinite_and_nan_activations():
    """An infinite or NaN activation gives the reference's non-finite
    outputs (f32: inf * w is +-inf, or NaN where w = 0; NaN spreads) in its
    row only, for M = 1 / 4 / 16 / 32; the other rows stay at the usual
    bars."""
    N, K = 256, 512
    w = prng.randn((K, N), 91, std=0.02)
    q4 = S.quantizeQ4(w)
    dq4 = O.dequant_q4s(dev_bytes(q4), K, N).astype(np.float64)
    for M in (1, 4, 16, 32):
        a = prng.randn((M, K), 92 + M)
        a[0, 33] = np.inf
        if M > 1:
            a[M - 1, 400] = np.nan
        y = S.matmulQ4(S.tensor(a), q4).data
        with np.errstate(invalid="ignore", over="ignore"):
            ref = a.astype(np.float64) @ dq4
        assert np.array_equal(np.isnan(y), np.isnan(ref)), M
        assert np.array_equal(np.isposinf(y), np.isposinf(ref)), M
        assert np.array_equal(np.isneginf(y), np.isneginf(ref)), M
        for m in range(1, M - 1):
            assert err(y[m], ref[m]) <= (TOL_HILO if M <= 8 else TOL), (M, m)


@pytest.mark.parametrize("N", [1024, 1040])
def test_q8_chunked_and_window_reads_agree(N):
    """Single-row Q8 matmuls read whole 16-column record runs as 16-byte
    chunks when N % 16 == 0 (two-tile blocks: N % 32 == 0) and the weight is
    16-byte aligned, else each record's own 36-byte window: the same records
    through both readers give bit-identical outputs (the weight copied to a
    2-byte offset forces the window reader), within the GEMV bar of the
    oracle."""
    K = 512
    w = prng.randn((K, N), 73, std=0.02)
    a = prng.randn((1, K), 74)
    q = S.quantizeQ8(w)
    raw = dev_bytes(q)
    ctx = device.ops_ctx()
    at = S.tensor(a)
    out0 = S.create([1, N])
    device.check(device.lib.smith_matmul_q8(ctx, at.buffer, q["buffer"], out0.buffer, 1, N, K, K // 32))
    buf = device.alloc(raw.size + 64)
    device.upload(buf, raw, 2)
    out1 = S.create([1, N])
    device.check(device.lib.smith_matmul_q8(ctx, at.buffer, buf + 2, out1.buffer, 1, N, K, K // 32))
    y0, y1 = out0.data, out1.data
    device.release_buffer(buf)
    assert np.array_equal(y0, y1)
    ref = a.astype(np.float64) @ O.dequant_q8(raw, K, N).astype(np.float64)
    assert err(y0, ref) <= TOL_HILO


def test_config2_q8_gemv_14336():
    K, N = 4096, 14336
    w = prng.randn((K, N), 1, std=0.02)
    a = prng.randn((1, K), 0)
    q = S.quantizeQ8(w)
    qb = dev_bytes(q)
    assert np.array_equal(qb, O.quantize_q8(w))
    y = S.matmulQ8(S.tensor(a), q).data
    ref = O.matmul_q8(a, qb, K, N)
    assert err(y, ref) <= TOL_HILO
    assert elem(y, ref, "cfg2 q8") <= ELEM_M2


@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_config3_batched_decode_sweep(N, K):
    w = prng.randn((K, N), 2, std=0.02)  # Smith weight [K, N]
    q = S.quantizeQ4(w)
    dq = O.dequant_q4s(dev_bytes(q), K, N).astype(np.float64)
    for M in (1, 4, 8, 16, 32):
        a = prng.randn((M, K), 10 + M)
        y = S.matmulQ4(S.tensor(a), q).data
        ref = a.astype(np.float64) @ dq
        e = err(y, ref)
        assert e <= (TOL_HILO if M <= 8 else TOL), (M, N, K, e)
        ee = elem(y, ref, "cfg3 q4s M=%d N=%d K=%d" % (M, N, K))
        assert ee <= elem_bar(M), (M, N, K, ee)


@pytest.mark.parametrize("N,K", [(2048, 1024), (512, 1024), (6144, 512), (2048, 8192), (4080, 4096)])
def test_batched_decode_variants_q4s_q8(N, K):
    """2 < M <= 32 on matmulQ4 / matmulQ8 at shapes that select each variant
    of the one-launch kernel (whole K per workgroup; 32-group K ranges over
    16- or 64-column tiles; 64-group ranges over 32 columns at M > 16,
    N = 4080 ending in a half-empty column block), every row bucket
    including partial ones."""
    w = prng.randn((K, N), 61, std=0.02)
    q4, q8 = S.quantizeQ4(w), S.quantizeQ8(w)
    dq4 = O.dequant_q4s(dev_bytes(q4), K, N).astype(np.float64)
    dq8 = O.dequant_q8(dev_bytes(q8), K, N).astype(np.float64)
    for M in (3, 6, 8, 12, 16, 20, 32):
        a = prng.randn((M, K), 62 + M)
        at = S.tensor(a)
        for name, y, dq in (("q4", S.matmulQ4(at, q4).data, dq4), ("q8", S.matmulQ8(at, q8).data, dq8)):
            e = err(y, a.astype(np.float64) @ dq)
            assert e <= (TOL_HILO if M <= 8 else TOL), (name, M, N, K, e)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_config4_prefill_gemm(N, K):
    """Config 4 on the MFMA GEMM: M=512 checked in full, M=2048 on 512
    random output columns (float64 reference over the dequantized bytes)."""
    w = prng.randn((K, N), 3, std=0.02)
    q = S.quantizeQ4(w)
    dq = O.dequant_q4s(dev_bytes(q), K, N).astype(np.float64)
    a = prng.randn((512, K), 20)
    y = S.matmulQ4(S.tensor(a), q).data
    e = err(y, a.astype(np.float64) @ dq)
    assert e <= TOL_GEMM, e
    a = prng.randn((2048, K), 21)
    y = S.matmulQ4(S.tensor(a), q).data
    cols = np.sort(np.random.default_rng(0).choice(N, 512, replace=False))
    e = err(y[:, cols], a.astype(np.float64) @ dq[:, cols])
    assert e <= TOL_GEMM, e


# ---------------- M >= 256: 256x256 tiles with K splits ----------------

@pytest.mark.parametrize("M,K,N", [(300, 4096, 300), (257, 1024, 520), (512, 14336, 96), (257, 2048, 18)])
def test_gemm_big_tiles_ragged(M, K, N):
    """M >= 256 runs 256x256 tiles with enough K splits to fill the chip
    (8 / 2 / 8 splits here) over ragged row and column tiles, Q4S and Q8."""
    w = prng.randn((K, N), 61, std=0.02)
    a = prng.randn((M, K), 62)
    q = S.quantizeQ4(w)
    ref = a.astype(np.float64) @ O.dequant_q4s(dev_bytes(q), K, N).astype(np.float64)
    assert err(S.matmulQ4(S.tensor(a), q).data, ref) <= TOL_GEMM
    q8 = S.quantizeQ8(w)
    ref8 = a.astype(np.float64) @ O.dequant_q8(dev_bytes(q8), K, N).astype(np.float64)
    assert err(S.matmulQ8(S.tensor(a), q8).data, ref8) <= TOL_GEMM


@pytest.mark.parametrize("epi", [1, 2])
@pytest.mark.parametrize("K", [2048, 1024])
def test_gemm_big_tiles_epilogues(epi, K):
    """The K-split finish applies the residual / SwiGLU epilogue (Q8 linear
    with a fused RMSNorm, M = 300 rows on 256x256 tiles): 4 splits summed by
    smith_gemm_reduce (K = 2048) and 2 (K = 1024)."""
    M, N, eps = 300, 320, 1e-5
    w = prng.randn((K, N), 63, std=0.02)
    x = prng.randn((M, K), 64)
    g = 1 + prng.randn((K,), 65, std=0.1)
    r = prng.randn((M, N), 66)
    q8 = S.quantizeQ8(w)
    wd = O.dequant_q8(dev_bytes(q8), K, N).astype(np.float64)
    x64 = x.astype(np.float64)
    xn = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + eps) * g.astype(np.float64)
    y = xn @ wd
    if epi == 1:
        y = y + r
    else:
        gt, up = y[:, 0::2], y[:, 1::2]
        y = gt / (1 + np.exp(-gt)) * up
    ctx = device.ops_ctx()
    xb, gb, rb = S.tensor(x), S.tensor(g), S.tensor(r)
    out = S.create([M, N if epi == 1 else N // 2])
    device.check(device.lib.smith_linear_q8(ctx, xb.buffer, q8["buffer"], out.buffer, M, N, K, gb.buffer, eps,
                                            rb.buffer, epi))
    assert err(out.data, y) <= TOL_GEMM


def test_decode_shapes_random_sweep():
    """matmulQ4 / matmulQ8 against the float64 reference on seeded random
    shapes: M in 1..40 (every GEMV path and row bucket), K with and without
    K % 32 == 0, N not a multiple of 16."""
    rng = np.random.default_rng(91)
    for case in range(16):
        M = int(rng.integers(1, 41))
        K = int(rng.choice([32, 96, 100, 256, 320, 736, 1024, 1056]))
        N = int(rng.integers(1, 700))
        w = prng.randn((K, N), 900 + case, std=0.02)
        a = prng.randn((M, K), 950 + case)
        q4, q8 = S.quantizeQ4(w), S.quantizeQ8(w)
        for name, q, dq in (("q4", q4, O.dequant_q4s(dev_bytes(q4), K, N)),
                            ("q8", q8, O.dequant_q8(dev_bytes(q8), K, N))):
            y = (S.matmulQ4 if name == "q4" else S.matmulQ8)(S.tensor(a), q).data
            e = err(y, a.astype(np.float64) @ dq.astype(np.float64))
            assert e <= tol_for(M, K), (case, name, M, K, N, e)


def test_hilo_buckets_random_sweep():
    """The 3 <= M <= 8 buckets of the one-launch batched GEMV (hi/lo
    activations, the zero term's row sums formed during the conversion and
    read from LDS) on seeded random shapes that reach each block variant
    (whole-K 16-column blocks, 32-group K ranges over 16 or 64 columns,
    ragged N, K % 32 == 0), on Q4S records and GGUF Q4_0 tile planes, with
    activation rows of mixed magnitude and one all-zero row (its sums are
    zero).  Bars as for configs 1-3 (normwise 2e-5, elementwise 1e-3)."""
    rng = np.random.default_rng(2027)
    ctx = device.ops_ctx()
    for case in range(10):
        M = int(rng.integers(3, 9))
        K = int(rng.choice([32, 64, 96, 256, 1024, 4096]))
        N = int(rng.choice([int(rng.integers(17, 700)), int(rng.integers(2000, 2600)), int(rng.integers(5200, 6000))]))
        a = prng.randn((M, K), 3000 + case)
        a[1] *= 64.0  # a row far from the others' magnitude
        a[M - 1] = 0.0
        # Q4S records, ragged N
        w = prng.randn((K, N), 3100 + case, std=0.02)
        q = S.quantizeQ4(w)
        y = S.matmulQ4(S.tensor(a), q).data
        ref = a.astype(np.float64) @ O.dequant_q4s(dev_bytes(q), K, N).astype(np.float64)
        what = "hilo q4s case %d M=%d K=%d N=%d" % (case, M, K, N)
        assert err(y, ref) <= TOL_HILO, what
        assert elem(y, ref, what) <= ELEM_HILO, what
        assert not y[M - 1].any(), what
        # GGUF Q4_0 tile planes (the decode path's layout), N a multiple of 16
        N16 = max(16, N // 16 * 16)
        wq = prng.randn((N16, K), 3200 + case, std=0.02)  # GGUF listing [out, in]
        blocks = O.quantize_rows(O.GGML_Q4_0, wq)
        G = K // 32
        src, nib, dsc = device.alloc(blocks.size), device.alloc(N16 * G * 16), device.alloc(N16 * G * 2)
        device.upload(src, blocks)
        device.check(device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N16, K, 0, 1, N16))
        at = S.tensor(a)
        out = S.create([M, N16])
        device.check(device.lib.smith_linear_q4_0_t(ctx, at.buffer, nib, dsc, out.buffer, M, N16, K, None, 0.0,
                                                    None, 0))
        wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N16 * K).reshape(N16, K).astype(np.float64)
        ref = a.astype(np.float64) @ wd.T
        what = "hilo q4_0 tiles case %d M=%d K=%d N=%d" % (case, M, K, N16)
        assert err(out.data, ref) <= TOL_HILO, what
        assert elem(out.data, ref, what) <= ELEM_HILO, what
        for b in (src, nib, dsc):
            device.release_buffer(b)
