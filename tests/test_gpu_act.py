"""GPU parity of the tile-major Q4_0 layout and the single-row act path
(smith_repack_q4_0_t_into, smith_linear_q4_0_t, smith_linear_q4_0_t_act and
the act outputs of smith_embed / the GEMV epilogues) against float64
references built from the oracle's Q4_0 dequantization.

Bars: the repack is byte-exact; GEMV outputs are within normwise 2e-5 of the
float64 reference (hi/lo f16 activations keep ~22 bits, the same bar as the
f32-activation Q4_0 GEMV tests); a SwiGLU output silu(g)*u carries the
relative errors of both of its GEMV columns and silu's slope (<= 1.1), so
its bar is 3x that, 6e-5.  The LM head is f32 FMA throughout (bar 2e-6).
"""
import numpy as np
import pytest

from oracle import oracle as O
from smith_amd import device, prng

pytestmark = pytest.mark.gpu

TOL = 2e-5
TOL_F32 = 2e-6  # f32 FMA paths (no f16 operand)
TOL_SWIGLU = 6e-5
EPS = 1e-5


def _q4_0(N, K, seed):
    """GGUF [out=N, in=K] Q4_0 blocks, tile-major planes on the device, and
    the dequantized float64 weight [N, K]."""
    w = prng.randn((N, K), seed, std=0.02)
    blocks = O.quantize_rows(O.GGML_Q4_0, w)
    G = K // 32
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    nib = device.alloc(N * G * 16)
    dsc = device.alloc(N * G * 2)
    device.check(device.lib.smith_repack_q4_0_t_into(device.ops_ctx(), src, nib, dsc, N, K, 0, 1, N))
    device.sync()
    device.release_buffer(src)
    wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, N * K).reshape(N, K).astype(np.float64)
    return blocks, nib, dsc, wd


def _buf(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = device.alloc(a.nbytes)
    device.upload(b, a)
    return b


def _get(b, n):
    device.sync()
    return device.download(b, n * 4, np.float32).astype(np.float64)


def _act_bytes(K):
    return K * 4 + K // 8 * 12


def _act_of(x, gamma):
    """An act of vector x (times gamma) through the embedding's act output."""
    K = x.size
    E = _buf(x)
    tok = device.alloc(4)
    device.upload(tok, np.zeros(1, np.int32))
    out = device.alloc(K * 4)
    act = device.alloc(_act_bytes(K))
    g = _buf(gamma) if gamma is not None else None
    device.check(device.lib.smith_embed(device.ops_ctx(), E, tok, out, 1, K, act, g))
    return act


def _rms(x, g):
    return x / np.sqrt(np.mean(x * x) + EPS) * g


def _silu_mul(y):
    g, u = y[0::2], y[1::2]
    return g / (1 + np.exp(-g)) * u


def test_tiles_repack_layout_and_interleave():
    N, K = 48, 96
    G = K // 32
    w = prng.randn((N, K), 7, std=0.02)
    blocks = O.quantize_rows(O.GGML_Q4_0, w)
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    Nt = 2 * N  # two weights column-interleaved
    nib = device.alloc(Nt * G * 16)
    dsc = device.alloc(Nt * G * 2)
    ctx = device.ops_ctx()
    for j in range(2):
        device.check(device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N, K, j, 2, Nt))
    got_nib = device.download(nib, Nt * G * 16, np.uint8).reshape(Nt // 16, G, 16, 16)
    got_d = device.download(dsc, Nt * G * 2, np.uint8).reshape(Nt // 16, G, 16, 2)
    b = blocks.reshape(N, G, 18)
    for col in range(Nt):
        n = col // 2
        t, c = divmod(col, 16)
        assert np.array_equal(got_nib[t, :, c], b[n, :, 2:]), col
        assert np.array_equal(got_d[t, :, c], b[n, :, :2]), col
    # rejected shapes
    assert device.lib.smith_repack_q4_0_t_into(ctx, src, nib, dsc, N, K, 0, 1, 40) != 0


@pytest.mark.parametrize("M", [1, 2, 3, 17, 70, 200])
def test_linear_t_all_epilogues(M):
    N, K = 160, 320
    _, nib, dsc, wd = _q4_0(N, K, 11)
    x = prng.randn((M, K), 12)
    g = 1 + prng.randn((K,), 13, std=0.1)
    r = prng.randn((M, N), 14)
    ctx = device.ops_ctx()
    xb, gb, rb, ob = _buf(x), _buf(g), _buf(r), device.alloc(M * N * 4)
    xn = np.stack([_rms(x[m].astype(np.float64), g) for m in range(M)])
    for epi in (0, 1, 2):
        device.check(device.lib.smith_linear_q4_0_t(ctx, xb, nib, dsc, ob, M, N, K, gb, EPS, rb, epi))
        y = xn @ wd.T
        if epi == 1:
            y = y + r
        if epi == 2:
            y = np.stack([_silu_mul(y[m]) for m in range(M)])
        got = _get(ob, y.size).reshape(y.shape)
        tol = (TOL_SWIGLU if epi == 2 else TOL) if M <= 8 else (1e-3 if M < 64 else 1e-2)  # M >= 64: f16 MFMA GEMM
        assert O.normwise_rel_err(got, y) <= tol, (M, epi)


@pytest.mark.parametrize("N,K", [(2048, 1024), (6144, 512), (512, 1024), (2048, 8192)])
def test_linear_t_batched_decode_variants(N, K):
    """2 < M <= 32 on the one-launch kernel's variants (whole K in a
    workgroup: 2048 x 1024; 32-group K ranges over 16-column tiles: 512 x
    1024; over 64-column tiles: 6144 x 512 and the long K 2048 x 8192), every
    row bucket (hi/lo M <= 8, plain f16 M <= 16, two row blocks M <= 32) and
    every epilogue with the RMSNorm in front."""
    _, nib, dsc, wd = _q4_0(N, K, 21)
    ctx = device.ops_ctx()
    for M in (3, 6, 8, 12, 16, 20, 32):
        x = prng.randn((M, K), 22 + M)
        g = 1 + prng.randn((K,), 23, std=0.1)
        r = prng.randn((M, N), 24 + M)
        xb, gb, rb, ob = _buf(x), _buf(g), _buf(r), device.alloc(M * N * 4)
        xn = np.stack([_rms(x[m].astype(np.float64), g) for m in range(M)])
        for epi in (0, 1, 2):
            device.check(device.lib.smith_linear_q4_0_t(ctx, xb, nib, dsc, ob, M, N, K, gb, EPS, rb, epi))
            y = xn @ wd.T
            if epi == 1:
                y = y + r
            if epi == 2:
                y = np.stack([_silu_mul(y[m]) for m in range(M)])
            got = _get(ob, y.size).reshape(y.shape)
            tol = (TOL_SWIGLU if epi == 2 else TOL) if M <= 8 else 1e-3
            assert O.normwise_rel_err(got, y) <= tol, (M, N, K, epi)
        for b in (xb, gb, rb, ob):
            device.release_buffer(b)


@pytest.mark.parametrize("N,K", [(64, 256), (5120, 3072), (96, 9600), (48, 32 * 7)])
@pytest.mark.parametrize("norm", [0, 1])
def test_act_gemv_matches_reference(N, K, norm):
    _, nib, dsc, wd = _q4_0(N, K, 21 + N)
    x = prng.randn((K,), 22).astype(np.float64)
    g = 1 + prng.randn((K,), 23, std=0.1).astype(np.float64)
    act = _act_of(x, g if norm else None)
    out = device.alloc(N * 4)
    device.check(device.lib.smith_linear_q4_0_t_act(device.ops_ctx(), act, norm, EPS, nib, dsc, out, N, K, None, 0,
                                                    None, None))
    xn = _rms(x, g) if norm else x
    assert O.normwise_rel_err(_get(out, N), wd @ xn) <= TOL


def test_act_chain_residual_swiglu_down():
    """x -> [norm] q|k|v-like GEMV; o-proj with residual writing the act of
    x2 (next norm's gamma folded in) -> gate|up with SwiGLU writing h's act ->
    down with residual: every act output checked through its consumer."""
    D, F = 256, 512
    ctx = device.ops_ctx()
    _, nib_o, d_o, wo = _q4_0(D, D, 31)
    _, nib_gu, d_gu, wgu = _q4_0(2 * F, D, 32)
    _, nib_dn, d_dn, wdn = _q4_0(D, F, 33)
    a_in = prng.randn((D,), 34).astype(np.float64)
    x = prng.randn((D,), 35).astype(np.float64)
    g2 = 1 + prng.randn((D,), 36, std=0.1).astype(np.float64)
    act_a = _act_of(a_in, None)
    xb, g2b = _buf(x), _buf(g2)
    x2b = device.alloc(D * 4)
    act_x2 = device.alloc(_act_bytes(D))
    device.check(device.lib.smith_linear_q4_0_t_act(ctx, act_a, 0, 0.0, nib_o, d_o, x2b, D, D, xb, 1, act_x2, g2b))
    x2 = _get(x2b, D)
    assert O.normwise_rel_err(x2, x + wo @ a_in) <= TOL
    hb = device.alloc(F * 4)
    act_h = device.alloc(_act_bytes(F))
    device.check(device.lib.smith_linear_q4_0_t_act(ctx, act_x2, 1, EPS, nib_gu, d_gu, hb, 2 * F, D, None, 2,
                                                    act_h, None))
    h = _get(hb, F)
    assert O.normwise_rel_err(h, _silu_mul(wgu @ _rms(x2, g2))) <= TOL_SWIGLU
    outb = device.alloc(D * 4)
    device.check(device.lib.smith_linear_q4_0_t_act(ctx, act_h, 0, 0.0, nib_dn, d_dn, outb, D, F, x2b, 1, None,
                                                    None))
    assert O.normwise_rel_err(_get(outb, D), x2 + wdn @ h) <= TOL


def test_act_gemv_rejects_bad_shapes():
    ctx = device.ops_ctx()
    assert device.lib.smith_linear_q4_0_t_act(ctx, None, 0, 0.0, None, None, None, 64, 256, None, 0, None,
                                              None) != 0
    dummy = device.alloc(4096)
    assert device.lib.smith_linear_q4_0_t_act(ctx, dummy, 0, 0.0, dummy, dummy, dummy, 64, 100, None, 0, None,
                                              None) != 0
    assert device.lib.smith_linear_q4_0_t_act(ctx, dummy, 0, 0.0, dummy, dummy, dummy, 48, 256, None, 0, dummy,
                                              None) != 0


@pytest.mark.parametrize("K,N", [(200, 96), (3072, 32000), (8192, 320)])
def test_lmhead_planes_match_reference(K, N):
    """Q4_0 output.weight read as lmHead[K][N] (blocks along N): planes from
    smith_repack_lmhead_q4_0, y = rmsnorm(x) . lmHead, vs float64."""
    w = prng.randn((K, N), 61, std=0.02)
    blocks = O.quantize_rows(O.GGML_Q4_0, w)  # rows of N: blocks run along the vocab axis
    wd = O.dequantize_tensor(O.GGML_Q4_0, blocks, K * N).reshape(K, N).astype(np.float64)
    ctx = device.ops_ctx()
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    nib = device.alloc(K * N // 2)
    dsc = device.alloc(K * N // 16)
    device.check(device.lib.smith_repack_lmhead_q4_0(ctx, src, nib, dsc, K, N))
    x = prng.randn((K,), 62).astype(np.float64)
    g = 1 + prng.randn((K,), 63, std=0.1).astype(np.float64)
    xb, gb, yb = _buf(x), _buf(g), device.alloc(N * 4)
    device.check(device.lib.smith_lmhead_q4_0_nb(ctx, xb, gb, EPS, nib, dsc, yb, K, N))
    assert O.normwise_rel_err(_get(yb, N), _rms(x, g) @ wd) <= TOL_F32
    device.check(device.lib.smith_lmhead_q4_0_nb(ctx, xb, None, 0.0, nib, dsc, yb, K, N))
    assert O.normwise_rel_err(_get(yb, N), x @ wd) <= TOL_F32


def _greedy_state(ctx, dim, wq, wk, count, pos):
    st = {"x": device.alloc(dim * 4), "toks": device.alloc(64 * 4), "cnt": device.alloc(4), "pos": device.alloc(4),
          "act": device.alloc(_act_bytes(dim)), "rr": device.alloc((4 + wq + wk) * 4)}
    device.upload(st["toks"], np.full(64, -7, np.int32))
    # the act is written only when dim % 32 == 0; zeroed so both states
    # compare equal when it is not
    device.upload(st["act"], np.zeros(_act_bytes(dim), np.uint8))
    device.upload(st["cnt"], np.array([count], np.int32))
    device.upload(st["pos"], np.array([pos], np.int32))
    row = np.zeros(4 + wq + wk, np.float32)
    row[:1] = np.array([-1], np.int32).view(np.float32)  # no position yet; header pads stay zero
    device.upload(st["rr"], row)
    return st


def _greedy_read(st, dim, wq, wk, N, logits):
    device.sync()
    return {"toks": device.download(st["toks"], 64 * 4, np.int32), "cnt": device.download(st["cnt"], 4, np.int32),
            "pos": device.download(st["pos"], 4, np.int32), "x": device.download(st["x"], dim * 4, np.float32),
            "act": device.download(st["act"], _act_bytes(dim), np.uint8),
            "rr": device.download(st["rr"], (4 + wq + wk) * 4, np.uint8),
            "logits": device.download(logits, N * 4, np.float32)}


@pytest.mark.parametrize("K,N,case", [(1024, 32000, "ties"), (1024, 32000, "nan0"), (1024, 32000, "nan5"),
                                      (200, 96, "ties"), (3072, 4096, "plain")])
def test_lmhead_greedy_matches_two_step(K, N, case):
    """smith_lmhead_q4_0_greedy == smith_lmhead_q4_0_nb then
    smith_argmax_embed, bit for bit (logits, token, count, position, x, its
    act, rope row), on two calls in a row.  "ties": vocab blocks copied to
    a later block of the same 512-column tile and of another tile, with a
    dominant column, so equal maxima sit in three tiles and the first must
    win; "nan0": a NaN scale in block 0 (logits 0..31 NaN, the reference's
    scan returns 0); "nan5": NaNs in block 5 only (skipped)."""
    nh, hd = 4, 8
    wq, wk = nh * hd, 2 * hd
    w = prng.randn((K, N), 71, std=0.02)
    xs = [prng.randn((K,), 72), prng.randn((K,), 73)]
    if case == "ties":
        w[:, 32 * 1 + 5] = 0.06 * np.sign(xs[0])
        nb = N // 32
        for b in (2, nb - 1):
            w[:, 32 * b:32 * b + 32] = w[:, 32:64]
    blocks = O.quantize_rows(O.GGML_Q4_0, w)
    if case in ("nan0", "nan5"):
        b = 0 if case == "nan0" else 5
        view = blocks.reshape(K, N // 32, 18)
        view[K // 2, b, 0:2] = np.frombuffer(np.array([0x7E00], np.uint16).tobytes(), np.uint8)
    ctx = device.ops_ctx()
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    nib, dsc = device.alloc(K * N // 2), device.alloc(K * N // 16)
    device.check(device.lib.smith_repack_lmhead_q4_0(ctx, src, nib, dsc, K, N))
    E = device.alloc(N * K * 4)
    device.check(device.lib.smith_randn(ctx, E, N * K, 74, 0, 1.0, 0.0))
    g = _buf(1 + prng.randn((K,), 75, std=0.1))
    gout = _buf(1 + prng.randn((K,), 76, std=0.1))
    rope_len = 64 * hd // 2 * nh
    cos, sin = _buf(prng.randn((rope_len,), 77)), _buf(prng.randn((rope_len,), 78))
    xin = device.alloc(K * 4)
    la, lb = device.alloc(N * 4), device.alloc(N * 4)
    sa = _greedy_state(ctx, K, wq, wk, 3, 20)
    sb = _greedy_state(ctx, K, wq, wk, 3, 20)
    act = sa["act"] if K % 32 == 0 else None
    actb = sb["act"] if K % 32 == 0 else None
    for call, xv in enumerate(xs):
        device.upload(xin, xv.astype(np.float32))
        device.check(device.lib.smith_lmhead_q4_0_nb(ctx, xin, g, EPS, nib, dsc, la, K, N))
        device.check(device.lib.smith_argmax_embed(ctx, la, N, E, K, sa["x"], sa["toks"], sa["cnt"], sa["pos"], act,
                                                   gout, cos, sin, rope_len, wq, wk, sa["rr"]))
        device.check(device.lib.smith_lmhead_q4_0_greedy(ctx, xin, g, EPS, nib, dsc, lb, K, N, E, sb["x"],
                                                         sb["toks"], sb["cnt"], sb["pos"], actb, gout, cos, sin,
                                                         rope_len, wq, wk, sb["rr"]))
        ra, rb = _greedy_read(sa, K, wq, wk, N, la), _greedy_read(sb, K, wq, wk, N, lb)
        for k in ra:
            assert np.array_equal(ra[k].view(np.uint8), rb[k].view(np.uint8)), (call, k)
        lg = ra["logits"].astype(np.float64)
        tok = int(rb["toks"][3 + call])
        if case == "nan0":
            assert tok == 0
        else:
            finite = np.where(np.isnan(lg), -np.inf, lg)
            assert tok == int(np.argmax(finite)), (call, tok)
        if case == "ties" and call == 0:
            assert tok == 32 + 5 and lg[32 + 5] == lg[64 + 5] == lg[N - 32 + 5]
        assert rb["cnt"][0] == 4 + call and rb["pos"][0] == 21 + call
        Eh = device.download(E, K * 4, np.float32, offset=tok * K * 4)
        assert np.array_equal(rb["x"], Eh)


@pytest.mark.parametrize("K,N,case", [(1024, 32000, "ties"), (3072, 4096, "plain"), (256, 512, "ties")])
def test_lmhead_q6_k_greedy_matches_two_step(K, N, case):
    """smith_lmhead_q6_k_greedy == smith_lmhead_q6_k_nb then
    smith_argmax_embed, bit for bit (logits, token, count, position, x, its
    act, rope row), on two calls in a row.  "ties": 256-column Q6_K blocks
    copied into the same 512-column tile and into the last tile, with a
    dominant column, so equal maxima sit in two tiles and the first wins."""
    nh, hd = 4, 8
    wq, wk = nh * hd, 2 * hd
    w = prng.randn((K, N), 81, std=0.02)
    xs = [prng.randn((K,), 82), prng.randn((K,), 83)]
    if case == "ties":
        w[:, 5] = 0.06 * np.sign(xs[0])
        nb = N // 256
        for b in (1, nb - 1):
            w[:, 256 * b:256 * b + 256] = w[:, 0:256]
    blocks = O.quantize_rows(O.GGML_Q6_K, w)
    ctx = device.ops_ctx()
    src = device.alloc(blocks.size)
    device.upload(src, blocks)
    planes = device.alloc(int(device.lib.smith_lmhead_q6_k_bytes(K, N)))
    device.check(device.lib.smith_repack_lmhead_q6_k(ctx, src, planes, K, N))
    E = device.alloc(N * K * 4)
    device.check(device.lib.smith_randn(ctx, E, N * K, 84, 0, 1.0, 0.0))
    g = _buf(1 + prng.randn((K,), 85, std=0.1))
    gout = _buf(1 + prng.randn((K,), 86, std=0.1))
    rope_len = 64 * hd // 2 * nh
    cos, sin = _buf(prng.randn((rope_len,), 87)), _buf(prng.randn((rope_len,), 88))
    xin = device.alloc(K * 4)
    la, lb = device.alloc(N * 4), device.alloc(N * 4)
    sa = _greedy_state(ctx, K, wq, wk, 3, 20)
    sb = _greedy_state(ctx, K, wq, wk, 3, 20)
    for call, xv in enumerate(xs):
        device.upload(xin, xv.astype(np.float32))
        device.check(device.lib.smith_lmhead_q6_k_nb(ctx, xin, g, EPS, planes, la, K, N))
        device.check(device.lib.smith_argmax_embed(ctx, la, N, E, K, sa["x"], sa["toks"], sa["cnt"], sa["pos"],
                                                   sa["act"], gout, cos, sin, rope_len, wq, wk, sa["rr"]))
        device.check(device.lib.smith_lmhead_q6_k_greedy(ctx, xin, g, EPS, planes, lb, K, N, E, sb["x"], sb["toks"],
                                                         sb["cnt"], sb["pos"], sb["act"], gout, cos, sin, rope_len,
                                                         wq, wk, sb["rr"]))
        ra, rb = _greedy_read(sa, K, wq, wk, N, la), _greedy_read(sb, K, wq, wk, N, lb)
        for k in ra:
            assert np.array_equal(ra[k].view(np.uint8), rb[k].view(np.uint8)), (call, k)
        lg = ra["logits"].astype(np.float64)
        tok = int(rb["toks"][3 + call])
        assert tok == int(np.argmax(lg)), (call, tok)
        if case == "ties" and call == 0:
            assert tok == 5 and lg[5] == lg[256 + 5] == lg[N - 256 + 5]
        assert rb["cnt"][0] == 4 + call and rb["pos"][0] == 21 + call
    assert device.lib.smith_lmhead_q6_k_greedy(ctx, xin, g, EPS, planes, lb, K, N, None, sb["x"], sb["toks"],
                                               sb["cnt"], sb["pos"], None, None, None, None, 0, 0, 0, None) != 0
