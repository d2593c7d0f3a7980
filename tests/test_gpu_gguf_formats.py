"""GPU parity of the other GGUF block types (Q4_1, Q5_0, Q4_K, Q6_K; Q4_0
and Q8_0 alongside where the entry point takes them):

  * smith_dequantize_gguf vs the oracle's dequantizeTensor: bit-exact, also
    on random block bytes (finite f16 fields) and a ragged element count;
  * smith_repack_gguf_tiles_into: the planes decoded on the host by the
    documented layout (nib / permuted high bits / prm / sup in 16-column
    tiles) reproduce the oracle's f32 weights exactly, for side-by-side and
    interleaved placement;
  * smith_linear_gguf_tiles_act / _attn (exact weights): normwise 5e-5 of
    the float64 product with the oracle's weights (SwiGLU 1.5e-4).  The
    exponent-bias operand (f16 1024 + q) makes each group's f32 MFMA sum
    about 1024 * sum|a| before the offset is taken off, so a group carries
    ~2^-24 * 1024 * sum|a| of rounding: normwise ~1e-5 .. 2.5e-5 at
    K = 3072 (Q4_0 seeds included), hence 5e-5;
  * smith_linear_gguf_tiles (MFMA GEMM, f16 weights and activations):
    normwise 1e-2, the GEMM bar of the Q4_0 tests;
  * loadGGUF(...).generate on a tiny model with the Q4_K_M mix (Q4_K
    q/k/o/gate/up, Q6_K v/down, Q6_K output.weight, Q4_K token_embd) and on
    Q4_1 / Q5_0 / Q6_K models, against the Llama oracle (as test_gpu_llama).
"""
import numpy as np
import pytest

from oracle import llama_oracle as LO
from oracle import oracle as O
from oracle.oracle import normwise_rel_err
from smith_amd import device, prng
from tests.llama_fixtures import write_tiny_llama

pytestmark = pytest.mark.gpu

TOL = 5e-5
TOL_SWIGLU = 1.5e-4
TOL_GEMM = 1e-2
EPS = 1e-5
KQ = [O.GGML_Q4_1, O.GGML_Q5_0, O.GGML_Q4_K, O.GGML_Q6_K]
ALL_TILE = [O.GGML_Q4_0] + KQ


def _buf(a):
    a = np.ascontiguousarray(a)
    b = device.alloc(max(a.nbytes, 4))
    device.upload(b, a)
    return b


def _get(b, n, dt=np.float32):
    device.sync()
    return device.download(b, n * np.dtype(dt).itemsize, dt)


def _rms(x, g):
    return x / np.sqrt(np.mean(x * x) + EPS) * g


def _silu_mul(y):
    g, u = y[0::2], y[1::2]
    return g / (1 + np.exp(-g)) * u


def _weights(t, N, K, seed):
    w = prng.randn((N, K), seed, std=0.02)
    blocks = O.quantize_rows(t, w)
    wd = O.dequantize_tensor(t, blocks, N * K).reshape(N, K)
    return blocks, wd


def _planes(t, blocks, N, K, parts=None):
    nbytes = int(device.lib.smith_gguf_tiles_bytes(t, N, K))
    assert nbytes
    pl = device.alloc(nbytes)
    ctx = device.ops_ctx()
    for (b, n, off, stride) in parts or [(blocks, N, 0, 1)]:
        src = _buf(b)
        device.check(device.lib.smith_repack_gguf_tiles_into(ctx, t, src, pl, n, K, off, stride, N))
        device.sync()
        device.release_buffer(src)
    return pl, nbytes


# ---------------- dequantizeTensor ----------------

@pytest.mark.parametrize("t", [O.GGML_F16, O.GGML_BF16, O.GGML_Q4_0, O.GGML_Q8_0] + KQ)
def test_dequantize_bit_exact(t):
    be, bb = O.BLOCK[t]
    ctx = device.ops_ctx()
    rng = np.random.default_rng(t)
    if be == 1:
        raw = rng.integers(0, 1 << 16, 4099, dtype=np.uint16)
        if t == O.GGML_F16:
            raw[(raw & 0x7C00) == 0x7C00] &= 0xBFFF  # finite halves
        raw = raw.view(np.uint8)
        numel = 4099
    else:
        enc = O.quantize_rows(t, prng.randn((6, 4 * be), 90 + t, std=0.05))
        rnd = rng.integers(0, 256, 40 * bb, dtype=np.uint8).reshape(40, bb)
        # finite f16 fields in the random blocks
        f16_at = {O.GGML_Q4_0: [0], O.GGML_Q8_0: [0], O.GGML_Q4_1: [0, 2], O.GGML_Q5_0: [0],
                  O.GGML_Q4_K: [0, 2], O.GGML_Q6_K: [208]}[t]
        for o in f16_at:
            rnd[:, o + 1] &= 0x3B  # exponent < 31, magnitude < 1
        raw = np.concatenate([enc, rnd.ravel()])
        numel = (raw.size // bb) * be - 5  # ragged tail
    src, dst = _buf(raw), device.alloc(numel * 4)
    device.check(device.lib.smith_dequantize_gguf(ctx, t, src, dst, numel))
    got = _get(dst, numel)
    want = O.dequantize_tensor(t, raw, numel)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------- tile planes ----------------

def _decode_planes(t, data, N, K):
    """Host decoder of the tile planes (layout of gguf_tiles.h) -> [N, K]."""
    G = K // 32
    R = N * G
    al = lambda x: (x + 255) & ~255
    hbB = {O.GGML_Q5_0: 4, O.GGML_Q6_K: 8}.get(t, 0)
    pB = 4 if t == O.GGML_Q4_1 else 2
    supB = {O.GGML_Q4_K: 4, O.GGML_Q6_K: 2}.get(t, 0)
    o_hb = al(R * 16)
    o_p = al(o_hb + R * hbB)
    o_s = al(o_p + R * pB)
    h16 = lambda u: float(np.array([u & 0xFFFF], np.uint16).view(np.float16)[0])
    out = np.zeros((N, K), np.float64)
    for n in range(N):
        for g in range(G):
            rec = ((n // 16) * G + g) * 16 + n % 16
            nb = data[rec * 16:rec * 16 + 16]
            q = np.array([(nb[e // 2] >> (4 * (e % 2))) & 15 for e in range(32)], np.int64)
            if hbB:
                words = data[o_hb + rec * hbB:o_hb + rec * hbB + hbB].view(np.uint32)
                for e in range(32):
                    i, k = e >> 3, e & 7
                    if t == O.GGML_Q5_0:
                        q[e] |= ((int(words[0]) >> (4 * i + (k & 3) + 16 * (k >> 2))) & 1) << 4
                    else:
                        pos = 2 * (4 * (i & 1) + (k & 3)) + 16 * (k >> 2)
                        q[e] |= ((int(words[i >> 1]) >> pos) & 3) << 4
            p = int(data[o_p + rec * pB:o_p + rec * pB + pB].view(np.uint32 if pB == 4 else np.uint16)[0])
            srec = ((n // 16) * (G // 8) + g // 8) * 16 + n % 16
            sp = int(data[o_s + srec * supB:o_s + srec * supB + supB].view(np.uint32 if supB == 4 else np.uint16)[0]) \
                if supB else 0
            if t == O.GGML_Q4_0:
                v = h16(p) * (q - 8)
            elif t == O.GGML_Q5_0:
                v = h16(p) * (q - 16)
            elif t == O.GGML_Q4_1:
                v = h16(p) * q + h16(p >> 16)
            elif t == O.GGML_Q4_K:
                v = np.float32(h16(sp) * (p & 63)) * q - np.float32(h16(sp >> 16) * ((p >> 8) & 63))
            else:
                sc = np.array([p & 0xFF, (p >> 8) & 0xFF], np.uint8).view(np.int8).astype(np.float64)
                v = h16(sp) * np.repeat(sc, 16) * (q - 32)
            out[n, 32 * g:32 * g + 32] = v
    return out.astype(np.float32)


@pytest.mark.parametrize("t", ALL_TILE)
def test_repack_planes_decode_to_oracle_weights(t):
    K = 512
    b1, w1 = _weights(t, 32, K, 11 + t)
    b2, w2 = _weights(t, 16, K, 12 + t)
    pl, nb = _planes(t, None, 48, K, parts=[(b1, 32, 0, 1), (b2, 16, 32, 1)])
    got = _decode_planes(t, _get(pl, nb, np.uint8), 48, K)
    assert np.array_equal(got, np.concatenate([w1, w2]))
    # interleaved (gate/up) placement
    pl, nb = _planes(t, None, 64, K, parts=[(b1, 32, 0, 2), (b1, 32, 1, 2)])
    got = _decode_planes(t, _get(pl, nb, np.uint8), 64, K)
    assert np.array_equal(got[0::2], w1) and np.array_equal(got[1::2], w1)


def test_tiles_rejects_bad_shapes():
    assert device.lib.smith_gguf_tiles_bytes(O.GGML_Q4_K, 64, 288) == 0  # K % 256
    assert device.lib.smith_gguf_tiles_bytes(O.GGML_Q5_0, 40, 288) == 0  # N % 16
    assert device.lib.smith_gguf_tiles_bytes(O.GGML_Q8_0, 64, 256) == 0  # no tile layout
    assert device.lib.smith_gguf_tiles_bytes(O.GGML_Q5_0, 64, 288) > 0
    ctx = device.ops_ctx()
    d = device.alloc(4096)
    assert device.lib.smith_linear_gguf_tiles_act(ctx, O.GGML_Q6_K, d, 0, 0.0, d, d, 64, 288, None, 0, None,
                                                  None) != 0


# ---------------- act GEMV (exact weights) ----------------

def _act_of(x, gamma):
    K = x.size
    E = _buf(np.asarray(x, np.float32))
    tok = _buf(np.zeros(1, np.int32))
    out = device.alloc(K * 4)
    act = device.alloc(K * 4 + K // 8 * 12)
    g = _buf(np.asarray(gamma, np.float32)) if gamma is not None else None
    device.check(device.lib.smith_embed(device.ops_ctx(), E, tok, out, 1, K, act, g))
    return act


@pytest.mark.parametrize("t", ALL_TILE)
@pytest.mark.parametrize("N,K", [(64, 256), (3072, 3072), (96, 9216), (48, 768)])
def test_act_gemv_all_types(t, N, K):
    blocks, wd = _weights(t, N, K, 21 + N + t)
    pl, _ = _planes(t, blocks, N, K)
    x = prng.randn((K,), 22).astype(np.float64)
    g = 1 + prng.randn((K,), 23, std=0.1).astype(np.float64)
    out = device.alloc(N * 4)
    ctx = device.ops_ctx()
    for norm in (0, 1):
        act = _act_of(x, g if norm else None)
        device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act, norm, EPS, pl, out, N, K, None, 0, None,
                                                            None))
        xn = _rms(x, g) if norm else x
        assert normwise_rel_err(_get(out, N), wd.astype(np.float64) @ xn) <= TOL, norm


@pytest.mark.parametrize("t", KQ)
def test_act_gemv_epilogues_and_act_output(t):
    """residual + act output -> SwiGLU -> residual chain on one type."""
    D, F = 256, 512
    ctx = device.ops_ctx()
    b_o, wo = _weights(t, D, D, 31)
    b_gu, wgu = _weights(t, 2 * F, D, 32)
    b_dn, wdn = _weights(t, D, F, 33)
    p_o, _ = _planes(t, b_o, D, D)
    p_gu, _ = _planes(t, b_gu, 2 * F, D)
    p_dn, _ = _planes(t, b_dn, D, F)
    wo, wgu, wdn = (w.astype(np.float64) for w in (wo, wgu, wdn))
    a_in = prng.randn((D,), 34).astype(np.float64)
    x = prng.randn((D,), 35).astype(np.float64)
    g2 = 1 + prng.randn((D,), 36, std=0.1).astype(np.float64)
    act_a = _act_of(a_in, None)
    xb, g2b = _buf(x.astype(np.float32)), _buf(g2.astype(np.float32))
    x2b, act_x2 = device.alloc(D * 4), device.alloc(D * 4 + D // 8 * 12)
    device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act_a, 0, 0.0, p_o, x2b, D, D, xb, 1, act_x2, g2b))
    x2 = _get(x2b, D).astype(np.float64)
    assert normwise_rel_err(x2, x + wo @ a_in) <= TOL
    hb, act_h = device.alloc(F * 4), device.alloc(F * 4 + F // 8 * 12)
    device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act_x2, 1, EPS, p_gu, hb, 2 * F, D, None, 2, act_h,
                                                        None))
    h = _get(hb, F).astype(np.float64)
    assert normwise_rel_err(h, _silu_mul(wgu @ _rms(x2, g2))) <= TOL_SWIGLU
    outb = device.alloc(D * 4)
    device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act_h, 0, 0.0, p_dn, outb, D, F, x2b, 1, None, None))
    assert normwise_rel_err(_get(outb, D), x2 + wdn @ h) <= TOL


# ---------------- M-row linear (GEMM) ----------------

@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("M", [1, 5, 70, 200])
def test_linear_gemm_all_epilogues(t, M):
    N, K = 160, 512
    blocks, wd = _weights(t, N, K, 41 + t)
    pl, _ = _planes(t, blocks, N, K)
    x = prng.randn((M, K), 42)
    g = 1 + prng.randn((K,), 43, std=0.1)
    r = prng.randn((M, N), 44)
    ctx = device.ops_ctx()
    xb, gb, rb, ob = _buf(x), _buf(g), _buf(r), device.alloc(M * N * 4)
    xn = np.stack([_rms(x[m].astype(np.float64), g) for m in range(M)])
    for epi in (0, 1, 2):
        device.check(device.lib.smith_linear_gguf_tiles(ctx, t, xb, pl, ob, M, N, K, gb, EPS, rb, epi))
        y = xn @ wd.astype(np.float64).T
        if epi == 1:
            y = y + r
        if epi == 2:
            y = np.stack([_silu_mul(y[m]) for m in range(M)])
        got = _get(ob, y.size).reshape(y.shape)
        assert normwise_rel_err(got, y) <= TOL_GEMM, (M, epi)


# ---------------- end to end ----------------

SMALL = dict(dim=256, layers=2, heads=4, kv_heads=2, ffn=512, vocab=320, context=2048)
Q4_K_M = dict(linear_type="q4_k", types={"attn_v": "q6_k", "ffn_down": "q6_k"}, embd_type="q4_k", head_type="q6_k")


def check_tokens(gpu_tokens, ref_logits):
    for i, (tk, lg) in enumerate(zip(gpu_tokens, ref_logits)):
        top2 = np.sort(lg)[-2:]
        if tk != int(np.argmax(lg)):
            assert top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])), (i, tk, int(np.argmax(lg)))


@pytest.mark.parametrize("kw", [Q4_K_M, dict(linear_type="q4_1"), dict(linear_type="q5_0", head_type="q8_0"),
                                dict(linear_type="q5_0", dim=288, heads=6, kv_heads=3, ffn=768),  # head_dim 48
                                dict(linear_type="q6_k", tie=True),
                                dict(types={"attn_v": "q6_k", "ffn_down": "q6_k"})])  # Q4_0 + Q6_K pair
def test_generate_mixed_formats(tmp_path_factory, kw):
    from smith_amd.gguf_loader import loadGGUF
    p = str(tmp_path_factory.mktemp("ggufk") / "m.gguf")
    write_tiny_llama(p, **dict(SMALL, **kw))
    m = loadGGUF(p)
    ref = LO.LlamaOracle(p)
    prompt = [3, 77, 150, 9, 210]
    caches = m.createCache()
    assert normwise_rel_err(m.forwardPrefill(prompt, caches)["logits"], ref.forward(prompt, 0)) <= 1e-2
    out = m.generate(prompt, {"maxTokens": 8, "temperature": 0})
    gen = out[len(prompt):]
    ref.reset()
    _, logits = ref.generate_greedy(prompt, 8, teacher=gen)
    check_tokens(gen, logits)
    caches = m.createCache()
    m.forwardPrefill(prompt, caches)
    ref.reset()
    ref.forward(prompt, 0)
    for i, tk in enumerate([5, 250, 17]):
        g = m.forwardDecode(tk, len(prompt) + i, caches)["logits"]
        w = ref.forward([tk], len(prompt) + i)
        # the path's 1e-2: these steps read K/V written by the f16-MFMA prefill
        # (f16 weights, and on Q4_K / Q6_K an f16-rounded scale): ~1e-3 observed
        assert normwise_rel_err(g, w) <= 1e-2, i


@pytest.mark.parametrize("t1,t2", [(O.GGML_Q4_K, O.GGML_Q6_K), (O.GGML_Q4_K, O.GGML_Q5_0), (O.GGML_Q5_0, O.GGML_Q6_K),
                                   (O.GGML_Q4_0, O.GGML_Q6_K), (O.GGML_Q4_K, O.GGML_Q4_0)])
@pytest.mark.parametrize("K", [256, 3072, 9216])
def test_pair_act_gemv(t1, t2, K):
    """Two block types in one launch (q|k of one type, v of another)."""
    N1, N2 = 80, 48
    b1, w1 = _weights(t1, N1, K, 51)
    b2, w2 = _weights(t2, N2, K, 52)
    p1, _ = _planes(t1, b1, N1, K)
    p2, _ = _planes(t2, b2, N2, K)
    assert device.lib.smith_gguf_tiles_pair_ok(t1, t2) == 1
    x = prng.randn((K,), 53).astype(np.float64)
    g = 1 + prng.randn((K,), 54, std=0.1).astype(np.float64)
    act = _act_of(x, g)
    out = device.alloc((N1 + N2) * 4)
    device.check(device.lib.smith_linear_gguf_tiles_pair_act(device.ops_ctx(), t1, p1, N1, t2, p2, N2, act, 1, EPS,
                                                             out, K))
    want = np.concatenate([w1, w2]).astype(np.float64) @ _rms(x, g)
    assert normwise_rel_err(_get(out, N1 + N2), want) <= TOL
    assert device.lib.smith_gguf_tiles_pair_ok(O.GGML_Q6_K, O.GGML_Q4_1) == 0


@pytest.mark.parametrize("K,N", [(256, 256), (3072, 32000), (8192, 512), (48, 768)])
def test_lmhead_q6_k_matches_reference(K, N):
    """Q6_K output.weight read as lmHead[K][N] (256-element blocks along N):
    planes from smith_repack_lmhead_q6_k, y = rmsnorm(x) . lmHead vs float64
    of the oracle's weights (f32 FMA throughout: 2e-6)."""
    w = prng.randn((K, N), 81, std=0.02)
    blocks = O.quantize_rows(O.GGML_Q6_K, w)  # rows of N: blocks run along the vocab axis
    wd = O.dequantize_tensor(O.GGML_Q6_K, blocks, K * N).reshape(K, N).astype(np.float64)
    ctx = device.ops_ctx()
    src = _buf(blocks)
    planes = device.alloc(int(device.lib.smith_lmhead_q6_k_bytes(K, N)))
    device.check(device.lib.smith_repack_lmhead_q6_k(ctx, src, planes, K, N))
    x = prng.randn((K,), 82).astype(np.float64)
    g = 1 + prng.randn((K,), 83, std=0.1).astype(np.float64)
    xb, gb, yb = _buf(x.astype(np.float32)), _buf(g.astype(np.float32)), device.alloc(N * 4)
    device.check(device.lib.smith_lmhead_q6_k_nb(ctx, xb, gb, EPS, planes, yb, K, N))
    assert normwise_rel_err(_get(yb, N), _rms(x, g) @ wd) <= 2e-6
    device.check(device.lib.smith_lmhead_q6_k_nb(ctx, xb, None, 0.0, planes, yb, K, N))
    assert normwise_rel_err(_get(yb, N), x @ wd) <= 2e-6
    assert device.lib.smith_lmhead_q6_k_nb(ctx, xb, None, 0.0, planes, yb, 40, N) != 0  # K % 16


@pytest.mark.parametrize("t", [O.GGML_Q4_0, O.GGML_Q4_K])
def test_prep_next_chain_matches_unhinted(t):
    """smith_prep_next on a prompt-shaped chain (M = 128 rows on the MFMA
    GEMM, every GEMM split over K): o-proj (+ residual) -> gate|up (RMSNorm,
    SwiGLU) -> down (+ residual) -> next q|k|v (RMSNorm), hinted so each
    reduce also writes the next GEMM's operand.  Same outputs as the chain
    without hints (the first GEMM bit for bit, the others within 2e-4
    normwise: the fused RMSNorm sums its squares in another order, which can
    move an f16 operand by one unit in the last place), one prep
    launch instead of four, and the oracle's chain within the GEMM bar."""
    M, D, F = 128, 1024, 1536
    ctx = device.ops_ctx()
    x0 = prng.randn((M, D), 81)
    res = prng.randn((M, D), 82)
    g2 = 1 + prng.randn((D,), 83, std=0.1)
    g1 = 1 + prng.randn((D,), 84, std=0.1)
    ws = [_weights(t, n, k, s) for (n, k, s) in ((D, D, 85), (2 * F, D, 86), (D, F, 87), (D, D, 88))]
    pls = [_planes(t, b, n, k)[0] for (b, _), (n, k) in zip(ws, ((D, D), (2 * F, D), (D, F), (D, D)))]
    xb, rb, g2b, g1b = _buf(x0), _buf(res), _buf(g2), _buf(g1)

    def chain(hint):
        y1, y2, y3, y4 = device.alloc(M * D * 4), device.alloc(M * F * 4), device.alloc(M * D * 4), device.alloc(M * D * 4)
        steps = [(pls[0], xb, y1, D, D, None, 0.0, rb, 1, (g2b, EPS)),
                 (pls[1], y1, y2, 2 * F, D, g2b, EPS, None, 2, (None, 0.0)),
                 (pls[2], y2, y3, D, F, None, 0.0, y1, 1, (g1b, EPS)),
                 (pls[3], y3, y4, D, D, g1b, EPS, None, 0, None)]
        device.profile_kernels(True)
        for pl, a, o, n, k, g, e, r, epi, nxt in steps:
            if hint and nxt is not None:
                device.check(device.lib.smith_prep_next(ctx, nxt[0], nxt[1]))
            device.check(device.lib.smith_linear_gguf_tiles(ctx, t, a, pl, o, M, n, k, g, e, r, epi))
        _, preps = device.profile_read("smith_gemm_prep_a")
        device.profile_read("")
        device.profile_kernels(False)
        outs = [_get(b, M * d).reshape(M, d) for b, d in ((y1, D), (y2, F), (y3, D), (y4, D))]
        for b in (y1, y2, y3, y4):
            device.release_buffer(b)
        return outs, preps

    plain, p0 = chain(False)
    fused, p1 = chain(True)
    assert (p0, p1) == (4, 1)
    assert np.array_equal(plain[0], fused[0])
    for a, b in zip(plain[1:], fused[1:]):
        assert normwise_rel_err(b, a) <= 2e-4
    wd = [w for _, w in ws]
    r1 = x0.astype(np.float64) @ wd[0].T.astype(np.float64) + res
    h = np.stack([_silu_mul(row) for row in (np.stack([_rms(r, g2) for r in r1]) @ wd[1].T)])
    r3 = h @ wd[2].T + r1
    r4 = np.stack([_rms(r, g1) for r in r3]) @ wd[3].T
    for got, ref in zip(fused, (r1, h, r3, r4)):
        assert normwise_rel_err(got, ref) <= 1e-2


@pytest.mark.parametrize("between", ["act_gemv", "fill_zero", "copy"])
def test_prep_next_hint_dropped_by_other_calls(between):
    """A smith_prep_next hint followed by any other launch or copy is gone by
    the time the next K-split GEMM runs: that GEMM ends in the plain reduce
    (no smith_gemm_reduce_prep reading the hinted gamma), and its output
    equals the unhinted call's bit for bit."""
    t = O.GGML_Q4_0
    M, D = 128, 1024
    ctx = device.ops_ctx()
    blocks, _ = _weights(t, D, D, 91)
    pl = _planes(t, blocks, D, D)[0]
    xb, rb = _buf(prng.randn((M, D), 92)), _buf(prng.randn((M, D), 93))
    gb = _buf(1 + prng.randn((D,), 94, std=0.1))
    scratch = device.alloc(4096)

    def run(hint):
        y = device.alloc(M * D * 4)
        if hint:
            device.check(device.lib.smith_prep_next(ctx, gb, EPS))
            if between == "fill_zero":
                device.check(device.lib.smith_fill_zero(ctx, scratch, 4096))
            elif between == "copy":
                device.check(device.lib.smith_copy_d2d(ctx, scratch, 0, xb, 0, 4096))
            else:  # a decode act GEMV (row 0 of x through the embedding's act output)
                tok, row = _buf(np.zeros(1, np.int32)), device.alloc(D * 4)
                act = device.alloc(D * 4 + D // 8 * 12)
                device.check(device.lib.smith_embed(ctx, xb, tok, row, 1, D, act, None))
                device.check(device.lib.smith_prep_next(ctx, gb, EPS))  # the embed dropped the first hint
                device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act, 0, 0.0, pl, row, D, D,
                                                                     None, 0, None, None))
        device.profile_kernels(True)
        device.check(device.lib.smith_linear_gguf_tiles(ctx, t, xb, pl, y, M, D, D, None, 0.0, rb, 1))
        _, n_fused = device.profile_read("smith_gemm_reduce_prep")
        _, n_plain = device.profile_read("smith_gemm_reduce")
        device.profile_read("")
        device.profile_kernels(False)
        out = _get(y, M * D)
        device.release_buffer(y)
        return out, n_fused, n_plain

    want, f0, p0 = run(False)
    got, f1, p1 = run(True)
    assert (f0, p0) == (0, 1) and (f1, p1) == (0, 1), (f0, p0, f1, p1)
    assert np.array_equal(got, want)


def test_q4_k_gate_up_two_tiles_per_wave_at_config5_width():
    """The Q4_K gate|up act GEMV at the config-5 width (N = 2 x 9216
    interleaved gate/up columns = 1152 column tiles, K = 3072) runs two
    column tiles per wave (the _c2 variant); with the RMSNorm scale, the
    SwiGLU epilogue and the act of h emitted for the down projection, which
    then consumes that act: both outputs against the float64 products of
    the oracle's weights."""
    t = O.GGML_Q4_K
    D, F = 3072, 9216
    ctx = device.ops_ctx()
    b_gu, wgu = _weights(t, 2 * F, D, 41)
    b_dn, wdn = _weights(t, D, F, 42)
    p_gu, _ = _planes(t, b_gu, 2 * F, D)
    p_dn, _ = _planes(t, b_dn, D, F)
    wgu, wdn = wgu.astype(np.float64), wdn.astype(np.float64)
    x = prng.randn((D,), 43).astype(np.float64)
    g = 1 + prng.randn((D,), 44, std=0.1).astype(np.float64)
    act_x = _act_of(x, g)
    hb, act_h = device.alloc(F * 4), device.alloc(F * 4 + F // 8 * 12)
    device.profile_kernels(True)
    device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act_x, 1, EPS, p_gu, hb, 2 * F, D, None, 2, act_h,
                                                        None))
    _, n_c2 = device.profile_read("smith_agemv_q4kt_k96_c2")
    device.profile_read("")
    device.profile_kernels(False)
    assert n_c2 == 1
    h = _get(hb, F).astype(np.float64)
    assert normwise_rel_err(h, _silu_mul(wgu @ _rms(x, g))) <= TOL_SWIGLU
    outb = device.alloc(D * 4)
    device.check(device.lib.smith_linear_gguf_tiles_act(ctx, t, act_h, 0, 0.0, p_dn, outb, D, F, None, 0, None, None))
    assert normwise_rel_err(_get(outb, D), wdn @ h) <= TOL
    for b in (p_gu, p_dn, hb, act_h, outb):
        device.release_buffer(b)
