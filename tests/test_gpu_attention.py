"""GPU parity of smith_attention for prompt rows (S > 1: KV append + the
f32-MFMA flash attention) and single rows (S == 1), against a float64
reference built from the Llama oracle's RoPE (whole-row indexing,
oracle/llama_oracle.py rope_rows) and its causal GQA softmax attention
(attend; gguf_cache.js:128-157, 212-231).  Keys before p0 come from caches filled
with random rows, so chunked prefill is covered.

Bar: normwise 1e-5 (f32 products and sums throughout; softmax exponentials
in f32), and the caches' new rows bit-exact to the kernels' own RoPE rows
within 1e-6.
"""
import numpy as np
import pytest

from oracle import llama_oracle as LO
from oracle.oracle import normwise_rel_err
from smith_amd import device, prng

pytestmark = pytest.mark.gpu


def _ref(q_all, k_new, v_new, kc, vc, p0, nH, nKV, hd, cos, sin):
    S = q_all.shape[0]
    Wq, Wk = nH * hd, nKV * hd
    q = LO.rope_rows(q_all, p0, cos, sin)            # [S, Wq]
    k = LO.rope_rows(k_new, p0, cos, sin)            # [S, Wk]
    K = kc.copy()
    V = vc.copy()
    for s in range(S):
        K[:, p0 + s, :] = k[s].reshape(nKV, hd)
        V[:, p0 + s, :] = v_new[s].reshape(nKV, hd)
    out = np.zeros((S, Wq))
    rep = nH // nKV
    for s in range(S):
        T = p0 + s + 1
        for h in range(nH):
            kv = h // rep  # the oracle's pinned attention (two-key closed form in test_llama_oracle)
            out[s, h * hd:(h + 1) * hd] = LO.attend(q[s, h * hd:(h + 1) * hd], K[kv, :T], V[kv, :T], 1 / np.sqrt(hd))
    return out, K, V


@pytest.mark.parametrize("S,p0,nH,nKV,hd", [(128, 0, 4, 2, 128), (70, 200, 4, 2, 128), (200, 0, 4, 4, 64),
                                           (33, 5, 6, 3, 48), (1, 77, 4, 2, 128), (256, 300, 8, 2, 64)])
def test_attention_matches_reference(S, p0, nH, nKV, hd):
    maxSeq = 8192
    Wq, Wk = nH * hd, nKV * hd
    ld = Wq + 2 * Wk
    cos, sin = LO.precompute_rope(hd, maxSeq, 10000.0)
    assert (p0 + S) * Wq // 2 <= maxSeq * hd // 2  # whole-row RoPE stays inside the table
    qkv = prng.randn((S, ld), 7 + S)
    kc = np.zeros((nKV, maxSeq, hd), np.float32)
    vc = np.zeros((nKV, maxSeq, hd), np.float32)
    kc[:, :p0] = prng.randn((nKV, p0, hd), 8)
    vc[:, :p0] = prng.randn((nKV, p0, hd), 9)
    ctx = device.ops_ctx()
    b = {}
    for name, a in (("qkv", qkv), ("cos", cos.astype(np.float32)), ("sin", sin.astype(np.float32)), ("kc", kc),
                    ("vc", vc)):
        a = np.ascontiguousarray(a, np.float32)
        b[name] = device.alloc(a.nbytes)
        device.upload(b[name], a)
    pos = device.alloc(4)
    device.upload(pos, np.array([p0], np.int32))
    out = device.alloc(S * Wq * 4)
    device.check(device.lib.smith_attention(ctx, b["qkv"], ld, pos, S, nH, nKV, hd, b["cos"], b["sin"], cos.size,
                                            b["kc"], b["vc"], maxSeq, out, None))
    device.sync()
    got = device.download(out, S * Wq * 4, np.float32).reshape(S, Wq)
    q64 = qkv.astype(np.float64)
    want, K, V = _ref(q64[:, :Wq], q64[:, Wq:Wq + Wk], q64[:, Wq + Wk:], kc.astype(np.float64),
                      vc.astype(np.float64), p0, nH, nKV, hd, cos, sin)
    assert normwise_rel_err(got, want) <= 1e-5
    gk = device.download(b["kc"], kc.nbytes, np.float32).reshape(kc.shape)
    gv = device.download(b["vc"], vc.nbytes, np.float32).reshape(vc.shape)
    assert np.abs(gk[:, :p0 + S] - K[:, :p0 + S]).max() <= 1e-6 * max(1.0, np.abs(K).max())
    assert np.array_equal(gv[:, :p0 + S], V[:, :p0 + S].astype(np.float32))


# ---------------- single-row attention as key-split partials ----------------

MAXSPLIT, STRIDE = 8, 132  # smith_attention_parts' partial records


def _combine(parts, p0, nH, hd):
    """Host combination of the (m, l, o) split partials of every head (the
    o-projection does this on the device): sum_z e^(m_z - M) o_z / sum_z e^(m_z - M) l_z."""
    nsplit = min(MAXSPLIT, (p0 + 1 + 31) // 32)
    out = np.zeros(nH * hd)
    for h in range(nH):
        rec = parts[h * MAXSPLIT:(h + 1) * MAXSPLIT][:nsplit].astype(np.float64)
        m, l, o = rec[:, 0], rec[:, 1], rec[:, 4:4 + hd]
        w = np.exp(m - m.max())
        out[h * hd:(h + 1) * hd] = (w[:, None] * o).sum(0) / (w * l).sum()
    return out


@pytest.mark.parametrize("p0,nH,nKV,hd,rope", [(0, 4, 2, 128, "none"), (31, 4, 2, 128, "tag"), (32, 4, 2, 128, "tag"),
                                               (77, 6, 3, 64, "stale"), (255, 4, 2, 128, "tag"),
                                               (256, 8, 8, 32, "none"), (300, 4, 2, 128, "tag"),
                                               (700, 4, 1, 128, "stale")])
def test_attention_parts_matches_reference(p0, nH, nKV, hd, rope):
    """smith_attention_parts at positions on and around the 32-row tiles and
    past 8 x 32 keys (splits of several tiles), with the rope row absent,
    current (tag == position) or stale (another position's tag, garbage
    entries: the table must be used).  Cache rows past the position hold NaN:
    they must not reach the result."""
    maxSeq = 1024
    Wq, Wk = nH * hd, nKV * hd
    ld = Wq + 2 * Wk
    cos, sin = LO.precompute_rope(hd, (p0 + 2) * nH, 10000.0)  # whole-row RoPE reads pos * Wq/2 + i
    qkv = prng.randn((1, ld), 40 + p0)
    kc = np.full((nKV, maxSeq, hd), np.nan, np.float32)
    vc = np.full((nKV, maxSeq, hd), np.nan, np.float32)
    kc[:, :p0] = prng.randn((nKV, p0, hd), 41)
    vc[:, :p0] = prng.randn((nKV, p0, hd), 42)
    ctx = device.ops_ctx()
    b = {}
    for name, a in (("qkv", qkv), ("cos", cos.astype(np.float32)), ("sin", sin.astype(np.float32)), ("kc", kc),
                    ("vc", vc)):
        a = np.ascontiguousarray(a, np.float32)
        b[name] = device.alloc(a.nbytes)
        device.upload(b[name], a)
    pos = device.alloc(4)
    device.upload(pos, np.array([p0], np.int32))
    rr = None
    if rope != "none":
        hq, hk = Wq // 2, Wk // 2
        row = np.full(4 + Wq + Wk, 7.5, np.float32)  # stale: garbage entries
        tag = p0 if rope == "tag" else p0 + 3
        if rope == "tag":
            row[4:4 + hq] = cos[p0 * hq:(p0 + 1) * hq]
            row[4 + hq:4 + Wq] = sin[p0 * hq:(p0 + 1) * hq]
            row[4 + Wq:4 + Wq + hk] = cos[p0 * hk:(p0 + 1) * hk]
            row[4 + Wq + hk:] = sin[p0 * hk:(p0 + 1) * hk]
        row[:1] = np.array([tag], np.int32).view(np.float32)
        rr = device.alloc(row.nbytes)
        device.upload(rr, row)
    parts = device.alloc(nH * MAXSPLIT * STRIDE * 4)
    device.check(device.lib.smith_attention_parts(ctx, b["qkv"], pos, nH, nKV, hd, b["cos"], b["sin"], cos.size, rr,
                                                  b["kc"], b["vc"], maxSeq, parts))
    device.sync()
    got = _combine(device.download(parts, nH * MAXSPLIT * STRIDE * 4, np.float32).reshape(-1, STRIDE), p0, nH, hd)
    q64 = qkv.astype(np.float64)
    kc0 = np.where(np.isnan(kc), 0.0, kc).astype(np.float64)
    vc0 = np.where(np.isnan(vc), 0.0, vc).astype(np.float64)
    want, K, V = _ref(q64[:, :Wq], q64[:, Wq:Wq + Wk], q64[:, Wq + Wk:], kc0, vc0, p0, nH, nKV, hd, cos, sin)
    assert np.isfinite(got).all()
    assert normwise_rel_err(got, want[0]) <= 1e-5
    gk = device.download(b["kc"], kc.nbytes, np.float32).reshape(kc.shape)
    gv = device.download(b["vc"], vc.nbytes, np.float32).reshape(vc.shape)
    assert np.abs(gk[:, p0] - K[:, p0]).max() <= 1e-6 * max(1.0, np.abs(K[:, :p0 + 1]).max())
    assert np.array_equal(gv[:, p0], V[:, p0].astype(np.float32))


def test_argmax_embed_writes_rope_row():
    """smith_argmax_embed: first-max token, x = E[token], count / position
    advance, and the rope row of the new position (tag and the cos / sin
    table entries of the q and k row widths)."""
    nH, nKV, hd, maxSeq, dim, N = 4, 2, 64, 256, 256, 1000
    Wq, Wk = nH * hd, nKV * hd
    cos, sin = LO.precompute_rope(hd, maxSeq, 10000.0)
    logits = prng.randn((N,), 50)
    logits[[17, 640]] = logits.max() + 1.0  # tie: the first index wins
    E = prng.randn((N, dim), 51)
    ctx = device.ops_ctx()
    bl, bE, bc, bs = (device.alloc(a.nbytes) for a in (logits, E, cos.astype(np.float32), sin.astype(np.float32)))
    device.upload(bl, logits)
    device.upload(bE, E)
    device.upload(bc, cos.astype(np.float32))
    device.upload(bs, sin.astype(np.float32))
    x, toks, cnt, pos = device.alloc(dim * 4), device.alloc(64), device.alloc(4), device.alloc(4)
    device.upload(cnt, np.array([3], np.int32))
    device.upload(pos, np.array([40], np.int32))
    rr = device.alloc((4 + Wq + Wk) * 4)
    device.check(device.lib.smith_set_i32(ctx, rr, -1))
    device.check(device.lib.smith_argmax_embed(ctx, bl, N, bE, dim, x, toks, cnt, pos, None, None, bc, bs,
                                               cos.size, Wq, Wk, rr))
    device.sync()
    assert device.download(toks, 16, np.int32)[3] == 17
    assert device.download(cnt, 4, np.int32)[0] == 4
    assert device.download(pos, 4, np.int32)[0] == 41
    assert np.array_equal(device.download(x, dim * 4, np.float32), E[17])
    row = device.download(rr, (4 + Wq + Wk) * 4, np.float32)
    assert row[:1].view(np.int32)[0] == 41
    hq, hk, p = Wq // 2, Wk // 2, 41
    want = np.concatenate([cos[p * hq:(p + 1) * hq], sin[p * hq:(p + 1) * hq], cos[p * hk:(p + 1) * hk],
                           sin[p * hk:(p + 1) * hk]]).astype(np.float32)
    assert np.array_equal(row[4:], want)


# ---------------- device-side position bounds ----------------

@pytest.mark.parametrize("entry,S", [("attention", 16), ("attention", 1), ("parts", 1)])
@pytest.mark.parametrize("case", ["short_table", "past_cache", "negative"])
def test_position_bounds_fail_cleanly(entry, S, case):
    """A position outside the KV cache, or one whose whole-row RoPE would
    read past the tables (here one entry short), makes the launch touch no
    cache or table entry and the next synchronising call report it; the
    error is reported once, and a valid call afterwards works."""
    nH, nKV, hd, maxSeq = 4, 2, 64, 64
    Wq, Wk = nH * hd, nKV * hd
    ld = Wq + 2 * Wk
    p0 = {"short_table": 10, "past_cache": maxSeq - S + 1, "negative": -1}[case]
    cos, sin = LO.precompute_rope(hd, maxSeq * nH, 10000.0)  # ample: every row's whole-row entries
    n_tab = cos.size if case != "short_table" else (p0 + S) * (Wq // 2) - 1
    print("bounds case", entry, S, case, p0, n_tab, flush=True)
    qkv = prng.randn((S, ld), 60)
    kc = prng.randn((nKV, maxSeq, hd), 61)
    vc = prng.randn((nKV, maxSeq, hd), 62)
    ctx = device.ops_ctx()
    b = {}
    for name, a in (("qkv", qkv), ("cos", cos[:n_tab]), ("sin", sin[:n_tab]), ("kc", kc), ("vc", vc)):
        a = np.ascontiguousarray(a, np.float32)
        b[name] = device.alloc(a.nbytes)
        device.upload(b[name], a)
    pos = device.alloc(4)
    device.upload(pos, np.array([p0], np.int32))
    out = device.alloc(S * Wq * 4)
    parts = device.alloc(nH * MAXSPLIT * STRIDE * 4)

    def call(p):
        if entry == "attention":
            return device.lib.smith_attention(ctx, b["qkv"], ld, p, S, nH, nKV, hd, b["cos"], b["sin"], n_tab,
                                              b["kc"], b["vc"], maxSeq, out, None)
        return device.lib.smith_attention_parts(ctx, b["qkv"], p, nH, nKV, hd, b["cos"], b["sin"], n_tab, None,
                                                b["kc"], b["vc"], maxSeq, parts)
    assert call(pos) == 0  # enqueued: the position is only known on the device
    assert device.lib.smith_sync(ctx) != 0
    msg = device.lib.smith_last_error(ctx).decode()
    assert "outside the KV cache or the whole-row RoPE table" in msg and str(p0) in msg, msg
    device.sync()  # reported once
    assert np.array_equal(device.download(b["kc"], kc.nbytes, np.float32).reshape(kc.shape), kc)
    assert np.array_equal(device.download(b["vc"], vc.nbytes, np.float32).reshape(vc.shape), vc)
    # a position inside both bounds runs normally afterwards
    device.upload(pos, np.array([0], np.int32))
    assert call(pos) == 0
    device.sync()
