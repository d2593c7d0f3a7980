"""GPU parity of smith_attention for prompt rows (S > 1: KV append + the
f32-MFMA flash attention) and single rows (S == 1), against a float64
reference built from the Llama oracle's RoPE (whole-row indexing,
oracle/llama_oracle.py rope_rows) and causal GQA softmax attention
(gguf_cache.js:128-157, 212-231).  Keys before p0 come from caches filled
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
            kv = h // rep
            sc = K[kv, :T] @ q[s, h * hd:(h + 1) * hd] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            out[s, h * hd:(h + 1) * hd] = (p / p.sum()) @ V[kv, :T]
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
    device.check(device.lib.smith_attention(ctx, b["qkv"], ld, pos, S, nH, nKV, hd, b["cos"], b["sin"], b["kc"],
                                            b["vc"], maxSeq, out, None))
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
