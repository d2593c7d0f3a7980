"""Pins the Llama oracle (oracle/llama_oracle.py) on the CPU.

  rmsnorm           closed form on a 2-vector
  precompute_rope   table entries vs cos/sin of pos * f32(1/base^(2i/d))
  rope_rows         position 0 is the identity; one row of width headDim is
                    the textbook pairwise rotation; whole-row pairing of a
                    [1, dim] row uses pos*(dim/2)+i (finding 6)
  cache / causality prefill logits == logits of token-by-token decode
                    (tests/gguf_cache.test.js:343-378 checks 0.1; f64 gives ~0)
  GQA mapping       nKV < nH equals nKV = nH with kv heads repeated h -> h/rep
                    (single position: RoPE is the identity at position 0)
  lm-head layout    output.weight flat data read as [dim, vocab]: an F32
                    output.weight holding E^T equals weight tying
  GGUF parsing      the product writer's file read back by the oracle reader
  silu / SwiGLU     silu(0) = 0, silu(1) = sigmoid(1), silu(-x) = silu(x) - x,
                    the limits; silu(gate) * up on an asymmetric pair, and the
                    layer's FFN wiring on a hand-built layer (gate != up)
  attention         two keys at head_dim 4: weights e^(s_i / sqrt(4)) / sum,
                    directly and through a hand-built layer (causal row 0)
"""
import os

import numpy as np
import pytest

from oracle import llama_oracle as LO
from smith_amd import gguf as G
from tests.llama_fixtures import write_tiny_llama


def test_rmsnorm_closed_form():
    y = LO.rmsnorm(np.array([3.0, 4.0]), np.array([1.0, 2.0]), 0.0)
    r = np.sqrt((9 + 16) / 2)
    assert np.allclose(y, [3 / r, 8 / r], rtol=0, atol=1e-15)


def test_rope_table_and_rotation():
    hd, base = 8, 10000.0
    cos, sin = LO.precompute_rope(hd, 16, base)
    for pos in (0, 3, 15):
        for i in range(hd // 2):
            f = np.float32(1.0 / base ** (2 * i / hd))
            assert cos[pos * 4 + i] == np.float32(np.cos(pos * float(f)))
            assert sin[pos * 4 + i] == np.float32(np.sin(pos * float(f)))
    x = np.arange(1.0, 9.0)[None, :]
    assert np.array_equal(LO.rope_rows(x, 0, cos, sin), x)
    y = LO.rope_rows(x, 5, cos, sin)[0]
    for i in range(4):  # textbook rotation of (x_i, x_{i+4}) by angle 5 * f_i
        a = 5 * float(np.float32(1.0 / base ** (2 * i / hd)))
        c, s = np.float32(np.cos(a)), np.float32(np.sin(a))
        assert np.isclose(y[i], x[0, i] * c - x[0, i + 4] * s)
        assert np.isclose(y[i + 4], x[0, i] * s + x[0, i + 4] * c)
    # a [1, 16] row (two heads) at position 2 uses table entries 2*8 + i
    x = np.arange(16.0)[None, :]
    cos2, sin2 = LO.precompute_rope(hd, 64, base)
    y = LO.rope_rows(x, 2, cos2, sin2)[0]
    assert np.isclose(y[3], x[0, 3] * cos2[16 + 3] - x[0, 11] * sin2[16 + 3])


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("llama")
    path = str(d / "tiny.gguf")
    write_tiny_llama(path)
    return path


def test_gguf_round_trip(tiny):
    parsed = G.loadGGUFFile(tiny)
    cfg = G.extractConfig(parsed["metadata"])
    assert (cfg["dim"], cfg["numLayers"], cfg["numHeads"], cfg["numKVHeads"], cfg["vocabSize"]) == (64, 2, 4, 2, 96)
    buf, meta, tensors, data0 = LO.read_gguf(tiny)
    assert data0 == parsed["dataOffset"]
    assert [t[0] for t in tensors] == [t["name"] for t in parsed["tensors"]]


def test_prefill_equals_sequential_decode(tiny):
    m = LO.LlamaOracle(tiny)
    toks = [5, 17, 3, 88, 42, 7]
    pre = m.forward(toks, 0)
    m.reset()
    dec = np.stack([m.forward([t], i)[0] for i, t in enumerate(toks)])
    assert np.max(np.abs(pre - dec)) < 1e-9


def test_gqa_repeat_mapping(tmp_path):
    dim, heads, hd = 64, 4, 16
    rng = np.random.default_rng(0)
    kv = {L: (rng.normal(0, 0.05, (2 * hd, dim)).astype(np.float32),
              rng.normal(0, 0.05, (2 * hd, dim)).astype(np.float32)) for L in range(2)}

    def rep(w):  # kv heads [0, 1] -> [0, 0, 1, 1]
        return np.concatenate([w[:hd], w[:hd], w[hd:], w[hd:]])

    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    write_tiny_llama(a, kv_heads=2, kv_override=lambda L: kv[L])
    write_tiny_llama(b, kv_heads=4, kv_override=lambda L: (rep(kv[L][0]), rep(kv[L][1])))
    # position 0 only: RoPE is the identity there, while at later positions
    # the whole-row pairing (k[i] with k[i + kvDim/2]) differs between the
    # two kv widths; one key means each q head returns its kv head's value
    for t in (1, 50):
        la = LO.LlamaOracle(a).forward([t], 0)
        lb = LO.LlamaOracle(b).forward([t], 0)
        assert np.max(np.abs(la - lb)) < 1e-9
    # and the mapping matters: h % nKV instead of h / rep gives other logits
    m = LO.LlamaOracle(a)
    blk = m.blocks[0]
    assert not np.allclose(blk["v"][:, :hd], blk["v"][:, hd:])


def test_lm_head_layout_matches_tying(tmp_path):
    a, b = str(tmp_path / "tied.gguf"), str(tmp_path / "head.gguf")
    E = write_tiny_llama(a, tie=True)
    write_tiny_llama(b, head_f32=np.ascontiguousarray(E.T))
    toks = [9, 4, 60]
    la = LO.LlamaOracle(a).forward(toks, 0)
    lb = LO.LlamaOracle(b).forward(toks, 0)
    assert np.max(np.abs(la - lb)) < 1e-9


# --- SwiGLU and attention pins (closed forms and hand-computed numbers) ---
SIG1 = 0.7310585786300049  # sigmoid(1) = 1 / (1 + e^-1)


def test_silu_closed_forms():
    assert LO.silu(np.array(0.0)) == 0.0
    assert np.isclose(LO.silu(np.array(1.0)), SIG1, rtol=0, atol=1e-15)
    x = np.array([0.3, 1.7, 4.0, 11.0])
    assert np.allclose(LO.silu(-x), LO.silu(x) - x, rtol=0, atol=1e-14)  # silu(-x) = silu(x) - x
    assert np.isclose(LO.silu(np.array(40.0)), 40.0, rtol=1e-15)  # silu(x) -> x
    assert abs(LO.silu(np.array(-40.0))) < 1e-15  # silu(x) -> 0 for x -> -inf


def test_swiglu_operand_order():
    # silu(gate) * up: silu(2) * 3 = 3 * 2 / (1 + e^-2); the swapped form gives silu(3) * 2
    got = LO.swiglu(np.array([2.0]), np.array([3.0]))[0]
    assert np.isclose(got, 5.284782467867515, rtol=0, atol=1e-12)
    assert not np.isclose(got, LO.swiglu(np.array([3.0]), np.array([2.0]))[0], atol=1e-3)


def test_attend_two_keys_scale():
    # hd = 4: scale 1/sqrt(4) = 0.5; scores 2 and 4 -> 1 and 2; weights e^1/(e^1+e^2), e^2/(e^1+e^2)
    q = np.array([2.0, 0, 0, 0])
    K = np.array([[1.0, 1, 1, 1], [2.0, 0, 0, 0]])
    V = np.array([[1.0, 0, 5, 0], [0.0, 1, 0, 7]])
    out = LO.attend(q, K, V, 0.5)
    w0, w1 = 1 - SIG1, SIG1  # e/(e+e^2) = 1/(1+e) = 1 - sigmoid(1)
    assert np.allclose(out, [w0, w1, 5 * w0, 7 * w1], rtol=0, atol=1e-15)


def _toy(dim, ffn, blocks):
    """A one-layer, one-head model built in memory (RoPE switched off by an
    all-cos-1 table, eps 0) so a layer's output can be written down by hand."""
    m = object.__new__(LO.LlamaOracle)
    m.dim, m.L, m.nH, m.nKV, m.hd, m.kvd, m.ffn = dim, 1, 1, 1, dim, dim, ffn
    m.eps, m.max_seq, m.lazy = 0.0, 8, False
    m.cos, m.sin = np.ones(8 * dim), np.zeros(8 * dim)
    m.blocks = [blocks]
    m.reset()
    return m


def test_layer_attention_scale_and_causality():
    """Two positions, identity q/k/v/o, FFN off: row 0 attends only to key 0
    (out = 2 x0); row 1 mixes values 0 and 1 with softmax weights of the
    scores q1.k / sqrt(hd) = (2, 4) / 2.  A 1/hd scale, a missing scale or a
    non-causal mask each give other numbers."""
    I4, Z = np.eye(4), np.zeros((4, 2))
    m = _toy(4, 2, dict(g1=np.ones(4), g2=np.ones(4), q=I4, k=I4, v=I4, o=I4, gate=Z, up=Z, down=np.zeros((2, 4))))
    x = np.array([[1.0, 1, 1, 1], [2.0, 0, 0, 0]])  # both rows have rms 1
    y = m._layer(0, x, 0)
    assert np.allclose(y[0], 2 * x[0], rtol=0, atol=1e-15)
    w0, w1 = 1 - SIG1, SIG1
    assert np.allclose(y[1], x[1] + w0 * x[0] + w1 * x[1], rtol=0, atol=1e-15)


def test_layer_swiglu_wiring():
    """Attention off (zero v), x = (3, 4, 0, 0) so rmsnorm gives (1.2, 1.6, 0, 0);
    gate = (1.2, 1.6), up = (0.5, 2.0); down scatters the two FFN outputs to
    elements 0 and 2: out = x + (silu(1.2) * 0.5, 0, silu(1.6) * 2.0, 0)."""
    Z4 = np.zeros((4, 4))
    gate = np.zeros((4, 2)); gate[0, 0] = 1; gate[1, 1] = 1
    up = np.zeros((4, 2)); up[0, 0] = 0.5 / 1.2; up[1, 1] = 2.0 / 1.6
    down = np.zeros((2, 4)); down[0, 0] = 1; down[1, 2] = 1
    m = _toy(4, 2, dict(g1=np.ones(4), g2=np.ones(4), q=Z4, k=Z4, v=Z4, o=Z4, gate=gate, up=up, down=down))
    x = np.array([[3.0, 4, 0, 0]])
    y = m._layer(0, x, 0)[0]
    s12 = 1.2 / (1 + np.exp(-1.2)) * 0.5
    s16 = 1.6 / (1 + np.exp(-1.6)) * 2.0
    assert np.allclose(y, [3 + s12, 4, s16, 0], rtol=0, atol=1e-14)


def test_layer_at_a_time_decode_equals_resident_weights(tiny):
    """The layer-at-a-time weight decoding used for config-5-sized models
    gives the same logits as keeping every layer decoded."""
    toks = [5, 17, 3, 88]
    a = LO.LlamaOracle(tiny, lazy=False).forward(toks, 0)
    b = LO.LlamaOracle(tiny, lazy=True).forward(toks, 0)
    assert np.max(np.abs(a - b)) <= 1e-12 * np.max(np.abs(a))  # BLAS order only
