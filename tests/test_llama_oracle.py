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
