"""loadGGUF on the non-Llama architectures the reference maps (phi, phi2,
phi3, gpt2: gguf_loader.js:48-91): weights loaded under the reference's
names and shapes, the same loaded / skipped lists, forward refused with the
reference's message (gguf_loader.js:394-396).

Expected lists follow from the reference's rules read by hand: a name the
map does not resolve is skipped as itself; a name it resolves to a
parameter the model lacks (biases, qkvProj, ln1Beta, posWeight) is skipped
as "name → path (not found in model)"; the loaded 2-D weights listed
[out, in] are transposed into [in, out].  Values: bit-exact to the oracle's
dequantizeTensor.
"""
import numpy as np
import pytest

from oracle import oracle as O
from smith_amd import gguf as G
from smith_amd import prng

pytestmark = pytest.mark.gpu

DIM, FFN, VOCAB = 256, 512, 96


def _write(path, arch):
    T = G.GGUF_TYPE
    meta = {
        "general.architecture": (T["STRING"], arch),
        "%s.embedding_length" % arch: (T["UINT32"], DIM),
        "%s.block_count" % arch: (T["UINT32"], 1),
        "%s.attention.head_count" % arch: (T["UINT32"], 4),
        "%s.context_length" % arch: (T["UINT32"], 64),
        "%s.feed_forward_length" % arch: (T["UINT32"], FFN),
        "%s.vocab_size" % arch: (T["UINT32"], VOCAB),
    }
    seed = [100]
    raw = {}

    def f32(name, shape):
        seed[0] += 1
        a = prng.randn(shape, seed[0], std=0.05)
        raw[name] = (O.GGML_F32, a.astype(np.float32).view(np.uint8).ravel(), shape)
        return (name, list(shape), O.GGML_F32, a.size * 4, lambda a=a: a)

    def q(name, shape, t):
        seed[0] += 1
        blocks = O.quantize_rows(t, prng.randn(shape, seed[0], std=0.02))
        raw[name] = (t, blocks, shape)
        return (name, list(shape), t, blocks.size, lambda b=blocks: b)

    tensors = [f32("token_embd.weight", (VOCAB, DIM)), f32("output_norm.weight", (DIM,)),
               f32("output_norm.bias", (DIM,)), f32("blk.0.attn_norm.weight", (DIM,)),
               f32("blk.0.attn_norm.bias", (DIM,)), q("blk.0.attn_qkv.weight", (3 * DIM, DIM), O.GGML_Q4_0),
               f32("blk.0.attn_qkv.bias", (3 * DIM,)), q("blk.0.attn_output.weight", (DIM, DIM), O.GGML_Q4_0),
               f32("blk.0.ffn_norm.weight", (DIM,)), q("blk.0.ffn_up.weight", (FFN, DIM), O.GGML_Q4_K),
               q("blk.0.ffn_down.weight", (DIM, FFN), O.GGML_Q6_K), f32("rope_freqs.weight", (32,))]
    if arch != "gpt2":
        tensors.append(q("output.weight", (DIM, VOCAB), O.GGML_Q8_0))
    else:
        tensors.append(f32("position_embd.weight", (64, DIM)))
    G.write_gguf(path, meta, tensors)
    return raw


def _f32(raw, name):
    t, data, shape = raw[name]
    return O.dequantize_tensor(t, data, int(np.prod(shape))).reshape(shape)


@pytest.mark.parametrize("arch", ["phi2", "gpt2"])
def test_other_architectures_load_like_the_reference(tmp_path, arch):
    from smith_amd.gguf_loader import loadGGUF
    p = str(tmp_path / ("%s.gguf" % arch))
    raw = _write(p, arch)
    m = loadGGUF(p)
    qkv_path = "qkvProj" if arch != "gpt2" else "qkvFused"
    want_loaded = ["token_embd.weight", "output_norm.weight", "output_norm.bias", "blk.0.attn_norm.weight",
                   "blk.0.attn_output.weight", "blk.0.ffn_norm.weight", "blk.0.ffn_up.weight",
                   "blk.0.ffn_down.weight"] + (["output.weight"] if arch != "gpt2" else [])
    want_skipped = ["blk.0.attn_norm.bias → blocks.0.ln1Beta (not found in model)",
                    "blk.0.attn_qkv.weight → blocks.0.mha.%s.weight (not found in model)" % qkv_path,
                    "blk.0.attn_qkv.bias → blocks.0.mha.%s.bias (not found in model)" % qkv_path,
                    "rope_freqs.weight"] + (["position_embd.weight → embedding.posWeight (not found in model)"]
                                            if arch == "gpt2" else [])
    assert sorted(m.loaded) == sorted(want_loaded)
    assert sorted(m.skipped) == sorted(want_skipped)
    P = m.model["params"]
    # [out, in] listings transposed to Smith's [in, out]; bit-exact values
    assert np.array_equal(P["blocks.0.mha.outProj.weight"].numpy(), _f32(raw, "blk.0.attn_output.weight").T)
    assert np.array_equal(P["blocks.0.ffn1.weight"].numpy(), _f32(raw, "blk.0.ffn_up.weight").T)
    assert np.array_equal(P["blocks.0.ffn2.weight"].numpy(), _f32(raw, "blk.0.ffn_down.weight").T)
    assert np.array_equal(P["lnFBeta"].numpy().ravel(), _f32(raw, "output_norm.bias"))
    if arch != "gpt2":
        # lmHead: the flat data untransposed (its path does not end in ".weight")
        assert np.array_equal(P["lmHead"].numpy().ravel(), _f32(raw, "output.weight").ravel())
        assert "rope" in m.model
    else:
        assert m.model.get("weightTied") and "rope" not in m.model
    with pytest.raises(RuntimeError, match="Forward not implemented for %s via GGUF loader" % arch):
        m.forward([1, 2, 3])
    with pytest.raises(RuntimeError):
        m.generate([1, 2, 3], {"maxTokens": 2})
