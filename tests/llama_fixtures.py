"""Tiny Llama GGUF files written on the CPU (numpy + the oracle's block
encoders), with the same layout choices as smith_amd.synthetic_gguf.

linear_type sets every linear weight's block type; `types` overrides it per
linear ({"attn_v": "q6_k", ...}); embd_type / head_type set token_embd's and
output.weight's types (f32 / q4_0 by default)."""
import numpy as np

from oracle import oracle as O
from smith_amd import gguf as G
from smith_amd import prng


def write_tiny_llama(path, dim=64, layers=2, heads=4, kv_heads=2, ffn=96, vocab=96, context=512, seed=3,
                     linear_type="q4_0", tie=False, kv_override=None, head_f32=None, std=0.05, types=None,
                     embd_type="f32", head_type="q4_0"):
    hd = dim // heads
    kvd = kv_heads * hd
    T = G.GGUF_TYPE
    meta = {
        "general.architecture": (T["STRING"], "llama"),
        "llama.embedding_length": (T["UINT32"], dim),
        "llama.block_count": (T["UINT32"], layers),
        "llama.attention.head_count": (T["UINT32"], heads),
        "llama.attention.head_count_kv": (T["UINT32"], kv_heads),
        "llama.context_length": (T["UINT32"], context),
        "llama.feed_forward_length": (T["UINT32"], ffn),
        "llama.rope.freq_base": (T["FLOAT32"], 10000.0),
        "llama.attention.layer_norm_rms_epsilon": (T["FLOAT32"], 1e-5),
        "llama.vocab_size": (T["UINT32"], vocab),
    }
    types = dict(types or {})

    def ttype(name):
        return G.GGML_TYPE[name.upper()]
    s = [seed * 7919]

    def nxt():
        s[0] += 1
        return s[0]

    def f32(name, shape, std_=std, mean=0.0, arr=None):
        a = prng.randn(shape, nxt(), std=std_, mean=mean) if arr is None else np.asarray(arr, np.float32)
        return (name, list(shape), G.GGML_TYPE["F32"], a.size * 4, lambda a=a: a)

    def lin(name, out_, in_, arr=None):
        w = prng.randn((out_, in_), nxt(), std=std) if arr is None else arr
        t = ttype(types.get(name.split(".")[2], linear_type))
        q = O.quantize_rows(t, w)
        return (name, [out_, in_], t, q.size, lambda q=q: q)

    tensors = []
    E = prng.randn((vocab, dim), nxt(), std=std)
    if embd_type == "f32":
        tensors.append(f32("token_embd.weight", (vocab, dim), arr=E))
    else:
        qe = O.quantize_rows(ttype(embd_type), E)
        tensors.append(("token_embd.weight", [vocab, dim], ttype(embd_type), qe.size, lambda q=qe: q))
    for L in range(layers):
        p = "blk.%d." % L
        tensors.append(f32(p + "attn_norm.weight", (dim,), 0.02, 1.0))
        tensors.append(lin(p + "attn_q.weight", dim, dim))
        if kv_override is not None:
            kw, vw = kv_override(L)
            tensors.append(lin(p + "attn_k.weight", kvd, dim, kw))
            tensors.append(lin(p + "attn_v.weight", kvd, dim, vw))
        else:
            tensors.append(lin(p + "attn_k.weight", kvd, dim))
            tensors.append(lin(p + "attn_v.weight", kvd, dim))
        tensors.append(lin(p + "attn_output.weight", dim, dim))
        tensors.append(lin(p + "ffn_gate.weight", ffn, dim))
        tensors.append(lin(p + "ffn_up.weight", ffn, dim))
        tensors.append(lin(p + "ffn_down.weight", dim, ffn))
        tensors.append(f32(p + "ffn_norm.weight", (dim,), 0.02, 1.0))
    tensors.append(f32("output_norm.weight", (dim,), 0.02, 1.0))
    if head_f32 is not None:
        tensors.append(f32("output.weight", (dim, vocab), arr=head_f32))
    elif not tie:
        # flat data = lmHead[dim][vocab], quantized along vocab
        w = prng.randn((dim, vocab), nxt(), std=std)
        q = O.quantize_rows(ttype(head_type), w)
        tensors.append(("output.weight", [dim, vocab], ttype(head_type), q.size, lambda q=q: q))
    G.write_gguf(path, meta, tensors)
    return E
