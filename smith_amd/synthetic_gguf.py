"""Seeded random-init Llama GGUF files (config 5 and small test models).

Weights are generated and quantized on the GPU (smith_randn +
smith_quantize_q4_0: ggml q4_0 rounding in the reference decoder's
interleaved nibble order) and streamed to the file one tensor at a time.
mix="q4_k_m" writes the llama.cpp Q4_K_M type mix instead (Q4_K q/k/o/gate/
up and token_embd, Q6_K v/down and output.weight) with seeded random block
fields -- nibbles, 6-bit scales, int8 scales uniform, each Q4_K min equal to
its scale with dmin = 7.5 d so the weights have zero mean, f16 scales chosen
for weights of about N(0, 0.02) size: a random init in quantized form.
Layout choices (so the reference's own loader would read the same model):
  * linear weights are listed [out, in] with blocks along `in`
    (gguf_loader.js:243-253 transposes such a listing into Smith's [in, out]);
  * output.weight's flat data is written as lmHead[dim][vocab] (the loader
    copies it untransposed, gguf_loader.js:256-259), quantized along vocab;
  * token_embd is f32 [vocab, dim]; norms are f32 ~ N(1, 0.02);
  * llama.context_length defaults to 8192 so the reference's whole-row RoPE
    indexing stays inside its table for 256 positions.
"""
import numpy as np

from . import device
from . import gguf as G

CONFIG5 = dict(dim=3072, layers=32, heads=24, kv_heads=8, ffn=9216, vocab=32000, context=8192, eps=1e-5,
               rope_base=10000.0)


def _gpu_randn(n, seed, std, mean):
    buf = device.alloc(n * 4)
    device.check(device.lib.smith_randn(device.ops_ctx(), buf, n, seed, 0, std, mean), "randn")
    return buf


def _f32_producer(n, seed, std, mean):
    def run():
        b = _gpu_randn(n, seed, std, mean)
        out = device.download(b, n * 4, np.float32)
        device.release_buffer(b)
        return out
    return run


def _q4_0_producer(rows, cols, seed, std):
    def run():
        n = rows * cols
        b = _gpu_randn(n, seed, std, 0.0)
        q = device.alloc(n // 32 * 18)
        device.check(device.lib.smith_quantize_q4_0(device.ops_ctx(), b, q, rows, cols), "quantize_q4_0")
        out = device.download(q, n // 32 * 18, np.uint8)
        device.release_buffer(b)
        device.release_buffer(q)
        return out
    return run


def _f16_bytes(v, n):
    return np.full(n, v, np.float16).view(np.uint8).reshape(n, 2)


def _kquant_producer(ggml, rows, cols, seed):
    """Random Q4_K / Q6_K blocks of a [rows, cols] tensor (cols % 256 == 0)."""
    def run():
        nb = rows * cols // 256
        rng = np.random.default_rng(seed)
        if ggml == G.GGML_TYPE["Q4_K"]:
            b = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
            b[:, 0:2] = _f16_bytes(1.0e-4, nb)   # d: 63 * 15 * 1e-4 ~ 0.09 full scale
            b[:, 2:4] = _f16_bytes(7.5e-4, nb)   # dmin = 7.5 d
            # every sub-block's 6-bit min equal to its 6-bit scale: bytes 4-7
            # repeat bytes 0-3 and each of bytes 8-11 carries the same nibble
            # twice, so w = d*sc*q - 7.5*d*sc = d*sc*(q - 7.5) has zero mean
            # over the uniform nibbles (uniform mins would give every weight a
            # positive offset and a degenerate model)
            b[:, 8:12] = b[:, 4:8]
            lo = b[:, 12:16] & 0x0F
            b[:, 12:16] = lo | (lo << 4)
        else:
            b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
            b[:, 208:210] = _f16_bytes(2.0e-5, nb)  # d: 127 * 32 * 2e-5 ~ 0.08 full scale
        return b.ravel()
    return run


def build_llama_gguf(path, dim, layers, heads, kv_heads, ffn, vocab, context=8192, eps=1e-5, rope_base=10000.0,
                     seed=1, std=0.02, tie_embeddings=False, mix="q4_0"):
    """Write a seeded random-init Llama GGUF (Q4_0 linears, or the Q4_K_M
    mix) to `path`."""
    if mix not in ("q4_0", "q4_k_m"):
        raise ValueError("mix must be q4_0 or q4_k_m")
    if mix == "q4_k_m" and (dim % 256 or ffn % 256 or vocab % 256):
        raise ValueError("the Q4_K_M mix needs dim, ffn and vocab multiples of 256")
    if dim % 32 or ffn % 32 or vocab % 32:
        raise ValueError("dim, ffn and vocab must be multiples of 32 for Q4_0")
    hd = dim // heads
    kvd = kv_heads * hd
    T = G.GGUF_TYPE
    meta = {
        "general.architecture": (T["STRING"], "llama"),
        "general.name": (T["STRING"], "smith-synthetic-llama"),
        "general.alignment": (T["UINT32"], 32),
        "llama.embedding_length": (T["UINT32"], dim),
        "llama.block_count": (T["UINT32"], layers),
        "llama.attention.head_count": (T["UINT32"], heads),
        "llama.attention.head_count_kv": (T["UINT32"], kv_heads),
        "llama.context_length": (T["UINT32"], context),
        "llama.feed_forward_length": (T["UINT32"], ffn),
        "llama.rope.freq_base": (T["FLOAT32"], rope_base),
        "llama.attention.layer_norm_rms_epsilon": (T["FLOAT32"], eps),
        "llama.vocab_size": (T["UINT32"], vocab),
    }
    F32, Q40 = G.GGML_TYPE["F32"], G.GGML_TYPE["Q4_0"]
    Q4K, Q6K = G.GGML_TYPE["Q4_K"], G.GGML_TYPE["Q6_K"]
    kbytes = {Q4K: 144, Q6K: 210}
    tensors = []
    s = seed * 1000003

    def nxt():
        nonlocal s
        s += 1
        return s

    if mix == "q4_k_m":
        tensors.append(("token_embd.weight", [vocab, dim], Q4K, vocab * dim // 256 * 144,
                        _kquant_producer(Q4K, vocab, dim, nxt())))
    else:
        tensors.append(("token_embd.weight", [vocab, dim], F32, vocab * dim * 4,
                        _f32_producer(vocab * dim, nxt(), std, 0.0)))
    for L in range(layers):
        p = "blk.%d." % L
        tensors.append((p + "attn_norm.weight", [dim], F32, dim * 4, _f32_producer(dim, nxt(), 0.02, 1.0)))
        for name, out_, in_ in (("attn_q", dim, dim), ("attn_k", kvd, dim), ("attn_v", kvd, dim),
                                ("attn_output", dim, dim), ("ffn_gate", ffn, dim), ("ffn_up", ffn, dim),
                                ("ffn_down", dim, ffn)):
            if mix == "q4_k_m":
                t = Q6K if name in ("attn_v", "ffn_down") else Q4K
                tensors.append((p + name + ".weight", [out_, in_], t, out_ * in_ // 256 * kbytes[t],
                                _kquant_producer(t, out_, in_, nxt())))
            else:
                tensors.append((p + name + ".weight", [out_, in_], Q40, out_ * in_ // 32 * 18,
                                _q4_0_producer(out_, in_, nxt(), std)))
        tensors.append((p + "ffn_norm.weight", [dim], F32, dim * 4, _f32_producer(dim, nxt(), 0.02, 1.0)))
    tensors.append(("output_norm.weight", [dim], F32, dim * 4, _f32_producer(dim, nxt(), 0.02, 1.0)))
    if not tie_embeddings and mix == "q4_k_m":
        tensors.append(("output.weight", [dim, vocab], Q6K, dim * vocab // 256 * 210,
                        _kquant_producer(Q6K, dim, vocab, nxt())))
    elif not tie_embeddings:
        tensors.append(("output.weight", [dim, vocab], Q40, dim * vocab // 32 * 18,
                        _q4_0_producer(dim, vocab, nxt(), std)))
    return G.write_gguf(path, meta, tensors)
