"""CPU oracle of the GGUF Llama path: loadGGUF + forwardLlamaCachedPrefill /
forwardLlamaCachedDecode + greedy generateGGUF (src/gguf_loader.js,
src/gguf_cache.js), in numpy float64 on the f32 weights the reference
builds.

TEST INFRASTRUCTURE ONLY (tests/, smoke, bench's cpu_baseline).  It has its
own GGUF reader (a restatement of gguf.js:127-165) and decodes blocks with
the C oracle (oracle_dequantize_tensor), so it shares no code with the
product package.  Pinning: tests/test_llama_oracle.py.
"""
import struct

import numpy as np

from . import oracle as O

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
_BLOCK = O.BLOCK


def read_gguf(path):
    """gguf.js:127-165 (header, metadata, tensor infos, 32-byte aligned data)."""
    buf = np.memmap(path, dtype=np.uint8, mode="r")
    pos = 0

    def rd(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, buf, pos)[0]
        pos += struct.calcsize(fmt)
        return v

    def rstr():
        nonlocal pos
        n = rd("<Q")
        s = bytes(buf[pos:pos + n]).decode()
        pos += n
        return s

    scal = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}

    def rval(t):
        if t in scal:
            return rd(scal[t])
        if t == 8:
            return rstr()
        if t == 9:
            et, n = rd("<I"), rd("<Q")
            return [rval(et) for _ in range(n)]
        raise ValueError(t)

    assert rd("<I") == 0x46554747, "Not a GGUF file"
    ver = rd("<I")
    assert 2 <= ver <= 3
    nt, nkv = rd("<Q"), rd("<Q")
    meta = {}
    for _ in range(nkv):
        k = rstr()
        meta[k] = rval(rd("<I"))
    tensors = []
    for _ in range(nt):
        name = rstr()
        nd = rd("<I")
        shape = [rd("<Q") for _ in range(nd)]
        t, off = rd("<I"), rd("<Q")
        tensors.append((name, shape, t, off))
    align = meta.get("general.alignment", 32)
    data0 = -(-pos // align) * align
    return buf, meta, tensors, data0


def _tensor_f32(buf, data0, shape, t, off, out=None, stage=None):
    """dequantizeTensor, gguf.js:343-394, widened to f64.  `out` (f64) and
    `stage` (f32), when given, are arrays of numel elements reused across
    calls, so a layer-at-a-time forward does not fault in fresh pages for
    every layer."""
    numel = int(np.prod(shape))
    bs, bpb = _BLOCK[t]
    nbytes = -(-numel // bs) * bpb
    raw = np.asarray(buf[data0 + off:data0 + off + nbytes])
    if t == F32:
        src = raw.view(np.float32)
    elif t == F16:
        src = raw.view(np.float16)
    else:
        src = O.dequantize_tensor(t, raw, numel, out=stage)
    if out is None:
        return src.astype(np.float64)
    np.copyto(out, src)
    return out


def precompute_rope(hd, max_seq, base):
    """ops/rope.js:10-30 (f32 freqs, f64 angle, f32 cos/sin)."""
    half = hd // 2
    freqs = np.array([np.float32(1.0 / (float(base) ** ((2 * i) / hd))) for i in range(half)], dtype=np.float32)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * freqs.astype(np.float64)[None, :]
    return np.cos(ang).astype(np.float32).ravel().astype(np.float64), np.sin(ang).astype(np.float32).ravel().astype(
        np.float64)


def rope_rows(x, start, cos, sin):
    """shaders/rope.metal:18-37 applied to whole rows [S, W] (gguf_cache.js:130,
    213): element i pairs with i + W/2, table entry pos*(W/2) + i."""
    S, W = x.shape
    half = W // 2
    out = np.empty_like(x)
    for s in range(S):
        idx = (start + s) * half + np.arange(half)
        c, sn = cos[idx], sin[idx]
        x0, x1 = x[s, :half], x[s, half:]
        out[s, :half] = x0 * c - x1 * sn
        out[s, half:] = x0 * sn + x1 * c
    return out


def rmsnorm(x, g, eps):
    """shaders/rmsnorm.metal:15-47."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g


def silu(x):
    """shaders/swiglu.metal:12-21: g / (1 + exp(-g))."""
    return x / (1.0 + np.exp(-x))


def swiglu(gate, up):
    """shaders/swiglu.metal:12-21: out = silu(gate) * up (gate is the first
    operand, gguf_cache.js:168-170 passes ffn_gate's product first)."""
    return silu(gate) * up


def attend(q, K, V, scale):
    """Decode attention of one query row over the cached keys
    (gguf_cache.js:149-154): scores = K q * scale, softmax over all T keys,
    output = weights @ V.  K, V [T, hd]."""
    sc = (K @ q) * scale
    w = np.exp(sc - sc.max())
    w /= w.sum()
    return w @ V


class LlamaOracle:
    def __init__(self, path, lazy=None):
        buf, meta, tensors, data0 = read_gguf(path)
        arch = meta["general.architecture"]
        assert arch == "llama"

        def g(k, d=None):
            return meta.get("llama." + k, d)

        self.dim = g("embedding_length")
        self.L = g("block_count")
        self.nH = g("attention.head_count")
        self.nKV = g("attention.head_count_kv") or self.nH
        self.max_seq = g("context_length", 2048)
        self.ffn = g("feed_forward_length")
        self.eps = g("attention.layer_norm_rms_epsilon", 1e-5)
        self.vocab = g("vocab_size", 32000)
        self.hd = self.dim // self.nH
        self.kvd = self.nKV * self.hd
        self.cos, self.sin = precompute_rope(self.hd, self.max_seq, g("rope.freq_base", 10000))
        T = {name: (shape, t, off) for name, shape, t, off in tensors}

        scratch = {}

        def reuse(role, numel, dtype):
            a = scratch.get((role, dtype))
            if a is None or a.size != numel:
                a = scratch[(role, dtype)] = np.empty(numel, dtype)
            return a

        def dense(name, role=None):
            shape, t, off = T[name]
            if role is None:
                return _tensor_f32(buf, data0, shape, t, off)
            numel = int(np.prod(shape))
            return _tensor_f32(buf, data0, shape, t, off, reuse(role, numel, np.float64),
                               reuse("stage%d" % numel, numel, np.float32))

        def linear(name, n_in, n_out):
            # gguf_loader.js:238-257: [rows, cols] listing; transpose when the
            # Smith shape [in, out] equals [cols, rows], else flat copy
            shape, t, off = T[name]
            data = dense(name, name.split(".")[2] if self.lazy else None)
            rows, cols = shape
            if n_in == cols and n_out == rows:
                w = data.reshape(rows, cols).T
                return w if self.lazy else w.copy()
            return data.reshape(n_in, n_out)

        self.E = dense("token_embd.weight").reshape(self.vocab, self.dim)
        # A model whose f64 weights would not fit comfortably in host memory
        # (config 5: 3.5 G parameters) is decoded one layer at a time inside
        # forward(), into arrays reused from layer to layer; small models
        # keep every layer decoded.
        per_layer = self.dim * (2 * self.dim + 2 * self.kvd + 3 * self.ffn)
        self.lazy = per_layer * self.L > (64 << 20) if lazy is None else bool(lazy)

        def block(l):
            p = "blk.%d." % l
            return dict(
                g1=dense(p + "attn_norm.weight"), g2=dense(p + "ffn_norm.weight"),
                q=linear(p + "attn_q.weight", self.dim, self.dim), k=linear(p + "attn_k.weight", self.dim, self.kvd),
                v=linear(p + "attn_v.weight", self.dim, self.kvd), o=linear(p + "attn_output.weight", self.dim, self.dim),
                gate=linear(p + "ffn_gate.weight", self.dim, self.ffn), up=linear(p + "ffn_up.weight", self.dim, self.ffn),
                down=linear(p + "ffn_down.weight", self.ffn, self.dim))
        self._block = block
        self.blocks = None if self.lazy else [block(l) for l in range(self.L)]
        self.gF = dense("output_norm.weight")
        if "output.weight" in T:
            # lmHead [dim, vocab] gets the flat data untransposed (gguf_loader.js:256-259)
            self.head = dense("output.weight").reshape(self.dim, self.vocab)
        else:
            self.head = self.E.T  # weight tying (gguf_loader.js:266-270)
        self.reset()

    def reset(self):
        # np.zeros maps untouched pages lazily: only the positions written
        # take host memory
        self.kc = [np.zeros((self.nKV, self.max_seq, self.hd)) for _ in range(self.L)]
        self.vc = [np.zeros((self.nKV, self.max_seq, self.hd)) for _ in range(self.L)]

    def _layer(self, l, x, start):
        """x [S, dim] at positions start..start+S-1 (gguf_cache.js:116-172 and
        :199-247: keys/values of earlier positions from the cache, causal)."""
        b = self._block(l) if self.lazy else self.blocks[l]
        S = x.shape[0]
        n1 = rmsnorm(x, b["g1"], self.eps)
        q = rope_rows(n1 @ b["q"], start, self.cos, self.sin)
        k = rope_rows(n1 @ b["k"], start, self.cos, self.sin)
        v = n1 @ b["v"]
        for h in range(self.nKV):
            self.kc[l][h, start:start + S] = k[:, h * self.hd:(h + 1) * self.hd]
            self.vc[l][h, start:start + S] = v[:, h * self.hd:(h + 1) * self.hd]
        rep = self.nH // self.nKV
        att = np.empty((S, self.dim))
        scale = 1.0 / np.sqrt(self.hd)
        for h in range(self.nH):
            kv = h // rep  # repeatKV: q head h -> kv head h / rep (gguf_cache.js:90-105)
            qh = q[:, h * self.hd:(h + 1) * self.hd]
            for s in range(S):
                T = start + s + 1
                att[s, h * self.hd:(h + 1) * self.hd] = attend(qh[s], self.kc[l][kv, :T], self.vc[l][kv, :T], scale)
        x2 = x + att @ b["o"]
        n2 = rmsnorm(x2, b["g2"], self.eps)
        return x2 + swiglu(n2 @ b["gate"], n2 @ b["up"]) @ b["down"]

    def forward(self, tokens, start):
        """Logits [S, vocab] for tokens at positions start.. (cache updated)."""
        x = self.E[np.asarray(tokens)]
        for l in range(self.L):
            x = self._layer(l, x, start)
        return rmsnorm(x, self.gF, self.eps) @ self.head

    def generate_greedy(self, prompt, max_tokens, teacher=None):
        """generateGGUF with temperature 0 (gguf_cache.js:309-371); argmax
        keeps the first maximum (generate.js:70-76).  With `teacher`, step i
        consumes teacher[i] instead of the oracle's own token (teacher
        forcing), and the logits of every step are returned."""
        self.reset()
        n = len(prompt)
        logits = [self.forward(prompt, 0)[-1]]
        toks = [int(np.argmax(logits[-1]))]
        for i in range(1, max_tokens):
            pos = n + i - 1
            if pos >= self.max_seq:
                break
            feed = toks[-1] if teacher is None else teacher[i - 1]
            logits.append(self.forward([feed], pos)[0])
            toks.append(int(np.argmax(logits[-1])))
        return toks, logits
