"""KV-cached Llama forward and generation -- mirror of src/gguf_cache.js.

Per layer the decode step is five kernels (the reference issues ~16
blocking submissions per layer, gguf_cache.js:116-172):
  1. RMSNorm(x) fused into the q|k|v GEMV                 -> qkv
  2. RoPE + KV-cache append + GQA softmax attention       -> attn
  3. o-proj GEMV with the residual add fused              -> x2 = x + o
  4. RMSNorm(x2) fused into the gate|up GEMV, SwiGLU fused -> h
  5. down GEMV with the residual add fused                -> x = x2 + down
then the LM head (final RMSNorm fused) and a device-side greedy step
(argmax, embedding of the chosen token, position advance).  The position
lives in device memory, so the greedy decode step is captured once as a HIP
graph and replayed.

Single-row steps on models whose linears have tile layouts (Q4_0, Q4_1,
Q5_0, Q4_K, Q6_K) pass activations between kernels as "acts" (the vector
already in the GEMV's MFMA operand form, with per-8-element sums and sums of
squares; smith_linear_q4_0_t_act / smith_linear_gguf_tiles_act): every producer -- embedding,
o-proj, gate|up, down -- writes the act its consumer reads, with the next
RMSNorm's gamma folded in, and the consumer applies the norm's rms as one
scalar.  Attention leaves its key-split partials to the o-projection, which
combines them while it builds its operand (smith_attention_parts +
smith_linear_*_attn; head_dim % 32 == 0, else attention writes an act).
Prefill rows (M > 1) take the f32 path.
"""
import os

import numpy as np

from . import device

# SMITH_DECODE_GRAPH=0 runs every decode step eagerly (kernel-level profilers
# that cannot trace graph replays); results are identical.
USE_GRAPH = os.environ.get("SMITH_DECODE_GRAPH", "1") != "0"
# Q4_0 / Q6_K LM head and the greedy step in one launch (smith_lmhead_*_greedy)
FUSED_GREEDY = os.environ.get("SMITH_FUSED_GREEDY", "1") != "0"
PREP_NEXT = os.environ.get("SMITH_PREP_NEXT", "1") != "0"

PREFILL_CHUNK = 256


def _chunk_rows(cfg):
    """Rows per prefill launch (bounded by the activation buffers)."""
    return PREFILL_CHUNK


def createGGUFCache(config):
    """gguf_cache.js:14-28: per layer k, v of [kvHeads, maxSeqLen, headDim]."""
    from .gguf_loader import DeviceArray
    shape = (config["numKVHeads"], config["maxSeqLen"], config["headDim"])
    caches = [{"k": DeviceArray(shape), "v": DeviceArray(shape), "len": 0} for _ in range(config["numLayers"])]
    return caches


def resetCache(caches):
    """gguf_cache.js:31-33."""
    for c in caches:
        c["len"] = 0


class _Engine:
    """Activation buffers and the device-side step state of one model."""

    def __init__(self, model):
        from .gguf_loader import DeviceArray
        cfg = model["config"]
        self.cfg = cfg
        R = PREFILL_CHUNK
        dim, kv, ffn = cfg["dim"], cfg["kvDim"], cfg["ffnDim"]
        self.qkv_ld = dim + 2 * kv
        self.x = DeviceArray((R, dim))
        self.x2 = DeviceArray((R, dim))
        self.qkv = DeviceArray((R, self.qkv_ld))
        self.attn = DeviceArray((R, dim))
        self.h = DeviceArray((R, ffn))
        self.logits = DeviceArray((cfg["vocabSize"],))
        self.pos = DeviceArray((1,), np.int32)
        self.count = DeviceArray((1,), np.int32)
        self.tokens = DeviceArray((cfg["maxSeqLen"] + 1,), np.int32)
        self.tok_in = DeviceArray((R,), np.int32)
        self.graph = None
        self.graph_caches = None
        hd = cfg["headDim"]
        self.use_act = (all(b[k].has_act for b in model["blocks"] for k in ("qkv", "outProj", "gateUp", "ffnDown"))
                        and dim % 32 == 0 and ffn % 32 == 0 and hd % 8 == 0 and cfg["numHeads"] * hd == dim)

        def act(K):
            return DeviceArray((K * 4 + K // 8 * 12,), np.uint8)
        if self.use_act:
            self.act_x, self.act_a, self.act_x2, self.act_h = act(dim), act(dim), act(dim), act(ffn)
        # attention partials combined by the o-projection (hd % 32 == 0)
        self.use_parts = self.use_act and hd % 32 == 0 and hd <= 128
        if self.use_parts:
            self.att_parts = DeviceArray((cfg["numHeads"] * 8 * 132,))
            # cos / sin of the current decode position, written by the greedy
            # step for the next one (tag -1: none yet, the attention reads the table)
            self.rope_row = DeviceArray((4 + cfg["numHeads"] * hd + cfg["numKVHeads"] * hd,))
            device.check(device.lib.smith_set_i32(device.ops_ctx(), self.rope_row.ptr, -1), "rope row")

    def set_pos(self, p):
        device.check(device.lib.smith_set_i32(device.ops_ctx(), self.pos.ptr, int(p)), "set_pos")

    def layers(self, model, caches, M):
        """Run every layer on rows x[0:M] at positions *pos .. *pos+M-1."""
        if M == 1 and self.use_act:
            return self.layers_act(model, caches)
        cfg, ctx, eps = self.cfg, device.ops_ctx(), model["normEps"]
        dim = cfg["dim"]
        x, x2, qkv, attn, h = self.x.ptr, self.x2.ptr, self.qkv.ptr, self.attn.ptr, self.h.ptr
        rope = model["rope"]
        blocks = model["blocks"]
        # each residual / SwiGLU GEMM's K-split reduce also writes the next
        # GEMM's f16 operand (with its RMSNorm), which then skips its prep
        hint = PREP_NEXT and M > 1
        for li, (blk, cache) in enumerate(zip(blocks, caches)):
            blk["qkv"](x, qkv, M, gamma=blk["ln1Gamma"].ptr, eps=eps)
            if hint:
                device.check(device.lib.smith_prep_next(ctx, None, 0.0), "prep hint")
            device.check(device.lib.smith_attention(
                ctx, qkv, self.qkv_ld, self.pos.ptr, M, cfg["numHeads"], cfg["numKVHeads"], cfg["headDim"],
                rope["cos"].ptr, rope["sin"].ptr, rope["cos"].shape[0], cache["k"].ptr, cache["v"].ptr, cfg["maxSeqLen"], attn, None),
                "attention")
            if hint:
                device.check(device.lib.smith_prep_next(ctx, blk["ln2Gamma"].ptr, eps), "prep hint")
            blk["outProj"](attn, x2, M, resid=x, epilogue=1)
            if hint:
                device.check(device.lib.smith_prep_next(ctx, None, 0.0), "prep hint")
            blk["gateUp"](x2, h, M, gamma=blk["ln2Gamma"].ptr, eps=eps, epilogue=2)
            if hint and li + 1 < len(blocks):
                device.check(device.lib.smith_prep_next(ctx, blocks[li + 1]["ln1Gamma"].ptr, eps), "prep hint")
            blk["ffnDown"](h, x, M, resid=x2, epilogue=1)
        del dim

    def layers_act(self, model, caches):
        """One row through every layer on acts; needs self.act_x written (with
        layer 0's attention-norm gamma) by the embedding of the row."""
        cfg, ctx, eps = self.cfg, device.ops_ctx(), model["normEps"]
        x, x2, qkv, attn = self.x.ptr, self.x2.ptr, self.qkv.ptr, self.attn.ptr
        ax, aa, ax2, ah = self.act_x.ptr, self.act_a.ptr, self.act_x2.ptr, self.act_h.ptr
        rope = model["rope"]
        blocks = model["blocks"]
        for li, (blk, cache) in enumerate(zip(blocks, caches)):
            blk["qkv"].act(ax, True, eps, qkv)
            if self.use_parts:
                parts = self.att_parts.ptr
                device.check(device.lib.smith_attention_parts(
                    ctx, qkv, self.pos.ptr, cfg["numHeads"], cfg["numKVHeads"], cfg["headDim"], rope["cos"].ptr,
                    rope["sin"].ptr, rope["sin"].shape[0], self.rope_row.ptr, cache["k"].ptr, cache["v"].ptr, cfg["maxSeqLen"], parts),
                    "attention")
                blk["outProj"].attn(parts, self.pos.ptr, cfg["headDim"], x2, x, 1, ax2, blk["ln2Gamma"].ptr)
            else:
                device.check(device.lib.smith_attention(
                    ctx, qkv, self.qkv_ld, self.pos.ptr, 1, cfg["numHeads"], cfg["numKVHeads"], cfg["headDim"],
                    rope["cos"].ptr, rope["sin"].ptr, rope["cos"].shape[0], cache["k"].ptr, cache["v"].ptr, cfg["maxSeqLen"], attn, aa),
                    "attention")
                blk["outProj"].act(aa, False, 0.0, x2, resid=x, epilogue=1, act_out=ax2,
                                   gamma_out=blk["ln2Gamma"].ptr)
            blk["gateUp"].act(ax2, True, eps, None, epilogue=2, act_out=ah)
            last = li + 1 == len(blocks)
            blk["ffnDown"].act(ah, False, 0.0, x, resid=x2, epilogue=1, act_out=None if last else ax,
                               gamma_out=None if last else blocks[li + 1]["ln1Gamma"].ptr)

    def _act0(self, model):
        """(act, gamma) the embedding of a single decode row writes."""
        if not self.use_act:
            return None, None
        return self.act_x.ptr, model["blocks"][0]["ln1Gamma"].ptr

    def lm_head(self, model, x_ptr):
        """Final RMSNorm fused into the LM head (gguf_cache.js:174-184)."""
        cfg, ctx = self.cfg, device.ops_ctx()
        head, g, eps = model["lmHead"], model["lnFGamma"].ptr, model["normEps"]
        if head["kind"] == "q4_0_nb":
            rc = device.lib.smith_lmhead_q4_0_nb(ctx, x_ptr, g, eps, head["nib"].ptr, head["d"].ptr, self.logits.ptr,
                                                 cfg["dim"],
                                                 cfg["vocabSize"])
        elif head["kind"] == "q6_k_nb":
            rc = device.lib.smith_lmhead_q6_k_nb(ctx, x_ptr, g, eps, head["planes"].ptr, self.logits.ptr, cfg["dim"],
                                                 cfg["vocabSize"])
        elif head["kind"] == "f32_kn":
            rc = device.lib.smith_gemv_f32(ctx, x_ptr, g, eps, head["w"].ptr, self.logits.ptr, cfg["dim"],
                                           cfg["vocabSize"], 0)
        else:
            rc = device.lib.smith_gemv_f32(ctx, x_ptr, g, eps, model["embedding"].ptr, self.logits.ptr, cfg["dim"],
                                           cfg["vocabSize"], 1)
        device.check(rc, "lm head")

    def greedy_step(self, model):
        cfg = self.cfg
        a0, g0 = self._act0(model)
        rope, hd = model["rope"], cfg["headDim"]
        rr = self.rope_row.ptr if self.use_parts else None
        device.check(device.lib.smith_argmax_embed(device.ops_ctx(), self.logits.ptr, cfg["vocabSize"],
                                                   self.model_embedding, cfg["dim"], self.x.ptr, self.tokens.ptr,
                                                   self.count.ptr, self.pos.ptr, a0, g0, rope["cos"].ptr,
                                                   rope["sin"].ptr, rope["cos"].shape[0], cfg["numHeads"] * hd,
                                                   cfg["numKVHeads"] * hd, rr), "argmax")

    def head_greedy(self, model):
        """LM head on x, then the greedy step: one launch for a Q4_0 or Q6_K
        head."""
        head = model["lmHead"]
        if not (FUSED_GREEDY and head["kind"] in ("q4_0_nb", "q6_k_nb")):
            self.lm_head(model, self.x.ptr)
            self.greedy_step(model)
            return
        cfg = self.cfg
        a0, g0 = self._act0(model)
        rope, hd = model["rope"], cfg["headDim"]
        rr = self.rope_row.ptr if self.use_parts else None
        tail = (self.logits.ptr, cfg["dim"], cfg["vocabSize"], self.model_embedding, self.x.ptr, self.tokens.ptr,
                self.count.ptr, self.pos.ptr, a0, g0, rope["cos"].ptr, rope["sin"].ptr, rope["cos"].shape[0],
                cfg["numHeads"] * hd, cfg["numKVHeads"] * hd, rr)
        ctx, g, eps = device.ops_ctx(), model["lnFGamma"].ptr, model["normEps"]
        if head["kind"] == "q4_0_nb":
            rc = device.lib.smith_lmhead_q4_0_greedy(ctx, self.x.ptr, g, eps, head["nib"].ptr, head["d"].ptr, *tail)
        else:
            rc = device.lib.smith_lmhead_q6_k_greedy(ctx, self.x.ptr, g, eps, head["planes"].ptr, *tail)
        device.check(rc, "lm head + greedy step")

    def embed(self, model, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        device.upload(self.tok_in.ptr, t)
        a0, g0 = self._act0(model) if len(t) == 1 else (None, None)
        device.check(device.lib.smith_embed(device.ops_ctx(), model["embedding"].ptr, self.tok_in.ptr, self.x.ptr,
                                            len(t), self.cfg["dim"], a0, g0), "embed")

    def prefill(self, model, tokens, caches, all_logits=False):
        """Prompt rows in chunks of <= 256 (attention keeps a chunk's keys in
        LDS); returns the logits of every row if asked, else of the last."""
        n = len(tokens)
        rows = []
        step = _chunk_rows(self.cfg)
        for r0 in range(0, n, step):
            r1 = min(n, r0 + step)
            self.embed(model, tokens[r0:r1])
            self.set_pos(r0)
            self.layers(model, caches, r1 - r0)
            if all_logits:
                for r in range(r1 - r0):
                    self.lm_head(model, self.x.ptr + r * self.cfg["dim"] * 4)
                    rows.append(self.logits.numpy().copy())
        last = (n - 1) % step
        if not all_logits:
            self.lm_head(model, self.x.ptr + last * self.cfg["dim"] * 4)
        for c in caches:
            c["len"] = n
        return np.stack(rows) if all_logits else None


def _engine(model):
    if "_engine" not in model:
        model["_engine"] = _Engine(model)
        model["_engine"].model_embedding = model["embedding"].ptr
    return model["_engine"]


def _check_rope_range(cfg, last_pos):
    # whole-row RoPE reads table entry pos*(W/2) + i < maxSeqLen*headDim/2 for
    # W = dim (q); beyond that the reference reads past its table
    if (last_pos + 1) * (cfg["dim"] // 2) > cfg["maxSeqLen"] * cfg["headDim"] // 2:
        raise ValueError("position %d: whole-row RoPE indexing needs context_length >= %d"
                         % (last_pos, (last_pos + 1) * cfg["dim"] // cfg["headDim"]))


def forwardLlamaCachedPrefill(model, tokenIds, caches):
    """gguf_cache.js:191-265; returns {'logits': [seqLen, vocab]} (host)."""
    e = _engine(model)
    _check_rope_range(e.cfg, len(tokenIds) - 1)
    logits = e.prefill(model, list(tokenIds), caches, all_logits=True)
    return {"logits": logits}


def forwardLlamaCachedDecode(model, tokenId, position, caches):
    """gguf_cache.js:109-187; returns {'logits': [1, vocab]} (host)."""
    e = _engine(model)
    _check_rope_range(e.cfg, position)
    e.embed(model, [tokenId])
    e.set_pos(position)
    e.layers(model, caches, 1)
    e.lm_head(model, e.x.ptr)
    for c in caches:
        c["len"] = position + 1
    return {"logits": e.logits.numpy()[None, :].copy()}


# --- host sampling (generate.js:11-70), used when temperature > 0 or a
#     repetition penalty is set; greedy decoding runs entirely on the device

def _sample(logits, generated, cfg, rng):
    t, k, p, rp = cfg["temperature"], cfg["topK"], cfg["topP"], cfg["repetitionPenalty"]
    lg = np.array(logits, dtype=np.float64)
    if rp > 1:
        for i in set(generated):
            if i < lg.size:
                lg[i] = lg[i] / rp if lg[i] > 0 else lg[i] * rp
    if t not in (0, 1):
        lg = lg / t
    if 0 < k < lg.size:
        thr = np.sort(lg)[::-1][k - 1]
        lg = np.where(lg >= thr, lg, -np.inf)
    if p < 1:
        order = np.argsort(-lg, kind="stable")
        pr = np.exp(lg - lg.max())
        pr /= pr.sum()
        keep = np.zeros(lg.size, bool)
        cum = 0.0
        for i in order:
            cum += pr[i]
            keep[i] = True
            if cum >= p:
                break
        lg = np.where(keep, lg, -np.inf)
    if t == 0:
        return int(np.argmax(lg))
    pr = np.exp(lg - lg.max())
    pr /= pr.sum()
    r = rng.random()
    c = np.cumsum(pr)
    idx = int(np.searchsorted(c, r, side="right"))
    return min(idx, lg.size - 1)


def generateGGUF(model, promptIds, config=None, callbacks=None):
    """gguf_cache.js:309-371: prefill, then one token per step; returns
    [...prompt, ...generated]."""
    config = dict(config or {})
    callbacks = callbacks or {}
    cfg = dict(maxTokens=config.get("maxTokens", 50), temperature=config.get("temperature", 1.0),
               topK=config.get("topK", 0), topP=config.get("topP", 1.0),
               repetitionPenalty=config.get("repetitionPenalty", 1.0))
    eos = config.get("eosToken")
    on_token = callbacks.get("onToken")
    e = _engine(model)
    mcfg = e.cfg
    generated = [int(t) for t in promptIds]
    prompt = generated[-mcfg["maxSeqLen"]:] if len(generated) > mcfg["maxSeqLen"] else generated
    n = len(prompt)
    last_pos = min(n + cfg["maxTokens"] - 2, mcfg["maxSeqLen"] - 1)
    _check_rope_range(mcfg, max(n - 1, last_pos))
    caches = model.get("_gen_caches")
    if caches is None:
        caches = model["_gen_caches"] = createGGUFCache(mcfg)
    resetCache(caches)
    greedy = cfg["temperature"] == 0 and cfg["repetitionPenalty"] <= 1
    rng = np.random.default_rng(config.get("seed"))

    e.prefill(model, prompt, caches)
    if greedy:
        device.check(device.lib.smith_set_i32(device.ops_ctx(), e.count.ptr, 0), "count")
        e.set_pos(n - 1)
        e.greedy_step(model)  # token 1; pos -> n; x = E[token]
        steps = 0
        for i in range(1, cfg["maxTokens"]):
            if n + i - 1 >= mcfg["maxSeqLen"]:
                break
            steps += 1
        sync_each = eos is not None or on_token is not None
        tok = int(e.tokens.numpy()[0]) if sync_each else None
        if sync_each:
            generated.append(tok)
            if eos is not None and tok == eos:
                return generated
            if on_token and on_token(tok, 1):
                return generated
        graph = None
        for i in range(1, steps + 1):
            if USE_GRAPH and graph is None and i >= 2:
                graph = _decode_graph(model, e, caches)
            if graph is not None:
                device.check(device.lib.smith_graph_launch(device.ops_ctx(), graph), "graph launch")
            else:
                e.layers(model, caches, 1)
                e.head_greedy(model)
            if sync_each:
                tok = int(e.tokens.numpy()[i])
                generated.append(tok)
                if eos is not None and tok == eos:
                    break
                if on_token and on_token(tok, i + 1):
                    break
        if not sync_each:
            generated.extend(int(t) for t in e.tokens.numpy()[:steps + 1])
        for c in caches:
            c["len"] = n + steps
        return generated

    # sampling path: logits to the host each step (generate.js:sampleToken CPU path)
    tok = _sample(e.logits.numpy(), generated, cfg, rng)
    generated.append(tok)
    if eos is not None and tok == eos:
        return generated
    if on_token and on_token(tok, 1):
        return generated
    for i in range(1, cfg["maxTokens"]):
        position = n + i - 1
        if position >= mcfg["maxSeqLen"]:
            break
        logits = forwardLlamaCachedDecode(model, generated[-1], position, caches)["logits"][0]
        tok = _sample(logits, generated, cfg, rng)
        generated.append(tok)
        if eos is not None and tok == eos:
            break
        if on_token and on_token(tok, i + 1):
            break
    return generated


def _decode_graph(model, e, caches):
    """Capture one greedy decode step (layers, LM head, argmax/embed/advance);
    every argument is fixed, the position and token count live on the device."""
    if e.graph is not None and e.graph_caches is caches:
        return e.graph
    if e.graph is not None:
        device.lib.smith_graph_destroy(e.graph)
        e.graph = None
    ctx = device.ops_ctx()
    device.check(device.lib.smith_graph_begin(ctx), "graph begin")
    try:
        e.layers(model, caches, 1)
        e.head_greedy(model)
    finally:
        g = device.lib.smith_graph_end(ctx)
    if not g:
        device.check(-1, "graph end")
    e.graph, e.graph_caches = g, caches
    return g
