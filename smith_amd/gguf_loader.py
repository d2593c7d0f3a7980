"""loadGGUF on MI355X -- mirror of src/gguf_loader.js for the Llama path.

Differences from the reference, all on purpose: the
reference dequantizes every tensor to f32 at load (gguf_loader.js:236) and
runs f32 GEMMs; here Q4_0 / Q4_1 / Q5_0 / Q8_0 / Q4_K / Q6_K linear weights
stay quantized on the device and `linear` runs the quantized GEMV.  The
blocks are only moved (never changed) into the kernels' layouts:
  * q|k|v of a layer side by side in one buffer (one GEMV per layer) when
    they share a block type, else three GEMVs writing the column ranges of
    the same q|k|v rows (Q4_K_M files keep attn_v in Q6_K),
  * gate/up interleaved column by column (the SwiGLU epilogue pairs them),
  * output.weight kept as stored: the reference reads its flat data as
    lmHead[dim][vocab] (gguf_loader.js:240-259 only transposes paths ending
    in ".weight"), so its Q4_0 blocks run along the vocab axis and it gets
    its own GEMV (smith_lmhead_q4_0_nb).
Norms and the token embedding are f32 on the device (a quantized
token_embd, or an output.weight of a type without its own GEMV, is decoded
on the device by smith_dequantize_gguf, bit-identical to dequantizeTensor).
"""
import numpy as np

from . import device
from . import gguf as G
from .gguf_cache import (createGGUFCache, forwardLlamaCachedDecode, forwardLlamaCachedPrefill, generateGGUF,
                         resetCache)

LLAMA_MAP = {
    "token_embd.weight": "embedding.tokenWeight",
    "output_norm.weight": "lnFGamma",
    "output.weight": "lmHead",
    "blk.{L}.attn_norm.weight": "blocks.{L}.ln1Gamma",
    "blk.{L}.ffn_norm.weight": "blocks.{L}.ln2Gamma",
    "blk.{L}.attn_q.weight": "blocks.{L}.mha.qProj.weight",
    "blk.{L}.attn_k.weight": "blocks.{L}.mha.kProj.weight",
    "blk.{L}.attn_v.weight": "blocks.{L}.mha.vProj.weight",
    "blk.{L}.attn_output.weight": "blocks.{L}.mha.outProj.weight",
    "blk.{L}.ffn_gate.weight": "blocks.{L}.ffnGate.weight",
    "blk.{L}.ffn_up.weight": "blocks.{L}.ffnUp.weight",
    "blk.{L}.ffn_down.weight": "blocks.{L}.ffnDown.weight",
}


# gguf_loader.js:48-84: name maps of the other architectures (their weights
# are only loaded; forward is Llama-only, gguf_loader.js:394-396)
PHI_MAP = {
    "token_embd.weight": "embedding.tokenWeight",
    "output_norm.weight": "lnFGamma",
    "output_norm.bias": "lnFBeta",
    "output.weight": "lmHead",
    "blk.{L}.attn_norm.weight": "blocks.{L}.ln1Gamma",
    "blk.{L}.attn_norm.bias": "blocks.{L}.ln1Beta",
    "blk.{L}.ffn_norm.weight": "blocks.{L}.ln2Gamma",
    "blk.{L}.ffn_norm.bias": "blocks.{L}.ln2Beta",
    "blk.{L}.attn_qkv.weight": "blocks.{L}.mha.qkvProj.weight",
    "blk.{L}.attn_qkv.bias": "blocks.{L}.mha.qkvProj.bias",
    "blk.{L}.attn_output.weight": "blocks.{L}.mha.outProj.weight",
    "blk.{L}.attn_output.bias": "blocks.{L}.mha.outProj.bias",
    "blk.{L}.ffn_up.weight": "blocks.{L}.ffn1.weight",
    "blk.{L}.ffn_up.bias": "blocks.{L}.ffn1.bias",
    "blk.{L}.ffn_down.weight": "blocks.{L}.ffn2.weight",
    "blk.{L}.ffn_down.bias": "blocks.{L}.ffn2.bias",
}
GPT2_MAP = dict(PHI_MAP)
del GPT2_MAP["output.weight"]
GPT2_MAP["position_embd.weight"] = "embedding.posWeight"
GPT2_MAP["blk.{L}.attn_qkv.weight"] = "blocks.{L}.mha.qkvFused.weight"
GPT2_MAP["blk.{L}.attn_qkv.bias"] = "blocks.{L}.mha.qkvFused.bias"


def getWeightMap(arch):
    """gguf_loader.js:86-91."""
    if arch == "llama":
        return LLAMA_MAP
    if arch in ("phi", "phi2", "phi3"):
        return PHI_MAP
    if arch == "gpt2":
        return GPT2_MAP
    raise ValueError("Unsupported GGUF architecture: %s" % arch)


def resolveWeight(name, weightMap):
    """gguf_loader.js:94-109."""
    if name in weightMap:
        return weightMap[name]
    parts = name.split(".", 2)
    if len(parts) == 3 and parts[0] == "blk" and parts[1].isdigit():
        pat = "blk.{L}." + parts[2]
        if pat in weightMap:
            return weightMap[pat].replace("{L}", parts[1])
    return None


def precomputeRoPE(dim, maxSeqLen, freqBase=10000):
    """ops/rope.js:10-30: f32 inverse frequencies, f64 angles, f32 cos/sin,
    flat [maxSeqLen, dim/2]."""
    half = dim // 2
    freqs = (1.0 / np.power(float(freqBase), (2.0 * np.arange(half)) / dim)).astype(np.float32)
    ang = np.arange(maxSeqLen, dtype=np.float64)[:, None] * freqs.astype(np.float64)[None, :]
    return np.cos(ang).astype(np.float32).ravel(), np.sin(ang).astype(np.float32).ravel()


class DeviceArray:
    """A device buffer with a shape (f32 unless stated)."""

    def __init__(self, shape, dtype=np.float32, nbytes=None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(nbytes if nbytes is not None else np.prod(self.shape) * self.dtype.itemsize)
        self.ptr = device.alloc(max(self.nbytes, 4))

    @classmethod
    def from_host(cls, arr, dtype=np.float32):
        a = np.ascontiguousarray(arr, dtype=dtype)
        d = cls(a.shape, dtype)
        device.upload(d.ptr, a)
        return d

    def numpy(self):
        return device.download(self.ptr, self.nbytes, self.dtype).reshape(self.shape)


GT_TYPES = {G.GGML_TYPE[t] for t in ("Q4_0", "Q4_1", "Q5_0", "Q4_K", "Q6_K")}


class QLinear:
    """A quantized linear weight on the device: y = x . W with W [in=K, out=N].
    kind 'q4_0t': tile-major nib/d planes; kind 'q8': matmulQ8 records;
    kind 'gt': the tile planes of another GGUF block type (ggml_type)."""

    def __init__(self, kind, K, N, a, b=None, ggml_type=None):
        self.kind, self.K, self.N, self.a, self.b, self.ggml_type = kind, K, N, a, b, ggml_type

    def __call__(self, x_ptr, out_ptr, M, gamma=None, eps=0.0, resid=None, epilogue=0):
        ctx = device.ops_ctx()
        if self.kind == "q4_0t":
            rc = device.lib.smith_linear_q4_0_t(ctx, x_ptr, self.a.ptr, self.b.ptr, out_ptr, M, self.N, self.K,
                                                gamma, eps, resid, epilogue)
        elif self.kind == "gt":
            rc = device.lib.smith_linear_gguf_tiles(ctx, self.ggml_type, x_ptr, self.a.ptr, out_ptr, M, self.N,
                                                    self.K, gamma, eps, resid, epilogue)
        else:
            rc = device.lib.smith_linear_q8(ctx, x_ptr, self.a.ptr, out_ptr, M, self.N, self.K, gamma, eps,
                                            resid, epilogue)
        device.check(rc, "linear")

    @property
    def has_act(self):
        return self.kind in ("q4_0t", "gt")

    def act(self, act_in, norm, eps, out_ptr, resid=None, epilogue=0, act_out=None, gamma_out=None):
        """Single-row linear on a prepared activation (smith_linear_*_act)."""
        if self.kind == "q4_0t":
            rc = device.lib.smith_linear_q4_0_t_act(device.ops_ctx(), act_in, 1 if norm else 0, eps, self.a.ptr,
                                                    self.b.ptr, out_ptr, self.N, self.K, resid, epilogue, act_out,
                                                    gamma_out)
        else:
            rc = device.lib.smith_linear_gguf_tiles_act(device.ops_ctx(), self.ggml_type, act_in, 1 if norm else 0,
                                                        eps, self.a.ptr, out_ptr, self.N, self.K, resid, epilogue,
                                                        act_out, gamma_out)
        device.check(rc, "linear (act)")

    def attn(self, parts, pos_ptr, head_dim, out_ptr, resid, epilogue, act_out, gamma_out):
        """Single-row linear on attention split partials (smith_linear_*_attn)."""
        ctx = device.ops_ctx()
        if self.kind == "q4_0t":
            rc = device.lib.smith_linear_q4_0_t_attn(ctx, parts, pos_ptr, head_dim, self.a.ptr, self.b.ptr, out_ptr,
                                                     self.N, self.K, resid, epilogue, act_out, gamma_out)
        else:
            rc = device.lib.smith_linear_gguf_tiles_attn(ctx, self.ggml_type, parts, pos_ptr, head_dim, self.a.ptr,
                                                         out_ptr, self.N, self.K, resid, epilogue, act_out, gamma_out)
        device.check(rc, "o-proj (attention partials)")


class QGroup:
    """Linears of different block types sharing one input and writing the
    column ranges [off, off + N_i) of one [M, N] output (q|k|v)."""

    def __init__(self, parts):
        self.parts = parts  # [(QLinear, column offset)]
        self.K = parts[0][0].K
        self.N = sum(q.N for q, _ in parts)
        self.kind = "group"
        self._tmp = None
        # one launch for two tile-plane runs with a two-format kernel
        self.pair = (len(parts) == 2 and all(q.kind == "gt" for q, _ in parts)
                     and bool(device.lib.smith_gguf_tiles_pair_ok(parts[0][0].ggml_type, parts[1][0].ggml_type)))

    @property
    def has_act(self):
        return all(q.has_act for q, _ in self.parts)

    def __call__(self, x_ptr, out_ptr, M, gamma=None, eps=0.0, resid=None, epilogue=0):
        if resid is not None or epilogue:
            raise NotImplementedError("epilogues on a mixed-type linear group")
        if M == 1:
            for q, off in self.parts:
                q(x_ptr, out_ptr + off * 4, 1, gamma, eps)
            return
        need = M * max(q.N for q, _ in self.parts) * 4
        if self._tmp is None or self._tmp.nbytes < need:
            self._tmp = DeviceArray((need // 4,))
        ctx = device.ops_ctx()
        for q, off in self.parts:
            q(x_ptr, self._tmp.ptr, M, gamma, eps)
            device.check(device.lib.smith_copy_2d(ctx, out_ptr + off * 4, self.N * 4, self._tmp.ptr, q.N * 4, q.N * 4,
                                                  M), "group copy")

    def act(self, act_in, norm, eps, out_ptr, resid=None, epilogue=0, act_out=None, gamma_out=None):
        if resid is not None or epilogue or act_out is not None:
            raise NotImplementedError("epilogues on a mixed-type linear group")
        if self.pair:
            (q1, _), (q2, _) = self.parts
            device.check(device.lib.smith_linear_gguf_tiles_pair_act(
                device.ops_ctx(), q1.ggml_type, q1.a.ptr, q1.N, q2.ggml_type, q2.a.ptr, q2.N, act_in,
                1 if norm else 0, eps, out_ptr, self.K), "linear pair (act)")
            return
        for q, off in self.parts:
            q.act(act_in, norm, eps, out_ptr + off * 4)


def _pack_group(parsed, infos, K, cols, interleave, gt_q4_0=False):
    """Repack one or more [out, in] quantized weights into one device buffer:
    side by side (interleave=False) or column-interleaved.  Weights of
    different block types side by side become a QGroup of same-type runs,
    every run in tile planes (Q4_0 included: gt_q4_0) so that a two-run
    group takes the two-format kernel."""
    types = [i["type"] for i in infos]
    if len(set(types)) != 1:
        if interleave:
            raise NotImplementedError("interleaved weights of different GGML types (%s)"
                                      % ", ".join(G.GGML_TYPE_NAME.get(t, str(t)) for t in types))
        # runs of equal type stay fused (q|k of Q4_K, v of Q6_K)
        parts, off, i = [], 0, 0
        while i < len(infos):
            j = i
            while j < len(infos) and types[j] == types[i]:
                j += 1
            run_cols = cols[i:j]
            parts.append((_pack_group(parsed, infos[i:j], K, run_cols, False, gt_q4_0=True), off))
            off += sum(run_cols)
            i = j
        return QGroup(parts)
    t = types[0]
    Ntot = sum(cols)
    Gk = K // 32
    ctx = device.ops_ctx()
    dsc = None
    if t == G.GGML_TYPE["Q4_0"] and not gt_q4_0:
        nib = DeviceArray((Gk * Ntot * 16,), np.uint8)
        dsc = DeviceArray((Gk * Ntot,), np.uint16)
        kind = "q4_0t"
    elif t == G.GGML_TYPE["Q8_0"]:
        nib = DeviceArray((Gk * Ntot * 34,), np.uint8)
        kind = "q8"
    elif t in GT_TYPES:
        nbytes = int(device.lib.smith_gguf_tiles_bytes(t, Ntot, K))
        if not nbytes:
            raise NotImplementedError("%s weight [%d, %d]: needs out %% 16 == 0 and in %% %d == 0"
                                      % (G.GGML_TYPE_NAME[t], Ntot, K, 256 if t in (12, 14) else 32))
        nib = DeviceArray((nbytes,), np.uint8)
        kind = "gt"
    else:
        raise NotImplementedError("linear weight type %s is not on the quantized path "
                                  "(Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q6_K)" % G.GGML_TYPE_NAME.get(t, t))
    off = 0
    for j, (info, n) in enumerate(zip(infos, cols)):
        raw = G.readTensorData(parsed, info)
        src = DeviceArray.from_host(np.asarray(raw), np.uint8)
        n_off, stride = (j, len(infos)) if interleave else (off, 1)
        if kind == "q4_0t":
            rc = device.lib.smith_repack_q4_0_t_into(ctx, src.ptr, nib.ptr, dsc.ptr, n, K, n_off, stride, Ntot)
        elif kind == "gt":
            rc = device.lib.smith_repack_gguf_tiles_into(ctx, t, src.ptr, nib.ptr, n, K, n_off, stride, Ntot)
        else:
            rc = device.lib.smith_repack_q8_0_into(ctx, src.ptr, nib.ptr, n, K, n_off, stride, Ntot)
        device.check(rc, "repack %s" % info["name"])
        device.sync()
        device.release_buffer(src.ptr)
        off += n
    return QLinear(kind, K, Ntot, nib, dsc, ggml_type=t)


def device_f32(parsed, info):
    """Any dequantizable tensor as an f32 device array (dequantizeTensor,
    src/gguf.js:343-394, on the device)."""
    numel = int(np.prod(info["shape"]))
    out = DeviceArray((numel,))
    raw = DeviceArray.from_host(np.asarray(G.readTensorData(parsed, info)), np.uint8)
    device.check(device.lib.smith_dequantize_gguf(device.ops_ctx(), info["type"], raw.ptr, out.ptr, numel),
                 "dequantize %s" % info["name"])
    device.sync()
    device.release_buffer(raw.ptr)
    return out


def createGGUFModel(config):
    """gguf_loader.js:151-212: derived sizes and the RoPE tables."""
    dim, nH = config["dim"], config["numHeads"]
    headDim = dim // nH
    kvHeads = config["numKVHeads"] or nH
    ffn = config["ffnDim"] or int(round(dim * 8 / 3 / 256) * 256)
    cfg = dict(config, headDim=headDim, kvDim=kvHeads * headDim, ffnDim=ffn, numKVHeads=kvHeads)
    cos, sin = precomputeRoPE(headDim, config["maxSeqLen"], config["ropeFreqBase"])
    return {"config": cfg, "arch": config["arch"], "normEps": float(config["normEps"]),
            "rope": {"cos": DeviceArray.from_host(cos), "sin": DeviceArray.from_host(sin)},
            "blocks": [{} for _ in range(config["numLayers"])]}


def loadWeights(parsed, model):
    """gguf_loader.js:216-273 with the quantized blocks kept (see module doc)."""
    cfg = model["config"]
    wmap = getWeightMap(model["arch"])
    dim, kvDim, ffn, vocab = cfg["dim"], cfg["kvDim"], cfg["ffnDim"], cfg["vocabSize"]
    by_path, loaded, skipped = {}, [], []
    for info in parsed["tensors"]:
        path = resolveWeight(info["name"], wmap)
        if path is None:
            skipped.append(info["name"])
            continue
        by_path[path] = info
        loaded.append(info["name"])

    def expect_linear(info, n_in, n_out):
        shp = info["shape"]
        if len(shp) != 2 or int(np.prod(shp)) != n_in * n_out:
            raise ValueError("%s: shape %s, expected %d x %d" % (info["name"], shp, n_out, n_in))
        rows, cols = shp
        if not (cols == n_in and rows == n_out):
            # listed [in, out]: the reference copies the flat data untransposed
            # (gguf_loader.js:254-256), i.e. blocks along out -- not supported
            raise NotImplementedError("%s is listed [in, out]; only [out, in] listings are on the quantized path"
                                      % info["name"])

    def dense(path, n):
        info = by_path.get(path)
        if info is None:
            return DeviceArray.from_host(np.ones(n, np.float32))  # createGGUFModel default (T.ones)
        return DeviceArray.from_host(G.dense_f32(parsed, info).reshape(n))

    E = by_path.get("embedding.tokenWeight")
    if E is None:
        raise ValueError("token_embd.weight missing")
    if E["type"] in (G.GGML_TYPE["F32"], G.GGML_TYPE["F16"]):
        model["embedding"] = DeviceArray.from_host(G.dense_f32(parsed, E).reshape(vocab, dim))
    else:
        model["embedding"] = device_f32(parsed, E)
    for L, blk in enumerate(model["blocks"]):
        p = "blocks.%d." % L
        q, k, v = (by_path[p + "mha.%sProj.weight" % n] for n in ("q", "k", "v"))
        o = by_path[p + "mha.outProj.weight"]
        g, u, d = (by_path[p + n + ".weight"] for n in ("ffnGate", "ffnUp", "ffnDown"))
        for info, n_in, n_out in ((q, dim, dim), (k, dim, kvDim), (v, dim, kvDim), (o, dim, dim), (g, dim, ffn),
                                  (u, dim, ffn), (d, ffn, dim)):
            expect_linear(info, n_in, n_out)
        blk["ln1Gamma"] = dense(p + "ln1Gamma", dim)
        blk["ln2Gamma"] = dense(p + "ln2Gamma", dim)
        blk["qkv"] = _pack_group(parsed, [q, k, v], dim, [dim, kvDim, kvDim], interleave=False)
        blk["outProj"] = _pack_group(parsed, [o], dim, [dim], interleave=False)
        blk["gateUp"] = _pack_group(parsed, [g, u], dim, [ffn, ffn], interleave=True)
        blk["ffnDown"] = _pack_group(parsed, [d], ffn, [dim], interleave=False)
    model["lnFGamma"] = dense("lnFGamma", dim)
    head = by_path.get("lmHead")
    if head is None:
        # weight tying (gguf_loader.js:266-270): logits = x . E^T
        model["lmHead"] = {"kind": "tied"}
        model["weightTied"] = True
    elif head["type"] == G.GGML_TYPE["Q4_0"]:
        if vocab % 32:
            raise NotImplementedError("Q4_0 output.weight needs vocab % 32 == 0")
        raw = DeviceArray.from_host(np.asarray(G.readTensorData(parsed, head)), np.uint8)
        nibp = DeviceArray((dim * vocab // 2,), np.uint8)
        dscp = DeviceArray((dim * vocab // 32,), np.uint16)
        device.check(device.lib.smith_repack_lmhead_q4_0(device.ops_ctx(), raw.ptr, nibp.ptr, dscp.ptr, dim, vocab),
                     "repack output.weight")
        device.sync()
        device.release_buffer(raw.ptr)
        model["lmHead"] = {"kind": "q4_0_nb", "nib": nibp, "d": dscp}
    elif head["type"] in (G.GGML_TYPE["F32"], G.GGML_TYPE["F16"]):
        model["lmHead"] = {"kind": "f32_kn", "w": DeviceArray.from_host(G.dense_f32(parsed, head))}
    elif head["type"] == G.GGML_TYPE["Q6_K"] and vocab % 256 == 0 and dim % 16 == 0 and dim <= 8192:
        raw = DeviceArray.from_host(np.asarray(G.readTensorData(parsed, head)), np.uint8)
        planes = DeviceArray((int(device.lib.smith_lmhead_q6_k_bytes(dim, vocab)),), np.uint8)
        device.check(device.lib.smith_repack_lmhead_q6_k(device.ops_ctx(), raw.ptr, planes.ptr, dim, vocab),
                     "repack output.weight")
        device.sync()
        device.release_buffer(raw.ptr)
        model["lmHead"] = {"kind": "q6_k_nb", "planes": planes}
    else:
        # other block types: decoded once to the f32 [dim][vocab] the reference
        # builds (its blocks run along vocab, so no K-blocked GEMV applies)
        model["lmHead"] = {"kind": "f32_kn", "w": device_f32(parsed, head)}
    device.sync()
    return {"loaded": loaded, "skipped": skipped}


class GGUFModel(dict):
    """The object loadGGUF returns (gguf_loader.js:388-404)."""

    def __getattr__(self, k):
        try:
            return self[k]
        except KeyError:
            raise AttributeError(k)


def _load_other(parsed, config):
    """createGGUFModel + loadWeights (gguf_loader.js:151-273) for the
    non-Llama architectures, whose weights the reference loads but never
    runs: the same parameter set (q/k/v/out projections, ffn1/ffn2, the
    final norm's beta; no RoPE table for gpt2), the same loaded / skipped
    lists ("name → path (not found in model)" when the map names a parameter
    the model lacks), each loaded tensor decoded on the device and stored f32
    in the Smith shape (transposed when listed [out, in], :240-259), and
    weight tying when output.weight is absent (:266-270)."""
    dim, nH = config["dim"], config["numHeads"]
    hd = dim // nH
    kvd = (config["numKVHeads"] or nH) * hd
    ffn = config["ffnDim"] or int(round(dim * 8 / 3 / 256) * 256)
    vocab = config["vocabSize"]
    shapes = {"embedding.tokenWeight": (vocab, dim), "lnFGamma": (dim,), "lnFBeta": (dim,), "lmHead": (dim, vocab)}
    for L in range(config["numLayers"]):
        b = "blocks.%d." % L
        shapes.update({b + "ln1Gamma": (dim,), b + "ln2Gamma": (dim,), b + "mha.qProj.weight": (dim, dim),
                       b + "mha.kProj.weight": (dim, kvd), b + "mha.vProj.weight": (dim, kvd),
                       b + "mha.outProj.weight": (dim, dim), b + "ffn1.weight": (dim, ffn),
                       b + "ffn2.weight": (ffn, dim)})
    wmap = getWeightMap(config["arch"])
    params, loaded, skipped = {}, [], []
    for info in parsed["tensors"]:
        path = resolveWeight(info["name"], wmap)
        if path is None:
            skipped.append(info["name"])
            continue
        if path not in shapes:
            skipped.append("%s \u2192 %s (not found in model)" % (info["name"], path))
            continue
        flat = device_f32(parsed, info)
        shp = shapes[path]
        is_weight = path.endswith(".weight") and not any(t in path for t in ("embd", "norm", "Gamma"))
        if is_weight and len(info["shape"]) == 2 and tuple(shp) == (info["shape"][1], info["shape"][0]):
            rows, cols = info["shape"]
            host = flat.numpy().reshape(rows, cols).T
            device.release_buffer(flat.ptr)
            params[path] = DeviceArray.from_host(host)
        else:
            flat.shape = tuple(shp) if int(np.prod(shp)) == flat.shape[0] else flat.shape
            params[path] = flat
        loaded.append(info["name"])
    model = {"config": dict(config, headDim=hd, kvDim=kvd, ffnDim=ffn), "arch": config["arch"],
             "normEps": float(config["normEps"]), "params": params}
    if "output.weight" not in loaded:
        params["lmHead"] = params.get("embedding.tokenWeight")
        model["weightTied"] = True
    if config["arch"] != "gpt2":
        cos, sin = precomputeRoPE(hd, config["maxSeqLen"], config["ropeFreqBase"])
        model["rope"] = {"cos": DeviceArray.from_host(cos), "sin": DeviceArray.from_host(sin)}
    device.sync()
    return model, loaded, skipped


def loadGGUF(path):
    """gguf_loader.js:381-405."""
    parsed = G.loadGGUFFile(path)
    config = G.extractConfig(parsed["metadata"])
    if config["arch"] != "llama":
        model, loaded, skipped = _load_other(parsed, config)

        def unsupported(*_a, **_k):
            # the reference's forward throws this (gguf_loader.js:394-396); its
            # cached entry points fail on the missing Llama FFN for these models
            raise RuntimeError("Forward not implemented for %s via GGUF loader" % config["arch"])
        return GGUFModel(model=model, config=config, metadata=parsed["metadata"], loaded=loaded, skipped=skipped,
                         forward=unsupported, createCache=lambda: createGGUFCache(model["config"]),
                         forwardPrefill=unsupported, forwardDecode=unsupported, generate=unsupported,
                         resetCache=resetCache)
    model = createGGUFModel(config)
    res = loadWeights(parsed, model)
    return GGUFModel(
        model=model, config=config, metadata=parsed["metadata"], loaded=res["loaded"], skipped=res["skipped"],
        forward=lambda tokenIds: forwardLlamaCachedPrefill(model, tokenIds, createGGUFCache(model["config"])),
        createCache=lambda: createGGUFCache(model["config"]),
        forwardPrefill=lambda tokenIds, caches: forwardLlamaCachedPrefill(model, tokenIds, caches),
        forwardDecode=lambda tokenId, position, caches: forwardLlamaCachedDecode(model, tokenId, position, caches),
        generate=lambda promptIds, genConfig=None, callbacks=None: generateGGUF(model, promptIds, genConfig or {},
                                                                               callbacks or {}),
        resetCache=resetCache,
    )
