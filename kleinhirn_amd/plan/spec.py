"""Model descriptions (ModelSpec / HeadSpec) for the encoder families the HIP runner executes.

Plain dicts with the field names of the reference's TypeScript types (src/plan/spec.ts:12-85), so a
spec serialises to the same JSON the reference's plan builder reads. The family rules (positions,
offsets, norms, heads) follow the reference's Hugging Face adapter (src/plan/hf.ts:157-458); only
the five families of the benchmark configurations are described here.
"""
from __future__ import annotations

import math


def position_rows(pad_id: int, ids) -> list[int]:
    """RoBERTa/XLM-R position rows: a pad id keeps row pad_id, every other id gets pad_id plus the
    count of non-pad ids up to and including it (src/plan/spec.ts:60-66)."""
    count = 0
    out = []
    for t in ids:
        if t == pad_id:
            out.append(pad_id)
        else:
            count += 1
            out.append(pad_id + count)
    return out


# ---- tensor names (src/plan/spec.ts:109-183) -------------------------------------------------

def _deberta_layer(l: int) -> dict:
    return {
        "qkvW": f"layers.{l}.qkv.weight", "qkvB": f"layers.{l}.qkv.bias",
        "posKey": f"layers.{l}.pos_key", "posQuery": f"layers.{l}.pos_query",
        "attnOutW": f"layers.{l}.attn_out.weight", "attnOutB": f"layers.{l}.attn_out.bias",
        "attnNormW": f"layers.{l}.attn_ln.weight", "attnNormB": f"layers.{l}.attn_ln.bias",
        "ffnInW": f"layers.{l}.ffn_in.weight", "ffnInB": f"layers.{l}.ffn_in.bias",
        "ffnOutW": f"layers.{l}.ffn_out.weight", "ffnOutB": f"layers.{l}.ffn_out.bias",
        "ffnNormW": f"layers.{l}.ffn_ln.weight", "ffnNormB": f"layers.{l}.ffn_ln.bias",
    }


def _bert_layer(l: int) -> dict:
    t = _deberta_layer(l)
    del t["posKey"], t["posQuery"]
    return t


class TensorNames:
    def __init__(self, embed_w, embed_b, layer, final_w=None, final_b=None):
        self.embedNormW = embed_w
        self.embedNormB = embed_b
        self.finalNormW = final_w
        self.finalNormB = final_b
        self.layer = layer


def modernbert_tensors(attention_bias: bool, mlp_bias: bool, norm_bias: bool) -> TensorNames:
    def layer(l):
        return {
            "qkvW": f"layers.{l}.wqkv.weight",
            "qkvB": f"layers.{l}.wqkv.bias" if attention_bias else None,
            "attnOutW": f"layers.{l}.attn_out.weight",
            "attnOutB": f"layers.{l}.attn_out.bias" if attention_bias else None,
            "attnNormW": f"layers.{l}.attn_norm.weight",
            "attnNormB": f"layers.{l}.attn_norm.bias" if norm_bias else None,
            "ffnInW": f"layers.{l}.mlp_in.weight",
            "ffnInB": f"layers.{l}.mlp_in.bias" if mlp_bias else None,
            "ffnOutW": f"layers.{l}.mlp_out.weight",
            "ffnOutB": f"layers.{l}.mlp_out.bias" if mlp_bias else None,
            "ffnNormW": f"layers.{l}.mlp_norm.weight",
            "ffnNormB": f"layers.{l}.mlp_norm.bias" if norm_bias else None,
        }
    return TensorNames("embeddings.norm.weight", "embeddings.norm.bias" if norm_bias else None,
                       layer, "final_norm.weight", "final_norm.bias" if norm_bias else None)


def tensor_names_for(spec: dict) -> TensorNames:
    fam = spec["family"]
    if fam in ("bert", "electra", "roberta", "xlm-roberta", "distilbert"):
        return TensorNames("embeddings.LayerNorm.weight", "embeddings.LayerNorm.bias", _bert_layer)
    if fam == "deberta-v2":
        return TensorNames("embeddings.LayerNorm.weight", "embeddings.LayerNorm.bias", _deberta_layer)
    if fam == "modernbert":
        return modernbert_tensors(spec["attention"]["bias"], spec["ffn"]["bias"],
                                  spec["block"]["norm"]["bias"])
    raise ValueError(f"no tensor names for family {fam}")


# ---- family rules (src/plan/hf.ts) ------------------------------------------------------------

def _dense(name, i, o, act, bias=True):
    return {"op": "dense", "name": name, "in": i, "out": o, "act": act, "bias": bias}


def bert_like(family: str, hidden: int, layers: int, heads: int, intermediate: int, vocab: int,
              max_positions: int = 512, type_vocab: int = 2, eps: float = 1e-12, act: str = "gelu",
              pad_id: int | None = None, position_offset: int = 0) -> dict:
    """BERT, RoBERTa and XLM-R rows of src/plan/hf.ts:179-221: post-norm, absolute positions,
    RoBERTa/XLM-R count position rows from the pad id (offset pad + 1, src/plan/hf.ts:116-125)."""
    head_dim = hidden // heads
    norm = {"eps": eps, "bias": True}
    embed = {"positions": "absolute", "positionOffset": position_offset,
             "maxPositions": max_positions, "typeVocab": type_vocab, "norm": norm,
             "maskMultiply": False, "project": False}
    if pad_id is not None:
        embed["padId"] = pad_id
    return {
        "family": family, "hidden": hidden, "layers": layers, "heads": heads, "headDim": head_dim,
        "intermediate": intermediate, "vocab": vocab, "embeddingSize": hidden, "embed": embed,
        "attention": {"kind": "standard", "bias": True, "scale": head_dim ** -0.5},
        "block": {"order": "post", "firstNormIdentity": False, "finalNorm": False, "norm": norm},
        "ffn": {"kind": "mlp", "act": act, "bias": True},
    }


def roberta_classify_head(hidden: int, classes: int) -> dict:
    """RobertaClassificationHead: first token, dense tanh, out_proj (src/plan/hf.ts:238-243)."""
    return {"type": "classify", "pool": "first", "classes": classes,
            "steps": [_dense("head.dense", hidden, hidden, "tanh"),
                      _dense("head.out_proj", hidden, classes, "none")]}


def deberta_v3(hidden: int, layers: int, heads: int, intermediate: int, vocab: int,
               buckets: int = 256, max_relative: int = 512, eps: float = 1e-7) -> dict:
    """DeBERTa-v3 row of src/plan/hf.ts:282-345: relative c2p+p2c attention with shared
    projections, no absolute positions, no type table, embedding LayerNorm times the mask."""
    head_dim = hidden // heads
    norm = {"eps": eps, "bias": True}
    return {
        "family": "deberta-v2", "hidden": hidden, "layers": layers, "heads": heads,
        "headDim": head_dim, "intermediate": intermediate, "vocab": vocab, "embeddingSize": hidden,
        "embed": {"positions": "none", "positionOffset": 0, "maxPositions": 512, "typeVocab": 0,
                  "norm": norm, "maskMultiply": True, "project": False},
        "attention": {"kind": "deberta-relative", "bias": True, "scale": 1 / math.sqrt(3 * head_dim),
                      "rel": {"buckets": buckets, "maxPositions": max_relative,
                              "types": ["c2p", "p2c"]}},
        "block": {"order": "post", "firstNormIdentity": False, "finalNorm": False, "norm": norm},
        "ffn": {"kind": "mlp", "act": "gelu", "bias": True},
    }


def deberta_v2_absolute(hidden: int, layers: int, heads: int, intermediate: int, vocab: int,
                        max_positions: int = 512, eps: float = 1e-7, act: str = "gelu") -> dict:
    """DeBERTa-v2 without relative attention (src/plan/hf.ts:327-345, polyBERT): absolute positions
    added before the embedding LayerNorm, the standard attention, the embeddings times the mask."""
    head_dim = hidden // heads
    norm = {"eps": eps, "bias": True}
    return {
        "family": "deberta-v2", "hidden": hidden, "layers": layers, "heads": heads,
        "headDim": head_dim, "intermediate": intermediate, "vocab": vocab, "embeddingSize": hidden,
        "embed": {"positions": "absolute", "positionOffset": 0, "maxPositions": max_positions, "typeVocab": 0,
                  "norm": norm, "maskMultiply": True, "project": False},
        "attention": {"kind": "standard", "bias": True, "scale": head_dim ** -0.5},
        "block": {"order": "post", "firstNormIdentity": False, "finalNorm": False, "norm": norm},
        "ffn": {"kind": "mlp", "act": act, "bias": True},
    }


def gliner(enc: dict, temperature: float, head_hidden: int | None = None, markers: int = 16) -> tuple[dict, dict]:
    """specFromGlinerManifest (src/plan/spec.ts:214-246): the DeBERTa-v2 encoder of a GLiNER2
    manifest (relative c2p+p2c attention, embedding LayerNorm times the mask, no position or type
    table) and the gliner2 span head. `enc` holds the manifest's encoder fields (hiddenSize,
    layers, heads, intermediateSize, positionBuckets, maxRelativePositions, layerNormEps,
    vocabSize)."""
    spec = deberta_v3(enc["hiddenSize"], enc["layers"], enc["heads"], enc["intermediateSize"],
                      enc.get("vocabSize", 0), enc["positionBuckets"], enc["maxRelativePositions"],
                      enc["layerNormEps"])
    spec["embed"]["maxPositions"] = 0
    head = {"type": "gliner2", "hidden": int(head_hidden or 768), "temperature": temperature, "markers": markers}
    return spec, head


def deberta_classify_head(hidden: int, classes: int, pooler_act: str = "gelu") -> dict:
    """ContextPooler (first token, dense, pooler_hidden_act) then the classifier
    (src/plan/hf.ts:354-364)."""
    return {"type": "classify", "pool": "first", "classes": classes,
            "steps": [_dense("head.pooler", hidden, hidden, pooler_act),
                      _dense("head.classifier", hidden, classes, "none")]}


def modernbert(hidden: int, layers: int, heads: int, intermediate: int, vocab: int,
               theta_global: float = 160000.0, theta_local: float = 10000.0,
               local_attention: int = 128, global_every: int = 3, eps: float = 1e-5,
               max_positions: int = 8192, bias: bool = False) -> dict:
    """ModernBERT row of src/plan/hf.ts:395-442: pre-norm, RoPE with a theta per layer type,
    sliding window half = local_attention / 2 on layers l % every != 0, GeGLU, layer 0 without
    attn_norm, a final norm."""
    head_dim = hidden // heads
    norm = {"eps": eps, "bias": bias}
    return {
        "family": "modernbert", "hidden": hidden, "layers": layers, "heads": heads,
        "headDim": head_dim, "intermediate": intermediate, "vocab": vocab, "embeddingSize": hidden,
        "embed": {"positions": "none", "positionOffset": 0, "maxPositions": max_positions,
                  "typeVocab": 0, "norm": norm, "maskMultiply": False, "project": False},
        "attention": {"kind": "standard", "bias": bias, "scale": head_dim ** -0.5,
                      "rope": {"thetaGlobal": theta_global, "thetaLocal": theta_local},
                      "window": {"half": local_attention // 2, "globalEvery": global_every}},
        "block": {"order": "pre", "firstNormIdentity": True, "finalNorm": True, "norm": norm},
        "ffn": {"kind": "geglu", "act": "gelu", "bias": bias},
    }


def julia(hidden: int, layers: int, heads: int, intermediate: int, vocab: int, norm_eps: float,
          rope_theta: float, local_attention: int, global_every: int, head_layers: int, head_ffn: int,
          options: int, max_pos: int = 0) -> tuple[dict, dict]:
    """specFromJuliaManifest (src/plan/spec.ts:248-277): a ModernBERT encoder with one RoPE theta,
    window half = localAttention, no biases, a final norm; the julia head (type row, head layers,
    scorer over `options` marker slots)."""
    head_dim = hidden // heads
    norm = {"eps": norm_eps, "bias": False}
    spec = {
        "family": "modernbert", "hidden": hidden, "layers": layers, "heads": heads,
        "headDim": head_dim, "intermediate": intermediate, "vocab": vocab, "embeddingSize": hidden,
        "embed": {"positions": "none", "positionOffset": 0, "maxPositions": max_pos,
                  "typeVocab": 0, "norm": norm, "maskMultiply": False, "project": False},
        "attention": {"kind": "standard", "bias": False, "scale": head_dim ** -0.5,
                      "rope": {"thetaGlobal": rope_theta, "thetaLocal": rope_theta},
                      "window": {"half": local_attention, "globalEvery": global_every}},
        "block": {"order": "pre", "firstNormIdentity": True, "finalNorm": True, "norm": norm},
        "ffn": {"kind": "geglu", "act": "gelu", "bias": False},
    }
    return spec, {"type": "julia", "layers": head_layers, "ffn": head_ffn, "options": options}


# rows of the Julia type table: the request types choice, score, noul (src/tokenizer/julia-input.ts:21)
JULIA_TYPES = 3


def julia_head_layer(i: int) -> dict:
    """Tensor names of Julia head layer i (src/plan/build.ts:387-396)."""
    p = f"head.{i}"
    return {"qkvW": f"{p}.in_proj.weight", "qkvB": f"{p}.in_proj.bias",
            "attnOutW": f"{p}.out_proj.weight", "attnOutB": f"{p}.out_proj.bias",
            "attnNormW": f"{p}.norm1.weight", "attnNormB": f"{p}.norm1.bias",
            "ffnNormW": f"{p}.norm2.weight", "ffnNormB": f"{p}.norm2.bias",
            "ffnInW": f"{p}.linear1.weight", "ffnInB": f"{p}.linear1.bias",
            "ffnOutW": f"{p}.linear2.weight", "ffnOutB": f"{p}.linear2.bias"}


def embed_head(pool: str, normalize: bool = True, steps=None) -> dict:
    """Embeddings head: pooling as sentence-transformers, optional dense steps
    (src/plan/hf.ts:272-278)."""
    return {"type": "embed", "pool": pool, "steps": list(steps or []), "normalize": normalize}


def manifest_tensors(spec: dict, head: dict) -> list[tuple[str, tuple[int, ...], str]]:
    """Every canonical tensor of a spec + head as (name, shape, kind) with kind in
    {'matrix', 'bias', 'gamma', 'beta', 'table', 'rel'}; names and shapes follow the reference
    converter (src/convert/names.ts:160-232)."""
    H, I, E = spec["hidden"], spec["intermediate"], spec["embeddingSize"]
    emb = spec["embed"]
    names = tensor_names_for(spec)
    out: list[tuple[str, tuple[int, ...], str]] = []
    out.append(("embeddings.word.weight", (spec["vocab"], E), "table"))
    if emb["positions"] == "absolute":
        out.append(("embeddings.position.weight", (emb["maxPositions"], E), "table"))
    if emb["typeVocab"] > 0:
        out.append(("embeddings.type.weight", (emb["typeVocab"], E), "table"))
    out.append((names.embedNormW, (E,), "gamma"))
    if names.embedNormB:
        out.append((names.embedNormB, (E,), "beta"))
    ffn_in = 2 * I if spec["ffn"]["kind"] == "geglu" else I
    for l in range(spec["layers"]):
        t = names.layer(l)
        if spec["family"] == "modernbert" and spec["block"]["firstNormIdentity"] and l == 0:
            t = dict(t, attnNormW=None, attnNormB=None)
        for key, shape, kind in (
            ("qkvW", (3 * H, H), "matrix"), ("qkvB", (3 * H,), "bias"),
            ("attnOutW", (H, H), "matrix"), ("attnOutB", (H,), "bias"),
            ("attnNormW", (H,), "gamma"), ("attnNormB", (H,), "beta"),
            ("ffnInW", (ffn_in, H), "matrix"), ("ffnInB", (ffn_in,), "bias"),
            ("ffnOutW", (H, I), "matrix"), ("ffnOutB", (H,), "bias"),
            ("ffnNormW", (H,), "gamma"), ("ffnNormB", (H,), "beta"),
        ):
            if t.get(key):
                out.append((t[key], shape, kind))
        if t.get("posKey") and spec["attention"]["kind"] == "deberta-relative":
            rows = 2 * spec["attention"]["rel"]["buckets"]
            out.append((t["posKey"], (rows, H), "rel"))
            out.append((t["posQuery"], (rows, H), "rel"))
    if names.finalNormW:
        out.append((names.finalNormW, (H,), "gamma"))
        if names.finalNormB:
            out.append((names.finalNormB, (H,), "beta"))
    if head["type"] == "julia":
        F = int(head["ffn"])
        out.append(("type_emb.weight", (JULIA_TYPES, H), "table"))
        for i in range(int(head["layers"])):
            t = julia_head_layer(i)
            for key, shape, kind in (
                ("qkvW", (3 * H, H), "matrix"), ("qkvB", (3 * H,), "bias"),
                ("attnOutW", (H, H), "matrix"), ("attnOutB", (H,), "bias"),
                ("attnNormW", (H,), "gamma"), ("attnNormB", (H,), "beta"),
                ("ffnNormW", (H,), "gamma"), ("ffnNormB", (H,), "beta"),
                ("ffnInW", (F, H), "matrix"), ("ffnInB", (F,), "bias"),
                ("ffnOutW", (H, F), "matrix"), ("ffnOutB", (H,), "bias"),
            ):
                out.append((t[key], shape, kind))
        out += [("scorer.norm.weight", (H,), "gamma"), ("scorer.norm.bias", (H,), "beta"),
                ("scorer.fc1.weight", (H, H), "matrix"), ("scorer.fc1.bias", (H,), "bias"),
                ("scorer.fc2.weight", (1, H), "matrix"), ("scorer.fc2.bias", (1,), "bias")]
    if head["type"] == "gliner2":
        # the span head's two products (src/plan/build.ts:367-370)
        hh = int(head["hidden"])
        out += [("head.fc1.weight", (hh, H), "matrix"), ("head.fc1.bias", (hh,), "bias"),
                ("head.fc2.weight", (1, hh), "matrix"), ("head.fc2.bias", (1,), "bias")]
    for step in head.get("steps", []):
        if step["op"] == "dense":
            out.append((f"{step['name']}.weight", (step["out"], step["in"]), "matrix"))
            if step["bias"]:
                out.append((f"{step['name']}.bias", (step["out"],), "bias"))
        else:
            out.append((f"{step['name']}.weight", (H,), "gamma"))
            if step["bias"]:
                out.append((f"{step['name']}.bias", (H,), "beta"))
    return out
