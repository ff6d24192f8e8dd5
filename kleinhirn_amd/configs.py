"""The benchmark workloads: model shape, head, bucket length and the seeded ragged batch.

c1 BERT MiniLM-L6 (f32, B=1, n=128, mean pool), c2 RoBERTa-base (f16, ragged B=256, 3 classes),
c3 DeBERTa-v3-base (f16, B=32 at n=512 and ragged B=256, 2 classes), c4 ModernBERT-small (f16,
B=64, n uniform 256..8192, CLS embedding), c5 XLM-R MiniLM-L12 cross-encoder (f16, 4096 pairs,
one relevance logit). Shapes follow the family rules of the reference's HF adapter; lengths and
ids come from the streams of kleinhirn_amd.synth (per-config stream seed + k).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import synth
from .plan import spec as S


@dataclass
class Workload:
    name: str
    spec: dict
    head: dict
    f16: bool
    length: int          # bucket length L of the plan
    lengths: list        # tokens per sequence (special tokens included)
    cls_id: int
    sep_id: int
    ids_seed: int
    pairs: list | None = None

    @property
    def batch(self) -> int:
        return len(self.lengths)

    @property
    def tokens(self) -> int:
        return int(sum(self.lengths))

    def ids(self) -> list[np.ndarray]:
        return synth.draw_ids(self.ids_seed, self.lengths, self.spec["vocab"], self.cls_id,
                              self.sep_id, self.pairs)


def minilm_spec():
    return S.bert_like("bert", 384, 6, 12, 1536, 30522, max_positions=512, type_vocab=2, eps=1e-12)


def roberta_base_spec():
    return S.bert_like("roberta", 768, 12, 12, 3072, 50265, max_positions=514, type_vocab=1,
                       eps=1e-5, pad_id=1, position_offset=2)


def deberta_v3_base_spec():
    return S.deberta_v3(768, 12, 12, 3072, 128100)


def modernbert_small_spec():
    return S.modernbert(384, 22, 6, 1536, 50368)


def xlmr_minilm_spec():
    return S.bert_like("xlm-roberta", 384, 12, 12, 1536, 250002, max_positions=514, type_vocab=1,
                       eps=1e-5, pad_id=1, position_offset=2)


def c1() -> Workload:
    return Workload("c1-minilm-l6-f32", minilm_spec(), S.embed_head("mean"), False, 128, [128],
                    101, 102, synth.SEED + 1)


def c2(batch: int = 256) -> Workload:
    st = synth.Lcg(synth.SEED + 2)
    lengths = synth.lognormal_lengths(st, batch)
    return Workload("c2-roberta-base-f16-ragged256", roberta_base_spec(),
                    S.roberta_classify_head(768, 3), True, 512, lengths, 0, 2, synth.SEED + 102)


def c3a(batch: int = 32) -> Workload:
    return Workload("c3a-deberta-v3-base-f16-b32x512", deberta_v3_base_spec(),
                    S.deberta_classify_head(768, 2), True, 512, [512] * batch, 1, 2, synth.SEED + 103)


def c3b(batch: int = 256) -> Workload:
    st = synth.Lcg(synth.SEED + 3)
    lengths = synth.lognormal_lengths(st, batch)
    return Workload("c3b-deberta-v3-base-f16-ragged256", deberta_v3_base_spec(),
                    S.deberta_classify_head(768, 2), True, 512, lengths, 1, 2, synth.SEED + 203)


def c4(batch: int = 64) -> Workload:
    st = synth.Lcg(synth.SEED + 4)
    lengths = [256 + math.floor(st.next() * 7937) for _ in range(batch)]
    return Workload("c4-modernbert-small-f16-b64", modernbert_small_spec(),
                    S.embed_head("cls", normalize=False), True, 8192, lengths, 50281, 50282,
                    synth.SEED + 104)


def c5(pairs: int = 4096) -> Workload:
    st = synth.Lcg(synth.SEED + 5)
    qp = []
    for _ in range(pairs):
        q = 8 + math.floor(st.next() * 25)
        p = 64 + math.floor(st.next() * 417)
        if q + p + 4 > 512:   # the XLM-R position table holds 512 tokens after the offset
            p = 512 - q - 4
        qp.append((q, p))
    lengths = [q + p + 4 for q, p in qp]
    head = {"type": "classify", "pool": "first", "classes": 1,
            "steps": [{"op": "dense", "name": "head.dense", "in": 384, "out": 384, "act": "tanh", "bias": True},
                      {"op": "dense", "name": "head.out_proj", "in": 384, "out": 1, "act": "none", "bias": True}]}
    return Workload("c5-xlmr-minilm-l12-f16-pairs4096", xlmr_minilm_spec(), head, True, 512,
                    lengths, 0, 2, synth.SEED + 105, pairs=qp)


ALL = {"c1": c1, "c2": c2, "c3a": c3a, "c3b": c3b, "c4": c4, "c5": c5}


# ---- weights -----------------------------------------------------------------------------------

def make_weights(spec: dict, head: dict, seed: int = synth.SEED) -> dict[str, np.ndarray]:
    """Every canonical tensor of the model as f32: matrices, biases and tables N(0, 0.02) from
    their own streams, LayerNorm gamma 1 and beta 0, DeBERTa pos_key / pos_query derived from
    N(0, 0.02) rel_embeddings as the reference converter does: LayerNorm (eps of the block norm)
    of the first 2 * buckets rows, times the layer's key / query projection transposed, plus its
    bias, in f64, rounded once to f32 (src/convert/manifest.ts:72-120)."""
    out: dict[str, np.ndarray] = {}
    rel_ln = None
    H = spec["hidden"]
    for name, shape, kind in S.manifest_tensors(spec, head):
        if kind == "gamma":
            out[name] = np.ones(shape, dtype=np.float32)
        elif kind == "beta":
            out[name] = np.zeros(shape, dtype=np.float32)
        elif kind == "rel":
            if rel_ln is None:
                rows = shape[0]
                rel = synth.tensor_values("encoder.rel_embeddings.weight", (rows, H), seed=seed).astype(np.float64)
                mean = rel.mean(axis=1, keepdims=True)
                var = ((rel - mean) ** 2).mean(axis=1, keepdims=True)
                eps = spec["block"]["norm"]["eps"]
                rel_ln = (rel - mean) / np.sqrt(var + eps)          # gamma 1, beta 0
            layer = name.split(".")[1]
            # key / query projections are the k and q row blocks of the fused qkv weight
            qkv_w = out[f"layers.{layer}.qkv.weight"].astype(np.float64)
            qkv_b = out[f"layers.{layer}.qkv.bias"].astype(np.float64)
            blk = 1 if name.endswith("pos_key") else 0
            w = qkv_w[blk * H:(blk + 1) * H]
            b = qkv_b[blk * H:(blk + 1) * H]
            out[name] = (rel_ln @ w.T + b).astype(np.float32)
        else:
            out[name] = synth.tensor_values(name, shape, seed=seed)
    return out


def storage(weights: dict[str, np.ndarray], f16: bool) -> dict[str, np.ndarray]:
    """The tensors in the plan's storage dtype (f16: round-to-nearest-even cast of the f32 values)."""
    if not f16:
        return weights
    return {k: synth.to_f16(v) for k, v in weights.items()}
