"""Independent restatements of the five families: Hugging Face transformers models built from a
config dict (no checkpoint download) and loaded with the same seeded canonical weights the oracle
and the HIP runner use. They pin the wiring the oracle and the HIP path could share by mistake
(which tensor feeds which residual, position rows, the c2p/p2c index direction, the ModernBERT
layer-0 identity norm, pooling and heads)."""
from __future__ import annotations

import numpy as np
import torch
import transformers


def _t(x):
    return torch.tensor(np.asarray(x, dtype=np.float32))


def _split_qkv(W, l, H, prefix, names):
    q = W[f"layers.{l}.qkv.weight"]
    qb = W[f"layers.{l}.qkv.bias"]
    sd = {}
    for i, n in enumerate(names):
        sd[f"{prefix}.{n}.weight"] = q[i * H:(i + 1) * H]
        sd[f"{prefix}.{n}.bias"] = qb[i * H:(i + 1) * H]
    return sd


def _bert_layers(W, spec, enc, attn_names=("query", "key", "value")):
    H = spec["hidden"]
    sd = {}
    for l in range(spec["layers"]):
        p = f"{enc}.layer.{l}"
        sd.update(_split_qkv(W, l, H, f"{p}.attention.self", attn_names))
        for dst, src in (("attention.output.dense", "attn_out"), ("intermediate.dense", "ffn_in"),
                         ("output.dense", "ffn_out"), ("attention.output.LayerNorm", "attn_ln"),
                         ("output.LayerNorm", "ffn_ln")):
            sd[f"{p}.{dst}.weight"] = W[f"layers.{l}.{src}.weight"]
            sd[f"{p}.{dst}.bias"] = W[f"layers.{l}.{src}.bias"]
    return sd


def _load(model, sd):
    missing, unexpected = model.load_state_dict({k: _t(v) for k, v in sd.items()}, strict=False)
    return missing, unexpected


def bert_embed_model(spec, W):
    """BertModel; the plan's embed head is the masked mean of the last hidden state."""
    cfg = transformers.BertConfig(
        vocab_size=spec["vocab"], hidden_size=spec["hidden"], num_hidden_layers=spec["layers"],
        num_attention_heads=spec["heads"], intermediate_size=spec["intermediate"],
        max_position_embeddings=spec["embed"]["maxPositions"], type_vocab_size=spec["embed"]["typeVocab"],
        layer_norm_eps=spec["block"]["norm"]["eps"], hidden_act="gelu")
    m = transformers.BertModel(cfg, add_pooling_layer=False).eval()
    sd = {"embeddings.word_embeddings.weight": W["embeddings.word.weight"],
          "embeddings.position_embeddings.weight": W["embeddings.position.weight"],
          "embeddings.token_type_embeddings.weight": W["embeddings.type.weight"],
          "embeddings.LayerNorm.weight": W["embeddings.LayerNorm.weight"],
          "embeddings.LayerNorm.bias": W["embeddings.LayerNorm.bias"]}
    sd.update(_bert_layers(W, spec, "encoder"))
    missing, _ = _load(m, sd)
    assert not [k for k in missing if "position_ids" not in k], missing

    def run(ids):
        with torch.no_grad():
            h = m(input_ids=torch.tensor(np.asarray(ids, dtype=np.int64))[None]).last_hidden_state[0]
        return h.mean(0).numpy()
    return run


def roberta_classify_model(spec, head, W, xlm: bool = False):
    cls = transformers.XLMRobertaConfig if xlm else transformers.RobertaConfig
    cfg = cls(vocab_size=spec["vocab"], hidden_size=spec["hidden"], num_hidden_layers=spec["layers"],
              num_attention_heads=spec["heads"], intermediate_size=spec["intermediate"],
              max_position_embeddings=spec["embed"]["maxPositions"],
              type_vocab_size=spec["embed"]["typeVocab"], layer_norm_eps=spec["block"]["norm"]["eps"],
              pad_token_id=spec["embed"]["padId"], num_labels=head["classes"], hidden_act="gelu")
    model_cls = (transformers.XLMRobertaForSequenceClassification if xlm
                 else transformers.RobertaForSequenceClassification)
    m = model_cls(cfg).eval()
    sd = {"roberta.embeddings.word_embeddings.weight": W["embeddings.word.weight"],
          "roberta.embeddings.position_embeddings.weight": W["embeddings.position.weight"],
          "roberta.embeddings.token_type_embeddings.weight": W["embeddings.type.weight"],
          "roberta.embeddings.LayerNorm.weight": W["embeddings.LayerNorm.weight"],
          "roberta.embeddings.LayerNorm.bias": W["embeddings.LayerNorm.bias"],
          "classifier.dense.weight": W["head.dense.weight"], "classifier.dense.bias": W["head.dense.bias"],
          "classifier.out_proj.weight": W["head.out_proj.weight"],
          "classifier.out_proj.bias": W["head.out_proj.bias"]}
    sd.update(_bert_layers(W, spec, "roberta.encoder"))
    missing, _ = _load(m, sd)
    assert not [k for k in missing if "position_ids" not in k], missing

    def run(ids):
        with torch.no_grad():
            return m(input_ids=torch.tensor(np.asarray(ids, dtype=np.int64))[None]).logits[0].numpy()
    return run


def deberta_classify_model(spec, head, W):
    H = spec["hidden"]
    rel = spec["attention"]["rel"]
    cfg = transformers.DebertaV2Config(
        vocab_size=spec["vocab"], hidden_size=H, num_hidden_layers=spec["layers"],
        num_attention_heads=spec["heads"], intermediate_size=spec["intermediate"],
        max_position_embeddings=512, type_vocab_size=0, layer_norm_eps=spec["block"]["norm"]["eps"],
        relative_attention=True, position_buckets=rel["buckets"], max_relative_positions=rel["maxPositions"],
        pos_att_type=["p2c", "c2p"], share_att_key=True, norm_rel_ebd="layer_norm",
        position_biased_input=False, pooler_hidden_size=H, pooler_hidden_act="gelu",
        num_labels=head["classes"], hidden_act="gelu", pad_token_id=0)
    m = transformers.DebertaV2ForSequenceClassification(cfg).eval()
    from kleinhirn_amd import synth
    rows = 2 * rel["buckets"]
    sd = {"deberta.embeddings.word_embeddings.weight": W["embeddings.word.weight"],
          "deberta.embeddings.LayerNorm.weight": W["embeddings.LayerNorm.weight"],
          "deberta.embeddings.LayerNorm.bias": W["embeddings.LayerNorm.bias"],
          "deberta.encoder.rel_embeddings.weight": synth.tensor_values("encoder.rel_embeddings.weight", (rows, H)),
          "deberta.encoder.LayerNorm.weight": np.ones(H, np.float32),
          "deberta.encoder.LayerNorm.bias": np.zeros(H, np.float32),
          "pooler.dense.weight": W["head.pooler.weight"], "pooler.dense.bias": W["head.pooler.bias"],
          "classifier.weight": W["head.classifier.weight"], "classifier.bias": W["head.classifier.bias"]}
    sd.update(_bert_layers(W, spec, "deberta.encoder", ("query_proj", "key_proj", "value_proj")))
    missing, _ = _load(m, sd)
    assert not [k for k in missing if "position_ids" not in k], missing

    def run(ids):
        with torch.no_grad():
            return m(input_ids=torch.tensor(np.asarray(ids, dtype=np.int64))[None]).logits[0].numpy()
    return run


def modernbert_cls_model(spec, W):
    H = spec["hidden"]
    a = spec["attention"]
    every = a["window"]["globalEvery"]
    cfg = transformers.ModernBertConfig(
        vocab_size=spec["vocab"], hidden_size=H, num_hidden_layers=spec["layers"],
        num_attention_heads=spec["heads"], intermediate_size=spec["intermediate"],
        max_position_embeddings=spec["embed"]["maxPositions"], norm_eps=spec["block"]["norm"]["eps"],
        norm_bias=False, attention_bias=False, mlp_bias=False, local_attention=2 * a["window"]["half"],
        global_attn_every_n_layers=every, hidden_activation="gelu",
        layer_types=["full_attention" if l % every == 0 else "sliding_attention" for l in range(spec["layers"])],
        rope_parameters={"full_attention": {"rope_type": "default", "rope_theta": a["rope"]["thetaGlobal"]},
                         "sliding_attention": {"rope_type": "default", "rope_theta": a["rope"]["thetaLocal"]}},
        pad_token_id=50283, attn_implementation="eager")
    m = transformers.ModernBertModel(cfg).eval()
    sd = {"embeddings.tok_embeddings.weight": W["embeddings.word.weight"],
          "embeddings.norm.weight": W["embeddings.norm.weight"], "final_norm.weight": W["final_norm.weight"]}
    for l in range(spec["layers"]):
        p = f"layers.{l}"
        if l > 0:
            sd[f"{p}.attn_norm.weight"] = W[f"layers.{l}.attn_norm.weight"]
        sd[f"{p}.attn.Wqkv.weight"] = W[f"layers.{l}.wqkv.weight"]
        sd[f"{p}.attn.Wo.weight"] = W[f"layers.{l}.attn_out.weight"]
        sd[f"{p}.mlp_norm.weight"] = W[f"layers.{l}.mlp_norm.weight"]
        sd[f"{p}.mlp.Wi.weight"] = W[f"layers.{l}.mlp_in.weight"]
        sd[f"{p}.mlp.Wo.weight"] = W[f"layers.{l}.mlp_out.weight"]
    missing, unexpected = _load(m, sd)
    assert not missing, missing

    def run(ids):
        with torch.no_grad():
            h = m(input_ids=torch.tensor(np.asarray(ids, dtype=np.int64))[None]).last_hidden_state[0]
        return h[0].numpy()
    return run
