"""Writes tests/golden/hf_esm2_8m.npz: HuggingFace ESM-2 forwards of the
config-1 synthetic model, the independent pin of the forward composition.

The reference's own acceptance check for embed -> N x TransformerBlock ->
final LN -> lm head is HuggingFace parity
(tests/python/test_against_hf.py:86-160, goldens captured by
tools/capture_golden.py:94-140). Its golden tensors are not in the
reference tree and no checkpoint can be fetched here, so this script builds
transformers' EsmForMaskedLM locally with the config-1 synthetic weights
(seed 20261201 + 1, no download) and records what that independent
implementation computes:

  * seq_logits       16 config-1 sequences, each run alone (batch of one,
                     no padding), logits concatenated in packed order;
  * mask_*           a packed batch of three sequences holding mask tokens
                     (token dropout), each run alone: logits and every hidden
                     state, hidden_0 = post-embed, hidden_1..5 = layer
                     outputs, hidden_6 = post-final-LN (the reference's
                     ForwardWithHiddenStates layout, include/esm_cpp/model.h:
                     184-191; model.cpp:1149-1189);
  * pad_*            two sequences with pads (attention_mask 0) run as one
                     padded HF batch: the post-embed state only. HF zeroes
                     pad rows and counts real tokens in the token-dropout
                     ratio, as the reference's Embed does (model.cpp:745-775);
                     past the embedding the two differ on purpose (HF masks
                     pad keys in attention, the reference's AttentionVarlen
                     takes no mask), so later states are not recorded.

Only this .npz is used by the tests; transformers is imported here alone.
Run:  python tests/golden/make_hf_fixture.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "esm-cpp_amd"))

from esm_gfx950 import synthetic as syn  # noqa: E402

OUT = os.path.join(HERE, "hf_esm2_8m.npz")
SEED = 20261201 + 1


def mask_batch() -> syn.PackedBatch:
    """Three sequences with mask tokens at fixed positions (ratios 0.1-0.3)."""
    b = syn.batch_from_lengths([26, 41, 19], seed=11)
    ids = b.ids.copy()
    cu = b.cu
    marks = {0: [3, 7, 8, 20], 1: [1, 2, 15, 30], 2: [5, 6, 9, 10, 11]}
    for s, pos in marks.items():
        for p in pos:
            ids[cu[s] + p] = syn.MASK
    return syn.PackedBatch(ids, cu.copy(), b.lengths.copy())


def pad_batch():
    """(ids, masks, cu): two 30-token sequences; the first ends in six pads,
    the second has three pads inside it and two mask tokens."""
    b = syn.batch_from_lengths([30, 30], seed=12)
    ids = b.ids.copy()
    masks = np.ones_like(ids)
    masks[24:30] = 0
    ids[24:30] = syn.PAD
    for p in (30 + 10, 30 + 11, 30 + 20):
        masks[p] = 0
        ids[p] = syn.PAD
    ids[30 + 4] = ids[30 + 15] = syn.MASK
    return ids, masks, b.cu.copy()


def run_padded(m, ids, masks, cu):
    """HF's post-embed state of the sequences as one padded batch."""
    import torch

    caps = []
    h = m.esm.embeddings.register_forward_hook(lambda _m, _i, o: caps.append(o.clone()))
    try:
        with torch.no_grad():
            x = torch.from_numpy(np.stack([ids[cu[i]:cu[i + 1]] for i in range(len(cu) - 1)]).astype(np.int64))
            am = torch.from_numpy(np.stack([masks[cu[i]:cu[i + 1]] for i in range(len(cu) - 1)]).astype(np.int64))
            m(input_ids=x, attention_mask=am)
    finally:
        h.remove()
    return caps[0].numpy().reshape(-1, caps[0].shape[-1]).astype(np.float32)


def hf_model(w):
    import torch
    from transformers import EsmConfig, EsmForMaskedLM

    cfg = w.cfg
    hc = EsmConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, num_hidden_layers=cfg.num_layers,
                   num_attention_heads=cfg.num_heads, intermediate_size=cfg.intermediate_size,
                   hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0, max_position_embeddings=1026,
                   position_embedding_type="rotary", layer_norm_eps=cfg.layer_norm_eps, token_dropout=True,
                   mask_token_id=syn.MASK, pad_token_id=syn.PAD, emb_layer_norm_before=False, hidden_act="gelu",
                   attn_implementation="eager")
    m = EsmForMaskedLM(hc).eval()
    F = w.f32
    names = {"esm.embeddings.word_embeddings.weight": "embed",
             "lm_head.decoder.weight": "embed",
             "lm_head.bias": "lm_head.decoder.bias",
             "lm_head.dense.weight": "lm_head.dense.weight",
             "lm_head.dense.bias": "lm_head.dense.bias",
             "lm_head.layer_norm.weight": "lm_head.ln.weight",
             "lm_head.layer_norm.bias": "lm_head.ln.bias",
             "esm.encoder.emb_layer_norm_after.weight": "final_ln.weight",
             "esm.encoder.emb_layer_norm_after.bias": "final_ln.bias"}
    per_layer = {"attention.self.query": "q", "attention.self.key": "k", "attention.self.value": "v",
                 "attention.output.dense": "out", "intermediate.dense": "fc1", "output.dense": "fc2",
                 "attention.LayerNorm": "attn_ln", "LayerNorm": "ffn_ln"}
    for i in range(cfg.num_layers):
        for hf, ours in per_layer.items():
            for p in ("weight", "bias"):
                names[f"esm.encoder.layer.{i}.{hf}.{p}"] = f"layers.{i}.{ours}.{p}"
    sd = m.state_dict()
    loaded = set()
    with torch.no_grad():
        for k, src in names.items():
            t = torch.from_numpy(np.ascontiguousarray(F[src]))
            assert sd[k].shape == t.shape, (k, sd[k].shape, t.shape)
            sd[k].copy_(t)
            loaded.add(k)
    missing = [k for k in sd if k not in loaded and not k.startswith("esm.contact_head")
               and not k.endswith("inv_freq")]
    assert not missing, missing
    return m


def run_one(m, ids: np.ndarray):
    """Logits [L, V] and hidden states [N + 1, L, d] of one sequence."""
    import torch

    caps = []
    hooks = [m.esm.embeddings.register_forward_hook(lambda _m, _i, o: caps.append(o[0].clone()))]
    for layer in m.esm.encoder.layer:
        hooks.append(layer.register_forward_hook(
            lambda _m, _i, o: caps.append((o[0] if isinstance(o, tuple) else o)[0].clone())))
    hooks.append(m.esm.encoder.emb_layer_norm_after.register_forward_hook(
        lambda _m, _i, o: caps.append(o[0].clone())))
    try:
        with torch.no_grad():
            x = torch.from_numpy(ids.astype(np.int64))[None]
            out = m(input_ids=x, attention_mask=torch.ones_like(x))
    finally:
        for h in hooks:
            h.remove()
    n = len(m.esm.encoder.layer)
    assert len(caps) == n + 2, len(caps)
    hidden = [c.numpy() for c in caps]
    # ForwardWithHiddenStates layout: the last layer's raw output is replaced
    # by the post-final-LN state (model.cpp:1187-1189).
    hidden = hidden[:n] + [hidden[n + 1]]
    return out.logits[0].numpy().astype(np.float32), np.stack(hidden).astype(np.float32)


def main():
    import torch
    import transformers

    torch.manual_seed(0)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    w = syn.make_weights(syn.ESM2_8M, seed=SEED, int8=False)
    m = hf_model(w)

    b1 = syn.config1_batch()
    logits = []
    for s in range(len(b1.lengths)):
        lg, _ = run_one(m, b1.ids[b1.cu[s]:b1.cu[s + 1]])
        logits.append(lg)
    bm = mask_batch()
    m_logits, m_hidden = [], []
    for s in range(len(bm.lengths)):
        lg, hs = run_one(m, bm.ids[bm.cu[s]:bm.cu[s + 1]])
        m_logits.append(lg)
        m_hidden.append(hs)
    p_ids, p_masks, p_cu = pad_batch()
    p_hidden0 = run_padded(m, p_ids, p_masks, p_cu)
    np.savez_compressed(
        OUT,
        pad_ids=p_ids, pad_masks=p_masks, pad_cu=p_cu, pad_hidden0=p_hidden0,
        seq_ids=b1.ids, seq_cu=b1.cu, seq_logits=np.concatenate(logits),
        mask_ids=bm.ids, mask_cu=bm.cu, mask_logits=np.concatenate(m_logits),
        mask_hidden=np.concatenate(m_hidden, axis=1),
        weights_seed=np.int64(SEED),
        transformers_version=np.array(transformers.__version__),
        torch_version=np.array(torch.__version__))
    print(f"wrote {OUT}: {len(b1.lengths)} sequences ({b1.total_tokens} tokens), mask batch "
          f"{bm.total_tokens} tokens, transformers {transformers.__version__}")


if __name__ == "__main__":
    main()
