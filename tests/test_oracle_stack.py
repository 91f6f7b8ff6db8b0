"""Pins the stack oracle (oracle/stack.py) against transformers' Qwen2ForCausalLM, and checks the
host-side packing (rus_amd.ops.pack_varlen) and model adapter on the CPU."""

from __future__ import annotations


import pytest
import torch

from oracle import stack as ostack
from rus_amd import model as M
from rus_amd.ops import pack_varlen, scatter_per_token


def tiny_config(layers=2) -> M.Qwen2Config:
    return M.Qwen2Config(hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, vocab_size=300,
                         lora_r=4, lora_alpha=8.0, lora_dropout=0.0)


def _batch(cfg, lengths, S, seed=0):
    g = torch.Generator().manual_seed(seed)
    B = len(lengths)
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=g)
    mask = torch.zeros(B, S, dtype=torch.long)
    for b, L in enumerate(lengths):
        mask[b, :L] = 1
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    labels[0, :3] = -100  # a masked prompt
    return ids, mask, labels


def test_pack_varlen_matches_reference_rules():
    ids = torch.tensor([[5, 6, 7, 0, 0], [1, 2, 3, 4, 9]])
    mask = torch.tensor([[1, 1, 1, 0, 0], [1, 1, 1, 1, 1]])
    labels = torch.tensor([[5, 6, 7, -100, -100], [-100, -100, 3, 4, 9]])
    pb = pack_varlen(ids, mask, labels)
    assert pb.row_lengths == [3, 5]
    assert pb.input_ids.tolist() == [5, 6, 7, 1, 2, 3, 4, 9]
    assert pb.pos_ids.tolist() == [0, 1, 2, 0, 1, 2, 3, 4]
    # shifted labels: position t predicts labels[t + 1]; the last position of each row is -100
    assert pb.shift_labels.tolist() == [6, 7, -100, -100, 3, 4, 9, -100]
    back = scatter_per_token(pb.input_ids, pb, -1)
    assert back.tolist() == [[5, 6, 7, -1, -1], [1, 2, 3, 4, 9]]
    # the id check looks at kept tokens only: padding may hold anything
    ids_pad = ids.clone()
    ids_pad[0, 3:] = 10**6
    assert pack_varlen(ids_pad, mask, labels, vocab_size=10).row_lengths == [3, 5]
    for bad in (-1, 10):
        ids_bad = ids.clone()
        ids_bad[1, 2] = bad
        with pytest.raises(IndexError):
            pack_varlen(ids_bad, mask, labels, vocab_size=10)


def test_stack_oracle_matches_transformers_qwen2():
    from transformers import Qwen2Config as HFConfig
    from transformers import Qwen2ForCausalLM

    cfg = tiny_config()
    model = M.build_random_qlora_qwen2(cfg, "cpu", seed=1, std=0.05)
    deq = ostack.dequant_model(model)
    lora = ostack.lora_leaves(model)
    lengths, S = [9, 14, 5], 14
    ids, mask, labels = _batch(cfg, lengths, S)
    pb = pack_varlen(ids, mask, labels)
    loss, _ = ostack.step_loss(model, deq, lora, pb.input_ids, pb.pos_ids, pb.shift_labels,
                               pb.row_lengths, rope_dtype=torch.float32)

    hf_cfg = HFConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, vocab_size=300,
                      rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                      tie_word_embeddings=True, attention_dropout=0.0,
                      max_position_embeddings=64)
    hf_cfg._attn_implementation = "eager"
    hf = Qwen2ForCausalLM(hf_cfg).float().eval()
    s = cfg.lora_scaling
    with torch.no_grad():
        hf.model.embed_tokens.weight.copy_(model.embed.float())
        hf.model.norm.weight.copy_(model.final_norm)
        for li, (L, layer) in enumerate(zip(model.layers, hf.model.layers)):
            W = deq[li]
            qA, qB, vA, vB = (t.detach() for t in lora[4 * li: 4 * li + 4])
            at, mlp = layer.self_attn, layer.mlp
            at.q_proj.weight.copy_(W["q"] + s * qB @ qA)
            at.k_proj.weight.copy_(W["k"])
            at.v_proj.weight.copy_(W["v"] + s * vB @ vA)
            at.o_proj.weight.copy_(W["o"])
            at.q_proj.bias.copy_(L.q_bias.float())
            at.k_proj.bias.copy_(L.k_bias.float())
            at.v_proj.bias.copy_(L.v_bias.float())
            mlp.gate_proj.weight.copy_(W["gate"])
            mlp.up_proj.weight.copy_(W["up"])
            mlp.down_proj.weight.copy_(W["down"])
            layer.input_layernorm.weight.copy_(L.ln1)
            layer.post_attention_layernorm.weight.copy_(L.ln2)
        out = hf(input_ids=ids, attention_mask=mask, labels=labels)
    assert torch.allclose(loss.detach(), out.loss, rtol=1e-5, atol=1e-5), (float(loss), float(out.loss))


def test_stack_oracle_lora_grads_match_finite_differences():
    cfg = tiny_config(layers=1)
    model = M.build_random_qlora_qwen2(cfg, "cpu", seed=2, std=0.05)
    deq = ostack.dequant_model(model)
    lora = [p.double().detach().requires_grad_(True) for p in ostack.lora_leaves(model)]
    ids, mask, labels = _batch(cfg, [6, 4], 6, seed=3)
    pb = pack_varlen(ids, mask, labels)
    with torch.no_grad():
        for d in deq:
            for k in d:
                d[k] = d[k].double()

    def f(params):
        # double-precision evaluation of the same composition (rope tables in float64)
        return _loss64(model, deq, params, pb)

    loss = f(lora)
    loss.backward()
    g = lora[1].grad  # q_B
    eps = 1e-6
    for idx in [(0, 0), (3, 1), (17, 2)]:
        plus = [p.detach().clone() for p in lora]
        minus = [p.detach().clone() for p in lora]
        plus[1][idx] += eps
        minus[1][idx] -= eps
        fd = (f(plus) - f(minus)) / (2 * eps)
        assert abs(float(fd) - float(g[idx])) <= 1e-6 + 1e-5 * abs(float(fd))


def _loss64(model, deq, lora, pb):
    import torch.nn.functional as F

    cfg = model.config
    hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    from oracle import ops as ref

    cos, sin = ref.rope_tables(int(pb.pos_ids.max()) + 1, hd, cfg.rope_theta, torch.float64)
    c, s = cos[pb.pos_ids], sin[pb.pos_ids]
    eps = cfg.rms_norm_eps
    h = model.embed.double()[pb.input_ids]
    n = h.shape[0]
    for li, L in enumerate(model.layers):
        W = deq[li]
        qA, qB, vA, vB = lora[4 * li: 4 * li + 4]
        x = ostack._rms(h, L.ln1.double(), eps)
        q = x @ W["q"].t() + L.q_bias.double() + cfg.lora_scaling * ((x @ qA.t()) @ qB.t())
        k = x @ W["k"].t() + L.k_bias.double()
        v = x @ W["v"].t() + L.v_bias.double() + cfg.lora_scaling * ((x @ vA.t()) @ vB.t())
        q = ostack._rope(q.view(n, hq, hd), c, s)
        k = ostack._rope(k.view(n, hkv, hd), c, s)
        att = _att64(q, k, v.view(n, hkv, hd), pb.row_lengths)
        h = h + att @ W["o"].t()
        x2 = ostack._rms(h, L.ln2.double(), eps)
        h = h + (F.silu(x2 @ W["gate"].t()) * (x2 @ W["up"].t())) @ W["down"].t()
    f = ostack._rms(h, model.final_norm.double(), eps)
    logits = f @ model.embed.double().t()
    return F.cross_entropy(logits, pb.shift_labels, ignore_index=-100)


def _att64(q, k, v, row_lengths):
    import math

    n, hq, d = q.shape
    groups = hq // k.shape[1]
    outs = []
    cur = 0
    for L in row_lengths:
        qs, ks, vs = q[cur:cur + L], k[cur:cur + L], v[cur:cur + L]
        ks = ks.repeat_interleave(groups, dim=1)
        vs = vs.repeat_interleave(groups, dim=1)
        sc = torch.einsum("ihd,jhd->hij", qs, ks) / math.sqrt(d)
        sc = sc.masked_fill(~torch.ones(L, L, dtype=torch.bool).tril(), float("-inf"))
        outs.append(torch.einsum("hij,jhd->ihd", torch.softmax(sc, -1), vs))
        cur += L
    return torch.cat(outs).reshape(n, hq * d)


def test_model_from_duck_typed_causal_lm():
    """The adapter reads the attribute layout of a PEFT + bitsandbytes Qwen2 (no libraries)."""
    from duck_hf import duck_causal_lm

    from rus_amd.adapters import model_from_causal_lm

    cfg = tiny_config(layers=1)
    m = M.build_random_qlora_qwen2(cfg, "cpu", seed=4)
    L = m.layers[0]
    causal = duck_causal_lm(m)
    got = model_from_causal_lm(causal)
    assert got.config.lora_r == 4 and abs(got.config.lora_scaling - cfg.lora_scaling) < 1e-12
    G = got.layers[0]
    assert torch.equal(G.q.packed, L.q.packed) and torch.equal(G.down.absmax2, L.down.absmax2)
    assert G.q_A is L.q_A and G.v_B is L.v_B
    assert got.meta["layer_lora_meta"][0]["p_q"] == 0.05


def test_stack_oracle_dropout_uses_branch_masks():
    # p > 0 with a seed changes the loss; the q-branch mask enters only through x A_q^T, so a
    # zero A_q / A_v (no LoRA signal) makes dropout invisible.
    cfg = M.Qwen2Config(**{**tiny_config().__dict__, "lora_dropout": 0.1})
    model = M.build_random_qlora_qwen2(cfg, "cpu", seed=2, std=0.05)
    deq = ostack.dequant_model(model)
    lengths, S = [9, 14], 14
    ids, mask, labels = _batch(cfg, lengths, S)
    pb = pack_varlen(ids, mask, labels)
    args = (pb.input_ids, pb.pos_ids, pb.shift_labels, pb.row_lengths)
    lora = ostack.lora_leaves(model)
    base, _ = ostack.step_loss(model, deq, lora, *args)
    dropped, _ = ostack.step_loss(model, deq, lora, *args, dropout_seed=5)
    again, _ = ostack.step_loss(model, deq, lora, *args, dropout_seed=5)
    assert float(dropped) != float(base) and float(again) == float(dropped)
    for li in range(cfg.num_hidden_layers):
        for j in (4 * li, 4 * li + 2):  # A_q, A_v
            lora[j] = torch.zeros_like(lora[j])
    z0, _ = ostack.step_loss(model, deq, lora, *args)
    z1, _ = ostack.step_loss(model, deq, lora, *args, dropout_seed=5)
    assert float(z0) == float(z1)
