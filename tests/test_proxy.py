"""CPU tests of the TRL / Soup integration surface (solution/ops.py:352-596, 1016-1238).

* ``ChunkedLogitsProxy`` built from per-position statistics answers what trainers compute from
  logits, against the same quantities computed from real logits (the reference's own proxy test,
  solution/test_kernels.py:228-241, plus the reshape / gather / dtype paths): entropy within
  2e-3, argmax exact, cross-entropy within 2e-3 (here exact up to fp32 summation order, since
  the statistics come from the same logits); unsupported operations raise.
* ``install_runtime_patches``: the transformers Qwen2 forward keeps the library's results for
  calls the fused path does not take (CPU inputs, no QLoRA layers); the TRL entropy helper reads
  the proxy and defers to the original for real logits.
"""

from __future__ import annotations

import sys
import types

import pytest
import torch
import torch.nn.functional as F

from rus_amd import ops
from rus_amd.proxy import ChunkedLogitsProxy


def _stats(B=2, S=32, V=4099, seed=3):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, S, V, generator=g) * 2.0
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[:, :8] = -100
    shift = torch.full((B, S), -100, dtype=torch.long)
    shift[:, :-1] = labels[:, 1:]
    lse = torch.logsumexp(logits, -1)
    ent = lse - (F.softmax(logits, -1) * logits).sum(-1)
    nll = F.cross_entropy(logits.reshape(-1, V), shift.reshape(-1), ignore_index=-100,
                          reduction="none").view(B, S)
    amax = logits.argmax(-1)
    return logits, labels, shift, nll, ent, amax, lse


@pytest.mark.parametrize("with_lse", [False, True])
def test_proxy_answers_trainer_reductions(with_lse):
    logits, labels, shift, nll, ent, amax, lse = _stats()
    B, S, V = logits.shape
    proxy = ChunkedLogitsProxy(nll, ent, amax, V, per_token_lse=lse if with_lse else None)
    assert proxy.shape == (B, S, V) and proxy.dtype == torch.float16 and proxy.dim() == 3
    assert proxy.size(-1) == V and len(proxy) == B
    # TRL's entropy expression
    got = torch.logsumexp(proxy, dim=-1) - torch.sum(F.softmax(proxy, dim=-1) * proxy, dim=-1)
    torch.testing.assert_close(got, ent, rtol=2e-3, atol=2e-3)
    if with_lse:  # each term on its own, not only their difference
        torch.testing.assert_close(torch.logsumexp(proxy, -1), lse)
        want = (F.softmax(logits, -1) * logits).sum(-1)
        torch.testing.assert_close((F.softmax(proxy, -1) * proxy).sum(-1), want, rtol=1e-4,
                                   atol=1e-4)
    # argmax (TRL mean_token_accuracy), before and after the causal shift
    assert torch.equal(proxy[:, :-1].argmax(dim=-1), amax[:, :-1])
    assert torch.equal(proxy.argmax(dim=-1)[:, :-1], amax[:, :-1])
    assert torch.equal(proxy[..., :-1, :].argmax(-1), amax[:, :-1])
    # per-row loss as Soup's rewind log computes it (reference test line 240)
    row0 = F.cross_entropy(proxy[0, :-1].float(), labels[0, 1:], ignore_index=-100)
    ref0 = F.cross_entropy(logits[0, :-1], labels[0, 1:], ignore_index=-100)
    torch.testing.assert_close(row0, ref0, rtol=2e-3, atol=2e-3)
    # the trainer's flattened shifted loss, all reductions
    flat = proxy[:, :-1].contiguous().view(-1, V)
    assert flat.shape == (B * (S - 1), V)
    tgt = labels[:, 1:].reshape(-1)
    for red in ("mean", "sum", "none"):
        a = F.cross_entropy(flat, tgt, ignore_index=-100, reduction=red)
        b = F.cross_entropy(logits[:, :-1].reshape(-1, V), tgt, ignore_index=-100, reduction=red)
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    # log-probabilities of the targets
    lp = F.log_softmax(proxy, dim=-1)[:, :-1].gather(-1, labels[:, 1:].clamp(min=0)[..., None])
    want = torch.log_softmax(logits, -1)[:, :-1].gather(-1, labels[:, 1:].clamp(min=0)[..., None])
    valid = (labels[:, 1:] != -100)[..., None]
    torch.testing.assert_close(lp[valid], want[valid], rtol=1e-5, atol=1e-5)
    # reshape with -1, row indexing, casts and no-op layout calls keep the statistics
    r = proxy.reshape(-1, V)
    assert r.shape == (B * S, V) and torch.equal(r.argmax(-1), amax.reshape(-1))
    assert proxy[1].shape == (S, V) and torch.equal(proxy[1].argmax(-1), amax[1])
    assert proxy.float().dtype == torch.float32 and proxy.to(torch.bfloat16).dtype == torch.bfloat16
    assert proxy.detach() is proxy and proxy.contiguous() is proxy
    assert "ChunkedLogitsProxy" in repr(proxy)


def test_proxy_rejects_what_needs_the_logits():
    logits, labels, shift, nll, ent, amax, lse = _stats(B=1, S=4, V=50)
    proxy = ChunkedLogitsProxy(nll, ent, amax, 50)
    for bad in (lambda: proxy + 1, lambda: proxy.sum(), lambda: proxy[..., :10],
                lambda: proxy.max(-1), lambda: proxy.reshape(2, 100),
                lambda: F.cross_entropy(proxy.view(-1, 50), shift.view(-1), label_smoothing=0.1),
                lambda: F.softmax(proxy, -1) + 1):
        with pytest.raises(TypeError):
            bad()
    with pytest.raises(ValueError):
        ChunkedLogitsProxy(nll, ent, amax, 50, virtual_shape=(1, 5, 50))


@pytest.fixture
def keep_qwen2_forward(monkeypatch):
    """install_runtime_patches replaces transformers' Qwen2 causal-LM, MLP and RMSNorm forwards;
    restore them afterwards."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except ImportError:
        return
    for cls in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                modeling_qwen2.Qwen2RMSNorm):
        monkeypatch.setattr(cls, "forward", cls.forward)


def test_trl_entropy_patch_reads_the_proxy(monkeypatch, keep_qwen2_forward):
    calls = []

    def entropy_from_logits(logits, chunk_size=128):
        calls.append(chunk_size)
        return torch.logsumexp(logits, -1) - (F.softmax(logits, -1) * logits).sum(-1)

    pkg, sub, mod = (types.ModuleType(n) for n in ("trl", "trl.trainer", "trl.trainer.sft_trainer"))
    mod.entropy_from_logits = entropy_from_logits
    pkg.trainer, sub.sft_trainer = sub, mod
    for name, m in (("trl", pkg), ("trl.trainer", sub), ("trl.trainer.sft_trainer", mod)):
        monkeypatch.setitem(sys.modules, name, m)
    got = ops.install_runtime_patches()
    assert got["trl_entropy"] and ops.install_runtime_patches()["trl_entropy"]  # idempotent
    logits, labels, shift, nll, ent, amax, lse = _stats(B=1, S=6, V=80)
    proxy = ChunkedLogitsProxy(nll, ent, amax, 80)
    assert mod.entropy_from_logits(proxy) is proxy.per_token_entropy and not calls
    torch.testing.assert_close(mod.entropy_from_logits(logits, chunk_size=7), ent)
    assert calls == [7]


def test_qwen2_patch_keeps_unfused_calls(keep_qwen2_forward):
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen2 import modeling_qwen2

    cfg = transformers.Qwen2Config(vocab_size=97, hidden_size=32, intermediate_size=64,
                                   num_hidden_layers=1, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(0)
    model = modeling_qwen2.Qwen2ForCausalLM(cfg).eval()
    ids = torch.randint(0, 97, (2, 9))
    with torch.no_grad():
        before = model(input_ids=ids, labels=ids)
    assert ops.install_runtime_patches()["transformers_qwen2"]
    assert getattr(modeling_qwen2.Qwen2ForCausalLM.forward, "_rus_fused", False)
    with torch.no_grad():
        after = model(input_ids=ids, labels=ids)  # CPU, no QLoRA layers: the library's path
    torch.testing.assert_close(after.loss, before.loss)
    torch.testing.assert_close(after.logits, before.logits)
    assert not ops._fusable(model, ids, ids)


def test_qwen2_mlp_and_rmsnorm_patches_keep_cpu_calls(keep_qwen2_forward):
    # Qwen2MLP / Qwen2RMSNorm are routed to the kernels only for device tensors: on CPU tensors
    # (and for a trainable norm weight under autograd) the library's own code runs, bit for bit.
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen2 import modeling_qwen2

    cfg = transformers.Qwen2Config(vocab_size=97, hidden_size=32, intermediate_size=64,
                                   num_hidden_layers=1, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(1)
    mlp, norm = modeling_qwen2.Qwen2MLP(cfg), modeling_qwen2.Qwen2RMSNorm(32, eps=1e-6)
    x = torch.randn(3, 5, 32)
    with torch.no_grad():
        want_mlp, want_norm = mlp(x), norm(x)
    got = ops.install_runtime_patches()
    assert got["qwen2_mlp"] and got["qwen2_rmsnorm"]
    for cls in (modeling_qwen2.Qwen2MLP, modeling_qwen2.Qwen2RMSNorm):
        assert getattr(cls.forward, "_rus_fused", False) and cls.forward.__wrapped__ is not None
    fwd = modeling_qwen2.Qwen2MLP.forward
    assert ops.install_runtime_patches()["qwen2_mlp"] and modeling_qwen2.Qwen2MLP.forward is fwd
    with torch.no_grad():
        assert torch.equal(mlp(x), want_mlp) and torch.equal(norm(x), want_norm)
    y = norm(x.requires_grad_())  # trainable weight: transformers' code, weight gradient formed
    y.sum().backward()
    assert norm.weight.grad is not None


def test_apply_is_idempotent(keep_qwen2_forward, monkeypatch):
    # rus_amd.apply(): loads the library, installs the patches once; a second call changes
    # nothing and returns the same answer (solution/__init__.py:111-116). No GPU here, so no
    # warm-up launches.
    pytest.importorskip("transformers")
    import rus_amd
    from transformers.models.qwen2 import modeling_qwen2

    monkeypatch.setattr(rus_amd, "_ACTIVE", None)
    first = rus_amd.apply()
    assert first["transformers_qwen2"] and first["qwen2_mlp"] and first["qwen2_rmsnorm"]
    fwds = [c.forward for c in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                                modeling_qwen2.Qwen2RMSNorm)]
    assert rus_amd.apply() == first
    assert fwds == [c.forward for c in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                                        modeling_qwen2.Qwen2RMSNorm)]
