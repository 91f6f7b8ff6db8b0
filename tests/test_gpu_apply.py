"""GPU tests of ``rus_amd.apply()`` and the Qwen2MLP / Qwen2RMSNorm patches it installs (the
reference's installer and fallback patches, solution/__init__.py:111-125, solution/ops.py:1029-1039,
1186-1188).

* ``apply()`` warms every kernel family up on the device, installs the patches, and a second call
  is a no-op.
* Patched fp16 ``Qwen2RMSNorm`` equals transformers' within one fp16 ulp per rounding (rtol 1e-3);
  patched fp16 ``Qwen2MLP`` (SwiGLU on the kernel, one rounding where transformers rounds twice)
  within 2e-3 relative Frobenius norm of transformers' output.
* An eval forward without labels of a transformers ``Qwen2ForCausalLM`` (not fusable: no labels,
  so its MLP and norm calls take the patched kernels) matches the unpatched forward. The model is
  fp32, so that transformers' attention runs in fp32 on both sides; logits within 1e-4 relative
  Frobenius norm, and the kernels are shown to have run.
"""

from __future__ import annotations

import pytest
import torch

from rus_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def fresh_patches(monkeypatch):
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen2 import modeling_qwen2

    import rus_amd

    for cls in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                modeling_qwen2.Qwen2RMSNorm):
        monkeypatch.setattr(cls, "forward", cls.forward)
    monkeypatch.setattr(rus_amd, "_ACTIVE", None)
    return transformers, modeling_qwen2, rus_amd


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def test_apply_warms_up_and_is_idempotent(fresh_patches):
    _, modeling_qwen2, rus_amd = fresh_patches
    first = rus_amd.apply()
    assert first["transformers_qwen2"] and first["qwen2_mlp"] and first["qwen2_rmsnorm"]
    fwds = [c.forward for c in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                                modeling_qwen2.Qwen2RMSNorm)]
    assert all(getattr(f, "_rus_fused", False) for f in fwds)
    assert rus_amd.apply() == first
    assert fwds == [c.forward for c in (modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2MLP,
                                        modeling_qwen2.Qwen2RMSNorm)]


def test_patched_rmsnorm_and_mlp_match_transformers_fp16(fresh_patches):
    transformers, modeling_qwen2, rus_amd = fresh_patches
    rus_amd.apply()
    cfg = transformers.Qwen2Config(vocab_size=1000, hidden_size=1536, intermediate_size=8960,
                                   num_hidden_layers=1, num_attention_heads=12,
                                   num_key_value_heads=2, rms_norm_eps=1e-6)
    torch.manual_seed(3)
    norm = modeling_qwen2.Qwen2RMSNorm(1536, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.05 * torch.randn(1536))
    norm = norm.to(DEV, torch.float16)
    norm.weight.requires_grad_(False)  # frozen, as under QLoRA
    mlp = modeling_qwen2.Qwen2MLP(cfg)
    with torch.no_grad():
        for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            lin.weight.normal_(0, 0.02)
    mlp = mlp.to(DEV, torch.float16)
    x = torch.randn(311, 1536, device=DEV).half()
    with torch.no_grad():
        got_n = norm(x)
        want_n = modeling_qwen2.Qwen2RMSNorm.forward.__wrapped__(norm, x)
        got_m = mlp(x)
        want_m = modeling_qwen2.Qwen2MLP.forward.__wrapped__(mlp, x)
    torch.cuda.synchronize()
    assert got_n.dtype == torch.float16 and got_n.shape == want_n.shape
    # one fp16 ulp at each of the two roundings (h * rstd, then * w)
    torch.testing.assert_close(got_n.float(), want_n.float(), rtol=2e-3, atol=2e-3)
    assert got_m.dtype == torch.float16 and got_m.shape == want_m.shape
    assert _rel(got_m, want_m) <= 2e-3


def test_eval_forward_without_labels_matches_unpatched(fresh_patches, monkeypatch):
    transformers, modeling_qwen2, rus_amd = fresh_patches
    cfg = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                                   num_hidden_layers=2, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=128,
                                   rms_norm_eps=1e-6)
    torch.manual_seed(5)
    model = modeling_qwen2.Qwen2ForCausalLM(cfg).to(DEV).eval()
    ids = torch.randint(0, 512, (2, 37), device=DEV)
    with torch.no_grad():
        want = model(input_ids=ids).logits
    calls = {"norm": 0, "glu": 0}
    fwd, glu = K.rms_norm_fwd, K.mlp_glu_fwd

    def count_norm(*a, **k):
        calls["norm"] += 1
        return fwd(*a, **k)

    def count_glu(*a, **k):
        calls["glu"] += 1
        return glu(*a, **k)

    monkeypatch.setattr(K, "rms_norm_fwd", count_norm)
    monkeypatch.setattr(K, "mlp_glu_fwd", count_glu)
    rus_amd.apply()
    calls.update(norm=0, glu=0)  # the warm-up's launches do not count
    with torch.no_grad():
        got = model(input_ids=ids).logits
    torch.cuda.synchronize()
    # 2 layers x (input + post-attention norm) + the final norm; one SwiGLU per layer
    assert calls == {"norm": 5, "glu": 2}
    assert got.shape == want.shape and got.dtype == want.dtype
    assert _rel(got, want) <= 1e-4
