"""Autograd functions, the fused Qwen2 stack and the chunked lm_head (solution/ops.py surface).

Names, signatures and return values follow the reference so its callers can switch to this
module: ``rms_norm`` / ``FusedRMSNormFn``, ``mlp_glu`` / ``FusedMLPGLUFn``, ``qkv_lora_rope`` /
``FusedQKVLoRARoPEFn``, ``chunked_lm_head`` / ``FusedChunkedLMHeadFn`` / ``PRESCALE_GRAD``,
``Qwen2FusedEngine`` and ``FusedQwen2StackFn.apply(h_packed, pos_ids, row_lengths, engine,
training, *lora_params)``. Every elementwise / normalisation / rotary / dequant / LoRA /
attention / lm_head step runs a gfx950 kernel from ``rus_amd.kernels``; the base-weight
projections are library GEMMs (hipBLASLt) on the dequantised fp16 weights, or the fused NF4 GEMM
kernel with ``gemm="fused"``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kernels as K
from .hostload import MAX_MLP_TOKENS, V_CHUNK_DEFAULT, HostHead, InputStream, WeightStream
from .proxy import ChunkedLogitsProxy

PRESCALE_GRAD = 65536.0  # solution/ops.py:171: gradients of the loss are formed times 2^16


# ---------------------------------------------------------------------------------------------
# Per-op autograd functions (solution/ops.py:30-164)
# ---------------------------------------------------------------------------------------------


class FusedRMSNormFn(torch.autograd.Function):
    """Residual + RMSNorm; saves (h, weight, rstd) only and returns the same gradient for x and
    residual (solution/ops.py:30-50)."""

    @staticmethod
    def forward(ctx, x, weight, eps=1e-6, residual=None):
        y, h, rstd = K.rms_norm_fwd(x, weight, eps=eps, residual=residual)
        ctx.save_for_backward(h, weight, rstd)
        ctx.with_residual = residual is not None
        return (y, h) if residual is not None else y

    @staticmethod
    def backward(ctx, *grads):
        h, weight, rstd = ctx.saved_tensors
        # with a residual, h = x + residual feeds both the norm and the next residual add
        d_h = grads[1] if ctx.with_residual else None
        dx = K.rms_norm_bwd(grads[0], h, weight, rstd, dresidual=d_h)
        return dx, None, None, (dx if ctx.with_residual else None)


def rms_norm(x, weight, eps: float = 1e-6, residual=None):
    return FusedRMSNormFn.apply(x, weight, eps, residual)


class FusedMLPGLUFn(torch.autograd.Function):
    """SwiGLU over fused [gate|up] (up=None) or separate tensors (solution/ops.py:57-81)."""

    @staticmethod
    def forward(ctx, gate_or_gu, up=None):
        ctx.one_buffer = up is None
        ctx.save_for_backward(gate_or_gu, *(() if up is None else (up,)))
        return K.mlp_glu_fwd(gate_or_gu, up)

    @staticmethod
    def backward(ctx, dout):
        if not ctx.one_buffer:
            return K.mlp_glu_bwd(dout, *ctx.saved_tensors)
        (gu,) = ctx.saved_tensors
        d_gu = torch.empty_like(gu)  # the saved pre-activation stays intact
        K.mlp_glu_bwd(dout, gu, None, dgu_out=d_gu)
        return d_gu, None


def mlp_glu(gate_or_gu, up=None):
    return FusedMLPGLUFn.apply(gate_or_gu, up)


class FusedQKVLoRARoPEFn(torch.autograd.Function):
    """LoRA delta + NeoX RoPE; the backward returns dqkv and the scaled LoRA-delta gradients from
    one kernel (solution/ops.py:88-148)."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, pos_ids, q_lora=None, v_lora=None, scale_q=2.0, scale_v=2.0,
                h_q=12, h_kv=2, head_dim=128):
        q_out, k_out, v_out = K.qkv_rope_fwd(qkv, cos, sin, pos_ids, q_lora=q_lora, v_lora=v_lora,
                                             scale_q=scale_q, scale_v=scale_v, h_q=h_q, h_kv=h_kv,
                                             head_dim=head_dim)
        ctx.save_for_backward(cos, sin, pos_ids)
        ctx.has_lora = q_lora is not None and v_lora is not None
        ctx.scale_q, ctx.scale_v = float(scale_q), float(scale_v)
        ctx.h_q, ctx.h_kv, ctx.head_dim = h_q, h_kv, head_dim
        return q_out, k_out, v_out

    @staticmethod
    def backward(ctx, dq_rot, dk_rot, dv_out):
        cos, sin, pos_ids = ctx.saved_tensors
        if not ctx.has_lora:
            dqkv = K.qkv_rope_bwd(dq_rot, dk_rot, dv_out, cos, sin, pos_ids, h_q=ctx.h_q,
                                  h_kv=ctx.h_kv, head_dim=ctx.head_dim)
            return dqkv, None, None, None, None, None, None, None, None, None, None
        dqkv, dq_lora, dv_lora = K.qkv_rope_bwd_lora(dq_rot, dk_rot, dv_out, cos, sin, pos_ids,
                                                     ctx.scale_q, ctx.scale_v, h_q=ctx.h_q,
                                                     h_kv=ctx.h_kv, head_dim=ctx.head_dim)
        return dqkv, None, None, None, dq_lora, dv_lora, None, None, None, None, None


def qkv_lora_rope(qkv, cos, sin, pos_ids, q_lora=None, v_lora=None, scale_q=2.0, scale_v=2.0,
                  h_q=12, h_kv=2, head_dim=128):
    return FusedQKVLoRARoPEFn.apply(qkv, cos, sin, pos_ids, q_lora, v_lora, scale_q, scale_v, h_q,
                                    h_kv, head_dim)


# ---------------------------------------------------------------------------------------------
# Chunked lm_head cross-entropy (solution/ops.py:174-349)
# ---------------------------------------------------------------------------------------------


def _lm_head_streamed(h_2d, labels, head: HostHead, num_items_in_batch, need_grad):
    """lm_head over a HostHead streamed from pinned host memory: one pass over the vocabulary
    chunks in order (``K.LMHeadPass``), each chunk copied once through the head's two-slot ring
    while the previous one computes and transposed on the device for the gradient GEMM; the label
    rows of the hidden gradient are read from the host by the finishing kernel. The reference
    streams W twice, forward chunks in order and gradient chunks in reverse
    (solution/ops.py:217-322)."""
    n_tok, d = h_2d.shape
    V, vc = head.vocab_size, head.v_chunk
    starts = list(range(0, V, vc))
    hp = K.LMHeadPass(n_tok, d, V, vc, h_2d.device, need_grad)
    head.prefetch_chunk(0, 0, min(vc, V))
    for c, s in enumerate(starts):
        e = min(s + vc, V)
        if c + 1 < len(starts):
            head.prefetch_chunk(c + 1, starts[c + 1], min(starts[c + 1] + vc, V))
        rows = head.get_chunk(c, s, e)
        rows_t = head.get_chunk_t(c, s, e) if need_grad else None
        hp.add_chunk(h_2d, rows, rows_t, s, labels)
        head.release_chunk(c)
    return hp.finish(labels, num_items_in_batch, head.cpu_weight)


class FusedChunkedLMHeadFn(torch.autograd.Function):
    """Cross-entropy loss, per-token NLL, entropy and argmax without the [N, V] logits (one pass
    over W in vocabulary chunks, ``K.LMHeadPass``); the hidden gradient (times 2^16) is formed in
    forward and rescaled by the incoming loss gradient in backward (solution/ops.py:174-339).
    Accumulation is fp32 (the reference's is fp16)."""

    @staticmethod
    def forward(ctx, hidden_states, shift_labels, weight_or_host_head, num_items_in_batch=None,
                v_chunk=None):
        h_2d = hidden_states.contiguous().view(-1, hidden_states.shape[-1])
        labels = shift_labels.contiguous().view(-1).to(torch.int64)
        is_head = isinstance(weight_or_host_head, HostHead)
        # Function.forward always runs with grad mode off, so torch.is_grad_enabled() (what the
        # reference tests, ops.py:280) is False here; ask autograd whether dH is needed instead.
        need_grad = bool(ctx.needs_input_grad[0])
        if is_head and not weight_or_host_head.resident:
            nll, lse, ent, amax, denom, dh_pre, loss = _lm_head_streamed(
                h_2d, labels, weight_or_host_head, num_items_in_batch, need_grad)
            loss = loss[0]
        else:
            if is_head:
                w, wt = weight_or_host_head.gpu_weight, weight_or_host_head.gpu_weight_t
            else:
                w, wt = weight_or_host_head.detach(), None
            v_chunk = lm_head_layout(v_chunk, h_2d.shape[0], w.shape[0], h_2d.device)
            nll, lse, ent, amax, denom, dh_pre, loss = K.lm_head_ce(
                h_2d, w, labels, num_items_in_batch=num_items_in_batch, v_chunk=v_chunk,
                need_grad=need_grad, weight_t=wt)
            loss = loss[0]
        ctx.save_for_backward(dh_pre)
        ctx.orig_shape = hidden_states.shape
        ctx.orig_dtype = hidden_states.dtype
        ctx.mark_non_differentiable(nll, ent, amax)
        return loss, nll, ent, amax

    @staticmethod
    def backward(ctx, grad_loss, _g_nll=None, _g_ent=None, _g_arg=None):
        (dh_pre,) = ctx.saved_tensors
        if dh_pre is None:
            return None, None, None, None, None
        g = grad_loss.detach().to(torch.float32).reshape(1)
        d_h = K.lm_head_dh_reduce(dh_pre.unsqueeze(0), 1.0 / PRESCALE_GRAD, ctx.orig_dtype,
                                  scale_dev=g)
        return d_h.view(ctx.orig_shape), None, None, None, None


def lm_head_layout(v_chunk, n_tok: int, n_vocab: int, device):
    """``v_chunk`` argument of K.lm_head_ce for a head layout choice: None or negative -> the
    single pass with the chunk chosen for ``n_tok`` tokens (K.lm_head_chunk_cols), and at least
    two chunks, so that no buffer holds a logit row of the whole vocabulary; a positive multiple
    of 256 -> that chunk; 0 -> None (the token-blocked head)."""
    if v_chunk is None or v_chunk < 0:
        c = K.lm_head_chunk_cols(n_tok, n_vocab, K.cu_count(device))
        if c >= n_vocab and n_vocab > K.LM_TILE:  # two chunks of whole 256-row tiles
            return K._round_up(-(-n_vocab // 2), K.LM_TILE)
        return c
    return int(v_chunk) if v_chunk > 0 else None


def chunked_lm_head(hidden_states, shift_labels, weight_or_host_head, num_items_in_batch=None,
                    v_chunk=None):
    """(loss, nll, entropy, argmax) of the lm_head cross-entropy (solution/ops.py:342-349).
    ``v_chunk`` sets the vocabulary rows per chunk, i.e. the [N, v_chunk] fp16 logit buffer
    (default: chosen for the token count within K.LM_CHUNK_BUDGET; 0: the token-blocked head; a
    streamed HostHead uses its own chunk)."""
    return FusedChunkedLMHeadFn.apply(hidden_states, shift_labels, weight_or_host_head,
                                      num_items_in_batch, v_chunk)


# ---------------------------------------------------------------------------------------------
# Fused 28-layer engine (solution/ops.py:599-1009)
# ---------------------------------------------------------------------------------------------


def rope_cache(max_pos: int, head_dim: int, theta: float, device, dtype=torch.float16):
    """cos/sin [max_pos, head_dim] of Qwen2's default rotary embedding (built once, in fp32 on the
    host, then cast; the reference takes it from the model's rotary module, ops.py:658-666)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(device, dtype).contiguous(), emb.sin().to(device, dtype).contiguous()


class Qwen2FusedEngine:
    """Streams, RoPE cache, norm weights and LoRA references of a QLoRA Qwen2 (ops.py:603-666).

    ``model`` is a ``rus_amd.model.QLoRAQwen2`` or a transformers/PEFT/bitsandbytes causal LM
    (read through ``rus_amd.adapters.layers_from_causal_lm``). ``layer_biases`` is defined here
    (the reference reads it from the engine but only defines it on its WeightStream).
    """

    def __init__(self, model, device, resident_weights: bool = False, resident_head: bool = True,
                 offload_inputs: bool = False, max_pos: int = 2048,
                 max_mlp_tokens: int = MAX_MLP_TOKENS, v_chunk: int = V_CHUNK_DEFAULT,
                 attention: str = "varlen", dropout_seed: int | None = None,
                 stream_unit: str = "layer", lora_kernels: bool = True, recompute: bool = True,
                 overlap: bool = False, gemm: str = "dequant", dequant_once: bool = False):
        from .model import QLoRAQwen2

        if not isinstance(model, QLoRAQwen2):
            from .adapters import model_from_causal_lm

            model = model_from_causal_lm(model)
        cfg = model.config
        self.device = torch.device(device)
        self.config = cfg
        self.num_layers = len(model.layers)
        self.hidden_size = cfg.hidden_size
        self.intermediate_size = cfg.intermediate_size
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.hidden_size // cfg.num_attention_heads
        self.rms_eps = float(cfg.rms_norm_eps)
        self.max_mlp_tokens = max_mlp_tokens
        self.weight_stream = WeightStream(model.layers, self.device, resident=resident_weights,
                                          unit=stream_unit)
        self.layer_biases = self.weight_stream.layer_biases
        self.host_head = HostHead(model.embed, self.device, v_chunk=v_chunk, resident=resident_head)
        self.input_stream = InputStream(self.num_layers, self.hidden_size, 2048, self.device,
                                        offload=offload_inputs)
        self.ln1_weights = [L.ln1.to(self.device) for L in model.layers]
        self.ln2_weights = [L.ln2.to(self.device) for L in model.layers]
        self.final_norm_weight = model.final_norm.to(self.device)
        self.lora_params = model.lora_parameters()
        self.layer_lora_meta = model.meta.get("layer_lora_meta") or [
            {"scale_q": cfg.lora_scaling, "scale_v": cfg.lora_scaling, "p_q": cfg.lora_dropout,
             "p_v": cfg.lora_dropout} for _ in model.layers]
        self.cos_table, self.sin_table = rope_cache(max_pos, self.head_dim, cfg.rope_theta,
                                                    self.device)
        if attention != "varlen":
            raise ValueError("attention must be 'varlen': the gfx950 varlen causal GQA kernels "
                             "over all packed rows are the engine's only attention path")
        if self.head_dim != K.ATTN_HEAD_DIM:
            raise ValueError(f"the varlen attention kernels run head_dim {K.ATTN_HEAD_DIM} only "
                             f"(got {self.head_dim})")
        self.attention = attention
        # recompute=True re-forms every layer's activations in the backward from its saved input
        # (the reference's memory-lean checkpointing); False keeps them from the forward (about
        # 60 bytes per token and hidden unit per layer for Qwen2.5-1.5B shapes), so the backward
        # skips three GEMMs, both norms, LoRA-down, RoPE and the attention forward per layer.
        self.recompute = bool(recompute)
        # overlap=True: each layer's NF4 dequant runs on a second stream one layer ahead (into
        # a second workspace set) while the current layer computes; needs the weights' packed
        # bytes on the device for the whole step (resident or stream_unit="model").
        # gemm="dequant": each layer's four NF4 segments are dequantised into fp16 workspaces
        # (one launch) and the products run on the library GEMM; "fused": the products decode
        # the NF4 bytes inside their MFMA main loop (K.nf4_gemm; no fp16 weight in HBM).
        if gemm not in ("dequant", "fused"):
            raise ValueError("gemm must be 'dequant' or 'fused'")
        if gemm == "fused" and overlap:
            raise ValueError("overlap (dequant one layer ahead) applies to gemm='dequant' only")
        self.gemm = gemm
        self.overlap = bool(overlap)
        if self.overlap:
            self.weight_stream.enable_dequant_ahead()
            self.side_stream = torch.cuda.Stream(device=self.device)  # default priority
        # dequant_once=True: the forward dequantises each layer into fp16 weights of the layer's
        # own (2.6 GB for Qwen2.5-1.5B) and the backward reads them, so a step runs one dequant
        # per layer instead of one per pass (the reference dequantises every segment again in
        # its backward, solution/ops.py:872-992, after the forward's ops.py:770-816).
        if dequant_once and (gemm != "dequant" or self.overlap):
            raise ValueError("dequant_once applies to gemm='dequant' without overlap")
        self.dequant_once = bool(dequant_once)
        if self.dequant_once:
            self.weight_stream.enable_dequant_once()
        self._flatten_lora()
        # The fused LoRA kernels (one launch for dropout + both A products, the B products inside
        # RoPE, two backward launches) cover ranks 4/8/16/32; other ranks use library GEMMs.
        ranks = {int(p.shape[0]) for p in self.lora_params[0::2]}
        self.fused_lora = bool(lora_kernels) and len(ranks) == 1 and ranks <= set(K.LORA_RANKS)
        # LoRA-down by blocks of four token rows (ranks 4/8/16, hidden a multiple of 64): the
        # product the layer's dequant launch can carry beside the input norm; every LoRA-down of
        # the engine then takes it, so all paths give the same bits.
        self.lora_rows = self.fused_lora and ranks <= set(K.LORA_ROWS_RANKS) and \
            self.hidden_size % 64 == 0
        # carry_lora_down: the input norm's blocks of the layer's dequant launch form its
        # LoRA-down (else a launch of its own, the same bits).
        self.carry_lora_down = self.lora_rows
        # lm_block_tokens: most tokens per block of the token-blocked lm_head (whole 256-token
        # tiles; None: the tiles whose fp16 logits fit K.LM_BLOCK_BUDGET).
        self.lm_block_tokens = None
        # lm_v_chunk: the lm_head layout, eager and captured. None (or negative): one pass over
        # vocabulary chunks (K.LMHeadPass: W read once, an [N, chunk] logit buffer) with the
        # chunk chosen for the token count within K.LM_CHUNK_BUDGET; a positive multiple of 256:
        # that chunk; 0: the token-blocked head ([block, V] logit buffers).
        self.lm_v_chunk = None
        # LoRA dropout: the counter-based masks of step k use seed (base + k), held on the device
        # so that a captured graph advances it by itself. The base comes from torch's CPU
        # generator unless given.
        if dropout_seed is None:
            dropout_seed = int(torch.randint(0, 2**62, (1,)).item())
        self.dropout_seed = torch.tensor([dropout_seed], dtype=torch.int64, device=self.device)
        self.last_dropout_seed = self.dropout_seed

    def next_dropout_seed(self) -> torch.Tensor:
        """Advances the device seed and returns a copy for one forward/backward pair."""
        self.dropout_seed.add_(1)
        self.last_dropout_seed = self.dropout_seed.clone()
        return self.last_dropout_seed

    @property
    def lora_numel(self) -> int:
        return self._lora_flat.numel()

    def lora_views(self, flat: torch.Tensor) -> list[torch.Tensor]:
        """Views of a flat buffer shaped like the LoRA parameters, in their order."""
        out, off = [], 0
        for p in self.lora_params:
            n = p.numel()
            out.append(flat[off: off + n].view(p.shape))
            off += n
        return out

    def _flatten_lora(self) -> None:
        """Makes the LoRA parameters views of one flat fp32 device buffer (same Parameter
        objects, so optimizers keep working) so that their fp16 copies for a step are one cast."""
        params = self.lora_params
        flat = torch.cat([p.detach().reshape(-1).to(self.device, torch.float32) for p in params])
        if getattr(self, "_lora_flat", None) is not None and self._lora_flat.numel() == flat.numel():
            self._lora_flat.copy_(flat)  # keep the address a captured graph reads
            flat = self._lora_flat
        off = 0
        for p in params:
            n = p.numel()
            p.data = flat[off: off + n].view(p.shape)
            off += n
        self._lora_flat = flat
        self._lora_ptrs = [p.data_ptr() for p in params]

    @property
    def flat_param(self):
        """The Parameter of ``flat_lora_parameter`` if it has been made, else None."""
        return getattr(self, "_flat_param", None)

    def flat_lora_parameter(self) -> torch.nn.Parameter:
        """One fp32 Parameter over the flat buffer that holds every LoRA factor (the LoRA
        parameters are views of it), so that an optimizer over it updates all factors with one
        fused launch; elementwise optimizers (AdamW) give the same values as over the separate
        factors. A captured step sets its ``.grad`` to the step's flat gradient."""
        if self.flat_param is None:
            self.sync_lora_storage()
            self._flat_param = torch.nn.Parameter(self._lora_flat, requires_grad=True)
        return self._flat_param

    def sync_lora_storage(self) -> None:
        """Re-points the LoRA parameters at the flat buffer if any was re-assigned (values kept)."""
        if [p.data_ptr() for p in self.lora_params] != self._lora_ptrs:
            self._flatten_lora()

    def _lora_layer_shapes(self) -> list[tuple[int, int]] | None:
        """[(rows, cols)] of one layer's four factors when every layer has the first layer's."""
        first = [tuple(p.shape) for p in self.lora_params[:4]]
        if len(first) != 4 or any(len(sh) != 2 for sh in first):
            return None
        for l in range(1, self.num_layers):
            if [tuple(p.shape) for p in self.lora_params[4 * l: 4 * l + 4]] != first:
                return None
        return first

    def lora_fp16(self) -> list[torch.Tensor]:
        """fp16 copies of [q_A, q_B, v_A, v_B] per layer for one step, one launch
        (rus_lora_cast_t); with the fused LoRA kernels the same launch writes their rank-major
        copies, which ``lora_fp16_t`` then returns."""
        self.sync_lora_storage()
        n = self._lora_flat.numel()
        flat16 = torch.empty(n, dtype=torch.float16, device=self.device)
        shapes = self._lora_layer_shapes() if n else None
        flat16t = torch.empty_like(flat16) if (self.fused_lora and shapes) else None
        if n:
            if shapes:
                K.lora_cast_t(self._lora_flat, self.num_layers, shapes, flat16, flat16t)
            else:
                K.lora_cast_t(self._lora_flat, 1, [(n, 1)], flat16)
        views = self.lora_views(flat16)
        self._lora16t = None
        if flat16t is not None:
            L = self.num_layers
            t_views = [None] * (4 * L)
            off = 0
            for j, (r0, c0) in enumerate(shapes):
                region = flat16t[L * off: L * (off + r0 * c0)].view(L, c0, r0)
                for l in range(L):
                    t_views[4 * l + j] = region[l]
                off += r0 * c0
            self._lora16t = (flat16, t_views)
        return views

    def lora_fp16_t(self, lora16: list[torch.Tensor]) -> list[torch.Tensor] | None:
        """Rank-major copies [q_A^T [D, r], q_B^T [r, Dq], v_A^T, v_B^T] per layer of a step's
        fp16 factors, for the fused LoRA backward: those ``lora_fp16`` wrote beside them, or (for
        factors from elsewhere) four batched transposes over all layers (the factors of every
        layer lie at one stride in the flat buffer). None without fused LoRA."""
        if not self.fused_lora:
            return None
        cached = getattr(self, "_lora16t", None)
        if cached is not None and lora16 and cached[0].data_ptr() == lora16[0].data_ptr():
            return cached[1]
        L = self.num_layers
        base = lora16[0]
        per_layer = sum(t.numel() for t in lora16[:4])
        out = [None] * (4 * L)
        off = 0
        for j in range(4):
            r0, c0 = lora16[j].shape
            v = torch.as_strided(base, (L, r0, c0), (per_layer, c0, 1),
                                 base.storage_offset() + off)
            t = v.transpose(1, 2).contiguous()  # [L, c0, r0]
            for l in range(L):
                out[4 * l + j] = t[l]
            off += r0 * c0
        return out


class VarlenMeta:
    """cu_seqlens of the packed rows (int32 on the device) and the longest row."""

    def __init__(self, row_lengths, device):
        lens = [int(L) for L in row_lengths if L > 0]
        cu = [0]
        for L in lens:
            cu.append(cu[-1] + L)
        self.cu = torch.tensor(cu, dtype=torch.int32, device=device)
        self.max_len = max(lens) if lens else 0
        self.lens = lens  # host copy (FLOP counts of the kernel timer only)

    @classmethod
    def from_device(cls, cu: torch.Tensor, max_len: int) -> "VarlenMeta":
        """From an existing int32 device buffer (a captured graph's static cu_seqlens)."""
        vm = cls.__new__(cls)
        vm.cu = cu
        vm.max_len = int(max_len)
        vm.lens = None
        return vm


def _varlen_attn_fwd(q, k, v, vm: VarlenMeta):
    """Causal GQA attention over all packed rows in one launch: q [N, Hq, D], k/v [N, Hkv, D]
    (the RoPE kernel's output layout) -> (out [N, Hq, D], lse [Hq, N]) (replaces the per-row SDPA
    loop with K/V expanded per group, solution/ops.py:669-696)."""
    return K.attn_varlen_fwd(q, k, v, vm.cu, lens=vm.lens)


def _varlen_attn_bwd(dout, q, k, v, out, lse, vm: VarlenMeta):
    return K.attn_varlen_bwd(dout, q, k, v, out, lse, vm.cu, lens=vm.lens)


def _dropout_on(meta, training) -> bool:
    return bool(training) and (meta["p_q"] > 0 or meta["p_v"] > 0)


def _lora_inputs(norm1, layer, meta, training, seed):
    """(x_q, x_v): the q- and v-branch LoRA inputs, dropped out with the counter-based masks of
    streams 2*layer and 2*layer + 1 (one kernel), or norm1 itself without dropout."""
    if _dropout_on(meta, training):
        return K.lora_dropout_fwd(norm1, seed, 2 * layer, 2 * layer + 1, meta["p_q"], meta["p_v"])
    return norm1, norm1


def _dropout_masks(engine, n_tok, training, seed):
    """Packed keep bits of every layer's two LoRA dropout masks for this step (streams 2l, 2l+1
    of the counter-based generator): per layer an int32 [2, n_tok, ceil(D / 32)] tensor, or None
    for a layer without dropout; one launch when all layers share their probabilities."""
    L = engine.num_layers
    metas = engine.layer_lora_meta
    if not training or not any(_dropout_on(m, training) for m in metas) or n_tok == 0:
        return [None] * L
    d = engine.hidden_size
    ps = {(m["p_q"], m["p_v"]) for m in metas}
    if len(ps) == 1:
        p_q, p_v = ps.pop()
        bits = K.dropout_keep_bits(seed, 0, 2 * L, n_tok, d, p_q, p_v)
        return [bits[2 * l: 2 * l + 2] for l in range(L)]
    return [K.dropout_keep_bits(seed, 2 * l, 2, n_tok, d, m["p_q"], m["p_v"])
            if _dropout_on(m, training) else None for l, m in enumerate(metas)]


def _lora_bits(masks, layer, meta):
    """(bits_q, bits_v, p_q, p_v) for the fused LoRA kernels of one layer (None: no dropout)."""
    m = masks[layer]
    if m is None:
        return None, None, 0.0, 0.0
    # both branches' bits (a branch with p = 0 keeps every element at scale 1)
    return m[0], m[1], meta["p_q"], meta["p_v"]


def _lora_deltas(x_q, x_v, qA, qB, vA, vB):
    """(mid_q, q_lora, mid_v, v_lora) = (x_q A_q^T, mid_q B_q^T, x_v A_v^T, mid_v B_v^T)."""
    mid_q = F.linear(x_q, qA)
    mid_v = F.linear(x_v, vA)
    return mid_q, F.linear(mid_q, qB), mid_v, F.linear(mid_v, vB)


def _lin(x, w, bias=None):
    """x W^T (+ bias) (F.linear, solution/ops.py:710-724, 771, 810): W is a dequantised fp16
    weight (library GEMM) or an NF4 operand (the fused dequant-in-GEMM kernel)."""
    if isinstance(w, K.NF4Operand):
        return K.nf4_gemm(x, w, bias=bias)
    return F.linear(x, w, bias)


def _mm_w(x, w):
    """x W, the input-gradient product (torch.mm, solution/ops.py:934, 939, 949, 993)."""
    if isinstance(w, K.NF4Operand):
        return K.nf4_gemm(x, w, trans=True)
    if x.shape[1] >= SPLIT_K_MIN:
        return _mm_split_k(x, w)
    return torch.mm(x, w)


def _mlp_fwd(norm2, w_gu, w_down, max_tokens):
    n = norm2.shape[0]
    if n <= max_tokens:
        return _lin(K.mlp_glu_fwd(_lin(norm2, w_gu)), w_down)
    out = torch.empty((n, w_down.shape[0]), dtype=norm2.dtype, device=norm2.device)
    for s in range(0, n, max_tokens):
        e = min(s + max_tokens, n)
        out[s:e] = _lin(K.mlp_glu_fwd(_lin(norm2[s:e], w_gu)), w_down)
    return out


SPLIT_K_MIN = 8192  # reduction length from which the [N, K] x [K, D] backward GEMM is split
# Output tiles (256 x 256) up to which the split-K MFMA kernel takes a long-K input gradient.
MFMA_SPLIT_TILES = 36


def _mm_split_k(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [M, K] @ b [K, D] (fp16) with K split: fp32 partials and one reduce kernel that rounds
    the sum to fp16 once (the single GEMM's rounding). For the long-K, narrow-output MLP backward
    product (K = 17920, D = 1536), where one GEMM leaves most of the GPU idle."""
    parts = _input_grad_parts(a, b)
    return torch.mm(a, b) if parts is None else K.sum_splits(parts, a.dtype)


def _input_grad_parts(a: torch.Tensor, b: torch.Tensor):
    """fp32 split-K partials [S, M, D] of the long-K input gradient a [M, K] @ b [K, D]
    (d_norm2 = torch.mm(d_gu, W_gu), solution/ops.py:939), or None where no split applies.
    Up to MFMA_SPLIT_TILES output tiles the split-K MFMA kernel (rus_gemm_parts, b read as
    stored) takes it, with S chosen so that its (tile, split) blocks fill one round of the 256
    CUs and every split keeps at least 512 columns; larger outputs fill the GPU by themselves
    and take the library's batched GEMM over 4 slices."""
    M, Kd = a.shape
    D = b.shape[1]
    if Kd < SPLIT_K_MIN or a.stride(1) != 1 or b.stride(1) != 1:
        return None
    tiles = -(-M // 256) * -(-D // 256)
    if (tiles <= MFMA_SPLIT_TILES and Kd % K.LM_K == 0 and D % 8 == 0 and a.stride(0) % 8 == 0
            and b.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0):
        return K.gemm_parts(a, b, True, max(1, min(64, 256 // tiles, Kd // 512)))
    return _split_k_parts(a, b)


def _split_k_parts(a: torch.Tensor, b: torch.Tensor, splits: int = 4):
    """The fp32 partial products [splits, M, D] of a [M, K] @ b [K, D] over K slices (one batched
    GEMM), or None where the split does not apply (short K, indivisible, non-contiguous)."""
    M, Kd = a.shape
    D = b.shape[1]
    if Kd < SPLIT_K_MIN or Kd % splits or a.stride(1) != 1 or not b.is_contiguous():
        return None
    ks = Kd // splits
    return torch.bmm(a.view(M, splits, ks).permute(1, 0, 2), b.view(splits, ks, D),
                     out_dtype=torch.float32)


class StackState:
    """What the stack's backward needs from its forward: final-norm input and rstd, positions,
    attention metadata, the step's fp16 LoRA copies, the dropout seed tensor, whether it ran
    in training mode, and (without recompute) each layer's saved activations (layer inputs live
    in the engine's InputStream)."""

    __slots__ = ("pos_ids", "h_last", "final_rstd", "vm", "row_lengths", "lora16", "training",
                 "seed", "buf", "saved", "masks", "lora16t")

    def __init__(self, **kw):
        self.saved = None
        self.masks = None
        self.lora16t = None
        for k, v in kw.items():
            setattr(self, k, v)


def _lora_down(engine, norm1, qA, vA, bits, out=None):
    """(mid_q, mid_v) of the fused LoRA path: by row blocks (``K.lora_down_rows``, the
    arithmetic a dequant launch carries) where the engine's rank allows, else by
    ``K.lora_down_fwd``."""
    if engine.lora_rows:
        return K.lora_down_rows(norm1, qA, vA, *bits, out=out)
    return K.lora_down_fwd(norm1, qA, vA, *bits, out=out)


def _layer_front(engine, l, norm1, w_qkv, lora16, training, seed, masks, pos_ids, mids=None):
    """q/k/v projection, LoRA deltas and RoPE of layer ``l`` (solution/ops.py:768-790) ->
    (q_rot, k_rot, v_out, lora) where lora = (mid_q, mid_v, x_q, x_v, bits): the rank-r
    intermediates, the dropped LoRA inputs of the library path (None with the fused kernels,
    which re-form them from norm1 and the keep bits) and the fused kernels' dropout arguments.
    ``mids``: (mid_q, mid_v) already formed (carried by the launch that formed norm1)."""
    cos, sin = engine.cos_table, engine.sin_table
    hq, hkv, hd = engine.num_heads, engine.num_kv_heads, engine.head_dim
    meta = engine.layer_lora_meta[l]
    qA, qB, vA, vB = lora16[4 * l: 4 * l + 4]
    bits = None
    if engine.fused_lora:  # dropout + A products in one launch, B products inside RoPE
        bits = _lora_bits(masks, l, meta)
        if mids is not None:
            mid_q, mid_v = mids
            qkv = _lin(norm1, w_qkv, engine.layer_biases[l])
        elif engine.overlap:  # the rank-r products on the side stream, beside the q/k/v GEMM
            main = torch.cuda.current_stream(norm1.device)
            n, r = norm1.shape[0], qA.shape[0]
            mids = (torch.empty((n, r), dtype=torch.float16, device=norm1.device),
                    torch.empty((n, r), dtype=torch.float16, device=norm1.device))
            side = engine.side_stream
            side.wait_stream(main)
            with torch.cuda.stream(side):
                _lora_down(engine, norm1, qA, vA, bits, out=mids)
            qkv = _lin(norm1, w_qkv, engine.layer_biases[l])
            main.wait_stream(side)
            mid_q, mid_v = mids
        else:
            mid_q, mid_v = _lora_down(engine, norm1, qA, vA, bits)
            qkv = _lin(norm1, w_qkv, engine.layer_biases[l])
        x_q = x_v = None
        q_rot, k_rot, v_out = K.qkv_rope_fwd_mid(
            qkv, mid_q, mid_v, qB, vB, cos, sin, pos_ids, meta["scale_q"], meta["scale_v"],
            hq, hkv, hd)
    else:
        qkv = _lin(norm1, w_qkv, engine.layer_biases[l])
        x_q, x_v = _lora_inputs(norm1, l, meta, training, seed)
        mid_q, q_lora, mid_v, v_lora = _lora_deltas(x_q, x_v, qA, qB, vA, vB)
        q_rot, k_rot, v_out = K.qkv_rope_fwd(qkv, cos, sin, pos_ids, q_lora=q_lora,
                                             v_lora=v_lora, scale_q=meta["scale_q"],
                                             scale_v=meta["scale_v"], h_q=hq, h_kv=hkv,
                                             head_dim=hd)
    return q_rot, k_rot, v_out, (mid_q, mid_v, x_q, x_v, bits)


def _norm_rides_dequant(engine) -> bool:
    """Whether a layer's RMSNorm can be deferred into the next dequant launch: the dequant runs
    on the current stream (not ahead on its own stream, not inside the fused products) and layer
    inputs stay in HBM (an offloaded input's slot is recycled once the layer releases it)."""
    return engine.gemm != "fused" and not engine.weight_stream.dequant_ahead and \
        not engine.input_stream.offload


def stack_forward(engine, h_packed, pos_ids, row_lengths, training, lora16, seed, vm=None,
                  save=False):
    """All decoder layers over packed tokens (solution/ops.py:736-830) -> (final_norm, state).

    No host synchronisation and no allocation outside torch's caching allocator, so it can run
    inside a captured HIP graph. Each layer's input residual add is fused into the RMSNorm kernel
    (h_{l+1} = h_mid + mlp is formed by the next layer's input norm) and the four weight segments
    of a layer are dequantised in one launch. With ``save`` every layer keeps what its backward
    reads (norm outputs and rstd, LoRA intermediates, rotated q/k/v, attention output and lse,
    the [gate|up] pre-activation), so the backward recomputes nothing; the values are the ones
    the recompute would produce, bit for bit."""
    ws, ins = engine.weight_stream, engine.input_stream
    L = engine.num_layers
    eps = engine.rms_eps
    h = h_packed.contiguous()
    carry = None  # (h_mid, mlp_out) of the previous layer, added inside the next norm
    n_tok = h.shape[0]
    hq, hd = engine.num_heads, engine.head_dim
    if vm is None:
        vm = VarlenMeta(row_lengths, engine.device)
    saved = [] if save else None
    masks = _dropout_masks(engine, n_tok, training, seed) if engine.fused_lora else [None] * L
    if L > 0:
        ws.prefetch(0)
    ahead = ws.dequant_ahead
    if ahead and L > 0:
        ws.issue_dequant(0)
    for l in range(L):
        if l + 1 < L:
            ws.prefetch(l + 1)
        if ahead and l + 1 < L:
            ws.issue_dequant(l + 1)  # beside this layer's compute
        # The input norm rides in the layer's dequant launch when that launch is on this stream.
        fused_gemm = engine.gemm == "fused"
        defer = _norm_rides_dequant(engine)
        if carry is None:
            norm1, _, rstd1, *pend = K.rms_norm_fwd(h, engine.ln1_weights[l], eps=eps,
                                                    defer=defer)
        else:
            norm1, h, rstd1, *pend = K.rms_norm_fwd(carry[1], engine.ln1_weights[l], eps=eps,
                                                    residual=carry[0], defer=defer)
        pend = pend[0] if pend else None
        mids = None
        if pend is not None and engine.carry_lora_down:  # LoRA-down in norm1's launch
            qA, vA = lora16[4 * l], lora16[4 * l + 2]
            bits = _lora_bits(masks, l, engine.layer_lora_meta[l])
            mids = pend.carry_lora_down(qA, vA, *bits)
        if fused_gemm:  # NF4 operands: the products decode the packed bytes themselves
            ws.wait_slot(l)
            W = ws.nf4_layer(l)
        elif ahead:
            W = ws.take_dequant(l)
        else:
            ws.wait_slot(l)
            W = ws.forward_weights(l, norm=pend)  # one launch: [q|k|v], o, [gate|up], down, norm
            ws.release_slot(l)
        if pend is not None:
            pend.run()  # no-op when the dequant launch carried it
        del pend
        ins.save(l, h)
        q_rot, k_rot, v_out, lora = _layer_front(engine, l, norm1, W["qkv"], lora16, training,
                                                 seed, masks, pos_ids, mids=mids)
        attn, lse = _varlen_attn_fwd(q_rot, k_rot, v_out, vm)
        attn = attn.view(n_tok, hq * hd)
        o_out = _lin(attn, W["o"])
        norm2, h_mid, rstd2 = K.rms_norm_fwd(o_out, engine.ln2_weights[l], eps=eps, residual=h)
        del o_out
        if save:
            gu = _lin(norm2, W["gu"])
            mlp_out = _lin(K.mlp_glu_fwd(gu), W["down"])
            saved.append({"norm1": norm1, "rstd1": rstd1, "lora": lora, "q_rot": q_rot,
                          "k_rot": k_rot, "v_out": v_out, "attn": attn, "lse": lse,
                          "h_mid": h_mid, "rstd2": rstd2, "norm2": norm2, "gu": gu})
        else:
            mlp_out = _mlp_fwd(norm2, W["gu"], W["down"], engine.max_mlp_tokens)
        if fused_gemm:
            ws.release_slot(l)  # the layer's last read of the packed slot is enqueued
        del norm1, lora, q_rot, k_rot, v_out, attn, norm2, W
        carry = (h_mid, mlp_out)
    if carry is None:
        final_norm, h_last, final_rstd = K.rms_norm_fwd(h, engine.final_norm_weight, eps=eps)
    else:
        final_norm, h_last, final_rstd = K.rms_norm_fwd(carry[1], engine.final_norm_weight,
                                                        eps=eps, residual=carry[0])
    st = StackState(pos_ids=pos_ids, h_last=h_last, final_rstd=final_rstd, vm=vm,
                    row_lengths=row_lengths, lora16=lora16, training=training, seed=seed,
                    masks=masks,
                    buf=ws.active if ws.unit == "model" else 0, saved=saved)
    return final_norm, st


def stack_backward(engine, st: StackState, d_final_norm, grad16) -> torch.Tensor:
    """Manual backward of every layer (solution/ops.py:832-1009), recomputing each layer's
    forward from its saved input as the reference does unless the forward saved its
    activations. Writes the fp16 LoRA gradients into ``grad16`` (flat, in the engine's
    parameter order) and returns the gradient of the packed embedding output."""
    ws, ins = engine.weight_stream, engine.input_stream
    L = engine.num_layers
    cos, sin, eps = engine.cos_table, engine.sin_table, engine.rms_eps
    training, seed, pos_ids = st.training, st.seed, st.pos_ids
    n_tokens = pos_ids.shape[0]
    hq, hkv, hd = engine.num_heads, engine.num_kv_heads, engine.head_dim
    q_dim = hq * hd
    gviews = engine.lora_views(grad16)

    # Each norm backward (the final norm's, then every layer's attention norm) is deferred into
    # the next layer's dequant launch when that launch runs on this stream (with dequant-once
    # the backward has no dequant launches: each norm runs on its own).
    defer = _norm_rides_dequant(engine) and not ws.dequant_once
    got = K.rms_norm_bwd(d_final_norm.contiguous(), st.h_last, engine.final_norm_weight,
                         st.final_rstd, defer=defer)
    dh, pend = got if defer else (got, None)
    st.lora16t = engine.lora_fp16_t(st.lora16)  # rank-major factors of the fused LoRA backward
    ws.use_buffer(st.buf)
    ahead = ws.dequant_ahead
    if L > 0:
        ws.prefetch(L - 1)
        if ahead:
            ws.issue_dequant(L - 1)
    for l in range(L - 1, -1, -1):
        if l - 1 >= 0:
            ws.prefetch(l - 1)
            ins.prefetch(l - 1, n_tokens)
            if ahead:
                ws.issue_dequant(l - 1)  # beside this layer's backward
        h_in = ins.load(l, n_tokens)
        fused_gemm = engine.gemm == "fused"
        if fused_gemm:
            ws.wait_slot(l)
            W = ws.nf4_layer(l)
        elif ahead:
            W = ws.take_dequant(l)
        elif ws.dequant_once:
            W = ws.stored_weights(l)  # the forward's dequant of this layer
        else:
            ws.wait_slot(l)
            W = ws.dequant_layer(l, norm=pend)
            ws.release_slot(l)  # every read of the packed slot is enqueued
        if pend is not None:
            pend.run()  # no-op when the dequant launch carried it
        pend = None
        w_qkv, w_o, w_gu, w_down = W["qkv"], W["o"], W["gu"], W["down"]
        meta = engine.layer_lora_meta[l]
        qA, qB, vA, vB = st.lora16[4 * l: 4 * l + 4]
        fused = engine.fused_lora
        gu = None
        if st.saved is not None:
            rec = st.saved[l]
            st.saved[l] = None  # freed as the backward moves down the stack
            norm1, rstd1 = rec["norm1"], rec["rstd1"]
            mid_q, mid_v, x_q, x_v, bits = rec["lora"]
            q_rot, k_rot, v_out = rec["q_rot"], rec["k_rot"], rec["v_out"]
            attn2d = rec["attn"]
            attn = attn2d.view(n_tokens, hq, hd)
            lse = rec["lse"]
            h_mid, rstd2, norm2, gu = rec["h_mid"], rec["rstd2"], rec["norm2"], rec["gu"]
            del rec
        else:
            # Recompute the layer forward (same dropout masks: same seed and streams).
            norm1, _, rstd1 = K.rms_norm_fwd(h_in, engine.ln1_weights[l], eps=eps)
            q_rot, k_rot, v_out, lora = _layer_front(engine, l, norm1, w_qkv, st.lora16,
                                                     training, seed, st.masks, pos_ids)
            mid_q, mid_v, x_q, x_v, bits = lora
            del lora
            attn, lse = _varlen_attn_fwd(q_rot, k_rot, v_out, st.vm)
            attn2d = attn.view(n_tokens, q_dim)
            o_out = _lin(attn2d, w_o)
            norm2, h_mid, rstd2 = K.rms_norm_fwd(o_out, engine.ln2_weights[l], eps=eps,
                                                 residual=h_in)
            del o_out

        # MLP backward: d_act = dh . W_down; SwiGLU backward in place over gu; d_norm2.
        step = min(engine.max_mlp_tokens, n_tokens)
        d_parts = None
        if gu is not None or step >= n_tokens:
            if gu is None:
                gu = _lin(norm2, w_gu)
            K.mlp_glu_bwd(_mm_w(dh, w_down), gu)
            if not isinstance(w_gu, K.NF4Operand):  # split-K partials go straight to the norm
                d_parts = _input_grad_parts(gu, w_gu)
            d_norm2 = _mm_w(gu, w_gu) if d_parts is None else None
            del gu
        else:
            d_norm2 = torch.empty_like(norm2)
            for s in range(0, n_tokens, step):
                e = min(s + step, n_tokens)
                gu = _lin(norm2[s:e], w_gu)
                K.mlp_glu_bwd(_mm_w(dh[s:e], w_down), gu)
                d_norm2[s:e] = _mm_w(gu, w_gu)
                del gu
        del norm2
        if d_parts is not None:
            dh_mid = K.rms_norm_bwd_parts(d_parts, h_mid, engine.ln2_weights[l], rstd2,
                                          dresidual=dh)
        else:
            dh_mid = K.rms_norm_bwd(d_norm2, h_mid, engine.ln2_weights[l], rstd2, dresidual=dh)
        del d_norm2, d_parts, h_mid, rstd2, dh

        # Attention backward, adjoint RoPE with [dQ|dK|dV] packing and LoRA-delta gradients.
        d_attn = _mm_w(dh_mid, w_o)
        # Fused LoRA at rank 16: d_mid from the RoPE backward's launch (which also sums each KV
        # group's per-query-head dK / dV partials left by the attention backward); the
        # input-gradient expansion beside the weight gradients in one launch.
        mid_fused = fused and K.rope_bwd_mid_supported(hq, hkv, hd, qA.shape[0])
        if mid_fused and hq // hkv <= 8:
            dq, dk, dv = K.attn_varlen_bwd_parts(d_attn.view(n_tokens, hq, hd), q_rot, k_rot,
                                                 v_out, attn, lse, st.vm.cu, lens=st.vm.lens)
        else:
            dq, dk, dv = _varlen_attn_bwd(d_attn.view(n_tokens, hq, hd), q_rot, k_rot, v_out,
                                          attn, lse, st.vm)
        del lse
        del attn, attn2d, d_attn, q_rot, k_rot, v_out
        if mid_fused:
            qBt, vBt = st.lora16t[4 * l + 1], st.lora16t[4 * l + 3]
            mid_fn = K.qkv_rope_bwd_lora_mid_parts if hq // hkv <= 8 else K.qkv_rope_bwd_lora_mid
            dqkv, dq_scaled, dv_scaled, d_mid_q, d_mid_v = mid_fn(
                dq, dk, dv, cos, sin, pos_ids, meta["scale_q"], meta["scale_v"], qBt, vBt,
                h_q=hq, h_kv=hkv, head_dim=hd)
        else:
            dqkv, dq_scaled, dv_scaled = K.qkv_rope_bwd_lora(dq, dk, dv, cos, sin, pos_ids,
                                                             meta["scale_q"], meta["scale_v"],
                                                             h_q=hq, h_kv=hkv, head_dim=hd)
        del dq, dk, dv

        # LoRA gradients (solution/ops.py:975-992): weight gradients into the flat buffer, input
        # gradients (through the forward's dropout masks) added into d_norm1.
        g_qA, g_qB, g_vA, g_vB = gviews[4 * l: 4 * l + 4]
        d_norm1 = _mm_w(dqkv, w_qkv)
        del dqkv
        if fused_gemm:
            ws.release_slot(l)  # the layer's last read of the packed slot is enqueued
        if mid_fused:  # the expansion into d_norm1 and all four weight gradients, one launch
            qAt, vAt = st.lora16t[4 * l], st.lora16t[4 * l + 2]
            K.lora_bwd_w(norm1, dq_scaled, dv_scaled, mid_q, mid_v, d_mid_q, d_mid_v, g_qA, g_qB,
                         g_vA, g_vB, *bits, expand=(qAt, vAt, d_norm1))
        elif fused:  # d_mid, the expansion, masks and both adds; then all four weight gradients
            qAt, qBt, vAt, vBt = st.lora16t[4 * l: 4 * l + 4]
            d_mid_q, d_mid_v = K.lora_bwd_x(dq_scaled, dv_scaled, qAt, vAt, qBt, vBt, d_norm1,
                                            *bits)
            K.lora_bwd_w(norm1, dq_scaled, dv_scaled, mid_q, mid_v, d_mid_q, d_mid_v, g_qA, g_qB,
                         g_vA, g_vB, *bits)
        else:
            torch.mm(dq_scaled.t(), mid_q, out=g_qB)
            d_mid_q = torch.mm(dq_scaled, qB)
            torch.mm(d_mid_q.t(), x_q, out=g_qA)
            dx_q = torch.mm(d_mid_q, qA)
            torch.mm(dv_scaled.t(), mid_v, out=g_vB)
            d_mid_v = torch.mm(dv_scaled, vB)
            torch.mm(d_mid_v.t(), x_v, out=g_vA)
            dx_v = torch.mm(d_mid_v, vA)
            if _dropout_on(meta, training):  # the forward's masks, then the two adds
                K.lora_dropout_bwd_add(d_norm1, dx_q, dx_v, seed, 2 * l, 2 * l + 1, meta["p_q"],
                                       meta["p_v"])
            else:
                d_norm1.add_(dx_q).add_(dx_v)
            del dx_q, dx_v
        del mid_q, mid_v, x_q, x_v, d_mid_q, d_mid_v, dq_scaled, dv_scaled, norm1
        got = K.rms_norm_bwd(d_norm1, h_in, engine.ln1_weights[l], rstd1, dresidual=dh_mid,
                             defer=defer)
        dh, pend = got if defer else (got, None)
        del got
        ins.release(l)
        del d_norm1, h_in, rstd1, dh_mid
    if pend is not None:
        pend.run()
    return dh


class FusedQwen2StackFn(torch.autograd.Function):
    """All decoder layers on packed tokens with layer-input checkpointing and recompute in
    backward (solution/ops.py:729-1009); with the engine's ``recompute=False`` the forward keeps
    every layer's activations instead (same values, no recompute). Returns the final-norm hidden
    states; the gradient flows to the LoRA parameters only.

    LoRA dropout masks come from a counter-based generator keyed by a per-forward seed (a device
    tensor drawn from the engine), so the recompute draws the same masks without saving or
    restoring torch's generator state."""

    @staticmethod
    def forward(ctx, h_packed, pos_ids, row_lengths, engine, training, *lora_params):
        seed = engine.next_dropout_seed() if training else engine.dropout_seed
        lora16 = engine.lora_fp16()
        ws = engine.weight_stream
        buf = ws.begin_step()
        save = not engine.recompute and any(ctx.needs_input_grad[5:])
        final_norm, st = stack_forward(engine, h_packed, pos_ids, row_lengths, training, lora16,
                                       seed, save=save)
        ws.end_step(buf)  # released again after the backward
        ctx.save_for_backward(*lora_params)
        ctx.st = st
        ctx.engine = engine
        return final_norm

    @staticmethod
    def backward(ctx, d_final_norm):
        engine = ctx.engine
        grad16 = torch.empty(engine.lora_numel, dtype=torch.float16, device=engine.device)
        dh = stack_backward(engine, ctx.st, d_final_norm, grad16)
        engine.weight_stream.end_step(ctx.st.buf)
        grads = engine.lora_views(grad16.float())  # the reference's .to(param dtype), one cast
        ctx.d_h_packed = dh  # gradient w.r.t. the embedding output (frozen), kept for tests
        del ctx.st
        return (None, None, None, None, None, *grads)


# ---------------------------------------------------------------------------------------------
# Padding-free varlen packing (solution/ops.py:1103-1127) and scatter back (ops.py:1151-1164)
# ---------------------------------------------------------------------------------------------


@dataclass
class PackedBatch:
    input_ids: torch.Tensor  # [N] int64
    pos_ids: torch.Tensor  # [N] int64, restarting per row
    shift_labels: torch.Tensor  # [N] int64, -100 where ignored
    row_lengths: list[int]
    valid_idx: torch.Tensor  # [N] flat indices into [B*S]
    batch_shape: tuple[int, int]


def pack_varlen(input_ids, attention_mask=None, labels=None, position_ids=None,
                vocab_size: int | None = None) -> PackedBatch:
    """keep = attention_mask | (shifted label != -100); positions = cumsum(mask) - 1 per row;
    the kept tokens of every row, concatenated (solution/ops.py:1103-1127). With ``vocab_size``,
    a kept token id outside [0, vocab_size) raises IndexError (checked in the one host
    synchronisation the row lengths need, so device inputs cost no extra round trip)."""
    B, S = input_ids.shape
    dev = input_ids.device
    if attention_mask is None:
        attention_mask = torch.ones((B, S), dtype=torch.long, device=dev)
    shift = torch.full((B, S), -100, dtype=torch.int64, device=dev)
    if labels is not None and S > 1:
        shift[:, :-1] = labels[:, 1:].to(torch.int64)
    keep = attention_mask.bool() | (shift != -100)
    if not keep.any():
        keep[:, 0] = True
    lens = keep.sum(dim=-1, dtype=torch.int64)
    if vocab_size is not None:
        bad = (keep & ((input_ids < 0) | (input_ids >= vocab_size))).sum().reshape(1)
        lens = torch.cat([lens, bad])
    row_lengths = lens.tolist()
    if vocab_size is not None and row_lengths.pop():
        raise IndexError(f"pack_varlen: a token id lies outside [0, {vocab_size})")
    valid_idx = torch.nonzero(keep.reshape(-1), as_tuple=False).squeeze(-1)
    pos_full = (position_ids.to(torch.long) if position_ids is not None
                else (attention_mask.to(torch.long).cumsum(dim=-1) - 1).clamp_(min=0))
    return PackedBatch(input_ids.reshape(-1).index_select(0, valid_idx),
                       pos_full.reshape(-1).index_select(0, valid_idx),
                       shift.reshape(-1).index_select(0, valid_idx), row_lengths, valid_idx, (B, S))


def scatter_per_token(values: torch.Tensor, packed: PackedBatch, fill=0.0) -> torch.Tensor:
    """[N] packed values -> [B, S], ``fill`` at positions that were not packed."""
    B, S = packed.batch_shape
    out = torch.full((B * S,), fill, dtype=values.dtype, device=values.device)
    out.index_copy_(0, packed.valid_idx, values)
    return out.view(B, S)


def fused_causal_lm_forward(engine: Qwen2FusedEngine, input_ids, attention_mask=None, labels=None,
                            num_items_in_batch=None, training: bool = True, position_ids=None):
    """Packed forward of the whole model with the fused lm_head (the body of the reference's
    patched Qwen2ForCausalLM.forward, solution/ops.py:1097-1164). Returns (loss, per-token nll,
    entropy, argmax) scattered back to [B, S]; padding positions get the mean entropy."""
    pb = pack_varlen(input_ids, attention_mask, labels, position_ids,
                     vocab_size=engine.host_head.vocab_size)
    h = engine.host_head.embed(pb.input_ids)
    final = FusedQwen2StackFn.apply(h, pb.pos_ids, pb.row_lengths, engine, training, *engine.lora_params)
    loss, nll, ent, amax = chunked_lm_head(final, pb.shift_labels, engine.host_head,
                                           num_items_in_batch=num_items_in_batch,
                                           v_chunk=engine.lm_v_chunk)
    mean_ent = ent.mean() if ent.numel() else torch.zeros((), device=ent.device)
    full_ent = mean_ent.expand(pb.batch_shape[0] * pb.batch_shape[1]).clone()
    full_ent.index_copy_(0, pb.valid_idx, ent)
    return (loss, scatter_per_token(nll, pb), full_ent.view(pb.batch_shape),
            scatter_per_token(amax, pb, 0))


def causal_lm_output(engine: Qwen2FusedEngine, input_ids, attention_mask=None, labels=None,
                     num_items_in_batch=None, training: bool = True, position_ids=None):
    """(loss, logits) of the fused packed forward where ``logits`` is a ``ChunkedLogitsProxy``
    [B, S, V] over the per-position statistics (solution/ops.py:1140-1186): what the patched
    ``Qwen2ForCausalLM.forward`` hands to the trainer."""
    loss, nll, ent, amax = fused_causal_lm_forward(engine, input_ids, attention_mask, labels,
                                                   num_items_in_batch, training, position_ids)
    proxy = ChunkedLogitsProxy(nll, ent, amax, engine.host_head.vocab_size,
                               dtype=torch.float16)
    return loss, proxy


def _fusable(causal_lm, input_ids, labels) -> bool:
    """Whether a transformers causal LM call can take the fused path: CUDA (HIP) token ids and
    labels, and PEFT LoRA on q_proj / v_proj over bitsandbytes 4-bit base layers (the attribute
    layout ``rus_amd.adapters`` reads; solution/ops.py:1041-1061 guards the same way)."""
    if not (isinstance(input_ids, torch.Tensor) and isinstance(labels, torch.Tensor)):
        return False
    if input_ids.device.type != "cuda" or labels.device.type != "cuda":
        return False
    layers = getattr(getattr(causal_lm, "model", None), "layers", None)
    if not layers:
        return False
    attn = getattr(layers[0], "self_attn", None)
    q, v = getattr(attn, "q_proj", None), getattr(attn, "v_proj", None)
    if not (hasattr(q, "lora_A") and hasattr(v, "lora_A")):
        return False
    base = getattr(q, "base_layer", q)
    return getattr(getattr(base, "weight", None), "quant_state", None) is not None


def _patch_transformers_qwen2() -> bool:
    try:
        from transformers.modeling_outputs import CausalLMOutputWithPast
        from transformers.models.qwen2 import modeling_qwen2
    except ImportError:
        return False
    cls = modeling_qwen2.Qwen2ForCausalLM
    if getattr(cls.forward, "_rus_fused", False):
        return True
    unfused = cls.forward

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, labels=None, use_cache=None, output_attentions=None,
                output_hidden_states=None, return_dict=None, **kwargs):
        if (inputs_embeds is not None or past_key_values is not None or output_attentions
                or output_hidden_states or not _fusable(self, input_ids, labels)):
            extra = {k: v for k, v in (("output_attentions", output_attentions),
                                        ("output_hidden_states", output_hidden_states),
                                        ("return_dict", return_dict)) if v is not None}
            return unfused(self, input_ids=input_ids, attention_mask=attention_mask,
                           position_ids=position_ids, past_key_values=past_key_values,
                           inputs_embeds=inputs_embeds, labels=labels, use_cache=use_cache,
                           **extra, **kwargs)
        engine = self.__dict__.get("_rus_fused_engine")
        if engine is None:
            engine = Qwen2FusedEngine(self, input_ids.device)
            self.__dict__["_rus_fused_engine"] = engine
        loss, proxy = causal_lm_output(engine, input_ids, attention_mask, labels,
                                       kwargs.get("num_items_in_batch"), self.training,
                                       position_ids)
        if return_dict is False:
            return (loss, proxy)
        return CausalLMOutputWithPast(loss=loss, logits=proxy)

    forward._rus_fused = True
    forward.__wrapped__ = unfused
    cls.forward = forward
    return True


_KERNEL_DTYPES = (torch.float16, torch.float32)


def _patch_qwen2_mlp() -> bool:
    """``Qwen2MLP.forward`` → down_proj(mlp_glu(gate_proj(x), up_proj(x))) for device tensors of
    a kernel dtype with the SiLU activation, for the calls the fused stack does not take (eval
    without labels, generation); anything else keeps transformers' code (solution/ops.py:1029-1033,
    1186)."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except ImportError:
        return False
    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_rus_fused", False):
        return True
    unfused = cls.forward

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not isinstance(x, torch.Tensor) or not x.is_cuda:
            return unfused(self, x)
        gate, up = self.gate_proj(x), self.up_proj(x)
        if gate.dtype not in _KERNEL_DTYPES or up.dtype != gate.dtype:
            return self.down_proj(self.act_fn(gate) * up)
        return self.down_proj(mlp_glu(gate, up))

    forward._rus_fused = True
    forward.__wrapped__ = unfused
    cls.forward = forward
    return True


def _patch_qwen2_rmsnorm() -> bool:
    """``Qwen2RMSNorm.forward`` → ``rms_norm`` (one-pass kernel, output in the input's dtype, the
    reference's behaviour, solution/ops.py:1035-1039, 1187) for device tensors of a kernel dtype.
    The kernel's backward forms no weight gradient (the norms are frozen under QLoRA), so a norm
    whose weight requires grad under autograd keeps transformers' code."""
    try:
        from transformers.models.qwen2 import modeling_qwen2
    except ImportError:
        return False
    cls = modeling_qwen2.Qwen2RMSNorm
    if getattr(cls.forward, "_rus_fused", False):
        return True
    unfused = cls.forward

    def forward(self, hidden_states):
        w = self.weight
        if (not isinstance(hidden_states, torch.Tensor) or not hidden_states.is_cuda
                or hidden_states.dtype not in _KERNEL_DTYPES or w.dtype not in _KERNEL_DTYPES
                or (w.requires_grad and torch.is_grad_enabled())):
            return unfused(self, hidden_states)
        eps = float(getattr(self, "variance_epsilon", getattr(self, "eps", 1e-6)))
        return rms_norm(hidden_states, w, eps=eps)

    forward._rus_fused = True
    forward.__wrapped__ = unfused
    cls.forward = forward
    return True


def _patch_trl_entropy() -> bool:
    try:
        import trl.trainer.sft_trainer as sft  # TRL 0.29.1 (solution/ops.py:1223-1238)
    except ImportError:
        return False
    plain = getattr(sft, "entropy_from_logits", None)
    if plain is None:
        return False
    if getattr(plain, "_rus_fused", False):
        return True

    def entropy_from_logits(logits, *args, **kwargs):
        if isinstance(logits, ChunkedLogitsProxy):
            return logits.per_token_entropy
        return plain(logits, *args, **kwargs)

    entropy_from_logits._rus_fused = True
    entropy_from_logits.__wrapped__ = plain
    sft.entropy_from_logits = entropy_from_logits
    return True


def install_runtime_patches() -> dict[str, bool]:
    """Routes a transformers ``Qwen2ForCausalLM`` training forward with QLoRA (PEFT LoRA on q / v
    over bitsandbytes NF4) and CUDA inputs through the fused engine, returning the loss and a
    ``ChunkedLogitsProxy``; routes the remaining ``Qwen2MLP`` / ``Qwen2RMSNorm`` calls on device
    tensors through the SwiGLU and RMSNorm kernels; and makes TRL's ``entropy_from_logits`` read
    the proxy's entropy (solution/ops.py:1016-1238). Any other call keeps the library's own code.
    Idempotent; returns which patches are active (a library that is not importable is skipped,
    where the reference swallows every exception)."""
    return {"transformers_qwen2": _patch_transformers_qwen2(),
            "qwen2_mlp": _patch_qwen2_mlp(),
            "qwen2_rmsnorm": _patch_qwen2_rmsnorm(),
            "trl_entropy": _patch_trl_entropy()}
