"""One DSpark draft layer's training step on MI355X (the full one-layer step of the benchmark
configurations: Qwen3-8B dims, hidden 4096, GQA 32/8 x 128, SwiGLU FFN 12288, RMSNorm, RoPE
theta 1e6, fwd + CE/L1 loss + bwd + AdamW).

Follows the reference's DFlash/DSpark draft model (aspec/models/draft/dflash.py):
  context  = RMSNorm(context_proj(target_hidden))                       (dflash.py:1258-1284)
  draft    = embed_tokens(draft_input_ids)                              (dflash.py:1315-1318)
  layer    : r = draft; x = input_layernorm(draft)                      (dflash.py:1015-1062)
             q = q_proj(x); k/v from context and draft (shared k/v_proj) (dflash.py:470-481)
             q, k = Q/K RMSNorm + RoPE (fused kernel)                    (dflash.py:826-877)
             attention over the DSpark block-sparse mask (direct CP at CP=1)
             h = r + o_proj(attn); x = post_attention_layernorm(h)
             h = h + down_proj(silu(gate_proj(x)) * up_proj(x))         (dflash.py:967-980)
  hidden   = final_norm(h)                                               (dflash.py:1471)
  logits   = hidden @ W_head^T (frozen), loss = 0.1 CE + 0.9 L1 against the frozen head's
             logits of the aligned target hidden states, weighted by the DSpark decay weights
and the reference's optimizer (`BF16Optimizer`, aspec/training/optimizer.py:40-164).

MI355X-specific layout: the residual adds are fused into the following RMSNorm (one pass writes
the sum and its normalisation), gate and up are one [2F, H] weight and one GEMM feeding the SwiGLU
kernel, and the optimizer keeps every trainable parameter as a view of one flat bf16 buffer with
flat fp32 master / moment buffers, updated by one fused kernel pass that reads each gradient where
autograd left it (a table of per-parameter segments), with the clip norm and the skip decision on
the device.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch
import torch.nn as nn
from torch.autograd.function import once_differentiable

from . import _lib, _timing

__all__ = ["rms_norm", "swiglu", "DSparkDraftLayerModel", "FusedBF16Optimizer",
           "warmup_decay_lr", "rope_tables", "dspark_layer_step", "layer_batch"]


def _check_rows(name, t, width):
    if not t.is_cuda or t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be a bf16 CUDA tensor")
    if not t.is_contiguous() or t.shape[-1] != width:
        raise ValueError(f"{name} must be contiguous with last dimension {width}")


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, residual, weight, eps):
        hidden = x.shape[-1]
        _check_rows("x", x, hidden)
        if residual is not None:
            _check_rows("residual", residual, hidden)
            if residual.shape != x.shape:
                raise ValueError("residual must match x")
        if weight.dtype != torch.bfloat16 or weight.numel() != hidden or not weight.is_contiguous():
            raise ValueError("RMSNorm weight must be a contiguous bf16 [hidden] tensor")
        rows = x.numel() // hidden
        out = torch.empty_like(x)
        y = torch.empty_like(x) if residual is not None else None
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        with _timing.region("rmsnorm_fwd"):
            _lib.call("aspec_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(residual), _lib.ptr(weight), rows,
                      hidden, float(eps), _lib.ptr(y), _lib.ptr(out), _lib.ptr(rstd),
                      _lib.stream_handle(x.device))
        ctx.save_for_backward(y if y is not None else x, weight, rstd)
        ctx.has_residual = residual is not None
        if residual is not None:
            return y, out
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, *grads):
        y, weight, rstd = ctx.saved_tensors
        if ctx.has_residual:
            dy_extra, dout = grads
        else:
            (dout,) = grads
            dy_extra = None
        hidden = y.shape[-1]
        rows = y.numel() // hidden
        if dout is None:
            dout = torch.zeros_like(y)
        dout = dout.to(torch.bfloat16).contiguous()
        dy_extra = None if dy_extra is None else dy_extra.to(torch.bfloat16).contiguous()
        dy = torch.empty_like(y)
        dw = torch.empty(hidden, dtype=torch.float32, device=y.device)
        size = ctypes.c_size_t()
        _lib.call("aspec_rmsnorm_bwd_workspace_bytes", hidden, ctypes.byref(size))
        workspace = torch.empty(size.value, dtype=torch.uint8, device=y.device)
        with _timing.region("rmsnorm_bwd"):
            _lib.call("aspec_rmsnorm_bwd", _lib.ptr(dout), _lib.ptr(dy_extra), _lib.ptr(y),
                      _lib.ptr(weight), _lib.ptr(rstd), rows, hidden, _lib.ptr(dy), _lib.ptr(dw),
                      _lib.ptr(workspace), _lib.stream_handle(y.device))
        dweight = dw.to(weight.dtype)
        if ctx.has_residual:
            return dy, dy, dweight, None
        return dy, None, dweight, None


def rms_norm(x, weight, eps, residual=None):
    """RMSNorm of x (or of y = x + residual, returned first): `_dflash_rms_norm`
    (aspec/models/draft/dflash.py:282-293) with one bf16 rounding, fused residual add."""
    return _RMSNorm.apply(x, residual, weight, eps)


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate_up):
        ffn = gate_up.shape[-1] // 2
        _check_rows("gate_up", gate_up, 2 * ffn)
        rows = gate_up.numel() // (2 * ffn)
        out = torch.empty(*gate_up.shape[:-1], ffn, dtype=gate_up.dtype, device=gate_up.device)
        with _timing.region("swiglu_fwd"):
            _lib.call("aspec_swiglu_fwd", _lib.ptr(gate_up), rows, ffn, _lib.ptr(out),
                      _lib.stream_handle(gate_up.device))
        ctx.save_for_backward(gate_up)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        (gate_up,) = ctx.saved_tensors
        ffn = gate_up.shape[-1] // 2
        rows = gate_up.numel() // (2 * ffn)
        dout = dout.to(torch.bfloat16).contiguous()
        dgu = torch.empty_like(gate_up)
        with _timing.region("swiglu_bwd"):
            _lib.call("aspec_swiglu_bwd", _lib.ptr(dout), _lib.ptr(gate_up), rows, ffn,
                      _lib.ptr(dgu), _lib.stream_handle(gate_up.device))
        return dgu


def swiglu(gate_up):
    """silu(gate) * up for gate_up = [gate | up] (`DFlashMLP`, dflash.py:967-980)."""
    return _SwiGLU.apply(gate_up)


def rope_tables(max_positions, head_dim, theta, device, dtype=torch.bfloat16):
    """cos / sin [1, 1, P, D] as `DFlashRotaryEmbedding` builds them (dflash.py:191-239): fp32
    phases of the default rope type, cast to the activation dtype."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    t = torch.arange(max_positions, device=device, dtype=torch.float32)
    emb = torch.cat((torch.outer(t, inv),) * 2, dim=-1)
    return emb.cos()[None, None].to(dtype), emb.sin()[None, None].to(dtype)


class DSparkDraftLayerModel(nn.Module):
    """A one-layer DSpark draft model (dense FFN) with its frozen embedding and head."""

    def __init__(self, *, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288,
                 num_target_layers=3, vocab=151936, draft_vocab=32000, rope_theta=1e6, eps=1e-6,
                 max_positions=8192, device=None, dtype=torch.bfloat16, seed=0):
        super().__init__()
        self.hidden, self.heads, self.kv_heads, self.head_dim, self.ffn = hidden, heads, kv_heads, head_dim, ffn
        self.eps = eps
        g = torch.Generator(device=device or "cpu").manual_seed(seed)

        def param(*shape, std=0.02, ones=False, trainable=True):
            if ones:
                t = torch.ones(*shape, device=device)
            else:
                t = torch.randn(*shape, generator=g, device=device) * std
            return nn.Parameter(t.to(dtype), requires_grad=trainable)

        self.embed_tokens = param(vocab, hidden, trainable=False)      # frozen Target copy
        self.lm_head = param(draft_vocab, hidden, trainable=False)     # frozen Target head slice
        self.context_proj = param(hidden, num_target_layers * hidden)
        self.context_norm = param(hidden, ones=True)
        self.input_layernorm = param(hidden, ones=True)
        self.q_proj = param(heads * head_dim, hidden)
        self.k_proj = param(kv_heads * head_dim, hidden)
        self.v_proj = param(kv_heads * head_dim, hidden)
        self.q_norm = param(head_dim, ones=True)
        self.k_norm = param(head_dim, ones=True)
        self.o_proj = param(hidden, heads * head_dim)
        self.post_attention_layernorm = param(hidden, ones=True)
        self.gate_up_proj = param(2 * ffn, hidden)                     # [gate; up]
        self.down_proj = param(hidden, ffn)
        self.final_norm = param(hidden, ones=True)
        cos, sin = rope_tables(max_positions, head_dim, rope_theta, device, dtype)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        # the frozen head's transposed copy: the logits' dgrad runs in the TN layout
        self.register_buffer("lm_head_t", self.lm_head.detach().t().contiguous(), persistent=False)

    def forward(self, target_hidden, draft_input_ids, context_positions, draft_positions, metadata):
        """target_hidden [1, T, L*H] bf16, draft_input_ids / draft_positions [1, Nq] int64,
        context_positions [1, T] int64 (RoPE ids), metadata: DirectCPMetadata -> [Nq, H]."""
        from .direct_cp import direct_cp_attention_from_kv
        from .dspark_qk_norm_rope import dspark_qk_norm_rope

        H, D, hq, hkv = self.hidden, self.head_dim, self.heads, self.kv_heads
        T, nq = target_hidden.shape[1], draft_input_ids.shape[1]
        ctx = rms_norm(target_hidden.reshape(T, -1) @ self.context_proj.t(), self.context_norm, self.eps)
        draft = self.embed_tokens[draft_input_ids.reshape(-1)]
        x = rms_norm(draft, self.input_layernorm, self.eps)
        q = (x @ self.q_proj.t()).view(1, nq, hq * D)
        k_ctx = (ctx @ self.k_proj.t()).view(1, T, hkv * D)
        k_draft = (x @ self.k_proj.t()).view(1, nq, hkv * D)
        v = torch.cat((ctx @ self.v_proj.t(), x @ self.v_proj.t()), dim=0).view(1, T + nq, hkv, D)
        q, k = dspark_qk_norm_rope(q, k_ctx, k_draft, self.q_norm, self.k_norm, self.eps, self.rope_cos,
                                   self.rope_sin, draft_positions, context_positions, draft_positions,
                                   hq, hkv, D)
        attn, _ = direct_cp_attention_from_kv(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                              metadata)
        o = attn.transpose(1, 2).reshape(nq, hq * D) @ self.o_proj.t()
        h, x2 = rms_norm(o, self.post_attention_layernorm, self.eps, residual=draft)
        mlp = swiglu(x2 @ self.gate_up_proj.t()) @ self.down_proj.t()
        _, hidden = rms_norm(mlp, self.final_norm, self.eps, residual=h)
        return hidden


def warmup_decay_lr(step, *, max_lr, total_steps, warmup_steps=0, min_lr=0.0, init_lr=0.0,
                    decay_style="cosine"):
    """`LRSchedulerWithWarmup._get_lr_for_group` (aspec/training/lr_scheduler.py) for the
    constant, linear and cosine decay styles."""
    if warmup_steps > 0 and step <= warmup_steps:
        return init_lr + (max_lr - init_lr) * step / warmup_steps
    if decay_style == "constant":
        return max_lr
    if step > total_steps:
        return min_lr
    ratio = min(1.0, max(0.0, (step - warmup_steps) / float(total_steps - warmup_steps)))
    if decay_style == "linear":
        coeff = 1.0 - ratio
    elif decay_style == "cosine":
        coeff = 0.5 * (math.cos(math.pi * ratio) + 1.0)
    else:
        raise NotImplementedError(f"decay style {decay_style!r} is not implemented here")
    return min_lr + coeff * (max_lr - min_lr)


class FusedBF16Optimizer:
    """`BF16Optimizer` (aspec/training/optimizer.py:40-164) as one fused HIP pass: bf16 model
    parameters become views of one flat buffer with fp32 master weights and moments. `step()` reads
    each gradient where autograd left it (one segment per parameter; a parameter whose grad is None
    is skipped, as torch's optimizers do), clips to max_grad_norm, skips a non-finite step, applies
    AdamW (torch's fused semantics, one step count per parameter) and refreshes the bf16 weights;
    it returns the pre-clip gradient norm as a device scalar (no host synchronization) and, as the
    reference's step does, leaves every grad None. `zero_grad(set_to_none=False)` instead keeps every gradient as a view of one flat bf16 buffer
    that autograd accumulates into. With more than 64 trainable parameters, or one whose size is
    not a multiple of 8, the gradients are gathered into that buffer and updated as one segment;
    that path cannot skip a single parameter, so a step in which some parameter has no gradient
    raises NotImplementedError there (the reference's AdamW would leave it untouched)."""

    def __init__(self, model, lr, weight_decay=0.0, max_grad_norm=0.5, total_steps=800_000,
                 warmup_ratio=0.015, decay_style="cosine", min_lr=0.0, betas=(0.9, 0.999), eps=1e-8):
        self.params = [p for p in model.parameters() if p.requires_grad]
        if not self.params:
            raise ValueError("no trainable parameters")
        dev = self.params[0].device
        if any(p.dtype != torch.bfloat16 or p.device != dev for p in self.params):
            raise ValueError("the fused optimizer serves bf16 parameters on one device")
        self.numel = sum(p.numel() for p in self.params)
        self._pad = (-self.numel) % 8
        self.flat = torch.empty(self.numel + self._pad, dtype=torch.bfloat16, device=dev)
        self._grads = None  # the flat gradient buffer, made on first use
        off = 0
        for p in self.params:
            n = p.numel()
            self.flat[off:off + n].copy_(p.detach().reshape(-1))
            p.data = self.flat[off:off + n].view_as(p)
            p.grad = None
            off += n
        if self._pad:
            self.flat[self.numel:].zero_()
        self.master = self.flat.float()
        self.exp_avg = torch.zeros_like(self.master)
        self.exp_avg_sq = torch.zeros_like(self.master)
        self.state = torch.zeros(_lib.load().aspec_adamw_state_bytes(), dtype=torch.uint8, device=dev)
        size = ctypes.c_size_t()
        _lib.call("aspec_adamw_workspace_bytes", ctypes.byref(size))
        self.workspace = torch.empty(size.value, dtype=torch.uint8, device=dev)
        self.lr, self.weight_decay, self.max_grad_norm = lr, weight_decay, max_grad_norm
        self.betas, self.eps = betas, eps
        self.schedule = dict(max_lr=lr, total_steps=total_steps,
                             warmup_steps=int(warmup_ratio * total_steps), min_lr=min_lr,
                             decay_style=decay_style)
        self.last_step = 0  # scheduler position (advances every step, as the reference's does)
        numel = [p.numel() for p in self.params]
        self._seg_numel = (ctypes.c_int64 * len(numel))(*numel)
        self._segments_ok = len(numel) <= 64 and all(n % 8 == 0 for n in numel[:-1])

    @property
    def grads(self):
        """The flat bf16 gradient buffer (zeroed when first made)."""
        if self._grads is None:
            self._grads = torch.zeros(self.numel + self._pad, dtype=torch.bfloat16, device=self.flat.device)
        return self._grads

    def get_learning_rate(self):
        return warmup_decay_lr(self.last_step, **self.schedule)

    def zero_grad(self, set_to_none=True):
        if set_to_none:
            for p in self.params:
                p.grad = None
            return
        self.grads.zero_()
        for p, off in zip(self.params, self._offsets()):
            if p.grad is None or p.grad.data_ptr() != self.grads[off:].data_ptr():
                p.grad = self.grads[off:off + p.numel()].view_as(p)

    def _offsets(self):
        off = 0
        for p in self.params:
            yield off
            off += p.numel()

    def _segment_grads(self):
        """Device pointers of the gradients, one segment per parameter (0 for a grad of None); a
        gradient that is not a contiguous, 16-byte aligned bf16 tensor of the parameter's shape is
        first copied into the parameter's slice of the flat gradient buffer."""
        ptrs = []
        for p, off in zip(self.params, self._offsets()):
            g = p.grad
            if g is None:
                ptrs.append(0)
            elif (g.dtype == torch.bfloat16 and g.device == p.device and g.shape == p.shape
                  and g.is_contiguous() and g.data_ptr() % 16 == 0):
                ptrs.append(g.data_ptr())
            else:
                view = self.grads[off:off + p.numel()].view_as(p)
                view.copy_(g)
                ptrs.append(view.data_ptr())
        return (ctypes.c_void_p * len(ptrs))(*ptrs)

    def step(self, closure=None):
        del closure
        lr = self.get_learning_rate()
        args = (float(lr), float(self.weight_decay), float(self.betas[0]), float(self.betas[1]),
                float(self.eps), float(self.max_grad_norm), _lib.ptr(self.state),
                _lib.ptr(self.workspace), _lib.stream_handle(self.flat.device))
        with _timing.region("adamw_step"):
            if self._segments_ok:
                _lib.call("aspec_adamw_step_segments", _lib.ptr(self.flat), _lib.ptr(self.master),
                          _lib.ptr(self.exp_avg), _lib.ptr(self.exp_avg_sq), self._segment_grads(),
                          self._seg_numel, len(self.params), *args)
            else:
                # more than 64 parameters, or one whose size is not a multiple of 8: every gradient
                # is gathered into the flat buffer and the update runs as one segment, which has
                # one step count and applies decay to every element, so a parameter without a
                # gradient cannot be skipped as the reference's AdamW skips it (optimizer.py:99-109)
                missing = sum(p.grad is None for p in self.params)
                if 0 < missing < len(self.params):
                    raise NotImplementedError(
                        f"{missing} of {len(self.params)} trainable parameters have no gradient; the "
                        "gathered AdamW path (more than 64 parameters, or a parameter whose size is "
                        "not a multiple of 8) cannot skip them")
                if missing == len(self.params):
                    # nothing to update (every parameter is skipped); the norm of no gradients is 0
                    self.grad_norm().zero_()
                else:
                    for p, off in zip(self.params, self._offsets()):
                        view = self.grads[off:off + p.numel()].view_as(p)
                        if p.grad.data_ptr() != view.data_ptr():
                            view.copy_(p.grad)
                    _lib.call("aspec_adamw_step", _lib.ptr(self.flat), _lib.ptr(self.master),
                              _lib.ptr(self.exp_avg), _lib.ptr(self.exp_avg_sq), _lib.ptr(self.grads),
                              self.flat.numel(), *args)
        self.last_step += 1
        for p in self.params:  # as the reference's step does: the gradients are consumed
            p.grad = None
        return self.grad_norm()

    def grad_norm(self):
        """The last step's gradient norm before clipping (device scalar)."""
        return self.state[24:28].view(torch.float32)[0]

    def optimizer_steps(self):
        """Steps taken (non-finite steps excluded) -- synchronizes."""
        return int(self.state[0:8].view(torch.int64)[0].item())


def layer_batch(model, workload, *, seed=0, num_target_layers=3, mask_token=None, decay_gamma=4.0):
    """Synthetic inputs of one packed row for `dspark_layer_step`, on the model's device:
    target hidden states [1, T, L*H] and the aligned teacher hidden states [1, T, H] (N(0, 1), bf16),
    token ids uniform over the embedding vocabulary, mapped into the draft vocabulary by id modulo
    its size (a synthetic choice: the reference's DSpark path has no vocabulary map), draft inputs
    [anchor token, mask, ..., mask] per block (dflash.py:1315-1318), document-local RoPE positions
    for the context and anchor position + offset for the draft, the direct-CP metadata (CP = 1)
    and the DSpark targets (dspark.py:240-272)."""
    from .anchors import validate_injected_anchors
    from .direct_cp import DirectCPMetadata
    from .targets import dspark_targets

    dev = model.lm_head.device
    w = workload
    T, nb, B = w.context_length, w.num_blocks, w.block_size
    vocab, draft_vocab = model.embed_tokens.shape[0], model.lm_head.shape[0]
    g = torch.Generator(device="cpu").manual_seed(seed)
    target_hidden = torch.randn(1, T, num_target_layers * model.hidden, generator=g).to(dev, torch.bfloat16)
    teacher_hidden = torch.randn(1, T, model.hidden, generator=g).to(dev, torch.bfloat16)
    ids = torch.randint(0, vocab, (1, T), generator=g).to(dev)
    loss_mask = torch.ones(1, T, dtype=torch.long, device=dev)
    t = lambda a, dt: torch.as_tensor(a, dtype=dt, device=dev)[None]  # noqa: E731
    anchors, keep = t(w.anchors, torch.long), t(w.keep, torch.bool)
    docs, adocs = t(w.ctx_doc_ids, torch.long), t(w.anchor_doc_ids, torch.long)
    anchors, keep = validate_injected_anchors(anchors, keep, loss_mask=loss_mask, num_anchors=nb,
                                              block_size=B, ctx_doc_ids=docs)
    starts = torch.as_tensor(np.cumsum([0] + list(w.lengths[:-1])), device=dev)
    local = torch.arange(T, device=dev) - starts[docs.clamp(min=0)][0]
    mask = vocab - 1 if mask_token is None else mask_token
    draft_ids = torch.full((nb, B), mask, dtype=torch.long, device=dev)
    draft_ids[:, 0] = ids[0, anchors[0]]
    offsets = torch.arange(B, device=dev)
    draft_pos = (local[anchors[0]][:, None] + offsets[None]).reshape(1, -1)
    meta = DirectCPMetadata(anchors, keep, t(w.context_positions, torch.long), B, 0, 1, None,
                            context_doc_ids=docs, anchor_doc_ids=adocs, sequence_length=w.sequence_length)
    targets = dspark_targets(anchors, keep, ids % draft_vocab, loss_mask, B,
                             loss_decay_gamma=decay_gamma, ctx_doc_ids=docs)
    return {"target_hidden": target_hidden, "teacher_hidden": teacher_hidden,
            "draft_input_ids": draft_ids.reshape(1, -1), "draft_positions": draft_pos.contiguous(),
            "context_positions": local[None].contiguous(), "metadata": meta, "targets": targets}


def dspark_layer_step(model, optimizer, batch, *, ce_alpha=0.1, l1_alpha=0.9):
    """One training step: forward, CE + L1 loss against the frozen head's teacher logits,
    backward, optimizer step. `batch` holds target_hidden [1, T, L*H], teacher_hidden [1, T, H],
    draft_input_ids / draft_positions [1, Nq], context_positions [1, T], metadata, and the DSpark
    targets (target_ids, teacher_index, weights as `dspark_targets` returns them).
    Returns (loss, grad_norm) as device tensors."""
    from .head_loss import selective_head_objective

    optimizer.zero_grad()
    with torch.no_grad(), _timing.region("teacher_gemm"):
        teacher = batch["teacher_hidden"].reshape(-1, model.hidden) @ model.lm_head.t()
    hidden = model(batch["target_hidden"], batch["draft_input_ids"], batch["context_positions"],
                   batch["draft_positions"], batch["metadata"])
    targets = batch["targets"]
    # (a_ce sum(w ce) + a_l1 sum(w l1)) / sum(w): the normalised weights go into the fused
    # vocabulary-GEMM + loss + dlogits pass, which returns the objective itself
    w = targets.weights.reshape(-1).float()
    w = w / w.sum().clamp(min=1e-6)
    loss, _, _ = selective_head_objective(hidden.reshape(-1, model.hidden), model.lm_head,
                                          targets.target_ids.reshape(-1), teacher,
                                          ce_weights=w * ce_alpha, l1_weights=w * l1_alpha,
                                          teacher_indices=targets.teacher_index.reshape(-1),
                                          weight_t=model.lm_head_t)
    loss.backward()
    norm = optimizer.step()
    return loss.detach(), norm
