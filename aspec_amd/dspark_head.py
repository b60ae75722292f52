"""DSpark selective-head terms on MI355X.

Drop-in for the head side of `DSparkModel._prediction_terms` (aspec/models/dspark.py:553-636) and
its modules `VanillaMarkov` / `AcceptRatePredictor` (aspec/models/draft/dspark.py:79-127).

The vocabulary projection and the Markov bias run as ONE library GEMM over the concatenated
reduction dimension:

    logits = h W^T + markov_w2 (markov_w1[prev])^T = [h | markov_w1[prev]] [W | markov_w2]^T

so the bias is never materialised as its own [rows, V] tensor and added (the reference's
`apply_block_logits` writes and reads one extra logits-sized tensor). The concatenated weight is
kept per head weight; only the rank-R Markov columns are copied in on each call. The cross-entropy
and softmax-L1 come from the fused HIP loss pass (`aspec_amd.loss.ce_l1_from_logits`), which also
returns the row argmax for the accuracy metric, so the logits are read once for CE, L1 and
accuracy. The confidence head and the acceptance statistics are small per-row tensor operations.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import _timing
from .loss import ce_l1_from_logits
from .sampling import DEFAULT_SAMPLING, compiled_l1_from_logits

__all__ = [
    "VanillaMarkov",
    "AcceptRatePredictor",
    "build_markov_head",
    "markov_head_logits",
    "acceptance_statistics",
    "dspark_prediction_terms",
]


class VanillaMarkov(nn.Module):
    """Rank-R Markov bias over the previous token (aspec/models/draft/dspark.py:79-114): the same
    parameters and methods; `head_logits` is the fused projection + bias."""

    def __init__(self, *, vocab_size: int, markov_rank: int):
        super().__init__()
        self.vocab_size = int(vocab_size)
        self.markov_rank = int(markov_rank)
        self.markov_head_type = "vanilla"
        if self.markov_rank <= 0:
            raise ValueError(f"VanillaMarkov requires markov_rank > 0, got {self.markov_rank}.")
        self.markov_w1 = nn.Embedding(self.vocab_size, self.markov_rank)
        self.markov_w2 = nn.Linear(self.markov_rank, self.vocab_size, bias=False)

    def get_prev_embeddings(self, token_ids: torch.Tensor) -> torch.Tensor:
        return self.markov_w1(token_ids.long())

    def project_bias(self, latent_states: torch.Tensor) -> torch.Tensor:
        return self.markov_w2(latent_states)

    def compute_step_bias(self, token_ids: torch.Tensor) -> torch.Tensor:
        return self.project_bias(self.get_prev_embeddings(token_ids))

    def apply_block_logits(self, base_logits: torch.Tensor, *, token_ids: torch.Tensor) -> torch.Tensor:
        if base_logits.size(2) == 0:
            return base_logits
        return base_logits + self.compute_step_bias(token_ids)

    def head_logits(self, hidden: torch.Tensor, head_weight: torch.Tensor,
                    token_ids: torch.Tensor) -> torch.Tensor:
        """`apply_block_logits(F.linear(hidden, head_weight), token_ids=token_ids)` as one GEMM."""
        return markov_head_logits(hidden, head_weight, token_ids, self.markov_w1.weight,
                                  self.markov_w2.weight)


class AcceptRatePredictor(nn.Module):
    """Confidence head (aspec/models/draft/dspark.py:117-127)."""

    def __init__(self, input_dim: int):
        super().__init__()
        self.proj = nn.Linear(int(input_dim), 1)

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        return self.proj(features).squeeze(-1)


def build_markov_head(config):
    """`build_markov_head` (aspec/models/draft/dspark.py:130-143)."""
    markov_rank = int(getattr(config, "markov_rank", 0))
    if markov_rank < 0:
        raise ValueError(f"markov_rank must be >= 0, got {markov_rank}")
    if markov_rank == 0:
        return None
    markov_head_type = str(getattr(config, "markov_head_type", "vanilla")).lower()
    if markov_head_type == "vanilla":
        return VanillaMarkov(vocab_size=config.vocab_size, markov_rank=markov_rank)
    raise NotImplementedError(
        f"markov_head_type={markov_head_type!r} is not supported yet; only 'vanilla' is implemented.")


# [W | markov_w2] per head weight (data pointer, version, shape): W is usually the frozen Target
# head, so it is copied once; the Markov columns are refreshed on every call.
_concat_cache: dict = {}


def _concat_weight(head_weight: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    key = (head_weight.data_ptr(), head_weight._version, tuple(head_weight.shape), head_weight.dtype,
           w2.shape[1])
    wcat = _concat_cache.get(key)
    if wcat is None:
        _concat_cache.clear()
        wcat = torch.empty(head_weight.shape[0], head_weight.shape[1] + w2.shape[1],
                           dtype=head_weight.dtype, device=head_weight.device)
        wcat[:, :head_weight.shape[1]].copy_(head_weight)
        _concat_cache[key] = wcat
    wcat[:, head_weight.shape[1]:].copy_(w2)
    return wcat


class _MarkovHeadLogits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden2d, prev, head_weight, w1, w2):
        hdim = hidden2d.shape[1]
        e = w1.index_select(0, prev).to(hidden2d.dtype)
        x = torch.cat((hidden2d, e), dim=1)
        wcat = _concat_weight(head_weight, w2.detach().to(head_weight.dtype))
        with _timing.region("head_gemm_fwd"):
            logits = x @ wcat.t()
        ctx.save_for_backward(x, prev, wcat)
        ctx.hdim = hdim
        ctx.shapes = (w1.shape, w1.dtype, w2.dtype, head_weight.dtype)
        return logits

    @staticmethod
    @once_differentiable
    def backward(ctx, dlogits):
        x, prev, wcat = ctx.saved_tensors
        hdim = ctx.hdim
        w1_shape, w1_dtype, w2_dtype, w_dtype = ctx.shapes
        dlogits = dlogits.to(x.dtype).contiguous()
        dh = de = dw = dw1 = dw2 = None
        need_h, _, need_w, need_w1, need_w2 = ctx.needs_input_grad
        if need_h or need_w1:
            with _timing.region("head_gemm_dgrad"):
                dx = dlogits @ wcat
            dh = dx[:, :hdim] if need_h else None
            de = dx[:, hdim:]
        if need_w or need_w2:
            dwcat = dlogits.t() @ x if need_w else None
            if need_w:
                dw = dwcat[:, :hdim].to(w_dtype)
                dw2 = dwcat[:, hdim:].to(w2_dtype) if need_w2 else None
            else:
                dw2 = (dlogits.t() @ x[:, hdim:]).to(w2_dtype)
        if need_w1:
            dw1 = torch.zeros(w1_shape, dtype=torch.float32, device=x.device)
            dw1.index_add_(0, prev, de.float())
            dw1 = dw1.to(w1_dtype)
        return dh, None, dw, dw1, dw2


def markov_head_logits(hidden: torch.Tensor, head_weight: torch.Tensor, prev_ids: torch.Tensor,
                       markov_w1: torch.Tensor, markov_w2: torch.Tensor) -> torch.Tensor:
    """hidden @ head_weight^T + markov_w2(markov_w1[prev_ids]) as one GEMM (autograd to hidden,
    head_weight, markov_w1 and markov_w2): the logits of dspark.py:560-566."""
    if hidden.shape[:-1] != prev_ids.shape:
        raise ValueError("prev_ids must index every hidden row")
    if head_weight.shape[0] != markov_w2.shape[0] or markov_w1.shape[1] != markov_w2.shape[1]:
        raise ValueError("Markov factors do not match the head: w1 [V', R], w2 [V, R], head [V, H]")
    rows = hidden.reshape(-1, hidden.shape[-1])
    prev = prev_ids.reshape(-1).long()
    logits = _MarkovHeadLogits.apply(rows, prev, head_weight, markov_w1, markov_w2)
    return logits.view(*hidden.shape[:-1], head_weight.shape[0])


def acceptance_statistics(accept_rate: torch.Tensor, eval_mask: torch.Tensor) -> torch.Tensor:
    """[[sum alpha per position..., sum tau], [mask count per position..., valid blocks]]
    (aspec/models/ops/acceptance.py:15-30)."""
    if accept_rate.ndim != 3 or accept_rate.shape != eval_mask.shape:
        raise ValueError("Acceptance and supervision must have matching [batch, blocks, positions] shapes")
    mask = eval_mask.detach().float()
    alpha = accept_rate.detach().float() * mask
    valid_blocks = mask.bool().any(dim=-1)
    tau = 1.0 + alpha.cumprod(dim=-1).sum(dim=-1)
    numerators = torch.cat((alpha.sum(dim=(0, 1)), (tau * valid_blocks).sum().reshape(1)))
    denominators = torch.cat((mask.sum(dim=(0, 1)), valid_blocks.sum().float().reshape(1)))
    return torch.stack((numerators, denominators))


def dspark_prediction_terms(hidden, target_ids, prev_ids, head_weight, aligned_target_hidden,
                            eval_mask, weights, *, markov_head=None, confidence_head=None,
                            confidence_head_with_markov=True, l1_loss_alpha=1.0,
                            confidence_head_alpha=0.0, prediction_start=0, block_size=None,
                            cached_target_logits=None, cached_draft_logits=None,
                            cached_target_positions=None, loss_cache=None, l1_sampling=None):
    """Additive DSpark head terms for one block slice (aspec/models/dspark.py:553-636):
    (ce_num, l1_num, conf_num, position_loss, position_correct, acceptance_totals).

    hidden [B, N, K, H], target_ids / prev_ids [B, N, K], eval_mask / weights [B, N, K]. The
    teacher logits are, as in the reference's unsampled L1 path:
      - with `cached_target_positions` [B, N, K]: rows of the teacher table `cached_target_logits`
        [B, context, V] at those context positions, read through int64 row indices by the loss
        kernel itself (the indexed teacher of dspark.py:576-585; never gathered into a copy);
      - else `cached_target_logits` (the logits' shape) or aligned_target_hidden projected by
        head_weight (no Markov bias).
    `loss_cache` is the head chunk's checkpoint-replay dict (dspark.py:473, 602): filled by the
    first forward, replayed without a loss forward kernel on the checkpoint recompute.
    `l1_sampling` = (target_sampling, draft_sampling), each (temperature, top_p, top_k), filters
    both distributions before the L1 (`DSparkModel(l1_target_sampling=..., l1_draft_sampling=...)`,
    dspark.py:111-112, 606-609): CE and the argmax still come from the raw logits, the L1 from
    `aspec_amd.sampling.compiled_l1_from_logits`; as in the reference, `loss_cache` then serves
    neither term.
    """
    if cached_draft_logits is not None:
        logits = cached_draft_logits
        if markov_head is not None:
            logits = markov_head.apply_block_logits(logits, token_ids=prev_ids)
    elif markov_head is not None:
        logits = markov_head.head_logits(hidden, head_weight, prev_ids)
    else:
        logits = F.linear(hidden.reshape(-1, hidden.shape[-1]), head_weight).view(
            *hidden.shape[:-1], head_weight.shape[0])
    vocab = logits.shape[-1]
    teacher = teacher_index = None
    if aligned_target_hidden is not None:
        if cached_target_positions is not None:
            if cached_target_logits is None or cached_target_logits.ndim != 3:
                raise ValueError("cached_target_positions index a [batch, context, vocab] teacher table")
            batch, context, _ = cached_target_logits.shape
            positions = cached_target_positions.flatten(1).long()
            if batch > 1:
                positions = positions + torch.arange(batch, device=positions.device)[:, None] * context
            teacher_index = positions.reshape(-1).contiguous()
            teacher = cached_target_logits.detach().reshape(-1, vocab).contiguous()
        else:
            teacher = cached_target_logits if cached_target_logits is not None else F.linear(
                aligned_target_hidden.reshape(-1, aligned_target_hidden.shape[-1]), head_weight
            ).view_as(logits)
            teacher = teacher.detach().contiguous().reshape(-1, vocab)
    flat = logits.reshape(-1, vocab).contiguous()
    sampled = l1_sampling is not None and tuple(map(tuple, l1_sampling)) != (DEFAULT_SAMPLING,
                                                                              DEFAULT_SAMPLING)
    if sampled and teacher is not None:
        ce, _, argmax = ce_l1_from_logits(flat, target_ids.reshape(-1).long().contiguous(), None,
                                          return_argmax=True)
        l1 = compiled_l1_from_logits(flat, teacher, l1_sampling[0], l1_sampling[1],
                                     teacher_indices=teacher_index)
    else:
        ce, l1, argmax = ce_l1_from_logits(
            flat, target_ids.reshape(-1).long().contiguous(), teacher, teacher_indices=teacher_index,
            return_argmax=True, _replay_cache=loss_cache)
    ce = ce.view_as(weights)
    ce_num = (ce * weights).sum()
    l1_num = logits.new_zeros((), dtype=torch.float32)
    accept_rate = None
    if teacher is not None:
        l1 = l1.view_as(weights)
        if l1_loss_alpha > 0:
            l1_num = (l1 * weights).sum()
        accept_rate = (1.0 - 0.5 * l1).clamp(0.0, 1.0)
    conf_num = logits.new_zeros((), dtype=torch.float32)
    if confidence_head is not None and confidence_head_alpha > 0:
        if accept_rate is None:
            raise ValueError("the confidence head needs teacher logits (aligned_target_hidden)")
        if confidence_head_with_markov:
            prev_emb = markov_head.get_prev_embeddings(prev_ids).to(hidden.dtype)
            conf_features = torch.cat([hidden, prev_emb], dim=-1)
        else:
            conf_features = hidden
        prediction = confidence_head(conf_features).float()
        conf_num = (F.binary_cross_entropy_with_logits(
            prediction, accept_rate.detach(), reduction="none") * weights).sum()
    with torch.no_grad():
        correct = (argmax.view_as(target_ids) == target_ids) & (eval_mask > 0.5)
        position_loss = (ce * eval_mask).sum((0, 1))
        position_correct = correct.float().sum((0, 1))
        if accept_rate is not None:
            acceptance_totals = F.pad(acceptance_statistics(
                accept_rate[..., prediction_start:], eval_mask[..., prediction_start:]),
                (prediction_start, 0))
        else:
            size = block_size if block_size is not None else target_ids.shape[-1]
            acceptance_totals = logits.new_zeros((2, size + 1), dtype=torch.float32)
    return ce_num, l1_num, conf_num, position_loss, position_correct, acceptance_totals
