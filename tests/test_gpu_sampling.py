"""Sampled L1 and sampling_logits on the GPU (csrc/sampling.hip) against the fp64 oracle
(oracle/sampling.py) on the same bf16 inputs.

* `sampling_logits`: the filtered fp32 values equal the oracle's bit for bit (kept values and the
  -inf positions), on the reference test's sampling cases, rows with heavy ties (bf16 values on a
  coarse grid), -inf tokens, a register-resident row of each size class and a row read from
  global memory (V = 151936). A row whose top-p boundary lies within 1e-7 (relative) of a token's
  preceding mass may differ in that one token: the exp values carry fp32 rounding (the reference's
  own fp32 cumulative sum carries more). Tie groups cut by top-p or top-k are exact (closed form);
  the gradient within bf16;
* `compiled_l1_from_logits`: L1 and the draft gradient within the reference's CUDA bars
  (tests/test_dspark_l1_sampling.py:254-269: atol 2e-6 / rtol 2e-5, gradient atol 2e-5 /
  rtol 0.02), on the reference's sampling pairs, gathered and indexed teachers;
* identical rows with one sampling: zero L1 and gradient exactly; the default sampling is the
  tiled-L1 kernel; invalid samplings and teacher indices raise; NaN rows propagate.
"""

import numpy as np
import pytest
import torch

from aspec_amd.sampling import compiled_l1_from_logits, sampling_logits
from aspec_amd.tiled_l1 import tiled_l1_from_logits
from oracle import sampling as S

pytestmark = pytest.mark.gpu

DEFAULT = (1.0, 1.0, -1)
TARGET = (0.8, 0.85, 5)
DRAFT = (1.2, 0.9, 7)
CASES = [(0.4, 1.0, -1), (1.0, 1.0, 1), (1.0, 1.0, 100), (1.0, 0.5, 10**30), (1.0, 0.5, -1), TARGET, DRAFT,
         (0.7, 0.3, -1), (1.0, 0.999, 2000)]
PAIRS = [(TARGET, DEFAULT), (DEFAULT, DRAFT), (TARGET, DRAFT), ((0.8, 0.7, -1), DEFAULT),
         (DEFAULT, (1.2, 0.8, -1)), ((0.8, 0.7, -1), (1.2, 0.8, -1))]
VOCABS = [17, 4097, 8192, 32000, 98304, 151936]


def _rows(gpu, rows, vocab, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = (torch.randn(rows, vocab, device=gpu, generator=g) * 2.0)
    x[1] = torch.randint(-8, 8, (vocab,), device=gpu, generator=g).float() / 4  # heavy ties
    x[2, ::3] = -torch.inf
    x[3] = 0.0  # one tie group
    return x.to(torch.bfloat16)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("vocab", VOCABS)
def test_sampling_logits_bitwise(gpu, vocab):
    x = _rows(gpu, 6, vocab, vocab)
    xn = _np(x)
    for sampling in CASES:
        got = sampling_logits(x, sampling).cpu()
        want = torch.from_numpy(S.sampling_logits(xn, sampling).astype(np.float32))
        margin = S.top_p_margin(xn, sampling)
        mism = (got != want).sum(-1)
        print(f"V={vocab} sampling={sampling}: kept {int(torch.isfinite(want).sum())} "
              f"mismatches {mism.tolist()} min margin {margin.min():.1e}")
        for r in range(x.shape[0]):
            if margin[r] >= 1e-7:
                assert torch.equal(got[r], want[r]), (vocab, sampling, r)
            else:  # at most the boundary token toggles
                diff = got[r] != want[r]
                n = int(diff.sum())
                assert n == 0 or (n == 1 and torch.isinf(torch.cat([got[r][diff], want[r][diff]])).any())


@pytest.mark.parametrize("vocab", [17, 4096, 32000, 151936])
def test_tie_groups_exact(gpu, vocab):
    """All-equal rows: top-p keeps floor(float32(top_p) * V) + 1 tokens, top-k keeps top_k, the
    lowest indices first (the reference's stable order)."""
    x = torch.zeros(3, vocab, device=gpu, dtype=torch.bfloat16)
    x[1] = 1.5
    x[2] = -3.0
    for sampling in ((1.0, 0.5, -1), (1.0, 0.3, -1), (0.7, 0.25, -1), (1.0, 1.0, 7), (0.5, 0.5, 5),
                     (1.0, 0.999, -1)):
        temperature, top_p, top_k = sampling
        n = vocab
        if top_p < 1.0:
            n = min(n, int(np.floor(float(np.float32(top_p)) * vocab)) + 1)
        if 0 < top_k < vocab:
            n = min(n, top_k)
        out = sampling_logits(x, sampling)
        kept = torch.isfinite(out)
        assert torch.equal(kept.sum(-1).cpu(), torch.full((3,), n)), sampling
        assert kept[:, :n].all() and not kept[:, n:].any()


@pytest.mark.parametrize("vocab", [4097, 32000, 151936])
def test_sampling_logits_gradient(gpu, vocab):
    x = _rows(gpu, 5, vocab, 3).requires_grad_()
    g = torch.Generator(device=gpu).manual_seed(4)
    for sampling in ((1.0, 0.8, 50), (0.6, 0.9, -1), (0.5, 1.0, -1)):
        w = torch.randn(5, vocab, device=gpu, generator=g)
        out = sampling_logits(x, sampling)
        (grad,) = torch.autograd.grad((torch.where(torch.isfinite(out), out, 0.0) * w).sum(), x)
        # the upstream gradient the kernel receives: zero where the output is -inf
        g_up = torch.where(torch.isfinite(out), w, 0.0).detach().cpu().double().numpy()
        want = torch.from_numpy(S.sampling_logits_grad(_np(x.detach()), g_up, sampling))
        torch.testing.assert_close(grad.cpu().double(), want, atol=1e-6, rtol=1e-2)


@pytest.mark.parametrize("vocab", [8192, 32000, 151936])
@pytest.mark.parametrize("target,draft", PAIRS)
def test_sampled_l1_matches_oracle(gpu, vocab, target, draft):
    x = _rows(gpu, 8, vocab, 19).requires_grad_()
    y = _rows(gpu, 8, vocab, 20)
    g = torch.Generator(device=gpu).manual_seed(5)
    w = torch.rand(8, device=gpu, generator=g)
    l1 = compiled_l1_from_logits(x, y, target, draft)
    (grad,) = torch.autograd.grad((l1 * w).sum(), x)
    xn, yn = _np(x.detach()), _np(y)
    ref = S.sampled_l1(xn, yn, target, draft)
    ref_g = S.sampled_l1_grad(xn, yn, w.cpu().double().numpy(), target, draft)
    # rows whose top-p boundary sits within the exp values' rounding are not comparable
    ok = np.minimum(S.top_p_margin(xn, draft), S.top_p_margin(yn, target)) >= 1e-7
    assert ok.sum() >= 5
    got, got_g = l1.detach().cpu().double().numpy()[ok], grad.cpu().double().numpy()[ok]
    err = np.abs(got - ref[ok]).max()
    rel = float(np.linalg.norm(got_g - ref_g[ok]) / max(np.linalg.norm(ref_g[ok]), 1e-30))
    # (a zero exact gradient, every kept draft token above the teacher, shows rel_l2 1: the
    # oracle's fp64 rounding against the kernel's exact zero)
    print(f"V={vocab} target={target} draft={draft}: {ok.sum()} rows, l1 max_abs {err:.2e}, "
          f"grad max_abs {np.abs(got_g - ref_g[ok]).max():.2e} rel_l2 {rel:.2e}")
    torch.testing.assert_close(torch.from_numpy(got), torch.from_numpy(ref[ok]), atol=2e-6, rtol=2e-5)
    torch.testing.assert_close(torch.from_numpy(got_g), torch.from_numpy(ref_g[ok]), atol=2e-5, rtol=0.02)


def test_identical_rows_and_default(gpu):
    x = _rows(gpu, 6, 32000, 8).requires_grad_()
    for sampling in (DRAFT, TARGET, (0.5, 1.0, -1)):
        l1 = compiled_l1_from_logits(x, x.detach(), sampling, sampling)
        (grad,) = torch.autograd.grad(l1.sum(), x)
        assert torch.count_nonzero(l1) == 0 and torch.count_nonzero(grad) == 0
    y = _rows(gpu, 6, 32000, 9)
    assert torch.equal(compiled_l1_from_logits(x.detach(), y), tiled_l1_from_logits(x.detach(), y))


def test_indexed_teacher_and_fail_closed(gpu):
    x = _rows(gpu, 8, 4097, 12)
    table = _rows(gpu, 5, 4097, 13)
    idx = torch.tensor([0, 4, 2, 2, 1, 3, 0, 4], device=gpu)
    a = compiled_l1_from_logits(x, table, TARGET, DRAFT, teacher_indices=idx)
    b = compiled_l1_from_logits(x, table[idx], TARGET, DRAFT)
    assert torch.equal(a, b)
    bad = idx.clone()
    bad[5] = 5
    with pytest.raises(ValueError, match="teacher index out of range"):
        compiled_l1_from_logits(x, table, TARGET, DRAFT, teacher_indices=bad)
    for sampling in ((0.0, 1.0, -1), (float("nan"), 1.0, -1), (1.0, 0.0, -1), (1.0, 1.1, -1), (1.0, 1.0, 0),
                     (1.0, 1.0, -2)):
        with pytest.raises(ValueError):
            compiled_l1_from_logits(x, table[idx], sampling, DEFAULT)
    nan_rows = x.clone()
    nan_rows[3, 7] = torch.nan
    out = compiled_l1_from_logits(nan_rows, table[idx], TARGET, DRAFT)
    assert torch.isnan(out[3]) and torch.isfinite(out[torch.arange(8, device=gpu) != 3]).all()


def test_prediction_terms_with_l1_sampling(gpu):
    """dspark_prediction_terms(l1_sampling=(target, draft)) (dspark.py:606-609): the L1 numerator
    from the filtered distributions (oracle), CE unchanged, the cached-teacher path equal."""
    from aspec_amd.dspark_head import dspark_prediction_terms

    g = torch.Generator(device=gpu).manual_seed(21)
    B, N, K, H, V = 1, 4, 3, 64, 4096
    hidden = (torch.randn(B, N, K, H, device=gpu, generator=g)).to(torch.bfloat16)
    head = (torch.randn(V, H, device=gpu, generator=g) * 0.3).to(torch.bfloat16)
    aligned = (torch.randn(B, N, K, H, device=gpu, generator=g)).to(torch.bfloat16)
    ids = torch.randint(0, V, (B, N, K), device=gpu, generator=g)
    weights = torch.rand(B, N, K, device=gpu, generator=g)
    eval_mask = weights > 0.2
    kwargs = dict(l1_loss_alpha=1.0, block_size=K)
    plain = dspark_prediction_terms(hidden, ids, ids, head, aligned, eval_mask, weights, **kwargs)
    h = hidden.clone().requires_grad_()
    terms = dspark_prediction_terms(h, ids, ids, head, aligned, eval_mask, weights,
                                    l1_sampling=(TARGET, DRAFT), **kwargs)
    assert torch.equal(terms[0], plain[0]) and torch.equal(terms[4], plain[4])
    logits = torch.matmul(hidden.reshape(-1, H), head.t())
    teacher = torch.matmul(aligned.reshape(-1, H), head.t())
    ref = S.sampled_l1(_np(logits), _np(teacher), TARGET, DRAFT)
    want = float((torch.from_numpy(ref) * weights.reshape(-1).cpu().double()).sum())
    torch.testing.assert_close(terms[1].double().cpu(), torch.tensor(want, dtype=torch.float64),
                               atol=2e-6, rtol=2e-5)
    (dh,) = torch.autograd.grad(terms[1], h)
    assert torch.isfinite(dh).all()
    # the cached teacher table at explicit positions gives the same terms
    table = teacher.reshape(B, N * K, V)
    positions = torch.arange(N * K, device=gpu).reshape(B, N, K)
    cached = dspark_prediction_terms(hidden, ids, ids, head, aligned, eval_mask, weights,
                                     cached_target_logits=table, cached_target_positions=positions,
                                     l1_sampling=(TARGET, DRAFT), **kwargs)
    assert torch.equal(cached[1], terms[1])
