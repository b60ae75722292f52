"""DSpark head terms on the GPU: the loss pass's fused argmax (bit-exact against torch.argmax and
the oracle, with ties, NaN and infinite rows, on the persistent and streaming kernels), the
Markov-fused head GEMM and its gradients, and the composed prediction terms, against the fp64
oracle (bf16 tolerances stated per test)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from aspec_amd import _lib
from aspec_amd.dspark_head import (AcceptRatePredictor, VanillaMarkov, acceptance_statistics,
                                   dspark_prediction_terms, markov_head_logits)
from aspec_amd.loss import ce_l1_from_logits
from oracle import dspark_head as odh
from oracle import loss as oloss

pytestmark = pytest.mark.gpu


def _planted_rows(gpu, rows, vocab, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = (torch.randn(rows, vocab, device=gpu, generator=g) * 3).to(torch.bfloat16)
    # ties of the row maximum far apart (several threads / chunks hold it)
    top = x.float().amax(-1)
    x[0, vocab - 1] = top[0].to(torch.bfloat16)
    x[0, vocab // 2] = top[0].to(torch.bfloat16)
    x[1, :] = 1.0  # a constant row: index 0
    x[2, 5] = float("nan")
    x[2, 3] = float("nan")
    x[3, vocab - 3] = float("inf")
    x[3, 17] = float("inf")
    x[4, :] = float("-inf")
    x[5, : vocab // 2] = float("-inf")
    # tiny maxima, where exp2 cannot tell the maximum from its neighbours
    x[6, :] = 0.0
    x[6, vocab - 5] = 1e-7
    x[7, :] = -1e-30
    x[7, 100] = 0.0
    return x


@pytest.mark.parametrize("vocab", [1000, 12000, 32000, 40000, 32001])
def test_fused_argmax_is_bit_exact(gpu, vocab):
    rows = 9
    x = _planted_rows(gpu, rows, vocab, 11 + vocab)
    t = torch.randint(0, vocab, (rows,), device=gpu)
    y = torch.randn_like(x.float()).to(torch.bfloat16)
    ce_a, l1_a, amax = ce_l1_from_logits(x, t, y, return_argmax=True)
    ce_b, l1_b = ce_l1_from_logits(x, t, y)
    torch.cuda.synchronize()
    print(f"argmax V={vocab}: {amax.tolist()}")
    assert torch.equal(amax, torch.argmax(x, dim=-1))
    np.testing.assert_array_equal(amax.cpu().numpy(), odh.argmax(x.float().cpu().numpy()))
    # the argmax leaves the loss outputs untouched
    assert torch.equal(torch.nan_to_num(ce_a, nan=7.0), torch.nan_to_num(ce_b, nan=7.0))
    assert torch.equal(torch.nan_to_num(l1_a, nan=7.0), torch.nan_to_num(l1_b, nan=7.0))


def test_fused_argmax_random_rows_large(gpu):
    g = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(2048, 32000, device=gpu, generator=g).to(torch.bfloat16)
    t = torch.randint(0, 32000, (2048,), device=gpu, generator=g)
    _, _, amax = ce_l1_from_logits(x, t, return_argmax=True)
    assert torch.equal(amax, torch.argmax(x, dim=-1))


def _head_case(gpu, rows=48, hidden=256, vocab=1024, rank=32, seed=0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    h = (torch.randn(rows, hidden, device=gpu, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    w1 = (torch.randn(vocab, rank, device=gpu, generator=g) * 0.5).to(torch.bfloat16)
    w2 = (torch.randn(vocab, rank, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    prev = torch.randint(0, vocab, (rows,), device=gpu, generator=g)
    prev[1] = prev[0]  # a repeated previous token: its embedding gradient accumulates
    return h, w, w1, w2, prev


def test_markov_head_logits_and_gradients(gpu):
    h, w, w1, w2, prev = _head_case(gpu)
    hr, w1r, w2r = (a.clone().requires_grad_() for a in (h, w1, w2))
    logits = markov_head_logits(hr, w, prev, w1r, w2r)
    g = torch.randn(logits.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(9))
    logits.backward(g.to(logits.dtype))
    np_ = lambda a: a.double().cpu().numpy()
    ref = odh.markov_logits(np_(h), np_(w), prev.cpu().numpy(), np_(w1), np_(w2))
    dh, dw1, dw2 = odh.markov_logits_grad(np_(h), np_(w), prev.cpu().numpy(), np_(w1), np_(w2),
                                          np_(g.to(torch.bfloat16)))
    for name, got, want in (("logits", logits, ref), ("dh", hr.grad, dh), ("dw1", w1r.grad, dw1),
                            ("dw2", w2r.grad, dw2)):
        got = np_(got.detach())
        err = np.abs(got - want).max()
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        print(f"markov {name}: max_abs={err:.3e} rel_l2={rel:.3e}")
        # bf16 inputs, fp32 accumulation, one bf16 rounding of the output
        assert rel < 1e-2
        np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2 * np.abs(want).max())


def test_vanilla_markov_fused_equals_bias_added(gpu):
    torch.manual_seed(0)
    head = VanillaMarkov(vocab_size=512, markov_rank=16).to(gpu, torch.bfloat16)
    h = torch.randn(2, 3, 4, 128, device=gpu, dtype=torch.bfloat16)
    w = torch.randn(512, 128, device=gpu, dtype=torch.bfloat16) * 0.05
    prev = torch.randint(0, 512, (2, 3, 4), device=gpu)
    fused = head.head_logits(h, w, prev)
    added = head.apply_block_logits(F.linear(h, w), token_ids=prev)
    torch.testing.assert_close(fused.float(), added.float(), rtol=2e-2, atol=2e-2)


def test_acceptance_statistics_matches_oracle(gpu):
    g = torch.Generator(device=gpu).manual_seed(3)
    accept = torch.rand(2, 5, 7, device=gpu, generator=g)
    mask = (torch.rand(2, 5, 7, device=gpu, generator=g) > 0.3).float()
    mask[1, 2] = 0
    got = acceptance_statistics(accept, mask).double().cpu().numpy()
    want = odh.acceptance_statistics(accept.double().cpu().numpy(), mask.double().cpu().numpy())
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_prediction_terms_match_oracle(gpu):
    B, N, K, H, V, R = 1, 6, 16, 256, 1024, 32
    gen = torch.Generator(device=gpu).manual_seed(21)
    rnd = lambda *s, scale=1.0: (torch.randn(*s, device=gpu, generator=gen) * scale).to(torch.bfloat16)
    h, th = rnd(B, N, K, H, scale=0.5), rnd(B, N, K, H, scale=0.5)
    w = rnd(V, H, scale=0.05)
    markov = VanillaMarkov(vocab_size=V, markov_rank=R).to(gpu, torch.bfloat16)
    conf = AcceptRatePredictor(H + R).to(gpu, torch.bfloat16)
    tgt = torch.randint(0, V, (B, N, K), device=gpu, generator=gen)
    prev = torch.randint(0, V, (B, N, K), device=gpu, generator=gen)
    mask = torch.ones(B, N, K, device=gpu)
    mask[0, 2, 10:] = 0
    weights = mask * torch.exp(-torch.arange(K, device=gpu) / 4.0)
    # half the positions predict their row's arg-max token, so the accuracy count is exercised
    ref_logits = odh.markov_logits(h.double().cpu().numpy().reshape(-1, H), w.double().cpu().numpy(),
                                   prev.cpu().numpy().reshape(-1),
                                   markov.markov_w1.weight.detach().double().cpu().numpy(),
                                   markov.markov_w2.weight.detach().double().cpu().numpy())
    top = torch.as_tensor(odh.argmax(ref_logits).reshape(B, N, K), device=gpu)
    tgt[..., : K // 2] = top[..., : K // 2]
    out = dspark_prediction_terms(h, tgt, prev, w, th, mask, weights, markov_head=markov,
                                  confidence_head=conf, confidence_head_alpha=1.0, prediction_start=1)
    np_ = lambda a: a.detach().double().cpu().numpy()
    ref = odh.prediction_terms(np_(h), np_(tgt).astype(np.int64), np_(prev).astype(np.int64), np_(w),
                               np_(th), np_(mask), np_(weights), w1=np_(markov.markov_w1.weight),
                               w2=np_(markov.markov_w2.weight), conf_w=np_(conf.proj.weight)[0],
                               conf_b=float(conf.proj.bias.item()), conf_alpha=1.0, prediction_start=1)
    names = ["ce_num", "l1_num", "conf_num", "position_loss", "position_correct", "acceptance"]
    for name, got, want in zip(names, out, ref):
        got = np.asarray(np_(got), np.float64)
        print(f"{name}: got={np.ravel(got)[:4]} want={np.ravel(want)[:4]}")
        # bf16 logits: CE / L1 sums within 1%, the accuracy count within one flipped argmax
        if name == "position_correct":
            assert want[: K // 2].sum() > 0
            assert np.abs(got - want).sum() <= 2
        else:
            np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)


def test_prediction_terms_indexed_teacher_and_checkpoint_replay(gpu):
    """The production path of _prediction_terms (aspec/models/dspark.py:573-605): teacher rows
    read from the cached [batch, context, V] teacher table through cached_target_positions (batch 2,
    so the per-row offsets b * context apply), against (a) the same terms with the rows gathered
    into a copy (bitwise equal: the loss reads the same values) and (b) the fp64 oracle; then a
    checkpoint replay through loss_cache reuses the first forward's statistics (no loss forward
    kernel runs) and gives bitwise the same terms and gradient."""
    from aspec_amd import _timing

    B, N, K, H, V, C = 2, 5, 16, 128, 1024, 48
    gen = torch.Generator(device=gpu).manual_seed(31)
    rnd = lambda *s, scale=1.0: (torch.randn(*s, device=gpu, generator=gen) * scale).to(torch.bfloat16)  # noqa: E731
    h = rnd(B, N, K, H, scale=0.5)
    w = rnd(V, H, scale=0.05)
    table = rnd(B, C, V, scale=2.0)
    positions = torch.randint(0, C, (B, N, K), device=gpu, generator=gen)
    tgt = torch.randint(0, V, (B, N, K), device=gpu, generator=gen)
    prev = torch.randint(0, V, (B, N, K), device=gpu, generator=gen)
    mask = (torch.rand(B, N, K, device=gpu, generator=gen) > 0.2).float()
    weights = mask * torch.exp(-torch.arange(K, device=gpu) / 4.0)
    gathered = table.gather(1, positions.flatten(1).unsqueeze(-1).expand(-1, -1, V)).view(B, N, K, V)
    aligned = torch.zeros(B, N, K, H, device=gpu, dtype=torch.bfloat16)  # presence switches L1 on

    def run(**teacher):
        hh = h.clone().requires_grad_()
        terms = dspark_prediction_terms(hh, tgt, prev, w, aligned, mask, weights, prediction_start=1,
                                        **teacher)
        (terms[0] * 0.1 + terms[1] * 0.9).backward()
        return [t.detach().clone() for t in terms], hh.grad

    indexed, g_indexed = run(cached_target_logits=table, cached_target_positions=positions)
    copied, g_copied = run(cached_target_logits=gathered)
    for a, b in zip(indexed, copied):
        assert torch.equal(a, b)
    assert torch.equal(g_indexed, g_copied)
    np_ = lambda a: a.detach().double().cpu().numpy()  # noqa: E731
    ref = odh.prediction_terms(np_(h), np_(tgt).astype(np.int64), np_(prev).astype(np.int64), np_(w), None,
                               np_(mask), np_(weights), teacher_logits=np_(gathered).reshape(-1, V),
                               prediction_start=1)
    for name, got, want in zip(["ce_num", "l1_num", "conf_num", "position_loss", "position_correct",
                                "acceptance"], indexed, ref):
        got = np.asarray(np_(got), np.float64)
        if name == "position_correct":
            assert np.abs(got - want).sum() <= 2
        else:
            np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)
    cache = {}
    _timing.reset()
    _timing.enable(True)
    try:
        first, g_first = run(cached_target_logits=table, cached_target_positions=positions, loss_cache=cache)
        assert "statistics" in cache and _timing.summary()["loss_fwd"]["launches"] == 1
        replay, g_replay = run(cached_target_logits=table, cached_target_positions=positions, loss_cache=cache)
        assert _timing.summary()["loss_fwd"]["launches"] == 1  # the replay ran no forward kernel
    finally:
        _timing.enable(False)
        _timing.reset()
    for a, b, c in zip(first, replay, indexed):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert torch.equal(g_first, g_replay) and torch.equal(g_first, g_indexed)
    with pytest.raises(ValueError, match="different head chunk"):
        dspark_prediction_terms(h[:, :2], tgt[:, :2], prev[:, :2], w, aligned[:, :2], mask[:, :2],
                                weights[:, :2], cached_target_logits=table,
                                cached_target_positions=positions[:, :2], loss_cache=cache)
