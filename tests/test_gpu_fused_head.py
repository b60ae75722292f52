"""The fused loss pass (CE + L1 + the objective's dlogits in one pass over the logits) and the
selective-head objective operator built on it.

* `ce_l1_fused_grad` against the two-kernel path (`ce_l1_from_logits` forward and its backward with
  the same per-row gradients): CE, L1 and the argmax bitwise equal (the same forward arithmetic),
  dlogits within one bf16 rounding (rel-L2 < 1e-3, atol 1e-6 / rtol 0.02), on the persistent
  walk's three chunk counts, gathered and indexed teachers, ignored targets and zero weights;
* against the fp64 oracle (oracle/loss.py) with the reference's gradient bar (rel-L2 < 0.01,
  tests/test_tiled_l1.py:26-148);
* identical draft and teacher rows: the L1 part of dlogits is exactly zero (the CE-only result);
* in place equals out of place bitwise; out-of-range indices raise; uncovered vocabularies raise
  NotImplementedError;
* the device-scalar scale of dh (`aspec_scale_bf16_by_device_scalar`) equals torch's fp32 product
  rounded once, on aligned, unaligned and tail elements, and leaves the buffer untouched for 1;
* `selective_head_objective` (GEMM + fused pass, dh = g dlogits W) against the unfused composition
  of the same library GEMM, `ce_l1_from_logits` and autograd (CE, L1 bitwise, the objective), and
  both against dh in fp64, also on the fallback vocabulary.
"""

import numpy as np
import pytest
import torch

from aspec_amd.head_loss import selective_head_objective
from aspec_amd.loss import ce_l1_from_logits, ce_l1_fused_grad
from oracle import loss as L

pytestmark = pytest.mark.gpu


def _case(gpu, rows, vocab, *, indexed, seed, scale=2.0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = (torch.randn(rows, vocab, device=gpu, generator=g) * scale).to(torch.bfloat16)
    trows = max(1, rows // 2) if indexed else rows
    y = (torch.randn(trows, vocab, device=gpu, generator=g) * scale).to(torch.bfloat16)
    idx = torch.randint(0, trows, (rows,), device=gpu, generator=g) if indexed else None
    t = torch.randint(0, vocab, (rows,), device=gpu, generator=g)
    t[::5] = -100  # ignored rows
    w_ce = torch.rand(rows, device=gpu, generator=g)
    w_l1 = torch.rand(rows, device=gpu, generator=g)
    w_ce[3::7] = 0.0
    w_l1[4::9] = 0.0
    return x, y, idx, t, w_ce, w_l1


def _two_kernel(x, y, idx, t, w_ce, w_l1):
    xi = x.clone().requires_grad_()
    ce, l1, amax = ce_l1_from_logits(xi, t, y, teacher_indices=idx, return_argmax=True)
    (torch.dot(ce, w_ce) + torch.dot(l1, w_l1)).backward()
    return ce.detach(), l1.detach(), xi.grad, amax


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp(min=1e-30)).item()


@pytest.mark.parametrize("vocab", [1000, 12000, 32000])
@pytest.mark.parametrize("indexed", [False, True])
def test_fused_pass_equals_two_kernel_path(gpu, vocab, indexed):
    x, y, idx, t, w_ce, w_l1 = _case(gpu, 300, vocab, indexed=indexed, seed=vocab + indexed)
    ce_f, l1_f, dx_f, amax_f = ce_l1_fused_grad(x, t, y, ce_weights=w_ce, l1_weights=w_l1,
                                                teacher_indices=idx, return_argmax=True)
    ce_u, l1_u, dx_u, amax_u = _two_kernel(x, y, idx, t, w_ce, w_l1)
    assert torch.equal(ce_f, ce_u) and torch.equal(l1_f, l1_u) and torch.equal(amax_f, amax_u)
    rel = _rel(dx_f, dx_u)
    print(f"fused V={vocab} indexed={indexed}: dlogits rel_l2 vs two-kernel = {rel:.2e}")
    assert rel < 1e-3
    torch.testing.assert_close(dx_f, dx_u, atol=1e-6, rtol=0.02)


@pytest.mark.parametrize("vocab", [4104, 32000])
def test_fused_pass_matches_fp64_oracle(gpu, vocab):
    x, y, idx, t, w_ce, w_l1 = _case(gpu, 6, vocab, indexed=False, seed=31)
    t[0] = 3  # no ignored row among the few rows checked here
    ce, l1, dx = ce_l1_fused_grad(x, t, y, ce_weights=w_ce, l1_weights=w_l1)
    xd, yd = x.double().cpu().numpy(), y.double().cpu().numpy()
    td, gce, gl1 = t.cpu().numpy(), w_ce.double().cpu().numpy(), w_l1.double().cpu().numpy()
    np.testing.assert_allclose(l1.double().cpu().numpy(), L.l1(xd, yd), atol=2e-6, rtol=2e-6)
    np.testing.assert_allclose(ce.double().cpu().numpy(), L.cross_entropy(xd, td), atol=2e-5, rtol=2e-6)
    ref = L.l1_grad(xd, yd, gl1) + L.cross_entropy_grad(xd, td, gce)
    ref = torch.as_tensor(ref)
    rel = _rel(dx.cpu(), ref)
    print(f"fused V={vocab}: dlogits rel_l2 vs fp64 = {rel:.2e}")
    assert rel < 0.01
    torch.testing.assert_close(dx.cpu(), ref.to(torch.bfloat16), atol=1e-7, rtol=0.02)


def test_identical_rows_have_no_l1_gradient(gpu):
    for vocab in (4104, 32000):
        x = torch.randn(7, vocab, device=gpu, dtype=torch.bfloat16)
        t = torch.randint(0, vocab, (7,), device=gpu)
        w_ce = torch.rand(7, device=gpu)
        w_l1 = torch.rand(7, device=gpu)
        ce, l1, dx = ce_l1_fused_grad(x, t, x, ce_weights=w_ce, l1_weights=w_l1)
        _, _, dx_ce_only = ce_l1_fused_grad(x, t, x, ce_weights=w_ce, l1_weights=torch.zeros_like(w_l1))
        assert torch.count_nonzero(l1) == 0
        assert torch.equal(dx, dx_ce_only)


def test_in_place_equals_out_of_place(gpu):
    x, y, idx, t, w_ce, w_l1 = _case(gpu, 257, 32000, indexed=True, seed=5)
    ce_o, l1_o, dx_o = ce_l1_fused_grad(x, t, y, ce_weights=w_ce, l1_weights=w_l1, teacher_indices=idx)
    buf = x.clone()
    ce_i, l1_i, dx_i = ce_l1_fused_grad(buf, t, y, ce_weights=w_ce, l1_weights=w_l1,
                                        teacher_indices=idx, in_place=True)
    assert dx_i.data_ptr() == buf.data_ptr()
    assert torch.equal(ce_i, ce_o) and torch.equal(l1_i, l1_o) and torch.equal(dx_i, dx_o)


def test_fused_pass_fails_closed(gpu):
    x, y, idx, t, w_ce, w_l1 = _case(gpu, 64, 4104, indexed=True, seed=9)
    bad = idx.clone()
    bad[17] = y.shape[0]
    with pytest.raises(ValueError, match="teacher index out of range"):
        ce_l1_fused_grad(x, t, y, ce_weights=w_ce, l1_weights=w_l1, teacher_indices=bad)
    bad_t = t.clone()
    bad_t[3] = 4104
    with pytest.raises(ValueError, match="cross-entropy target out of range"):
        ce_l1_fused_grad(x, bad_t, y, ce_weights=w_ce, l1_weights=w_l1, teacher_indices=idx)
    odd = torch.randn(4, 4103, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        ce_l1_fused_grad(odd, t[:4].clamp(max=4102), odd.clone(), ce_weights=w_ce[:4], l1_weights=w_l1[:4])


@pytest.mark.parametrize("vocab", [32000, 40000])
def test_selective_head_objective_equals_unfused_composition(gpu, vocab):
    g = torch.Generator(device=gpu).manual_seed(vocab)
    rows, hid, trows = 512, 256, 200
    h = (torch.randn(rows, hid, device=gpu, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(vocab, hid, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    th = (torch.randn(trows, hid, device=gpu, generator=g) * 0.5).to(torch.bfloat16)
    teacher = torch.matmul(th, w.t())
    idx = torch.randint(0, trows, (rows,), device=gpu, generator=g)
    t = torch.randint(0, vocab, (rows,), device=gpu, generator=g)
    t[::11] = -100
    w_ce = torch.rand(rows, device=gpu, generator=g) * 0.1
    w_l1 = torch.rand(rows, device=gpu, generator=g) * 0.9

    hf = h.clone().requires_grad_()
    obj, ce, l1 = selective_head_objective(hf, w, t, teacher, teacher_indices=idx, ce_weights=w_ce,
                                           l1_weights=w_l1)
    (obj * 3.0).backward()

    hu = h.clone().requires_grad_()
    logits = torch.matmul(hu, w.t())
    ce_u, l1_u = ce_l1_from_logits(logits, t, teacher, teacher_indices=idx)
    obj_u = torch.dot(ce_u, w_ce) + torch.dot(l1_u, w_l1)
    (obj_u * 3.0).backward()

    assert torch.equal(ce, ce_u.detach()) and torch.equal(l1, l1_u.detach())
    torch.testing.assert_close(obj, obj_u, rtol=1e-6, atol=1e-6)
    # Both paths against dh in fp64: the oracle's dlogits at the same bf16 logits times W. The
    # fused path rounds once more than the unfused one (dlogits is formed before the upstream
    # gradient g is known, so g scales the bf16 dh), hence the bound relative to the unfused error.
    xd = logits.detach().double().cpu().numpy()
    yd = teacher.double().cpu().numpy()[idx.cpu().numpy()]
    td = t.cpu().numpy()
    dl = L.l1_grad(xd, yd, 3.0 * w_l1.double().cpu().numpy()) + L.cross_entropy_grad(
        xd, td, 3.0 * w_ce.double().cpu().numpy())
    ref = torch.as_tensor(dl @ w.double().cpu().numpy())
    err_f, err_u = _rel(hf.grad.cpu(), ref), _rel(hu.grad.cpu(), ref)
    print(f"objective V={vocab}: dh rel_l2 vs fp64 fused {err_f:.2e} unfused {err_u:.2e}")
    assert err_f < 1e-2 and err_f < 1.6 * err_u + 1e-4


@pytest.mark.parametrize("offset,n", [(0, 8 * 1000), (0, 8 * 1000 + 5), (3, 777), (1, 3)])
def test_device_scalar_scale(gpu, offset, n):
    from aspec_amd import _lib

    base = torch.randn(n + offset, device=gpu).to(torch.bfloat16)
    base[offset::97] = torch.inf
    x = base[offset:]
    before = x.clone()
    for value in (0.37, -3.0, 1.0):
        s = torch.tensor(value, device=gpu)
        y = base.clone()[offset:]  # the same alignment as x
        _lib.call("aspec_scale_bf16_by_device_scalar", y.data_ptr(), n, s.data_ptr(),
                  _lib.stream_handle(gpu))
        expect = (x.float() * value).to(torch.bfloat16)  # fp32 product, one round to nearest even
        assert torch.equal(y.view(torch.int16), expect.view(torch.int16)), value
    z = torch.full((1,), float("nan"), device=gpu, dtype=torch.bfloat16)
    _lib.call("aspec_scale_bf16_by_device_scalar", z.data_ptr(), 1, torch.tensor(1.0, device=gpu).data_ptr(),
              _lib.stream_handle(gpu))
    assert torch.isnan(z).all() and torch.equal(x, before)


def test_objective_unit_upstream_gradient_is_dlogits_times_w(gpu):
    g = torch.Generator(device=gpu).manual_seed(3)
    rows, hid, vocab = 256, 128, 4096
    h = (torch.randn(rows, hid, device=gpu, generator=g) * 0.5).to(torch.bfloat16).requires_grad_()
    w = (torch.randn(vocab, hid, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    teacher = (torch.randn(rows, vocab, device=gpu, generator=g)).to(torch.bfloat16)
    t = torch.randint(0, vocab, (rows,), device=gpu, generator=g)
    w_ce = torch.rand(rows, device=gpu, generator=g)
    w_l1 = torch.rand(rows, device=gpu, generator=g)
    obj, _, _ = selective_head_objective(h, w, t, teacher, ce_weights=w_ce, l1_weights=w_l1)
    obj.backward()
    logits = torch.matmul(h.detach(), w.t())
    _, _, dlogits = ce_l1_fused_grad(logits, t, teacher, ce_weights=w_ce, l1_weights=w_l1)
    assert torch.equal(h.grad, torch.matmul(dlogits, w.t().contiguous().t()))
