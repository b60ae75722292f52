"""Pins the attention and loss oracles (CPU): independent per-row loops, closed forms, special
values and finite-difference gradients."""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from oracle import attention as A
from oracle import loss as L
from oracle import metadata as M


def _dense(w):
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    return M.endpoints_to_dense(ends, w.num_keys)


def _small():
    g = torch.Generator().manual_seed(47)
    w = W.from_layout("small", [9, 17, 7], np.array([0, 4, 7, 9, 12, 20, 28, 31]),
                      np.array([0, 0, 0, 1, 1, 1, 2, 2]), 2,
                      keep=[True, True, False, True, True, True, True, True])
    q = torch.randn(4, w.num_queries, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, w.num_keys, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, w.num_keys, 16, generator=g, dtype=torch.float64)
    return w, q, k, v


def test_attention_matches_per_row_loop():
    w, q, k, v = _small()
    vis = _dense(w)
    out, lse = A.attention(q, k, v, vis, 0.25)
    for head in range(4):
        for row in range(w.num_queries):
            o_ref, l_ref = A.attention_row_loop(q, k, v, vis, 0.25, head, row)
            np.testing.assert_allclose(out[head, row].numpy(), o_ref, rtol=1e-12, atol=1e-12)
            assert abs(float(lse[head, row]) - l_ref) < 1e-10


def test_dropped_rows_and_single_key_rows():
    w, q, k, v = _small()
    vis = _dense(w)
    out, lse = A.attention(q, k, v, vis, 0.25)
    # block 2 (rows 4, 5) is dropped: O = 0 and LSE = MASK_VALUE (direct_cp.py:470-477)
    assert torch.all(out[:, 4:6] == 0) and torch.all(lse[:, 4:6] == A.MASK_VALUE)
    # block 0 (anchor 0) sees only its two draft keys 33, 34; restrict to one key by hand:
    vis1 = np.zeros_like(vis)
    vis1[0, 33] = True
    out1, lse1 = A.attention(q, k, v, vis1, 0.25)
    torch.testing.assert_close(out1[0, 0], v[0, 33], rtol=0, atol=1e-15)
    assert abs(float(lse1[0, 0]) - 0.25 * float(q[0, 0] @ k[0, 33])) < 1e-12


def test_attention_gradients_match_finite_differences():
    w, q, k, v = _small()
    vis = _dense(w)
    g = torch.Generator().manual_seed(3)
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    dlse = torch.randn(q.shape[:2], generator=g, dtype=torch.float64)
    _, _, (dq, dk, dv) = A.attention(q, k, v, vis, 0.25, dout=dout, dlse=dlse)

    def objective(qq, kk, vv):
        o, l = A.attention(qq, kk, vv, vis, 0.25)
        keep = torch.as_tensor(vis.any(-1))
        return float((o * dout).sum() + (l * dlse * keep).sum())

    eps = 1e-6
    for tensor, grad, idx in ((q, dq, (1, 7, 3)), (k, dk, (0, 10, 5)), (v, dv, (1, 41, 2)), (k, dk, (1, 35, 0))):
        plus, minus = tensor.clone(), tensor.clone()
        plus[idx] += eps
        minus[idx] -= eps
        args_p = [plus if t is tensor else t for t in (q, k, v)]
        args_m = [minus if t is tensor else t for t in (q, k, v)]
        fd = (objective(*args_p) - objective(*args_m)) / (2 * eps)
        assert abs(fd - float(grad[idx])) < 1e-6 * max(1.0, abs(fd))


def test_l1_special_values():
    x = np.array([[0.0, -np.inf], [1.0, 2.0], [3.0, 3.0]])
    y = np.array([[-np.inf, 0.0], [1.0, 2.0], [0.0, 0.0]])
    np.testing.assert_allclose(L.l1(x, y), [2.0, 0.0, 0.0], atol=1e-15)
    np.testing.assert_array_equal(L.l1_grad(x[1:], y[1:], np.ones(2)), 0.0)
    # two-point closed form: |p - q| summed = 2 |sigmoid(a) - sigmoid(b)|
    a, b = 0.3, -1.2
    expected = 2 * abs(1 / (1 + np.exp(-a)) - 1 / (1 + np.exp(-b)))
    np.testing.assert_allclose(L.l1([[a, 0.0]], [[b, 0.0]]), [expected], rtol=1e-14)


def test_ce_special_values():
    x = np.zeros((2, 7))
    np.testing.assert_allclose(L.cross_entropy(x, [3, -100]), [np.log(7), 0.0], rtol=1e-15)
    g = L.cross_entropy_grad(x, [3, -100], [1.0, 1.0])
    np.testing.assert_allclose(g[0], np.full(7, 1 / 7) - np.eye(7)[3], rtol=1e-14)
    assert not g[1].any()


@pytest.mark.parametrize("fn", ["l1", "ce"])
def test_loss_gradients_match_finite_differences(fn):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 11)) * 2
    y = rng.standard_normal((3, 11)) * 2
    t = np.array([1, 4, 10])
    g = rng.standard_normal(3)

    def f(xx):
        return float((L.l1(xx, y) * g).sum()) if fn == "l1" else float((L.cross_entropy(xx, t) * g).sum())

    grad = L.l1_grad(x, y, g) if fn == "l1" else L.cross_entropy_grad(x, t, g)
    eps = 1e-6
    for idx in [(0, 0), (1, 4), (2, 10), (2, 3)]:
        p, m = x.copy(), x.copy()
        p[idx] += eps
        m[idx] -= eps
        assert abs((f(p) - f(m)) / (2 * eps) - grad[idx]) < 1e-7


def test_sampled_group_oracle_equals_dense_oracle():
    """`attention_group_sampled` (the chunked single-KV-group form used at config 4) against the
    dense `attention` on a small ragged layout with a dropped block and an LSE gradient: O and
    LSE for every row, dQ for sampled rows and dK/dV for key ranges that straddle the context /
    draft boundary, all in float64, for several chunk sizes (chunk edges inside blocks)."""
    w, q, k, v = _small()
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    vis = M.endpoints_to_dense(ends, w.num_keys)
    g = torch.Generator().manual_seed(3)
    dout = torch.randn(4, w.num_queries, 16, generator=g, dtype=torch.float64)
    dlse = torch.randn(4, w.num_queries, generator=g, dtype=torch.float64)
    out, lse, (dq, dk, dv) = A.attention(q, k, v, vis, 0.3, dout=dout, dlse=dlse)
    rows = [0, 3, 5, w.num_queries - 1]
    ranges = [(0, 5), (w.context_length - 3, w.context_length + 4), (w.num_keys - 2, w.num_keys)]
    for kv in range(2):
        sl = slice(2 * kv, 2 * kv + 2)
        for chunk in (3, 7, 64):
            got = A.attention_group_sampled(q[sl], k[kv], v[kv], ends, 0.3, dout[sl], dlse[sl],
                                            dq_rows=rows, key_ranges=ranges, chunk=chunk,
                                            dtype=torch.float64)
            torch.testing.assert_close(got["out"], out[sl], rtol=1e-12, atol=1e-12)
            torch.testing.assert_close(got["lse"], lse[sl], rtol=1e-12, atol=1e-12)
            torch.testing.assert_close(got["dq"], dq[sl][:, rows], rtol=1e-10, atol=1e-12)
            for (k0, k1), (gk, gv) in zip(ranges, got["dkv"]):
                torch.testing.assert_close(gk, dk[kv, k0:k1], rtol=1e-10, atol=1e-12)
                torch.testing.assert_close(gv, dv[kv, k0:k1], rtol=1e-10, atol=1e-12)


def test_dense_oracle_kv_head_subset_equals_full_run():
    w, q, k, v = _small()
    vis = _dense(w)
    g = torch.Generator().manual_seed(4)
    dout = torch.randn(4, w.num_queries, 16, generator=g, dtype=torch.float64)
    full = A.attention(q, k, v, vis, 0.25, dout=dout)
    part = A.attention(q, k, v, vis, 0.25, dout=dout, kv_heads=[1])
    torch.testing.assert_close(part[0][2:], full[0][2:])
    torch.testing.assert_close(part[1][2:], full[1][2:])
    for a, b in zip(part[2], full[2]):
        torch.testing.assert_close(a[2:] if a.shape[0] == 4 else a[1:], b[2:] if b.shape[0] == 4 else b[1:])
    assert not part[0][:2].any()
