"""The one-GPU part of Direct CP: each rank's share of the attention (all gathered queries against
the rank's context shard and its own draft blocks, direct_cp.py:1077-1093) run one virtual rank
after another on one GPU, and the ranks' (O, LSE) partials merged exactly
(`merge_attention_partials`, direct_cp.py:362-367,460-467). No collectives: the all-gather of the
queries and the all-to-all of the partials are index permutations here.

* The shard endpoints (`aspec_thd_cp_shard_endpoints`) equal `oracle.metadata.cp_endpoints` bit
  for bit, for cp in {2, 4}, contiguous and zigzag ownership, with and without windows / causal
  draft blocks, on packed multi-document rows.
* Config 2 sharded over cp in {2, 4} ranks, both layouts: the merged output and LSE match the
  unsharded HIP result within the reference's attention bars (atol = rtol = 0.025,
  tests/test_thd_attention.py:218-225), and so do dQ (summed over the ranks' partials), dK and dV
  (each key's gradient from the rank that holds it) within 0.04, through autograd of the merge and
  each partial (which therefore carries an LSE gradient).
"""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.direct_cp import (DirectCPMetadata, build_context_positions, cp_shard_endpoints,
                                 direct_cp_attention_from_kv, direct_cp_partial_attention,
                                 merge_attention_partials)
from oracle import metadata as M

pytestmark = pytest.mark.gpu


def _rank_metadata(w, rank, cp, layout, device, n=None, **opts):
    n = w.num_blocks if n is None else n
    pos = build_context_positions(w.context_length, rank, cp, layout=layout)
    t = lambda x, dt: torch.as_tensor(x, dtype=dt, device=device)[None]  # noqa: E731
    return pos.numpy(), DirectCPMetadata(
        t(w.anchors[:n], torch.long), t(w.keep[:n], torch.bool), pos[None].to(device), w.block_size, rank, cp,
        "virtual", context_doc_ids=t(w.ctx_doc_ids[pos.numpy()], torch.long),
        anchor_doc_ids=t(w.anchor_doc_ids[:n], torch.long), sequence_length=w.sequence_length,
        layout=layout, **opts)


@pytest.mark.parametrize("cp", [2, 4])
@pytest.mark.parametrize("layout", ["contiguous", "zigzag"])
@pytest.mark.parametrize("opts", [{}, {"draft_is_causal": True, "context_window": 300}, {"query_window": 5}])
def test_shard_endpoints_bit_exact(gpu, cp, layout, opts):
    for w in (W.config1(0), W.config2(), W.config3(0, 0)):
        n = w.num_blocks - w.num_blocks % (2 * cp)
        for rank in range(cp):
            pos, meta = _rank_metadata(w, rank, cp, layout, gpu, n, **opts)
            got = cp_shard_endpoints(meta, gpu).cpu().numpy()
            collective, local = M.cp_blocks(n, rank, cp, layout)
            want = M.cp_endpoints(w.anchors[:n], w.keep[:n], w.anchor_doc_ids[:n], pos, w.ctx_doc_ids[pos],
                                  w.block_size, w.sequence_length, collective, local, **opts)
            np.testing.assert_array_equal(got, want, err_msg=f"{w.name} rank {rank}/{cp} {layout} {opts}")


@pytest.mark.parametrize("cp", [2, 4])
@pytest.mark.parametrize("layout", ["contiguous", "zigzag"])
def test_config2_sharded_partials_merge_to_the_unsharded_attention(gpu, cp, layout):
    w = W.config2()
    B, T, n = w.block_size, w.context_length, w.num_blocks
    g = torch.Generator(device=gpu).manual_seed(60 + cp)

    def rows(count, heads, scale):
        return (torch.randn(1, count, heads, w.head_dim, device=gpu, generator=g) * scale).to(torch.bfloat16)

    q_tok, k_tok, v_tok = rows(w.num_queries, w.q_heads, 0.5), rows(w.num_keys, w.kv_heads, 0.5), rows(w.num_keys, w.kv_heads, 0.5)
    dout_tok = rows(w.num_queries, w.q_heads, 1.0)
    view = lambda x: x.transpose(1, 2)  # noqa: E731  token-major storage as [1, H, L, D]
    # unsharded reference
    q0, k0, v0 = (view(x).detach().requires_grad_() for x in (q_tok, k_tok, v_tok))
    out0, lse0 = direct_cp_attention_from_kv(q0, k0, v0, W.metadata_for(w, gpu))
    (out0.float() * view(dout_tok).float()).sum().backward()
    # sharded: every rank's partial of all gathered queries, merged
    q, k, v = (view(x).detach().requires_grad_() for x in (q_tok, k_tok, v_tok))
    collective = M.cp_blocks(n, 0, cp, layout)[0]
    qrows = torch.as_tensor(np.repeat(collective, B) * B + np.tile(np.arange(B), n), device=gpu)
    outs, lses = [], []
    for rank in range(cp):
        pos, meta = _rank_metadata(w, rank, cp, layout, gpu)
        local = meta.local_block_ids.numpy()
        keys = np.concatenate([pos, T + np.repeat(local, B) * B + np.tile(np.arange(B), local.size)])
        kidx = torch.as_tensor(keys, device=gpu)
        o, l = direct_cp_partial_attention(q.index_select(2, qrows), k.index_select(2, kidx),
                                           v.index_select(2, kidx), meta)
        outs.append(o.float())
        lses.append(l)
    out, lse = merge_attention_partials(torch.stack(outs), torch.stack(lses))
    inverse = torch.empty_like(qrows)
    inverse[qrows] = torch.arange(qrows.numel(), device=gpu)
    out, lse = out.index_select(2, inverse), lse.index_select(2, inverse)  # back to block order
    (out * view(dout_tok).float()).sum().backward()
    torch.cuda.synchronize()

    def check(name, got, ref, tol):
        got, ref = got.double().cpu(), ref.double().cpu()
        err = (got - ref).abs().max().item()
        rel = ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()
        print(f"cp={cp} {layout} {name}: max_abs {err:.2e} rel_l2 {rel:.2e}", flush=True)
        torch.testing.assert_close(got, ref, atol=tol, rtol=tol)

    kept = lse0 > -1e29
    check("O", out, out0.float(), 0.025)
    check("LSE", lse[kept], lse0[kept], 0.025)
    assert torch.all(lse[~kept] == -1e30)
    check("dQ", q.grad, q0.grad, 0.04)
    check("dK", k.grad, k0.grad, 0.04)
    check("dV", v.grad, v0.grad, 0.04)


def test_merge_keeps_the_mask_value_for_rows_without_keys(gpu):
    """`_merge_partials`' conventions: a row with keys in one partial only takes that partial
    exactly; a row whose every partial is -1e30 keeps LSE = -1e30."""
    outs = torch.randn(3, 1, 2, 4, 8, device=gpu)
    lses = torch.randn(3, 1, 2, 4, device=gpu)
    lses[1:, :, :, 0] = -1e30
    lses[:, :, :, 1] = -1e30
    outs[:, :, :, 1] = 0
    out, lse = merge_attention_partials(outs, lses)
    torch.testing.assert_close(out[:, :, 0], outs[0, :, :, 0])
    torch.testing.assert_close(lse[:, :, 0], lses[0, :, :, 0])
    assert torch.all(lse[:, :, 1] <= -1e29) and not out[:, :, 1].any()
    ref = torch.logsumexp(lses[:, :, :, 2:], dim=0)
    torch.testing.assert_close(lse[:, :, 2:], ref)
    w = torch.softmax(lses[:, :, :, 2:], dim=0)
    torch.testing.assert_close(out[:, :, 2:], (w.unsqueeze(-1) * outs[:, :, :, 2:]).sum(0))
