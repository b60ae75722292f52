"""Elementwise parity at the BASELINE headline configurations, with both error figures recorded.

Attention (bf16 inputs, fp32 accumulation) against the fp32 oracle, every output elementwise:
  * config 2 (Qwen3-8B 4K, 512 x 16 anchors, GQA 32/8): O, LSE, dQ, dK, dV for all 8 KV groups;
  * config 3 (both ragged 32K bins): all outputs of two KV groups per bin;
  * config 4 (32K document, 2048 x 16 anchors, GQA 40/8): all outputs of one KV group.
The oracle is `oracle.attention.attention_group_sampled`, pinned against the dense math-path
oracle on CPU. Tolerances are the reference's bf16-GPU-vs-math bars
(tests/test_thd_attention.py:218-225): atol = rtol = 0.025 for O and LSE, 0.04 for gradients.

Loss at config 2's shape (8192 rows x V = 32000, a 4096-row teacher table addressed by the DSpark
teacher indices, CE targets from the DSpark labels): CE and L1 of every row against the fp64 oracle
(the reference's bars, tests/test_tiled_l1.py:28-46: L1 atol = rtol = 2e-6; CE 2e-5 / 2e-6) and the
gradient of >= 96 sampled rows spread over the persistent kernel's row walk (rel-L2 < 0.01,
atol 1e-6 / rtol 0.02 in bf16, the bar of the fused CE + L1 gradient test), for the two-kernel
path (forward walk, then the backward kernel) and for the one-pass kernel the draft step runs
(`ce_l1_fused_grad`: the forward walk writes the objective's dlogits, with the DSpark
eval-mask x decay weights).

The reference's B = 7 attention study workload (10 x 4096 + 40960 + 49152 context tokens, 6144
captured anchors; tests/golden/dspark_b7_workload.json): every output of two KV groups.

Each output's max-abs and relative-L2 error is printed and, when ASPEC_PARITY_DIR is set, appended
as one JSON line to $ASPEC_PARITY_DIR/parity.jsonl.
"""

import json
import os
import time

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.direct_cp import direct_cp_attention_from_kv
from oracle import attention as A
from oracle import loss as L
from oracle import metadata as M

pytestmark = pytest.mark.gpu


def record(case, name, got, ref, *, atol, rtol):
    got, ref = got.double().cpu(), ref.double().cpu()
    diff = (got - ref).abs()
    max_abs = float(diff.max()) if diff.numel() else 0.0
    rel = float((got - ref).norm() / ref.norm().clamp_min(1e-30))
    line = {"case": case, "output": name, "max_abs": max_abs, "rel_l2": rel, "elements": ref.numel(),
            "atol": atol, "rtol": rtol}
    print(json.dumps(line), flush=True)
    out_dir = os.environ.get("ASPEC_PARITY_DIR")
    if out_dir:
        os.makedirs(out_dir, exist_ok=True)
        with open(os.path.join(out_dir, "parity.jsonl"), "a") as f:
            f.write(json.dumps(line) + "\n")
    torch.testing.assert_close(got, ref, atol=atol, rtol=rtol)
    return max_abs, rel


def _attention_inputs(w, seed):
    g = torch.Generator().manual_seed(seed)
    hq, hkv, d = w.q_heads, w.kv_heads, w.head_dim
    q = (torch.randn(w.num_queries, hq, d, generator=g) * 0.5).bfloat16()
    k = (torch.randn(w.num_keys, hkv, d, generator=g) * 0.5).bfloat16()
    v = (torch.randn(w.num_keys, hkv, d, generator=g) * 0.5).bfloat16()
    dout = torch.randn(w.num_queries, hq, d, generator=g).bfloat16()
    dlse = torch.randn(hq, w.num_queries, generator=g) * 0.1
    return q, k, v, dout, dlse


def _attention_parity(w, device, groups, seed, case):
    """GPU forward + backward (with an LSE gradient) of a whole workload, then every output of the
    listed KV groups against the chunked fp32 oracle."""
    t0 = time.perf_counter()
    q, k, v, dout, dlse = _attention_inputs(w, seed)
    dev = lambda x: x.to(device)[None].transpose(1, 2).requires_grad_()  # noqa: E731
    qd, kd, vd = dev(q), dev(k), dev(v)
    meta = W.metadata_for(w, device)
    out, lse = direct_cp_attention_from_kv(qd, kd, vd, meta)
    obj = (out.float() * dout.to(device)[None].transpose(1, 2).float()).sum() + (lse * dlse.to(device)[None]).sum()
    obj.backward()
    torch.cuda.synchronize()
    got = {"O": out.detach()[0].float().cpu(), "LSE": lse.detach()[0].cpu(), "dQ": qd.grad[0].float().cpu(),
           "dK": kd.grad[0].float().cpu(), "dV": vd.grad[0].float().cpu()}
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    group = w.q_heads // w.kv_heads
    qt, dt = q.float().transpose(0, 1), dout.float().transpose(0, 1)  # [Hq, Nq, D]
    all_rows = np.arange(w.num_queries)
    figures = {}
    for kv in groups:
        sl = slice(kv * group, (kv + 1) * group)
        ref = A.attention_group_sampled(qt[sl], k[:, kv].float(), v[:, kv].float(), ends,
                                        w.head_dim ** -0.5, dt[sl], dlse[sl], dq_rows=all_rows,
                                        key_ranges=[(0, w.num_keys)], chunk=256)
        keep = ref["lse"][0] > A.MASK_VALUE / 2
        tag = f"{case}/kv{kv}"
        figures[kv] = {
            "O": record(tag, "O", got["O"][sl], ref["out"], atol=0.025, rtol=0.025),
            "LSE": record(tag, "LSE", got["LSE"][sl][:, keep], ref["lse"][:, keep], atol=0.025, rtol=0.025),
            "dQ": record(tag, "dQ", got["dQ"][sl], ref["dq"], atol=0.04, rtol=0.04),
            "dK": record(tag, "dK", got["dK"][kv], ref["dkv"][0][0], atol=0.04, rtol=0.04),
            "dV": record(tag, "dV", got["dV"][kv], ref["dkv"][0][1], atol=0.04, rtol=0.04),
        }
        assert torch.all(got["LSE"][sl][:, ~keep] == A.MASK_VALUE)
        assert not got["O"][sl][:, ~keep].any()
    print(f"{case}: {len(groups)} KV group(s) in {time.perf_counter() - t0:.1f} s", flush=True)
    return figures


def test_config2_attention_all_kv_groups_elementwise(gpu):
    w = W.config2()
    _attention_parity(w, gpu, range(w.kv_heads), seed=21, case="config2")


@pytest.mark.parametrize("bin_index", [0, 1])
def test_config3_attention_two_kv_groups_elementwise(gpu, bin_index):
    w = W.config3(0, bin_index)
    _attention_parity(w, gpu, (0, w.kv_heads - 1), seed=30 + bin_index, case=f"config3_bin{bin_index}")


def test_config4_attention_one_kv_group_elementwise(gpu):
    """GQA 40/8 (a group of five): O, LSE, dQ for all 32768 rows of KV group 3's five query heads,
    and dK / dV for all 65536 keys of KV head 3 (the first context key tiles are split over many
    work units, so their dK/dV go through the split-tile accumulation)."""
    w = W.config4()
    _attention_parity(w, gpu, (3,), seed=41, case="config4")


def test_reference_b7_workload_two_kv_groups_elementwise(gpu):
    """The reference's published attention workload (docs/dspark_attn_kernel_optimization.md:49-51):
    B = 7 blocks straddle the kernels' 32-row query tiles and 64/128-key tiles, twelve documents
    share one key space, and the anchors are in the sampler's order (one wraparound per
    document). O, LSE, dQ of all 43008 rows and dK, dV of all 174080 keys for KV groups 0 and 7."""
    w = W.reference_b7()
    _attention_parity(w, gpu, (0, w.kv_heads - 1), seed=70, case="reference_b7")


def _config2_loss_inputs(gpu, seed):
    from aspec_amd.targets import dspark_targets

    w = W.config2()
    vocab, rows = 32000, w.num_queries
    g = torch.Generator(device=gpu).manual_seed(seed)
    anchors = torch.as_tensor(w.anchors, device=gpu)[None]
    keep = torch.as_tensor(w.keep, device=gpu)[None]
    input_ids = torch.randint(0, vocab, (1, w.context_length), device=gpu, generator=g)
    loss_mask = torch.ones(1, w.context_length, dtype=torch.long, device=gpu)
    docs = torch.as_tensor(w.ctx_doc_ids, device=gpu)[None]
    tg = dspark_targets(anchors, keep, input_ids, loss_mask, w.block_size, loss_decay_gamma=4.0,
                        ctx_doc_ids=docs)
    targets = tg.target_ids.reshape(-1).clone()
    targets[::97] = -100  # ignored rows
    tidx = tg.teacher_index.reshape(-1).contiguous()
    x = (torch.randn(rows, vocab, device=gpu, generator=g) * 2).bfloat16()
    table = (torch.randn(w.context_length, vocab, device=gpu, generator=g) * 2).bfloat16()
    return w, tg, targets, tidx, x, table


def _loss_oracle_check(case, x, table, targets, tidx, ce, l1, dlogits, gce, gl1):
    """CE and L1 of every row, and dlogits of >= 96 rows spread over the persistent walk, against
    the fp64 oracle."""
    rows = x.shape[0]
    xc, tc, ic = x.cpu(), targets.cpu().numpy(), tidx.cpu().numpy()
    table_c = table.cpu()
    ref_ce, ref_l1 = np.empty(rows), np.empty(rows)
    for r0 in range(0, rows, 512):
        xd = xc[r0:r0 + 512].double().numpy()
        yd = table_c[torch.as_tensor(ic[r0:r0 + 512])].double().numpy()
        ref_ce[r0:r0 + 512] = L.cross_entropy(xd, tc[r0:r0 + 512])
        ref_l1[r0:r0 + 512] = L.l1(xd, yd)
    record(case, "CE", ce.detach().cpu(), torch.as_tensor(ref_ce), atol=2e-5, rtol=2e-6)
    record(case, "L1", l1.detach().cpu(), torch.as_tensor(ref_l1), atol=2e-6, rtol=2e-6)
    # the walk's first and last rows, rows at the CU-count stride (start, middle and end of each
    # CU's share) and a few at an odd stride
    sample = np.unique(np.concatenate([np.arange(4), np.arange(rows - 4, rows), np.arange(1, rows, 256),
                                       np.arange(128, rows, 256), np.arange(255, rows, 256),
                                       np.arange(1, rows, 97)[:8]]))
    assert sample.size >= 96
    xd = xc[sample].double().numpy()
    yd = table_c[torch.as_tensor(ic[sample])].double().numpy()
    ref_g = (L.cross_entropy_grad(xd, tc[sample], gce.cpu().double().numpy()[sample])
             + L.l1_grad(xd, yd, gl1.cpu().double().numpy()[sample]))
    got_g = dlogits[torch.as_tensor(sample, device=dlogits.device)].cpu()
    _, rel = record(case, "dlogits (sampled rows)", got_g.double(), torch.as_tensor(ref_g),
                    atol=1e-6, rtol=0.02)
    assert rel < 0.01
    torch.testing.assert_close(got_g, torch.as_tensor(ref_g).to(torch.bfloat16), atol=1e-6, rtol=0.02)


def test_config2_fused_loss_all_rows_indexed_teacher(gpu):
    """The one-pass loss the draft step ships (`ce_l1_fused_grad`: the persistent forward walk,
    32 rows per CU at 8192 rows, writing the objective's dlogits as each row's statistics are
    final) with the DSpark indexed teacher and the step's weights (0.1 / 0.9 times the eval mask x
    exp(-k/4) decay over their sum): CE and L1 of every row, dlogits of >= 96 rows over the walk."""
    from aspec_amd.loss import ce_l1_fused_grad

    w, tg, targets, tidx, x, table = _config2_loss_inputs(gpu, 53)
    wts = tg.weights.reshape(-1).float()
    gce, gl1 = 0.1 * wts / wts.sum(), 0.9 * wts / wts.sum()
    ce, l1, dlogits = ce_l1_fused_grad(x, targets, table, ce_weights=gce, l1_weights=gl1,
                                       teacher_indices=tidx)
    torch.cuda.synchronize()
    _loss_oracle_check("config2_fused_loss", x, table, targets, tidx, ce, l1, dlogits, gce, gl1)


def test_config2_loss_all_rows_indexed_teacher(gpu):
    """CE + L1 at 8192 x 32000 with the DSpark indexed teacher: the bench's persistent forward
    (one workgroup per CU walking 32 rows each, the next row's teacher index and target prefetched
    while the current row is reduced) checked on every row, and the fused backward on 96 rows:
    the first and last rows of the walk and rows at the CU-count strides."""
    from aspec_amd.loss import ce_l1_from_logits

    w, tg, targets, tidx, x, table = _config2_loss_inputs(gpu, 52)
    rows = x.shape[0]
    g = torch.Generator(device=gpu).manual_seed(152)
    gce = torch.randn(rows, device=gpu, generator=g)
    gl1 = torch.randn(rows, device=gpu, generator=g)
    xin = x.clone().requires_grad_()
    ce, l1 = ce_l1_from_logits(xin, targets, table, teacher_indices=tidx)
    ((ce * gce).sum() + (l1 * gl1).sum()).backward()
    torch.cuda.synchronize()
    _loss_oracle_check("config2_loss", x, table, targets, tidx, ce, l1, xin.grad, gce, gl1)
