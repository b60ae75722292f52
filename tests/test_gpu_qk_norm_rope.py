"""HIP fused Q/K RMSNorm + RoPE (forward and backward) vs the float64 oracle.

Cases and tolerances are the reference's (tests/test_dspark_qk_cutedsl.py:213-309): batch /
context / draft lengths (1,5,3), (1,17,7), (2,5,3), 8 query and 2 KV heads, head_dim 128,
eps 1e-6, positions drawn from a 67-row cos/sin table of random angles; outputs and input
gradients within atol = rtol = 2e-2, the fp32 weight gradients (read through the C ABI; autograd
rounds them to the bf16 weights) within rtol 1e-5 / atol 2e-5, and two backward runs bitwise
equal. Max-abs and relative-L2 errors are printed for every tensor. The same cases run with fp16
activations (the reference's kernel serves bf16 and fp16, dspark_qk_norm_rope.py:169-170; its
tests run bf16): outputs and input gradients within 2e-3, one fp16 rounding of the fp64 result on
the same fp16 inputs.
"""

import ctypes

import numpy as np
import pytest
import torch

from aspec_amd import _lib
from aspec_amd.dspark_qk_norm_rope import dspark_qk_norm_rope, last_position_error
from oracle import qk_norm_rope as Q

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _inputs(device, batch, lc, ld, hq=8, hkv=2, positions=67, seed=None, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed if seed is not None else batch * 10_000 + lc * 100 + ld)
    bf = dtype
    query = torch.randn(batch, ld, hq * 128, generator=g).to(bf)
    ctx = torch.randn(batch, lc, hkv * 128, generator=g).to(bf)
    drf = torch.randn(batch, ld, hkv * 128, generator=g).to(bf)
    wq = torch.randn(128, generator=g).to(bf)
    wk = torch.randn(128, generator=g).to(bf)
    ang = torch.randn(positions, 64, generator=g)
    ang = torch.cat((ang, ang), dim=-1)
    cos, sin = ang.cos().to(bf), ang.sin().to(bf)
    pq = torch.randint(positions, (batch, ld), generator=g)
    pc = torch.randint(positions, (batch, lc), generator=g)
    pd = torch.randint(positions, (batch, ld), generator=g)
    cpu = dict(query=query, ctx=ctx, drf=drf, wq=wq, wk=wk, cos=cos, sin=sin, pq=pq, pc=pc, pd=pd)
    dev = {k: v.to(device) for k, v in cpu.items()}
    return cpu, dev


def _run(dev, hq, hkv, grads=None, requires_grad=True):
    t = {k: (v.clone().requires_grad_() if requires_grad and k in ("query", "ctx", "drf", "wq", "wk") else v)
         for k, v in dev.items()}
    q, k = dspark_qk_norm_rope(t["query"], t["ctx"], t["drf"], t["wq"], t["wk"], EPS,
                               t["cos"][None, None], t["sin"][None, None], t["pq"], t["pc"], t["pd"],
                               hq, hkv, 128)
    if grads is None:
        return q, k, None
    torch.autograd.backward((q, k), grads)
    return q, k, tuple(t[n].grad for n in ("query", "ctx", "drf", "wq", "wk"))


def _abi_weight_grads(dev, hq, hkv, gq, gk):
    """fp32 dw_q, dw_k straight from the C ABI (autograd rounds them to the bf16 weights' dtype)."""
    b, ld = dev["pq"].shape
    lc = dev["pc"].shape[1]
    d = dev["query"].device
    q_out = torch.empty(b * ld, hq, 128, device=d, dtype=dev["query"].dtype)
    k_out = torch.empty(b * (lc + ld), hkv, 128, device=d, dtype=dev["query"].dtype)
    rq = torch.empty(b * ld, hq, device=d)
    rk = torch.empty(b * (lc + ld), hkv, device=d)
    flags = torch.zeros(1, dtype=torch.int32, device=d)
    stream = _lib.stream_handle(d)
    cos, sin = dev["cos"], dev["sin"]
    common = (dev["wq"].data_ptr(), dev["wk"].data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
              cos.stride(0), dev["pq"].data_ptr(), dev["pc"].data_ptr(), dev["pd"].data_ptr(), b, lc, ld,
              hq, hkv, 128, EPS, _lib.mask_dtype_code(dev["query"]))
    _lib.call("aspec_qk_norm_rope_fwd", dev["query"].data_ptr(), dev["ctx"].data_ptr(), dev["drf"].data_ptr(),
              *common, q_out.data_ptr(), k_out.data_ptr(), rq.data_ptr(), rk.data_ptr(), flags.data_ptr(),
              stream)
    size = ctypes.c_size_t()
    _lib.call("aspec_qk_norm_rope_bwd_workspace_bytes", b, lc, ld, hq, hkv, ctypes.byref(size))
    ws = torch.empty(size.value, dtype=torch.uint8, device=d)
    dq, dc, dd = torch.empty_like(dev["query"]), torch.empty_like(dev["ctx"]), torch.empty_like(dev["drf"])
    dwq, dwk = torch.empty(128, device=d), torch.empty(128, device=d)
    gq, gk = gq.contiguous(), gk.contiguous()
    _lib.call("aspec_qk_norm_rope_bwd", gq.data_ptr(), gk.data_ptr(), dev["query"].data_ptr(),
              dev["ctx"].data_ptr(), dev["drf"].data_ptr(), rq.data_ptr(), rk.data_ptr(), *common,
              dq.data_ptr(), dc.data_ptr(), dd.data_ptr(), dwq.data_ptr(), dwk.data_ptr(), ws.data_ptr(),
              flags.data_ptr(), stream)
    return dwq, dwk


def _oracle(cpu, hq, hkv):
    b, ld = cpu["pq"].shape
    lc = cpu["pc"].shape[1]
    f = lambda x: x.double().numpy()  # noqa: E731
    args = (f(cpu["query"]).reshape(b, ld, hq, 128), f(cpu["ctx"]).reshape(b, lc, hkv, 128),
            f(cpu["drf"]).reshape(b, ld, hkv, 128), f(cpu["wq"]), f(cpu["wk"]), f(cpu["cos"]),
            f(cpu["sin"]), cpu["pq"].numpy(), cpu["pc"].numpy(), cpu["pd"].numpy(), EPS)
    return args


def _report(name, got, ref, atol, rtol):
    got = got.detach().double().cpu().numpy().reshape(ref.shape)
    err = np.abs(got - ref).max()
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    print(f"{name}: max_abs={err:.3e} rel_l2={rel:.3e}")
    np.testing.assert_allclose(got, ref, atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize(("batch", "lc", "ld"), [(1, 5, 3), (1, 17, 7), (2, 5, 3)])
def test_forward_backward_match_oracle_and_are_deterministic(gpu, batch, lc, ld, dtype):
    hq, hkv = 8, 2
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-3
    cpu, dev = _inputs(gpu, batch, lc, ld, dtype=dtype)
    g = torch.Generator().manual_seed(7)
    gq = torch.randn(batch, ld, hq, 128, generator=g).to(dtype)
    gk = torch.randn(batch, lc + ld, hkv, 128, generator=g).to(dtype)
    q, k, grads = _run(dev, hq, hkv, (gq.to(gpu), gk.to(gpu)))
    assert q.dtype == dtype and k.dtype == dtype and all(t.dtype == dtype for t in grads)
    args = _oracle(cpu, hq, hkv)
    rq, rk, _, _ = Q.prepare_qk(*args)
    _report("q", q, rq, tol, tol)
    _report("k", k, rk, tol, tol)
    ref = Q.prepare_qk_grad(*args, gq.double().numpy(), gk.double().numpy())
    # input gradients, and the weight gradients autograd hands the weights (rounded to their dtype;
    # the bar of the reference's bf16 test for those two)
    for name, got, r, t in zip(("dquery", "dcontext_key", "ddraft_key", "dwq(act)", "dwk(act)"),
                               grads, ref, (tol, tol, tol, 2e-2, 2e-2)):
        _report(name, got, r, t, t)
    # the kernel's fp32 weight gradients, at the reference's bar
    dwq, dwk = _abi_weight_grads(dev, hq, hkv, gq.to(gpu), gk.to(gpu))
    _report("dwq(fp32)", dwq, ref[3], 2e-5, 1e-5)
    _report("dwk(fp32)", dwk, ref[4], 2e-5, 1e-5)
    _, _, again = _run(dev, hq, hkv, (gq.to(gpu), gk.to(gpu)))
    for first, second in zip(grads, again):
        assert torch.equal(first, second)
    assert not last_position_error()


def test_rstd_and_key_join_layout(gpu):
    cpu, dev = _inputs(gpu, 2, 4, 3)
    q, k, _ = _run(dev, 8, 2, requires_grad=False)
    rq, rk, _, _ = Q.prepare_qk(*_oracle(cpu, 8, 2))
    assert q.shape == (2, 3, 8, 128) and k.shape == (2, 7, 2, 128)
    # the first context token of batch row 1 sits right after batch row 0's draft tokens
    _report("k[1, 0]", k[1, 0], rk[1, 0], 2e-2, 2e-2)


def test_config2_geometry_against_sampled_rows_and_full_weight_gradients(gpu):
    # one 4096-token context, 512 anchors x 16 = 8192 draft tokens, GQA 32/8
    hq, hkv, lc, ld = 32, 8, 4096, 8192
    cpu, dev = _inputs(gpu, 1, lc, ld, hq=hq, hkv=hkv, positions=lc + 64, seed=11)
    g = torch.Generator().manual_seed(12)
    gq = torch.randn(1, ld, hq, 128, generator=g).bfloat16()
    gk = torch.randn(1, lc + ld, hkv, 128, generator=g).bfloat16()
    q, k, grads = _run(dev, hq, hkv, (gq.to(gpu), gk.to(gpu)))
    args = _oracle(cpu, hq, hkv)
    rows_q = np.random.default_rng(0).choice(ld, 64, replace=False)
    rows_k = np.random.default_rng(1).choice(lc + ld, 64, replace=False)
    rq, rk, _, _ = Q.prepare_qk(*args)
    _report("q[sample]", q[0, rows_q], rq[0, rows_q], 2e-2, 2e-2)
    _report("k[sample]", k[0, rows_k], rk[0, rows_k], 2e-2, 2e-2)
    dq, dc, dd, dwq, dwk = Q.prepare_qk_grad(*args, gq.double().numpy(), gk.double().numpy())
    _report("dquery[sample]", grads[0].view(1, ld, hq, 128)[0, rows_q], dq[0, rows_q], 2e-2, 2e-2)
    # fp32 sums over 262,144 (q) and 98,304 (k) head rows: relative 1e-4 of the largest entry
    fq, fk = _abi_weight_grads(dev, hq, hkv, gq.to(gpu), gk.to(gpu))
    _report("dwq(fp32)", fq, dwq, 1e-4 * np.abs(dwq).max(), 1e-4)
    _report("dwk(fp32)", fk, dwk, 1e-4 * np.abs(dwk).max(), 1e-4)


def test_positions_outside_the_table_give_nan_rows(gpu):
    cpu, dev = _inputs(gpu, 1, 5, 3)
    dev["pq"] = dev["pq"].clone()
    dev["pq"][0, 1] = 67  # one past the table
    q, k, _ = _run(dev, 8, 2, requires_grad=False)
    assert torch.isnan(q[0, 1]).all() and torch.isfinite(q[0, 0]).all() and torch.isfinite(k).all()
    assert last_position_error()


def test_unsupported_inputs_fail_closed(gpu):
    cpu, dev = _inputs(gpu, 1, 5, 3)
    with pytest.raises(ValueError, match="bf16/f16"):
        dspark_qk_norm_rope(dev["query"].float(), dev["ctx"].float(), dev["drf"].float(), dev["wq"].float(),
                            dev["wk"].float(), EPS, dev["cos"][None, None], dev["sin"][None, None],
                            dev["pq"], dev["pc"], dev["pd"], 8, 2, 128)
    with pytest.raises(ValueError, match="share one dtype"):
        dspark_qk_norm_rope(dev["query"].half(), dev["ctx"], dev["drf"], dev["wq"], dev["wk"], EPS,
                            dev["cos"][None, None], dev["sin"][None, None], dev["pq"], dev["pc"],
                            dev["pd"], 8, 2, 128)
    with pytest.raises(ValueError, match="query width"):
        dspark_qk_norm_rope(dev["query"], dev["ctx"], dev["drf"], dev["wq"], dev["wk"], EPS,
                            dev["cos"][None, None], dev["sin"][None, None], dev["pq"], dev["pc"], dev["pd"],
                            4, 2, 128)
