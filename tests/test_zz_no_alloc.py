"""aspec_qk_norm_rope_bwd_noalloc (the workspace-free Q/K norm + RoPE backward, its scratch a static
device array) against aspec_qk_norm_rope_bwd with a caller-allocated workspace, through the C ABI:
two calls in a row, the second with a smaller input, every output bitwise equal (the same
deterministic kernels), for bf16 and fp16 activations. Also: an invalid size is rejected, and the
workspace-free call allocates nothing at either level the process can observe: torch's caching
allocator reserves no more memory, and the device's free memory as HIP reports it
(hipMemGetInfo, through torch.cuda.mem_get_info) is the same before and after the call."""

import ctypes

import pytest
import torch

from aspec_amd import _lib

pytestmark = pytest.mark.gpu

EPS = 1e-6
BF16 = 4  # ASPEC_MASK_BF16
F16 = 5  # ASPEC_MASK_F16
DTYPES = {BF16: torch.bfloat16, F16: torch.float16}


def _case(device, batch, lc, ld, hq, hkv, seed, code=BF16):
    g = torch.Generator().manual_seed(seed)
    bf = DTYPES[code]
    rnd = lambda *s: torch.randn(*s, generator=g).to(bf).to(device)  # noqa: E731
    x = dict(query=rnd(batch * ld, hq, 128), ctx=rnd(batch * lc, hkv, 128), drf=rnd(batch * ld, hkv, 128),
             wq=rnd(128), wk=rnd(128))
    ang = torch.randn(97, 64, generator=g)
    ang = torch.cat((ang, ang), dim=-1)
    x["cos"], x["sin"] = ang.cos().to(bf).to(device), ang.sin().to(bf).to(device)
    for name, n in (("pq", ld), ("pc", lc), ("pd", ld)):
        x[name] = torch.randint(97, (batch, n), generator=g).to(device)
    x["q_out"] = torch.empty(batch * ld, hq, 128, dtype=bf, device=device)
    x["k_out"] = torch.empty(batch * (lc + ld), hkv, 128, dtype=bf, device=device)
    x["rstd_q"] = torch.empty(batch * ld, hq, dtype=torch.float32, device=device)
    x["rstd_k"] = torch.empty(batch * (lc + ld), hkv, dtype=torch.float32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _lib.stream_handle(device)
    _lib.call("aspec_qk_norm_rope_fwd", x["query"].data_ptr(), x["ctx"].data_ptr(), x["drf"].data_ptr(),
              x["wq"].data_ptr(), x["wk"].data_ptr(), x["cos"].data_ptr(), x["sin"].data_ptr(), 97, 128,
              x["pq"].data_ptr(), x["pc"].data_ptr(), x["pd"].data_ptr(), batch, lc, ld, hq, hkv, 128, EPS,
              code, x["q_out"].data_ptr(), x["k_out"].data_ptr(), x["rstd_q"].data_ptr(), x["rstd_k"].data_ptr(),
              flags.data_ptr(), stream)
    x["gq"] = rnd(batch * ld, hq, 128)
    x["gk"] = rnd(batch * (lc + ld), hkv, 128)
    x["sizes"] = (batch, lc, ld, hq, hkv)
    x["code"] = code
    return x


def _outputs(x):
    return [torch.full_like(x["query"], float("nan")), torch.full_like(x["ctx"], float("nan")),
            torch.full_like(x["drf"], float("nan")), torch.full((128,), float("nan"), device=x["wq"].device),
            torch.full((128,), float("nan"), device=x["wq"].device),
            torch.zeros(1, dtype=torch.int32, device=x["wq"].device)]


def _args_head(x):
    batch, lc, ld, hq, hkv = x["sizes"]
    return (x["gq"].data_ptr(), x["gk"].data_ptr(), x["query"].data_ptr(), x["ctx"].data_ptr(),
            x["drf"].data_ptr(), x["rstd_q"].data_ptr(), x["rstd_k"].data_ptr(), x["wq"].data_ptr(),
            x["wk"].data_ptr(), x["cos"].data_ptr(), x["sin"].data_ptr(), 97, 128, x["pq"].data_ptr(),
            x["pc"].data_ptr(), x["pd"].data_ptr(), batch, lc, ld, hq, hkv, 128, EPS, x["code"])


def _with_workspace(x):
    out = _outputs(x)
    batch, lc, ld, hq, hkv = x["sizes"]
    size = ctypes.c_size_t()
    _lib.call("aspec_qk_norm_rope_bwd_workspace_bytes", batch, lc, ld, hq, hkv, ctypes.byref(size))
    ws = torch.empty(size.value, dtype=torch.uint8, device=x["wq"].device)
    _lib.call("aspec_qk_norm_rope_bwd", *_args_head(x), *(t.data_ptr() for t in out[:5]), ws.data_ptr(),
              out[5].data_ptr(), _lib.stream_handle(x["wq"].device))
    torch.cuda.synchronize()
    return out


def _without_workspace(x):
    out = _outputs(x)
    torch.cuda.synchronize()
    reserved = torch.cuda.memory_reserved()
    free = torch.cuda.mem_get_info()[0]
    _lib.call("aspec_qk_norm_rope_bwd_noalloc", *_args_head(x), *(t.data_ptr() for t in out[:5]),
              out[5].data_ptr(), _lib.stream_handle(x["wq"].device))
    torch.cuda.synchronize()
    assert torch.cuda.memory_reserved() == reserved
    assert torch.cuda.mem_get_info()[0] == free
    return out


@pytest.mark.parametrize("code", [BF16, F16])
def test_noalloc_backward_equals_workspace_backward(gpu, code):
    # the first call fills the grid (2048 workgroups: the scratch's full size), the second is
    # smaller, so stale partials of the first call sit beyond the second call's groups
    big = _case(gpu, 2, 2048, 512, 32, 8, seed=1, code=code)
    small = _case(gpu, 1, 40, 24, 4, 2, seed=2, code=code)
    for x in (big, small):
        want = _with_workspace(x)
        got = _without_workspace(x)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        assert int(got[5].item()) == 0
        assert torch.isfinite(got[3]).all() and torch.isfinite(got[4]).all()


def test_noalloc_backward_rejects_invalid_sizes(gpu):
    x = _case(gpu, 1, 8, 4, 4, 2, seed=3)
    out = _outputs(x)
    args = list(_args_head(x))
    args[18] = 0  # draft_len
    with pytest.raises(ValueError, match="positive"):
        _lib.call("aspec_qk_norm_rope_bwd_noalloc", *args, *(t.data_ptr() for t in out[:5]),
                  out[5].data_ptr(), _lib.stream_handle(gpu))
