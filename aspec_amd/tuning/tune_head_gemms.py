"""Writes the PyTorch TunableOp solution file for the selective-head GEMMs of the config-2 draft
step on gfx950 (run on the GPU box; the file travels with the tree).

The three products are plain library GEMMs (hipBLASLt / rocBLAS), bf16 in, fp32 accumulate:
  draft logits   [8192, 4096] x W^T            (W = frozen head [32000, 4096])
  teacher table  [4096, 4096] x W^T
  head dgrad     [8192, 32000] x W             (computed on W^T stored contiguous: TN layout)
With --layer-step, two config-5 one-layer training steps (aspec_amd.draft_layer) also run under
tuning, so the file records every GEMM of that step as well: the projections, the SwiGLU MLP and
the head, forward and backward.
TunableOp times every hipBLASLt and rocBLAS solution for each shape and records the fastest; with
tuning off and this file loaded, later processes reuse the choice. The file carries validators
(PyTorch, HIP, hipBLASLt, rocBLAS versions and the GPU arch); on a mismatch TunableOp ignores it
and the library defaults run.

    python -m aspec_amd.tuning.tune_head_gemms [--out PATH] [--layer-step] [--duration-ms N]
        [--iterations N] [--rotating-mb MB]
"""

from __future__ import annotations

import argparse
from pathlib import Path

DEFAULT_FILE = Path(__file__).resolve().parent / "head_gemms_gfx950.csv"


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--out", default=str(DEFAULT_FILE))
    p.add_argument("--rows", type=int, default=8192)
    p.add_argument("--context", type=int, default=4096)
    p.add_argument("--hidden", type=int, default=4096)
    p.add_argument("--vocab", type=int, default=32000)
    p.add_argument("--layer-step", action="store_true", help="also tune the config-5 layer step's GEMMs")
    p.add_argument("--duration-ms", type=int, default=30, help="timing budget per candidate solution")
    p.add_argument("--iterations", type=int, default=30, help="timed runs per candidate solution")
    p.add_argument("--rotating-mb", type=int, default=0,
                   help="rotate the operands through this many MB so candidates are timed on cold caches")
    args = p.parse_args()
    import torch

    out = Path(args.out)
    if out.exists():
        out.unlink()
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_filename(str(out))
    torch.cuda.tunable.set_max_tuning_duration(args.duration_ms)
    torch.cuda.tunable.set_max_tuning_iterations(args.iterations)
    if args.rotating_mb:
        torch.cuda.tunable.set_rotating_buffer_size(args.rotating_mb)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(args.rows, args.hidden, device=dev, dtype=torch.bfloat16, generator=g)
    th = torch.randn(args.context, args.hidden, device=dev, dtype=torch.bfloat16, generator=g)
    w = torch.randn(args.vocab, args.hidden, device=dev, dtype=torch.bfloat16, generator=g) * 0.02
    wt = w.t().contiguous()
    gr = torch.randn(args.rows, args.vocab, device=dev, dtype=torch.bfloat16, generator=g)
    for _ in range(2):
        torch.matmul(h, w.t())
        torch.matmul(th, w.t())
        torch.matmul(gr, wt.t())
    torch.cuda.synchronize()
    print("tuned the head GEMMs", flush=True)
    if args.layer_step:
        from aspec_amd import workloads as W
        from aspec_amd.draft_layer import (DSparkDraftLayerModel, FusedBF16Optimizer, dspark_layer_step,
                                           layer_batch)

        del h, th, w, wt, gr
        model = DSparkDraftLayerModel(device=dev)
        opt = FusedBF16Optimizer(model, lr=1e-4, total_steps=1000, warmup_ratio=0.0)
        batch = layer_batch(model, W.config5(), seed=0)
        for i in range(2):
            dspark_layer_step(model, opt, batch)
            torch.cuda.synchronize()
            print(f"tuned config-5 layer step {i + 1}", flush=True)
    print(f"solutions -> {out} (written at exit)", flush=True)


if __name__ == "__main__":
    main()
