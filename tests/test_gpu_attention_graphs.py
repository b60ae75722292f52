"""HIP-graph capture of the DSpark attention, as bench.py's kernel-bench contract times it
(`AttentionRunner.capture`): forward, backward and forward + backward each captured once through
`direct_cp_attention_from_kv`, with dQ's second stream forked and joined inside the capture.

Every replay must equal the eager result bit for bit (the kernels are deterministic): three rounds
of replays with eager calls and host synchronisations between them, the last after the inputs and
the upstream gradient change in place, so a replay that reused stale results, or a captured node
that only acts on the first replay (a memset node, say), fails. Eager forward and backward calls
on the default stream come first, as in the bench: the capture must not depend on the stream
those earlier autograd graphs were built on.
"""

import pytest
import torch

import bench
from aspec_amd import workloads as W

pytestmark = pytest.mark.gpu


def _check(name, got, want):
    for index, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"{name} output {index} differs from the eager result"


@pytest.mark.parametrize("overlap", [True, False])
def test_attention_graph_replays_equal_eager_results(gpu, overlap):
    from aspec_amd.direct_cp import backward_overlap, set_backward_overlap

    saved = backward_overlap()
    set_backward_overlap(overlap)
    try:
        w = W.config1(0)
        run = bench.AttentionRunner(w, gpu, seed=7)
        # eager calls on the default stream first, as the bench makes them before it captures
        for _ in range(2):
            run.combined()
        run.prepare_backward()
        run.backward()
        torch.cuda.synchronize()
        graphs = run.capture()
        g = torch.Generator(device=gpu).manual_seed(8)
        for trial in range(3):
            if trial == 2:
                # through .data, so the version counters stay put: the eager backward of the
                # captured forward then accepts the new values, as the graph's replay reads them
                for x in (run.q, run.k, run.v, run.dout):
                    x.data.copy_(torch.randn(x.shape, device=gpu, generator=g).to(x.dtype))
            for graph, _ in graphs.values():
                graph.replay()
            torch.cuda.synchronize()
            got = {"fwd": [graphs["fwd"][1].clone()], "bwd": [t.clone() for t in graphs["bwd"][1]],
                   "fb": [t.clone() for t in graphs["fb"][1]]}
            want = {"fwd": [run.forward().detach()], "bwd": list(run.backward()), "fb": list(run.combined())}
            torch.cuda.synchronize()
            print(f"overlap={overlap} trial {trial}: fwd max |O| {want['fwd'][0].abs().max().item():.3f}",
                  flush=True)
            for phase in ("fwd", "bwd", "fb"):
                _check(f"{phase} replay {trial}", got[phase], want[phase])
            assert torch.isfinite(got["fb"][0]).all()
        del graphs
    finally:
        set_backward_overlap(saved)
