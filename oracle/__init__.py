"""CPU oracle for the DSpark draft hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (integer metadata) and CPU torch / numpy fp64 (attention and loss
arithmetic), of the reference's algorithms on this path, each function citing the reference
file:line it follows. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker or the timed CPU baseline; the
`aspec_amd` product never imports it and never falls back to it.

How each part is pinned (besides agreeing with the HIP path):
  metadata.py  -- three independent restatements (mask_mod brute force, math `_visibility`,
                  searchsorted endpoints) must agree; hand-derived golden fixtures
                  (tests/golden/thd_small_case.json, dflash_truth_tables.json) from the reference's
                  own test cases; tile classes equal brute-force any/all (the reference's spec).
  attention.py -- reduces to textbook masked softmax attention; pinned by a per-row float64 loop,
                  single-visible-key closed forms and autograd-vs-finite-difference gradients.
  loss.py      -- fp64 closed forms pinned by special values (identical rows -> 0, disjoint
                  one-hots -> 2, uniform CE -> log V) and finite-difference gradients.
  rows.py      -- the reference's own packing / anchor / output-block / target test cases and
                  closed forms.
  qk_norm_rope.py -- RMSNorm and RoPE closed forms: constant rows normalize to +-1, cos=1/sin=0
                  is the identity, cos=0/sin=1 is rotate_half, the rotation keeps each (i, i+D/2)
                  pair's norm, and finite-difference gradients.
  layer.py     -- RMSNorm of constant rows gives +-w and its residual add comes first; RMSNorm and
                  SwiGLU gradients against finite differences; AdamW's closed-form first step,
                  clipping and non-finite skip; the fp64 one-layer forward is differentiable and
                  respects the mask.
  packing.py   -- the reference's own packing test cases with hand-derived placements, brute-force
                  eligible anchor starts, exact-double density ties, and a replay of every
                  placement (best fit, skips, seeds, capacity, rank order) on random pools.
  dspark_head.py -- the Markov logits reduce to h W^T for w2 = 0 and to a w2 column for a one-hot
                  w1 row; argmax against hand-stated indices (ties, NaN, +-inf rows); acceptance
                  statistics against a hand-computed block; BCE at 0 and its gradient; the Markov
                  gradients against finite differences.
"""
