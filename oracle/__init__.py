"""The oracle: a CPU restatement of the reference's BD3LM / Dream denoise step.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``diffusorrt_amd``)
imports, links or runs anything under ``oracle/``. The only callers are the
tests under ``tests/``, ``__graft_entry__.smoke()`` (as the checker of one small
GPU invocation) and the ``cpu_baseline`` leg of ``bench.py``.

Every function cites the reference file:line it restates (paths relative to the
reference's ``python/src/edllm/``). The reference's MLX code cannot run here
(no ``mlx``, Python 3.10 < 3.11), so each function is pinned instead by known
answers, closed forms and invariants in ``tests/test_oracle_*.py``; the
temperature sampler (whose key chaining only the reference's code fixes) by
vectors that the reference's own sampler wrote (``tests/golden/
sampling_vectors.json``, ``tests/test_sampling_vectors.py``). MLX's own
last-bit behaviour (quantized_matmul accumulation order, fused SDPA, bf16
matmul rounding) is parity unpinned: no reference test or golden logits ship.

Modules:
  ops      -- per-op math: RMSNorm, RoPE tables + split-half RoPE, SwiGLU,
              q4 g64 affine unpack/dequant (MLX packing), linear (bf16 / q4 /
              fp32 choreography), d2f_hybrid mask, GQA SDPA, float64 max-prob
              scoring, argsort top-k, splitmix64 sampling noise.
  forward  -- the full-context transformer forward (every visible row is
              recomputed each step, exactly as the reference does).
  policy   -- MaskState / BlockLayout / BD3 fixed-quota / fixed-quota commit
              policies and the decode loop, restated as plain loops.
"""
