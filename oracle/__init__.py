"""CPU oracle for the UniCache physical KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``unicache_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg use it, as the checker (never as the thing measured or shipped).

It restates, in numpy, the arithmetic of the reference files cited in each
function (paths relative to the UniCache repository):

- ``oracle.kivi``: KIVI group quantization, LSB-first int32 packing,
  dequantization, the kernel-native layout and fake quantization
  (unicache/storage/physical.py, unicache/storage/kivi_cuda.py,
  unicache/operators/builtin.py).
- ``oracle.attention``: GQA logits / probability-value products, softmax
  summaries with natural-log LSE and the LSE merge
  (unicache/storage/physical.py, unicache/storage/kivi_triton.py,
  unicache/adapters/bagel.py).
- ``oracle.h2o``: per-KV-head H2O scores, budget arithmetic, deterministic
  top-k selection (lowest index wins ties) and the GQA gather
  (unicache/operators/physical.py, unicache/storage/physical.py,
  unicache/storage/tensor_backend.py).

How each function is pinned (golden vectors, known answers, invariants) is
listed next to its tests in tests/test_oracle_*.py.  Parity status: every
function here has at least one known-answer or invariant check; none is
"parity unpinned".
"""
