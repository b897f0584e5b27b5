"""CPU oracle for the fused tile-local Strassen GEMM path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports, calls or
links this package. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or, for
the CPU baseline, as the timed CPU restatement) -- never as a fallback for the
GPU path.

``oracle.strassen_ref`` restates, in numpy, the arithmetic of the reference's
``strassen_pallas.py`` (kernel ``:156-879``, wrapper ``:882-1221``, relayouts
``:1315-1411``), the matched blocked-cubic control
(``experiments/qwen3/benchmark_cubic_control.py:76-113``), the measurement
helpers of ``experiments/qwen3/benchmark_common.py:17-91`` and the unfused
Qwen3 semantics of ``experiments/qwen3/benchmark_qwen3_32b_layer.py:258-341``.

Pinning (what checks each function, so a plausible mistake fails a test):

* ``bf16_round`` -- against torch's own float32->bfloat16 conversion on
  random, tie, overflow and special values; closed-form ties-to-even cases.
* ``strassen_matmul`` / ``cubic_blocked_matmul`` algebra (quadrant map,
  signs, K-panel accumulation, product order bookkeeping) -- exact-integer
  known-answer tests (result must equal ``A @ B`` bit-exactly), the technique
  of the reference's ``Strassen_MM_Focus/tests/test_kernels_v001.py:59-80``.
* bf16 operand-sum rounding and output rounding -- the reference's published
  accuracy-gate errors on regenerated inputs (``default_rng(20260833)``,
  shape (2048, 14336, 2048), tile (2048, 2048, 512):
  Strassen l2_relative 4.6988e-3, cubic 1.6595e-3,
  ``archive/initial-snapshot/evidence/strassen_cubic_control.jsonl:7``);
  a bounded-nonzero rounding test (``test_kernels_v001.py:82-96``).
* epilogues -- closed forms (``silu(g)*u``, ``acc+r``, ``acc+bias``) and, for
  ``qk_norm_rope``, the unfused RMSNorm+RoPE semantics composed with the
  relayout inverse (``benchmark_qwen3_32b_layer.py:270-284``, ``:322-341``).
* relayouts -- brute-force index maps on tiny sizes and round trips.
* ``packed_operand`` (the packed kernel's operand layout, no reference
  counterpart) -- a per-element index walk over every packed position on
  small shapes, and the cubic round trip (unpacked quadrants reassemble the
  input exactly); the operand sums it stores are the ones the known-answer
  tests above pin.

Parity at the rounding level of XLA/Mosaic internals (dot accumulation order,
``jax.nn.silu``/``rsqrt`` ulps) cannot be pinned without JAX, which is absent
here; those are bounded statistically by the gates above.
"""

from .strassen_ref import *  # noqa: F401,F403
