"""CPU oracle for the INT8 decode-attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (float32 arithmetic, one rounding per torch op),
the reference's PyTorch algorithm for the path the HIP kernels replace:

* ``oracle.quant``     affine per-block INT8 quantize / dequantize
                        (reference src/flashspec/quant.py:94-204)
* ``oracle.attention`` dense decode attention and the portable ``fused`` /
                        ``paged`` paths (reference src/flashspec/attention.py:70-223)
* ``oracle.paged``     paged-cache layouts, ``to_dense``, whole-store ``append``
                        and the allocator's per-page append
                        (reference src/flashspec/paged.py:17-557)

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker (or the timed CPU baseline),
never as part of the product path.  The ``flashspec_amd`` package must not
import it.

How each function is pinned (so that a plausible slip fails a check):

* quantize/dequantize: golden vectors written by the reference itself
  (tests/golden/), closed forms (constant block -> scale 1e-8; all-zero block
  -> int8 -128 that round-trips to 0; extremes map to 0/255), and a brute-force
  nearest-integer check of every code.
* reference_attention: float64 brute-force loops on tiny shapes, one-token and
  equal-key closed forms, mask == truncation.
* from_dense layouts: interleaved layout closed form; shuffled layout against
  the reference's golden tables.
* append / allocator append: golden vectors written by the reference itself.

No function here is "parity unpinned".
"""

from . import attention, paged, quant  # noqa: F401
