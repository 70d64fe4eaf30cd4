"""CPU oracle for the paged-attention decode path — TEST INFRASTRUCTURE ONLY.

A CPU restatement of the reference algorithms (VRAMancer's PyTorch paths),
used as the checker for the gfx950 kernels.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product (``vramancer_amd``) never calls it and has no CPU
fallback.

Modules and what pins each of them (beyond following the reference's code):
  paged_decode  restates core/paged_attention_cuda.py:187-231 and :291-348;
                pinned by an fp64 closed-form attention (``dense_attention``)
                and the reference test cases (zero / single-token context).
  kv_codecs     the int8 and fp8-e4m3 codecs this build defines (the
                reference has none); pinned by round-trip bounds, the exact
                scale/extreme-code identities and torch's float8_e4m3fn cast.
  turboquant    restates core/kv_quantizer.py:46-105, 217-572 (CPU path);
                pinned by golden vectors written from the reference itself
                (tests/golden/), the Sylvester Hadamard matrix, rotation
                invariants, tiny-dimension brute force and bit-order cases.
Nothing here is "parity unpinned"; see tests/test_oracle_pins.py.
"""
