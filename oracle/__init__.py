"""CPU oracle for the Gated DeltaNet decode and prefill operators.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import anything from this package, and
only as the checker (or the timed CPU baseline), never as the product path.
The product path (``gdn_amd``) never imports it and fails loudly when the HIP
library is missing.
"""
