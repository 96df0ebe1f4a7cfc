"""CPU oracle for the conv-chain upscaler path -- TEST INFRASTRUCTURE ONLY.

Restates the reference's per-op arithmetic on the CPU (plain C in oracle.c,
NumPy glue here) so the HIP engine can be checked against it. Only tests/,
``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may import this
package; the product (``arthip_amd``) never does.

Parity status of every function is recorded in tests/test_oracle.py, which pins
each one against library routines (numpy float16 casts, torch conv2d /
pixel_shuffle / silu), brute force on tiny inputs and closed-form invariants.
"""
