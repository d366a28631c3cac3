"""CPU oracle of the BS-RoFormer transformer stack - TEST INFRASTRUCTURE ONLY.

This package restates, in plain fp32/fp64 PyTorch on the CPU, what LoggeL/turbo-roformer computes on
the hot path, so that the gfx950 kernels can be checked against it.  It is the checker, never the
thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product (``turbo-roformer_amd/``) never imports it and has no CPU
fallback routed through it.

Modules
    reference  fp32 restatement of the reference module forward (src/turbo_roformer/model.py:28-278)
    folded     the restructured forward with folded norms (src/turbo_roformer/fast.py:163-266, 349-360)
    kernels    bf16-rounding emulations of the reference's fused ops (src/turbo_roformer/csrc/kernels.cpp)
    cpu_stack  the AVX512-BF16 CPU stack (cpu_stack.cpp, built by the Makefile here): the same-host
               kernel-class CPU baseline of bench.py, after the reference's published CPU kernel design
               (docs/how-it-works.md:120-151)

How each function is pinned (tests/test_oracle.py): closed forms and invariants (L2 norm, rotary as a
complex rotation, softmax rows summing to one), textbook/library routines (SDPA in fp64, ``math.erf``),
brute force on tiny inputs, folded vs unfolded agreement (>= 100 dB), axial permutation checks, the
reference's own known-answer tests (chunk schedule, Hamming window, state-dict keys, parameter count,
output length) and golden vectors written by the reference module itself (tests/golden/).  cpu_stack is
checked against folded.stack (tests/test_cpu_stack.py).
"""
