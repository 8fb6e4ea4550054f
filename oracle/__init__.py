"""CPU oracle for the FlashAttention forward/backward hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``flash-attn-v100_amd/``)
imports, links or calls anything in this directory.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker / the timed CPU baseline, never as the computation that
is measured or shipped.

Contents
--------
``attention``  restatement of the reference's math path
               (``tests/test_attention.py:39-79``, ``__init__.py:34-55`` of
               mini-kio/flash-attn-v100) in torch on the CPU, fp32 or fp64:
               forward O, true natural-log LSE, the backward by the explicit
               formulas and by autograd.
``philox``     numpy restatement of Philox4x32-10 (Salmon et al., SC'11,
               "Parallel random numbers: as easy as 1, 2, 3") and of Triton's
               ``tl.rand`` uint32 -> fp32 mapping (triton/language/random.py),
               i.e. the RNG behind the reference's dropout
               (``kernels/forward_kernel.py:198-203``).
``philox_ref.c`` the same Philox/dropout-mask restatement in C (fast path for
               full-size bit-exact mask checks); built by ``oracle/Makefile``
               into ``oracle/_build/liboracle.so``.

Each function is pinned by tests in ``tests/test_oracle.py`` (Random123
known-answer vectors, Triton-interpreter vectors committed under
``tests/golden/``, brute force on tiny shapes, closed forms and invariants).
"""
