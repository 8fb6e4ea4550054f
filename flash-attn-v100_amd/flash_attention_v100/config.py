"""Debug switches of the attention path (reference ``config.py:267-285``).

Only the two switches that act on this path are kept; the reference's tile
tables, autotuning and multi-GPU settings are replaced by the gfx950 kernels'
static configuration.  Both are off by default, and then cost nothing: no
tensor is read and the host never waits for the GPU.

* ``VALIDATE_OUTPUTS``: the autograd function checks its inputs (q, k, v, the
  bias), its outputs (O, LSE), the incoming gradient and the gradients it
  returns for NaN / Inf (reference ``ops/attention.py:163-168, 203-206,
  271-272, 304-310``), raising ``ValueError`` naming the tensor.  LSE is
  allowed ``-inf``: it is the defined value of a row with no visible key.
* ``CHECK_NUMERICAL_STABILITY``: ``validate_inputs_enhanced`` also scans q, k,
  v and the bias for NaN / Inf (``ValueError``) and warns about extreme
  magnitudes (reference ``utils.py:219-254``, which scans unconditionally; here
  the scan is opt-in because each scan is a host synchronisation).

Each check reads the tensor once on the GPU and synchronises once.
"""


class DebugConfig:
    VALIDATE_OUTPUTS = False
    CHECK_NUMERICAL_STABILITY = False
