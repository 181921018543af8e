"""CPU oracle for the fused-time spiking-neuron path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker or
as the timed CPU baseline.

Two independent restatements of myelin's ``torch`` backend live here:

* ``oracle.torch_ref`` restates the reference's PyTorch code paths op by op
  (same ATen ops, same evaluation order) so that forward results are
  bit-identical to what myelin's ``torch`` backend computes on the CPU and
  gradients come from ``torch.autograd`` exactly as in the reference.
* ``oracle/c/oracle.c`` restates the same recurrences and the packing
  arithmetic in plain C (``-ffp-contract=off``), with the surrogate backward
  written as a closed-form adjoint.  ``oracle.c_ref`` loads it with ctypes.

Pinning (what checks each function against something other than itself) is
listed per function in ``oracle.torch_ref``'s module docstring.
"""
