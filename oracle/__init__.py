"""CPU oracle for DiskMule's quantized-matrix path.

TEST INFRASTRUCTURE ONLY.  ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, as the checker
or the timed CPU baseline.  The product (``diskmule_amd``) never imports it
and never falls back to it.

Two independent restatements live here:

* ``dm_oracle.c`` (loaded through :mod:`oracle.capi`): the C restatement of
  ``src/cpu.rs`` that follows the reference's operation order bit for bit.
* :mod:`oracle.numpy_ref`: a vectorised numpy restatement of the block
  decoders that follows the indexing of ``metal/kernels.metal:377-484``
  instead, used to cross-check the C decoders.
"""
