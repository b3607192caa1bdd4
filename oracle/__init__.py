"""Test infrastructure only: the CPU oracle of the HFFN forward path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import, call, link or
run anything under ``oracle/``, and only as the checker (or, for ``x86_ref``, as the timed CPU baseline). The
product path (``hffn_amd``) never imports it and has no CPU fallback.

* ``oracle.reference`` - float64 forward of a compact hidden-major FFN: the slot walk of
  ``runtime/common/ffn/hffn_ffn_layers/reference.py:21-38``, the dense closed form of
  ``runtime/common/pythia/hffn_pythia/oracle.py:17-31``, and a pure-Python loop for tiny cases.
* ``oracle.transpose`` - the output-major transpose of the down store
  (``runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:55-67``): numpy stable argsort, and a pure-Python
  bucket version.
* ``oracle.x86_ref`` - ctypes binding of the reference x86 AVX2 kernel
  (``runtime/cpu/x86/common/kernels/hffn_compact_g4_inference.cpp``), compiled from its source where it lies by
  ``oracle/Makefile`` into ``oracle/_ref/`` (never copied into this repository).
"""
