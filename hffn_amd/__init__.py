"""MI355X-native HFFN inference runtime: hand-written HIP kernels for gfx950 behind the reference's Python API.

* ``hffn_amd.runtime``  - ``HFFNLayer``, ``HFFNRuntime``, ``up_mode``/``down_mode`` (as ``hffn_cuda.runtime``)
* ``hffn_amd.parity``   - forced-pair parity check (as ``hffn_cuda.parity``)
* ``hffn_amd.ffn``      - ``cuda_layer``/``hip_layer`` for compact test layers (as ``hffn_ffn_cuda``)
* ``hffn_amd.synth``    - the seeded compact layers and inputs (test layers of the reference, workload layers)
* ``hffn_amd.pythia``   - the Pythia two-arm loader and ``HFFNMLP`` hook (as ``hffn_pythia_cuda``)
"""
