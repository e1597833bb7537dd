"""CPU oracle for the selective-scan inference path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's (createcentury/mamba-metal) sequential
semantics on the CPU.  It is the parity checker for the HIP product path and the
CPU baseline in ``bench.py``.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it; the product package
``mamba_metal_amd`` never does and fails loudly if its HIP library is missing.

Contents:
  cscan.py      ctypes binding of the C restatement ``scan_ref.c`` (fp32 / fp64)
  numpy_ref.py  numpy restatement of the scan, pair scan, conv1d and decode step
  model_ref.py  torch-CPU restatement of MambaBlock / MambaModel prefill + step
  build.py      gcc build of ``liboracle_scan.so``

Pinning status of every function is recorded in each module's docstring.
"""
