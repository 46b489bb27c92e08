"""CPU oracle for the UnifiedLM fast-memory path (test infrastructure).

This package checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The HIP library under ``unifiedlm.c_amd/`` never calls into it.

Modules
-------
fastmem   float64 torch restatement of the reference's pure-PyTorch forms
          (test_all.py:28-75, model.py:26-111, 149-175).
runc      ctypes binding of ``_ref/librunc_ref.so``, which is the reference's
          own ``run.c`` compiled unchanged from its source (see Makefile).
ulme      writer for the ULMe v1 fp32 checkpoint that run.c reads
          (export.py:4-12, 37-82), used to feed the same weights to run.c.
"""
