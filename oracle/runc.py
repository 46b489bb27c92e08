"""ctypes binding of the reference's run.c built under oracle/_ref (ORACLE side).

``oracle/Makefile`` compiles the unmodified run.c from the reference checkout
into ``_ref/librunc_ref.so``. That file travels with the tree, so tests can use
it where the reference checkout is absent. ``available()`` is False when it
was never built.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_ref", "librunc_ref.so")
LIB_OMP = os.path.join(HERE, "_ref", "librunc_ref_omp.so")   # the reference's runomp flags
REFERENCE = "/root/reference"


def build():
    """Compile run.c when the reference checkout is present (a no-op otherwise)."""
    if os.path.exists(os.path.join(REFERENCE, "run.c")):
        subprocess.run(["make", "-s", "-C", HERE, f"REF={REFERENCE}"], check=True)


def available(omp=False):
    return os.path.exists(LIB_OMP if omp else LIB)


class RuncReference:
    """The reference decoder: load(path), reset(), forward(token) -> logits.
    omp=True loads the OpenMP build (its threads from OMP_NUM_THREADS)."""

    def __init__(self, checkpoint, omp=False):
        self._lib = ctypes.CDLL(LIB_OMP if omp else LIB)
        self._lib.runc_ref_load.argtypes = [ctypes.c_char_p]
        self._lib.runc_ref_forward.argtypes = [ctypes.c_int]
        self._lib.runc_ref_forward.restype = ctypes.POINTER(ctypes.c_float)
        self._lib.runc_ref_load(checkpoint.encode())
        self.vocab = self._lib.runc_ref_vocab()

    def reset(self):
        self._lib.runc_ref_reset()

    def forward(self, token):
        ptr = self._lib.runc_ref_forward(int(token))
        return np.ctypeslib.as_array(ptr, shape=(self.vocab,)).copy()

    def logits(self, tokens):
        """Logits for each position of one token sequence, from a reset state."""
        self.reset()
        return np.stack([self.forward(t) for t in tokens])
