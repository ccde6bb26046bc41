"""ctypes loader of oracle/cref.c (test infrastructure, see its header).

``build()`` compiles it with gcc into oracle/_cref.so; the library travels
with the tree, so GPU hosts load the prebuilt file.  When it is missing, the
numpy restatement in oracle/ref.py gives the same results, only slower.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cref.c")
LIB = os.path.join(HERE, "_cref.so")
_lib = None


def build() -> str:
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-shared", "-fPIC",
           SRC, "-o", LIB + ".tmp"]
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


def load():
    global _lib
    if _lib is None and os.path.exists(LIB):
        lib = ctypes.CDLL(LIB)
        lib.vq_assign_direct.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        lib.vq_assign_direct.restype = None
        _lib = lib
    return _lib


def vq_assign_direct(x, c):
    """oracle.ref.vq_assign_direct in C; x (n, d), c (k, d) -> int64 (n,)."""
    lib = load()
    if lib is None:
        from . import ref
        return ref.vq_assign_direct(x, c)
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    c = np.ascontiguousarray(np.asarray(c, np.float32))
    out = np.empty(x.shape[0], np.int64)
    lib.vq_assign_direct(x.ctypes.data, x.shape[0], x.shape[1], c.ctypes.data, c.shape[0],
                         out.ctypes.data)
    return out


def vq_assign_direct_t(x, c):
    """vq_assign_direct on CPU torch tensors, returning an int64 tensor (the
    ``assign`` rule for oracle.ref.kmeans / compress_layer)."""
    import torch
    return torch.from_numpy(vq_assign_direct(x.numpy(), c.numpy()))
