"""ctypes loader for the C fp64 oracle (attn_ref.c).  TEST INFRASTRUCTURE ONLY."""

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    if not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "attn_ref.c").stat().st_mtime:
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
    i = ctypes.c_int
    lib.oracle_gemm.argtypes = [f32p, f32p, f64p, i, i, i, i, i, i, i]
    lib.oracle_gemm.restype = None
    lib.oracle_attention.argtypes = [f32p, f32p, f32p, f32p, i, i, i, ctypes.c_double, i,
                                     f64p, f64p, f64p, f64p, f64p, f64p, f64p]
    lib.oracle_attention.restype = ctypes.c_int
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def gemm(a, b, m, n, k, sam, sak, sbk, sbn):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    c = np.zeros(m * n, np.float64)
    lib().oracle_gemm(a, b, c, m, n, k, sam, sak, sbk, sbn)
    return c.reshape(m, n)


def attention(q, k, v, d_out, scale, causal=False):
    q, k, v, d_out = (np.ascontiguousarray(x, np.float32) for x in (q, k, v, d_out))
    heads, seq, dim = q.shape
    out = {name: np.zeros(q.shape, np.float64) for name in ("o", "dq", "dk", "dv")}
    lse = np.zeros((heads, seq), np.float64)
    delta = np.zeros((heads, seq), np.float64)
    amp = np.zeros(3, np.float64)
    status = lib().oracle_attention(q, k, v, d_out, heads, seq, dim, float(scale), int(causal),
                                    out["o"], lse, delta, out["dq"], out["dk"], out["dv"], amp)
    if status != 0:
        raise MemoryError("oracle_attention could not allocate")
    out.update(lse=lse, delta=delta,
               amplification={"dq": amp[0], "dk": amp[1], "dv": amp[2]})
    return out
