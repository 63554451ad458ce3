"""Host drivers for the dense hot path, over the tm_* C ABI.

These are the reference's own callers restated for the built-in gfx950 kernels:
  - `matmul` follows python/examples/matmul.py:47-63 (grid (cdiv(M,BM), cdiv(N,BN)),
    the 12-argument matmul_kernel list);
  - `AttentionLayer` follows python/examples/attention_training.py:195-247
    (forward writes O and the log2 logsumexp L; backward runs preprocess, dq,
    dkdv with the reference's argument lists and grids);
  - `SAEEncoder` follows Sources/TritonMetalMLX/SAEEncoder.swift:116-160 and
    python/examples/sae_encode.py:73-107 (relu(x @ W_enc + b_enc) in one
    dispatch of sae_encode_kernel, grid (cdiv(M,64), cdiv(F,64))).
Every dispatch is a tm_launch (or tm_launch_async) call into the native library.
"""

import json
import math

import numpy as np

from . import _core
from .buffer import DeviceBuffer

_ELEMENTS = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}

#: Threads per workgroup the reference caller asks for (4 simdgroups of 32).
REFERENCE_THREADS = 128


def cdiv(a, b):
    return (a + b - 1) // b


class BuiltinLibrary:
    """One built-in library spec and its kernels, loaded once.  bwd="atomic"
    adds attn_bwd_fused, the backward in one call that sums dQ with fp32
    atomics (not deterministic)."""

    NAMES = ("matmul_kernel", "attn_fwd", "attn_bwd_preprocess", "attn_bwd_dq", "attn_bwd_dkdv",
             "sae_encode_kernel")

    def __init__(self, element="f32", head_dim=64, causal=False, bwd="split"):
        if element not in _ELEMENTS:
            raise ValueError(f"element must be one of {sorted(_ELEMENTS)}")
        if bwd not in ("split", "atomic"):
            raise ValueError("bwd must be 'split' or 'atomic'")
        self.element = element
        self.dtype = _ELEMENTS[element]
        self.head_dim = head_dim
        self.causal = causal
        self.bwd = bwd
        self.spec = f"builtin element={element} head_dim={head_dim} causal={int(causal)} bwd={bwd}"
        self.info = {k["name"]: k for k in json.loads(_core.kernel_info(self.spec))["kernels"]}
        self.handle = _core.compile_msl(self.spec)
        names = self.NAMES + (("attn_bwd_fused",) if bwd != "split" else ())
        self.kernels = {name: _core.load_kernel(self.handle, name) for name in names}

    def release(self):
        for handle in self.kernels.values():
            _core.release_kernel(handle)
        self.kernels = {}
        if self.handle:
            _core.release_library(self.handle)
            self.handle = 0


_CACHE = {}


def library(element="f32", head_dim=64, causal=False, bwd="split") -> BuiltinLibrary:
    key = (element, head_dim, bool(causal), bwd)
    if key not in _CACHE:
        _CACHE[key] = BuiltinLibrary(element, head_dim, causal, bwd)
    return _CACHE[key]


def _go(kernel, grid, kinds, values, synchronous=True):
    if synchronous:
        _core.launch(kernel, grid, REFERENCE_THREADS, kinds, values)
    else:
        _core.launch_async(kernel, grid, REFERENCE_THREADS, kinds, values)


# --------------------------------------------------------------------------- #
# GEMM
# --------------------------------------------------------------------------- #


def matmul_args(a, b, c, m, n, k, strides=None, block=(64, 64, 32)):
    """(grid, kinds, values) of one matmul_kernel dispatch, in the reference's
    12-argument order (GEMMKernel.swift:42-45).  Default strides: row-major."""
    sam, sak, sbk, sbn, scm, scn = strides or (k, 1, n, 1, n, 1)
    grid = (cdiv(m, block[0]), cdiv(n, block[1]), 1)
    kinds = [_core.ARG_BUFFER] * 3 + [_core.ARG_I32] * 9
    values = [a.tm_handle, b.tm_handle, c.tm_handle, m, n, k, sam, sak, sbk, sbn, scm, scn]
    return grid, kinds, values


def matmul(a: DeviceBuffer, b: DeviceBuffer, c: DeviceBuffer, m, n, k, strides=None,
           element=None, synchronous=True):
    """C = A @ B on the device through matmul_kernel."""
    element = element or {v: k for k, v in _ELEMENTS.items()}[a.dtype]
    lib = library(element)
    grid, kinds, values = matmul_args(a, b, c, m, n, k, strides)
    _go(lib.kernels["matmul_kernel"], grid, kinds, values, synchronous)


def matmul_numpy(a: np.ndarray, b: np.ndarray, element="f32") -> np.ndarray:
    """Convenience: host arrays in, float32 host array out."""
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    dtype = _ELEMENTS[element]
    bufs = [DeviceBuffer.from_numpy(np.asarray(x, np.float32), dtype) for x in (a, b)]
    c = DeviceBuffer((m, n), dtype)
    try:
        matmul(bufs[0], bufs[1], c, m, n, k, element=element)
        return c.float32()
    finally:
        for x in (*bufs, c):
            x.free()


# --------------------------------------------------------------------------- #
# SAE encoder: relu(x @ W_enc + b_enc)
# --------------------------------------------------------------------------- #


class SAEEncoder:
    """The fused sparse-autoencoder encoder `relu(x @ W_enc + b_enc)`, x [M, D],
    W_enc [D, F], b_enc [F], out [M, F], all row-major contiguous.

    Compiled once (the library cache), each call is one sae_encode_kernel
    dispatch, as SAEEncoder.Compiled (SAEEncoder.swift:116-160).  The shape
    checks and their messages are the Swift wrapper's (:127-143); the kernel
    itself checks buffer extents against M, D and F."""

    #: SAEEncoder.Blocking() defaults; the grid below is the reference caller's
    #: (sae_encode.py:36-37, :97-103).
    BLOCK_M = 64
    BLOCK_F = 64

    def __init__(self, element="f32"):
        self.element = element
        self.lib = library(element)
        self.kernel = self.lib.kernels["sae_encode_kernel"]

    @classmethod
    def args(cls, x, w, b, out, rows, model, features):
        """(grid, kinds, values) in the kernel's argument order (x, w, b, out, M, D, F)."""
        grid = (cdiv(rows, cls.BLOCK_M), cdiv(features, cls.BLOCK_F), 1)
        kinds = [_core.ARG_BUFFER] * 4 + [_core.ARG_I32] * 3
        values = [x.tm_handle, w.tm_handle, b.tm_handle, out.tm_handle, rows, model, features]
        return grid, kinds, values

    @staticmethod
    def check_shapes(x_shape, w_shape, b_shape):
        """(rows, model, features), or ValueError with the Swift wrapper's message."""
        x_shape, w_shape, b_shape = tuple(x_shape), tuple(w_shape), tuple(b_shape)
        if len(x_shape) != 2 or len(w_shape) != 2 or len(b_shape) != 1:
            raise ValueError(f"sae_encode expects x [M, D], W_enc [D, F], b_enc [F]; got "
                             f"{list(x_shape)}, {list(w_shape)}, {list(b_shape)}")
        rows, model = x_shape
        features = w_shape[1]
        if w_shape[0] != model:
            raise ValueError(f"x is [{rows}, {model}] and W_enc is {list(w_shape)}; their "
                             "contraction dimensions differ")
        if b_shape[0] != features:
            raise ValueError(f"W_enc has {features} features but b_enc has {b_shape[0]}")
        return rows, model, features

    def __call__(self, x: DeviceBuffer, w: DeviceBuffer, b: DeviceBuffer,
                 out: DeviceBuffer = None, synchronous=True) -> DeviceBuffer:
        rows, model, features = self.check_shapes(x.shape, w.shape, b.shape)
        if out is None:
            out = DeviceBuffer((rows, features), x.dtype)
        elif tuple(out.shape) != (rows, features):
            raise ValueError(f"out is {list(out.shape)}, expected [{rows}, {features}]")
        grid, kinds, values = self.args(x, w, b, out, rows, model, features)
        _go(self.kernel, grid, kinds, values, synchronous)
        return out

    def numpy(self, x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
        """Host arrays in, float32 host array out."""
        self.check_shapes(np.shape(x), np.shape(w), np.shape(b))
        dtype = _ELEMENTS[self.element]
        bufs = [DeviceBuffer.from_numpy(np.asarray(a, np.float32), dtype) for a in (x, w, b)]
        out = None
        try:
            out = self(*bufs)
            return out.float32()
        finally:
            for a in (*bufs, out):
                if a is not None:
                    a.free()


# --------------------------------------------------------------------------- #
# Attention
# --------------------------------------------------------------------------- #


class AttentionLayer:
    """Q, K, V, O, dO, dQ, dK, dV as [heads, seq, dim] device buffers plus the
    per-row L (log2 logsumexp) and Delta, and the four attention kernels.

    `heads` is batch*heads: the reference's layout [B*H, S, D] with
    stride_head = S*D and stride_seq = D (AttentionKernel.swift:25-28).
    bwd="atomic" runs the backward as preprocess + attn_bwd_fused
    instead of preprocess + dq + dkdv.
    """

    #: per-(head, row) tensors: the forward's L (log2 units) and the backward's Delta
    ROW_STATS = ("lse", "delta")
    #: per-(head, row, d) tensors in the element type
    TENSORS = ("q", "k", "v", "o", "do", "dq", "dk", "dv")

    def __init__(self, heads, seq, dim, element="f32", causal=False, scale=None,
                 block_m=16, block_n=32, bwd="split"):
        self.heads, self.seq, self.dim = heads, seq, dim
        self.element, self.causal = element, causal
        # the reference caller's tile sizes only shape the requested grids; the
        # library covers the problem with its own tiles
        self.block_m, self.block_n = block_m, block_n
        self.scale = scale if scale is not None else 1.0 / math.sqrt(dim)
        self.bwd = bwd
        self.lib = library(element, dim, causal, bwd)
        self.buffers = {}
        for name in self.TENSORS:
            self.buffers[name] = DeviceBuffer((heads, seq, dim), _ELEMENTS[element])
        for name in self.ROW_STATS:
            self.buffers[name] = DeviceBuffer((heads, seq), "float32")

    def free(self):
        """Release every buffer (the library stays cached for other layers)."""
        while self.buffers:
            _, buffer = self.buffers.popitem()
            buffer.free()

    def upload(self, name, array):
        self.buffers[name].write(np.asarray(array, dtype=np.float32)
                                 if self.element != "f32" else array)

    def read(self, name) -> np.ndarray:
        return self.buffers[name].float32()

    # -- dispatch descriptions (reference argument lists) ------------------

    def _h(self, name):
        return self.buffers[name].tm_handle

    def fwd_args(self, stats=True):
        B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
        grid = (cdiv(self.seq, self.block_m), self.heads, 1)
        kinds = [B, B, B, B, F, I, I, I]
        values = [self._h("q"), self._h("k"), self._h("v"), self._h("o"),
                  _core.float_bits(self.scale), self.seq * self.dim, self.dim, self.seq]
        if stats:
            kinds += [B, I]
            values += [self._h("lse"), self.seq]
        return grid, kinds, values

    def pre_args(self):
        B, I = _core.ARG_BUFFER, _core.ARG_I32
        grid = (cdiv(self.seq, self.block_m), self.heads, 1)
        kinds = [B, B, B, I, I, I, I]
        values = [self._h("o"), self._h("do"), self._h("delta"),
                  self.seq * self.dim, self.dim, self.seq, self.seq]
        return grid, kinds, values

    def dq_args(self):
        B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
        grid = (cdiv(self.seq, self.block_m), self.heads, 1)
        kinds = [B] * 7 + [F, I, I, I, I]
        values = [self._h(x) for x in ("q", "k", "v", "do", "dq", "lse", "delta")] + [
            _core.float_bits(self.scale), self.seq * self.dim, self.dim, self.seq, self.seq]
        return grid, kinds, values

    def dkdv_args(self):
        B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
        grid = (cdiv(self.seq, self.block_n), self.heads, 1)
        kinds = [B] * 8 + [F, I, I, I, I]
        values = [self._h(x) for x in ("q", "k", "v", "do", "dk", "dv", "lse", "delta")] + [
            _core.float_bits(self.scale), self.seq * self.dim, self.dim, self.seq, self.seq]
        return grid, kinds, values

    def fused_args(self):
        B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
        grid = (cdiv(self.seq, self.block_n), self.heads, 1)
        kinds = [B] * 9 + [F, I, I, I, I]
        values = [self._h(x) for x in ("q", "k", "v", "do", "dq", "dk", "dv", "lse", "delta")] + [
            _core.float_bits(self.scale), self.seq * self.dim, self.dim, self.seq, self.seq]
        return grid, kinds, values

    # -- passes --------------------------------------------------------------

    def run_forward(self, synchronous=True, stats=True):
        _go(self.lib.kernels["attn_fwd"], *self.fwd_args(stats), synchronous=synchronous)

    def run_backward(self, synchronous=True):
        k = self.lib.kernels
        _go(k["attn_bwd_preprocess"], *self.pre_args(), synchronous=False)
        if self.bwd != "split":
            _go(k["attn_bwd_fused"], *self.fused_args(), synchronous=synchronous)
            return
        _go(k["attn_bwd_dq"], *self.dq_args(), synchronous=False)
        _go(k["attn_bwd_dkdv"], *self.dkdv_args(), synchronous=synchronous)

    def forward(self, q, k, v):
        """Upload, run, return (O, L) as float32 host arrays."""
        self.upload("q", q)
        self.upload("k", k)
        self.upload("v", v)
        self.run_forward()
        return self.read("o"), self.read("lse")

    def backward(self, d_out):
        """Upload dO, run the three backward kernels, return (dQ, dK, dV)."""
        self.upload("do", d_out)
        self.run_backward()
        return self.read("dq"), self.read("dk"), self.read("dv")
