"""Shared drivers for the attention GPU tests: reference-ordered dispatches
through the tm_* ABI (attention_training.py:195-247)."""

import math

import numpy as np

from oracle import generators as G
from triton_metal import _core
from triton_metal.buffer import round_to
from triton_metal.ops import AttentionLayer

DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def inputs(heads, seq, dim, element="f32", spread=1.0, seeds=(1, 5, 9, 13)):
    """The reference's tensor() inputs, rounded to the element type."""
    count = heads * seq * dim
    return [round_to(G.tensor(count, s, spread).reshape(heads, seq, dim), element)
            for s in seeds]


def normal_inputs(heads, seq, dim, element, seed=0, scale=1.0, count=4):
    rng = np.random.default_rng(seed)
    return [round_to(rng.standard_normal((heads, seq, dim), dtype=np.float32) * np.float32(scale),
                     element) for _ in range(count)]


class Runner:
    def __init__(self, heads, seq, dim, element="f32", causal=False, scale=None, threads=128):
        self.layer = AttentionLayer(heads, seq, dim, element, causal, scale)
        self.threads = threads
        self.element = element

    @property
    def scale(self):
        return self.layer.scale

    def _go(self, name, args):
        grid, kinds, values = args
        kernel = self.layer.lib.kernels[name]
        _core.launch(kernel, grid, self.threads, kinds, values)
        return _core.kernel_variant(kernel)

    def forward(self, q, k, v, stats=True):
        for name, x in (("q", q), ("k", k), ("v", v)):
            self.layer.upload(name, x)
        self.variant = self._go("attn_fwd", self.layer.fwd_args(stats))
        return self.layer.read("o"), self.layer.read("lse")

    def backward(self, q, k, v, o, lse, d_out):
        """Backward from given O and L (the reference test feeds the oracle's)."""
        for name, x in (("q", q), ("k", k), ("v", v), ("o", o), ("do", d_out)):
            self.layer.upload(name, x)
        self.layer.buffers["lse"].write(np.asarray(lse, np.float32))
        return self.backward_resident()

    def backward_resident(self):
        self.variants = [self._go("attn_bwd_preprocess", self.layer.pre_args()),
                         self._go("attn_bwd_dq", self.layer.dq_args()),
                         self._go("attn_bwd_dkdv", self.layer.dkdv_args())]
        return (self.layer.read("delta"), self.layer.read("dq"), self.layer.read("dk"),
                self.layer.read("dv"))

    def free(self):
        self.layer.free()
