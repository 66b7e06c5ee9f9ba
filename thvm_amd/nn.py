"""thvm_amd.nn -- the layers the decode drivers use (reference py/thvm/nn.py:
Linear, LayerNorm, Embedding, RMSNorm :211-224), over thvm_amd.tensor.

Weights are initialised on the host from a seeded numpy generator and
uploaded once; ``Linear`` keeps tinygrad's [out_features, in_features]
layout, which is the row-major [N, K] weight the gfx950 GEMV streams."""
from __future__ import annotations

import math
import sys
from typing import Optional

import numpy as np

from thvm_amd import state as _state
from thvm_amd.tensor import Tensor, dtypes

_RNG = np.random.default_rng(0)


def manual_seed(seed: int) -> None:
    global _RNG
    _RNG = np.random.default_rng(seed)


def _uniform(shape, bound: float) -> np.ndarray:
    return _RNG.uniform(-bound, bound, size=shape).astype(np.float32)


class Linear:
    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        bound = 1.0 / math.sqrt(in_features)
        self.weight = Tensor(_uniform((out_features, in_features), bound))
        self.bias = Tensor(_uniform((out_features,), bound)) if bias else None

    def __call__(self, x: Tensor) -> Tensor:
        return x.linear(self.weight.transpose(), self.bias)


class LayerNorm:
    def __init__(self, normalized_shape: int, eps: float = 1e-5, elementwise_affine: bool = True):
        self.normalized_shape = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
        self.axis = tuple(-1 - i for i in range(len(self.normalized_shape)))
        self.eps = eps
        self.weight = Tensor(np.ones(self.normalized_shape, np.float32)) if elementwise_affine else None
        self.bias = Tensor(np.zeros(self.normalized_shape, np.float32)) if elementwise_affine else None

    def __call__(self, x: Tensor) -> Tensor:
        x = x.layernorm(axis=self.axis[0], eps=self.eps)
        if self.weight is None:
            return x
        return x * self.weight + self.bias


class RMSNorm:
    def __init__(self, dim: int, eps: float = 1e-6):
        self.eps = eps
        self.weight = Tensor(np.ones(dim, np.float32))

    def __call__(self, x: Tensor) -> Tensor:
        return x * ((x * x).mean(-1, keepdim=True) + self.eps).rsqrt() * self.weight


class Embedding:
    def __init__(self, vocab_size: int, embed_size: int):
        self.vocab_sz, self.embed_sz = vocab_size, embed_size
        self.weight = Tensor(_RNG.standard_normal((vocab_size, embed_size)).astype(np.float32))

    def __call__(self, idx: Tensor) -> Tensor:
        if idx.dtype.id != dtypes.int32.id:
            idx = idx.cast(dtypes.int32)
        return self.weight.gather_rows(idx)


def get_parameters(obj) -> list:
    """Every Tensor under obj (attributes, list items, dict values)."""
    return _state.get_parameters(obj)


# `thvm_amd.nn.state` as the reference's `thvm.nn.state` (safe_load,
# load_state_dict, ...)
state = _state
sys.modules[__name__ + ".state"] = _state
