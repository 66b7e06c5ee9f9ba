"""Checkpoint state for the Tensor host: the reference's state surface
(py/thvm/nn_state.py:42-280: safe_load, safe_save, safe_load_metadata,
torch_load, get_state_dict, get_parameters, load_state_dict, tinygrad's
nn/state.py semantics) over the file readers of thvm_amd.weights.

safe_load and torch_load return device Tensors: each stored dtype maps to
the host's (f32, f16, bf16, int32, uint8, bool; f64 and fp8 widen to f32,
int64 narrows to int32).  A tensor's dotted name is its attribute path, list
index or dict key under the model object."""
from __future__ import annotations

from typing import Dict, Optional

import numpy as np

from . import weights as W
from .tensor import Tensor, dtypes

_HOST = {W.DT_FP32: dtypes.float32, W.DT_FP16: dtypes.float16, W.DT_BF16: dtypes.bfloat16,
         W.DT_INT32: dtypes.int32, W.DT_UINT8: dtypes.uint8, W.DT_BOOL: dtypes.bool}


def _to_tensor(v) -> Tensor:
    if isinstance(v, Tensor):
        return v
    if isinstance(v, W.DiskTensor):
        dt = _HOST.get(v.dtype)
        if dt is not None and dt.id != dtypes.bfloat16.id:
            return Tensor(np.array(v.numpy()), dtype=dt)
        if dt is not None:                             # bf16: exact through f32
            return Tensor(v.float32(), dtype=dtypes.bfloat16)
        a = v.float32() if v.dtype in (W.DT_FP64, W.DT_FP8E4M3, W.DT_FP8E5M2) else np.array(v.numpy())
        return Tensor(a)
    return Tensor(np.asarray(v))


def safe_load_metadata(fn):
    return W.safe_load_metadata(fn)


def safe_load(fn) -> Dict[str, Tensor]:
    return {k: _to_tensor(v) for k, v in W.safe_load(fn).items()}


def safe_save(tensors: Dict[str, Tensor], fn, metadata: Optional[dict] = None) -> None:
    out = {}
    for k, t in tensors.items():
        if not isinstance(t, Tensor):
            out[k] = np.asarray(t)
        elif t.dtype.id == dtypes.bfloat16.id:
            out[k] = (W.f32_to_bf16(t.numpy().astype(np.float32)), W.DT_BF16)
        else:
            out[k] = t.numpy()
    W.safe_save(out, fn, metadata)


def torch_load(path) -> Dict[str, Tensor]:
    return {k: _to_tensor(v) for k, v in W.torch_load(path).items()}


def _walk(obj, prefix: str, out: Dict[str, Tensor]) -> None:
    if isinstance(obj, Tensor):
        out[prefix.rstrip(".")] = obj
    elif isinstance(obj, (list, tuple)):
        for i, x in enumerate(obj):
            _walk(x, f"{prefix}{i}.", out)
    elif isinstance(obj, dict):
        for k, v in obj.items():
            _walk(v, f"{prefix}{k}.", out)
    elif hasattr(obj, "__dict__"):
        for k, v in vars(obj).items():
            _walk(v, f"{prefix}{k}.", out)


def get_state_dict(obj, prefix: str = "") -> Dict[str, Tensor]:
    out: Dict[str, Tensor] = {}
    _walk(obj, prefix, out)
    return out


def get_parameters(obj) -> list:
    return list(get_state_dict(obj).values())


def load_state_dict(model, state_dict: Dict[str, object], strict: bool = True, verbose: bool = True,
                    consume: bool = False, realize: bool = True) -> list:
    """Each model Tensor replaced by its state_dict entry (a Tensor, array or
    disk tensor) and realized; a missing key raises under strict, a shape
    mismatch always does (except () against (1,)).  Returns the loaded
    Tensors."""
    ret = []
    for k, v in get_state_dict(model).items():
        if k not in state_dict:
            if strict:
                raise KeyError(f"missing key in state_dict: {k}")
            continue
        src = _to_tensor(state_dict[k])
        if tuple(src.shape) != tuple(v.shape):
            if {(), (1,)} == {tuple(src.shape), tuple(v.shape)}:
                src = src.reshape(*v.shape) if v.shape else src.reshape(())
            else:
                raise ValueError(f"shape mismatch in `{k}`: model {v.shape} vs ckpt {src.shape}")
        v.replace(src)
        if realize:
            v.realize()
        if consume:
            del state_dict[k]
        ret.append(v)
    return ret


__all__ = ["safe_save", "safe_load", "safe_load_metadata", "torch_load", "get_state_dict",
           "get_parameters", "load_state_dict"]
