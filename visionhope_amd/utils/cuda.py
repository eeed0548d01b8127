"""Device selection for native launches (reference ``utils/cuda.py:10-22``)."""

import functools

import torch


def _first_tensor(args, kwargs):
    for value in args:
        if isinstance(value, torch.Tensor):
            return value
    for value in kwargs.values():
        if isinstance(value, torch.Tensor):
            return value
    return None


def on_tensor_device(function):
    """Decorator: run ``function`` with the device of its first tensor argument current,
    so the native calls it makes launch on that device's current stream.  CPU tensors,
    and tensors already on the current device, run it unchanged."""
    @functools.wraps(function)
    def run_on_device(*args, **kwargs):
        tensor = _first_tensor(args, kwargs)
        if tensor is None or not tensor.is_cuda or tensor.get_device() == torch.cuda.current_device():
            return function(*args, **kwargs)
        with torch.cuda.device(tensor.device):
            return function(*args, **kwargs)
    return run_on_device
