"""Weight files with the model's own parameter names.

File format of the reference's ``tools/checkpoint.py:17-38``: a ``torch.save`` of
``{'state_dict': state}`` whose keys are the modules' native names (for example
``stages.0.0.operator.srnl.M_m_0``), read back with ``torch.load(weights_only=True)``;
reference weight files therefore load as they are, with no key conversion.
"""

from collections import OrderedDict
from collections.abc import Mapping

import torch

CONTAINER_KEY = "state_dict"


def _require_named_tensors(state):
    if not isinstance(state, Mapping) or len(state) == 0:
        raise ValueError("state_dict must be a nonempty mapping of tensor names to tensors")
    for key, value in state.items():
        if not isinstance(key, str) or not isinstance(value, torch.Tensor):
            raise TypeError("state_dict must contain only named tensors")


def read_weights(path, *, map_location="cpu"):
    """The state dict of a weight file (the container must hold nothing but it)."""
    payload = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(payload, Mapping) or list(payload) != [CONTAINER_KEY]:
        raise ValueError("A VisionHOPE weight file must contain only 'state_dict'")
    state = payload[CONTAINER_KEY]
    _require_named_tensors(state)
    return state


def save_weights(path, state_dict):
    """Write ``state_dict`` (parameters and buffers, copied to the CPU) with its names and
    the module version metadata ``load_state_dict`` uses."""
    _require_named_tensors(state_dict)
    cpu_state = OrderedDict()
    for key, value in state_dict.items():
        cpu_state[key] = value.detach().to("cpu")
    metadata = getattr(state_dict, "_metadata", None)
    if metadata is not None:
        cpu_state._metadata = metadata
    torch.save({CONTAINER_KEY: cpu_state}, path)


def load_checkpoint(model, path, *, strict=True, map_location="cpu"):
    """``model.load_state_dict`` of a weight file's native keys."""
    return model.load_state_dict(read_weights(path, map_location=map_location), strict=strict)
