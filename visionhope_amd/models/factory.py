"""The named VisionHOPE classifiers and their constructor (reference ``models/factory.py``).

``MODEL_CONFIGS`` holds the reference's published widths and depths.  timm is not a
dependency here: the model registry is a local dict and the ImageNet normalisation
constants are written out.
"""

from copy import deepcopy

from .hierarchical import HierarchicalVisionHOPE

IMAGENET_DEFAULT_MEAN = (0.485, 0.456, 0.406)
IMAGENET_DEFAULT_STD = (0.229, 0.224, 0.225)

MODEL_CONFIGS = {
    "visionhope_tiny": dict(embed_dims=(64, 128, 256, 512),
                            mixer_dims=(32, 64, 128, 256), depths=(3, 4, 18, 4)),
    "visionhope_small": dict(embed_dims=(64, 160, 320, 512),
                             mixer_dims=(32, 80, 160, 256), depths=(4, 8, 25, 8)),
    "visionhope_base": dict(embed_dims=(96, 192, 448, 640),
                            mixer_dims=(48, 96, 224, 320), depths=(4, 8, 25, 8)),
}

MODEL_REGISTRY = {}


def register_model(fn):
    MODEL_REGISTRY[fn.__name__] = fn
    return fn


# Arguments of timm's model factory that VisionHOPE accepts only at their neutral value.
_NEUTRAL_TIMM_ARGS = {"drop_rate": 0.0, "drop_connect_rate": None, "drop_block_rate": None,
                      "global_pool": "avg", "bn_momentum": None, "bn_eps": None, "scriptable": False,
                      "pretrained_cfg": None, "pretrained_cfg_overlay": None}


def _default_cfg():
    """The timm-style data configuration a classifier built here advertises."""
    return {"url": "", "num_classes": 1000, "input_size": (3, 224, 224), "pool_size": None,
            "crop_pct": 1.0, "interpolation": "bicubic", "mean": IMAGENET_DEFAULT_MEAN,
            "std": IMAGENET_DEFAULT_STD, "classifier": "head"}


def create_model(name, pretrained=False, checkpoint_path=None, **kwargs):
    """Build a registered VisionHOPE model; with ``checkpoint_path``, load its native-name
    weights (reference ``factory.py:19-43``).  ``pretrained`` needs a checkpoint path (no
    download exists)."""
    if name not in MODEL_CONFIGS:
        raise ValueError(f"Unknown model {name!r}; choose from {tuple(MODEL_CONFIGS)}")
    if pretrained and not checkpoint_path:
        raise ValueError("Provide checkpoint_path for pretrained weights")
    for key in [k for k in kwargs if k in _NEUTRAL_TIMM_ARGS]:
        value = kwargs.pop(key)
        if value is not None and value != _NEUTRAL_TIMM_ARGS[key]:
            raise ValueError(f"Unsupported {key}={value!r}")
    model = HierarchicalVisionHOPE(**{**deepcopy(MODEL_CONFIGS[name]), **kwargs})
    model.default_cfg = _default_cfg()
    if checkpoint_path:
        from ..tools.checkpoint import load_checkpoint
        load_checkpoint(model, checkpoint_path)
    return model


@register_model
def visionhope_tiny(pretrained=False, **kwargs):
    return create_model("visionhope_tiny", pretrained=pretrained, **kwargs)


@register_model
def visionhope_small(pretrained=False, **kwargs):
    return create_model("visionhope_small", pretrained=pretrained, **kwargs)


@register_model
def visionhope_base(pretrained=False, **kwargs):
    return create_model("visionhope_base", pretrained=pretrained, **kwargs)
