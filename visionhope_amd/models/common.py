"""Initialisation and the classifier interface shared by the VisionHOPE models.

Public surface of the reference's ``models/common.py``: ``initialize_weights`` and the
``ClassificationModel`` base (classifier access, activation checkpointing, the training
guard of prepared models).
"""

import torch
from torch import nn
from torch.nn.init import trunc_normal_
from torch.utils.checkpoint import checkpoint


def initialize_weights(module):
    """Linear and convolution weights: truncated normal, std 0.02; biases: zero."""
    if not isinstance(module, (nn.Linear, nn.Conv2d)):
        return
    trunc_normal_(module.weight, std=0.02)
    if module.bias is not None:
        nn.init.zeros_(module.bias)


class ClassificationModel(nn.Module):
    """Base of the classifiers: ``forward = head(forward_features(x))``.  Subclasses define
    ``forward_features``, ``head``, ``num_features`` and ``grad_checkpointing``."""

    def forward(self, x):
        return self.head(self.forward_features(x))

    def get_classifier(self):
        return self.head

    def reset_classifier(self, num_classes, global_pool=None):
        """A new linear classifier for ``num_classes`` (pooling is always the average)."""
        if global_pool is not None and global_pool != "avg":
            raise ValueError("VisionHOPE uses global average pooling")
        self.num_classes = num_classes
        self.head = nn.Linear(self.num_features, num_classes)
        initialize_weights(self.head)

    def set_grad_checkpointing(self, enable=True):
        self.grad_checkpointing = bool(enable)

    def _run_blocks(self, blocks, x):
        """The blocks of a stage, each recomputed in backward when checkpointing applies."""
        if not (self.grad_checkpointing and self.training and torch.is_grad_enabled()):
            return blocks(x)
        for block in blocks:
            x = checkpoint(block, x, use_reentrant=False)
        return x

    def train(self, mode=True):
        if mode and getattr(self, "_inference_prepared", False):
            raise RuntimeError("This model has folded inference weights; train an unfused model")
        return super().train(mode)
