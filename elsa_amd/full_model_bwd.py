"""Trainable twin of the toy encoder (public names of the reference's full_model_bwd.py:
``TrainableTransformerEncoder``, ``make_train_model_pair``).  The ELSA core runs the autograd
path: two-pass forward with row state, exact-recompute backward, gradients of the fused qkv
projection written back in its layout."""
from __future__ import annotations

from typing import Optional

from .full_model import SdpaKind, TransformerEncoder, _twin


class TrainableTransformerEncoder(TransformerEncoder):
    """``TransformerEncoder`` whose ELSA attention carries gradients (``qkv_attention_train``)."""

    trainable = True


def make_train_model_pair(*, dim: int = 192, depth: int = 1, heads: int = 3, mlp_ratio: float = 4.0,
                          sdpa_kind: SdpaKind = "auto", is_causal: bool = False,
                          elsa_kwargs: Optional[dict] = None) -> tuple[TrainableTransformerEncoder,
                                                                       TrainableTransformerEncoder]:
    """(SDPA baseline, ELSA) trainable encoders with identical weights."""
    baseline = TrainableTransformerEncoder(dim=dim, depth=depth, heads=heads, mlp_ratio=mlp_ratio, backend="sdpa",
                                           sdpa_kind=sdpa_kind, is_causal=is_causal)
    return _twin(baseline, elsa_kwargs)
