"""Trainable twin of the toy encoder: ELSA attention through ``twopass_attention_train``.

Mirrors the reference's full_model_bwd.py (``TrainableSelfAttention`` :48-92 ...
``make_train_model_pair`` :176-205).
"""
from __future__ import annotations

from typing import Optional

import torch

from .attention_bwd import twopass_attention_train
from .full_model import MLP, SdpaKind, SelfAttention, TransformerBlock, TransformerEncoder, _pair

TrainableMLP = MLP


def _train_elsa_kwargs(q: torch.Tensor, explicit: dict) -> dict:
    kwargs = dict(explicit)
    kwargs["algorithm"] = "paper_scan"
    if q.dtype != torch.float32 and int(q.shape[-2]) >= 4096:
        kwargs.setdefault("bwd_block_m", 32)
        kwargs.setdefault("bwd_block_n", 32)
    return kwargs


class TrainableSelfAttention(SelfAttention):
    def _attend(self, q, k, v):
        if self.backend == "elsa":
            return twopass_attention_train(q, k, v, is_causal=self.is_causal, **_train_elsa_kwargs(q, self.elsa_kwargs))
        return super()._attend(q, k, v)


class TrainableTransformerBlock(TransformerBlock):
    attention_cls = TrainableSelfAttention


class TrainableTransformerEncoder(TransformerEncoder):
    """Full-model training harness using the two-pass ELSA autograd attention."""

    block_cls = TrainableTransformerBlock


def make_train_model_pair(*, dim: int = 192, depth: int = 1, heads: int = 3, mlp_ratio: float = 4.0,
                          sdpa_kind: SdpaKind = "auto", is_causal: bool = False,
                          elsa_kwargs: Optional[dict] = None) -> tuple[TrainableTransformerEncoder,
                                                                       TrainableTransformerEncoder]:
    """(SDPA baseline, ELSA) trainable encoders with identical weights."""
    return _pair(TrainableTransformerEncoder, dim=dim, depth=depth, heads=heads, mlp_ratio=mlp_ratio,
                 sdpa_kind=sdpa_kind, is_causal=is_causal, elsa_kwargs=elsa_kwargs)
