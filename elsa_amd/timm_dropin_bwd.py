"""timm drop-in (training): ViT / Swin v1 attention through ``twopass_attention_train``.

Mirrors the reference's timm_dropin_bwd.py (``TrainPatchReport`` :13-20,
``ElsaTrainTimmVitAttention`` :23-77, ``ElsaTrainTimmSwinWindowAttention`` :80-172,
``patch_timm_attention_train`` :197-216).  The reference's sequence-length tile
table (:40-61) only picks Triton tiles; here the same kwargs are set (so callers see
the same defaults) and the HIP planner chooses its own tiles.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from .attention_bwd import twopass_attention_train
from .timm_dropin import _SwinWindowCommon, _patch, _swin_state, _vit_out, _vit_qkv, _vit_state


@dataclass(frozen=True)
class TrainPatchReport:
    vit_attention: int = 0
    swin_window_attention: int = 0

    @property
    def total(self) -> int:
        return self.vit_attention + self.swin_window_attention


class ElsaTrainTimmVitAttention(nn.Module):
    def __init__(self, source: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> None:
        super().__init__()
        _vit_state(self, source, elsa_kwargs)
        self.attn_drop = copy.deepcopy(source.attn_drop) if hasattr(source, "attn_drop") else nn.Dropout(0.0)

    def _elsa_kwargs_for_seq(self, seq_len: int, dtype: torch.dtype) -> dict:
        kwargs = dict(self.elsa_kwargs)
        kwargs["algorithm"] = "paper_scan"
        if dtype != torch.float32 and seq_len >= 4096:
            kwargs.setdefault("bwd_block_m", 32)
            kwargs.setdefault("bwd_block_n", 32)
        kwargs.setdefault("q_chunk_size", seq_len)
        return kwargs

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if attn_mask is not None:
            raise ValueError("ELSA ViT bwd drop-in currently supports unmasked attention only")
        if self.training and getattr(self.attn_drop, "p", 0.0):
            raise ValueError("ELSA ViT bwd drop-in does not implement attention dropout")
        q, k, v = _vit_qkv(self, x)
        y = twopass_attention_train(q, k, v, **self._elsa_kwargs_for_seq(x.shape[1], q.dtype))
        return _vit_out(self, y, x.shape[0], x.shape[1])


class ElsaTrainTimmSwinWindowAttention(_SwinWindowCommon):
    def __init__(self, source: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> None:
        super().__init__()
        _swin_state(self, source, elsa_kwargs)

    def _elsa_kwargs_for_window(self, seq_len: int) -> dict:
        kwargs = dict(self.elsa_kwargs)
        kwargs["algorithm"] = "paper_scan"
        kwargs.setdefault("block_m", 64)
        kwargs.setdefault("block_n", 64)
        kwargs.setdefault("q_chunk_size", seq_len)
        return kwargs

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.training and self.attn_drop.p:
            raise ValueError("ELSA Swin bwd drop-in does not implement attention dropout")
        q, k, v, bias = self._qkv_and_bias(x, mask)
        y = twopass_attention_train(q, k, v, bias=bias, **self._elsa_kwargs_for_window(x.shape[1]))
        return self._out(y, x.shape[0], x.shape[1])


def patch_timm_attention_train(model: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> TrainPatchReport:
    """Replace every timm ViT / Swin v1 attention module with its trainable ELSA twin (in place)."""
    vit, swin = _patch(model, ElsaTrainTimmVitAttention, ElsaTrainTimmSwinWindowAttention, elsa_kwargs)
    return TrainPatchReport(vit_attention=vit, swin_window_attention=swin)
