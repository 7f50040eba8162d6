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

from .attention_bwd import _train_bnhd, qkv_attention_train
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
        batch, seq_len, _ = x.shape
        if isinstance(self.q_norm, nn.Identity) and isinstance(self.k_norm, nn.Identity):
            # q, k, v straight from the fused projection; its gradient comes back in place
            qkv = self.qkv(x).reshape(batch, seq_len, 3, self.num_heads, self.head_dim)
            y = qkv_attention_train(qkv, **self._elsa_kwargs_for_seq(seq_len, qkv.dtype))
        else:
            q, k, v = _vit_qkv(self, x)
            y = _train_bnhd(q, k, v, **self._elsa_kwargs_for_seq(seq_len, q.dtype))
        return _vit_out(self, y, batch, seq_len)


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
        batch_windows, seq_len, _ = x.shape
        bias = self._bias(mask, batch_windows, seq_len)
        kwargs = self._elsa_kwargs_for_window(seq_len)
        qkv = self._qkv5(x)
        factor = self._q_factor()
        if factor == 1.0:
            y = qkv_attention_train(qkv, bias=bias, **kwargs)
        else:
            q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
            y = _train_bnhd(q * factor, k, v, bias=bias, **kwargs)
        return self._out(y, batch_windows, seq_len)


def patch_timm_attention_train(model: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> TrainPatchReport:
    """Replace every timm ViT / Swin v1 attention module with its trainable ELSA twin (in place)."""
    vit, swin = _patch(model, ElsaTrainTimmVitAttention, ElsaTrainTimmSwinWindowAttention, elsa_kwargs)
    return TrainPatchReport(vit_attention=vit, swin_window_attention=swin)
