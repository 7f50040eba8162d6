"""timm drop-in (inference): swap ViT / Swin v1 attention modules for two-pass ELSA.

Mirrors the reference's timm_dropin.py (``PatchReport`` :13-20, ``ElsaTimmVitAttention``
:23-59, ``ElsaTimmSwinWindowAttention`` :62-150, duck-typing predicates :153-172,
``patch_timm_attention`` :175-194): same class names, patched attributes, kwargs and
errors.  The attention call goes to ``twopass_attention`` (HIP two-pass kernels);
Swin windows pass the relative-position bias plus the shifted-window mask as one
broadcast bias.  ``set_window_size`` uses this package's own index/resize helpers
(elsa_amd.vision_models) instead of timm's.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import _twopass_attention
from .vision_models import relative_position_index, resize_rel_pos_bias_table


@dataclass(frozen=True)
class PatchReport:
    vit_attention: int = 0
    swin_window_attention: int = 0

    @property
    def total(self) -> int:
        return self.vit_attention + self.swin_window_attention


def _vit_state(module: nn.Module, source: nn.Module, elsa_kwargs: Optional[dict]) -> None:
    module.num_heads = int(source.num_heads)
    module.head_dim = int(source.head_dim)
    module.attn_dim = int(getattr(source, "attn_dim", module.num_heads * module.head_dim))
    module.qkv = copy.deepcopy(source.qkv)
    module.q_norm = copy.deepcopy(source.q_norm)
    module.k_norm = copy.deepcopy(source.k_norm)
    module.norm = copy.deepcopy(source.norm) if hasattr(source, "norm") else nn.Identity()
    module.proj = copy.deepcopy(source.proj)
    module.proj_drop = copy.deepcopy(source.proj_drop)
    module.elsa_kwargs = dict(elsa_kwargs or {})


def _vit_qkv(module: nn.Module, x: torch.Tensor):
    batch, seq_len, _ = x.shape
    # strided [B, H, N, D] views of the fused projection: the kernels read them in place
    qkv = module.qkv(x).reshape(batch, seq_len, 3, module.num_heads, module.head_dim).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    return module.q_norm(q), module.k_norm(k), v


def _attend(q, k, v, kwargs, bias=None):
    """twopass_attention with the output laid out as [B, N, H, D] (free transpose after)."""
    kw = dict(bias=None, is_causal=False, block_m=None, block_n=None, q_chunk_size=None, summary_dtype=None,
              phase1_warps=None, phase2_warps=None, phase1_stages=None, phase2_stages=None, input_precision="auto",
              algorithm="auto")
    kw.update(kwargs)
    if bias is not None:
        kw["bias"] = bias
    return _twopass_attention(q, k, v, out_bnhd=True, **kw)


def _vit_out(module: nn.Module, y: torch.Tensor, batch: int, seq_len: int) -> torch.Tensor:
    y = y.transpose(1, 2).reshape(batch, seq_len, module.attn_dim)
    return module.proj_drop(module.proj(module.norm(y)))


class ElsaTimmVitAttention(nn.Module):
    def __init__(self, source: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> None:
        super().__init__()
        _vit_state(self, source, elsa_kwargs)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if attn_mask is not None:
            raise ValueError("ELSA ViT drop-in currently supports unmasked attention only")
        q, k, v = _vit_qkv(self, x)
        y = _attend(q, k, v, self.elsa_kwargs)
        return _vit_out(self, y, x.shape[0], x.shape[1])


def _swin_state(module: nn.Module, source: nn.Module, elsa_kwargs: Optional[dict]) -> None:
    module.dim = int(source.dim)
    module.window_size = tuple(int(x) for x in source.window_size)
    module.window_area = int(source.window_area)
    module.num_heads = int(source.num_heads)
    module.qkv = copy.deepcopy(source.qkv)
    module.attn_drop = copy.deepcopy(source.attn_drop)
    module.proj = copy.deepcopy(source.proj)
    module.proj_drop = copy.deepcopy(source.proj_drop)
    module.softmax = copy.deepcopy(source.softmax)
    module.scale = float(source.scale)
    module.head_dim = int(module.qkv.out_features // (3 * module.num_heads))
    module.attn_dim = module.head_dim * module.num_heads
    module.relative_position_bias_table = nn.Parameter(source.relative_position_bias_table.detach().clone())
    module.register_buffer("relative_position_index", source.relative_position_index.detach().clone(),
                           persistent=False)
    module.elsa_kwargs = dict(elsa_kwargs or {})


class _SwinWindowCommon(nn.Module):
    """Shared pieces of the Swin v1 window-attention drop-ins (reference timm_dropin.py:85-144)."""

    def _get_rel_pos_bias(self) -> torch.Tensor:
        bias = self.relative_position_bias_table[self.relative_position_index.view(-1)].view(
            self.window_area, self.window_area, self.num_heads)
        return bias.permute(2, 0, 1).contiguous().unsqueeze(0)

    def set_window_size(self, window_size) -> None:
        if isinstance(window_size, int):
            window_size = (window_size, window_size)
        window_size = tuple(int(x) for x in window_size)
        if window_size == self.window_size:
            return
        self.window_size = window_size
        win_h, win_w = window_size
        self.window_area = win_h * win_w
        with torch.no_grad():
            self.relative_position_bias_table = nn.Parameter(
                resize_rel_pos_bias_table(self.relative_position_bias_table, window_size))
            self.register_buffer("relative_position_index",
                                 relative_position_index(win_h, win_w, device=self.relative_position_bias_table.device),
                                 persistent=False)

    def _q_factor(self) -> float:
        """Factor on q that turns the kernels' 1/sqrt(head_dim) into the module's own scale."""
        canonical_scale = self.head_dim ** -0.5
        return 1.0 if abs(self.scale - canonical_scale) <= 1e-12 else self.scale / canonical_scale

    def _qkv5(self, x: torch.Tensor) -> torch.Tensor:
        """The fused projection as [B_win, N, 3, H, D]."""
        batch_windows, seq_len, _ = x.shape
        return self.qkv(x).reshape(batch_windows, seq_len, 3, self.num_heads, self.head_dim)

    def _bias(self, mask: Optional[torch.Tensor], batch_windows: int, seq_len: int) -> torch.Tensor:
        """Relative-position bias plus the shifted-window mask, [B_win | 1, H, N, N].

        The values are the reference's sums (timm_dropin.py:85-90).  The tensor is built with
        rows padded to a multiple of 8 keys and returned as its [..., :N] view, so that the
        kernels read each row's keys with 16-byte loads (inference: when the table records no
        gradient).  The padding costs no launch: the
        table gather uses an index whose pad columns point at a valid table row (those keys
        are never read, and their gradient is zero), and the mask is padded once per mask."""
        npad = (-seq_len) % 8
        # with a gradient to the table, autograd would rebuild the padded layout in the
        # backward (a zero fill and a copy per layer): training keeps the dense bias
        needs_grad = torch.is_grad_enabled() and self.relative_position_bias_table.requires_grad
        if npad == 0 or needs_grad:
            bias = self._get_rel_pos_bias()
            if mask is not None:
                num_win = int(mask.shape[0])
                mask_bias = mask.view(1, num_win, 1, seq_len, seq_len).expand(
                    batch_windows // num_win, -1, self.num_heads, -1, -1)
                bias = bias + mask_bias.reshape(-1, self.num_heads, seq_len, seq_len)
            return bias
        width, h = seq_len + npad, self.num_heads
        rel = self.relative_position_bias_table[self._padded_index(seq_len, npad)]
        rel = rel.view(seq_len, width, h).permute(2, 0, 1).contiguous().unsqueeze(0)
        if mask is None:
            return rel[..., :seq_len]
        num_win = int(mask.shape[0])
        m = self._padded_mask(mask, npad)
        bias = rel.view(1, 1, h, seq_len, width) + m.view(1, num_win, 1, seq_len, width)
        bias = bias.expand(batch_windows // num_win, -1, -1, -1, -1).reshape(-1, h, seq_len, width)
        return bias[..., :seq_len]

    def _padded_index(self, seq_len: int, npad: int) -> torch.Tensor:
        idx = self.relative_position_index
        key = (idx.data_ptr(), tuple(idx.shape), idx.device, npad)
        cached = self.__dict__.get("_elsa_index_cache")
        if cached is None or cached[0] != key:
            padded = F.pad(idx.reshape(seq_len, seq_len), (0, npad)).reshape(-1)  # pads with index 0
            self.__dict__["_elsa_index_cache"] = (key, padded)
        return self.__dict__["_elsa_index_cache"][1]

    def _padded_mask(self, mask: torch.Tensor, npad: int) -> torch.Tensor:
        key = (mask.data_ptr(), tuple(mask.shape), mask.dtype, mask.device, mask._version, npad)
        cached = self.__dict__.get("_elsa_mask_cache")
        if cached is None or cached[0] != key:
            self.__dict__["_elsa_mask_cache"] = (key, F.pad(mask, (0, npad)))
        return self.__dict__["_elsa_mask_cache"][1]

    def _qkv_and_bias(self, x: torch.Tensor, mask: Optional[torch.Tensor]):
        batch_windows, seq_len, _ = x.shape
        q, k, v = self._qkv5(x).permute(2, 0, 3, 1, 4).unbind(0)
        factor = self._q_factor()
        if factor != 1.0:
            q = q * factor
        return q, k, v, self._bias(mask, batch_windows, seq_len)

    def _out(self, y: torch.Tensor, batch_windows: int, seq_len: int) -> torch.Tensor:
        y = y.transpose(1, 2).reshape(batch_windows, seq_len, self.attn_dim)
        return self.proj_drop(self.proj(y))


class ElsaTimmSwinWindowAttention(_SwinWindowCommon):
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
            raise ValueError("ELSA Swin drop-in forward is inference-only when attention dropout is nonzero")
        q, k, v, bias = self._qkv_and_bias(x, mask)
        y = _attend(q, k, v, self._elsa_kwargs_for_window(x.shape[1]), bias=bias)
        return self._out(y, x.shape[0], x.shape[1])


def _is_vit_attention(module: nn.Module) -> bool:
    required = ("qkv", "q_norm", "k_norm", "proj", "num_heads", "head_dim")
    return all(hasattr(module, name) for name in required)


def _is_swin_v1_window_attention(module: nn.Module) -> bool:
    required = ("qkv", "proj", "relative_position_bias_table", "relative_position_index", "window_area",
                "window_size", "scale", "num_heads", "dim")
    return all(hasattr(module, name) for name in required) and not hasattr(module, "logit_scale")


def _patch(model: nn.Module, vit_cls, swin_cls, elsa_kwargs: Optional[dict]) -> tuple[int, int]:
    vit_count = 0
    swin_count = 0

    def visit(parent: nn.Module) -> None:
        nonlocal vit_count, swin_count
        for name, child in list(parent.named_children()):
            if _is_vit_attention(child):
                setattr(parent, name, vit_cls(child, elsa_kwargs=elsa_kwargs))
                vit_count += 1
            elif _is_swin_v1_window_attention(child):
                setattr(parent, name, swin_cls(child, elsa_kwargs=elsa_kwargs))
                swin_count += 1
            else:
                visit(child)

    visit(model)
    if vit_count + swin_count == 0:
        raise ValueError("no compatible timm ViT or Swin v1 attention modules were patched")
    return vit_count, swin_count


def patch_timm_attention(model: nn.Module, *, elsa_kwargs: Optional[dict] = None) -> PatchReport:
    """Replace every timm ViT / Swin v1 attention module in ``model`` (in place)."""
    vit, swin = _patch(model, ElsaTimmVitAttention, ElsaTimmSwinWindowAttention, elsa_kwargs)
    return PatchReport(vit_attention=vit, swin_window_attention=swin)
