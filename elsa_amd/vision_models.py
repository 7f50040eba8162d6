"""ViT and Swin v1 modules with timm's module layout and attribute names.

timm is not a dependency of this package.  These modules reproduce the structure
the ELSA drop-ins patch (``blocks[i].attn`` with ``qkv``/``q_norm``/``k_norm``/
``norm``/``proj``; Swin ``WindowAttention`` with ``relative_position_bias_table``,
``relative_position_index``, ``window_area``, ``scale`` ...), so
``patch_timm_attention`` works on them exactly as on timm models
(reference timm_dropin.py:153-194).  Their own attention uses PyTorch SDPA, which
is the baseline the drop-in replaces.  Used by the ViT-T / Swin-T parity tests
and the img/s measurement (ViT-Tiny: patch 16, embed 192, depth 12, 3 heads;
Swin-Tiny: embed 96, depths 2-2-6-2, heads 3-6-12-24, window 7).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F


# ----------------------------------------------------------------------------- ViT
class Attention(nn.Module):
    """Multi-head self-attention with timm's ViT attribute names."""

    def __init__(self, dim: int, num_heads: int = 8, qkv_bias: bool = True) -> None:
        super().__init__()
        if dim % num_heads:
            raise ValueError("dim must be divisible by num_heads")
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.attn_dim = dim
        self.scale = self.head_dim ** -0.5
        self.qkv = nn.Linear(dim, 3 * dim, bias=qkv_bias)
        self.q_norm = nn.Identity()
        self.k_norm = nn.Identity()
        self.attn_drop = nn.Dropout(0.0)
        self.norm = nn.Identity()
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Dropout(0.0)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        b, n, _ = x.shape
        qkv = self.qkv(x).reshape(b, n, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        q, k = self.q_norm(q), self.k_norm(k)
        y = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, scale=self.scale)
        y = y.transpose(1, 2).reshape(b, n, self.attn_dim)
        return self.proj_drop(self.proj(self.norm(y)))


class Mlp(nn.Module):
    def __init__(self, dim: int, hidden: int) -> None:
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.act = nn.GELU()
        self.drop1 = nn.Dropout(0.0)
        self.norm = nn.Identity()
        self.fc2 = nn.Linear(hidden, dim)
        self.drop2 = nn.Dropout(0.0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.drop2(self.fc2(self.norm(self.drop1(self.act(self.fc1(x))))))


class Block(nn.Module):
    def __init__(self, dim: int, num_heads: int, mlp_ratio: float = 4.0) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(dim, eps=1e-6)
        self.attn = Attention(dim, num_heads)
        self.norm2 = nn.LayerNorm(dim, eps=1e-6)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))


class PatchEmbed(nn.Module):
    def __init__(self, img_size: int, patch_size: int, in_chans: int, embed_dim: int, flatten: bool = True,
                 norm: bool = False) -> None:
        super().__init__()
        self.img_size = img_size
        self.patch_size = patch_size
        self.grid_size = (img_size // patch_size, img_size // patch_size)
        self.num_patches = self.grid_size[0] * self.grid_size[1]
        self.flatten = flatten
        self.proj = nn.Conv2d(in_chans, embed_dim, kernel_size=patch_size, stride=patch_size)
        self.norm = nn.LayerNorm(embed_dim) if norm else nn.Identity()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.proj(x)
        if self.flatten:
            return self.norm(x.flatten(2).transpose(1, 2))  # B, N, C
        return self.norm(x.permute(0, 2, 3, 1))  # B, H, W, C


class VisionTransformer(nn.Module):
    """ViT with a class token, learned position embedding and a linear head."""

    def __init__(self, *, img_size: int = 224, patch_size: int = 16, in_chans: int = 3, num_classes: int = 1000,
                 embed_dim: int = 192, depth: int = 12, num_heads: int = 3, mlp_ratio: float = 4.0) -> None:
        super().__init__()
        self.patch_embed = PatchEmbed(img_size, patch_size, in_chans, embed_dim)
        n = self.patch_embed.num_patches
        self.cls_token = nn.Parameter(torch.zeros(1, 1, embed_dim))
        self.pos_embed = nn.Parameter(torch.randn(1, n + 1, embed_dim) * 0.02)
        self.blocks = nn.Sequential(*[Block(embed_dim, num_heads, mlp_ratio) for _ in range(depth)])
        self.norm = nn.LayerNorm(embed_dim, eps=1e-6)
        self.head = nn.Linear(embed_dim, num_classes)
        nn.init.normal_(self.cls_token, std=1e-6)

    @property
    def seq_len(self) -> int:
        return self.patch_embed.num_patches + 1

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.patch_embed(x)
        x = torch.cat([self.cls_token.expand(x.shape[0], -1, -1), x], dim=1) + self.pos_embed
        x = self.norm(self.blocks(x))
        return self.head(x[:, 0])


def vit_tiny_patch16(img_size: int = 224, num_classes: int = 1000) -> VisionTransformer:
    """ViT-Tiny/16: embed 192, depth 12, 3 heads (head dim 64), MLP 768, class token."""
    return VisionTransformer(img_size=img_size, patch_size=16, embed_dim=192, depth=12, num_heads=3,
                             num_classes=num_classes)


# ----------------------------------------------------------------------------- Swin v1
def relative_position_index(win_h: int, win_w: int, device=None) -> torch.Tensor:
    """Index into the (2*win_h-1)*(2*win_w-1) bias table for every (query, key) pair of a window."""
    coords = torch.stack(torch.meshgrid(torch.arange(win_h, device=device), torch.arange(win_w, device=device),
                                        indexing="ij")).flatten(1)  # 2, Wh*Ww
    rel = (coords[:, :, None] - coords[:, None, :]).permute(1, 2, 0)  # Wh*Ww, Wh*Ww, 2
    rel[:, :, 0] += win_h - 1
    rel[:, :, 1] += win_w - 1
    return rel[:, :, 0] * (2 * win_w - 1) + rel[:, :, 1]


def resize_rel_pos_bias_table(table: torch.Tensor, new_window_size: Sequence[int]) -> torch.Tensor:
    """Bicubic resize of a [(2h-1)*(2w-1), heads] bias table to a new window size."""
    heads = table.shape[1]
    old = int(round(math.sqrt(table.shape[0])))
    new_h, new_w = 2 * new_window_size[0] - 1, 2 * new_window_size[1] - 1
    grid = table.T.reshape(1, heads, old, old)
    grid = F.interpolate(grid.float(), size=(new_h, new_w), mode="bicubic", align_corners=False)
    return grid.reshape(heads, new_h * new_w).T.to(table.dtype)


def window_partition(x: torch.Tensor, ws: Sequence[int]) -> torch.Tensor:
    b, h, w, c = x.shape
    x = x.view(b, h // ws[0], ws[0], w // ws[1], ws[1], c)
    return x.permute(0, 1, 3, 2, 4, 5).reshape(-1, ws[0], ws[1], c)


def window_reverse(windows: torch.Tensor, ws: Sequence[int], h: int, w: int) -> torch.Tensor:
    c = windows.shape[-1]
    x = windows.view(-1, h // ws[0], w // ws[1], ws[0], ws[1], c)
    return x.permute(0, 1, 3, 2, 4, 5).reshape(-1, h, w, c)


class WindowAttention(nn.Module):
    """Swin v1 window attention with timm's attribute names (relative position bias, optional mask)."""

    def __init__(self, dim: int, num_heads: int, window_size: Sequence[int]) -> None:
        super().__init__()
        self.dim = dim
        self.window_size = tuple(window_size)
        self.window_area = self.window_size[0] * self.window_size[1]
        self.num_heads = num_heads
        head_dim = dim // num_heads
        self.scale = head_dim ** -0.5
        self.relative_position_bias_table = nn.Parameter(
            torch.zeros((2 * self.window_size[0] - 1) * (2 * self.window_size[1] - 1), num_heads))
        nn.init.trunc_normal_(self.relative_position_bias_table, std=0.02)
        self.register_buffer("relative_position_index", relative_position_index(*self.window_size),
                             persistent=False)
        self.qkv = nn.Linear(dim, 3 * dim)
        self.attn_drop = nn.Dropout(0.0)
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Dropout(0.0)
        self.softmax = nn.Softmax(dim=-1)

    def _get_rel_pos_bias(self) -> torch.Tensor:
        bias = self.relative_position_bias_table[self.relative_position_index.view(-1)].view(
            self.window_area, self.window_area, -1)
        return bias.permute(2, 0, 1).contiguous().unsqueeze(0)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        b_win, n, c = x.shape
        qkv = self.qkv(x).reshape(b_win, n, 3, self.num_heads, -1).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        bias = self._get_rel_pos_bias()
        if mask is not None:
            nw = mask.shape[0]
            bias = (bias.view(1, 1, self.num_heads, n, n) + mask.view(1, nw, 1, n, n)).expand(
                b_win // nw, -1, -1, -1, -1).reshape(-1, self.num_heads, n, n)
        y = F.scaled_dot_product_attention(q, k, v, attn_mask=bias.to(q.dtype), scale=self.scale)
        y = y.transpose(1, 2).reshape(b_win, n, -1)
        return self.proj_drop(self.proj(y))


class SwinTransformerBlock(nn.Module):
    def __init__(self, dim: int, input_resolution: Sequence[int], num_heads: int, window_size: int,
                 shift: bool, mlp_ratio: float = 4.0) -> None:
        super().__init__()
        h, w = input_resolution
        ws = min(window_size, h, w)  # a window never exceeds the feature map
        self.window_size = (ws, ws)
        self.shift_size = (ws // 2, ws // 2) if (shift and min(h, w) > window_size) else (0, 0)
        self.input_resolution = (h, w)
        self.norm1 = nn.LayerNorm(dim)
        self.attn = WindowAttention(dim, num_heads, self.window_size)
        self.norm2 = nn.LayerNorm(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.register_buffer("attn_mask", self._make_mask(), persistent=False)

    def _padded(self):
        h, w = self.input_resolution
        ws = self.window_size
        return h + (ws[0] - h % ws[0]) % ws[0], w + (ws[1] - w % ws[1]) % ws[1]

    def _make_mask(self) -> Optional[torch.Tensor]:
        if not any(self.shift_size):
            return None
        hp, wp = self._padded()
        ws, ss = self.window_size, self.shift_size
        img = torch.zeros(1, hp, wp, 1)
        cnt = 0
        for hsl in (slice(0, -ws[0]), slice(-ws[0], -ss[0]), slice(-ss[0], None)):
            for wsl in (slice(0, -ws[1]), slice(-ws[1], -ss[1]), slice(-ss[1], None)):
                img[:, hsl, wsl, :] = cnt
                cnt += 1
        mw = window_partition(img, ws).view(-1, ws[0] * ws[1])
        mask = mw.unsqueeze(1) - mw.unsqueeze(2)
        return mask.masked_fill(mask != 0, -100.0).masked_fill(mask == 0, 0.0)

    def _attn(self, x: torch.Tensor) -> torch.Tensor:
        b, h, w, c = x.shape
        ss = self.shift_size
        if any(ss):
            x = torch.roll(x, shifts=(-ss[0], -ss[1]), dims=(1, 2))
        hp, wp = self._padded()
        x = F.pad(x, (0, 0, 0, wp - w, 0, hp - h))
        win = window_partition(x, self.window_size).view(-1, self.window_size[0] * self.window_size[1], c)
        mask = None if self.attn_mask is None else self.attn_mask.to(x.dtype)
        win = self.attn(win, mask=mask)
        x = window_reverse(win.view(-1, self.window_size[0], self.window_size[1], c), self.window_size, hp, wp)
        x = x[:, :h, :w, :].contiguous()
        if any(ss):
            x = torch.roll(x, shifts=ss, dims=(1, 2))
        return x

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, h, w, c = x.shape
        x = x + self._attn(self.norm1(x))
        x = x.reshape(b, -1, c)
        x = x + self.mlp(self.norm2(x))
        return x.reshape(b, h, w, c)


class PatchMerging(nn.Module):
    def __init__(self, dim: int) -> None:
        super().__init__()
        self.norm = nn.LayerNorm(4 * dim)
        self.reduction = nn.Linear(4 * dim, 2 * dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, h, w, c = x.shape
        x = F.pad(x, (0, 0, 0, w % 2, 0, h % 2))
        x = x.reshape(b, x.shape[1] // 2, 2, x.shape[2] // 2, 2, c).permute(0, 1, 3, 4, 2, 5).flatten(3)
        return self.reduction(self.norm(x))


class SwinTransformerStage(nn.Module):
    def __init__(self, dim: int, out_dim: int, input_resolution: Sequence[int], depth: int, num_heads: int,
                 window_size: int, downsample: bool) -> None:
        super().__init__()
        self.downsample = PatchMerging(dim) if downsample else nn.Identity()
        res = tuple((r + 1) // 2 for r in input_resolution) if downsample else tuple(input_resolution)
        self.output_resolution = res
        self.blocks = nn.Sequential(*[
            SwinTransformerBlock(out_dim, res, num_heads, window_size, shift=(i % 2 == 1)) for i in range(depth)
        ])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.blocks(self.downsample(x))


class SwinTransformer(nn.Module):
    def __init__(self, *, img_size: int = 224, patch_size: int = 4, in_chans: int = 3, num_classes: int = 1000,
                 embed_dim: int = 96, depths: Sequence[int] = (2, 2, 6, 2), num_heads: Sequence[int] = (3, 6, 12, 24),
                 window_size: int = 7) -> None:
        super().__init__()
        self.patch_embed = PatchEmbed(img_size, patch_size, in_chans, embed_dim, flatten=False, norm=True)
        res = self.patch_embed.grid_size
        stages = []
        dim = embed_dim
        for i, (depth, heads) in enumerate(zip(depths, num_heads)):
            out_dim = embed_dim * 2 ** i
            stage = SwinTransformerStage(dim, out_dim, res, depth, heads, window_size, downsample=i > 0)
            res = stage.output_resolution
            stages.append(stage)
            dim = out_dim
        self.layers = nn.Sequential(*stages)
        self.norm = nn.LayerNorm(dim)
        self.head = nn.Linear(dim, num_classes)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.norm(self.layers(self.patch_embed(x)))
        return self.head(x.mean(dim=(1, 2)))


def swin_tiny_patch4_window7(img_size: int = 224, num_classes: int = 1000) -> SwinTransformer:
    """Swin-T: embed 96, depths (2,2,6,2), heads (3,6,12,24) (head dim 32), window 7 with shifts."""
    return SwinTransformer(img_size=img_size, embed_dim=96, depths=(2, 2, 6, 2), num_heads=(3, 6, 12, 24),
                           window_size=7, num_classes=num_classes)
